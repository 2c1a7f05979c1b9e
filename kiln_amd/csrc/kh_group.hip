// kh_group.hip — gather_qmm at prefill sizes: the rows of the batch grouped by
// expert and run through the MFMA GEMM once per expert tile.
//
// gather_qmm (crates/kiln-mlx/src/ops.rs:390-429) computes, for every batch
// pair b, x[b] @ dequantize(w[e_b])^T. SwitchGlu (crates/kiln-models/src/
// moe.rs:272-310) calls it with T*k pairs of one row each, sorted by expert
// when T*k >= 64. Run pair by pair, every row streams its expert's whole
// weight matrix; grouped, each expert's codes are read once per row tile.
//
//   1. group_plan_kernel (one workgroup): counts the pairs of each expert
//      (ids outside [-E, E) form one more group), pads each group's rows to
//      whole m-tiles of 16*mt rows, writes the expert of every m-tile and the
//      padded row of every pair's first row.
//   2. group_prep_x: each row of x as float16 (the GEMM's activation format)
//      at its padded row; rowmap[padded row] = its output row.
//   3. gemm_kernel in grouped mode: m-tile tm uses expert gtab[1 + tm]'s
//      codes, scales and biases; outputs go to rowmap's rows, padding rows
//      are dropped.
//
// A row's result depends only on its own activations and its expert, never
// on its padded position or its neighbours, so the order in which rows of one
// group receive their slots (LDS atomics) does not change any output bit.
#include <algorithm>

#include "kh_common.h"
#include "kh_kernels.h"

namespace kh {

namespace {

constexpr int kPlanThreads = 1024;  // one thread per group in the scan
constexpr int kChunk = 16;          // ids a thread loads at once
static_assert(kGroupMaxE + 1 <= kPlanThreads, "one scan slot per group");

// Thread tid takes the contiguous block of pairs [tid * per, (tid+1) * per),
// reads its ids kChunk at a time (all loads in flight together) and counts
// runs of equal experts, so sorted ids (SwitchGlu's sort path) cost one LDS
// atomic per run instead of one per pair on a shared counter.
__global__ __launch_bounds__(kPlanThreads) void group_plan_kernel(GatherArgs g, int M, int BM,
                                                                  int64_t padded, int* __restrict__ tab,
                                                                  int* __restrict__ pos,
                                                                  int* __restrict__ rowmap) {
  __shared__ int cnt[kPlanThreads];
  __shared__ int sc[kPlanThreads];
  const int tid = threadIdx.x;
  const int64_t per = (g.pairs + kPlanThreads - 1) / kPlanThreads;
  const int64_t b0 = min<int64_t>(g.pairs, tid * per), b1 = min<int64_t>(g.pairs, b0 + per);
  cnt[tid] = 0;
  __syncthreads();
  // experts of pairs base .. base+kChunk-1 (-1 past the block), loaded together
  auto chunk = [&](int64_t base, int (&ev)[kChunk]) {
#pragma unroll
    for (int j = 0; j < kChunk; ++j) {
      int64_t xo;
      ev[j] = base + j < b1 ? gather_expert(g, base + j, &xo) : -1;
    }
  };
  {
    int run_e = -1, run_n = 0;
    for (int64_t base = b0; base < b1; base += kChunk) {
      int ev[kChunk];
      chunk(base, ev);
#pragma unroll
      for (int j = 0; j < kChunk; ++j) {
        if (ev[j] < 0) break;
        if (ev[j] != run_e) {
          if (run_n) atomicAdd(&cnt[run_e], run_n);
          run_e = ev[j];
          run_n = 0;
        }
        ++run_n;
      }
    }
    if (run_n) atomicAdd(&cnt[run_e], run_n);
  }
  __syncthreads();
  // m-tiles of group tid, then their inclusive prefix sum (Hillis-Steele)
  const int nt = tid <= g.E ? (int)(((int64_t)cnt[tid] * M + BM - 1) / BM) : 0;
  sc[tid] = nt;
  __syncthreads();
  for (int off = 1; off < kPlanThreads; off <<= 1) {
    const int v = tid >= off ? sc[tid - off] : 0;
    __syncthreads();
    sc[tid] += v;
    __syncthreads();
  }
  const int t0 = sc[tid] - nt;  // first m-tile of group tid
  for (int j = 0; j < nt; ++j) tab[1 + t0 + j] = tid < g.E ? tid : 0;  // out-of-range rows: any expert
  if (tid == kPlanThreads - 1) tab[0] = sc[tid];
  __syncthreads();
  cnt[tid] = 0;        // now the slot cursor of each group
  sc[tid] = t0 * BM;   // now the first padded row of each group
  __syncthreads();
  for (int64_t r = tid; r < padded; r += kPlanThreads) rowmap[r] = -1;
  // slots: one atomic per run (within a chunk) reserves its consecutive slots
  for (int64_t base = b0; base < b1; base += kChunk) {
    int ev[kChunk];
    chunk(base, ev);
    int cur = ev[0], j0 = 0;  // the run being scanned: expert, first index
#pragma unroll
    for (int j = 1; j <= kChunk; ++j) {
      const int ej = j < kChunk ? ev[j] : -2;
      if (ej != cur) {
        if (cur >= 0) {
          const int first = atomicAdd(&cnt[cur], j - j0);
          for (int q = j0; q < j; ++q) pos[base + q] = sc[cur] + (first + q - j0) * M;
        }
        cur = ej;
        j0 = j;
      }
    }
  }
}

size_t align256(size_t b) { return (b + 255) / 256 * 256; }

}  // namespace

GroupPlan plan_group(const QmvArgs& a, const GatherArgs& g) {
  GroupPlan p;
  p.rows = g.pairs * a.M;
  // groups that can be non-empty; rows per group on average pick the tile height
  const int64_t groups = std::max<int64_t>(1, std::min<int64_t>(g.E + 1, g.pairs));
  const int64_t avg = (p.rows + groups - 1) / groups;
  int mt = 1;
  while (mt < 8 && 16 * mt < avg) mt *= 2;
  p.mt = mt;
  const int64_t BM = 16 * mt;
  // sum over groups of ceil(rows_e / BM) <= rows / BM + groups
  p.tiles_max = (p.rows + BM - 1) / BM + groups;
  p.padded = p.tiles_max * BM;
  return p;
}

size_t group_workspace_bytes(const GroupPlan& p, const QmvArgs& a, const GatherArgs& g) {
  return align256((size_t)p.padded * a.K * 2) + 2 * align256((size_t)p.padded * 4) +
         align256((size_t)g.pairs * 4) + align256((size_t)(1 + p.tiles_max) * 4);
}

hipError_t launch_gather_grouped(const QmvArgs& a, const GatherArgs& g, const GroupPlan& p, void* ws) {
  char* base = static_cast<char*>(ws);
  void* xh = base;
  base += align256((size_t)p.padded * a.K * 2);
  float* rsc = reinterpret_cast<float*>(base);
  base += align256((size_t)p.padded * 4);
  int* rowmap = reinterpret_cast<int*>(base);
  base += align256((size_t)p.padded * 4);
  int* pos = reinterpret_cast<int*>(base);
  base += align256((size_t)g.pairs * 4);
  int* tab = reinterpret_cast<int*>(base);
  hipLaunchKernelGGL(group_plan_kernel, dim3(1), dim3(kPlanThreads), 0, a.stream, g, a.M, 16 * p.mt,
                     p.padded, tab, pos, rowmap);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = launch_group_prep_x(a, g, pos, xh, rsc, rowmap);
  if (e != hipSuccess) return e;
  QmvArgs gp = a;
  gp.M = (int)p.padded;
  return launch_gemm_grouped(gp, p.mt, (int)p.tiles_max, xh, rsc, tab, rowmap);
}

}  // namespace kh
