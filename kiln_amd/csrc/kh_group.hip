// kh_group.hip — gather_qmm at prefill sizes: the rows of the batch grouped by
// expert and run through the MFMA GEMM once per expert tile.
//
// gather_qmm (crates/kiln-mlx/src/ops.rs:390-429) computes, for every batch
// pair b, x[b] @ dequantize(w[e_b])^T. SwitchGlu (crates/kiln-models/src/
// moe.rs:272-310) calls it with T*k pairs of one row each, sorted by expert
// when T*k >= 64. Run pair by pair, every row streams its expert's whole
// weight matrix; grouped, each expert's codes are read once per row tile.
//
//   1. the plan, over the whole GPU: group_count_kernel (1024 pairs per
//      workgroup) counts each workgroup's pairs per expert (ids outside
//      [-E, E) form one more group) and marks every padded row as padding; group_scan_kernel (one workgroup, one thread
//      per group) pads each group's rows to whole m-tiles of 16*mt rows,
//      writes the expert of every m-tile and turns the counts into each
//      workgroup's first slot per group; group_pos_kernel (the count
//      kernel's partition) gives every pair its padded row.
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

constexpr int kScanThreads = 1024;  // one thread per group in the scan
constexpr int kPairThreads = 256;   // threads of the count and slot kernels
constexpr int kPairsPerThread = 4;  // their pairs per thread (ids loaded together)
constexpr int kPairsPerWg = kPairThreads * kPairsPerThread;
constexpr int kBatch = 16;          // workgroup counts the scan loads at once
static_assert(kGroupMaxE + 1 <= kScanThreads, "one scan thread per group");

// wcnt[w * (E+1) + e] = pairs of workgroup w's block (kPairsPerWg pairs)
// with expert e.
// Also marks every padded row as padding (rowmap = -1; the rows' own
// entries are written after the scan).
__global__ __launch_bounds__(kPairThreads) void group_count_kernel(GatherArgs g, int* __restrict__ wcnt,
                                                                   int64_t padded, int* __restrict__ rowmap) {
  __shared__ int h[kGroupMaxE + 1];
  const int tid = threadIdx.x, G1 = g.E + 1;
  for (int i = tid; i < G1; i += kPairThreads) h[i] = 0;
  __syncthreads();
  int ev[kPairsPerThread];
#pragma unroll
  for (int j = 0; j < kPairsPerThread; ++j) {
    const int64_t b = (int64_t)blockIdx.x * kPairsPerWg + j * kPairThreads + tid;
    int64_t xo;
    ev[j] = b < g.pairs ? gather_expert(g, b, &xo) : -1;
  }
#pragma unroll
  for (int j = 0; j < kPairsPerThread; ++j)
    if (ev[j] >= 0) atomicAdd(&h[ev[j]], 1);
  __syncthreads();
  for (int i = tid; i < G1; i += kPairThreads) wcnt[(int64_t)blockIdx.x * G1 + i] = h[i];
  for (int64_t r = (int64_t)blockIdx.x * kPairThreads + tid; r < padded; r += (int64_t)gridDim.x * kPairThreads)
    rowmap[r] = -1;
}

// Thread e (one per group): the group's m-tiles, their prefix sum over the
// groups, tab (m-tile count, expert per m-tile), and in place of the counts
// the first padded row of each workgroup's pairs of the group.
__global__ __launch_bounds__(kScanThreads) void group_scan_kernel(GatherArgs g, int nwg, int* __restrict__ wcnt,
                                                                  int M, int BM, int* __restrict__ tab) {
  __shared__ int sc[kScanThreads];
  const int tid = threadIdx.x, G1 = g.E + 1;
  int64_t tot = 0;
  if (tid < G1)
    for (int w0 = 0; w0 < nwg; w0 += kBatch) {
      int c[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) c[j] = w0 + j < nwg ? wcnt[(int64_t)(w0 + j) * G1 + tid] : 0;
#pragma unroll
      for (int j = 0; j < kBatch; ++j) tot += c[j];
    }
  const int nt = tid < G1 ? (int)((tot * M + BM - 1) / BM) : 0;
  sc[tid] = nt;
  __syncthreads();
  for (int off = 1; off < kScanThreads; off <<= 1) {  // inclusive prefix sum (Hillis-Steele)
    const int v = tid >= off ? sc[tid - off] : 0;
    __syncthreads();
    sc[tid] += v;
    __syncthreads();
  }
  const int t0 = sc[tid] - nt;  // first m-tile of group tid
  for (int j = 0; j < nt; ++j) tab[1 + t0 + j] = tid < g.E ? tid : 0;  // out-of-range rows: any expert
  if (tid == kScanThreads - 1) tab[0] = sc[tid];
  if (tid < G1) {
    int run = t0 * BM;
    for (int w0 = 0; w0 < nwg; w0 += kBatch) {
      int c[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) c[j] = w0 + j < nwg ? wcnt[(int64_t)(w0 + j) * G1 + tid] : 0;
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        if (w0 + j < nwg) wcnt[(int64_t)(w0 + j) * G1 + tid] = run;
        run += c[j] * M;
      }
    }
  }
}

// pos[b] = padded row of pair b's first row: its workgroup's first slot in
// its group plus its rank among them (an LDS atomic: the order among one
// workgroup's pairs of a group does not change any result).
__global__ __launch_bounds__(kPairThreads) void group_pos_kernel(GatherArgs g, const int* __restrict__ woff,
                                                                 int M, int* __restrict__ pos) {
  __shared__ int cur[kGroupMaxE + 1];
  const int tid = threadIdx.x, G1 = g.E + 1;
  for (int i = tid; i < G1; i += kPairThreads) cur[i] = 0;
  __syncthreads();
  int ev[kPairsPerThread];
#pragma unroll
  for (int j = 0; j < kPairsPerThread; ++j) {
    const int64_t b = (int64_t)blockIdx.x * kPairsPerWg + j * kPairThreads + tid;
    int64_t xo;
    ev[j] = b < g.pairs ? gather_expert(g, b, &xo) : -1;
  }
#pragma unroll
  for (int j = 0; j < kPairsPerThread; ++j) {
    if (ev[j] < 0) continue;
    const int64_t b = (int64_t)blockIdx.x * kPairsPerWg + j * kPairThreads + tid;
    pos[b] = woff[(int64_t)blockIdx.x * G1 + ev[j]] + atomicAdd(&cur[ev[j]], 1) * M;
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

static int64_t plan_wgs(const GatherArgs& g) { return (g.pairs + kPairsPerWg - 1) / kPairsPerWg; }

size_t group_workspace_bytes(const GroupPlan& p, const QmvArgs& a, const GatherArgs& g) {
  return align256((size_t)p.padded * a.K * 2) + 2 * align256((size_t)p.padded * 4) +
         align256((size_t)g.pairs * 4) + align256((size_t)(1 + p.tiles_max) * 4) +
         align256((size_t)plan_wgs(g) * (g.E + 1) * 4);
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
  base += align256((size_t)(1 + p.tiles_max) * 4);
  int* wcnt = reinterpret_cast<int*>(base);
  const int64_t nwg = plan_wgs(g);
  hipLaunchKernelGGL(group_count_kernel, dim3((unsigned)nwg), dim3(kPairThreads), 0, a.stream, g, wcnt,
                     p.padded, rowmap);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(group_scan_kernel, dim3(1), dim3(kScanThreads), 0, a.stream, g, (int)nwg, wcnt, a.M,
                     16 * p.mt, tab);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL(group_pos_kernel, dim3((unsigned)nwg), dim3(kPairThreads), 0, a.stream, g, wcnt, a.M, pos);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  e = launch_group_prep_x(a, g, pos, xh, rsc, rowmap);
  if (e != hipSuccess) return e;
  QmvArgs gp = a;
  gp.M = (int)p.padded;
  return launch_gemm_grouped(gp, p.mt, (int)p.tiles_max, xh, rsc, tab, rowmap);
}

}  // namespace kh
