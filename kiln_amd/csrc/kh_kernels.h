// kh_kernels.h — host-side launcher interface between the C ABI and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kh_common.h"

namespace kh {

// Quantized matmul, transpose=true: x [M, K], w [N, K*bits/32],
// scales/biases [N, K/gs], out [M, N].
struct QmvArgs {
  const void* x;
  int xdt;
  const void* w;
  const void* scales;
  const void* biases;
  int sdt;
  void* out;
  int odt;
  int M, N, K, gs, bits;
  hipStream_t stream;
  // Linear::forward's optional bias [N] (nullptr: none), its dtype, and the
  // dtype the product is rounded to before the bias is added.
  const void* bias = nullptr;
  int bdt = 0, ydt = 0;
  Epilogue epi() const { return Epilogue{bias, bdt, ydt}; }
};

// Small batches (M <= kSkinnyMaxM, K % 128 == 0): weights streamed once,
// M rows on the matrix cores, exact products (kh_skinny.hip).
constexpr int kSkinnyMaxM = 32;
bool skinny_supported(int64_t M, int64_t N, int64_t K, int bits, int gs);
// Waves of the skinny launch with one 16-row tile per workgroup: ceil(N/16)
// times the waves that split K (the largest divisor of K/128 up to 8).
int64_t skinny_waves(int64_t N, int64_t K);
hipError_t launch_skinny(const QmvArgs& a);
// Up to 4 parts on one x (each skinny_supported, same M, K, bits, group size
// and x/scales dtypes), one launch; each part's result equals launch_skinny's.
hipError_t launch_skinny_multi(const QmvArgs* a, int n);
// act(gate) * up (ACT_SILU / ACT_GELU_APPROX) in one launch, each output
// summed as launch_skinny sums it; gate and up of equal shapes.
bool skinny_pairable(const QmvArgs& gate);
hipError_t launch_skinny_gate_up(const QmvArgs& gate, const QmvArgs& up, int act);

// Largest M served by the decode kernel; larger M takes the prefill GEMM.
constexpr int kDecodeMaxM = 16;

// Decode GEMV for the smallest batches: VALU dot products over one pass of
// the weights, activations held in registers. Serves 1 <= M <= gemv_max_m(K,
// bits) (4, or fewer for very long rows; 0 when K is too long for it).
int gemv_max_m(int K, int bits);
// The kernel addresses each operand with 32-bit byte offsets.
bool gemv_fits(int64_t M, int64_t N, int64_t K, int bits, int gs);
hipError_t launch_gemv(const QmvArgs& a);
// Up to 4 weight sets sharing x (and M, K, bits, group size, dtypes), one
// launch: q/k/v projections.
hipError_t launch_gemv_multi(const QmvArgs* a, int n);
// gather_qmm over expert stacks: a.w/scales/biases hold E slices of [N, ..];
// pair p (of `pairs`) uses activation block x + xoff(p) ([M, K]) and expert
// idx[ioff(p)], writing out + p*M*N. Offsets come from p's coordinates over
// `shape` (nd batch dims) times the strides xs (elements of x) and is
// (elements of idx).
struct GatherArgs {
  const void* idx;
  bool idx_signed;
  int E;
  int64_t pairs;
  int nd;
  int shape[8];
  int64_t xs[8], is[8];
};
// Element offset of pair b's id in idx; *xo = the pair's element offset in x.
__device__ __forceinline__ int64_t gather_io(const GatherArgs& g, int64_t b, int64_t* xo) {
  if (g.nd == 1) {  // one batch dimension (b < shape[0]): no division
    *xo = b * g.xs[0];
    return b * g.is[0];
  }
  int64_t xoff = 0, io = 0, rem = b;
  for (int d = g.nd - 1; d >= 0; --d) {
    const int64_t c = rem % g.shape[d];
    rem /= g.shape[d];
    xoff += c * g.xs[d];
    io += c * g.is[d];
  }
  *xo = xoff;
  return io;
}
__device__ __forceinline__ int gather_raw(const GatherArgs& g, int64_t io) {
  return g.idx_signed ? static_cast<const int32_t*>(g.idx)[io]
                      : (int)static_cast<const uint32_t*>(g.idx)[io];
}
// Expert of a raw id (g.E when the id is outside [-E, E)).
__device__ __forceinline__ int gather_to_expert(const GatherArgs& g, int raw) {
  int64_t e = g.idx_signed ? (int64_t)raw : (int64_t)(uint32_t)raw;
  if (e < 0) e += g.E;
  return e >= 0 && e < g.E ? (int)e : g.E;
}
// Expert of pair b; *xo = the pair's element offset in x.
__device__ __forceinline__ int gather_expert(const GatherArgs& g, int64_t b, int64_t* xo) {
  return gather_to_expert(g, gather_raw(g, gather_io(g, b, xo)));
}
hipError_t launch_gemv_gather(const QmvArgs& a, const GatherArgs& g);
// Any dtype/alignment/M: one thread per output, float32 fma chain.
hipError_t launch_gather_generic(const QmvArgs& a, const GatherArgs& g);

// gate.out = act(x gate^T [+ gate.bias]) * (x up^T [+ up.bias]) (act_mul
// sequence, act = ACT_SILU or ACT_GELU_APPROX), one launch; gate.N == up.N.
hipError_t launch_gemv_gate_up(const QmvArgs& gate, const QmvArgs& up, int act);

// Decode path (M <= kDecodeMaxM; correct up to M = 64), MFMA on unscaled
// codes with per-group fp32 scaling.
hipError_t launch_qmv(const QmvArgs& a);

// Set n 32-bit words to value (a kernel, so it is safe inside graph capture).
hipError_t launch_fill_u32(void* p, int64_t n, uint32_t value, hipStream_t stream);

// Prefill path (any M; chosen for M > kDecodeMaxM): LDS-tiled float16 MFMA
// GEMM. `ws` is a 16-byte aligned device workspace of qmm_workspace_bytes(M, K)
// bytes (float16 activations and per-row scales).
hipError_t launch_qmm(const QmvArgs& a, void* ws);
size_t qmm_workspace_bytes(int M, int K);

// x -> float16 rows scaled by an exact power of two (rsc[m] = 2^e_m), in the
// pair order of the code operands: xh holds M*K*2 bytes, 16-byte aligned.
hipError_t launch_prep_x(const QmvArgs& a, void* xh, float* rsc);

// gather_qmm at prefill sizes (kh_group.hip): the batch's rows grouped by
// expert, each group padded to whole m-tiles of 16*mt rows, through the
// GEMM in grouped mode. Experts 0..kGroupMaxE-1 (ids beyond give zero rows).
constexpr int kGroupMaxE = 1023;
struct GroupPlan {
  int mt;
  int64_t rows;       // pairs * M
  int64_t tiles_max;  // m-tiles the padded buffer holds
  int64_t padded;     // tiles_max * 16 * mt
};
GroupPlan plan_group(const QmvArgs& a, const GatherArgs& g);
// Workspace bytes of the grouped call (16-byte aligned pieces).
size_t group_workspace_bytes(const GroupPlan& p, const QmvArgs& a, const GatherArgs& g);
hipError_t launch_gather_grouped(const QmvArgs& a, const GatherArgs& g, const GroupPlan& p, void* ws);
hipError_t launch_group_prep_x(const QmvArgs& a, const GatherArgs& g, const int* pos, void* xh,
                               float* rsc, int* rowmap);
hipError_t launch_gemm_grouped(const QmvArgs& a, int mt, int tiles_max, const void* xh,
                               const float* rsc, const int* gtab, const int* rowmap);

// Quantized GEMM for every M above the VALU-GEMV range (K % 128 == 0): a
// (16*mt) x 256 tile per workgroup, float16 MFMA on weights dequantised once
// in registers, deterministic split-K. The plan depends on M only through mt.
struct GemmPlan {
  int mt, tiles_m, tiles_n, nsplit, kslice;
  int tail;  // last tiles run as two half-width workgroups each (a second launch)
};
GemmPlan plan_gemm(int M, int N, int K, int bits);
bool gemm_supported(int K);
size_t gemm_partial_bytes(const GemmPlan& p, int M, int N);
// xh/rsc from launch_prep_x; part: gemm_partial_bytes(p) bytes (unused if 0).
// reduce = false leaves a split-K launch's partial sums in part.
hipError_t launch_gemm(const QmvArgs& a, const GemmPlan& p, const void* xh, const float* rsc,
                       float* part, bool reduce = true);
// act(gate) * up from the partial sums of two split-K launches (nsplit > 1
// each) into g.out, bitwise as two reduced launches and launch_act_mul.
// n <= 4 GEMMs on one converted x as one launch (same bits, group size,
// scale dtype and m-tile, no tail launch: gemm_multi_compatible). Parts with
// nsplit > 1 leave their partial sums in part[i] (launch_gemm_reduce_multi);
// the others store their results.
bool gemm_multi_compatible(const QmvArgs* a, const GemmPlan* p, int n);
hipError_t launch_gemm_multi(const QmvArgs* a, const GemmPlan* p, const void* xh, const float* rsc,
                             float* const* part, int n);
// The reductions of n <= 4 split-K launches (nsplit > 1 each, partial sums
// in part[i]) in one launch, each output as launch_gemm's own reduction.
hipError_t launch_gemm_reduce_multi(const QmvArgs* a, const GemmPlan* p, float* const* part, int n);
hipError_t launch_gemm_reduce_gate_up(const QmvArgs& g, const GemmPlan& pg, const float* part_g,
                                      const QmvArgs& u, const GemmPlan& pu, const float* part_u, int act);

// Any dtype / alignment / transpose: one thread per output, fp32 fma chain.
hipError_t launch_qmm_generic(const QmvArgs& a, bool transpose);

// Dequantize rows: w [R, K*bits/32] -> out [R, K].
hipError_t launch_dequantize(const void* w, const void* scales, const void* biases, int sdt,
                             void* out, int odt, int64_t R, int64_t K, int gs, int bits,
                             hipStream_t stream);

// Quantized embedding: out[t, :] = dequantize(row ids[t]); V table rows.
hipError_t launch_embedding(const void* ids, bool ids_signed, int64_t T, const void* w,
                            const void* scales, const void* biases, int sdt, void* out, int odt,
                            int64_t V, int64_t H, int gs, int bits, hipStream_t stream);

// Affine quantization of rows x K values (dtype wdt) into packed codes
// [rows, K*bits/32] and scales/biases [rows, K/gs] of dtype wdt.
hipError_t launch_quantize(const void* w, int wdt, void* wq, void* scales, void* biases,
                           int64_t rows, int64_t K, int gs, int bits, hipStream_t stream);

// res[i] = act_mul(g[i], u[i], dt, act) (g, u, res all of dtype dt).
hipError_t launch_act_mul(const void* g, const void* u, void* res, int dt, int64_t n, int act,
                          hipStream_t stream);

// res[i] = a[i] + b[i % nb] (float32 sum, rounded once to rdt).
hipError_t launch_add(const void* a, int adt, const void* b, int bdt, void* res, int rdt, int64_t n,
                      int64_t nb, hipStream_t stream);

// res = a + b with numpy broadcasting: res has `shape` (nd dims); a and b are
// read with element strides as / bs (0 along their broadcast dimensions).
struct AddShape {
  int nd;
  int64_t shape[8], as[8], bs[8];
};
hipError_t launch_add_bcast(const void* a, int adt, const void* b, int bdt, void* res, int rdt, int64_t n,
                            const AddShape& sh, hipStream_t stream);

// take(a, ids, axis=0) on rows of row_bytes bytes.
hipError_t launch_take(const void* a, int64_t V, int64_t row_bytes, const void* ids,
                       bool ids_signed, int64_t T, void* out, hipStream_t stream);

}  // namespace kh
