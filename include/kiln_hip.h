/*
 * kiln_hip.h — C ABI of the MI355X (gfx950) affine-quantized linear path.
 *
 * Drop-in for the mlx-c entry points Kiln's quantized layers reach:
 *
 *   kh_quantized_matmul     replaces mlx_quantized_matmul, bound at
 *                           crates/kiln-mlx/src/ops.rs:374-385 and wrapped by
 *                           ops::quantized_matmul (ops.rs:359-388); callers
 *                           Linear::forward (crates/kiln-models/src/nn.rs:89)
 *                           and Embedding::as_linear (nn.rs:187).
 *   kh_dequantize           replaces mlx_dequantize, bound at ops.rs:467-480
 *                           (ops::dequantize, ops.rs:456-484).
 *   kh_take                 replaces mlx_take_axis for axis 0, bound at
 *                           ops.rs:250-254 (ops::take).
 *   kh_add                  replaces mlx_add for the bias add of Linear::forward
 *                           (nn.rs:98-100, ops::add): res = a + b, b broadcast
 *                           over a's leading dimensions.
 *   kh_quantized_matmul_multi  the q/k/v projections (nn.rs:724-726) on one x.
 *   kh_quantized_gate_up    silu(gate(x)) * up(x) of the gated MLP (nn.rs:284-294).
 *   kh_quantize             mlx_quantize (mode "affine"), the arithmetic of the
 *                           checkpoint conversion Kiln runs through mlx_lm
 *                           convert (crates/kiln-jobs/src/quantize.rs:72-91).
 *   kh_gather_qmm           replaces mlx_gather_qmm (ops.rs:390-429), the MoE
 *                           expert dispatch (moe.rs:124-176).
 *   kh_quantized_embedding  the fused form of Embedding::lookup
 *                           (nn.rs:159-176): three take(axis=0) calls
 *                           followed by dequantize, in one pass.
 *
 * Conventions (mirroring crates/kiln-mlx/src/error.rs:24-72, array.rs):
 *   - every call returns 0 on success and a non-zero kh_status on error; the
 *     message of the last failing call on the calling thread is returned by
 *     kh_last_error() (thread-local, valid until the next failing call on
 *     that thread). No call aborts the process on bad input.
 *   - arrays are plain descriptors of caller-owned, row-contiguous device
 *     memory. Inputs are borrowed; the result `res` is caller-allocated with
 *     the shape the operation produces (the call checks it) and its dtype
 *     selects the output element type.
 *   - all work is enqueued on the given HIP stream (NULL = the device's null
 *     stream) and is asynchronous; the caller synchronises at its step
 *     boundary, as Kiln does at eval/async_eval (array.rs:460-475).
 *   - a stream is driven from one thread at a time; calls on different
 *     streams may run concurrently.
 *   - device scratch: kernels that need scratch (the GEMM's float16
 *     activations and split-K partials, the gate/up intermediates, the MoE
 *     grouping plan) take it from a workspace kept per (device, stream). The
 *     first call on a stream that needs more than the workspace holds calls
 *     hipMalloc (under stream capture in relaxed capture mode); later calls
 *     of the same or smaller size allocate nothing. A workspace that a graph
 *     capture has used is never freed while the process runs: when it must
 *     grow it is retired (kept allocated) so captured graphs stay valid, and
 *     those buffers are released only at process exit. Callers that must
 *     never allocate use kh_quantized_matmul_noalloc.
 *   - shapes follow MLX: x is [..., K] (leading dims flattened to M), w is
 *     [N, K*bits/32] uint32 with the lowest `bits` bits holding the lowest
 *     column, scales and biases are [N, K/group_size]. mode must be "affine"
 *     (or NULL, meaning "affine").
 */
#ifndef KILN_HIP_H
#define KILN_HIP_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types; the numbering follows mlx_dtype (mlx-c v0.6.0), of which
 * Kiln uses the subset in crates/kiln-mlx/src/array.rs:22-69. */
typedef enum kh_dtype {
  KH_BOOL = 0,
  KH_UINT8 = 1,
  KH_UINT16 = 2,
  KH_UINT32 = 3,
  KH_UINT64 = 4,
  KH_INT8 = 5,
  KH_INT16 = 6,
  KH_INT32 = 7,
  KH_INT64 = 8,
  KH_FLOAT16 = 9,
  KH_FLOAT32 = 10,
  KH_FLOAT64 = 11,
  KH_BFLOAT16 = 12,
  KH_COMPLEX64 = 13
} kh_dtype;

#define KH_MAX_NDIM 8

/* A borrowed view of row-contiguous device memory. */
typedef struct kh_array {
  void* data;                 /* device pointer (HBM); may be NULL iff size 0 */
  int32_t dtype;              /* kh_dtype */
  int32_t ndim;               /* 0 .. KH_MAX_NDIM */
  int64_t shape[KH_MAX_NDIM]; /* row-major, contiguous */
} kh_array;

/* mlx_optional_int: has_value=false selects the MLX default
 * (group_size 64, bits 4). */
typedef struct kh_optional_int {
  int32_t value;
  bool has_value;
} kh_optional_int;

/* Opaque HIP stream handle (hipStream_t). */
typedef void* kh_stream;

typedef enum kh_status {
  KH_OK = 0,
  KH_ERR_INVALID_ARGUMENT = 1, /* shape, dtype, bits/group_size/mode domain */
  KH_ERR_UNSUPPORTED = 2,      /* valid MLX input this library does not run */
  KH_ERR_DEVICE = 3,           /* HIP runtime error (launch, memory) */
  KH_ERR_NO_DEVICE = 4         /* no usable gfx950 device */
} kh_status;

/* res = x @ dequantize(w, scales, biases)^T   (transpose = true)
 * res = x @ dequantize(w, scales, biases)     (transpose = false)
 *
 * transpose=true (every Kiln call site): x [..., K], w [N, K*bits/32],
 * scales/biases [N, K/gs], res [..., N].
 * transpose=false: x [..., K], w [K, N*bits/32], scales/biases [K, N/gs],
 * res [..., N].
 * x: bfloat16 | float16 | float32; scales/biases: bfloat16 | float16 | float32
 * (same dtype for both); res: bfloat16 | float16 | float32. Products are
 * accumulated in float32 and rounded once (round-to-nearest-even) to res.
 * With bf16/f16 x and bf16/f16 scales and transpose=true, the decode kernels
 * (M <= 16, and M <= 32 on shapes the small-batch kernel takes) use every
 * dequantised weight exactly; the GEMM path (larger M; kh_quantized_matmul_plan
 * names the kernel of a call) rounds each weight once to float16 (relative
 * error <= 2^-11) before the float32-accumulating MFMA, with x scaled per row
 * by an exact power of two into float16 range. Other combinations run an exact
 * float32 kernel.
 * bits in {4, 8}; group_size in {32, 64, 128}; K % group_size == 0. */
int kh_quantized_matmul(kh_array* res, const kh_array* x, const kh_array* w,
                        const kh_array* scales, const kh_array* biases,
                        bool transpose, kh_optional_int group_size,
                        kh_optional_int bits, const char* mode,
                        kh_stream stream);

/* res[r, k] = round(fma(f32(scales[r, k/gs]), f32(q[r, k]), f32(biases[r, k/gs])))
 * w [..., R, K*bits/32] -> res [..., R, K]; res dtype bfloat16|float16|float32
 * (MLX's default is the scales dtype, ops.rs:476-479 leaves it unset). */
/* Affine quantization, as mlx_quantize(w, group_size, bits, "affine") of
 * MLX v0.31.1 (Kiln reaches it through mlx_lm convert,
 * crates/kiln-jobs/src/quantize.rs:72-91): w [..., K] float16|bfloat16|float32
 * with K % group_size == 0 -> w_q uint32 [..., K*bits/32] (codes packed
 * lowest bits first), scales and biases [..., K/group_size] of w's dtype.
 * Per group, in float32: s = max((max - min) / (2^bits - 1), 1e-7), negated
 * unless |min| > |max|; edge = the larger-magnitude extreme; q0 = round(edge
 * / s); if q0 != 0, s = edge / q0 and b = edge, else b = 0; code =
 * clamp(round((w - b) / s), 0, 2^bits - 1), rounding half away from zero. */
int kh_quantize(kh_array* w_q, kh_array* scales, kh_array* biases, const kh_array* w,
                kh_optional_int group_size, kh_optional_int bits, const char* mode,
                kh_stream stream);

int kh_dequantize(kh_array* res, const kh_array* w, const kh_array* scales,
                  const kh_array* biases, kh_optional_int group_size,
                  kh_optional_int bits, const char* mode, kh_stream stream);

/* res = take(a, indices, axis=0): rows of a (any dtype, [V, ...]) gathered
 * at indices (uint32 | int32, any shape) -> res [indices.shape..., a.shape[1:]...].
 * Negative int32 indices count from the end (MLX's take). An index outside
 * [-V, V) yields a zero row (HBM is never read out of bounds). */
int kh_take(kh_array* res, const kh_array* a, const kh_array* indices,
            kh_stream stream);

/* Several quantized_matmul calls that share x: res[i] = x @ dequantize(w[i])^T
 * (transpose=true) for i < n, each exactly as kh_quantized_matmul computes it.
 * Replaces the q/k/v projection triple of the attention block
 * (crates/kiln-models/src/nn.rs:724-726: three Linear::forward on one x);
 * with transpose=true, 16-bit x and scales and M within the decode GEMV's
 * range, up to 4 parts run in one launch. */
int kh_quantized_matmul_multi(int n, kh_array* const* res, const kh_array* x,
                              const kh_array* const* w, const kh_array* const* scales,
                              const kh_array* const* biases, bool transpose,
                              kh_optional_int group_size, kh_optional_int bits,
                              const char* mode, kh_stream stream);

/* res = silu(x @ gate^T) * (x @ up^T): the input of the gated MLP's down
 * projection (crates/kiln-models/src/nn.rs:284-294, Activation::Silu), which
 * the reference forms with two quantized_matmul calls, sigmoid and two
 * multiplies. Every intermediate is rounded to res's dtype as those arrays
 * are: gate and up; sigmoid(gate), evaluated in float32; gate*sigmoid; and
 * the final product. Shapes as kh_quantized_matmul with transpose=true; gate
 * and up have equal shapes. One launch where the decode GEMV applies. */
int kh_quantized_gate_up(kh_array* res, const kh_array* x, const kh_array* w_gate,
                         const kh_array* scales_gate, const kh_array* biases_gate,
                         const kh_array* w_up, const kh_array* scales_up,
                         const kh_array* biases_up, kh_optional_int group_size,
                         kh_optional_int bits, const char* mode, kh_stream stream);

/* The gated MLP's activation (Kiln's Activation, crates/kiln-models/src/
 * nn.rs:259-294): silu(gate) for llama/qwen, gelu_approx(gate) for gemma. */
typedef enum kh_activation { KH_ACT_SILU = 0, KH_ACT_GELU_APPROX = 1 } kh_activation;

/* Linear::forward (crates/kiln-models/src/nn.rs:79-102) in one launch:
 * res = quantized_matmul(x, w, scales, biases, transpose=true) [+ bias].
 * bias: NULL, or a float [N] vector (Qwen2's q/k/v, mlp_bias models). The
 * product is an array of MLX's result dtype for (x, scales) (equal dtypes:
 * that dtype; otherwise float32) and the sum is formed in float32 from that
 * rounded product and the bias, then rounded to res, whose dtype must be the
 * dtype of product + bias: bit-identical to kh_quantized_matmul into an array
 * of the product's dtype followed by kh_add. Without a bias this is
 * kh_quantized_matmul with transpose=true. */
int kh_linear(kh_array* res, const kh_array* x, const kh_array* w, const kh_array* scales,
              const kh_array* biases, const kh_array* bias, kh_optional_int group_size,
              kh_optional_int bits, const char* mode, kh_stream stream);

/* n Linear::forward calls on one x (q/k/v, nn.rs:724-726), as
 * kh_quantized_matmul_multi with each part's optional bias (bias may be NULL
 * for no biases at all, or hold NULL entries); each part's result equals
 * kh_linear's. One launch where the decode GEMV applies. */
int kh_linear_multi(int n, kh_array* const* res, const kh_array* x, const kh_array* const* w,
                    const kh_array* const* scales, const kh_array* const* biases,
                    const kh_array* const* bias, kh_optional_int group_size, kh_optional_int bits,
                    const char* mode, kh_stream stream);

/* Mlp::forward's input to down_proj (crates/kiln-models/src/nn.rs:284-294):
 * res = act(gate_proj(x)) * up_proj(x), the projections as kh_linear (with
 * optional biases bias_gate / bias_up), act = silu or gelu_approx
 * (gelu_approx as nn.rs:221-235: 0.5x(1 + tanh(sqrt(2/pi)(x + 0.044715x^3)))
 * with every intermediate rounded to res's dtype as the reference's arrays
 * are; x^3 formed as (x*x)*x in float32). gate and up have equal shapes;
 * with biases res's dtype must be that of kh_linear's result. One launch
 * where the decode GEMV applies; kh_quantized_gate_up is this call with
 * silu and no biases. */
int kh_mlp_gate_up(kh_array* res, const kh_array* x, const kh_array* w_gate,
                   const kh_array* scales_gate, const kh_array* biases_gate,
                   const kh_array* bias_gate, const kh_array* w_up, const kh_array* scales_up,
                   const kh_array* biases_up, const kh_array* bias_up, int activation,
                   kh_optional_int group_size, kh_optional_int bits, const char* mode,
                   kh_stream stream);

/* Quantized gather-matmul over expert stacks (mlx_gather_qmm with null
 * lhs_indices, bound at crates/kiln-mlx/src/ops.rs:390-429; called by
 * SwitchLinear::forward, crates/kiln-models/src/moe.rs:124-176, for the MoE
 * expert dispatch of SwitchGlu, moe.rs:272-310):
 *   batch = broadcast(x.shape[:-2], rhs_indices.shape)     (numpy rules)
 *   res[b] = x[b] @ dequantize(w[e], scales[e], biases[e])^T,  e = rhs_indices[b]
 * x [..., M, K] bfloat16|float16|float32; w [E, N, K*bits/32] uint32;
 * scales/biases [E, N, K/gs]; rhs_indices uint32|int32; res [batch..., M, N].
 * transpose must be true (Kiln's only use). Negative int32 ids count from
 * the end; ids outside [-E, E) give zero rows. sorted_indices is the
 * reference's scheduling hint and does not change results. Small batches
 * run pair by pair with kh_quantized_matmul's decode numerics (exact
 * products). From 64 rows (pairs x M) and 2 rows per possible expert on
 * average, and for every M above the decode range, the rows are grouped by
 * expert on the device and run as one MFMA GEMM: each row then equals
 * kh_quantized_matmul's GEMM path on that row (float16 weights). float32 x
 * or scales take an exact float32 chain. */
int kh_gather_qmm(kh_array* res, const kh_array* x, const kh_array* w, const kh_array* scales,
                  const kh_array* biases, const kh_array* rhs_indices, bool transpose,
                  kh_optional_int group_size, kh_optional_int bits, const char* mode,
                  bool sorted_indices, kh_stream stream);

/* res = dequantize(take(w, ids), take(scales, ids), take(biases, ids)):
 * the quantized embedding lookup. ids uint32|int32 of any shape; w [V, H*bits/32];
 * scales/biases [V, H/gs]; res [ids.shape..., H], bfloat16|float16|float32.
 * Bit-identical to kh_take of the three tensors followed by kh_dequantize;
 * out-of-range ids give zero rows as in kh_take. */
int kh_quantized_embedding(kh_array* res, const kh_array* ids,
                           const kh_array* w, const kh_array* scales,
                           const kh_array* biases, kh_optional_int group_size,
                           kh_optional_int bits, const char* mode,
                           kh_stream stream);

/* res = a + b, elementwise, with numpy broadcasting (dimensions aligned from
 * the right; a dimension of size 1 stretches), as mlx_add. a, b, res:
 * bfloat16|float16|float32; res has the broadcast shape. Each sum is formed in
 * float32 and rounded once to res. */
int kh_add(kh_array* res, const kh_array* a, const kh_array* b, kh_stream stream);

/* kh_quantized_matmul without any device allocation. No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, validation and results (bit for bit) as kh_quantized_matmul.
 * The kernels' scratch (the prefill GEMM's float16 activations, row scales and
 * split-K partials) lives in one static device array per GPU of
 * kh_noalloc_scratch_bytes() bytes (64 MiB), held until the process ends; a
 * call that needs more fails with KH_ERR_UNSUPPORTED before launching
 * anything (e.g. M*K*2 + 4*M plus, with split-K, 4*nsplit*M*N bytes above
 * 64 MiB). Every call on one GPU shares that array: calls that overlap on one
 * GPU (concurrent streams, or threads) race and must be serialised by the
 * caller. Nothing in the array needs clearing between calls. */
int kh_quantized_matmul_noalloc(kh_array* res, const kh_array* x, const kh_array* w,
                                const kh_array* scales, const kh_array* biases,
                                bool transpose, kh_optional_int group_size,
                                kh_optional_int bits, const char* mode, kh_stream stream);

/* Bytes of kh_quantized_matmul_noalloc's per-GPU scratch array. */
size_t kh_noalloc_scratch_bytes(void);

/* Diagnostics, no counterpart in the reference: writes to buf the name of the
 * kernel plan kh_quantized_matmul runs for a transpose=true call of this
 * shape and these dtypes with 16-byte aligned operands ("gemv", "skinny",
 * "gemm mt=.. nsplit=.. tail=..", "qmv", "qmm" or "generic"). For tests and
 * profiling tools that need to know which kernel a shape exercises. */
int kh_quantized_matmul_plan(int64_t M, int64_t N, int64_t K, int group_size, int bits,
                             int x_dtype, int scales_dtype, char* buf, size_t len);

/* Message of the last failing call on this thread ("" if none). */
const char* kh_last_error(void);

/* Library version string. */
const char* kh_version(void);

#ifdef __cplusplus
}
#endif

#endif /* KILN_HIP_H */
