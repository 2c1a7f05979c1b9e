// kh_dequant.hip — dequantize, quantized embedding gather, take, and the
// general quantized matmul for gfx950.
//
// dequantize (crates/kiln-mlx/src/ops.rs:456-484) and the embedding lookup
// (Embedding::lookup, crates/kiln-models/src/nn.rs:159-176: take x3 then
// dequantize) are HBM-bound byte work: one thread expands one packed word
// (8 four-bit or 4 eight-bit codes) with one float32 fma per code, rounds once
// to the output type and writes the values with one vector store.
#include "kh_common.h"
#include "kh_kernels.h"

namespace kh {

namespace {

// Round CPW values to odt and store them at out + base (vector store when
// VEC, which the host selects when the output is suitably aligned).
template <int CPW, bool VEC>
__device__ __forceinline__ void store_codes(void* out, int odt, int64_t base, const float* v) {
  if constexpr (VEC) {
    if (odt == DT_F32) {
      f32x4* o = reinterpret_cast<f32x4*>(static_cast<float*>(out) + base);
#pragma unroll
      for (int c = 0; c < CPW; c += 4) o[c / 4] = f32x4{v[c], v[c + 1], v[c + 2], v[c + 3]};
    } else {
      uint32_t p[CPW / 2];
#pragma unroll
      for (int c = 0; c < CPW; c += 2) p[c / 2] = pack2(v[c], v[c + 1], odt);
      uint16_t* o16 = static_cast<uint16_t*>(out) + base;
      if constexpr (CPW == 8) {
        *reinterpret_cast<u32x4*>(o16) = u32x4{p[0], p[1], p[2], p[3]};
      } else {
        *reinterpret_cast<u32x2*>(o16) = u32x2{p[0], p[1]};
      }
    }
  } else {
#pragma unroll
    for (int c = 0; c < CPW; ++c) store_from_f32(out, odt, base + c, v[c]);
  }
}

template <int BITS>
__device__ __forceinline__ void expand_word(uint32_t u, float sc, float bi, float* v) {
  constexpr int CPW = 32 / BITS;
#pragma unroll
  for (int c = 0; c < CPW; ++c) v[c] = fmaf(sc, (float)((u >> (BITS * c)) & ((1u << BITS) - 1u)), bi);
}

template <int BITS, bool VEC>
__global__ void dequant_kernel(const uint32_t* __restrict__ w, const void* __restrict__ scales,
                               const void* __restrict__ biases, int sdt, void* __restrict__ out,
                               int odt, int64_t R, int64_t K, int gs) {
  constexpr int CPW = 32 / BITS;
  const int64_t WR = K / CPW;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= R * WR) return;
  const int64_t r = i / WR, wi = i % WR;
  const int64_t G = K / gs;
  const int64_t si = r * G + (wi * CPW) / gs;
  float v[CPW];
  expand_word<BITS>(__builtin_nontemporal_load(w + i), load_as_f32(scales, sdt, si),
                    load_as_f32(biases, sdt, si), v);
  store_codes<CPW, VEC>(out, odt, r * K + wi * CPW, v);
}

__device__ __forceinline__ int64_t resolve_id(const void* ids, bool ids_signed, int64_t t,
                                              int64_t V) {
  int64_t id = ids_signed ? (int64_t) static_cast<const int32_t*>(ids)[t]
                          : (int64_t) static_cast<const uint32_t*>(ids)[t];
  if (id < 0) id += V;
  return (id < 0 || id >= V) ? -1 : id;
}

// WPT = 2: a thread expands two consecutive words of a row (one 8-byte load,
// both in one group since gs >= 32 codes) and stores them back to back.
template <int BITS, bool VEC, int WPT>
__global__ void embedding_kernel(const void* __restrict__ ids, int ids_signed, int64_t T,
                                 const uint32_t* __restrict__ w, const void* __restrict__ scales,
                                 const void* __restrict__ biases, int sdt, void* __restrict__ out,
                                 int odt, int64_t V, int64_t H, int gs) {
  constexpr int CPW = 32 / BITS;
  const int64_t WR = H / CPW, UR = WR / WPT;  // words and thread units per row
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= T * UR) return;
  const int64_t t = i / UR, wi = (i % UR) * WPT;
  const int64_t id = resolve_id(ids, ids_signed != 0, t, V);
  float v[WPT][CPW];
  if (id < 0) {
#pragma unroll
    for (int k = 0; k < WPT; ++k)
#pragma unroll
      for (int c = 0; c < CPW; ++c) v[k][c] = 0.f;
  } else {
    const int64_t G = H / gs;
    const int64_t si = id * G + (wi * CPW) / gs;
    const float sc = load_as_f32(scales, sdt, si), bi = load_as_f32(biases, sdt, si);
    if constexpr (WPT == 2) {
      const u32x2 q = *reinterpret_cast<const u32x2*>(w + id * WR + wi);
      expand_word<BITS>(q[0], sc, bi, v[0]);
      expand_word<BITS>(q[1], sc, bi, v[1]);
    } else {
      expand_word<BITS>(w[id * WR + wi], sc, bi, v[0]);
    }
  }
#pragma unroll
  for (int k = 0; k < WPT; ++k) store_codes<CPW, VEC>(out, odt, t * H + (wi + k) * CPW, v[k]);
}

// take on rows of `units` elements of type U.
template <typename U>
__global__ void take_kernel(const U* __restrict__ a, int64_t V, int64_t units,
                            const void* __restrict__ ids, int ids_signed, int64_t T,
                            U* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= T * units) return;
  const int64_t t = i / units, e = i % units;
  const int64_t id = resolve_id(ids, ids_signed != 0, t, V);
  if (id < 0) {
    U z;
    __builtin_memset(&z, 0, sizeof(U));
    out[i] = z;
  } else {
    out[i] = a[id * units + e];
  }
}

// General quantized matmul: one thread per output, acc = fma(x, w, acc) over
// k in increasing order with w = fma(s, q, b) — the same float32 operation
// sequence as the CPU oracle's restatement.
template <int BITS>
__global__ void qmm_generic_kernel(const void* __restrict__ x, int xdt,
                                   const uint32_t* __restrict__ w, const void* __restrict__ scales,
                                   const void* __restrict__ biases, int sdt, void* __restrict__ out,
                                   int odt, int M, int N, int K, int gs, int transpose, Epilogue epi) {
  constexpr int CPW = 32 / BITS;
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  for (int m = blockIdx.y; m < M; m += gridDim.y) {
  float acc = 0.f;
  if (transpose) {
    const int64_t WR = K / CPW, G = K / gs;
    const uint32_t* row = w + (int64_t)n * WR;
    for (int k = 0; k < K; ++k) {
      const float sc = load_as_f32(scales, sdt, (int64_t)n * G + k / gs);
      const float bi = load_as_f32(biases, sdt, (int64_t)n * G + k / gs);
      const float wv = fmaf(sc, (float)((row[k / CPW] >> (BITS * (k % CPW))) & MASK), bi);
      acc = fmaf(load_as_f32(x, xdt, (int64_t)m * K + k), wv, acc);
    }
  } else {
    const int64_t WR = N / CPW, G = N / gs;
    for (int k = 0; k < K; ++k) {
      const float sc = load_as_f32(scales, sdt, (int64_t)k * G + n / gs);
      const float bi = load_as_f32(biases, sdt, (int64_t)k * G + n / gs);
      const uint32_t word = w[(int64_t)k * WR + n / CPW];
      const float wv = fmaf(sc, (float)((word >> (BITS * (n % CPW))) & MASK), bi);
      acc = fmaf(load_as_f32(x, xdt, (int64_t)m * K + k), wv, acc);
    }
  }
  store_from_f32(out, odt, (int64_t)m * N + n, epi(acc, n));
  }
}

__global__ void add_kernel(const void* __restrict__ a, int adt, const void* __restrict__ b, int bdt,
                           void* __restrict__ res, int rdt, int64_t n, int64_t nb) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  store_from_f32(res, rdt, i, load_as_f32(a, adt, i) + load_as_f32(b, bdt, i % nb));
}

// General broadcasting: element i of the result at coordinates over `shape`
// reads a and b through their strides (0 along broadcast dimensions).
__global__ void add_bcast_kernel(const void* __restrict__ a, int adt, const void* __restrict__ b, int bdt,
                                 void* __restrict__ res, int rdt, int64_t n, AddShape sh) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  int64_t ia = 0, ib = 0, rem = i;
  for (int d = sh.nd - 1; d >= 0; --d) {
    const int64_t c = rem % sh.shape[d];
    rem /= sh.shape[d];
    ia += c * sh.as[d];
    ib += c * sh.bs[d];
  }
  store_from_f32(res, rdt, i, load_as_f32(a, adt, ia) + load_as_f32(b, bdt, ib));
}

// gather_qmm, any dtype / alignment / M: one thread per output column n,
// pairs x rows over grid.y; float32 fma chain in k order (as the oracle).
template <int BITS>
__global__ void gather_generic_kernel(const void* __restrict__ x, int xdt, const uint32_t* __restrict__ w,
                                      const void* __restrict__ scales, const void* __restrict__ biases,
                                      int sdt, void* __restrict__ out, int odt, int M, int N, int K,
                                      int gs, GatherArgs g) {
  constexpr int CPW = 32 / BITS;
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const int64_t WR = K / CPW, G = K / gs;
  for (int64_t pm = blockIdx.y; pm < g.pairs * M; pm += gridDim.y) {
    const int64_t pair = pm / M;
    const int m = (int)(pm % M);
    int64_t xo = 0, io = 0, rem = pair;
    for (int d = g.nd - 1; d >= 0; --d) {
      const int64_t c = rem % g.shape[d];
      rem /= g.shape[d];
      xo += c * g.xs[d];
      io += c * g.is[d];
    }
    int64_t e = g.idx_signed ? (int64_t) static_cast<const int32_t*>(g.idx)[io]
                             : (int64_t) static_cast<const uint32_t*>(g.idx)[io];
    if (e < 0) e += g.E;
    float acc = 0.f;
    if (e >= 0 && e < g.E) {
      const int64_t rn = e * N + n;  // row of the flattened [E*N, ...] stack
      const uint32_t* row = w + rn * WR;
      for (int k = 0; k < K; ++k) {
        const float sc = load_as_f32(scales, sdt, rn * G + k / gs);
        const float bi = load_as_f32(biases, sdt, rn * G + k / gs);
        const float wv = fmaf(sc, (float)((row[k / CPW] >> (BITS * (k % CPW))) & MASK), bi);
        acc = fmaf(load_as_f32(x, xdt, xo + (int64_t)m * K + k), wv, acc);
      }
    }
    store_from_f32(out, odt, pm * N + n, acc);
  }
}

__global__ void act_mul_kernel(const void* __restrict__ g, const void* __restrict__ u,
                               void* __restrict__ res, int dt, int64_t n, int act) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  store_from_f32(res, dt, i, act_mul(load_as_f32(g, dt, i), load_as_f32(u, dt, i), dt, act));
}

__global__ void fill_u32_kernel(uint32_t* __restrict__ p, int64_t n, uint32_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// Affine quantization (mlx_quantize, mode "affine"; MLX v0.31.1's rule):
// per group of GS values, in float32,
//   s = max((hi - lo) / nb, 1e-7), negated unless |lo| > |hi|;
//   edge = the larger-magnitude extreme; q0 = round(edge / s);
//   if q0 != 0: s = edge / q0, b = edge, else b = 0;
//   code = min(max(round((w - b) / s), 0), nb)      (round: half away from 0)
// with s and b stored in w's dtype (round to nearest even) and the codes
// computed from the float32 s and b. Lane t takes the 8 values 8t .. 8t+7
// of the flattened rows (one output word at 4 bits, two at 8); the GS/8
// lanes of a group reduce lo and hi by cross-lane exchange, and groups never
// straddle a wave. Division is IEEE (the HIP default) and no product is
// contracted, so results are bit-identical to a sequential float32 evaluation.
template <int BITS, int GS, bool VEC>
__global__ __launch_bounds__(256) void quantize_kernel(const void* __restrict__ w, int wdt,
                                                       uint32_t* __restrict__ wq,
                                                       void* __restrict__ scales,
                                                       void* __restrict__ biases, int64_t blocks) {
#pragma clang fp contract(off)
  constexpr int L = GS / 8;  // lanes per group
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= blocks) return;  // whole groups: blocks is a multiple of L
  const float nb = (float)((1 << BITS) - 1);
  float v[8];
  if (VEC && wdt != DT_F32) {  // 8 values: one 16-byte load
    const u32x4 d = static_cast<const u32x4*>(w)[t];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t h = (d[i / 2] >> (16 * (i % 2))) & 0xffffu;
      v[i] = wdt == DT_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
    }
  } else if (VEC) {  // float32: two 16-byte loads
    const f32x4 a = static_cast<const f32x4*>(w)[2 * t], b = static_cast<const f32x4*>(w)[2 * t + 1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = a[i];
      v[4 + i] = b[i];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = load_as_f32(w, wdt, t * 8 + i);
  }
  float lo = v[0], hi = v[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) {
    lo = fminf(lo, v[i]);
    hi = fmaxf(hi, v[i]);
  }
#pragma unroll
  for (int o = L / 2; o > 0; o >>= 1) {
    lo = fminf(lo, __shfl_xor(lo, o));
    hi = fmaxf(hi, __shfl_xor(hi, o));
  }
  float sc = fmaxf((hi - lo) / nb, 1e-7f);
  const bool side = fabsf(lo) > fabsf(hi);
  sc = side ? sc : -sc;
  const float edge = side ? lo : hi;
  const float q0 = roundf(edge / sc);
  float bi = 0.f;
  if (q0 != 0.f) {
    sc = edge / q0;
    bi = edge;
  }
  if (t % L == 0) {
    store_from_f32(scales, wdt, t / L, sc);
    store_from_f32(biases, wdt, t / L, bi);
  }
  uint32_t word[BITS / 4] = {};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float c = fminf(fmaxf(roundf((v[i] - bi) / sc), 0.f), nb);
    word[i * BITS / 32] |= (uint32_t)c << (BITS * (i % (32 / BITS)));
  }
#pragma unroll
  for (int j = 0; j < BITS / 4; ++j) wq[t * (BITS / 4) + j] = word[j];
}

inline unsigned blocks_for(int64_t n, int threads) { return (unsigned)((n + threads - 1) / threads); }

}  // namespace

hipError_t launch_add(const void* a, int adt, const void* b, int bdt, void* res, int rdt, int64_t n,
                      int64_t nb, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(add_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, stream, a, adt, b, bdt, res,
                     rdt, n, nb);
  return hipGetLastError();
}

hipError_t launch_add_bcast(const void* a, int adt, const void* b, int bdt, void* res, int rdt, int64_t n,
                            const AddShape& sh, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(add_bcast_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, stream, a, adt, b, bdt, res,
                     rdt, n, sh);
  return hipGetLastError();
}

hipError_t launch_fill_u32(void* p, int64_t n, uint32_t value, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(fill_u32_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, stream,
                     static_cast<uint32_t*>(p), n, value);
  return hipGetLastError();
}

hipError_t launch_dequantize(const void* w, const void* scales, const void* biases, int sdt,
                             void* out, int odt, int64_t R, int64_t K, int gs, int bits,
                             hipStream_t stream) {
  const int64_t words = R * (K * bits / 32);
  if (words == 0) return hipSuccess;
  const bool vec = (reinterpret_cast<uintptr_t>(out) % 16) == 0;
  const dim3 grid(blocks_for(words, 256)), block(256);
  const uint32_t* wp = static_cast<const uint32_t*>(w);
  if (bits == 4) {
    if (vec) hipLaunchKernelGGL((dequant_kernel<4, true>), grid, block, 0, stream, wp, scales, biases, sdt, out, odt, R, K, gs);
    else hipLaunchKernelGGL((dequant_kernel<4, false>), grid, block, 0, stream, wp, scales, biases, sdt, out, odt, R, K, gs);
  } else {
    if (vec) hipLaunchKernelGGL((dequant_kernel<8, true>), grid, block, 0, stream, wp, scales, biases, sdt, out, odt, R, K, gs);
    else hipLaunchKernelGGL((dequant_kernel<8, false>), grid, block, 0, stream, wp, scales, biases, sdt, out, odt, R, K, gs);
  }
  return hipGetLastError();
}

hipError_t launch_embedding(const void* ids, bool ids_signed, int64_t T, const void* w,
                            const void* scales, const void* biases, int sdt, void* out, int odt,
                            int64_t V, int64_t H, int gs, int bits, hipStream_t stream) {
  const int64_t words = T * (H * bits / 32);
  if (words == 0) return hipSuccess;
  const bool vec = (reinterpret_cast<uintptr_t>(out) % 16) == 0;
  const uint32_t* wp = static_cast<const uint32_t*>(w);
  const int sg = ids_signed ? 1 : 0;
  const dim3 block(256);
  // two words per thread where rows hold an even number of 8-byte aligned words
  const bool two = vec && ((H * bits / 32) % 2) == 0 && (reinterpret_cast<uintptr_t>(w) % 8) == 0;
#define KH_EMB(B, VC, P)                                                                                 \
  hipLaunchKernelGGL((embedding_kernel<B, VC, P>), dim3(blocks_for(words / P, 256)), block, 0, stream, ids, \
                     sg, T, wp, scales, biases, sdt, out, odt, V, H, gs)
  if (bits == 4) {
    if (two) KH_EMB(4, true, 2); else if (vec) KH_EMB(4, true, 1); else KH_EMB(4, false, 1);
  } else {
    if (two) KH_EMB(8, true, 2); else if (vec) KH_EMB(8, true, 1); else KH_EMB(8, false, 1);
  }
#undef KH_EMB
  return hipGetLastError();
}

hipError_t launch_take(const void* a, int64_t V, int64_t row_bytes, const void* ids,
                       bool ids_signed, int64_t T, void* out, hipStream_t stream) {
  if (T == 0 || row_bytes == 0) return hipSuccess;
  const uintptr_t al = reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(out);
  const int sg = ids_signed ? 1 : 0;
  const dim3 block(256);
  if (row_bytes % 16 == 0 && al % 16 == 0) {
    const int64_t units = row_bytes / 16;
    hipLaunchKernelGGL(take_kernel<u32x4>, dim3(blocks_for(T * units, 256)), block, 0, stream,
                       static_cast<const u32x4*>(a), V, units, ids, sg, T, static_cast<u32x4*>(out));
  } else if (row_bytes % 4 == 0 && al % 4 == 0) {
    const int64_t units = row_bytes / 4;
    hipLaunchKernelGGL(take_kernel<uint32_t>, dim3(blocks_for(T * units, 256)), block, 0, stream,
                       static_cast<const uint32_t*>(a), V, units, ids, sg, T, static_cast<uint32_t*>(out));
  } else {
    hipLaunchKernelGGL(take_kernel<uint8_t>, dim3(blocks_for(T * row_bytes, 256)), block, 0, stream,
                       static_cast<const uint8_t*>(a), V, row_bytes, ids, sg, T, static_cast<uint8_t*>(out));
  }
  return hipGetLastError();
}

hipError_t launch_qmm_generic(const QmvArgs& a, bool transpose) {
  if (a.M == 0 || a.N == 0) return hipSuccess;
  const dim3 grid(blocks_for(a.N, 256), a.M < 65535 ? a.M : 65535), block(256);
  const uint32_t* wp = static_cast<const uint32_t*>(a.w);
  if (a.bits == 4)
    hipLaunchKernelGGL(qmm_generic_kernel<4>, grid, block, 0, a.stream, a.x, a.xdt, wp, a.scales,
                       a.biases, a.sdt, a.out, a.odt, a.M, a.N, a.K, a.gs, transpose ? 1 : 0, a.epi());
  else
    hipLaunchKernelGGL(qmm_generic_kernel<8>, grid, block, 0, a.stream, a.x, a.xdt, wp, a.scales,
                       a.biases, a.sdt, a.out, a.odt, a.M, a.N, a.K, a.gs, transpose ? 1 : 0, a.epi());
  return hipGetLastError();
}

hipError_t launch_act_mul(const void* g, const void* u, void* res, int dt, int64_t n, int act,
                          hipStream_t stream) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(act_mul_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, g, u, res,
                     dt, n, act);
  return hipGetLastError();
}

hipError_t launch_gather_generic(const QmvArgs& a, const GatherArgs& g) {
  const int64_t rows = g.pairs * a.M;
  if (rows == 0 || a.N == 0) return hipSuccess;
  const dim3 block(128), grid((a.N + 127) / 128, (unsigned)(rows < 65535 ? rows : 65535));
  if (a.bits == 4)
    hipLaunchKernelGGL(gather_generic_kernel<4>, grid, block, 0, a.stream, a.x, a.xdt, (const uint32_t*)a.w,
                       a.scales, a.biases, a.sdt, a.out, a.odt, a.M, a.N, a.K, a.gs, g);
  else
    hipLaunchKernelGGL(gather_generic_kernel<8>, grid, block, 0, a.stream, a.x, a.xdt, (const uint32_t*)a.w,
                       a.scales, a.biases, a.sdt, a.out, a.odt, a.M, a.N, a.K, a.gs, g);
  return hipGetLastError();
}

hipError_t launch_quantize(const void* w, int wdt, void* wq, void* scales, void* biases,
                           int64_t rows, int64_t K, int gs, int bits, hipStream_t stream) {
  const int64_t blocks = rows * K / 8;
  if (blocks == 0) return hipSuccess;
  const dim3 grid(blocks_for(blocks, 256)), block(256);
  uint32_t* q = static_cast<uint32_t*>(wq);
  const bool vec = (reinterpret_cast<uintptr_t>(w) & 15) == 0;
#define KH_Q(B, G)                                                                              \
  do {                                                                                          \
    if (vec)                                                                                    \
      hipLaunchKernelGGL((quantize_kernel<B, G, true>), grid, block, 0, stream, w, wdt, q,      \
                         scales, biases, blocks);                                               \
    else                                                                                        \
      hipLaunchKernelGGL((quantize_kernel<B, G, false>), grid, block, 0, stream, w, wdt, q,     \
                         scales, biases, blocks);                                               \
  } while (0)
  if (bits == 4) {
    if (gs == 32) KH_Q(4, 32); else if (gs == 64) KH_Q(4, 64); else KH_Q(4, 128);
  } else {
    if (gs == 32) KH_Q(8, 32); else if (gs == 64) KH_Q(8, 64); else KH_Q(8, 128);
  }
#undef KH_Q
  return hipGetLastError();
}

}  // namespace kh
