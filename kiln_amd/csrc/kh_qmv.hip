// kh_qmv.hip — decode / small-batch quantized GEMV for gfx950 (M <= 64).
//
// Computes y[m, n] = sum_k x[m, k] * (s[n, g(k)] * q[n, k] + b[n, g(k)])
// (the transpose=true form of quantized_matmul, crates/kiln-mlx/src/ops.rs:359-388,
// used by Linear::forward nn.rs:89 and Embedding::as_linear nn.rs:187).
//
// The affine dequantisation is factored per group g so that no dequantised
// weight is ever rounded:
//   y[m, n] = sum_g  s[n,g] * P'[m,n,g] + (b[n,g] - OFF*s[n,g]) * X[m,g]
//   P'[m,n,g] = sum_{k in g} x[m,k] * (OFF + q[n,k])      (MFMA, fp32 accumulate)
//   X[m,g]    = sum_{k in g} x[m,k]                        (MFMA against ones)
// OFF + q is exactly representable in the MFMA input type: it is built by
// OR-ing the code into the mantissa of OFF (bf16: OFF = 128, 7-bit mantissa;
// f16: OFF = 1024, 10-bit mantissa), except 8-bit codes with bf16 activations,
// which go through an exact int->float conversion with OFF = 0.
//
// Work decomposition: one workgroup owns 16 output rows (one MFMA column
// tile) and all M <= 64 activation rows (MT m-tiles of 16). Its NWK waves
// split the K groups into contiguous ranges and reduce their fp32 partials
// through LDS in fixed wave order, so every output's summation order depends
// only on (N, K, group_size, bits) — never on M or on scheduling.
//
// MFMA v_mfma_f32_16x16x32_{bf16,f16}: A = activations (16 m x 32 k),
// B = codes (32 k x 16 n). Lane l supplies row/column l%16 and the eight k of
// block l/16; D lane l holds column l%16, rows 4*(l/16)+0..3. Per step the
// four lane groups read four different words of the same group, so a group
// (gs/32 steps) is reduced inside one accumulator chain.
#include "kh_common.h"
#include "kh_kernels.h"

namespace kh {

// Pair order of the B operand built from packed codes; the activations are
// permuted to match. 4-bit word -> (c0,c4)(c1,c5)(c2,c6)(c3,c7);
// 8-bit word pair -> (c0,c2)(c1,c3)(c4,c6)(c5,c7).
template <int BITS>
__device__ __forceinline__ u32x4 permute_x(u32x4 d) {
  u32x4 r;
  if constexpr (BITS == 4) {
    r[0] = perm(d[2], d[0], 0x05040100u);
    r[1] = perm(d[2], d[0], 0x07060302u);
    r[2] = perm(d[3], d[1], 0x05040100u);
    r[3] = perm(d[3], d[1], 0x07060302u);
  } else {
    r[0] = perm(d[1], d[0], 0x05040100u);
    r[1] = perm(d[1], d[0], 0x07060302u);
    r[2] = perm(d[3], d[2], 0x05040100u);
    r[3] = perm(d[3], d[2], 0x07060302u);
  }
  return r;
}

template <bool XBF16>
struct MagicT;
template <>
struct MagicT<true> {  // bf16: 0x4300 = 128.0
  static constexpr uint32_t magic = 0x43004300u;
  static constexpr uint32_t ones = 0x3f803f80u;
};
template <>
struct MagicT<false> {  // f16: 0x6400 = 1024.0
  static constexpr uint32_t magic = 0x64006400u;
  static constexpr uint32_t ones = 0x3c003c00u;
};

template <int BITS, bool XBF16>
struct CodeOffset {
  static constexpr float value = (BITS == 8 && XBF16) ? 0.0f : (XBF16 ? 128.0f : 1024.0f);
};

// Eight codes (one 4-bit word, or two 8-bit words) -> B operand, values OFF + q.
template <int BITS, bool XBF16>
__device__ __forceinline__ u32x4 codes_to_b(const uint32_t* q) {
  u32x4 r;
  constexpr uint32_t MAG = MagicT<XBF16>::magic;
  if constexpr (BITS == 4) {
    const uint32_t u = q[0];
    r[0] = (u & 0x000f000fu) | MAG;
    r[1] = ((u >> 4) & 0x000f000fu) | MAG;
    r[2] = ((u >> 8) & 0x000f000fu) | MAG;
    r[3] = ((u >> 12) & 0x000f000fu) | MAG;
  } else if constexpr (!XBF16) {
    r[0] = (q[0] & 0x00ff00ffu) | MAG;
    r[1] = ((q[0] >> 8) & 0x00ff00ffu) | MAG;
    r[2] = (q[1] & 0x00ff00ffu) | MAG;
    r[3] = ((q[1] >> 8) & 0x00ff00ffu) | MAG;
  } else {
    // Integer codes 0..255 are exact in bf16: the bf16 value is the upper
    // half of the float32 bits.
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t u = q[h];
      const uint32_t f0 = __float_as_uint((float)(u & 0xffu));
      const uint32_t f1 = __float_as_uint((float)((u >> 8) & 0xffu));
      const uint32_t f2 = __float_as_uint((float)((u >> 16) & 0xffu));
      const uint32_t f3 = __float_as_uint((float)(u >> 24));
      r[2 * h + 0] = perm(f2, f0, 0x07060302u);
      r[2 * h + 1] = perm(f3, f1, 0x07060302u);
    }
  }
  return r;
}

template <bool XBF16>
__device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (XBF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

constexpr int QMV_MAX_WAVES = 16;

template <int BITS, int GS, bool XBF16, int MT>
__global__ __launch_bounds__(1024) void qmv_kernel(const uint16_t* __restrict__ x,
                                                   const uint32_t* __restrict__ w,
                                                   const void* __restrict__ scales,
                                                   const void* __restrict__ biases, int sdt,
                                                   void* __restrict__ out, int odt, int M, int N,
                                                   int K) {
  constexpr int CPW = 32 / BITS;   // codes per word
  constexpr int S = GS / 32;       // MFMA k-steps per group
  constexpr int WPS = 8 / CPW;     // words per lane per step
  constexpr int LW = S * WPS;      // words per lane per group
  constexpr int WPG = GS / CPW;    // words per group per row (= 4 * LW)
  constexpr float OFF = CodeOffset<BITS, XBF16>::value;

  __shared__ f32x4 red[QMV_MAX_WAVES * MT * 64];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwk = blockDim.x >> 6;
  const int col = lane & 15;
  const int lg = lane >> 4;
  const int n = blockIdx.x * 16 + col;
  const bool nvalid = n < N;
  const int G = K / GS;
  const int64_t WR = K / CPW;
  const int g0 = (int)((int64_t)G * wave / nwk);
  const int g1 = (int)((int64_t)G * (wave + 1) / nwk);

  const uint32_t* wrow = w + (int64_t)(nvalid ? n : 0) * WR + lg * LW;
  const int64_t sbase = (int64_t)(nvalid ? n : 0) * G;

  u32x4 ones;
  ones[0] = ones[1] = ones[2] = ones[3] = MagicT<XBF16>::ones;

  f32x4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int g = g0; g < g1; ++g) {
    uint32_t q[LW];
    if (nvalid) {
      const uint32_t* src = wrow + (int64_t)g * WPG;
      if constexpr (LW == 1) {
        q[0] = __builtin_nontemporal_load(src);
      } else if constexpr (LW == 2) {
        u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(src));
        q[0] = v[0];
        q[1] = v[1];
      } else {
#pragma unroll
        for (int i = 0; i < LW; i += 4) {
          u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + i));
          q[i] = v[0];
          q[i + 1] = v[1];
          q[i + 2] = v[2];
          q[i + 3] = v[3];
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < LW; ++i) q[i] = 0;
    }
    float sc = 0.f, bp = 0.f;
    if (nvalid) {
      sc = load_as_f32(scales, sdt, sbase + g);
      bp = fmaf(-OFF, sc, load_as_f32(biases, sdt, sbase + g));
    }

    f32x4 P[MT], X[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      P[t] = f32x4{0.f, 0.f, 0.f, 0.f};
      X[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int j = 0; j < S; ++j) {
      const u32x4 b = codes_to_b<BITS, XBF16>(q + j * WPS);
      const int64_t kx = (int64_t)g * GS + 8 * (lg * S + j);
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const int m = t * 16 + col;
        u32x4 a = u32x4{0u, 0u, 0u, 0u};
        if (m < M) a = permute_x<BITS>(*reinterpret_cast<const u32x4*>(x + (int64_t)m * K + kx));
        P[t] = mfma<XBF16>(a, b, P[t]);
        X[t] = mfma<XBF16>(a, ones, X[t]);
      }
    }
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[t][i] = fmaf(sc, P[t][i], acc[t][i]);
        acc[t][i] = fmaf(bp, X[t][i], acc[t][i]);
      }
  }

  if (nwk > 1) {
#pragma unroll
    for (int t = 0; t < MT; ++t) red[(wave * MT + t) * 64 + lane] = acc[t];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      f32x4 s = red[t * 64 + lane];
      for (int v = 1; v < nwk; ++v) {
        const f32x4 o = red[(v * MT + t) * 64 + lane];
        s[0] += o[0];
        s[1] += o[1];
        s[2] += o[2];
        s[3] += o[3];
      }
      acc[t] = s;
    }
  }
  if (!nvalid) return;
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = t * 16 + 4 * lg + i;
      if (m < M) store_from_f32(out, odt, (int64_t)m * N + n, acc[t][i]);
    }
}

// Waves per workgroup: enough waves in flight to cover the chip, at least two
// groups per wave. Depends only on (N, K, group_size) so that the summation
// order of an output row is the same for every M.
int qmv_waves(int N, int K, int gs) {
  const int tiles = (N + 15) / 16;
  const int G = K / gs;
  int nwk = 1;
  while (nwk < QMV_MAX_WAVES && tiles * nwk < 8192 && G / (nwk * 2) >= 2) nwk *= 2;
  return nwk;
}

template <int BITS, int GS, bool XBF16>
static hipError_t launch_mt(const QmvArgs& a, int nwk) {
  const dim3 grid((a.N + 15) / 16), block(64 * nwk);
  const int mt = (a.M + 15) / 16;
#define KH_QMV_LAUNCH(MTV)                                                                        \
  hipLaunchKernelGGL((qmv_kernel<BITS, GS, XBF16, MTV>), grid, block, 0, a.stream,                \
                     (const uint16_t*)a.x, (const uint32_t*)a.w, a.scales, a.biases, a.sdt, a.out, \
                     a.odt, a.M, a.N, a.K)
  switch (mt) {
    case 1: KH_QMV_LAUNCH(1); break;
    case 2: KH_QMV_LAUNCH(2); break;
    case 3: KH_QMV_LAUNCH(3); break;
    default: KH_QMV_LAUNCH(4); break;
  }
#undef KH_QMV_LAUNCH
  return hipGetLastError();
}

template <int BITS, bool XBF16>
static hipError_t launch_gs(const QmvArgs& a, int nwk) {
  switch (a.gs) {
    case 32: return launch_mt<BITS, 32, XBF16>(a, nwk);
    case 64: return launch_mt<BITS, 64, XBF16>(a, nwk);
    default: return launch_mt<BITS, 128, XBF16>(a, nwk);
  }
}

hipError_t launch_qmv(const QmvArgs& a) {
  const int nwk = qmv_waves(a.N, a.K, a.gs);
  const bool xbf16 = a.xdt == DT_BF16;
  if (a.bits == 4) return xbf16 ? launch_gs<4, true>(a, nwk) : launch_gs<4, false>(a, nwk);
  return xbf16 ? launch_gs<8, true>(a, nwk) : launch_gs<8, false>(a, nwk);
}

}  // namespace kh
