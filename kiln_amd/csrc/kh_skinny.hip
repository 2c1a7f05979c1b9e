// kh_skinny.hip — quantized matmul for small batches (5 <= M <= 32) on gfx950.
//
// y[m, n] = sum_k x[m, k] * w[n, k], w = s[n, g(k)] * q[n, k] + b[n, g(k)]
// (quantized_matmul, transpose=true: crates/kiln-mlx/src/ops.rs:359-388).
//
// The weights are streamed once, as in the decode GEMV, but the M rows go
// through the matrix cores, so the cost hardly grows with M.
//
// Numerics: exact products, as the decode GEMV. Codes enter an MFMA as the
// 16-bit values OFF + q built by OR-ing the code into the mantissa of OFF
// (bf16 x: OFF = 128, f16 x: OFF = 1024; exact), against x in its own dtype,
// accumulating in float32. Each MFMA step is restricted to one quantization
// group by zeroing the A-operand lanes of the other groups, and a second MFMA
// against ones gives the group sums X of x. Per group and piece:
//   acc += s * P + (b - OFF * s) * X,   P = sum x * (OFF + q).
// 8-bit codes with bf16 x, where OFF + q is not exact beyond q = 127, enter
// as two nibble operands: P = P_lo + 16 * P_hi with OFF_eff = 17 * 128.
//
// Work decomposition: a workgroup of W <= 8 waves owns 16 * NTW weight rows
// and all M rows of x (one or two 16-row m-tiles);
// the waves split K into 128-code pieces (wave w takes pieces w*ppw ..
// (w+1)*ppw - 1). Within a piece, lane (n = l % 16, kb = l / 16) of a 16-row
// tile loads the 32 codes kb*32 .. kb*32+31 of row n (16 or 32 bytes) and the
// matching 32 values of x row l % 16; MFMA step j (0..3) takes the lane's
// 8 codes 8j .. 8j+7. The loads of the next piece are in flight while a
// piece computes. The W partial tiles are summed through LDS in wave order.
#include <type_traits>

#include "kh_common.h"
#include "kh_kernels.h"

namespace kh {

namespace {

constexpr int kSkMaxWaves = 8;
constexpr int kPiece = 128;  // codes per piece

template <bool XBF16>
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (XBF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

template <int BITS, int NTW, int MT>
struct Piece {
  u32x4 q[NTW][BITS / 4];  // the lane's 32 codes per tile
  u32x4 x[MT][4];          // x[m, run .. run+31] per 16-row m-tile
};

template <int BITS, bool XBF16, bool SBF16, int GS, int NTW, int MT>
__global__ __launch_bounds__(64 * kSkMaxWaves) void skinny_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ w,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    void* __restrict__ out, int odt, int M, int N, int K, int ppw, Epilogue epi) {
  constexpr int GP = kPiece / GS;               // groups per piece
  constexpr bool SPLIT = XBF16 && BITS == 8;    // 8-bit codes as two nibble operands
  constexpr uint32_t MAG = XBF16 ? 0x43004300u : 0x64006400u;   // OFF in both halves
  constexpr uint32_t ONE = XBF16 ? 0x3F803F80u : 0x3C003C00u;   // 1.0 in both halves
  constexpr float OFF = SPLIT ? 17.f * 128.f : (XBF16 ? 128.f : 1024.f);
  using P_t = Piece<BITS, NTW, MT>;
  constexpr int ROWS = 16 * NTW;

  // LDS: the scales and biases of the workgroup's rows for all of K
  // ([2][ROWS][G] 16-bit values, loaded once), then the partial tiles of the
  // cross-wave sum ([W][MT][NTW][4][64] floats).
  extern __shared__ __align__(16) unsigned char smem[];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, W = blockDim.x >> 6;
  const int col = lane & 15, kb = lane >> 4;
  const int n0 = blockIdx.x * 16 * NTW;
  const int G = K / GS;
  const int wpr = K * BITS / 32;
  const int gl = (kb * 32) / GS;  // group of this lane's run within a piece

  int nrow[NTW];
#pragma unroll
  for (int t = 0; t < NTW; ++t) nrow[t] = min(n0 + t * 16 + col, N - 1);
  bool mval[MT];
  const u32x4* xr[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    mval[mt] = mt * 16 + col < M;
    xr[mt] = reinterpret_cast<const u32x4*>(x + (int64_t)min(mt * 16 + col, M - 1) * K);
  }

  uint16_t* sbl = reinterpret_cast<uint16_t*>(smem);
  float* red = reinterpret_cast<float*>(smem + (size_t)2 * ROWS * G * 2);

  auto load = [&](P_t& P, int piece) {
    const int run = piece * kPiece + kb * 32;  // first code of the lane's run
#pragma unroll
    for (int t = 0; t < NTW; ++t) {
      const u32x4* src = reinterpret_cast<const u32x4*>(w + (int64_t)nrow[t] * wpr + run * BITS / 32);
#pragma unroll
      for (int h = 0; h < BITS / 4; ++h) P.q[t][h] = __builtin_nontemporal_load(src + h);
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j) P.x[mt][j] = xr[mt][(run >> 3) + j];  // row min(m, M-1)
  };

  f32x4 acc[MT][NTW];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < NTW; ++t) acc[mt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const u32x4 ones = u32x4{ONE, ONE, ONE, ONE};

  auto compute = [&](const P_t& P, int piece) {
    f32x4 pa[MT][NTW][GP], pb[MT][NTW][GP], xs[MT][GP];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int g = 0; g < GP; ++g) {
        xs[mt][g] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < NTW; ++t) pa[mt][t][g] = pb[mt][t][g] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // the code operands of step j, per tile
      u32x4 lo[NTW], hi[NTW];
#pragma unroll
      for (int t = 0; t < NTW; ++t) {
        const uint32_t w0 = BITS == 4 ? P.q[t][0][j] : P.q[t][j >> 1][(j & 1) * 2];
        const uint32_t w1 = BITS == 4 ? 0u : P.q[t][j >> 1][(j & 1) * 2 + 1];
        if constexpr (BITS == 4) {
#pragma unroll
          for (int e = 0; e < 4; ++e) lo[t][e] = ((w0 >> (4 * e)) & 0x000f000fu) | MAG;
        } else {
          const uint32_t r[4] = {w0 & 0x00ff00ffu, (w0 >> 8) & 0x00ff00ffu, w1 & 0x00ff00ffu,
                                 (w1 >> 8) & 0x00ff00ffu};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if constexpr (SPLIT) {
              lo[t][e] = (r[e] & 0x000f000fu) | MAG;
              hi[t][e] = ((r[e] >> 4) & 0x000f000fu) | MAG;
            } else {
              lo[t][e] = r[e] | MAG;
            }
          }
        }
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const u32x4 a = mval[mt] ? permute_x<BITS>(P.x[mt][j]) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int g = 0; g < GP; ++g) {
          const u32x4 ag = (GP == 1 || gl == g) ? a : u32x4{0u, 0u, 0u, 0u};
          xs[mt][g] = mfma16<XBF16>(ag, ones, xs[mt][g]);
#pragma unroll
          for (int t = 0; t < NTW; ++t) {
            pa[mt][t][g] = mfma16<XBF16>(ag, lo[t], pa[mt][t][g]);
            if constexpr (SPLIT) pb[mt][t][g] = mfma16<XBF16>(ag, hi[t], pb[mt][t][g]);
          }
        }
      }
    }
    // acc += s * P + (b - OFF * s) * X per group, columns n = lane % 16
#pragma unroll
    for (int t = 0; t < NTW; ++t)
#pragma unroll
      for (int g = 0; g < GP; ++g) {
        const int si = (t * 16 + col) * G + piece * GP + g;
        const float s = SBF16 ? bf16_bits_to_f32(sbl[si]) : f16_bits_to_f32(sbl[si]);
        const float b = SBF16 ? bf16_bits_to_f32(sbl[ROWS * G + si]) : f16_bits_to_f32(sbl[ROWS * G + si]);
        const float c = b - OFF * s;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float p = SPLIT ? pa[mt][t][g][e] + 16.f * pb[mt][t][g][e] : pa[mt][t][g][e];
            acc[mt][t][e] += s * p + c * xs[mt][g][e];
          }
      }
  };

  P_t A, B;
  const int p0 = wave * ppw;
  load(A, p0);
  // the rows' scales and biases (rows n0 .. n0+ROWS-1 are consecutive, so
  // each array is one contiguous run; rows past N are not loaded and their
  // outputs are never stored)
  {
    const int nr = min(ROWS, N - n0);
    const int64_t cnt = (int64_t)nr * G;
    const uint16_t* src[2] = {scales + (int64_t)n0 * G, biases + (int64_t)n0 * G};
    if ((G & 7) == 0) {
      for (int64_t i = threadIdx.x; i < 2 * cnt / 8; i += blockDim.x) {
        const int a = i >= cnt / 8;
        const int64_t j = i - a * (cnt / 8);
        reinterpret_cast<u32x4*>(sbl + a * ROWS * G)[j] = reinterpret_cast<const u32x4*>(src[a])[j];
      }
    } else {
      for (int64_t i = threadIdx.x; i < 2 * cnt; i += blockDim.x) {
        const int a = i >= cnt;
        const int64_t j = i - a * cnt;
        sbl[a * ROWS * G + j] = src[a][j];
      }
    }
  }
  __syncthreads();
  for (int i = 0; i < ppw; i += 2) {
    if (i + 1 < ppw) load(B, p0 + i + 1);
    compute(A, p0 + i);
    if (i + 1 >= ppw) break;
    if (i + 2 < ppw) load(A, p0 + i + 2);
    compute(B, p0 + i + 1);
  }

  // Sum the W partial tiles in wave order. D lane l holds rows 4*(l/16)+e,
  // column l%16 of each 16x16 tile.
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < NTW; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        red[(((wave * MT + mt) * NTW + t) * 4 + e) * 64 + lane] = acc[mt][t][e];
  __syncthreads();
  for (int i = threadIdx.x; i < MT * NTW * 256; i += blockDim.x) {
    const int l = i & 63, e = (i >> 6) & 3, t = (i >> 8) % NTW, mt = (i >> 8) / NTW;
    const int m = mt * 16 + 4 * (l >> 4) + e, n = n0 + t * 16 + (l & 15);
    if (m >= M || n >= N) continue;
    const int base = ((mt * NTW + t) * 4 + e) * 64 + l, stride = MT * NTW * 256;
    float v = red[base];
    for (int ww = 1; ww < W; ++ww) v += red[base + ww * stride];
    store_from_f32(out, odt, (int64_t)m * N + n, epi(v, n));
  }
}

struct SkinnyPlan {
  int W, ppw, ntw, mt;
};

// Most 16-row tiles per wave that fit the registers (from the compiler's
// register counts: larger tilings spill).
constexpr int max_ntw(int bits, int gs, int mt) {
  return mt == 1 ? (bits == 4 ? (gs == 128 ? 4 : 2) : (gs == 32 ? 1 : 2))
                 : (bits == 4 && gs == 128 ? 2 : 1);
}

// W and the pieces per wave depend on K only, so a row's summation order
// is the same for every M this kernel serves.
SkinnyPlan plan_skinny(int M, int N, int K, int bits, int gs) {
  const int np = K / kPiece;
  int W = kSkMaxWaves;
  while (np % W) --W;
  SkinnyPlan p{W, np / W, 1, M > 16 ? 2 : 1};
  // as many rows per workgroup as keeps the launch at >= 2048 waves
  const int mx = max_ntw(bits, gs, p.mt);
  if (mx >= 4 && (int64_t)((N + 63) / 64) * W >= 2048) p.ntw = 4;
  else if (mx >= 2 && (int64_t)((N + 31) / 32) * W >= 2048) p.ntw = 2;
  return p;
}

// LDS of one workgroup: scales and biases of its rows, then the partial tiles.
size_t skinny_lds(const SkinnyPlan& p, int64_t K, int gs) {
  return (size_t)2 * 16 * p.ntw * (K / gs) * 2 + (size_t)p.W * p.mt * p.ntw * 4 * 64 * sizeof(float);
}
constexpr size_t kSkMaxLds = 96 * 1024;
constexpr int64_t kSkMaxWavesMt2 = 3 * 4 * 256;  // three waves per SIMD on 256 CUs  // keeps at least one workgroup per CU with room to spare

template <int BITS, bool XBF16, bool SBF16, int GS, int NTW, int MT>
hipError_t launch_t(const QmvArgs& a, const SkinnyPlan& p) {
  const int wgs = (a.N + 16 * NTW - 1) / (16 * NTW);
  const size_t lds = skinny_lds(p, a.K, GS);
  hipLaunchKernelGGL((skinny_kernel<BITS, XBF16, SBF16, GS, NTW, MT>), dim3(wgs), dim3(64 * p.W), lds,
                     a.stream, (const uint16_t*)a.x, (const uint32_t*)a.w,
                     (const uint16_t*)a.scales, (const uint16_t*)a.biases, a.out, a.odt, a.M, a.N,
                     a.K, p.ppw, a.epi());
  return hipGetLastError();
}

template <int BITS, bool XBF16, bool SBF16, int GS, int MT>
hipError_t launch_m(const QmvArgs& a, const SkinnyPlan& p) {
  if constexpr (max_ntw(BITS, GS, MT) >= 4)
    if (p.ntw == 4) return launch_t<BITS, XBF16, SBF16, GS, 4, MT>(a, p);
  if constexpr (max_ntw(BITS, GS, MT) >= 2)
    if (p.ntw == 2) return launch_t<BITS, XBF16, SBF16, GS, 2, MT>(a, p);
  return launch_t<BITS, XBF16, SBF16, GS, 1, MT>(a, p);
}

template <int BITS, bool XBF16, bool SBF16, int GS>
hipError_t launch_n(const QmvArgs& a, const SkinnyPlan& p) {
  return p.mt == 2 ? launch_m<BITS, XBF16, SBF16, GS, 2>(a, p) : launch_m<BITS, XBF16, SBF16, GS, 1>(a, p);
}

template <int BITS, bool XBF16, bool SBF16>
hipError_t launch_g(const QmvArgs& a, const SkinnyPlan& p) {
  if (a.gs == 32) return launch_n<BITS, XBF16, SBF16, 32>(a, p);
  if (a.gs == 64) return launch_n<BITS, XBF16, SBF16, 64>(a, p);
  return launch_n<BITS, XBF16, SBF16, 128>(a, p);
}

template <int BITS>
hipError_t launch_b(const QmvArgs& a, const SkinnyPlan& p) {
  const bool xb = a.xdt == DT_BF16, sb = a.sdt == DT_BF16;
  if (xb) return sb ? launch_g<BITS, true, true>(a, p) : launch_g<BITS, true, false>(a, p);
  return sb ? launch_g<BITS, false, true>(a, p) : launch_g<BITS, false, false>(a, p);
}

}  // namespace

int64_t skinny_waves(int64_t N, int64_t K) {
  const int np = (int)(K / kPiece);
  int W = kSkMaxWaves;
  while (W > 1 && np % W) --W;
  return (N + 15) / 16 * W;
}

bool skinny_supported(int64_t M, int64_t N, int64_t K, int bits, int gs) {
  const int64_t lim = (int64_t)1 << 31;
  if (!(M >= 1 && M <= kSkinnyMaxM && K % kPiece == 0 && N >= 1 && N * K * bits / 8 < lim &&
        M * K * 2 < lim && N * (K / gs) * 2 < lim))
    return false;
  const SkinnyPlan p = plan_skinny((int)M, (int)N, (int)K, bits, gs);
  // Two m-tiles take ~140-170 registers: three waves per SIMD. Beyond one
  // round of resident waves the GEMM is faster (measured), so M > 16 uses
  // this kernel only where ceil(N/16) * W waves fit (a rule on N and K only).
  if (M > 16 && (int64_t)((N + 15) / 16) * p.W > kSkMaxWavesMt2) return false;
  return skinny_lds(p, K, gs) <= kSkMaxLds;
}

hipError_t launch_skinny(const QmvArgs& a) {
  if (!skinny_supported(a.M, a.N, a.K, a.bits, a.gs)) return hipErrorInvalidValue;
  const SkinnyPlan p = plan_skinny(a.M, a.N, a.K, a.bits, a.gs);
  return a.bits == 4 ? launch_b<4>(a, p) : launch_b<8>(a, p);
}

}  // namespace kh
