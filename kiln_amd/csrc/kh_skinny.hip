// kh_skinny.hip — quantized matmul for small batches (5 <= M <= 16) on gfx950.
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
// Work decomposition: a workgroup of W <= 8 waves owns 16 * NTW weight rows;
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

template <int BITS, int NTW>
struct Piece {
  u32x4 q[NTW][BITS / 4];  // the lane's 32 codes per tile
  u32x4 x[4];              // x[m, run .. run+31]
};

template <int BITS, bool XBF16, bool SBF16, int GS, int NTW>
__global__ __launch_bounds__(64 * kSkMaxWaves) void skinny_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ w,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    void* __restrict__ out, int odt, int M, int N, int K, int ppw) {
  constexpr int GP = kPiece / GS;               // groups per piece
  constexpr bool SPLIT = XBF16 && BITS == 8;    // 8-bit codes as two nibble operands
  constexpr uint32_t MAG = XBF16 ? 0x43004300u : 0x64006400u;   // OFF in both halves
  constexpr uint32_t ONE = XBF16 ? 0x3F803F80u : 0x3C003C00u;   // 1.0 in both halves
  constexpr float OFF = SPLIT ? 17.f * 128.f : (XBF16 ? 128.f : 1024.f);
  using P_t = Piece<BITS, NTW>;
  constexpr int ROWS = 16 * NTW;

  // LDS: the scales and biases of the workgroup's rows for all of K
  // ([2][ROWS][G] 16-bit values, loaded once), then the partial tiles of the
  // cross-wave sum ([W][NTW][4][64] floats).
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
  const bool mval = col < M;
  const u32x4* xr = reinterpret_cast<const u32x4*>(x + (int64_t)min(col, M - 1) * K);

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
    for (int j = 0; j < 4; ++j) P.x[j] = xr[(run >> 3) + j];  // row min(col, M-1)
  };

  f32x4 acc[NTW];
#pragma unroll
  for (int t = 0; t < NTW; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const u32x4 ones = u32x4{ONE, ONE, ONE, ONE};

  auto compute = [&](const P_t& P, int piece) {
    f32x4 pa[NTW][GP], pb[NTW][GP], xs[GP];
#pragma unroll
    for (int g = 0; g < GP; ++g) {
      xs[g] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < NTW; ++t) pa[t][g] = pb[t][g] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u32x4 a = mval ? permute_x<BITS>(P.x[j]) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int g = 0; g < GP; ++g) {
        const u32x4 ag = (GP == 1 || gl == g) ? a : u32x4{0u, 0u, 0u, 0u};
        xs[g] = mfma16<XBF16>(ag, ones, xs[g]);
#pragma unroll
        for (int t = 0; t < NTW; ++t) {
          const uint32_t w0 = BITS == 4 ? P.q[t][0][j] : P.q[t][j >> 1][(j & 1) * 2];
          const uint32_t w1 = BITS == 4 ? 0u : P.q[t][j >> 1][(j & 1) * 2 + 1];
          u32x4 lo, hi;
          if constexpr (BITS == 4) {
#pragma unroll
            for (int e = 0; e < 4; ++e) lo[e] = ((w0 >> (4 * e)) & 0x000f000fu) | MAG;
          } else {
            const uint32_t r[4] = {w0 & 0x00ff00ffu, (w0 >> 8) & 0x00ff00ffu, w1 & 0x00ff00ffu,
                                   (w1 >> 8) & 0x00ff00ffu};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              if constexpr (SPLIT) {
                lo[e] = (r[e] & 0x000f000fu) | MAG;
                hi[e] = ((r[e] >> 4) & 0x000f000fu) | MAG;
              } else {
                lo[e] = r[e] | MAG;
              }
            }
          }
          pa[t][g] = mfma16<XBF16>(ag, lo, pa[t][g]);
          if constexpr (SPLIT) pb[t][g] = mfma16<XBF16>(ag, hi, pb[t][g]);
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
        for (int e = 0; e < 4; ++e) {
          const float p = SPLIT ? pa[t][g][e] + 16.f * pb[t][g][e] : pa[t][g][e];
          acc[t][e] += s * p + c * xs[g][e];
        }
      }
  };

  // Two pieces in flight: the loads of piece i+1 are issued before the
  // arithmetic of piece i (a deeper ring measured slower: its registers cost
  // more resident waves than it hides).
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
  for (int t = 0; t < NTW; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) red[((wave * NTW + t) * 4 + e) * 64 + lane] = acc[t][e];
  __syncthreads();
  for (int i = threadIdx.x; i < NTW * 256; i += blockDim.x) {
    const int l = i & 63, e = (i >> 6) & 3, t = i >> 8;
    const int m = 4 * (l >> 4) + e, n = n0 + t * 16 + (l & 15);
    if (m >= M || n >= N) continue;
    float v = red[((0 * NTW + t) * 4 + e) * 64 + l];
    for (int ww = 1; ww < W; ++ww) v += red[((ww * NTW + t) * 4 + e) * 64 + l];
    store_from_f32(out, odt, (int64_t)m * N + n, v);
  }
}

struct SkinnyPlan {
  int W, ppw, ntw;
};

// Most 16-row tiles per wave that fit the registers (from the compiler's
// register counts: larger tilings spill).
constexpr int max_ntw(int bits, int gs) {
  return bits == 4 ? (gs == 128 ? 4 : 2) : (gs == 32 ? 1 : 2);
}

SkinnyPlan plan_skinny(int N, int K, int bits, int gs) {
  const int np = K / kPiece;
  int W = kSkMaxWaves;
  while (np % W) --W;
  SkinnyPlan p{W, np / W, 1};
  // as many rows per workgroup as keeps the launch at >= 2048 waves
  if (max_ntw(bits, gs) >= 4 && (int64_t)((N + 63) / 64) * W >= 2048) p.ntw = 4;
  else if (max_ntw(bits, gs) >= 2 && (int64_t)((N + 31) / 32) * W >= 2048) p.ntw = 2;
  return p;
}

// LDS of one workgroup: scales and biases of its rows, then the partial tiles.
size_t skinny_lds(const SkinnyPlan& p, int64_t K, int gs) {
  return (size_t)2 * 16 * p.ntw * (K / gs) * 2 + (size_t)p.W * p.ntw * 4 * 64 * sizeof(float);
}
constexpr size_t kSkMaxLds = 96 * 1024;  // keeps at least one workgroup per CU with room to spare

template <int BITS, bool XBF16, bool SBF16, int GS, int NTW>
hipError_t launch_t(const QmvArgs& a, const SkinnyPlan& p) {
  const int wgs = (a.N + 16 * NTW - 1) / (16 * NTW);
  const size_t lds = skinny_lds(p, a.K, GS);
  hipLaunchKernelGGL((skinny_kernel<BITS, XBF16, SBF16, GS, NTW>), dim3(wgs), dim3(64 * p.W), lds,
                     a.stream, (const uint16_t*)a.x, (const uint32_t*)a.w,
                     (const uint16_t*)a.scales, (const uint16_t*)a.biases, a.out, a.odt, a.M, a.N,
                     a.K, p.ppw);
  return hipGetLastError();
}

template <int BITS, bool XBF16, bool SBF16, int GS>
hipError_t launch_n(const QmvArgs& a, const SkinnyPlan& p) {
  if constexpr (max_ntw(BITS, GS) >= 4)
    if (p.ntw == 4) return launch_t<BITS, XBF16, SBF16, GS, 4>(a, p);
  if constexpr (max_ntw(BITS, GS) >= 2)
    if (p.ntw == 2) return launch_t<BITS, XBF16, SBF16, GS, 2>(a, p);
  return launch_t<BITS, XBF16, SBF16, GS, 1>(a, p);
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

bool skinny_supported(int64_t M, int64_t N, int64_t K, int bits, int gs) {
  const int64_t lim = (int64_t)1 << 31;
  if (!(M >= 1 && M <= kSkinnyMaxM && K % kPiece == 0 && N >= 1 && N * K * bits / 8 < lim &&
        M * K * 2 < lim && N * (K / gs) * 2 < lim))
    return false;
  return skinny_lds(plan_skinny((int)N, (int)K, bits, gs), K, gs) <= kSkMaxLds;
}

hipError_t launch_skinny(const QmvArgs& a) {
  if (!skinny_supported(a.M, a.N, a.K, a.bits, a.gs)) return hipErrorInvalidValue;
  const SkinnyPlan p = plan_skinny(a.N, a.K, a.bits, a.gs);
  return a.bits == 4 ? launch_b<4>(a, p) : launch_b<8>(a, p);
}

}  // namespace kh
