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
#include <algorithm>
#include <type_traits>

#include "kh_common.h"
#include "kh_kernels.h"

namespace kh {

namespace {

constexpr int kSkMaxWaves = 8;
constexpr int kSkMaxParts = 4;
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

// Up to kSkMaxParts weight sets on one x per launch (q/k/v): workgroup b
// takes tile b - tile0 of the part whose range holds b. In paired mode (the
// gated MLP, act >= 0) a workgroup takes the same NTW/2 16-row tiles of part
// 0 (gate) and part 1 (up) and stores act(gate) * up into part 0's output.
// Each output is summed exactly as in a single-part launch.
struct SkPart {
  const uint32_t* w;
  const uint16_t* scales;
  const uint16_t* biases;
  void* out;
  int odt, N, tile0;
  Epilogue epi;
};
struct SkParts {
  SkPart part[kSkMaxParts];
  int n, act;
};

template <int BITS, int NTW, int MT>
struct Piece {
  u32x4 q[NTW][BITS / 4];  // the lane's 32 codes per tile
  u32x4 x[MT][4];          // x[m, run .. run+31] per 16-row m-tile
};

template <int BITS, bool XBF16, bool SBF16, int GS, int NTW, int MT>
__global__ __launch_bounds__(64 * kSkMaxWaves) void skinny_kernel(
    const uint16_t* __restrict__ x, SkParts parts, int M, int K, int ppw) {
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
  const bool paired = parts.act >= 0;  // uniform
  constexpr int HALF = NTW / 2 > 0 ? NTW / 2 : 1;  // tiles per part in paired mode (NTW even there)
  int pi = 0;                          // the part (independent mode)
  if (!paired)
    while (pi + 1 < parts.n && (int)blockIdx.x >= parts.part[pi + 1].tile0) ++pi;
  const int n0 = paired ? (int)blockIdx.x * 16 * HALF : ((int)blockIdx.x - parts.part[pi].tile0) * ROWS;
  const int G = K / GS;
  const int wpr = K * BITS / 32;
  const int gl = (kb * 32) / GS;  // group of this lane's run within a piece

  // slot t: its part and its first row (paired: slots 0..HALF-1 gate, the
  // rest up, over the same rows)
  auto slot_part = [&](int t) { return paired ? (t < HALF ? 0 : 1) : pi; };
  auto slot_row = [&](int t) { return n0 + (paired ? (t % HALF) : t) * 16; };
  const uint32_t* wrow[NTW];
#pragma unroll
  for (int t = 0; t < NTW; ++t) {
    const SkPart& sp = parts.part[slot_part(t)];
    wrow[t] = sp.w + (int64_t)min(slot_row(t) + col, sp.N - 1) * wpr;
  }
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
      const u32x4* src = reinterpret_cast<const u32x4*>(wrow[t] + run * BITS / 32);
#pragma unroll
      for (int h = 0; h < BITS / 4; ++h) P.q[t][h] = __builtin_nontemporal_load(src + h);
    }
    // padding rows (m >= M) load nothing: their lanes read zeros, so the
    // batch costs x bytes for its M rows only
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j) P.x[mt][j] = mval[mt] ? xr[mt][(run >> 3) + j] : u32x4{0u, 0u, 0u, 0u};
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
  // the rows' scales and biases: one run of consecutive rows per part (two
  // in paired mode, into LDS rows 0.. and 16*HALF..); rows past N are not
  // loaded and their outputs are never stored
  for (int r = 0; r < (paired ? 2 : 1); ++r) {
    const SkPart& sp = parts.part[paired ? r : pi];
    const int rows = paired ? 16 * HALF : ROWS, dst0 = paired ? r * 16 * HALF : 0;
    const int nr = min(rows, sp.N - n0);
    const int64_t cnt = (int64_t)nr * G;
    const uint16_t* src[2] = {sp.scales + (int64_t)n0 * G, sp.biases + (int64_t)n0 * G};
    uint16_t* dst[2] = {sbl + (int64_t)dst0 * G, sbl + ((int64_t)ROWS + dst0) * G};
    if ((G & 7) == 0) {
      for (int64_t i = threadIdx.x; i < 2 * cnt / 8; i += blockDim.x) {
        const int a = i >= cnt / 8;
        const int64_t j = i - a * (cnt / 8);
        reinterpret_cast<u32x4*>(dst[a])[j] = reinterpret_cast<const u32x4*>(src[a])[j];
      }
    } else {
      for (int64_t i = threadIdx.x; i < 2 * cnt; i += blockDim.x) {
        const int a = i >= cnt;
        const int64_t j = i - a * cnt;
        dst[a][j] = src[a][j];
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
  const int stride = MT * NTW * 256;
  auto sum = [&](int mt, int t, int e, int l) {
    const int base = ((mt * NTW + t) * 4 + e) * 64 + l;
    float v = red[base];
    for (int ww = 1; ww < W; ++ww) v += red[base + ww * stride];
    return v;
  };
  if (!paired) {
    const SkPart& sp = parts.part[pi];
    for (int i = threadIdx.x; i < MT * NTW * 256; i += blockDim.x) {
      const int l = i & 63, e = (i >> 6) & 3, t = (i >> 8) % NTW, mt = (i >> 8) / NTW;
      const int m = mt * 16 + 4 * (l >> 4) + e, n = n0 + t * 16 + (l & 15);
      if (m >= M || n >= sp.N) continue;
      store_from_f32(sp.out, sp.odt, (int64_t)m * sp.N + n, sp.epi(sum(mt, t, e, l), n));
    }
  } else {
    const SkPart &g = parts.part[0], &u = parts.part[1];
    for (int i = threadIdx.x; i < MT * HALF * 256; i += blockDim.x) {
      const int l = i & 63, e = (i >> 6) & 3, t = (i >> 8) % HALF, mt = (i >> 8) / HALF;
      const int m = mt * 16 + 4 * (l >> 4) + e, n = n0 + t * 16 + (l & 15);
      if (m >= M || n >= g.N) continue;
      const float v = act_mul(g.epi(sum(mt, t, e, l), n), u.epi(sum(mt, t + HALF, e, l), n), g.odt, parts.act);
      store_from_f32(g.out, g.odt, (int64_t)m * g.N + n, v);
    }
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
constexpr int64_t kSkMaxChainCycles = 20000;  // MFMA cycles per wave (measured bound, see skinny_supported)
constexpr int64_t kSkMaxMfma = 1000000;        // MFMAs per launch (measured crossover, see skinny_supported)
constexpr int64_t kSkMaxWavesMt2 = 3 * 4 * 256;  // three waves per SIMD on 256 CUs  // keeps at least one workgroup per CU with room to spare

// One launch over n parts sharing x, M, K and the plan (act >= 0: paired
// gate/up, n == 2, NTW even).
template <int BITS, bool XBF16, bool SBF16, int GS, int NTW, int MT>
hipError_t launch_t(const QmvArgs* a, int n, int act, const SkinnyPlan& p) {
  SkParts parts{};
  parts.n = n;
  parts.act = act;
  int wgs = 0;
  for (int i = 0; i < n; ++i) {
    parts.part[i] = SkPart{(const uint32_t*)a[i].w, (const uint16_t*)a[i].scales, (const uint16_t*)a[i].biases,
                           a[i].out, a[i].odt, a[i].N, wgs, a[i].epi()};
    if (act < 0) wgs += (a[i].N + 16 * NTW - 1) / (16 * NTW);
  }
  if (act >= 0) wgs = (a[0].N + 8 * NTW - 1) / (8 * NTW);
  const size_t lds = skinny_lds(p, a[0].K, GS);
  hipLaunchKernelGGL((skinny_kernel<BITS, XBF16, SBF16, GS, NTW, MT>), dim3(wgs), dim3(64 * p.W), lds,
                     a[0].stream, (const uint16_t*)a[0].x, parts, a[0].M, a[0].K, p.ppw);
  return hipGetLastError();
}

template <int BITS, bool XBF16, bool SBF16, int GS, int MT>
hipError_t launch_m(const QmvArgs* a, int n, int act, const SkinnyPlan& p) {
  if constexpr (max_ntw(BITS, GS, MT) >= 4)
    if (p.ntw == 4) return launch_t<BITS, XBF16, SBF16, GS, 4, MT>(a, n, act, p);
  if constexpr (max_ntw(BITS, GS, MT) >= 2)
    if (p.ntw == 2) return launch_t<BITS, XBF16, SBF16, GS, 2, MT>(a, n, act, p);
  if (act >= 0) return hipErrorInvalidValue;  // paired mode needs two tiles per workgroup
  return launch_t<BITS, XBF16, SBF16, GS, 1, MT>(a, n, act, p);
}

template <int BITS, bool XBF16, bool SBF16, int GS>
hipError_t launch_n(const QmvArgs* a, int n, int act, const SkinnyPlan& p) {
  return p.mt == 2 ? launch_m<BITS, XBF16, SBF16, GS, 2>(a, n, act, p)
                   : launch_m<BITS, XBF16, SBF16, GS, 1>(a, n, act, p);
}

template <int BITS, bool XBF16, bool SBF16>
hipError_t launch_g(const QmvArgs* a, int n, int act, const SkinnyPlan& p) {
  if (a[0].gs == 32) return launch_n<BITS, XBF16, SBF16, 32>(a, n, act, p);
  if (a[0].gs == 64) return launch_n<BITS, XBF16, SBF16, 64>(a, n, act, p);
  return launch_n<BITS, XBF16, SBF16, 128>(a, n, act, p);
}

template <int BITS>
hipError_t launch_b(const QmvArgs* a, int n, int act, const SkinnyPlan& p) {
  const bool xb = a[0].xdt == DT_BF16, sb = a[0].sdt == DT_BF16;
  if (xb) return sb ? launch_g<BITS, true, true>(a, n, act, p) : launch_g<BITS, true, false>(a, n, act, p);
  return sb ? launch_g<BITS, false, true>(a, n, act, p) : launch_g<BITS, false, false>(a, n, act, p);
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
  // Each wave computes its pieces in sequence. Where that chain of MFMAs
  // (per piece and 16-row tile: 4 steps x groups x m-tiles x (P + X, and
  // the high nibbles of 8-bit codes)) is long, the launch is compute-bound
  // with few waves in flight and the GEMM is faster: Qwen2.5-7B's down
  // projection (8-bit gs32, K = 18944) at M = 17..32 took 84-94 us here
  // against 45-47 on the GEMM. Bound: ~10 us of MFMA issue per wave.
  const int64_t per_piece = 4 * (kPiece / gs) * p.mt * (bits == 8 ? 3 : 2);  // MFMAs per piece and tile
  const int64_t chain = (int64_t)p.ppw * per_piece * p.ntw * 16;
  if (chain > kSkMaxChainCycles) return false;
  // Over the launch the MFMA work per code byte is fixed by (bits, gs, m-tiles);
  // its lower fixed cost wins on small matrices, the GEMM's throughput on
  // large ones: Qwen2.5-7B's gate (8-bit gs32, 68 MB) at M = 16 took 58 us
  // here against ~44 on the GEMM, its q (13 MB) 16 against 28.
  if ((N + 15) / 16 * (K / kPiece) * per_piece > kSkMaxMfma) return false;
  return skinny_lds(p, K, gs) <= kSkMaxLds;
}

hipError_t launch_skinny(const QmvArgs& a) {
  if (!skinny_supported(a.M, a.N, a.K, a.bits, a.gs)) return hipErrorInvalidValue;
  const SkinnyPlan p = plan_skinny(a.M, a.N, a.K, a.bits, a.gs);
  return a.bits == 4 ? launch_b<4>(&a, 1, -1, p) : launch_b<8>(&a, 1, -1, p);
}

hipError_t launch_skinny_multi(const QmvArgs* a, int n) {
  if (n < 1 || n > kSkMaxParts) return hipErrorInvalidValue;
  int64_t nsum = 0;
  for (int i = 0; i < n; ++i) {
    if (!skinny_supported(a[i].M, a[i].N, a[i].K, a[i].bits, a[i].gs)) return hipErrorInvalidValue;
    nsum += a[i].N;
  }
  // the tile width from the launch's total rows (the sums do not depend on
  // it), narrowed if its LDS would not fit
  SkinnyPlan p = plan_skinny(a[0].M, (int)std::min<int64_t>(nsum, INT32_MAX), a[0].K, a[0].bits, a[0].gs);
  while (p.ntw > 1 && skinny_lds(p, a[0].K, a[0].gs) > kSkMaxLds) p.ntw /= 2;
  return a[0].bits == 4 ? launch_b<4>(a, n, -1, p) : launch_b<8>(a, n, -1, p);
}

bool skinny_pairable(const QmvArgs& gate) {
  if (!skinny_supported(gate.M, gate.N, gate.K, gate.bits, gate.gs)) return false;
  const SkinnyPlan p = plan_skinny(gate.M, gate.N, gate.K, gate.bits, gate.gs);
  return max_ntw(gate.bits, gate.gs, p.mt) >= 2 && skinny_lds(SkinnyPlan{p.W, p.ppw, 2, p.mt}, gate.K, gate.gs) <= kSkMaxLds;
}

hipError_t launch_skinny_gate_up(const QmvArgs& gate, const QmvArgs& up, int act) {
  if (!skinny_pairable(gate)) return hipErrorInvalidValue;
  SkinnyPlan p = plan_skinny(gate.M, gate.N, gate.K, gate.bits, gate.gs);
  p.ntw = 2;  // one 16-row tile of each of gate and up per workgroup
  const QmvArgs a[2] = {gate, up};
  return gate.bits == 4 ? launch_b<4>(a, 2, act, p) : launch_b<8>(a, 2, act, p);
}

}  // namespace kh
