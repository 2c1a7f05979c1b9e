// kh_qmm.hip — prefill quantized GEMM for gfx950 (M > 16).
//
// y[m, n] = sum_k x[m, k] * w[n, k], w = s[n, g(k)] * q[n, k] + b[n, g(k)]
// (quantized_matmul, transpose=true: crates/kiln-mlx/src/ops.rs:359-388).
//
// Numerics. Each weight is dequantised once, in registers, to float16 with a
// single rounding: w16 = fma16(s, q, b) (v_pk_fma_f16; q is exact, produced
// as (1024 + q) - 1024 from the code OR-ed into the mantissa of 1024.0). The
// activations enter as float16 too: qmm_prep_x converts each row of x to
// float16 after an exact power-of-two scaling 2^-e_m chosen so that the row's
// largest magnitude stays below 2^15, and the result row is multiplied back
// by 2^e_m. Products accumulate in float32 (v_mfma_f32_16x16x32_f16). The
// only rounding beyond the float32 reference is that of w to float16
// (relative 2^-11): about 1e-4 relative error on typical outputs, an order
// of magnitude inside the 1e-3 mean tolerance (rounding w to bfloat16 instead
// would give ~1.7e-3). Float32 outputs of the same row do not depend on M.
//
// Tiling. A 256-thread workgroup owns a 256 (m) x 128 (n) output tile and
// walks K in stages of 64. Per stage it copies the (pre-permuted) float16
// activation tile and the raw code tile into LDS; each of its four waves
// (2 x 2, 128 x 64 each) expands its own code fragments to float16 in
// registers right before the MFMAs and accumulates directly into the output
// tile. Global loads of stage s+1 are in flight while stage s computes.
#include "kh_common.h"
#include "kh_kernels.h"

namespace kh {

namespace {

typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 h2;

constexpr int BM = 256, BN = 128, BK = 64, NT = 256;
constexpr int KB = BK / 8;  // 8-element k-blocks per stage
constexpr int WM = 128, WN = 64;  // wave tile
constexpr int MT = WM / 16, NTL = WN / 16;
constexpr int BPAD = 4;     // words of padding per k-block row of the code tile
constexpr int PF = 2;  // stages of global loads in flight

// Pairs of codes as float16 (1024 + q) in both halves (exact for q < 1024).
template <int BITS>
__device__ __forceinline__ void code_pairs(uint32_t q0, uint32_t q1, uint32_t mag, uint32_t* r) {
  if constexpr (BITS == 4) {
    r[0] = (q0 & 0x000f000fu) | mag;
    r[1] = ((q0 >> 4) & 0x000f000fu) | mag;
    r[2] = ((q0 >> 8) & 0x000f000fu) | mag;
    r[3] = ((q0 >> 12) & 0x000f000fu) | mag;
  } else {
    r[0] = (q0 & 0x00ff00ffu) | mag;
    r[1] = ((q0 >> 8) & 0x00ff00ffu) | mag;
    r[2] = (q1 & 0x00ff00ffu) | mag;
    r[3] = ((q1 >> 8) & 0x00ff00ffu) | mag;
  }
}

__device__ __forceinline__ f32x4 mfma_f16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

}  // namespace

// dst = permuted float16 of row * 2^-e, *rs = 2^e, with e >= 0 the smallest
// exponent keeping max|row| * 2^-e below 2^15. Called by all 256 threads of a
// workgroup (red: 256 floats of LDS). zero: write a zero row and *rs = 0.
template <int BITS, bool XBF16>
__device__ __forceinline__ void prep_row(const uint16_t* __restrict__ x, u32x4* __restrict__ dst,
                                         float* __restrict__ rs, int K, bool zero, float* red) {
  const int tid = threadIdx.x;
  const u32x4* row = reinterpret_cast<const u32x4*>(x);
  const int nb = K / 8;
  if (zero) {
    for (int c = tid; c < nb; c += 256) dst[c] = u32x4{0u, 0u, 0u, 0u};
    if (tid == 0) *rs = 0.f;
    return;
  }
  float mx = 0.f;
  for (int c = tid; c < nb; c += 256) {
    const u32x4 v = row[c];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = XBF16 ? bf16_bits_to_f32(v[e] & 0xffffu) : f16_bits_to_f32(v[e] & 0xffffu);
      const float hi = XBF16 ? bf16_bits_to_f32(v[e] >> 16) : f16_bits_to_f32(v[e] >> 16);
      mx = fmaxf(mx, fmaxf(fabsf(lo), fabsf(hi)));
    }
  }
  red[tid] = mx;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (tid < s) red[tid] = fmaxf(red[tid], red[tid + s]);
    __syncthreads();
  }
  mx = red[0];
  int ex = 0;
  if (mx >= 32768.f) {
    int e2;
    (void)frexpf(mx, &e2);  // mx = f * 2^e2, f in [0.5, 1)
    ex = e2 - 15;           // mx * 2^-ex < 2^15
  }
  const float inv = ldexpf(1.f, -ex);
  if (tid == 0) *rs = ldexpf(1.f, ex);
  for (int c = tid; c < nb; c += 256) {
    const u32x4 v = row[c];
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = XBF16 ? bf16_bits_to_f32(v[e] & 0xffffu) : f16_bits_to_f32(v[e] & 0xffffu);
      const float hi = XBF16 ? bf16_bits_to_f32(v[e] >> 16) : f16_bits_to_f32(v[e] >> 16);
      o[e] = f32_to_f16_bits(lo * inv) | (f32_to_f16_bits(hi * inv) << 16);
    }
    dst[c] = permute_x<BITS>(o);
  }
}

// prep_row by WPR waves (64 * WPR threads per row, WPR = 1 or 4), for rows
// of at most 64 * WPR * CPL 16-byte chunks: the row is read once into
// registers and its maximum reduced across lanes (and, for WPR = 4, across
// the workgroup's waves through LDS), then converted. Same values as
// prep_row: the maximum does not depend on the order it is taken in.
template <int BITS, bool XBF16, int CPL, int WPR>
__device__ __forceinline__ void prep_row_regs(const uint16_t* __restrict__ x, u32x4* __restrict__ dst,
                                              float* __restrict__ rs, int K, bool zero, float* red) {
  constexpr int TPR = 64 * WPR;  // threads per row
  const int tr = threadIdx.x % TPR;
  const u32x4* row = reinterpret_cast<const u32x4*>(x);
  const int nb = K / 8;
  if (zero) {  // uniform across the row's threads
    for (int c = tr; c < nb; c += TPR) dst[c] = u32x4{0u, 0u, 0u, 0u};
    if (tr == 0) *rs = 0.f;
    return;
  }
  u32x4 v[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int i = c * TPR + tr;
    v[c] = i < nb ? row[i] : u32x4{0u, 0u, 0u, 0u};
  }
  float mx = 0.f;
#pragma unroll
  for (int c = 0; c < CPL; ++c)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = XBF16 ? bf16_bits_to_f32(v[c][e] & 0xffffu) : f16_bits_to_f32(v[c][e] & 0xffffu);
      const float hi = XBF16 ? bf16_bits_to_f32(v[c][e] >> 16) : f16_bits_to_f32(v[c][e] >> 16);
      mx = fmaxf(mx, fmaxf(fabsf(lo), fabsf(hi)));
    }
  mx = wave_max(mx);
  if constexpr (WPR > 1) {
    if ((tr & 63) == 0) red[tr >> 6] = mx;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < WPR; ++w) mx = fmaxf(mx, red[w]);
    __syncthreads();  // red is reused by the next row
  }
  int ex = 0;
  if (mx >= 32768.f) {
    int e2;
    (void)frexpf(mx, &e2);
    ex = e2 - 15;
  }
  const float inv = ldexpf(1.f, -ex);
  if (tr == 0) *rs = ldexpf(1.f, ex);
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int i = c * TPR + tr;
    if (i >= nb) break;
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = XBF16 ? bf16_bits_to_f32(v[c][e] & 0xffffu) : f16_bits_to_f32(v[c][e] & 0xffffu);
      const float hi = XBF16 ? bf16_bits_to_f32(v[c][e] >> 16) : f16_bits_to_f32(v[c][e] >> 16);
      o[e] = f32_to_f16_bits(lo * inv) | (f32_to_f16_bits(hi * inv) << 16);
    }
    dst[i] = permute_x<BITS>(o);
  }
}

// 4 / WPR rows per workgroup of 256 threads.
template <int BITS, bool XBF16, int CPL, int WPR>
__global__ __launch_bounds__(256) void qmm_prep_x_w(const uint16_t* __restrict__ x, u32x4* __restrict__ xh,
                                                    float* __restrict__ rscale, int M, int K) {
  __shared__ float red[4];
  const int m = blockIdx.x * (4 / WPR) + (int)threadIdx.x / (64 * WPR);
  if (m >= M) return;  // WPR = 4: uniform per workgroup
  prep_row_regs<BITS, XBF16, CPL, WPR>(x + (int64_t)m * K, xh + (int64_t)m * (K / 8), rscale + m, K, false,
                                       red);
}

// group_prep_x with the row kernels' layout.
template <int BITS, bool XBF16, int CPL, int WPR>
__global__ __launch_bounds__(256) void group_prep_x_w(const uint16_t* __restrict__ x, GatherArgs g, int M,
                                                      const int* __restrict__ pos, u32x4* __restrict__ xh,
                                                      float* __restrict__ rscale, int* __restrict__ rowmap,
                                                      int K) {
  __shared__ float red[4];
  constexpr int RPW = 4 / WPR;  // rows per workgroup and step
  const int64_t rows = g.pairs * M;
  // every thread of a row (for WPR = 4: of the workgroup) runs the same trips
  for (int64_t r = (int64_t)blockIdx.x * RPW + (int)threadIdx.x / (64 * WPR); r < rows;
       r += (int64_t)gridDim.x * RPW) {
    const int64_t b = r / M;
    const int i = (int)(r % M);
    int64_t xo;
    const int e = gather_expert(g, b, &xo);
    const int64_t pr = pos[b] + i;
    prep_row_regs<BITS, XBF16, CPL, WPR>(x + xo + (int64_t)i * K, xh + pr * (K / 8), rscale + pr, K,
                                         e >= g.E, red);
    if ((int)threadIdx.x % (64 * WPR) == 0) rowmap[pr] = (int)r;
  }
}

// xh[m], rscale[m] = prep_row(x[m]). One workgroup per row.
template <int BITS, bool XBF16>
__global__ __launch_bounds__(256) void qmm_prep_x(const uint16_t* __restrict__ x,
                                                  u32x4* __restrict__ xh,
                                                  float* __restrict__ rscale, int K) {
  __shared__ float red[256];
  const int m = blockIdx.x;
  prep_row<BITS, XBF16>(x + (int64_t)m * K, xh + (int64_t)m * (K / 8), rscale + m, K, false, red);
}

// Grouped (gather_qmm) rows: row r = pair b * M + i of the batch goes to
// padded row pos[b] + i; rowmap records r there. Pairs whose expert id is
// out of range get a zero row and scale 0 (their outputs are zeros).
template <int BITS, bool XBF16>
__global__ __launch_bounds__(256) void group_prep_x(const uint16_t* __restrict__ x, GatherArgs g, int M,
                                                    const int* __restrict__ pos, u32x4* __restrict__ xh,
                                                    float* __restrict__ rscale, int* __restrict__ rowmap,
                                                    int K) {
  __shared__ float red[256];
  for (int64_t r = blockIdx.x; r < g.pairs * M; r += gridDim.x) {
    const int64_t b = r / M;
    const int i = (int)(r % M);
    int64_t xo;
    const int e = gather_expert(g, b, &xo);
    const int64_t pr = pos[b] + i;
    prep_row<BITS, XBF16>(x + xo + (int64_t)i * K, xh + pr * (K / 8), rscale + pr, K, e >= g.E, red);
    if (threadIdx.x == 0) rowmap[pr] = (int)r;
    __syncthreads();  // red is reused by the next row
  }
}

template <int BITS, int GS, bool SF16>
__global__ __launch_bounds__(NT) void qmm_kernel(const u32x4* __restrict__ xh,
                                                 const uint32_t* __restrict__ w,
                                                 const uint16_t* __restrict__ scales,
                                                 const uint16_t* __restrict__ biases,
                                                 const float* __restrict__ rscale,
                                                 void* __restrict__ out, int odt, int M, int N,
                                                 int K, Epilogue epi) {
  constexpr int CPW = 32 / BITS;
  constexpr int WPS = 8 / CPW;                 // words per 8-k block
  constexpr int WPR = BK / CPW;                // words per row per stage
  constexpr int GPS = GS >= BK ? 1 : BK / GS;  // groups touched per stage
  constexpr int BROW = BN * WPS + BPAD;        // words per k-block row of the code tile
  constexpr int AV = BM * KB / NT;             // 16-byte activation chunks per thread
  constexpr int BV = BN * WPR / 4 / NT;        // 16-byte code chunks per thread

  __shared__ u32x4 As[KB * BM];
  __shared__ uint32_t Bs[KB * BROW];
  __shared__ uint32_t Ss[GPS * BN];  // f16 scales: (s, s); bf16 scales: f32 bits of s
  __shared__ uint32_t Bb[GPS * BN];  // f16: (b, b);     bf16: f32 bits of b

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, lg = lane >> 4;
  const int wm = wave & 1, wn = wave >> 1;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int G = K / GS;
  const int64_t WR = K / CPW;
  const int KB8 = K / 8;
  const int nst = (K + BK - 1) / BK;

  // Prefetch ring: stage st lives in registers slot st % PF until stored to LDS.
  u32x4 ra[PF][AV], rb[PF][BV];
  uint32_t rs[PF], rbb[PF];

  auto load_stage = [&](int p, int st) {
    const int kb0 = st * KB;
#pragma unroll
    for (int r = 0; r < AV; ++r) {
      const int c = tid + r * NT;
      const int mm = c / KB, kb = c % KB;
      const int m = m0 + mm;
      ra[p][r] = (m < M && kb0 + kb < KB8) ? xh[(int64_t)m * KB8 + kb0 + kb] : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int r = 0; r < BV; ++r) {
      const int c = tid + r * NT;
      const int nn = c / (WPR / 4), wq = c % (WPR / 4);
      const int n = n0 + nn;
      const int64_t word = (int64_t)st * WPR + wq * 4;
      rb[p][r] = (n < N && word < WR) ? *reinterpret_cast<const u32x4*>(w + n * WR + word)
                                      : u32x4{0u, 0u, 0u, 0u};
    }
    if (tid < GPS * BN) {
      const int gi = tid / BN, nn = tid % BN;
      const int g = (st * BK) / GS + gi, n = n0 + nn;
      rs[p] = rbb[p] = 0u;
      if (n < N && g < G) {
        const uint32_t sh = scales[(int64_t)n * G + g], bh = biases[(int64_t)n * G + g];
        if constexpr (SF16) {
          rs[p] = sh | (sh << 16);
          rbb[p] = bh | (bh << 16);
        } else {
          rs[p] = __float_as_uint(bf16_bits_to_f32(sh));
          rbb[p] = __float_as_uint(bf16_bits_to_f32(bh));
        }
      }
    }
  };

  // Activation tile: k-block kb of row m at As[kb*BM + (m ^ kb)] — the XOR
  // spreads the eight k-blocks of a row (stored by neighbouring threads) over
  // different banks; readers of one k-block see a permutation of 16 rows.
  auto store_stage = [&](int p) {
#pragma unroll
    for (int r = 0; r < AV; ++r) {
      const int c = tid + r * NT;
      const int mm = c / KB, kb = c % KB;
      As[kb * BM + (mm ^ kb)] = ra[p][r];
    }
#pragma unroll
    for (int r = 0; r < BV; ++r) {
      const int c = tid + r * NT;
      const int nn = c / (WPR / 4), wq = c % (WPR / 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int word = wq * 4 + e;  // word within the stage row
        Bs[(word / WPS) * BROW + nn * WPS + word % WPS] = rb[p][r][e];
      }
    }
    if (tid < GPS * BN) {
      Ss[tid] = rs[p];
      Bb[tid] = rbb[p];
    }
  };

  uint32_t mag = 0x64006400u;  // float16 1024.0 in both halves
  asm volatile("" : "+v"(mag));  // a VGPR operand, so (mask, or) fuses into v_and_or_b32

  f32x4 acc[MT][NTL];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int u = 0; u < NTL; ++u) acc[t][u] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int p = 0; p < PF; ++p)
    if (p < nst) load_stage(p, p);
  for (int st0 = 0; st0 < nst; st0 += PF) {
#pragma unroll
  for (int p = 0; p < PF; ++p) {
    const int st = st0 + p;
    if (st >= nst) continue;  // uniform
    __syncthreads();
    store_stage(p);
    __syncthreads();
    if (st + PF < nst) load_stage(p, st + PF);

#pragma unroll
    for (int j = 0; j < BK / 32; ++j) {
      const int kb = 4 * j + lg;
      const int gi = GS >= BK ? 0 : (j * 32) / GS;
      u32x4 b[NTL];
#pragma unroll
      for (int u = 0; u < NTL; ++u) {
        const int nn = wn * WN + u * 16 + col;
        const uint32_t q0 = Bs[kb * BROW + nn * WPS];
        const uint32_t q1 = WPS == 2 ? Bs[kb * BROW + nn * WPS + 1] : 0u;
        uint32_t r[4];
        code_pairs<BITS>(q0, q1, mag, r);
        if constexpr (SF16) {
          const h2 s2 = __builtin_bit_cast(h2, Ss[gi * BN + nn]);
          const h2 b2 = __builtin_bit_cast(h2, Bb[gi * BN + nn]);
          const h2 k1024 = h2{(_Float16)1024.f, (_Float16)1024.f};
#pragma unroll
          for (int i = 0; i < 4; ++i)
            b[u][i] = __builtin_bit_cast(
                uint32_t, __builtin_elementwise_fma(s2, __builtin_bit_cast(h2, r[i]) - k1024, b2));
        } else {
          const float sf = __uint_as_float(Ss[gi * BN + nn]);
          const float bf = __uint_as_float(Bb[gi * BN + nn]);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            // (1024 + q) - 1024 is exact; one rounding in the fma, one to f16
            const float lo = fmaf(sf, f16_bits_to_f32(r[i] & 0xffffu) - 1024.f, bf);
            const float hi = fmaf(sf, f16_bits_to_f32(r[i] >> 16) - 1024.f, bf);
            b[u][i] = f32_to_f16_bits(lo) | (f32_to_f16_bits(hi) << 16);
          }
        }
      }
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const u32x4 a = As[kb * BM + ((wm * WM + t * 16 + col) ^ kb)];
#pragma unroll
        for (int u = 0; u < NTL; ++u) acc[t][u] = mfma_f16(a, b[u], acc[t][u]);
      }
    }
  }
  }

#pragma unroll
  for (int t = 0; t < MT; ++t) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = m0 + wm * WM + t * 16 + 4 * lg + i;
      if (m >= M) continue;
      const float rsc = rscale[m];
#pragma unroll
      for (int u = 0; u < NTL; ++u) {
        const int n = n0 + wn * WN + u * 16 + col;
        if (n < N) store_from_f32(out, odt, (int64_t)m * N + n, epi(acc[t][u][i] * rsc, n));
      }
    }
  }
}

size_t qmm_workspace_bytes(int M, int K) {
  return (size_t)M * K * 2 + (size_t)M * sizeof(float) + 256;
}

template <int BITS, int GS>
static hipError_t launch_sf(const QmvArgs& a, const u32x4* xh, const float* rsc) {
  const dim3 grid((a.N + BN - 1) / BN, (a.M + BM - 1) / BM), block(NT);
  if (a.sdt == DT_F16)
    hipLaunchKernelGGL((qmm_kernel<BITS, GS, true>), grid, block, 0, a.stream, xh,
                       (const uint32_t*)a.w, (const uint16_t*)a.scales, (const uint16_t*)a.biases,
                       rsc, a.out, a.odt, a.M, a.N, a.K, a.epi());
  else
    hipLaunchKernelGGL((qmm_kernel<BITS, GS, false>), grid, block, 0, a.stream, xh,
                       (const uint32_t*)a.w, (const uint16_t*)a.scales, (const uint16_t*)a.biases,
                       rsc, a.out, a.odt, a.M, a.N, a.K, a.epi());
  return hipGetLastError();
}

template <int BITS>
static hipError_t launch_gs(const QmvArgs& a, const u32x4* xh, const float* rsc) {
  switch (a.gs) {
    case 32: return launch_sf<BITS, 32>(a, xh, rsc);
    case 64: return launch_sf<BITS, 64>(a, xh, rsc);
    default: return launch_sf<BITS, 128>(a, xh, rsc);
  }
}

// `ws` holds qmm_workspace_bytes(M, K) bytes (16-byte aligned). Scales and
// biases are float16 or bfloat16.
// Layout of the register row kernels: (chunks per lane, waves per row), or
// cpl = 0 when the row is too long for registers (workgroup-per-row kernels).
struct PrepShape {
  int cpl, wpr;
};
static PrepShape prep_shape(int K) {
  const int nb = K / 8;
  for (int c : {2, 4, 8})
    if (nb <= 64 * c) return {c, 1};
  for (int c : {4, 8})
    if (nb <= 256 * c) return {c, 4};
  return {0, 0};
}

template <int BITS, bool X>
static hipError_t group_prep_b(const QmvArgs& a, const GatherArgs& g, const int* pos, u32x4* xh, float* rsc,
                               int* rowmap) {
  const int64_t rows = g.pairs * a.M;
  const PrepShape ps = prep_shape(a.K);
  if (ps.cpl == 0) {
    const unsigned grid = (unsigned)(rows < (1 << 20) ? rows : (1 << 20));
    hipLaunchKernelGGL((group_prep_x<BITS, X>), dim3(grid), dim3(256), 0, a.stream, (const uint16_t*)a.x, g,
                       a.M, pos, xh, rsc, rowmap, a.K);
    return hipGetLastError();
  }
  const int64_t wg = ps.wpr == 1 ? (rows + 3) / 4 : rows;
  const unsigned grid = (unsigned)(wg < (1 << 20) ? wg : (1 << 20));
#define KH_GW(C, W)                                                                                   \
  hipLaunchKernelGGL((group_prep_x_w<BITS, X, C, W>), dim3(grid), dim3(256), 0, a.stream,             \
                     (const uint16_t*)a.x, g, a.M, pos, xh, rsc, rowmap, a.K)
  if (ps.wpr == 1) {
    if (ps.cpl == 2) KH_GW(2, 1); else if (ps.cpl == 4) KH_GW(4, 1); else KH_GW(8, 1);
  } else {
    if (ps.cpl == 4) KH_GW(4, 4); else KH_GW(8, 4);
  }
#undef KH_GW
  return hipGetLastError();
}

hipError_t launch_group_prep_x(const QmvArgs& a, const GatherArgs& g, const int* pos, void* xh_,
                               float* rsc, int* rowmap) {
  u32x4* xh = static_cast<u32x4*>(xh_);
  const bool xbf16 = a.xdt == DT_BF16;
  if (a.bits == 4)
    return xbf16 ? group_prep_b<4, true>(a, g, pos, xh, rsc, rowmap) : group_prep_b<4, false>(a, g, pos, xh, rsc, rowmap);
  return xbf16 ? group_prep_b<8, true>(a, g, pos, xh, rsc, rowmap) : group_prep_b<8, false>(a, g, pos, xh, rsc, rowmap);
}

template <int BITS, bool X>
static hipError_t prep_b(const QmvArgs& a, u32x4* xh, float* rsc) {
  const PrepShape ps = prep_shape(a.K);
  if (ps.cpl == 0) {
    hipLaunchKernelGGL((qmm_prep_x<BITS, X>), dim3(a.M), dim3(256), 0, a.stream, (const uint16_t*)a.x, xh, rsc,
                       a.K);
    return hipGetLastError();
  }
  const dim3 grid(ps.wpr == 1 ? (a.M + 3) / 4 : a.M);
#define KH_PW(C, W)                                                                                 \
  hipLaunchKernelGGL((qmm_prep_x_w<BITS, X, C, W>), grid, dim3(256), 0, a.stream, (const uint16_t*)a.x, xh, \
                     rsc, a.M, a.K)
  if (ps.wpr == 1) {
    if (ps.cpl == 2) KH_PW(2, 1); else if (ps.cpl == 4) KH_PW(4, 1); else KH_PW(8, 1);
  } else {
    if (ps.cpl == 4) KH_PW(4, 4); else KH_PW(8, 4);
  }
#undef KH_PW
  return hipGetLastError();
}

hipError_t launch_prep_x(const QmvArgs& a, void* xh_, float* rsc) {
  u32x4* xh = static_cast<u32x4*>(xh_);
  const bool xbf16 = a.xdt == DT_BF16;
  if (a.bits == 4) return xbf16 ? prep_b<4, true>(a, xh, rsc) : prep_b<4, false>(a, xh, rsc);
  return xbf16 ? prep_b<8, true>(a, xh, rsc) : prep_b<8, false>(a, xh, rsc);
}

hipError_t launch_qmm(const QmvArgs& a, void* ws) {
  u32x4* xh = static_cast<u32x4*>(ws);
  float* rsc = reinterpret_cast<float*>(static_cast<char*>(ws) + (size_t)a.M * a.K * 2);
  hipError_t e = launch_prep_x(a, xh, rsc);
  if (e != hipSuccess) return e;
  return a.bits == 4 ? launch_gs<4>(a, xh, rsc) : launch_gs<8>(a, xh, rsc);
}

}  // namespace kh
