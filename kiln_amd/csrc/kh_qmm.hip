// kh_qmm.hip — prefill quantized GEMM for gfx950 (chosen for M > 64).
//
// Same factored arithmetic as the decode path (kh_qmv.hip):
//   y[m,n] = sum_g s[n,g] * P'[m,n,g] + (b[n,g] - OFF*s[n,g]) * X[m,g]
// with P' = x . (OFF + q) on bf16/f16 MFMA (fp32 accumulate, one fresh chain
// per group) and X[m,g] = sum of x over the group, computed once per call
// by qmm_xsum_kernel into a workspace.
//
// Tiling: a 256-thread workgroup owns a 128 (m) x 128 (n) output tile and
// walks K in stages of 64. Per stage it stages the activation tile in LDS as
// bf16/f16 (already permuted into the pair order of the B operand) and the
// packed code tile in LDS as raw words (0.5 or 1 byte per weight); each of
// the four waves (2 x 2, 64 x 64 each) expands its own code fragments in
// registers right before the MFMA. Global loads of stage s+1 are in flight
// while stage s computes.
#include "kh_common.h"
#include "kh_kernels.h"

namespace kh {

namespace {

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

template <int BITS, bool XBF16>
__device__ __forceinline__ u32x4 codes_to_b(uint32_t q0, uint32_t q1) {
  u32x4 r;
  constexpr uint32_t MAG = XBF16 ? 0x43004300u : 0x64006400u;
  if constexpr (BITS == 4) {
    r[0] = (q0 & 0x000f000fu) | MAG;
    r[1] = ((q0 >> 4) & 0x000f000fu) | MAG;
    r[2] = ((q0 >> 8) & 0x000f000fu) | MAG;
    r[3] = ((q0 >> 12) & 0x000f000fu) | MAG;
  } else if constexpr (!XBF16) {
    r[0] = (q0 & 0x00ff00ffu) | MAG;
    r[1] = ((q0 >> 8) & 0x00ff00ffu) | MAG;
    r[2] = (q1 & 0x00ff00ffu) | MAG;
    r[3] = ((q1 >> 8) & 0x00ff00ffu) | MAG;
  } else {
    const uint32_t qq[2] = {q0, q1};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t u = qq[h];
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

constexpr int BM = 128, BN = 128, BK = 64, NT = 256;
constexpr int KB = BK / 8;     // 8-element k-blocks per stage
constexpr int BPAD = 16;       // LDS row padding (words) of the code tile

}  // namespace

// xsum[m, g] = sum_{k in group g} x[m, k], float32, increasing k.
__global__ void qmm_xsum_kernel(const uint16_t* __restrict__ x, int xbf16, float* __restrict__ xsum,
                                int M, int K, int gs) {
  const int G = K / gs;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)M * G) return;
  const int64_t m = i / G, g = i % G;
  const u32x4* src = reinterpret_cast<const u32x4*>(x + m * K + g * gs);
  float s = 0.f;
  for (int c = 0; c < gs / 8; ++c) {
    const u32x4 v = src[c];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t lo = v[e] & 0xffffu, hi = v[e] >> 16;
      s += xbf16 ? bf16_bits_to_f32(lo) : f16_bits_to_f32(lo);
      s += xbf16 ? bf16_bits_to_f32(hi) : f16_bits_to_f32(hi);
    }
  }
  xsum[i] = s;
}

template <int BITS, int GS, bool XBF16>
__global__ __launch_bounds__(NT) void qmm_kernel(const uint16_t* __restrict__ x,
                                                 const uint32_t* __restrict__ w,
                                                 const void* __restrict__ scales,
                                                 const void* __restrict__ biases, int sdt,
                                                 const float* __restrict__ xsum,
                                                 void* __restrict__ out, int odt, int M, int N,
                                                 int K) {
  constexpr int CPW = 32 / BITS;
  constexpr int WPS = 8 / CPW;                 // words per 8-k block
  constexpr int WPR = BK / CPW;                // words per row per stage
  constexpr int GPS = GS >= BK ? 1 : BK / GS;  // groups touched per stage
  constexpr float OFF = (BITS == 8 && XBF16) ? 0.0f : (XBF16 ? 128.0f : 1024.0f);
  constexpr int BROW = BN * WPS + BPAD;        // words per k-block row of the code tile
  constexpr int AV = BM * KB / NT;             // 16-byte activation chunks per thread
  constexpr int BV = BN * WPR / 4 / NT;        // 16-byte code chunks per thread

  __shared__ u32x4 As[KB * BM];
  __shared__ uint32_t Bs[KB * BROW];
  __shared__ float2 Sc[GPS * BN];
  __shared__ float Xs[GPS * BM];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, lg = lane >> 4;
  const int wm = wave & 1, wn = wave >> 1;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int G = K / GS;
  const int64_t WR = K / CPW;
  const int nst = (K + BK - 1) / BK;

  u32x4 ra[AV], rb[BV];
  float2 rs = {0.f, 0.f};
  float rx = 0.f;

  auto load_stage = [&](int st) {
    const int k0 = st * BK;
#pragma unroll
    for (int r = 0; r < AV; ++r) {
      const int c = tid + r * NT;
      const int mm = c / KB, kb = c % KB;
      const int m = m0 + mm, k = k0 + kb * 8;
      ra[r] = (m < M && k < K) ? *reinterpret_cast<const u32x4*>(x + (int64_t)m * K + k)
                               : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int r = 0; r < BV; ++r) {
      const int c = tid + r * NT;
      const int nn = c / (WPR / 4), wq = c % (WPR / 4);
      const int n = n0 + nn;
      const int64_t word = (int64_t)k0 / CPW + wq * 4;
      rb[r] = (n < N && word < WR)
                  ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(w + n * WR + word))
                  : u32x4{0u, 0u, 0u, 0u};
    }
    if (tid < GPS * BN) {
      const int gi = tid / BN, nn = tid % BN;
      const int g = k0 / GS + gi, n = n0 + nn;
      rs = float2{0.f, 0.f};
      if (n < N && g < G) {
        const float sc = load_as_f32(scales, sdt, (int64_t)n * G + g);
        rs = float2{sc, fmaf(-OFF, sc, load_as_f32(biases, sdt, (int64_t)n * G + g))};
      }
    }
    if (tid >= NT - GPS * BM) {
      const int t2 = tid - (NT - GPS * BM);
      const int gi = t2 / BM, mm = t2 % BM;
      const int g = k0 / GS + gi, m = m0 + mm;
      rx = (m < M && g < G) ? xsum[(int64_t)m * G + g] : 0.f;
    }
  };

  auto store_stage = [&]() {
#pragma unroll
    for (int r = 0; r < AV; ++r) {
      const int c = tid + r * NT;
      const int mm = c / KB, kb = c % KB;
      As[kb * BM + mm] = permute_x<BITS>(ra[r]);
    }
#pragma unroll
    for (int r = 0; r < BV; ++r) {
      const int c = tid + r * NT;
      const int nn = c / (WPR / 4), wq = c % (WPR / 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int word = wq * 4 + e;  // word within the stage row
        const int kb = word / WPS, sub = word % WPS;
        Bs[kb * BROW + nn * WPS + sub] = rb[r][e];
      }
    }
    if (tid < GPS * BN) Sc[tid] = rs;
    if (tid >= NT - GPS * BM) Xs[tid - (NT - GPS * BM)] = rx;
  };

  f32x4 acc[4][4], P[4][4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[t][u] = P[t][u] = f32x4{0.f, 0.f, 0.f, 0.f};

  load_stage(0);
  for (int st = 0; st < nst; ++st) {
    __syncthreads();
    store_stage();
    __syncthreads();
    if (st + 1 < nst) load_stage(st + 1);

#pragma unroll
    for (int j = 0; j < BK / 32; ++j) {
      const int kabs = st * BK + j * 32;
      if (kabs % GS == 0) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int u = 0; u < 4; ++u) P[t][u] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
      const int kb = 4 * j + lg;
      u32x4 a[4], b[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) a[t] = As[kb * BM + wm * 64 + t * 16 + col];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int nn = wn * 64 + u * 16 + col;
        const uint32_t q0 = Bs[kb * BROW + nn * WPS];
        const uint32_t q1 = WPS == 2 ? Bs[kb * BROW + nn * WPS + 1] : 0u;
        b[u] = codes_to_b<BITS, XBF16>(q0, q1);
      }
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int u = 0; u < 4; ++u) P[t][u] = mfma<XBF16>(a[t], b[u], P[t][u]);

      if ((kabs + 32) % GS == 0) {
        const int gi = GS >= BK ? 0 : (j * 32) / GS;
        float2 sb[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) sb[u] = Sc[gi * BN + wn * 64 + u * 16 + col];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const f32x4 xs = *reinterpret_cast<const f32x4*>(&Xs[gi * BM + wm * 64 + t * 16 + 4 * lg]);
#pragma unroll
          for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              acc[t][u][i] = fmaf(sb[u].x, P[t][u][i], acc[t][u][i]);
              acc[t][u][i] = fmaf(sb[u].y, xs[i], acc[t][u][i]);
            }
        }
      }
    }
  }

#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int n = n0 + wn * 64 + u * 16 + col;
      if (n >= N) continue;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = m0 + wm * 64 + t * 16 + 4 * lg + i;
        if (m < M) store_from_f32(out, odt, (int64_t)m * N + n, acc[t][u][i]);
      }
    }
}

template <int BITS, bool XBF16>
static hipError_t launch_gs(const QmvArgs& a, float* xsum) {
  const dim3 grid((a.N + BN - 1) / BN, (a.M + BM - 1) / BM), block(NT);
#define KH_QMM_LAUNCH(GSV)                                                                      \
  hipLaunchKernelGGL((qmm_kernel<BITS, GSV, XBF16>), grid, block, 0, a.stream,                  \
                     (const uint16_t*)a.x, (const uint32_t*)a.w, a.scales, a.biases, a.sdt, xsum, \
                     a.out, a.odt, a.M, a.N, a.K)
  switch (a.gs) {
    case 32: KH_QMM_LAUNCH(32); break;
    case 64: KH_QMM_LAUNCH(64); break;
    default: KH_QMM_LAUNCH(128); break;
  }
#undef KH_QMM_LAUNCH
  return hipGetLastError();
}

hipError_t launch_qmm(const QmvArgs& a, float* xsum) {
  const int64_t total = (int64_t)a.M * (a.K / a.gs);
  hipLaunchKernelGGL(qmm_xsum_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, a.stream,
                     (const uint16_t*)a.x, a.xdt == DT_BF16 ? 1 : 0, xsum, a.M, a.K, a.gs);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const bool xbf16 = a.xdt == DT_BF16;
  if (a.bits == 4) return xbf16 ? launch_gs<4, true>(a, xsum) : launch_gs<4, false>(a, xsum);
  return xbf16 ? launch_gs<8, true>(a, xsum) : launch_gs<8, false>(a, xsum);
}

}  // namespace kh
