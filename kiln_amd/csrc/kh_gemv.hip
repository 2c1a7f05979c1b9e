// kh_gemv.hip — decode quantized GEMV for gfx950 at M <= 8: one pass over
// the packed weights, every load issued up front, VALU dot products.
//
// Computes y[m, n] = sum_k x[m, k] * (s[n, g(k)] * q[n, k] + b[n, g(k)])
// (the transpose=true form of quantized_matmul, crates/kiln-mlx/src/ops.rs:359-388,
// called by Linear::forward nn.rs:89 and Embedding::as_linear nn.rs:187).
//
// Layout. A row of packed codes is a sequence of 16-byte chunks (32 codes at
// 4 bits, 16 at 8 bits); a chunk never straddles a quantization group since
// group_size >= 32. Lane slot t of a workgroup (W waves, 64*W slots) owns
// chunks c = t + i*64*W, i < I, of every one of the workgroup's R rows, so
// one load instruction of a wave reads 1 KB of contiguous weight bytes, and
// the lane's activations for its chunks are loaded once and kept in
// registers for all R rows.
//
// Arithmetic. Per chunk, the codes become 16-bit pairs OFF + q (bf16
// OFF = 128, f16 OFF = 1024, built by OR-ing the code into the mantissa;
// 8-bit codes with bf16 activations convert exactly through float32 with
// OFF = 0) and meet the activations, permuted into the same pair order, in a
// v_dot2c_f32_{bf16,f16} chain. Every product is exact; the affine terms
// are applied per chunk as
//   acc += s * P + (b - OFF*s) * X,   P = sum x*(OFF+q),  X = sum x
// so no dequantised weight is ever rounded.
//
// Reduction, in a fixed order: chunks i ascending within a lane; across the
// 64 lanes of a wave a butterfly over lane offsets 32, 16, ..., 1 whose
// first steps also split the R*M partial sums among lanes; across waves in
// wave order through LDS. Each output's summation tree is the same whatever
// M is, so row r of the result is bitwise identical for every M this kernel
// serves.
#include "kh_common.h"
#include "kh_kernels.h"

namespace kh {

// Plan constants (measured on the Llama-3 shapes):
constexpr int kGemvWaves = 2048;      // waves per launch wanted before fewer rows per workgroup
constexpr int kGemvWavesWide = 4096;  // ... and, while a workgroup keeps more than 4 rows, this many
constexpr int kGemvMaxM1 = 8;         // largest M served with one chunk per lane slot
constexpr int kGemvRMax = 16;         // rows per workgroup with one chunk per lane slot

namespace {

constexpr int kGemvMaxWaves = 8;
constexpr int kGemvMaxParts = 4;

// Raw buffer loads: a descriptor per tensor (uniform, in SGPRs), the row
// offset as the scalar offset and a 32-bit lane offset, so no per-lane 64-bit
// address arithmetic. Tensors are below 4 GiB (checked by the host). The
// third descriptor word 0x00020000 is the gfx9-family raw buffer format.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const void* p) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, 0x7fffffff, 0x00020000);
}

constexpr int kCodeAux = 2;  // non-temporal: weights are streamed once

template <int BITS, bool XBF16>
struct GemvOff {
  static constexpr float value = (BITS == 8 && XBF16) ? 0.0f : (XBF16 ? 128.0f : 1024.0f);
};

template <bool XBF16>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  if constexpr (XBF16)
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a), __builtin_bit_cast(bf2, b), c,
                                           false);
  else
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a), __builtin_bit_cast(h2, b), c, false);
}

// One 16-byte chunk of codes -> NP operand pairs in permute_x order:
// 4-bit word j gives pairs 4j+t = (c_t, c_{t+4}) of that word; 8-bit word j
// gives pairs 2j = (c0, c2), 2j+1 = (c1, c3). `mag` holds OFF in both halves
// in a VGPR, so each (mask, or) is one v_and_or_b32.
template <int BITS, bool XBF16>
__device__ __forceinline__ void chunk_pairs(const uint32_t (&q)[4], uint32_t mag,
                                            uint32_t (&p)[64 / BITS]) {
  if constexpr (BITS == 4) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t u = q[j];
      p[4 * j + 0] = (u & 0x000f000fu) | mag;
      p[4 * j + 1] = ((u >> 4) & 0x000f000fu) | mag;
      p[4 * j + 2] = ((u >> 8) & 0x000f000fu) | mag;
      p[4 * j + 3] = ((u >> 12) & 0x000f000fu) | mag;
    }
  } else if constexpr (!XBF16) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      p[2 * j + 0] = (q[j] & 0x00ff00ffu) | mag;
      p[2 * j + 1] = ((q[j] >> 8) & 0x00ff00ffu) | mag;
    }
  } else {
    // Codes 0..255 are exact in bf16: the upper half of the float32 bits.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t u = q[j];
      const uint32_t f0 = __float_as_uint((float)(u & 0xffu));
      const uint32_t f1 = __float_as_uint((float)((u >> 8) & 0xffu));
      const uint32_t f2 = __float_as_uint((float)((u >> 16) & 0xffu));
      const uint32_t f3 = __float_as_uint((float)(u >> 24));
      p[2 * j + 0] = perm(f2, f0, 0x07060302u);
      p[2 * j + 1] = perm(f3, f1, 0x07060302u);
    }
  }
}

template <bool SBF16>
__device__ __forceinline__ float half_bits_to_f32(uint32_t h) {
  return SBF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
}

// The partner of lane l in the butterfly step at offset O <= 8, fetched by
// DPP within a row of 16 lanes: l ^ 1 and l ^ 2 (quad permutes), the mirror
// of l within its 8 lanes (O = 4) and within its 16 lanes (O = 8). Each
// pairs l with a lane whose bit O differs and whose bits above O agree, so
// the four steps sum each group of 16 lanes exactly once.
template <int O>
__device__ __forceinline__ float dpp_partner(float v) {
  constexpr int ctrl = O == 8 ? 0x140 : (O == 4 ? 0x141 : (O == 2 ? 0x4e : 0xb1));
  return __builtin_bit_cast(float,
                            __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), ctrl, 0xf, 0xf, false));
}

// Lanes l and l + O (O = 32, 16) exchange a and b: after
// v_permlane{32,16}_swap(a, b), lanes with bit O clear hold (own a, partner's
// a) and lanes with bit O set hold (partner's b, own b), so the sum of the
// pair is own + partner's copy of the half the lane keeps.
template <int O>
__device__ __forceinline__ float swap_sum(float a, float b) {
  const unsigned ua = __builtin_bit_cast(unsigned, a), ub = __builtin_bit_cast(unsigned, b);
  const auto r = O == 32 ? __builtin_amdgcn_permlane32_swap(ua, ub, false, false)
                         : __builtin_amdgcn_permlane16_swap(ua, ub, false, false);
  return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
}

// Wave butterfly at lane offset O, then O/2, ..., 1, by cross-lane moves that
// stay in the VALU (permlane swaps across 32 and 16 lanes, DPP below). While
// more than one partial remains (CNT > 1), a step halves the set each lane
// carries: the lane with bit O clear keeps the lower half, its partner the
// upper half, and each adds the partner's copy of the half it keeps; after
// log2(NV) steps lane l carries partial l >> (6 - log2(NV)). Later steps sum
// that survivor. Float addition is commutative, so both lanes of a pair form
// the same sum, and every output sees the same tree over the 64 lanes
// whatever NV is.
template <int CNT, int O>
__device__ __forceinline__ void butterfly(float* acc, int lane) {
  if constexpr (O >= 1) {
    if constexpr (CNT > 1) {
      constexpr int H = CNT / 2;
      const bool up = (lane & O) != 0;
#pragma unroll
      for (int j = 0; j < H; ++j) {
        if constexpr (O >= 16) {
          acc[j] = swap_sum<O>(acc[j], acc[j + H]);
        } else {
          const float send = up ? acc[j] : acc[j + H];
          const float keep = up ? acc[j + H] : acc[j];
          acc[j] = keep + dpp_partner<O>(send);
        }
      }
      butterfly<H, O / 2>(acc, lane);
    } else {
      if constexpr (O >= 16)
        acc[0] = swap_sum<O>(acc[0], acc[0]);
      else
        acc[0] += dpp_partner<O>(acc[0]);
      butterfly<1, O / 2>(acc, lane);
    }
  }
}

// Weight sets of one launch: parts share x (and K, bits, group size, dtypes);
// part i owns workgroups [wg0, next part's wg0). With GU the launch has two
// parts of equal N (gate, up) and every workgroup owns the same rows of both.
struct GemvParts {
  const uint32_t* w[kGemvMaxParts];
  const uint16_t* scales[kGemvMaxParts];
  const uint16_t* biases[kGemvMaxParts];
  void* out[kGemvMaxParts];
  const void* bias[kGemvMaxParts];  // Linear::forward's bias per part, or nullptr
  int bdt[kGemvMaxParts];
  int N[kGemvMaxParts];
  int wg0[kGemvMaxParts];
  int nparts;
  int ydt;  // dtype the products are rounded to before a bias is added
  int act;  // GU: the gated MLP's activation (ACT_SILU, ACT_GELU_APPROX)
};

// Gather mode (gather_qmm): workgroup b computes rows [rb*R, rb*R+R) of
// pair p = b / nrb; pair p's batch coordinates over `shape` give the offset
// of its [M, K] activation block in x (strides xs) and of its expert id in
// idx (strides is); the expert selects w/scales/biases slice e of part 0
// (strides ew, es). An id outside [-E, E) (negative ids count from the end)
// gives zero rows.
constexpr int kGatherMaxDims = 8;
constexpr int kModeOne = 0, kModeParts = 1, kModeGather = 2;
struct GemvGather {
  const void* idx;
  int idx_signed, E, nrb, nd;
  int shape[kGatherMaxDims];
  int64_t xs[kGatherMaxDims], is[kGatherMaxDims];
  int64_t ew, es;  // words per expert in w; halves per expert in scales/biases
};

// RT rows per workgroup: R rows of one part, or (GU) R = RT/2 rows of the
// gate and the same R rows of the up projection, stored as act(gate)*up.
// MODE: kModeOne (one part), kModeParts (several parts on one x) or
// kModeGather (gather mode: gth describes the pairs; otherwise it is unused).
template <int BITS, bool XBF16, bool SBF16, int M, int RT, int I, bool GU, int MODE>
__global__ __launch_bounds__(64 * kGemvMaxWaves) void gemv_kernel(
    const uint16_t* __restrict__ x, const GemvParts parts, const GemvGather gth, int odt, int Mrows,
    int K, int cshift) {
  constexpr int R = RT;
  constexpr int CPC = 128 / BITS;  // codes per chunk
  constexpr int NP = CPC / 2;      // operand pairs per chunk
  constexpr int NXV = CPC / 8;     // 16-byte activation loads per chunk
  constexpr int NV = R * M;        // partial sums per lane
  constexpr float OFF = GemvOff<BITS, XBF16>::value;
  static_assert(NV <= 64 && (NV & (NV - 1)) == 0, "partials must split evenly over lanes");

  __shared__ float red[kGemvMaxWaves][NV];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int nth = blockDim.x;
  const int nch = K / CPC;           // chunks per row
  const int wpr = nch * 4;           // words per row
  const int G = nch >> cshift;       // groups per row (cshift = log2(group_size / CPC))
  constexpr int RP = GU ? R / 2 : R;  // rows per part of this workgroup
  // This workgroup's part (GU: the gate's part; up is part 1), chosen by
  // selects over every slot of the table, so all kernel arguments are read
  // in one batch of scalar loads with no load depending on another.
  int part = 0;
  if constexpr (!GU && MODE == kModeParts) {
#pragma unroll
    for (int i = 1; i < kGemvMaxParts; ++i)
      part = (i < parts.nparts && (int)blockIdx.x >= parts.wg0[i]) ? i : part;
  }
  const uint32_t* wsel = parts.w[0];
  const uint16_t* ssel = parts.scales[0];
  const uint16_t* bsel = parts.biases[0];
  void* osel = parts.out[0];
  const void* bias_sel = parts.bias[0];
  int bdt_sel = parts.bdt[0], N_sel = parts.N[0], wg0_sel = parts.wg0[0];
  if constexpr (!GU && MODE == kModeParts) {
#pragma unroll
    for (int i = 1; i < kGemvMaxParts; ++i) {
      const bool t = part == i;
      wsel = t ? parts.w[i] : wsel;
      ssel = t ? parts.scales[i] : ssel;
      bsel = t ? parts.biases[i] : bsel;
      osel = t ? parts.out[i] : osel;
      bias_sel = t ? parts.bias[i] : bias_sel;
      bdt_sel = t ? parts.bdt[i] : bdt_sel;
      N_sel = t ? parts.N[i] : N_sel;
      wg0_sel = t ? parts.wg0[i] : wg0_sel;
    }
  }
  const int N = N_sel;
  int row0 = ((int)blockIdx.x - wg0_sel) * RP;
  // operand pointers of this workgroup (h = 1: the up projection under GU)
  const uint16_t* xp = x;
  const uint32_t* wp[2] = {wsel, GU ? parts.w[1] : wsel};
  const uint16_t* sp[2] = {ssel, GU ? parts.scales[1] : ssel};
  const uint16_t* bp[2] = {bsel, GU ? parts.biases[1] : bsel};
  void* outp = osel;
  if constexpr (MODE == kModeGather) {
    const int pair = (int)blockIdx.x / gth.nrb;
    row0 = ((int)blockIdx.x % gth.nrb) * RP;
    int64_t xo = 0, io = 0;
    int rem = pair;
    for (int d = gth.nd - 1; d >= 0; --d) {
      const int c = rem % gth.shape[d];
      rem /= gth.shape[d];
      xo += c * gth.xs[d];
      io += c * gth.is[d];
    }
    int64_t e = gth.idx_signed ? (int64_t) static_cast<const int32_t*>(gth.idx)[io]
                               : (int64_t) static_cast<const uint32_t*>(gth.idx)[io];
    if (e < 0) e += gth.E;
    outp = static_cast<char*>(outp) + (int64_t)pair * Mrows * N * (odt == DT_F32 ? 4 : 2);
    if (e < 0 || e >= gth.E) {  // uniform: zero rows, no loads
      for (int t = tid; t < RP * Mrows; t += nth) {
        const int r = t / Mrows, m = t % Mrows;
        if (row0 + r < N) store_from_f32(outp, odt, (int64_t)m * N + row0 + r, 0.f);
      }
      return;
    }
    xp = x + xo;
    wp[0] = wp[0] + e * gth.ew;
    sp[0] = sp[0] + e * gth.es;
    bp[0] = bp[0] + e * gth.es;
  }

  int cidx[I];
  bool live[I];
#pragma unroll
  for (int i = 0; i < I; ++i) {
    const int c = tid + i * nth;
    live[i] = c < nch;
    cidx[i] = live[i] ? c : nch - 1;  // clamped: every load stays in bounds
  }

  // ---- issue every load: activations, codes, scale/bias halves. Each
  // address is a row base (uniform across the wave) plus a 32-bit lane
  // offset, the form the scalar-base global loads take.
  const __amdgpu_buffer_rsrc_t bx = buffer_of(xp);
  // descriptors of the part (GU: [0] gate, [1] up)
  __amdgpu_buffer_rsrc_t bw[2], bs[2], bb[2];
#pragma unroll
  for (int h = 0; h < (GU ? 2 : 1); ++h) {
    bw[h] = buffer_of(wp[h]);
    bs[h] = buffer_of(sp[h]);
    bb[h] = buffer_of(bp[h]);
  }
  u32x4 xr[I][M][NXV];
#pragma unroll
  for (int i = 0; i < I; ++i)
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const int mm = m < Mrows ? m : Mrows - 1;
#pragma unroll
      for (int v = 0; v < NXV; ++v)
        xr[i][m][v] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(bx, cidx[i] * (CPC * 2) + v * 16, mm * K * 2, 0));
    }
  // Row by row (codes, then that row's scale and bias halves), so that row r
  // can be computed as soon as its own loads have landed.
  uint32_t q[R][I][4];
  uint32_t sr[R][I], br[R][I];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int h = GU && r >= RP ? 1 : 0;  // compile-time once unrolled
    const int n = row0 + r % RP < N ? row0 + r % RP : N - 1;
#pragma unroll
    for (int i = 0; i < I; ++i) {
      const u32x4 v = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(bw[h], cidx[i] * 16, n * wpr * 4, kCodeAux));
      q[r][i][0] = v[0];
      q[r][i][1] = v[1];
      q[r][i][2] = v[2];
      q[r][i][3] = v[3];
      const int go = (cidx[i] >> cshift) * 2;
      sr[r][i] = __builtin_amdgcn_raw_buffer_load_b16(bs[h], go, n * G * 2, 0);
      br[r][i] = __builtin_amdgcn_raw_buffer_load_b16(bb[h], go, n * G * 2, 0);
    }
  }

  // Nothing below may be scheduled above this point: every load of the wave
  // is in flight before the first one is waited for (one memory round trip).
  __builtin_amdgcn_sched_barrier(0);

  // ---- activations into pair order; X = sum of the chunk's activations
  uint32_t xw[I][M][NP];
  float X[I][M];
  const uint32_t one = XBF16 ? 0x3f803f80u : 0x3c003c00u;
#pragma unroll
  for (int i = 0; i < I; ++i)
#pragma unroll
    for (int m = 0; m < M; ++m) {
      // Lanes past the row end and rows m >= Mrows hold clamped (finite,
      // in-bounds) data: their sums are discarded, not masked here.
#pragma unroll
      for (int v = 0; v < NXV; ++v) {
        const u32x4 pv = permute_x<BITS>(xr[i][m][v]);
#pragma unroll
        for (int e = 0; e < 4; ++e) xw[i][m][4 * v + e] = pv[e];
      }
      float s = 0.f;
#pragma unroll
      for (int k = 0; k < NP; ++k) s = dot2<XBF16>(xw[i][m][k], one, s);
      X[i][m] = s;
    }

  uint32_t mag = XBF16 ? 0x43004300u : 0x64006400u;
  asm volatile("" : "+v"(mag));  // keep it in a VGPR (see chunk_pairs)

  float acc[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) acc[j] = 0.f;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int i = 0; i < I; ++i) {
      uint32_t p[NP];
      chunk_pairs<BITS, XBF16>(q[r][i], mag, p);
      const float sc = half_bits_to_f32<SBF16>(sr[r][i]);
      const float bp = fmaf(-OFF, sc, half_bits_to_f32<SBF16>(br[r][i]));
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float d = 0.f;
#pragma unroll
        for (int k = 0; k < NP; ++k) d = dot2<XBF16>(p[k], xw[i][m][k], d);
        // a select, not a branch: a branch would let the compiler sink this
        // row's loads into it, behind the waits for the other rows
        const float a = fmaf(bp, X[i][m], fmaf(sc, d, acc[r * M + m]));
        acc[r * M + m] = live[i] ? a : acc[r * M + m];
      }
    }

  // ---- wave butterfly over lane offsets 32..1
  butterfly<NV, 32>(acc, lane);
  constexpr int LNV = __builtin_ctz(NV);
  if ((lane & ((64 >> LNV) - 1)) == 0) red[wave][lane >> (6 - LNV)] = acc[0];
  __syncthreads();
  const int W = nth >> 6;
  if (!GU && tid < NV) {
    float s = red[0][tid];
    for (int v = 1; v < W; ++v) s += red[v][tid];
    const int r = tid / M, m = tid % M;
    const int n = row0 + r;
    const Epilogue epi{bias_sel, bdt_sel, parts.ydt};
    if (n < N && m < Mrows) store_from_f32(outp, odt, (int64_t)m * N + n, epi(s, n));
  }
  if (GU && tid < NV / 2) {  // partial j = r*M + m: gate rows first, then up rows
    float g = red[0][tid], u = red[0][tid + NV / 2];
    for (int v = 1; v < W; ++v) {
      g += red[v][tid];
      u += red[v][tid + NV / 2];
    }
    const int r = tid / M, m = tid % M;
    const int n = row0 + r;
    const Epilogue eg{parts.bias[0], parts.bdt[0], parts.ydt}, eu{parts.bias[1], parts.bdt[1], parts.ydt};
    if (n < N && m < Mrows)
      store_from_f32(parts.out[0], odt, (int64_t)m * N + n, act_mul(eg(g, n), eu(u, n), odt, parts.act));
  }
}

struct GemvPlan {
  int waves, I, R;
};

GemvPlan plan_gemv(int N, int K, int bits) {
  const int nch = K * bits / 128;
  int I = 1;
  while ((nch + 64 * I - 1) / (64 * I) > kGemvMaxWaves) ++I;
  const int waves = (nch + 64 * I - 1) / (64 * I);
  int R = I == 1 ? kGemvRMax : (I == 2 ? 4 : 2);
  while (R > 2 && (int64_t)((N + R - 1) / R) * waves < kGemvWaves) R >>= 1;
  // measured: 4 rows per workgroup with twice the waves beats 8 on the
  // Llama-3-8B shapes (gate 8.84 -> 8.63 us), while 2 rows instead of 4
  // costs 11% on the Llama-3.2-1B layer at M = 4
  while (R > 4 && (int64_t)((N + R - 1) / R) * waves < kGemvWavesWide) R >>= 1;
  return {waves, I, R};
}

struct GemvLaunch {
  const QmvArgs* a;  // shared fields (x, dtypes, M, K, gs, bits, stream) from a[0]
  GemvParts parts;
  int total_wgs;
  bool gu;
  GemvGather gth;  // idx == nullptr unless gather mode
  int64_t pairs;   // gather mode: number of (activation block, expert) pairs
};

template <int BITS, bool XBF16, bool SBF16, int M, int R, int I>
hipError_t launch_one(const GemvLaunch& L, const GemvPlan& p) {
  constexpr int CPC = 128 / BITS;
  const QmvArgs& a = *L.a;
  const int cshift = __builtin_ctz(a.gs / CPC);
  if (L.gu) {
    if constexpr (2 * R * M <= 64)
      hipLaunchKernelGGL((gemv_kernel<BITS, XBF16, SBF16, M, 2 * R, I, true, kModeParts>), dim3(L.total_wgs),
                         dim3(64 * p.waves), 0, a.stream, (const uint16_t*)a.x, L.parts, L.gth, a.odt,
                         a.M, a.K, cshift);
    else
      return hipErrorInvalidValue;
  } else {
    if (L.gth.idx != nullptr)
      hipLaunchKernelGGL((gemv_kernel<BITS, XBF16, SBF16, M, R, I, false, kModeGather>), dim3(L.total_wgs),
                         dim3(64 * p.waves), 0, a.stream, (const uint16_t*)a.x, L.parts, L.gth, a.odt, a.M,
                         a.K, cshift);
    else if (L.parts.nparts > 1)
      hipLaunchKernelGGL((gemv_kernel<BITS, XBF16, SBF16, M, R, I, false, kModeParts>), dim3(L.total_wgs),
                         dim3(64 * p.waves), 0, a.stream, (const uint16_t*)a.x, L.parts, L.gth, a.odt, a.M,
                         a.K, cshift);
    else
      hipLaunchKernelGGL((gemv_kernel<BITS, XBF16, SBF16, M, R, I, false, kModeOne>), dim3(L.total_wgs),
                         dim3(64 * p.waves), 0, a.stream, (const uint16_t*)a.x, L.parts, L.gth, a.odt, a.M,
                         a.K, cshift);
  }
  return hipGetLastError();
}

template <int BITS, bool XBF16, bool SBF16, int M>
hipError_t launch_m(const GemvLaunch& a, const GemvPlan& p) {
  if (p.I == 1) {
    // At M = 8 the activations take 8x16 registers: at most 4 rows per
    // workgroup. (R does not change any output's summation order.)
    if constexpr (M == 8) {
      if (p.R >= 4) return launch_one<BITS, XBF16, SBF16, 8, 4, 1>(a, p);
      return launch_one<BITS, XBF16, SBF16, 8, 2, 1>(a, p);
    } else {
      if (p.R == 16) return launch_one<BITS, XBF16, SBF16, M, 16, 1>(a, p);
      if (p.R == 8) return launch_one<BITS, XBF16, SBF16, M, 8, 1>(a, p);
      if (p.R == 4) return launch_one<BITS, XBF16, SBF16, M, 4, 1>(a, p);
      return launch_one<BITS, XBF16, SBF16, M, 2, 1>(a, p);
    }
  }
  if constexpr (M <= 2) {
    if (p.I == 2) {
      if (p.R == 4) return launch_one<BITS, XBF16, SBF16, M, 4, 2>(a, p);
      return launch_one<BITS, XBF16, SBF16, M, 2, 2>(a, p);
    }
  }
  if constexpr (M == 1) {
    if (p.I == 3) return launch_one<BITS, XBF16, SBF16, 1, 2, 3>(a, p);
    if (p.I == 4) return launch_one<BITS, XBF16, SBF16, 1, 2, 4>(a, p);
  }
  return hipErrorInvalidValue;
}

template <int BITS, bool XBF16, bool SBF16>
hipError_t launch_s(const GemvLaunch& L, const GemvPlan& p) {
  const int M = L.a->M;
  if (M == 1) return launch_m<BITS, XBF16, SBF16, 1>(L, p);
  if (M == 2) return launch_m<BITS, XBF16, SBF16, 2>(L, p);
  if (M <= 4) return launch_m<BITS, XBF16, SBF16, 4>(L, p);
  return launch_m<BITS, XBF16, SBF16, 8>(L, p);
}

template <int BITS, bool XBF16>
hipError_t launch_x(const GemvLaunch& L, const GemvPlan& p) {
  return L.a->sdt == DT_BF16 ? launch_s<BITS, XBF16, true>(L, p) : launch_s<BITS, XBF16, false>(L, p);
}

// Rows per workgroup actually launched (the instantiation launch_m picks).
int rows_launched(const GemvPlan& p, int M) {
  if (p.I == 1 && M > 4) return p.R >= 4 ? 4 : 2;
  return p.R;
}

hipError_t launch(GemvLaunch& L) {
  const QmvArgs& a = *L.a;
  int ntot = 0;
  for (int i = 0; i < L.parts.nparts; ++i) ntot += L.parts.N[i];
  GemvPlan p = plan_gemv(L.gu ? L.parts.N[0] : ntot, a.K, a.bits);
  if (L.gu)  // the gate and up rows of a workgroup share its partial-sum lanes
    while (p.R > 2 && 2 * rows_launched(p, a.M) * (a.M <= 2 ? a.M : (a.M <= 4 ? 4 : 8)) > 64) p.R >>= 1;
  const int R = rows_launched(p, a.M);
  if (L.gth.idx != nullptr) {
    L.gth.nrb = (L.parts.N[0] + R - 1) / R;
    const int64_t wgs = L.pairs * L.gth.nrb;
    if (wgs > 0x7fffffff) return hipErrorInvalidValue;
    L.total_wgs = (int)wgs;
    L.parts.wg0[0] = 0;
    const bool xbf16 = a.xdt == DT_BF16;
    if (a.bits == 4) return xbf16 ? launch_x<4, true>(L, p) : launch_x<4, false>(L, p);
    return xbf16 ? launch_x<8, true>(L, p) : launch_x<8, false>(L, p);
  }
  L.total_wgs = 0;
  for (int i = 0; i < L.parts.nparts; ++i) {
    L.parts.wg0[i] = L.total_wgs;
    if (!L.gu || i == 0) L.total_wgs += (L.parts.N[i] + R - 1) / R;
  }
  if (L.gu) L.parts.wg0[1] = 0;
  const bool xbf16 = a.xdt == DT_BF16;
  if (a.bits == 4) return xbf16 ? launch_x<4, true>(L, p) : launch_x<4, false>(L, p);
  return xbf16 ? launch_x<8, true>(L, p) : launch_x<8, false>(L, p);
}

void set_part(GemvParts& P, int i, const QmvArgs& a) {
  P.w[i] = (const uint32_t*)a.w;
  P.scales[i] = (const uint16_t*)a.scales;
  P.biases[i] = (const uint16_t*)a.biases;
  P.out[i] = a.out;
  P.bias[i] = a.bias;
  P.bdt[i] = a.bdt;
  P.N[i] = a.N;
  P.ydt = a.ydt;
}

}  // namespace

bool gemv_fits(int64_t M, int64_t N, int64_t K, int bits, int gs) {
  const int64_t lim = (int64_t)1 << 31;  // byte offsets are 32-bit signed
  return N * K * bits / 8 < lim && M * K * 2 < lim && N * (K / gs) * 2 < lim;
}

int gemv_max_m(int K, int bits) {
  const int I = plan_gemv(1, K, bits).I;
  return I == 1 ? kGemvMaxM1 : (I == 2 ? 2 : (I <= 4 ? 1 : 0));
}

hipError_t launch_gemv(const QmvArgs& a) {
  if (a.M < 1 || a.M > gemv_max_m(a.K, a.bits)) return hipErrorInvalidValue;
  GemvLaunch L{&a, {}, 0, false, {}, 0};
  L.parts.nparts = 1;
  set_part(L.parts, 0, a);
  return launch(L);
}

hipError_t launch_gemv_multi(const QmvArgs* a, int n) {
  if (n < 1 || n > kGemvMaxParts || a[0].M < 1 || a[0].M > gemv_max_m(a[0].K, a[0].bits))
    return hipErrorInvalidValue;
  GemvLaunch L{&a[0], {}, 0, false, {}, 0};
  L.parts.nparts = n;
  for (int i = 0; i < n; ++i) set_part(L.parts, i, a[i]);
  return launch(L);
}

hipError_t launch_gemv_gate_up(const QmvArgs& gate, const QmvArgs& up, int act) {
  if (gate.M < 1 || gate.M > gemv_max_m(gate.K, gate.bits) || gate.N != up.N) return hipErrorInvalidValue;
  GemvLaunch L{&gate, {}, 0, true, {}, 0};
  L.parts.nparts = 2;
  L.parts.act = act;
  set_part(L.parts, 0, gate);
  set_part(L.parts, 1, up);
  return launch(L);
}

hipError_t launch_gemv_gather(const QmvArgs& a, const GatherArgs& g) {
  if (a.M < 1 || a.M > gemv_max_m(a.K, a.bits) || g.nd > kGatherMaxDims) return hipErrorInvalidValue;
  GemvLaunch L{&a, {}, 0, false, {}, g.pairs};
  L.parts.nparts = 1;
  set_part(L.parts, 0, a);
  L.gth.idx = g.idx;
  L.gth.idx_signed = g.idx_signed ? 1 : 0;
  L.gth.E = g.E;
  L.gth.nd = g.nd;
  for (int d = 0; d < g.nd; ++d) {
    L.gth.shape[d] = g.shape[d];
    L.gth.xs[d] = g.xs[d];
    L.gth.is[d] = g.is[d];
  }
  L.gth.ew = (int64_t)a.N * a.K * a.bits / 32;
  L.gth.es = (int64_t)a.N * (a.K / a.gs);
  return launch(L);
}

}  // namespace kh
