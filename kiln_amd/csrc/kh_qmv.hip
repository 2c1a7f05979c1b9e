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
//   X[m,g]    = sum_{k in g} x[m,k]                        (MFMA against ones, fp32 accumulate)
// OFF + q is exactly representable in the MFMA input type: it is built by
// OR-ing the code into the mantissa of OFF (bf16: OFF = 128, 7-bit mantissa;
// f16: OFF = 1024, 10-bit mantissa), except 8-bit codes with bf16 activations,
// which go through an exact int->float conversion with OFF = 0.
//
// Work decomposition. One workgroup owns RT 16-row output tiles (MFMA column
// tiles; RT = 4, 2 or 1, as many as still leave enough workgroups) and all
// M <= 64 activation rows; its RT*KS waves are (row tile, K slice) pairs, so
// the staged activations are shared by RT row tiles. A block is 16 bytes per lane: the four lane groups of a wave read 4
// consecutive words each, 64 contiguous bytes per output row per load
// instruction (128 codes at 4 bits, 64 at 8). MFMA step j of a block takes
// word j (4-bit) or words 2j, 2j+1 (8-bit) from every lane group.
//
// When a block spans NC > 1 quantization groups (4-bit gs32/gs64, 8-bit
// gs32), lane groups of different groups must not share an accumulator. Each
// group ("chain") is given its own D rows instead: activation rows are packed
// as (chain, m) into the 16 MFMA rows, and the A operand of a row is the
// activation for lane groups of that row's chain and zero for the others
// (zero lanes read a zero area of LDS). At M = 1 one MFMA per step serves
// every chain; larger M uses more row tiles. Each D element sees the same
// inputs whatever the tiling, so results do not depend on M.
//
// Per workgroup the activations of the current windows are staged in LDS,
// permuted into the MFMA pair order, with the raw scale/bias halves of the
// workgroup's rows. The first chunk of code loads is issued
// before staging so both overlap. Final sums: for every output, chains in
// ascending order, and within a chain the KS slice partials in slice order.
// KS depends only on (N, K, group_size, bits), so every output's summation
// order is independent of M: row r of the result is bitwise identical for
// every M <= 64.
//
// MFMA v_mfma_f32_16x16x32_{bf16,f16}: A = activations (16 rows x 32 k),
// B = codes (32 k x 16 n). Lane l supplies row/column l%16 and the eight k of
// block l/16; D lane l holds column l%16, rows 4*(l/16)+0..3.
#include "kh_common.h"
#include "kh_kernels.h"

namespace kh {

template <int BITS, bool XBF16>
struct CodeOffset {
  static constexpr float value = (BITS == 8 && XBF16) ? 0.0f : (XBF16 ? 128.0f : 1024.0f);
};

// Eight codes (one 4-bit word, or two 8-bit words) -> B operand, values OFF + q.
// `mag` is the OFF bit pattern (bf16 0x4300 = 128.0, f16 0x6400 = 1024.0 in
// both halves) held in a VGPR, so each (mask, or) pair becomes one
// v_and_or_b32 (a VOP3 may carry only one non-VGPR constant).
template <int BITS, bool XBF16>
__device__ __forceinline__ u32x4 codes_to_b(const uint32_t* q, uint32_t mag) {
  u32x4 r;
  const uint32_t MAG = mag;
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

template <bool SBF16>
__device__ __forceinline__ float half_to_f32(uint32_t h) {
  return SBF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
}

constexpr int kQmvInflight = 16;     // VGPRs per lane for one chunk of code loads
constexpr int kQmvWaveTarget = 4096; // waves per launch to aim for
constexpr int kQmvMaxWaves = 8;      // waves per workgroup (row tiles x K slices)
constexpr int kQmvMinWgs = 256;      // workgroups wanted before packing more row tiles per workgroup
constexpr int kQmvLds = 49152;       // LDS bytes per workgroup for staged operands

constexpr int pow2_floor(int v) {
  int p = 1;
  while (p * 2 <= v) p *= 2;
  return p;
}

// Geometry shared by host and device.
template <int BITS, int GS>
struct QmvGeom {
  static constexpr int CPW = 32 / BITS;         // codes per word
  static constexpr int CB = 16 * CPW;           // codes per block (per output row)
  static constexpr int SPB = CB / 32;           // MFMA steps per block
  static constexpr int WPS = 8 / CPW;           // words per step per lane
  static constexpr int KBB = CB / 8;            // 8-element k-blocks per block
  static constexpr int NC = CB >= GS ? CB / GS : 1;   // groups (chains) per block
  static constexpr int BPG = GS > CB ? GS / CB : 1;   // blocks per group
  static constexpr int LGC = 4 / NC;            // lane groups per chain
  static constexpr int U = kQmvInflight / 8; // blocks per load chunk (two chunks in flight)
};

struct QmvPlan {
  int rt;      // 16-row output tiles per workgroup
  int ks;      // K slices per workgroup (waves = rt * ks)
  int nct;     // chains per row tile
  int tiles;   // MFMA row tiles
  int wu;      // units (BPG blocks) per slice staged per round (power of two)
  int batch;   // slices staged together (power of two, divides ks)
  size_t lds;  // dynamic LDS bytes
};

static int ceil_div(int a, int b) { return (a + b - 1) / b; }

template <int BITS, int GS>
static QmvPlan plan_qmv_t(int M, int N, int K) {
  using Gm = QmvGeom<BITS, GS>;
  const int NU = ceil_div(K, Gm::CB) / Gm::BPG;  // units per row
  const int tiles16 = ceil_div(N, 16);
  int rt = 4;
  while (rt > 1 && tiles16 / rt < kQmvMinWgs) rt /= 2;
  int ks = 1;
  while (rt * ks * 2 <= kQmvMaxWaves && ceil_div(tiles16, rt) * rt * ks * 2 <= kQmvWaveTarget &&
         NU / (ks * 2) >= 2)
    ks *= 2;
  const int rows = 16 * rt;
  int nct = 1;
  if (M <= 16) nct = pow2_floor(16 / M) < Gm::NC ? pow2_floor(16 / M) : Gm::NC;
  const int mt = 16 / nct;
  int mtiles = 1;  // m tiles, rounded up to a power of two (extra tiles see only rows >= M)
  while (mtiles < ceil_div(M, mt)) mtiles *= 2;
  const int tiles = (Gm::NC / nct) * mtiles;
  // LDS per staged unit: activations and raw scale/bias halves.
  const size_t per_unit = (size_t)Gm::BPG * Gm::CB * M * 2 + (size_t)rows * Gm::NC * 4;
  int batch = ks;
  while (batch > 1 && per_unit * batch > kQmvLds) batch /= 2;
  int wu = pow2_floor((int)(kQmvLds / (per_unit * batch)) > 0 ? (int)(kQmvLds / (per_unit * batch)) : 1);
  while (wu > 1 && wu / 2 >= ceil_div(NU, ks)) wu /= 2;
  size_t lds = (size_t)batch * wu * per_unit + (size_t)Gm::SPB * M * 16;
  const size_t red = (size_t)rt * ks * 64 * 16 + (size_t)M * rows * 4;
  if (red > lds) lds = red;
  return {rt, ks, nct, tiles, wu, batch, lds};
}

template <int BITS, int GS, bool XBF16, bool SBF16, int TILES>
__global__ __launch_bounds__(64 * kQmvMaxWaves) void qmv_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ w,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    void* __restrict__ out, int odt, int M, int N, int K, int RT, int nct, int wu, int batch, Epilogue epi) {
  using Gm = QmvGeom<BITS, GS>;
  constexpr int CB = Gm::CB, SPB = Gm::SPB, WPS = Gm::WPS, KBB = Gm::KBB;
  constexpr int NC = Gm::NC, BPG = Gm::BPG, LGC = Gm::LGC, U = Gm::U;
  constexpr float OFF = CodeOffset<BITS, XBF16>::value;

  extern __shared__ __align__(16) unsigned char smem[];

  const int tid = threadIdx.x;
  const int nthreads = blockDim.x;
  const int lrt = __builtin_ctz(RT);
  const int KS = (nthreads >> 6) >> lrt;        // K slices
  const int lks = __builtin_ctz(KS);
  const int ROWS = RT * 16;                     // output rows of this workgroup
  const int lrows = lrt + 4;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rt = wave & (RT - 1);               // row tile of this wave
  const int ks = wave >> lrt;                   // K slice of this wave
  const int col = lane & 15;
  const int lg = lane >> 4;
  const int row0 = blockIdx.x * ROWS;
  const int n = row0 + rt * 16 + col;
  const int nc = n < N ? n : N - 1;             // clamped: every weight load is in bounds
  const int G = K / GS;
  const int WR = K / Gm::CPW;                   // words per row
  const int NU = ((K + CB - 1) / CB) / BPG;     // units (BPG blocks) per row
  const int mt = 16 / nct;                      // rows per chain in a tile
  const int cgroups = NC / nct;                 // chain groups
  const int lwu = __builtin_ctz(wu), lbatch = __builtin_ctz(batch);

  // LDS for one staging step, `batch` slices x `wu` units, slot = sb_i*wu + ul:
  //   xs  [slot][BPG*KBB][M] u32x4   permuted activations
  //   sbh [slot][ROWS][NC]   uint32  scale | bias << 16 (raw halves)
  // then the zero area [SPB][M] u32x4.
  const int xs_u = BPG * KBB * M;
  const int nslots = batch * wu;
  u32x4* xs = reinterpret_cast<u32x4*>(smem);
  uint32_t* sbh = reinterpret_cast<uint32_t*>(xs + (size_t)nslots * xs_u);
  u32x4* zero = reinterpret_cast<u32x4*>(sbh + (size_t)nslots * ROWS * NC);

  // Units of slice k: [(NU*k) >> lks, (NU*(k+1)) >> lks).
  const int r0 = (NU * ks) >> lks;
  const int r1 = (NU * (ks + 1)) >> lks;
  const int longest = (NU + KS - 1) >> lks;

  // Lane roles per tile: A row = col; the lane's D rows 4*lg..4*lg+3 belong
  // to one chain because mt is a multiple of 4.
  int a_off[TILES];    // u32x4 offset of this lane's A operand inside a block (-1: zero lane)
  int d_chain[TILES];  // chain of this lane's D rows
#pragma unroll
  for (int t = 0; t < TILES; ++t) {
    const int cg = t % cgroups, mtile = t / cgroups;
    const int ca = cg * nct + col / mt, ma = mtile * mt + col % mt;
    const bool live = (lg / LGC) == ca && ma < M;
    a_off[t] = live ? (lg * SPB) * M + ma : -1;  // k-block lg*SPB + j, step j
    d_chain[t] = cg * nct + (4 * lg) / mt;
  }

  const uint32_t* wrow = w + (int64_t)nc * WR;
  uint32_t mag = XBF16 ? 0x43004300u : 0x64006400u;
  asm volatile("" : "+v"(mag));  // keep it in a VGPR (see codes_to_b)
  const uint32_t one = XBF16 ? 0x3f803f80u : 0x3c003c00u;  // 1.0 in both halves
  const u32x4 ones = u32x4{one, one, one, one};

  f32x4 acc[TILES];
#pragma unroll
  for (int t = 0; t < TILES; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int i = tid; i < SPB * M; i += nthreads) zero[i] = u32x4{0u, 0u, 0u, 0u};

  const int nbatch = KS >> lbatch;
  const int nsteps = ((longest + wu - 1) >> lwu) * nbatch;
  for (int step = 0; step < nsteps; ++step) {
    const int off = (step / nbatch) << lwu;    // unit offset within every slice
    const int kb0 = (step % nbatch) << lbatch; // first slice staged in this step
    const bool mine = ks >= kb0 && ks < kb0 + batch;
    const int my_units = mine ? min(wu, r1 - (r0 + off)) : 0;
    const int my_blocks = my_units * BPG;

    // ---- first two chunks of code loads, issued before staging
    uint32_t qa[U][4], qb[U][4];
    auto load_chunk = [&](uint32_t (&q)[U][4], int c0) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int blk = (r0 + off) * BPG + min(c0 + u, max(my_blocks - 1, 0));
        // a lane chunk past the row end (partial last block) reads the row's
        // last chunk instead; its activations are zero
        const int word = min(blk * 16 + lg * 4, WR - 4);
        const u32x4 v = *reinterpret_cast<const u32x4*>(wrow + word);
        q[u][0] = v[0];
        q[u][1] = v[1];
        q[u][2] = v[2];
        q[u][3] = v[3];
      }
    };
    if (my_blocks > 0) load_chunk(qa, 0);
    if (my_blocks > U) load_chunk(qb, U);

    // ---- stage activations and scale/bias halves for the batch's units
    __syncthreads();
    {
      constexpr int LKB = __builtin_ctz(BPG * KBB);
      const int items = (nslots << LKB);        // (slot, kb); rows m looped inside
      for (int it = tid; it < items; it += nthreads) {
        const int kb = it & (BPG * KBB - 1);
        const int slot = it >> LKB;
        const int ul = slot & (wu - 1), sb_i = slot >> lwu;
        const int k_sl = kb0 + sb_i;
        const int unit = ((NU * k_sl) >> lks) + off + ul;
        const int uend = (NU * (k_sl + 1)) >> lks;
        const int k = (unit * BPG * KBB + kb) * 8;
        const bool ok = unit < uend && k < K;
        u32x4* dst = xs + (size_t)slot * xs_u + kb * M;
        for (int m = 0; m < M; ++m)
          dst[m] = ok ? permute_x<BITS>(*reinterpret_cast<const u32x4*>(x + (int64_t)m * K + k))
                      : u32x4{0u, 0u, 0u, 0u};
      }
      constexpr int LNC = __builtin_ctz(NC);
      const int sitems = (nslots * ROWS) << LNC;  // (slot, row, chain)
      for (int it = tid; it < sitems; it += nthreads) {
        const int c = it & (NC - 1);
        const int ul = (it >> LNC) & (wu - 1);
        const int row = (it >> (LNC + lwu)) & (ROWS - 1);
        const int sb_i = it >> (LNC + lwu + lrows);
        const int k_sl = kb0 + sb_i;
        const int unit = ((NU * k_sl) >> lks) + off + ul;
        const int uend = (NU * (k_sl + 1)) >> lks;
        const int g = unit * NC + c;
        const int rn = min(row0 + row, N - 1);
        uint32_t e = 0u;
        if (unit < uend && g < G)
          e = (uint32_t)scales[(int64_t)rn * G + g] | ((uint32_t)biases[(int64_t)rn * G + g] << 16);
        sbh[((size_t)((sb_i << lwu) + ul) * ROWS + row) * NC + c] = e;
      }
    }
    __syncthreads();

    // ---- stream this wave's code blocks
    const int slot0 = (ks - kb0) * wu;
    static_assert(BPG == 1 || TILES <= 4, "chains spanning blocks keep one D per tile");
    f32x4 D[TILES], DX[TILES];  // persist across the BPG blocks of a group
    auto compute_chunk = [&](uint32_t (&q)[U][4], int c0) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int b = c0 + u;
        if (b >= my_blocks) continue;  // wave-uniform
        const int ul = b / BPG, bib = b % BPG;
        u32x4 B[SPB];
#pragma unroll
        for (int j = 0; j < SPB; ++j) B[j] = codes_to_b<BITS, XBF16>(&q[u][j * WPS], mag);
        const int slot = slot0 + ul;
        const u32x4* xunit = xs + (size_t)slot * xs_u + bib * KBB * M;
        const uint32_t* sbu = sbh + ((size_t)slot * ROWS + rt * 16 + col) * NC;
#pragma unroll
        for (int t = 0; t < TILES; ++t) {
          if (bib == 0) D[t] = DX[t] = f32x4{0.f, 0.f, 0.f, 0.f};
          const u32x4* ap = a_off[t] >= 0 ? xunit + a_off[t] : zero;
#pragma unroll
          for (int j = 0; j < SPB; ++j) {
            const u32x4 a = ap[j * M];
            D[t] = mfma<XBF16>(a, B[j], D[t]);
            DX[t] = mfma<XBF16>(a, ones, DX[t]);  // group sums X of the same rows
          }
          if (bib == BPG - 1) {
            const uint32_t e = sbu[d_chain[t]];
            const float sc = half_to_f32<SBF16>(e & 0xffffu);
            const float bp = fmaf(-OFF, sc, half_to_f32<SBF16>(e >> 16));
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              acc[t][i] = fmaf(sc, D[t][i], acc[t][i]);
              acc[t][i] = fmaf(bp, DX[t][i], acc[t][i]);
            }
          }
        }
      }
    };
    for (int c0 = 0; c0 < my_blocks; c0 += 2 * U) {
      compute_chunk(qa, c0);
      if (c0 + 2 * U < my_blocks) load_chunk(qa, c0 + 2 * U);
      if (c0 + U < my_blocks) {
        compute_chunk(qb, c0 + U);
        if (c0 + 3 * U < my_blocks) load_chunk(qb, c0 + 3 * U);
      }
    }
  }

  // ---- final sums per output: chains ascending, K slices in order
  __syncthreads();
  f32x4* red = reinterpret_cast<f32x4*>(smem);                       // [waves][64]
  float* outacc = reinterpret_cast<float*>(red + (size_t)nthreads);  // [M][ROWS]
  for (int i = tid; i < M * ROWS; i += nthreads) outacc[i] = 0.f;
#pragma unroll
  for (int t = 0; t < TILES; ++t) {
    __syncthreads();
    red[tid] = acc[t];
    __syncthreads();
    const int mtile = t / cgroups;
    for (int it = tid; it < 16 * ROWS; it += nthreads) {
      const int r_in = it >> lrows, row = it & (ROWS - 1);  // (row within chain block, output row)
      const int m = mtile * mt + r_in;
      if (r_in < mt && m < M) {
        const int tr = row >> 4, nl = row & 15;
        float s = outacc[m * ROWS + row];
        for (int cl = 0; cl < nct; ++cl) {
          const int r = cl * mt + r_in;  // D row
          const int ln = (r >> 2) * 16 + nl, el = r & 3;
          for (int k2 = 0; k2 < KS; ++k2) s += red[((k2 << lrt) + tr) * 64 + ln][el];
        }
        outacc[m * ROWS + row] = s;
      }
    }
  }
  __syncthreads();
  for (int i = tid; i < M * ROWS; i += nthreads) {
    const int m = i >> lrows, row = i & (ROWS - 1);
    const int nn = row0 + row;
    if (nn < N) store_from_f32(out, odt, (int64_t)m * N + nn, epi(outacc[i], nn));
  }
}

template <int BITS, int GS, bool XBF16, bool SBF16>
static hipError_t launch_tiles(const QmvArgs& a) {
  const QmvPlan p = plan_qmv_t<BITS, GS>(a.M, a.N, a.K);
  const dim3 grid((a.N + 16 * p.rt - 1) / (16 * p.rt)), block(64 * p.rt * p.ks);
#define KH_QMV_LAUNCH(TV)                                                                      \
  hipLaunchKernelGGL((qmv_kernel<BITS, GS, XBF16, SBF16, TV>), grid, block, p.lds, a.stream,  \
                     (const uint16_t*)a.x, (const uint32_t*)a.w, (const uint16_t*)a.scales,   \
                     (const uint16_t*)a.biases, a.out, a.odt, a.M, a.N, a.K, p.rt, p.nct, p.wu, p.batch, a.epi())
  switch (p.tiles) {
    case 1: KH_QMV_LAUNCH(1); break;
    case 2: KH_QMV_LAUNCH(2); break;
    case 4: KH_QMV_LAUNCH(4); break;
    case 8: if constexpr (QmvGeom<BITS, GS>::BPG == 1) { KH_QMV_LAUNCH(8); break; } else return hipErrorInvalidValue;
    case 16: if constexpr (QmvGeom<BITS, GS>::BPG == 1) { KH_QMV_LAUNCH(16); break; } else return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
#undef KH_QMV_LAUNCH
  return hipGetLastError();
}

template <int BITS, bool XBF16, bool SBF16>
static hipError_t launch_gs(const QmvArgs& a) {
  switch (a.gs) {
    case 32: return launch_tiles<BITS, 32, XBF16, SBF16>(a);
    case 64: return launch_tiles<BITS, 64, XBF16, SBF16>(a);
    default: return launch_tiles<BITS, 128, XBF16, SBF16>(a);
  }
}

template <int BITS, bool XBF16>
static hipError_t launch_st(const QmvArgs& a) {
  return a.sdt == DT_BF16 ? launch_gs<BITS, XBF16, true>(a) : launch_gs<BITS, XBF16, false>(a);
}

// Scales and biases must be float16 or bfloat16 here (float32 scales take the
// general kernel). Uses no device memory besides its arguments.
hipError_t launch_qmv(const QmvArgs& a) {
  const bool xbf16 = a.xdt == DT_BF16;
  if (a.bits == 4) return xbf16 ? launch_st<4, true>(a) : launch_st<4, false>(a);
  return xbf16 ? launch_st<8, true>(a) : launch_st<8, false>(a);
}

}  // namespace kh
