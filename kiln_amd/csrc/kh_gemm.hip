// kh_gemm.hip — quantized GEMM for gfx950, every M above the VALU-GEMV range.
//
// y[m, n] = sum_k x[m, k] * w[n, k], w = s[n, g(k)] * q[n, k] + b[n, g(k)]
// (quantized_matmul, transpose=true: crates/kiln-mlx/src/ops.rs:359-388).
//
// Numerics: as the prefill path of kh_qmm.hip. qmm_prep_x has written x as
// float16 rows scaled by an exact power of two (rscale = 2^e_m), permuted
// into the pair order of the code operand. Each weight is dequantised once,
// in registers, to float16 with one rounding, w16 = fma16(s, q, b), and the
// products accumulate in float32 (v_mfma_f32_16x16x32_f16). Outputs are
// multiplied back by rscale.
//
// Work decomposition. A workgroup of four waves owns a (16*MT) x 256 output
// tile and one K slice; the waves split N (64 columns each, four 16-column
// MFMA tiles), so every weight is dequantised exactly once. K is walked in
// stages of 128 codes:
//   - codes go from HBM straight into registers in MFMA operand layout
//     (lane (n, lg) holds 16 bytes of row n: one load per 16-row tile at 4
//     bits, two at 8 bits), prefetched three stages ahead, cached normally
//     (every row tile of the launch re-reads them);
//   - the activation tile of the stage (16*MT rows x 128 k, float16) is
//     copied HBM/L2 -> LDS by the direct global-to-LDS loads of gfx950 (each
//     instruction four whole rows, 1 KB contiguous), into a ring of LDS
//     buffers, row-major with the 16-byte blocks XOR-swizzled by row so the
//     MFMA operand reads are free of bank conflicts;
//   - one barrier per stage; a stage's loads go out in four parts, one
//     before each MFMA step of the stage three earlier (one wave per SIMD
//     would otherwise stall at issue with the matrix core idle), and the
//     weights of MFMA step j+1 are dequantised between the MFMAs of step j.
// K slices (split-K, chosen from N, K and M-tiles only) write float32
// partials that gemm_reduce sums in slice order, so results are
// deterministic. Tiles are ordered in bands of 4 m-tiles (m fastest within a
// band) and dealt to XCDs in consecutive runs, so the workgroups resident on
// one XCD share both the activation panels and the code rows in its L2.
#include "kh_common.h"
#include "kh_kernels.h"
#include "kh_lds.h"

namespace kh {

namespace {

typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 h2;

constexpr int kStage = 128;   // codes per K stage
constexpr int kWaves = 4;
constexpr int kNT = 4;        // 16-column tiles per wave
constexpr int kBN = kWaves * kNT * 16;  // 256
constexpr int kXcds = 8;
constexpr int kMaxMT = 8;     // largest m tile: 128 rows
constexpr int kCUs = 256;     // MI355X compute units
constexpr int kReduceParts = 4;
// epilogue store kinds
constexpr int kStPart = 0, kStBf16 = 1, kStF16 = 2, kStF32 = 3, kStAny = 4;

__device__ __forceinline__ f32x4 mfma_f16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// 16-bit scale/bias halves -> (v, v) float16 pair. bf16 values are converted
// through float32 to float16 (round to nearest even); scales and biases of
// the supported formats are far inside float16's normal range.
template <bool SF16>
__device__ __forceinline__ h2 half_pair(uint32_t h) {
  if constexpr (SF16) {
    return __builtin_bit_cast(h2, h | (h << 16));
  } else {
    const _Float16 v = (_Float16)bf16_bits_to_f32(h);
    return h2{v, v};
  }
}

// Stages kept in flight (measured on the Llama-3-8B shapes): 4 for the
// smallest tiles (latency-bound launches) and the largest (one wave per SIMD:
// the ring is what hides memory latency), 2 at 64 rows.
constexpr int kBandM = 4;     // m-tiles per band of the tile order (m fastest within a band)
constexpr int kSplitCap = 256;  // split-K target: workgroups per launch (one per CU)
// VALU ops scheduled after each MFMA when dequantising a step ahead
constexpr int kInterleave = 2;
constexpr int ring_depth(int bits, int mt) { return mt == 4 ? 2 : 4; }
// 16-column MFMA tiles per wave: tiles of up to 64 rows run as 128-column
// workgroups, so a launch has twice the workgroups and two of them share a
// CU, one wave's MFMAs running while another dequantises or waits (the
// Llama-3-8B linears at M = 64: 8-17% faster than 256-column workgroups).
// Each output accumulates over K in the same order whatever the width.
constexpr int nt_for(int mt) { return mt <= 4 ? kNT / 2 : kNT; }

// Scale/bias chunk: the groups of P stages (P*128 codes) of every row of the
// workgroup, copied to LDS by direct loads of SPIECE bytes.
template <int GS, int P, int BN, int KW>
struct ScaleChunk {
  static constexpr int GC = P * kStage / GS;            // groups per row
  static constexpr int BYTES = GC * 2;                  // per row and array
  // A piece never spans two stages (a stage is 2*128/GS bytes of a row), so
  // each piece lies wholly inside the row's groups or wholly past its end —
  // the row's valid groups end on a stage boundary.
  static constexpr int SPIECE = GS == 128 ? 2 : 4;      // direct-load size
  static constexpr int PIECES = BYTES / SPIECE;         // per row and array
  static_assert(PIECES * SPIECE == BYTES && (2 * kStage / GS) % SPIECE == 0, "pieces tile stages");
  // Direct loads of fewer than 4 bytes still write one dword per lane in LDS.
  static constexpr int SSTRIDE = SPIECE < 4 ? 4 : SPIECE;     // LDS bytes per piece
  static constexpr int LDS_BYTES = 2 * BN * PIECES * SSTRIDE;  // one chunk buffer
  // LDS byte offset of group g (within the chunk) of row `row`, array `arr`
  __device__ static constexpr int offset(int arr, int row, int g) {
    return ((arr * BN + row) * PIECES + g / (SPIECE / 2)) * SSTRIDE + (g % (SPIECE / 2)) * 2;
  }
  static constexpr int OPS = 2 * BN * PIECES / (64 * KW);  // direct loads per lane
  static_assert(OPS * 64 * KW == 2 * BN * PIECES, "every wave issues the same loads");
};

// One weight matrix of a launch: its work items are start .. start +
// cnt * (256 / BN) * nsplit - 1 of the launch (several parts sharing x, M, K
// and the kernel class run as one launch; each part's results are those of
// its own launch).
struct GemmPart {
  const uint32_t* w;
  const uint16_t* scales;
  const uint16_t* biases;
  float* part;
  void* out;
  int odt, N, kslice, tiles_n, tile0, cnt, nsplit, start;
  Epilogue epi;
};
constexpr int kGemmParts = 4;
struct GemmParts {
  GemmPart p[kGemmParts];
  int n, total;
};

// GR (grouped, gather_qmm): x holds the rows of every expert group, each
// group padded to whole m-tiles; gtab[0] is the number of m-tiles in use and
// gtab[1 + tm] the expert of m-tile tm (w, scales and biases are [E, N, ..]
// stacks); rowmap[m] is the output row of padded row m, or -1 for padding.
template <int BITS, bool SF16, int MT, int GS, int NT, bool GR>
__global__ __launch_bounds__(64 * kWaves) void gemm_kernel(
    const u32x4* __restrict__ xh, const float* __restrict__ rscale, GemmParts gp, int M, int K,
    const int* __restrict__ gtab, const int* __restrict__ rowmap) {
  // NT 16-column MFMA tiles per wave: 4 (a 256-column tile) or 2 (half of
  // one, for the last partial round of a launch)
  constexpr int KW = kWaves;               // waves per workgroup
  constexpr int MW = MT;                   // 16-row m-tiles per wave
  constexpr int BN = kWaves * NT * 16;
  constexpr int SUB = kBN / BN;           // workgroups per 256-column tile
  constexpr int BM = 16 * MT;
  constexpr int LW = BITS / 4;             // 16-byte code loads per lane per 16-row tile
  constexpr int SLOTS = 16 * BM;           // u32x4 activation slots per stage
  constexpr int DOPS = (SLOTS + 64 * KW - 1) / (64 * KW);  // activation loads per lane
  constexpr int P = ring_depth(BITS, MT);  // stages in flight
  using SC = ScaleChunk<GS, P, BN, KW>;
  constexpr int LGS = __builtin_ctz(GS);

  __shared__ u32x4 As[P][SLOTS];
  __shared__ __align__(16) unsigned char Ss[2][SC::LDS_BYTES];  // [chunk buf][scales|biases][row][piece]

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wc = wave;  // column group
  const int col = lane & 15, lg = lane >> 4;

  // XCD-aware tile order: workgroup b runs on XCD b % 8; the work items of
  // one XCD are consecutive in (split, tile, part of tile) order, with tiles
  // tile0 .. tile0+cnt-1 numbered m-tile-major, n fastest.
  // Grouped: only the m-tiles in use (a device-side count) are dealt out, so
  // they spread over all XCDs; the grid was sized for the most there can be.
  const int tiles_m = GR ? gtab[0] : (M + BM - 1) / BM;
  const int total = GR ? tiles_m * gp.p[0].tiles_n * SUB : gp.total;
  const int per = (total + kXcds - 1) / kXcds;
  if (GR && (int)blockIdx.x / kXcds >= per) return;
  int t = (blockIdx.x % kXcds) * per + blockIdx.x / kXcds;
  if (t >= total) return;
  // The part holding work item t (uniform), chosen by selects over every
  // slot of the part table: the kernel arguments are read in one batch of
  // scalar loads, none depending on another (a loop over the parts would
  // wait for each part's start before reading the next).
  GemmPart sel = gp.p[0];
#pragma unroll
  for (int i = 1; i < kGemmParts; ++i) {
    const bool take = i < gp.n && t >= gp.p[i].start;
    sel.w = take ? gp.p[i].w : sel.w;
    sel.scales = take ? gp.p[i].scales : sel.scales;
    sel.biases = take ? gp.p[i].biases : sel.biases;
    sel.part = take ? gp.p[i].part : sel.part;
    sel.out = take ? gp.p[i].out : sel.out;
    sel.odt = take ? gp.p[i].odt : sel.odt;
    sel.N = take ? gp.p[i].N : sel.N;
    sel.kslice = take ? gp.p[i].kslice : sel.kslice;
    sel.tiles_n = take ? gp.p[i].tiles_n : sel.tiles_n;
    sel.tile0 = take ? gp.p[i].tile0 : sel.tile0;
    sel.cnt = take ? gp.p[i].cnt : sel.cnt;
    sel.nsplit = take ? gp.p[i].nsplit : sel.nsplit;
    sel.start = take ? gp.p[i].start : sel.start;
    sel.epi.bias = take ? gp.p[i].epi.bias : sel.epi.bias;
    sel.epi.bdt = take ? gp.p[i].epi.bdt : sel.epi.bdt;
    sel.epi.ydt = take ? gp.p[i].epi.ydt : sel.epi.ydt;
  }
  t -= sel.start;
  const uint32_t* __restrict__ w = sel.w;
  const uint16_t* __restrict__ scales = sel.scales;
  const uint16_t* __restrict__ biases = sel.biases;
  float* __restrict__ part = sel.part;
  void* __restrict__ out = sel.out;
  const int odt = sel.odt, N = sel.N, kslice = sel.kslice, tiles_n = sel.tiles_n;
  const int tile0 = sel.tile0, cnt = sel.cnt, nsplit = sel.nsplit;
  const Epilogue epi = sel.epi;
  const int u0 = t % (cnt * SUB);
  const int sp = t / (cnt * SUB);
  const int tile = tile0 + u0 / SUB;
  int tn = tile % tiles_n, tm = tile / tiles_n;
  {
    // bands of kBandM m-tiles, m fastest within a band: the workgroups resident
    // on one XCD at a time share both activation panels and code rows in L2
    const int b0 = (tile / (kBandM * tiles_n)) * kBandM;
    const int bh = min(kBandM, tiles_m - b0);
    const int rr = tile - b0 * tiles_n;
    tm = b0 + rr % bh;
    tn = rr / bh;
  }

  if constexpr (GR) {
    const int64_t e = gtab[1 + tm];
    w += e * N * (K * BITS / 32);
    scales += e * N * (K >> LGS);
    biases += e * N * (K >> LGS);
  }
  const int m0 = tm * BM, n0 = tn * kBN + (u0 % SUB) * BN;
  const int k0 = sp * kslice;
  const int k1 = min(K, k0 + kslice);
  const int nst = (k1 - k0) / kStage;      // K and kslice are multiples of kStage
  const int G = K >> LGS;
  const int KB8 = K / 8;
  const int wpr = K * BITS / 32;           // words per row
  const int nchunks = (nst + P - 1) / P;

  // Rows of this lane's four code tiles (clamped: every load in bounds).
  int nrow[NT];
#pragma unroll
  for (int u = 0; u < NT; ++u) {
    const int n = n0 + wc * (NT * 16) + u * 16 + col;
    nrow[u] = n < N ? n : N - 1;
  }
  // The epilogue's per-row values (the activation row scale and, grouped,
  // the output row), loaded now so that their latency hides behind the main
  // loop rather than being paid at its end: lane l holds tile rows h*64+l.
  constexpr int RR = (BM + 63) / 64;
  float rsr[RR];
  int rmr[RR];
#pragma unroll
  for (int h = 0; h < RR; ++h) {
    const int m = m0 + h * 64 + lane;
    const bool in = h * 64 + lane < BM && m < M;
    rsr[h] = in ? rscale[m] : 0.f;
    if constexpr (GR) rmr[h] = in ? rowmap[m] : -1;
  }

  // ---- loaders (all in bounds: indices past the slice or the matrix are
  // clamped; what they fetch is never used)
  auto load_codes = [&](u32x4 (&q)[NT][LW], int st) {
    const int kc = k0 + st * kStage;
#pragma unroll
    for (int u = 0; u < NT; ++u) {
      const uint32_t* row = w + (int64_t)nrow[u] * wpr;
#pragma unroll
      for (int h = 0; h < LW; ++h) {
        const int code = kc + (BITS == 4 ? lg * 32 : h * 64 + lg * 16);
        const u32x4* src = reinterpret_cast<const u32x4*>(row + code * BITS / 32);
        q[u][h] = *src;
      }
    }
  };
  // Activation tile of a stage: row m's 16 blocks of 8 codes (256 bytes) at
  // slots m*16 + (kb ^ (m & 15)). One direct load fills 64 consecutive slots:
  // four whole rows, 1 KB of contiguous global memory; the XOR spreads the
  // 16 rows an MFMA operand read touches (same kb) over all LDS banks.
  auto load_acts = [&](int buf, int st) {
    const int kc8 = (k0 + st * kStage) >> 3;
#pragma unroll
    for (int d = 0; d < DOPS; ++d) {
      const int s = (d * KW + wave) * 64 + lane;
      const int sl = s < SLOTS ? s : SLOTS - 1;
      const int m = sl >> 4, kb = (sl & 15) ^ (m & 15);
      const int mm = m0 + m < M ? m0 + m : M - 1;
      if ((d * KW + wave) * 64 < SLOTS)  // wave-uniform
        __builtin_amdgcn_global_load_lds(
            (const void*)(xh + (int64_t)mm * KB8 + kc8 + kb),
            (lds_void*)&As[buf][(d * KW + wave) * 64], 16, 0, 0);
    }
  };
  // Scale/bias chunk c into buffer c & 1: lane op i = (array, row, piece),
  // consecutive lanes -> consecutive pieces of one row (contiguous memory).
  auto load_scales = [&](int c) {
    const int g0 = (k0 >> LGS) + c * SC::GC;
#pragma unroll
    for (int d = 0; d < SC::OPS; ++d) {
      const int i = (d * KW + wave) * 64 + lane;
      const int piece = i % SC::PIECES, row = (i / SC::PIECES) % BN, arr = i / (SC::PIECES * BN);
      const int n = n0 + row < N ? n0 + row : N - 1;
      // a piece past the row's last group (only in the last chunk of a slice
      // whose stage count is not a multiple of P, or past K) reads the
      // row's last piece instead: in bounds, never used
      const int gp = min(g0 + piece * (SC::SPIECE / 2), G - SC::SPIECE / 2);
      const uint16_t* src = (arr ? biases : scales) + (int64_t)n * G + gp;
      lds_void* dst = (lds_void*)&Ss[c & 1][((d * KW + wave) * 64) * SC::SSTRIDE];
      __builtin_amdgcn_global_load_lds((const void*)src, dst, SC::SPIECE, 0, 0);
    }
  };

  // Part j (of 4) of a stage's activation and code loads, for issuing a
  // stage's loads spread over the MFMA steps of the stage before.
  auto load_acts_part = [&](int buf, int st, int j) {
    const int kc8 = (k0 + st * kStage) >> 3;
#pragma unroll
    for (int d = j * (DOPS / 4); d < (j + 1) * (DOPS / 4); ++d) {
      const int s = (d * KW + wave) * 64 + lane;
      const int m = s >> 4, kb = (s & 15) ^ (m & 15);
      const int mm = m0 + m < M ? m0 + m : M - 1;
      __builtin_amdgcn_global_load_lds((const void*)(xh + (int64_t)mm * KB8 + kc8 + kb),
                                       (lds_void*)&As[buf][(d * KW + wave) * 64], 16, 0, 0);
    }
  };
  auto load_codes_part = [&](u32x4 (&q)[NT][LW], int st, int j) {
    if (j >= NT) return;
    const int kc = k0 + st * kStage;
    const uint32_t* row = w + (int64_t)nrow[j] * wpr;
#pragma unroll
    for (int h = 0; h < LW; ++h) {
      const int code = kc + (BITS == 4 ? lg * 32 : h * 64 + lg * 16);
      q[j][h] = *reinterpret_cast<const u32x4*>(row + code * BITS / 32);
    }
  };

  uint32_t mag = 0x64006400u;  // float16 1024.0 in both halves
  asm volatile("" : "+v"(mag));
  const h2 k1024 = h2{(_Float16)1024.f, (_Float16)1024.f};

  f32x4 acc[MW][NT];
#pragma unroll
  for (int i = 0; i < MW; ++i)
#pragma unroll
    for (int u = 0; u < NT; ++u) acc[i][u] = f32x4{0.f, 0.f, 0.f, 0.f};

  u32x4 q[P][NT][LW];  // code ring: slot p holds stage st with st % P == p

  // Issue order of vector-memory ops: scales(chunk 0); for t = 0..P-2:
  // activations(t), codes(t); then per stage st (p = st % P): wait for
  // activations(st), barrier (the buffers and slots of stage st-1, and at a
  // chunk start the scale buffer of chunk c-1, are free), activations(st+P-1),
  // scales(chunk c+1) if p == 0, codes(st+P-1), arithmetic of st. Clamped
  // indices keep this sequence free of branches, so the ops issued after
  // activations(st) are codes(st), P-2 stages of (activations, codes), and one
  // scale chunk unless p == 0: a compile-time count per p.
  constexpr int OPS = LW * NT;
  constexpr int BASE = OPS + (P - 2) * (DOPS + OPS);
  static_assert(BASE + SC::OPS < 64, "vmcnt holds 6 bits");
  // Spread issue (128- and 64-row tiles, one wave per SIMD): the loads of
  // stage st + P - 1 are issued in four parts, part j (activation loads
  // j*DOPS/4 .., code tile j) before MFMA step j of stage st, after the scale
  // chunk when p == 0. The last activation load of a stage is then followed
  // by its last code load and the P - 2 younger stages' loads, plus one scale
  // chunk when one of those was issued at p == 0 (1 <= p <= P - 2). The
  // prologue's stages go out in the plain order, which puts more ops after
  // their last activation load: the same counts only wait longer there.
  constexpr bool SPREAD = (MT == 8 || MT == 4) && DOPS % 4 == 0;
  // (code tile j goes out in part j: with NT = 2 parts 2 and 3 carry none)
  constexpr int WS0 = (NT == 4 ? LW : 0) + (P - 2) * (DOPS + OPS);
  // dequantisation a step ahead (measured 2-6% on the 4-bit gs64 prefill
  // shapes; group size 32 would spill with it)
  constexpr int IL = GS >= 64 ? kInterleave : 0;
  static_assert(WS0 + SC::OPS < 64, "vmcnt holds 6 bits");
  load_scales(0);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int t = 0; t < P - 1; ++t) {
    load_acts(t, min(t, nst - 1));
    __builtin_amdgcn_sched_barrier(0);
    load_codes(q[t], min(t, nst - 1));
    __builtin_amdgcn_sched_barrier(0);
  }

  for (int c = 0; c < nchunks; ++c) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int st = c * P + p;
      if constexpr (SPREAD) {
        if (p >= 1 && p <= P - 2)
          waitcnt_vm<WS0 + SC::OPS>();
        else
          waitcnt_vm<WS0>();
      } else {
        if (p == 0)
          waitcnt_vm<BASE>();
        else
          waitcnt_vm<BASE + SC::OPS>();
      }
      __builtin_amdgcn_s_barrier();
      const int pn = (p + P - 1) % P;  // slot and buffer of stage st + P - 1 (constant once unrolled)
      const int stn = min(st + P - 1, nst - 1);
      // The waits count the ops issued after a stage's last activation load,
      // so activation, scale and code loads leave in exactly this order (the
      // scheduler would otherwise move code loads above the activation load
      // of the same part, leaving that load outside the wait).
      auto issue = [&](int j) {  // part j of the spread issue
        if (j == 0 && p == 0) {
          load_scales(min(c + 1, nchunks - 1));
          __builtin_amdgcn_sched_barrier(0);
        }
        load_acts_part(pn, stn, j);
        __builtin_amdgcn_sched_barrier(0);
        load_codes_part(q[pn], stn, j);
        __builtin_amdgcn_sched_barrier(0);
      };
      if constexpr (!SPREAD) {
        load_acts(pn, stn);
        __builtin_amdgcn_sched_barrier(0);
        if (p == 0) load_scales(min(c + 1, nchunks - 1));
        __builtin_amdgcn_sched_barrier(0);
        load_codes(q[pn], stn);
      }
      // The waits above rely on program order of the vector memory ops.
      __builtin_amdgcn_sched_barrier(0);
      if (SPREAD && st >= nst) {  // uniform: nothing to compute, the loads still go out
#pragma unroll
        for (int j = 0; j < 4; ++j) issue(j);
      }
      if (st < nst) {  // uniform
        const unsigned char* sbuf = &Ss[c & 1][0];
        // this lane's scale and bias for each of its code runs in the stage
        // (one group per run), and the activation operands of step 0
        uint32_t sv[NT][LW], bv[NT][LW];
#pragma unroll
        for (int u = 0; u < NT; ++u)
#pragma unroll
          for (int h = 0; h < LW; ++h) {
            const int gl = (p * kStage + (BITS == 4 ? lg * 32 : h * 64 + lg * 16)) >> LGS;
            const int row = wc * (NT * 16) + u * 16 + col;
            sv[u][h] = lds_u16_nowait(sbuf + SC::offset(0, row, gl));
            bv[u][h] = lds_u16_nowait(sbuf + SC::offset(1, row, gl));
          }
        // activation operand (MFMA A layout: lane (row col, k-block lg)) of
        // m-tile i for step j, from the swizzled slot p
        u32x4 av[2][MW];
        auto read_a = [&](u32x4 (&a)[MW], int j) {
#pragma unroll
          for (int i = 0; i < MW; ++i) {
            const int m = i * 16 + col, kb = step_off<BITS>(j, lg) >> 3;
            a[i] = lds_b128_nowait(&As[p][m * 16 + (kb ^ (m & 15))]);
          }
        };
        read_a(av[0], 0);
        lds_wait_all();
#pragma unroll
        for (int u = 0; u < NT; ++u)
#pragma unroll
          for (int h = 0; h < LW; ++h) {
            ready(sv[u][h]);
            ready(bv[u][h]);
          }
#pragma unroll
        for (int i = 0; i < MW; ++i) ready(av[0][i]);
        // dequantised code operand (MFMA B layout) of each column tile for step j
        auto dequant = [&](u32x4 (&b)[NT], int j) {
#pragma unroll
          for (int u = 0; u < NT; ++u) {
            const int h = BITS == 4 ? 0 : (j >> 1);
            const uint32_t q0 = BITS == 4 ? q[p][u][0][j] : q[p][u][h][(j & 1) * 2];
            const uint32_t q1 = BITS == 4 ? 0u : q[p][u][h][(j & 1) * 2 + 1];
            uint32_t r[4];
            pairs_1024<BITS>(q0, q1, mag, r);
            const h2 s2 = half_pair<SF16>(sv[u][h]);
            const h2 b2 = half_pair<SF16>(bv[u][h]);
#pragma unroll
            for (int e = 0; e < 4; ++e)
              b[u][e] = __builtin_bit_cast(
                  uint32_t, __builtin_elementwise_fma(s2, __builtin_bit_cast(h2, r[e]) - k1024, b2));
          }
        };
        // IL: the operands of step j+1 are dequantised while the MFMAs of
        // step j run, interleaved by the scheduler (kInterleave VALU ops per MFMA)
        u32x4 bq[2][NT];
        if constexpr (IL > 0) dequant(bq[0], 0);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if constexpr (SPREAD) issue(j);
          if constexpr (IL == 0) dequant(bq[j & 1], j);
          // operands of step j were read during step j-1 (or above)
          if (j > 0) {
            lds_wait_all();
#pragma unroll
            for (int i = 0; i < MW; ++i) ready(av[j & 1][i]);
          }
          if (j < 3) read_a(av[(j + 1) & 1], j + 1);
          if constexpr (IL > 0)
            if (j < 3) dequant(bq[(j + 1) & 1], j + 1);
#pragma unroll
          for (int i = 0; i < MW; ++i)
#pragma unroll
            for (int u = 0; u < NT; ++u) acc[i][u] = mfma_f16(av[j & 1][i], bq[j & 1][u], acc[i][u]);
          if constexpr (IL > 0) {
#pragma unroll
            for (int i = 0; i < MW * NT; ++i) {
              __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
              __builtin_amdgcn_sched_group_barrier(0x002, IL, 0);  // then VALU
            }
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // ---- epilogue. D lane l holds column l%16, rows 4*(l/16)+e of each 16x16
  // tile. The tile goes through LDS (the activation ring, free once every
  // wave is past its last stage and no prefetch is in flight) as float32
  // rows of 256 columns, so that the stores leave as whole rows: 16-byte
  // blocks XOR-swizzled by row so the scattered writes spread over the banks.
  // Tiles taller than the ring holds go in passes of EP m-tiles.
  constexpr int RING_BYTES = P * SLOTS * 16;
  constexpr int EP_CAP = RING_BYTES / (16 * BN * 4) < MT ? RING_BYTES / (16 * BN * 4) : MT;
  constexpr int EP = EP_CAP >= 8 ? 8 : EP_CAP >= 4 ? 4 : EP_CAP >= 2 ? 2 : 1;  // divides MT
  static_assert(EP >= 1 && MT % EP == 0, "epilogue passes");
  float* T = reinterpret_cast<float*>(&As[0][0]);
  auto tidx = [](int r, int c) {  // float index of (row r, column c) in T
    return r * BN + ((((c >> 2) ^ (((r >> 2) & 3) << 2))) << 2) + (c & 3);
  };
  // whole-block stores need 4 | N and 16-byte aligned base pointers
  const bool vec = (N & 3) == 0 && (((uintptr_t)out | (uintptr_t)part) & 15) == 0;
  // Every global load the store loop needs is issued before it: vmcnt counts
  // stores too, so a load between stores would wait for every store before
  // it. A thread's four columns are the same in every round (64*KW blocks
  // per round is a whole number of rows), so its bias values load once; the
  // output rows of a pass load one per lane and travel by ds_bpermute.
  constexpr int BQ = BN / 4;  // 16-byte blocks per row
  static_assert((64 * KW) % BQ == 0, "fixed columns per thread");
  const int cfix = (tid % BQ) * 4;
  const bool add_bias = nsplit == 1 && epi.bias;  // uniform
  float bv[4] = {0.f, 0.f, 0.f, 0.f};
  if (add_bias) {
#pragma unroll
    for (int k = 0; k < 4; ++k) bv[k] = load_as_f32(epi.bias, epi.bdt, min(n0 + cfix + k, N - 1));
  }
#pragma unroll
  for (int i0 = 0; i0 < MT; i0 += EP) {
    __syncthreads();
#pragma unroll
    for (int il = 0; il < MW; ++il) {
      const int i = il;  // m-tile within the workgroup tile
      if (i < i0 || i >= i0 + EP) continue;  // another pass (uniform per wave)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = (i - i0) * 16 + 4 * lg + e;
        const float rs = __shfl(rsr[i * 16 / 64], (i * 16 + 4 * lg + e) & 63);  // 0 past M
#pragma unroll
        for (int u = 0; u < NT; ++u) T[tidx(r, wc * (NT * 16) + u * 16 + col)] = acc[il][u][e] * rs;
      }
    }
    __syncthreads();
    constexpr int BLOCKS = EP * 16 * (BN / 4);  // 16-byte blocks of the pass
    static_assert(BLOCKS % (64 * KW) == 0, "whole rounds of blocks");
    // One loop per kind of store, chosen once: the rounds are unrolled, and
    // uniform tests inside them (split, alignment, dtype, bias) cost scalar
    // branches and waits in every round.
    auto store_rounds = [&](auto kind_c, auto bias_c) {
      constexpr int KIND = decltype(kind_c)::value;
      constexpr bool BIAS = decltype(bias_c)::value;
#pragma unroll
      for (int b0 = 0; b0 < BLOCKS; b0 += 64 * KW) {
        const int b = b0 + tid, r = b / BQ, c = cfix;
        int m = m0 + i0 * 16 + r;
        const int n = n0 + c;
        if constexpr (GR) {
          // output row (split-K is never used here); every lane takes part
          const int rt = i0 * 16 + r;  // row in the tile
          int g = __shfl(rmr[0], rt & 63);
#pragma unroll
          for (int h = 1; h < RR; ++h) {
            const int gh = __shfl(rmr[h], rt & 63);
            g = (rt >> 6) == h ? gh : g;
          }
          if (m >= M || n >= N || g < 0) continue;
          m = g;
        } else {
          if (m >= M || n >= N) continue;
        }
        f32x4 v = *reinterpret_cast<const f32x4*>(&T[tidx(r, c)]);
        if constexpr (BIAS) {  // the same rounding as Epilogue
#pragma unroll
          for (int k = 0; k < 4; ++k) v[k] = round_to(v[k], epi.ydt) + bv[k];
        }
        if constexpr (KIND == kStPart) {
          *reinterpret_cast<f32x4*>(part + ((int64_t)sp * M + m) * N + n) = v;
        } else if constexpr (KIND == kStBf16 || KIND == kStF16) {
          const int dt = KIND == kStBf16 ? DT_BF16 : DT_F16;
          *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + (int64_t)m * N + n) =
              make_uint2(pack2(v[0], v[1], dt), pack2(v[2], v[3], dt));
        } else if constexpr (KIND == kStF32) {
          *reinterpret_cast<f32x4*>(static_cast<float*>(out) + (int64_t)m * N + n) = v;
        } else {  // any layout, element by element
          if (add_bias) {
#pragma unroll
            for (int k = 0; k < 4; ++k) v[k] = round_to(v[k], epi.ydt) + bv[k];
          }
          for (int k = 0; k < 4 && n + k < N; ++k) {
            if (nsplit > 1)
              part[((int64_t)sp * M + m) * N + n + k] = v[k];
            else
              store_from_f32(out, odt, (int64_t)m * N + n + k, v[k]);
          }
        }
      }
    };
    using std::integral_constant;
    using B0 = integral_constant<bool, false>;
    using B1 = integral_constant<bool, true>;
    if (!vec) {
      store_rounds(integral_constant<int, kStAny>{}, B0{});
    } else if (nsplit > 1) {  // no bias on partial sums
      store_rounds(integral_constant<int, kStPart>{}, B0{});
    } else if (odt == DT_BF16) {
      if (add_bias) store_rounds(integral_constant<int, kStBf16>{}, B1{});
      else store_rounds(integral_constant<int, kStBf16>{}, B0{});
    } else if (odt == DT_F16) {
      if (add_bias) store_rounds(integral_constant<int, kStF16>{}, B1{});
      else store_rounds(integral_constant<int, kStF16>{}, B0{});
    } else {
      if (add_bias) store_rounds(integral_constant<int, kStF32>{}, B1{});
      else store_rounds(integral_constant<int, kStF32>{}, B0{});
    }
  }
}

// The split-K reductions. Thread i serves outputs V*i .. V*i+V-1 (V = 4
// where every row is a whole number of 16-byte blocks and the pointers are
// aligned: one 16-byte load per slice and one store per thread), each
// output summed over the slices in slice order, so V changes no bit.
template <int V>
__device__ __forceinline__ void load_v(const float* p, float (&v)[V]) {
  if constexpr (V == 4) {
    const f32x4 q = *reinterpret_cast<const f32x4*>(p);
    v[0] = q[0]; v[1] = q[1]; v[2] = q[2]; v[3] = q[3];
  } else {
    v[0] = *p;
  }
}
template <int V>
__device__ __forceinline__ void add_slices(const float* part, int64_t i, int64_t MN, int nsplit, float (&s)[V]) {
  load_v<V>(part + i, s);
  for (int k = 1; k < nsplit; ++k) {
    float q[V];
    load_v<V>(part + k * MN + i, q);
#pragma unroll
    for (int e = 0; e < V; ++e) s[e] += q[e];
  }
}
template <int V>
__device__ __forceinline__ void store_v(void* out, int odt, int64_t i, const float (&v)[V]) {
  if constexpr (V == 4) {
    if (odt == DT_F32) {
      *reinterpret_cast<f32x4*>(static_cast<float*>(out) + i) = f32x4{v[0], v[1], v[2], v[3]};
    } else {
      *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(out) + i) = u32x2{pack2(v[0], v[1], odt), pack2(v[2], v[3], odt)};
    }
  } else {
    store_from_f32(out, odt, i, v[0]);
  }
}

// out[m, n] = sum over slices s (in order) of part[s, m, n].
template <int V>
__global__ void gemm_reduce(const float* __restrict__ part, void* __restrict__ out, int odt, int64_t MN, int N,
                            int nsplit, Epilogue epi) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * V;
  if (i >= MN) return;
  float s[V];
  add_slices<V>(part, i, MN, nsplit, s);
  const int n = (int)(i % N);
#pragma unroll
  for (int e = 0; e < V; ++e) s[e] = epi(s[e], n + e);
  store_v<V>(out, odt, i, s);
}

// The gated MLP after two split-K GEMMs (gate and up): each output sums its
// slices in order as gemm_reduce does, takes its epilogue, and the pair goes
// through the activation (act_mul rounds both to odt first, as the stored
// intermediates of separate calls would be).
template <int V>
__global__ void gemm_reduce_gate_up(const float* __restrict__ pg, int ng, const float* __restrict__ pu, int nu,
                                    void* __restrict__ out, int odt, int64_t MN, int N, Epilogue eg, Epilogue eu,
                                    int act) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * V;
  if (i >= MN) return;
  float g[V], u[V];
  add_slices<V>(pg, i, MN, ng, g);
  add_slices<V>(pu, i, MN, nu, u);
  const int n = (int)(i % N);
#pragma unroll
  for (int e = 0; e < V; ++e) g[e] = act_mul(eg(g[e], n + e), eu(u[e], n + e), odt, act);
  store_v<V>(out, odt, i, g);
}

// The split-K reductions of up to kReduceParts launches in one grid: thread
// i serves the part whose element range holds its outputs, exactly as
// gemm_reduce.
struct ReduceParts {
  const float* part[kReduceParts];
  void* out[kReduceParts];
  int odt[kReduceParts], N[kReduceParts], nsplit[kReduceParts];
  int64_t MN[kReduceParts], start[kReduceParts + 1];
  Epilogue epi[kReduceParts];
  int n;
};
template <int V>
__global__ void gemm_reduce_multi(ReduceParts r) {
  const int64_t g = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * V;
  if (g >= r.start[r.n]) return;
  int p = 0;
#pragma unroll
  for (int q = 1; q < kReduceParts; ++q) p = (q < r.n && g >= r.start[q]) ? q : p;
  const int64_t i = g - r.start[p];
  float s[V];
  add_slices<V>(r.part[p], i, r.MN[p], r.nsplit[p], s);
  const int n = (int)(i % r.N[p]);
#pragma unroll
  for (int e = 0; e < V; ++e) s[e] = r.epi[p](s[e], n + e);
  store_v<V>(r.out[p], r.odt[p], i, s);
}

// V = 4 for large reductions (measured: a Llama-3-8B gate/up call at M = 64,
// 0.9 M outputs, 28.3 -> 27.5 us; at 0.26-0.5 M outputs V = 4 was 0.3-0.8 us
// slower: a quarter of the threads leaves too few loads in flight) where
// every row is whole 16-byte blocks of partials and the output takes
// 4-element stores.
constexpr int64_t kReduceVecMin = 768 * 1024;
bool reduce_vec4(const void* out, int odt, const float* part, int N, int64_t MN) {
  const uintptr_t oa = reinterpret_cast<uintptr_t>(out), pa = reinterpret_cast<uintptr_t>(part);
  return MN >= kReduceVecMin && N % 4 == 0 && (pa & 15) == 0 && (oa & (odt == DT_F32 ? 15 : 7)) == 0;
}

}  // namespace

GemmPlan plan_gemm(int M, int N, int K, int bits) {
  (void)bits;
  GemmPlan p;
  int mt = 1;
  while (mt < kMaxMT && 16 * mt < M) mt *= 2;
  p.mt = mt;
  p.tiles_m = (M + 16 * mt - 1) / (16 * mt);
  p.tiles_n = (N + kBN - 1) / kBN;
  // Split K while the launch has fewer than one workgroup per CU (measured:
  // splitting further only adds partial-sum traffic) and each slice keeps at
  // least 4 stages. Below the largest tile the split depends
  // on (N, K, mt) only, so rows do not change with M inside one mt class.
  const int stages = K / kStage;
  const int tm = mt < kMaxMT ? 1 : p.tiles_m;
  int s = 1;
  while (p.tiles_n * tm * s * 2 <= kSplitCap && stages / (2 * s) >= 4) s *= 2;
  p.nsplit = s;
  p.kslice = ((stages + s - 1) / s) * kStage;
  p.nsplit = (K + p.kslice - 1) / p.kslice;
  // 128-row tiles run one workgroup per CU. When the tiles fill a last round
  // only partly (at most half), those tiles go to a second launch as two
  // 128-column workgroups each, so the last round takes half the time. Each
  // output element still accumulates over K in the same order: the rows are
  // bit-identical to the full-width kernel's.
  const int T = p.tiles_n * p.tiles_m, r = T % kCUs;
  p.tail = (mt == kMaxMT && p.nsplit == 1 && T > kCUs && r > 0 && r <= kCUs / 2) ? r : 0;
  return p;
}

size_t gemm_partial_bytes(const GemmPlan& p, int M, int N) {
  return p.nsplit > 1 ? (size_t)p.nsplit * M * N * sizeof(float) : 0;
}

bool gemm_supported(int K) { return K % kStage == 0; }

GemmPart part_of(const QmvArgs& a, const GemmPlan& p, float* part, int tile0, int cnt, int nsplit, int start,
                 bool gr) {
  return GemmPart{(const uint32_t*)a.w, (const uint16_t*)a.scales, (const uint16_t*)a.biases, part, a.out,
                  a.odt, a.N, p.kslice, p.tiles_n, tile0, cnt, nsplit, start,
                  gr ? Epilogue{nullptr, 0, 0} : a.epi()};
}

template <int BITS, bool SF16, int MT, int GS, int NT, bool GR>
static hipError_t launch_parts(const GemmParts& gp, const QmvArgs& a, const u32x4* xh, const float* rsc,
                               const int* gtab, const int* rowmap) {
  const int grid = ((gp.total + kXcds - 1) / kXcds) * kXcds;
  hipLaunchKernelGGL((gemm_kernel<BITS, SF16, MT, GS, NT, GR>), dim3(grid), dim3(64 * kWaves), 0, a.stream, xh,
                     rsc, gp, a.M, a.K, gtab, rowmap);
  return hipGetLastError();
}

template <int BITS, bool SF16, int MT, int GS, int NT, bool GR>
static hipError_t launch_range(const QmvArgs& a, const GemmPlan& p, const u32x4* xh,
                               const float* rsc, float* part, int tile0, int cnt, int nsplit,
                               const int* gtab, const int* rowmap) {
  GemmParts gp{};
  gp.n = 1;
  gp.total = cnt * (kNT / NT) * nsplit;
  gp.p[0] = part_of(a, p, part, tile0, cnt, nsplit, 0, GR);
  return launch_parts<BITS, SF16, MT, GS, NT, GR>(gp, a, xh, rsc, gtab, rowmap);
}

template <int BITS, bool SF16, int MT, int GS, bool GR>
static hipError_t launch_mt(const QmvArgs& a, const GemmPlan& p, const u32x4* xh, const float* rsc,
                            float* part, const int* gtab, const int* rowmap) {
  const int T = p.tiles_n * p.tiles_m;
  if constexpr (GR) {
    return launch_range<BITS, SF16, MT, GS, kNT, true>(a, p, xh, rsc, part, 0, T, 1, gtab, rowmap);
  } else {
    hipError_t e = launch_range<BITS, SF16, MT, GS, nt_for(MT), false>(a, p, xh, rsc, part, 0, T - p.tail, p.nsplit,
                                                                      nullptr, nullptr);
    if constexpr (MT == kMaxMT) {
      if (e == hipSuccess && p.tail > 0)
        e = launch_range<BITS, SF16, MT, GS, kNT / 2, false>(a, p, xh, rsc, part, T - p.tail, p.tail, 1, nullptr,
                                                       nullptr);
    }
    return e;
  }
}

template <int BITS, bool SF16, int GS, bool GR>
static hipError_t launch_g(const QmvArgs& a, const GemmPlan& p, const u32x4* xh, const float* rsc,
                           float* part, const int* gtab, const int* rowmap) {
  switch (p.mt) {
    case 1: return launch_mt<BITS, SF16, 1, GS, GR>(a, p, xh, rsc, part, gtab, rowmap);
    case 2: return launch_mt<BITS, SF16, 2, GS, GR>(a, p, xh, rsc, part, gtab, rowmap);
    case 4: return launch_mt<BITS, SF16, 4, GS, GR>(a, p, xh, rsc, part, gtab, rowmap);
    default: return launch_mt<BITS, SF16, 8, GS, GR>(a, p, xh, rsc, part, gtab, rowmap);
  }
}

template <int BITS, bool SF16, bool GR>
static hipError_t launch_s(const QmvArgs& a, const GemmPlan& p, const u32x4* xh, const float* rsc,
                           float* part, const int* gtab = nullptr, const int* rowmap = nullptr) {
  switch (a.gs) {
    case 32: return launch_g<BITS, SF16, 32, GR>(a, p, xh, rsc, part, gtab, rowmap);
    case 64: return launch_g<BITS, SF16, 64, GR>(a, p, xh, rsc, part, gtab, rowmap);
    default: return launch_g<BITS, SF16, 128, GR>(a, p, xh, rsc, part, gtab, rowmap);
  }
}

template <int BITS, bool SF16, int GS>
static hipError_t multi_mt(const GemmParts& gp, const QmvArgs& a, int mt, const u32x4* xh, const float* rsc) {
  switch (mt) {
    case 1: return launch_parts<BITS, SF16, 1, GS, nt_for(1), false>(gp, a, xh, rsc, nullptr, nullptr);
    case 2: return launch_parts<BITS, SF16, 2, GS, nt_for(2), false>(gp, a, xh, rsc, nullptr, nullptr);
    case 4: return launch_parts<BITS, SF16, 4, GS, nt_for(4), false>(gp, a, xh, rsc, nullptr, nullptr);
    default: return launch_parts<BITS, SF16, 8, GS, nt_for(8), false>(gp, a, xh, rsc, nullptr, nullptr);
  }
}
template <int BITS, bool SF16>
static hipError_t multi_gs(const GemmParts& gp, const QmvArgs& a, int mt, const u32x4* xh, const float* rsc) {
  switch (a.gs) {
    case 32: return multi_mt<BITS, SF16, 32>(gp, a, mt, xh, rsc);
    case 64: return multi_mt<BITS, SF16, 64>(gp, a, mt, xh, rsc);
    default: return multi_mt<BITS, SF16, 128>(gp, a, mt, xh, rsc);
  }
}

bool gemm_multi_compatible(const QmvArgs* a, const GemmPlan* p, int n) {
  if (n < 1 || n > kGemmParts) return false;
  for (int i = 0; i < n; ++i)
    if (a[i].bits != a[0].bits || a[i].gs != a[0].gs || a[i].sdt != a[0].sdt || p[i].mt != p[0].mt ||
        p[i].tail != 0)
      return false;
  return true;
}

hipError_t launch_gemm_multi(const QmvArgs* a, const GemmPlan* p, const void* xh, const float* rsc,
                             float* const* part, int n) {
  if (!gemm_multi_compatible(a, p, n)) return hipErrorInvalidValue;
  GemmParts gp{};
  gp.n = n;
  int start = 0;
  for (int i = 0; i < n; ++i) {
    const int cnt = p[i].tiles_n * p[i].tiles_m;
    gp.p[i] = part_of(a[i], p[i], part[i], 0, cnt, p[i].nsplit, start, false);
    start += cnt * p[i].nsplit * (kNT / nt_for(p[0].mt));
  }
  gp.total = start;
  const u32x4* x4 = static_cast<const u32x4*>(xh);
  const bool sf16 = a[0].sdt == DT_F16;
  if (a[0].bits == 4)
    return sf16 ? multi_gs<4, true>(gp, a[0], p[0].mt, x4, rsc) : multi_gs<4, false>(gp, a[0], p[0].mt, x4, rsc);
  return sf16 ? multi_gs<8, true>(gp, a[0], p[0].mt, x4, rsc) : multi_gs<8, false>(gp, a[0], p[0].mt, x4, rsc);
}

// `xh`/`rsc` as written by launch_prep_x; `part` holds gemm_partial_bytes.
hipError_t launch_gemm(const QmvArgs& a, const GemmPlan& p, const void* xh, const float* rsc,
                       float* part, bool reduce) {
  hipError_t e;
  const u32x4* x4 = static_cast<const u32x4*>(xh);
  const bool sf16 = a.sdt == DT_F16;
  if (a.bits == 4)
    e = sf16 ? launch_s<4, true, false>(a, p, x4, rsc, part) : launch_s<4, false, false>(a, p, x4, rsc, part);
  else
    e = sf16 ? launch_s<8, true, false>(a, p, x4, rsc, part) : launch_s<8, false, false>(a, p, x4, rsc, part);
  if (e != hipSuccess || p.nsplit == 1 || !reduce) return e;
  const int64_t MN = (int64_t)a.M * a.N;
  if (reduce_vec4(a.out, a.odt, part, a.N, MN))
    hipLaunchKernelGGL(gemm_reduce<4>, dim3((unsigned)((MN / 4 + 255) / 256)), dim3(256), 0, a.stream, part,
                       a.out, a.odt, MN, a.N, p.nsplit, a.epi());
  else
    hipLaunchKernelGGL(gemm_reduce<1>, dim3((unsigned)((MN + 255) / 256)), dim3(256), 0, a.stream, part,
                       a.out, a.odt, MN, a.N, p.nsplit, a.epi());
  return hipGetLastError();
}

hipError_t launch_gemm_reduce_gate_up(const QmvArgs& g, const GemmPlan& pg, const float* part_g,
                                      const QmvArgs& u, const GemmPlan& pu, const float* part_u, int act) {
  const int64_t MN = (int64_t)g.M * g.N;
  if (reduce_vec4(g.out, g.odt, part_g, g.N, MN) && reduce_vec4(g.out, g.odt, part_u, g.N, MN))
    hipLaunchKernelGGL(gemm_reduce_gate_up<4>, dim3((unsigned)((MN / 4 + 255) / 256)), dim3(256), 0, g.stream,
                       part_g, pg.nsplit, part_u, pu.nsplit, g.out, g.odt, MN, g.N, g.epi(), u.epi(), act);
  else
    hipLaunchKernelGGL(gemm_reduce_gate_up<1>, dim3((unsigned)((MN + 255) / 256)), dim3(256), 0, g.stream,
                       part_g, pg.nsplit, part_u, pu.nsplit, g.out, g.odt, MN, g.N, g.epi(), u.epi(), act);
  return hipGetLastError();
}

hipError_t launch_gemm_reduce_multi(const QmvArgs* a, const GemmPlan* p, float* const* part, int n) {
  if (n < 1 || n > kReduceParts) return hipErrorInvalidValue;
  ReduceParts r{};
  r.n = n;
  r.start[0] = 0;
  bool vec = true;
  for (int i = 0; i < n; ++i) {
    r.part[i] = part[i];
    r.out[i] = a[i].out;
    r.odt[i] = a[i].odt;
    r.N[i] = a[i].N;
    r.nsplit[i] = p[i].nsplit;
    r.MN[i] = (int64_t)a[i].M * a[i].N;
    r.epi[i] = a[i].epi();
    r.start[i + 1] = r.start[i] + r.MN[i];
    vec = vec && reduce_vec4(a[i].out, a[i].odt, part[i], a[i].N, kReduceVecMin);
  }
  if (vec && r.start[n] >= kReduceVecMin)
    hipLaunchKernelGGL(gemm_reduce_multi<4>, dim3((unsigned)((r.start[n] / 4 + 255) / 256)), dim3(256), 0,
                       a[0].stream, r);
  else
    hipLaunchKernelGGL(gemm_reduce_multi<1>, dim3((unsigned)((r.start[n] + 255) / 256)), dim3(256), 0,
                       a[0].stream, r);
  return hipGetLastError();
}

// Grouped GEMM over expert stacks: a.M is the padded row count
// (tiles_max * 16 * mt), a.out has the real rows; see gemm_kernel's GR mode.
hipError_t launch_gemm_grouped(const QmvArgs& a, int mt, int tiles_max, const void* xh,
                               const float* rsc, const int* gtab, const int* rowmap) {
  GemmPlan p;
  p.mt = mt;
  p.tiles_m = tiles_max;
  p.tiles_n = (a.N + kBN - 1) / kBN;
  p.nsplit = 1;
  p.kslice = a.K;
  p.tail = 0;
  const u32x4* x4 = static_cast<const u32x4*>(xh);
  const bool sf16 = a.sdt == DT_F16;
  if (a.bits == 4)
    return sf16 ? launch_s<4, true, true>(a, p, x4, rsc, nullptr, gtab, rowmap)
                : launch_s<4, false, true>(a, p, x4, rsc, nullptr, gtab, rowmap);
  return sf16 ? launch_s<8, true, true>(a, p, x4, rsc, nullptr, gtab, rowmap)
              : launch_s<8, false, true>(a, p, x4, rsc, nullptr, gtab, rowmap);
}

}  // namespace kh
