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
// accumulating in float32. MFMA step j of a 128-code piece covers the codes
// j*32 .. j*32+31, which lie in one quantization group (group size >= 32),
// and a second MFMA against ones gives the group sums X of x. Per group:
//   acc += s * P + (b - OFF * s) * X,   P = sum x * (OFF + q).
// 8-bit codes with bf16 x, where OFF + q is not exact beyond q = 127, enter
// as two nibble operands: P = P_lo + 16 * P_hi with OFF_eff = 17 * 128.
//
// Work decomposition: a workgroup of W <= 8 waves owns 16 * NTW weight rows
// and all M rows of x (one or two 16-row m-tiles); the waves split K into
// 128-code pieces, interleaved (wave w takes pieces w, w + W, ...), so at any
// time a workgroup reads W consecutive pieces of each of its rows. Lane
// (n = l % 16, kb = l / 16) of a 16-row tile loads the codes kb*32 ..
// kb*32+31 of row n (16 or 32 bytes); a 4x4 word transpose across the lane
// rows (permlane swaps) gives each lane its 8 codes of every step. x comes
// as the matching 16-byte runs of x row l % 16 (zeros past M), straight
// from memory. Every load is a buffer load whose offset is selected without
// branches (past the row, the piece range or M it reads zeros), so the
// compiler's waits cover exactly the piece computed while the next ones stay
// in flight. The scales and biases of the workgroup's rows for all of K are
// copied into LDS first, as contiguous 16-byte words. The W partial tiles
// are summed through LDS in wave order.
#include <algorithm>
#include <type_traits>

#include "kh_common.h"
#include "kh_kernels.h"

namespace kh {

namespace {

constexpr int kSkMaxWaves = 8;
constexpr int kSkMaxParts = 4;
constexpr int kPiece = 128;  // codes per piece
// Pieces a wave keeps in flight: one while it has at most kSkDepth1Max
// pieces to do (measured best: more outstanding loads of this access
// pattern only slowed the launch), two for longer runs of K.
constexpr int kSkDepth1Max = 16;

template <bool XBF16>
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (XBF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// 4x4 transpose of words across the four 16-lane rows of a wave: word a of
// row b becomes word b of row a.
__device__ __forceinline__ void xpose4(uint32_t* w) {
  const auto r = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
  const auto q = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
  const auto u = __builtin_amdgcn_permlane16_swap(r[0], q[0], false, false);
  const auto v = __builtin_amdgcn_permlane16_swap(r[1], q[1], false, false);
  w[0] = u[0];
  w[1] = u[1];
  w[2] = v[0];
  w[3] = v[1];
}

// Raw buffer descriptor over `bytes` bytes (gfx9-family raw format word):
// loads at offsets >= bytes return zeros without a memory access.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t sk_buf(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, bytes, 0x00020000);
}
// OR-ed into an offset it puts it past every tensor (all are < 2 GiB).
constexpr uint32_t kOob = 0xFFFFF000u;

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

// One piece's operands in registers: the lane's 32 codes per tile and x for
// the four MFMA steps per m-tile.
template <int BITS, int NTW, int MT>
struct Piece {
  u32x4 q[NTW][BITS / 4];
  u32x4 x[MT][4];
};

// SOLO: a launch of one part (no part table walk: every kernel argument is
// read at a fixed offset, in one batch of scalar loads).
template <int BITS, bool XBF16, bool SBF16, int GS, int NTW, int MT, int D, bool SOLO>
__global__ __launch_bounds__(64 * kSkMaxWaves) void skinny_kernel(
    const uint16_t* __restrict__ x, SkParts parts, int M, int K, int ppw) {
  using P_t = Piece<BITS, NTW, MT>;
  constexpr int GP = kPiece / GS;  // groups per piece
  constexpr bool SPLIT = XBF16 && BITS == 8;    // 8-bit codes as two nibble operands
  constexpr uint32_t MAG = XBF16 ? 0x43004300u : 0x64006400u;   // OFF in both halves
  constexpr uint32_t ONE = XBF16 ? 0x3F803F80u : 0x3C003C00u;   // 1.0 in both halves
  constexpr float OFF = SPLIT ? 17.f * 128.f : (XBF16 ? 128.f : 1024.f);

  // LDS: the scales and biases of the workgroup's rows for all of K
  // ([2][ROWS][G] 16-bit values), then the partial tiles of the cross-wave
  // sum ([W][MT][NTW][4][64] floats).
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int ROWS = 16 * NTW;
  uint16_t* sbl = reinterpret_cast<uint16_t*>(smem);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, W = blockDim.x >> 6;
  const int col = lane & 15, kb = lane >> 4;
  const bool paired = !SOLO && parts.act >= 0;  // uniform
  constexpr int HALF = NTW / 2 > 0 ? NTW / 2 : 1;  // tiles per part in paired mode (NTW even there)
  int pi = 0;                          // the part (independent mode)
  if constexpr (!SOLO) {
    if (!paired)
      while (pi + 1 < parts.n && (int)blockIdx.x >= parts.part[pi + 1].tile0) ++pi;
  }
  const int n0 = paired ? (int)blockIdx.x * 16 * HALF : ((int)blockIdx.x - parts.part[pi].tile0) * 16 * NTW;
  const int G = K / GS;
  const int rowb = K * BITS / 8;  // bytes per row of codes

  // slot t: its part and its first row (paired: slots 0..HALF-1 gate, the
  // rest up, over the same rows)
  auto slot_part = [&](int t) { return paired ? (t < HALF ? 0 : 1) : pi; };
  auto slot_row = [&](int t) { return n0 + (paired ? (t % HALF) : t) * 16; };
  __amdgpu_buffer_rsrc_t wb[NTW];
  uint32_t wro[NTW], rmask[NTW];  // byte offset of the lane's row; rows past N read zeros
#pragma unroll
  for (int t = 0; t < NTW; ++t) {
    const SkPart& sp = parts.part[slot_part(t)];
    wb[t] = sk_buf(sp.w, (uint32_t)((int64_t)sp.N * rowb));
    const int r = slot_row(t) + col;
    rmask[t] = r < sp.N ? 0u : kOob;
    wro[t] = (uint32_t)min(r, sp.N - 1) * rowb;
  }
  // x rows past M (padding of the m-tile) read zeros: the batch costs x
  // bytes for its M rows only
  uint32_t xro[MT], xmask[MT];
  const __amdgpu_buffer_rsrc_t xb = sk_buf(x, (uint32_t)((int64_t)M * K * 2));
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + col;
    xmask[mt] = m < M ? 0u : kOob;
    xro[mt] = (uint32_t)min(m, M - 1) * K * 2;
  }

  // The wave's i-th piece is piece wave + i*W of the row: a workgroup reads
  // W consecutive pieces of each row at a time. Pieces i >= ppw read zeros
  // (and add nothing). The offsets are selected without branches, so the
  // compiler's waits for a piece leave the later pieces' loads in flight.
  auto load = [&](P_t& P, int i) {
    const uint32_t pmask = (uint32_t)((ppw - 1 - i) >> 31) & kOob;  // i >= ppw
    const int piece = wave + i * W;
    const uint32_t cofs = (uint32_t)piece * (kPiece * BITS / 8) + kb * (BITS * 4);
#pragma unroll
    for (int t = 0; t < NTW; ++t) {
#pragma unroll
      for (int h = 0; h < BITS / 4; ++h)
        P.q[t][h] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(wb[t], (wro[t] + cofs + 16 * h) | rmask[t] | pmask, 0, 2));
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t xc = (uint32_t)(piece * kPiece + j * 32 + kb * 8) * 2;
        P.x[mt][j] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(xb, (xro[mt] + xc) | xmask[mt] | pmask, 0, 0));
      }
  };

  f32x4 acc[MT][NTW];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < NTW; ++t) acc[mt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const u32x4 ones = u32x4{ONE, ONE, ONE, ONE};

  // MFMA step j of a piece covers its codes j*32 .. j*32+31 (lane row kb:
  // j*32 + kb*8 .. +7), inside one quantization group (group size >= 32).
  auto compute = [&](P_t& P, int i) {
    const int piece = min(wave + i * W, W * ppw - 1);  // pieces past the wave's read zeros
    // lane row kb loaded codes kb*32 .. kb*32+31 (4 or 8 words); step j
    // wants word kb of lane row j: a 4x4 transpose of words across rows
#pragma unroll
    for (int t = 0; t < NTW; ++t) {
      if constexpr (BITS == 4) {
        uint32_t w[4] = {P.q[t][0][0], P.q[t][0][1], P.q[t][0][2], P.q[t][0][3]};
        xpose4(w);
        P.q[t][0] = u32x4{w[0], w[1], w[2], w[3]};
      } else {
        uint32_t e[4] = {P.q[t][0][0], P.q[t][0][2], P.q[t][1][0], P.q[t][1][2]};
        uint32_t o[4] = {P.q[t][0][1], P.q[t][0][3], P.q[t][1][1], P.q[t][1][3]};
        xpose4(e);
        xpose4(o);
        P.q[t][0] = u32x4{e[0], o[0], e[1], o[1]};
        P.q[t][1] = u32x4{e[2], o[2], e[3], o[3]};
      }
    }
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
      const int g = (j * 32) / GS;
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
        const u32x4 a = permute_x<BITS>(P.x[mt][j]);
        xs[mt][g] = mfma16<XBF16>(a, ones, xs[mt][g]);
#pragma unroll
        for (int t = 0; t < NTW; ++t) {
          pa[mt][t][g] = mfma16<XBF16>(a, lo[t], pa[mt][t][g]);
          if constexpr (SPLIT) pb[mt][t][g] = mfma16<XBF16>(a, hi[t], pb[mt][t][g]);
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

  // Scales and biases of the workgroup's rows for all of K, staged in LDS
  // ([2][ROWS][G] 16-bit values): one contiguous [rows][G] block per array
  // and part, copied in 16-byte words (issued before the pieces' loads, so
  // the wait for them leaves the pieces in flight).
  constexpr int SREG = 2;  // staged words per thread held in registers
  u32x4 sv[SREG];
  const int srows = paired ? 16 * HALF : 16 * NTW;  // rows per part
  const int scnt = (paired ? 4 : 2) * srows * G / 8;  // words over (part, array)
  const bool svec = (G & 7) == 0;
  if (svec) {
#pragma unroll
    for (int r = 0; r < SREG; ++r) {
      const int i = min((int)threadIdx.x + r * (int)blockDim.x, scnt - 1);
      const int per = srows * G / 8, blk = i / per, j = i - blk * per;  // blk = part * 2 + array
      const SkPart& sp = parts.part[paired ? (blk >> 1) : pi];
      const uint16_t* src = (blk & 1) ? sp.biases : sp.scales;
      // rows past N repeat the last row's words (never used)
      const int64_t e = min((int64_t)n0 * G + (int64_t)j * 8, (int64_t)sp.N * G - 8);
      sv[r] = *reinterpret_cast<const u32x4*>(src + e);
    }
  }
  P_t buf[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    load(buf[d], d);
    __builtin_amdgcn_sched_barrier(0);
  }
  {
    const int per = srows * G / 8;
    auto dst_of = [&](int i) {
      const int blk = i / per, j = i - blk * per;
      const int row0 = paired ? (blk >> 1) * 16 * HALF : 0;
      return reinterpret_cast<u32x4*>(sbl + (int64_t)(blk & 1) * ROWS * G + (int64_t)row0 * G) + j;
    };
    if (svec) {
#pragma unroll
      for (int r = 0; r < SREG; ++r) {
        const int i = (int)threadIdx.x + r * (int)blockDim.x;
        if (i < scnt) *dst_of(i) = sv[r];
      }
      for (int i = (int)threadIdx.x + SREG * (int)blockDim.x; i < scnt; i += blockDim.x) {
        const int blk = i / per, j = i - blk * per;
        const SkPart& sp = parts.part[paired ? (blk >> 1) : pi];
        const uint16_t* src = (blk & 1) ? sp.biases : sp.scales;
        const int64_t e = min((int64_t)n0 * G + (int64_t)j * 8, (int64_t)sp.N * G - 8);
        *dst_of(i) = *reinterpret_cast<const u32x4*>(src + e);
      }
    } else {
      const int per16 = srows * G;
      for (int i = threadIdx.x; i < scnt * 8; i += blockDim.x) {
        const int blk = i / per16, j = i - blk * per16;
        const SkPart& sp = parts.part[paired ? (blk >> 1) : pi];
        const uint16_t* src = (blk & 1) ? sp.biases : sp.scales;
        const int row0 = paired ? (blk >> 1) * 16 * HALF : 0;
        sbl[(int64_t)(blk & 1) * ROWS * G + (int64_t)row0 * G + j] = src[min((int64_t)n0 * G + j, (int64_t)sp.N * G - 1)];
      }
    }
    __syncthreads();
  }
  for (int i = 0; i < ppw; i += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      compute(buf[d], i + d);
      // the refill goes out before the next piece's arithmetic
      load(buf[d], i + d + D);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // Sum the W partial tiles in wave order. D lane l holds rows 4*(l/16)+e,
  // column l%16 of each 16x16 tile.
  float* red = reinterpret_cast<float*>(smem + (size_t)2 * ROWS * G * 2);
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

// Most 16-row tiles per wave that fit the registers with two pieces in
// flight (from the compiler's register counts: larger tilings spill).
constexpr int max_ntw(int bits, int gs, int mt) {
  return mt == 1 ? (bits == 8 && gs == 32 ? 2 : 4) : (bits == 8 && gs == 32 ? 1 : 2);
}
// Widest tiling a single-part launch chooses (measured: wider tiles of one
// matrix leave CUs without work before they save x loads).
constexpr int pref_ntw(int bits, int gs, int mt) {
  return mt == 1 ? (bits == 4 ? (gs == 128 ? 4 : 2) : (gs == 32 ? 1 : 2))
                 : (bits == 4 && gs == 128 ? 2 : 1);
}

// W and the pieces per wave depend on K only, so a row's summation order
// is the same for every M this kernel serves. The tile width keeps at least
// 2048 waves in a single-part launch; a multi-part launch (q|k|v) widens to
// 1024 waves with the full register budget (measured: Llama-3-8B q|k|v at
// M = 16..32 took 11-15 us against 14-22 us on one tile per wave).
SkinnyPlan plan_skinny(int M, int N, int K, int bits, int gs, bool multi = false) {
  const int np = K / kPiece;
  int W = kSkMaxWaves;
  while (np % W) --W;
  SkinnyPlan p{W, np / W, 1, M > 16 ? 2 : 1};
  const int mx = multi ? max_ntw(bits, gs, p.mt) : pref_ntw(bits, gs, p.mt);
  const int64_t thr = multi ? 1024 : 2048;
  if (mx >= 4 && (int64_t)((N + 63) / 64) * W >= thr) p.ntw = 4;
  else if (mx >= 2 && (int64_t)((N + 31) / 32) * W >= thr) p.ntw = 2;
  return p;
}

// LDS of one workgroup: scales and biases of its rows, then the partial tiles.
size_t skinny_lds(const SkinnyPlan& p, int64_t K, int gs) {
  return (size_t)2 * 16 * p.ntw * (K / gs) * 2 + (size_t)p.W * p.mt * p.ntw * 4 * 64 * sizeof(float);
}
constexpr size_t kSkMaxLds = 96 * 1024;
constexpr int64_t kSkMaxChainCycles = 20000;  // MFMA cycles per wave (measured bound, see skinny_supported)
constexpr int64_t kSkMaxMfma = 1000000;        // MFMAs per launch (measured crossover, see skinny_supported)
constexpr int64_t kSkMaxXBytes = (int64_t)150 << 20;  // x reads of a launch at M = 17..32 (measured, see skinny_supported)
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
  const bool one = n == 1 && act < 0;
  if (p.ppw <= kSkDepth1Max) {
    if (one)
      hipLaunchKernelGGL((skinny_kernel<BITS, XBF16, SBF16, GS, NTW, MT, 1, true>), dim3(wgs), dim3(64 * p.W), lds,
                         a[0].stream, (const uint16_t*)a[0].x, parts, a[0].M, a[0].K, p.ppw);
    else
      hipLaunchKernelGGL((skinny_kernel<BITS, XBF16, SBF16, GS, NTW, MT, 1, false>), dim3(wgs), dim3(64 * p.W), lds,
                         a[0].stream, (const uint16_t*)a[0].x, parts, a[0].M, a[0].K, p.ppw);
  } else {
    if (one)
      hipLaunchKernelGGL((skinny_kernel<BITS, XBF16, SBF16, GS, NTW, MT, 2, true>), dim3(wgs), dim3(64 * p.W), lds,
                         a[0].stream, (const uint16_t*)a[0].x, parts, a[0].M, a[0].K, p.ppw);
    else
      hipLaunchKernelGGL((skinny_kernel<BITS, XBF16, SBF16, GS, NTW, MT, 2, false>), dim3(wgs), dim3(64 * p.W), lds,
                         a[0].stream, (const uint16_t*)a[0].x, parts, a[0].M, a[0].K, p.ppw);
  }
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
  // Every 16-row tile reads all of x: at M = 17..32 a long-K matrix makes
  // that stream several times the code bytes (Llama-3-8B down 4096x14336 at
  // M = 32: 235 MB of x reads against 29 MB of codes, 31.7 us against 27.8
  // on the GEMM; at M = 17, 125 MB, 22.9 us against 26.7).
  if (M > 16 && (int64_t)((N + 15) / 16) * K * 2 * M > kSkMaxXBytes) return false;
  // MFMAs per piece: 4 steps x m-tiles of P per tile (two with the nibble
  // operands of 8-bit codes; bf16 x, the case the bounds are measured on),
  // and the X sums shared by the wave's tiles.
  const int64_t p_tile = 4 * p.mt * (bits == 8 ? 2 : 1), x_sums = 4 * p.mt;
  // Each wave computes its pieces in sequence. Where that chain of MFMAs is
  // long the launch is compute-bound with few waves in flight and the GEMM
  // is faster: Qwen2.5-7B's down projection (8-bit gs32, K = 18944) at
  // M = 17..32 took 84-94 us on a four-times longer chain than this kernel
  // has now, against 45-47 on the GEMM. Bound: ~10 us of MFMA issue per wave.
  const int64_t chain = (int64_t)p.ppw * (p_tile * p.ntw + x_sums) * 16;
  if (chain > kSkMaxChainCycles) return false;
  // Over the launch the MFMA work per code byte is fixed by (bits, m-tiles);
  // its lower fixed cost wins on small matrices, the GEMM's throughput on
  // large ones (measured crossover).
  if ((N + 15) / 16 * (K / kPiece) * (p_tile + x_sums) > kSkMaxMfma) return false;
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
  SkinnyPlan p = plan_skinny(a[0].M, (int)std::min<int64_t>(nsum, INT32_MAX), a[0].K, a[0].bits, a[0].gs, n > 1);
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
