/*
 * kh_oracle.c — CPU restatement of Kiln's affine-quantized linear path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker the HIP library is
 * compared against (tests/, __graft_entry__.smoke(), and the cpu_baseline leg
 * of bench.py). Nothing in the product path links or calls it.
 *
 * What it restates:
 *   - the mlx-lm affine format as Kiln loads it
 *     (crates/kiln-models/src/weights.rs:86-102: U32 packed codes, F16/BF16/F32
 *     scales and biases; crates/kiln-models/src/config.rs:137-148: bits 4|8,
 *     group_size 32|64|128) and as MLX v0.31.1 (pinned through mlx-c v0.6.0,
 *     docs/decisions/0001-mlx-c-pin.md:16-21) packs it: code j of a uint32
 *     word is (word >> (bits*j)) & (2^bits - 1) and belongs to column
 *     word_index*(32/bits) + j;
 *   - ops::dequantize (crates/kiln-mlx/src/ops.rs:456-484):
 *     w = scale*q + bias per group of group_size consecutive columns,
 *     evaluated as one float32 fma and rounded once (round-to-nearest-even)
 *     to the output dtype;
 *   - ops::quantized_matmul (ops.rs:359-388), transpose=true
 *     (the form every Kiln call site uses: nn.rs:89, nn.rs:187) and
 *     transpose=false: y = x @ dequant(w)^T or x @ dequant(w), accumulated in
 *     float32 in increasing k order, rounded once to the output dtype;
 *   - Embedding::lookup (crates/kiln-models/src/nn.rs:159-176):
 *     take(w|scales|biases, ids, axis 0) then dequantize;
 *   - the affine quantize of the checkpoint conversion
 *     (crates/kiln-jobs/src/quantize.rs:72-91 runs mlx_lm convert): kho_quantize,
 *     pinned by known answers and round-trip bounds; its bit-level agreement
 *     with MLX itself is "parity unpinned".
 *
 * MLX itself is absent (no install, no network); see the pinning tests for
 * what fixes each function independently.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { O_F16 = 9, O_F32 = 10, O_BF16 = 12, O_U32 = 3, O_I32 = 7 };

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float kho_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* float32 -> bfloat16, round-to-nearest-even; NaN stays a quiet NaN. */
uint16_t kho_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}

/* IEEE binary16 -> float32 (exact). */
float kho_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  if (exp == 0) {
    /* zero or subnormal: man * 2^-24 */
    float v = (float)man * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  if (exp == 31) return u2f(sign | 0x7f800000u | (man << 13) | (man ? 0x400000u : 0));
  return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

/* float32 -> IEEE binary16, round-to-nearest-even, overflow to inf. */
uint16_t kho_f32_to_f16(float f) {
  uint32_t u = f2u(f);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7e00u;           /* NaN */
  if (a >= 0x477ff000u) return sign | 0x7c00u;          /* >= 65520 -> inf */
  if (a < 0x38800000u) {                                /* below 2^-14: subnormal */
    /* value = m * 2^-24 with m = round(a_value * 2^24) */
    float av = u2f(a);
    float scaled = av * 16777216.0f;                    /* exact (power of two) */
    /* round half to even on the integer */
    float fl = floorf(scaled);
    float diff = scaled - fl;
    uint32_t m = (uint32_t)fl;
    if (diff > 0.5f || (diff == 0.5f && (m & 1u))) m += 1u;
    return sign | (uint16_t)m;                          /* m == 0x400 is the min normal */
  }
  uint32_t exp = (a >> 23) - 112u;
  uint32_t man = a & 0x7fffffu;
  uint32_t h = (exp << 10) | (man >> 13);
  uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
  return sign | (uint16_t)h;
}

static inline float load_f(const void* p, int dtype, int64_t i) {
  switch (dtype) {
    case O_F16: return kho_f16_to_f32(((const uint16_t*)p)[i]);
    case O_BF16: return kho_bf16_to_f32(((const uint16_t*)p)[i]);
    default: return ((const float*)p)[i];
  }
}

static inline void store_f(void* p, int dtype, int64_t i, float v) {
  switch (dtype) {
    case O_F16: ((uint16_t*)p)[i] = kho_f32_to_f16(v); break;
    case O_BF16: ((uint16_t*)p)[i] = kho_f32_to_bf16(v); break;
    default: ((float*)p)[i] = v; break;
  }
}

static inline uint32_t code_at(const uint32_t* row, int64_t k, int bits) {
  int per = 32 / bits;
  return (row[k / per] >> (bits * (k % per))) & ((1u << bits) - 1u);
}

/* codes[r, k] for a [rows, K*bits/32] packed matrix. */
void kho_unpack(const uint32_t* w, int64_t rows, int64_t K, int bits, uint8_t* codes) {
  int64_t wpr = K * bits / 32;
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t k = 0; k < K; ++k) codes[r * K + k] = (uint8_t)code_at(w + r * wpr, k, bits);
}

/* Pack codes[rows, K] (values < 2^bits) little-end-first into uint32. */
void kho_pack(const uint8_t* codes, int64_t rows, int64_t K, int bits, uint32_t* w) {
  int per = 32 / bits;
  int64_t wpr = K / per;
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t i = 0; i < wpr; ++i) {
      uint32_t word = 0;
      for (int j = 0; j < per; ++j)
        word |= ((uint32_t)codes[r * K + i * per + j] & ((1u << bits) - 1u)) << (bits * j);
      w[r * wpr + i] = word;
    }
}

static inline float dq(const uint32_t* wrow, const void* s, const void* b, int sdt,
                       int64_t sbase, int64_t k, int gs, int bits) {
  float sc = load_f(s, sdt, sbase + k / gs);
  float bi = load_f(b, sdt, sbase + k / gs);
  return fmaf(sc, (float)code_at(wrow, k, bits), bi);
}

/* res[r, k] = round_odt(fma(s, q, b)); rows of K columns. */
void kho_dequantize(const uint32_t* w, const void* s, const void* b, int sdt, int64_t rows,
                    int64_t K, int gs, int bits, void* out, int odt) {
  int64_t wpr = K * bits / 32, G = K / gs;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t k = 0; k < K; ++k)
      store_f(out, odt, r * K + k, dq(w + r * wpr, s, b, sdt, r * G, k, gs, bits));
}

/* Affine quantization of rows of K values (dtype wdt) in groups of gs, as
 * MLX v0.31.1 computes it (mlx_quantize, mode "affine"; the algorithm of
 * MLX's affine_quantize, restated: Kiln itself quantizes through mlx_lm
 * convert, crates/kiln-jobs/src/quantize.rs:72-91). Per group, in float32:
 *   lo, hi = min, max of the group;  nb = 2^bits - 1
 *   s = max((hi - lo) / nb, 1e-7);  side = |lo| > |hi|
 *   s = side ? s : -s;  edge = side ? lo : hi
 *   q0 = round(edge / s)                      (round: half away from zero)
 *   s = q0 != 0 ? edge / q0 : s;  b = q0 != 0 ? edge : 0
 *   code_k = min(max(round((w_k - b) / s), 0), nb)
 * scales and biases are stored in wdt (round to nearest even); the codes use
 * the float32 s and b. Codes are packed lowest bits first. */
void kho_quantize(const void* w, int wdt, int64_t rows, int64_t K, int gs, int bits,
                  uint32_t* wq, void* s_out, void* b_out) {
  const float nb = (float)((1 << bits) - 1);
  const int64_t G = K / gs, wpr = K * bits / 32;
  const int per = 32 / bits;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t g = 0; g < G; ++g) {
      const int64_t base = r * K + g * gs;
      float lo = load_f(w, wdt, base), hi = lo;
      for (int k = 1; k < gs; ++k) {
        const float v = load_f(w, wdt, base + k);
        lo = fminf(lo, v);
        hi = fmaxf(hi, v);
      }
      float sc = fmaxf((hi - lo) / nb, 1e-7f);
      const int side = fabsf(lo) > fabsf(hi);
      sc = side ? sc : -sc;
      const float edge = side ? lo : hi;
      const float q0 = roundf(edge / sc);
      float bi = 0.f;
      if (q0 != 0.f) {
        sc = edge / q0;
        bi = edge;
      }
      store_f(s_out, wdt, r * G + g, sc);
      store_f(b_out, wdt, r * G + g, bi);
      for (int k = 0; k < gs; k += per) {
        uint32_t word = 0;
        for (int j = 0; j < per; ++j) {
          const float v = roundf((load_f(w, wdt, base + k + j) - bi) / sc);
          const float c = fminf(fmaxf(v, 0.f), nb);
          word |= (uint32_t)c << (bits * j);
        }
        wq[r * wpr + (g * gs + k) / per] = word;
      }
    }
  }
}

/* Float32 result of quantized_matmul (before output rounding), x [M,K].
 * transpose=1: w [N, K*bits/32], s/b [N, K/gs]; y[m,n] = sum_k x[m,k]*W[n,k].
 * transpose=0: w [K, N*bits/32], s/b [K, N/gs]; y[m,n] = sum_k x[m,k]*W[k,n].
 * Accumulation: acc = fma(x, w, acc) for k = 0..K-1 in order, acc from 0. */
void kho_qmm_f32(const void* x, int xdt, const uint32_t* w, const void* s, const void* b,
                 int sdt, int64_t M, int64_t N, int64_t K, int gs, int bits, int transpose,
                 float* y) {
  if (transpose) {
    int64_t wpr = K * bits / 32, G = K / gs;
#pragma omp parallel
    {
      float* wrow = (float*)malloc(sizeof(float) * (size_t)(K > 0 ? K : 1));
#pragma omp for schedule(static)
      for (int64_t n = 0; n < N; ++n) {
        for (int64_t k = 0; k < K; ++k) wrow[k] = dq(w + n * wpr, s, b, sdt, n * G, k, gs, bits);
        for (int64_t m = 0; m < M; ++m) {
          float acc = 0.0f;
          for (int64_t k = 0; k < K; ++k) acc = fmaf(load_f(x, xdt, m * K + k), wrow[k], acc);
          y[m * N + n] = acc;
        }
      }
      free(wrow);
    }
  } else {
    int64_t wpr = N * bits / 32, G = N / gs;
#pragma omp parallel
    {
      float* wcol = (float*)malloc(sizeof(float) * (size_t)(K > 0 ? K : 1));
#pragma omp for schedule(static)
      for (int64_t n = 0; n < N; ++n) {
        for (int64_t k = 0; k < K; ++k) wcol[k] = dq(w + k * wpr, s, b, sdt, k * G, n, gs, bits);
        for (int64_t m = 0; m < M; ++m) {
          float acc = 0.0f;
          for (int64_t k = 0; k < K; ++k) acc = fmaf(load_f(x, xdt, m * K + k), wcol[k], acc);
          y[m * N + n] = acc;
        }
      }
      free(wcol);
    }
  }
}

/* quantized_matmul rounded to odt. */
void kho_qmm(const void* x, int xdt, const uint32_t* w, const void* s, const void* b, int sdt,
             int64_t M, int64_t N, int64_t K, int gs, int bits, int transpose, void* out,
             int odt) {
  float* y = (float*)malloc(sizeof(float) * (size_t)(M * N > 0 ? M * N : 1));
  kho_qmm_f32(x, xdt, w, s, b, sdt, M, N, K, gs, bits, transpose, y);
  for (int64_t i = 0; i < M * N; ++i) store_f(out, odt, i, y[i]);
  free(y);
}

/* take(a, ids, axis 0) for rows of `row_bytes`; out-of-range ids -> zero row,
 * negative int32 ids wrap once (MLX take). */
static int64_t resolve_id(const void* ids, int idt, int64_t t, int64_t V) {
  int64_t id = idt == O_I32 ? (int64_t)((const int32_t*)ids)[t] : (int64_t)((const uint32_t*)ids)[t];
  if (id < 0) id += V;
  return (id < 0 || id >= V) ? -1 : id;
}

void kho_take(const void* a, int64_t V, int64_t row_bytes, const void* ids, int idt, int64_t T,
              void* out) {
  for (int64_t t = 0; t < T; ++t) {
    int64_t id = resolve_id(ids, idt, t, V);
    if (id < 0) memset((char*)out + t * row_bytes, 0, (size_t)row_bytes);
    else memcpy((char*)out + t * row_bytes, (const char*)a + id * row_bytes, (size_t)row_bytes);
  }
}

/* Embedding::lookup: gather rows then dequantize them. */
void kho_embedding(const void* ids, int idt, int64_t T, const uint32_t* w, const void* s,
                   const void* b, int sdt, int64_t V, int64_t H, int gs, int bits, void* out,
                   int odt) {
  int64_t wpr = H * bits / 32, G = H / gs;
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < T; ++t) {
    int64_t id = resolve_id(ids, idt, t, V);
    for (int64_t k = 0; k < H; ++k) {
      float v = id < 0 ? 0.0f : dq(w + id * wpr, s, b, sdt, id * G, k, gs, bits);
      store_f(out, odt, t * H + k, v);
    }
  }
}

/* Threads the OpenMP loops above run with. */
int kho_threads(void) {
#ifdef _OPENMP
  extern int omp_get_max_threads(void);
  return omp_get_max_threads();
#else
  return 1;
#endif
}
