// kh_common.h — shared device helpers for the gfx950 quantized-linear kernels.
#pragma once

#include <type_traits>

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/kiln_hip.h"

namespace kh {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;
typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2;

// Element types the kernels read and write (values of kh_dtype).
enum : int { DT_F16 = KH_FLOAT16, DT_F32 = KH_FLOAT32, DT_BF16 = KH_BFLOAT16 };

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}

// float -> bfloat16 bits, round-to-nearest-even; NaN stays a quiet NaN.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  // round to nearest even; NaN keeps its top bits with the quiet bit set.
  // Both results are computed and one selected (an if compiles to an
  // exec-mask branch per element).
  const uint32_t u = __float_as_uint(f);
  const uint32_t rne = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const uint32_t qnan = (u >> 16) | 0x40u;
  return (u & 0x7fffffffu) > 0x7f800000u ? qnan : rne;
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// float -> binary16 bits, round-to-nearest-even (hardware conversion).
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

// Load element i of a float array of dtype dt as float32 (exact).
__device__ __forceinline__ float load_as_f32(const void* p, int dt, int64_t i) {
  if (dt == DT_F32) return static_cast<const float*>(p)[i];
  uint32_t h = static_cast<const uint16_t*>(p)[i];
  return dt == DT_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
}

// Round v to dtype dt and store it as element i.
__device__ __forceinline__ void store_from_f32(void* p, int dt, int64_t i, float v) {
  if (dt == DT_F32) {
    static_cast<float*>(p)[i] = v;
  } else {
    uint32_t h = dt == DT_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
    static_cast<uint16_t*>(p)[i] = (uint16_t)h;
  }
}

// Maximum of v over the 64 lanes of a wave, in every lane, by cross-lane
// moves that stay in the VALU: DPP within 16-lane rows (l ^ 1, l ^ 2, the
// mirror within 8 and within 16 lanes), then v_permlane16_swap and
// v_permlane32_swap across rows (a ds_bpermute per step would be a round
// trip through the LDS crossbar). The maximum does not depend on the order.
__device__ __forceinline__ float wave_max(float v) {
  auto dpp = [](float a, auto ctrl) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, a), decltype(ctrl)::value, 0xf, 0xf, false));
  };
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0xb1>{}));
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0x4e>{}));
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0x141>{}));
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0x140>{}));
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto r16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  v = fmaxf(__builtin_bit_cast(float, (unsigned)r16[0]), __builtin_bit_cast(float, (unsigned)r16[1]));
  const unsigned w = __builtin_bit_cast(unsigned, v);
  const auto r32 = __builtin_amdgcn_permlane32_swap(w, w, false, false);
  return fmaxf(__builtin_bit_cast(float, (unsigned)r32[0]), __builtin_bit_cast(float, (unsigned)r32[1]));
}

// v rounded to dtype dt (round-to-nearest-even) and read back as float32.
__device__ __forceinline__ float round_to(float v, int dt) {
  if (dt == DT_F32) return v;
  return dt == DT_BF16 ? bf16_bits_to_f32(f32_to_bf16_bits(v)) : f16_bits_to_f32(f32_to_f16_bits(v));
}

// The gated-MLP activation of Kiln's llama/qwen MLP (crates/kiln-models/src/
// nn.rs:284-294): silu(gate) * up = gate * sigmoid(gate) * up, with every
// intermediate an array of the output dtype dt as in the reference's op
// graph: gate and up rounded to dt, sigmoid evaluated in float32 from the
// rounded gate and rounded, gate*sigmoid rounded, and the final product
// returned in float32 for the caller's single rounding store.
__device__ __forceinline__ float silu_mul(float g, float u, int dt) {
  g = round_to(g, dt);
  u = round_to(u, dt);
  const float sg = round_to(1.f / (1.f + expf(-g)), dt);
  const float a = round_to(g * sg, dt);
  return a * u;
}

// gelu_approx(gate) * up of Kiln's gemma MLP (crates/kiln-models/src/nn.rs:
// 221-235, 284-294), with every intermediate an array of dtype dt as in the
// reference's op graph (scalars are weak: converted to dt first):
//   cube = g^3; inner = g + 0.044715*cube; scaled = sqrt(2/pi)*inner;
//   gate = 1 + tanh(scaled); act = (0.5*g)*gate; result act*up,
// each op evaluated in float32 and rounded to dt. The cube is formed as
// (g*g)*g in float32 (MLX's power(x, 3) differs at most in the last float32
// bit). Returned in float32 for the caller's single rounding store.
__device__ __forceinline__ float gelu_mul(float g, float u, int dt) {
  g = round_to(g, dt);
  u = round_to(u, dt);
  const float c1 = round_to(0.044715f, dt), c2 = round_to(0.7978845608028654f, dt);
  const float cube = round_to((g * g) * g, dt);
  const float inner = round_to(g + round_to(c1 * cube, dt), dt);
  const float scaled = round_to(c2 * inner, dt);
  const float gate = round_to(1.f + round_to(tanhf(scaled), dt), dt);
  const float act = round_to(round_to(0.5f * g, dt) * gate, dt);
  return act * u;
}

// Activation of the gated MLP (Kiln's Activation enum, nn.rs:259-294).
enum : int { ACT_SILU = 0, ACT_GELU_APPROX = 1 };
__device__ __forceinline__ float act_mul(float g, float u, int dt, int act) {
  return act == ACT_GELU_APPROX ? gelu_mul(g, u, dt) : silu_mul(g, u, dt);
}

// Epilogue of Linear::forward (crates/kiln-models/src/nn.rs:79-102): the
// product is an array of dtype ydt, then `+ bias` (ops::add) forms the sum of
// that rounded product and the bias in float32; the caller's store rounds the
// sum to the result dtype. Without a bias the product passes unchanged.
struct Epilogue {
  const void* bias;  // [N] or nullptr
  int bdt, ydt;
  __device__ __forceinline__ float operator()(float v, int64_t n) const {
    return bias ? round_to(v, ydt) + load_as_f32(bias, bdt, n) : v;
  }
};

// Round a pair to dt and pack the two 16-bit results (lo = a).
__device__ __forceinline__ uint32_t pack2(float a, float b, int dt) {
  uint32_t ha = dt == DT_BF16 ? f32_to_bf16_bits(a) : f32_to_f16_bits(a);
  uint32_t hb = dt == DT_BF16 ? f32_to_bf16_bits(b) : f32_to_f16_bits(b);
  return ha | (hb << 16);
}

// v_perm_b32: byte i of the result is byte sel_i of the 8-byte value {hi, lo}.
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// Pair order in which the decode kernels turn packed codes into 16-bit
// operand pairs; activations are permuted to match. 4-bit word -> (c0,c4)(c1,c5)(c2,c6)(c3,c7);
// 8-bit word pair -> (c0,c2)(c1,c3)(c4,c6)(c5,c7).
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

// Pairs of codes as float16 (1024 + q) in both halves (exact for q < 1024),
// in the pair order of permute_x: 4-bit word -> (c0,c4)(c1,c5)(c2,c6)(c3,c7);
// 8-bit word pair -> (c0,c2)(c1,c3)(c4,c6)(c5,c7).
template <int BITS>
__device__ __forceinline__ void pairs_1024(uint32_t q0, uint32_t q1, uint32_t mag, uint32_t* r) {
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

// Offset (codes) of the 8-code block lane group lg contributes to MFMA step j
// of a stage: 4-bit lanes hold 32 consecutive codes (16 bytes), step j takes
// word j; 8-bit lanes hold two 16-code runs 64 apart, step j takes words
// 2(j%2), 2(j%2)+1 of run j/2.
template <int BITS>
__device__ __forceinline__ int step_off(int j, int lg) {
  return BITS == 4 ? lg * 32 + 8 * j : (j >> 1) * 64 + lg * 16 + (j & 1) * 8;
}

}  // namespace kh
