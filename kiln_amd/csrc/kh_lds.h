// kh_lds.h — direct global->LDS loads and hand-counted waits, shared by the
// kernels that stream operands through LDS rings (kh_gemm.hip, kh_skinny.hip).
#pragma once

#include "kh_common.h"

namespace kh {

typedef __attribute__((address_space(3))) void lds_void;

// s_waitcnt vmcnt(N) leaving expcnt and lgkmcnt unconstrained (gfx9
// encoding: vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14).
template <int N>
__device__ __forceinline__ void waitcnt_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// LDS reads issued by inline asm, which the compiler's wait insertion does
// not see: it treats an LDS read as possibly aliasing the direct-to-LDS
// loads in flight and would put a full wait before it, exposing the LDS
// latency at every read. The data read must have been completed by a vmcnt
// wait and a barrier. lds_wait_all() waits for these reads; ready(v) orders
// a use of v after that wait.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}
__device__ __forceinline__ uint32_t lds_u16_nowait(const void* p) {
  uint32_t v;
  asm volatile("ds_read_u16 %0, %1" : "=v"(v) : "v"(lds_addr(p)));
  return v;
}
__device__ __forceinline__ uint32_t lds_b32_nowait(const void* p) {
  uint32_t v;
  asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(lds_addr(p)));
  return v;
}
__device__ __forceinline__ u32x2 lds_b64_nowait(const void* p) {
  u32x2 v;
  asm volatile("ds_read_b64 %0, %1" : "=v"(v) : "v"(lds_addr(p)));
  return v;
}
__device__ __forceinline__ u32x4 lds_b128_nowait(const void* p) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(lds_addr(p)));
  return v;
}
__device__ __forceinline__ void lds_wait_all() { asm volatile("s_waitcnt lgkmcnt(0)" ::); }
__device__ __forceinline__ void ready(uint32_t& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void ready(u32x2& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void ready(u32x4& v) { asm volatile("" : "+v"(v)); }

}  // namespace kh
