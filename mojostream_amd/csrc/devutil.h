// Device helpers shared by the Q4 kernels (GEMV and GEMM).
#pragma once
#include "common.h"

namespace ms {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Global-memory loads through an explicit global pointer: generic (flat)
// loads also count against the LDS wait counter, so an LDS wait would stall
// on them.
template <class T>
__device__ inline T ldg(const void *p) {
  return *(const __attribute__((address_space(1))) T *)p;
}
template <>
__device__ inline float4 ldg<float4>(const void *p) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  const f32x4 v = *(const __attribute__((address_space(1))) f32x4 *)p;
  return float4{v.x, v.y, v.z, v.w};
}

// Streaming load (non-temporal hint): data read once, which should not
// displace reused data from the caches.
template <class T>
__device__ inline T ldg_nt(const void *p) {
  return __builtin_nontemporal_load((const __attribute__((address_space(1))) T *)p);
}

// A uniform value passed through an opaque register move: the compiler can no
// longer turn selects between such values back into an indexed memory access
// (which would put them in scratch memory or re-read the argument struct).
template <class T>
__device__ inline T launder(T v) {
  asm volatile("" : "+s"(v));
  return v;
}

// Low nibbles of the four bytes of d as bytes 0..15 (the zero point is added
// separately, with a constant -8 operand).
__device__ inline int nib_u8(uint32_t d) { return (int)(d & 0x0F0F0F0Fu); }

// Low nibbles of the four bytes of d as signed bytes n - 8 (the Q4 zero point
// folded into the operand): n + 0x78 stays inside its byte for n <= 15, and
// flipping bit 7 turns it into the two's complement of n - 8.
__device__ inline int nib_s8(uint32_t d) {
  return (int)(((d & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u);
}

}  // namespace ms
