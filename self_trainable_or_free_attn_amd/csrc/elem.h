// Token element type of the VSA kernels. Every VSA source is compiled twice: as is for bf16, and with ES_ELEM_F16
// defined for fp16, in which build the C entry points that read or write token tensors carry the suffix _f16
// (the reference dispatches the same kernels on the tensor dtype, csrc/vsa/vsa2_api.cpp:51 and its run_* switches).
// The kernels are written once against these names:
//   e16_t         raw 16-bit token value in global / LDS memory
//   elem_t, ev8   the scalar / 8-wide MFMA operand type
//   emfma         v_mfma_f32_32x32x16_{bf16,f16}
//   e2f, f2e      16-bit bits <-> float (round to nearest even)
//   epack8, esum8 floats -> one MFMA operand; the fp32 sum of an operand's 8 values (v_dot2 against 1.0)
//   elds16, ecat_tr  LDS row read / two transposed half-reads as one operand
#pragma once
#include "common.h"

namespace es {

typedef unsigned short e16_t;

#ifdef ES_ELEM_F16

typedef _Float16 elem_t;
typedef _Float16 ev8 __attribute__((ext_vector_type(8)));
typedef _Float16 ev2 __attribute__((ext_vector_type(2)));
#define ES_VSA_API(name) name##_f16

__device__ __forceinline__ f32x16 emfma(ev8 a, ev8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float e2f(e16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
__device__ __forceinline__ e16_t f2e(float f) { return __builtin_bit_cast(e16_t, (_Float16)f); }
__device__ __forceinline__ float esum8(ev8 v, float acc) {
  const ev2 one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
  for (int i = 0; i < 8; i += 2) acc = __builtin_amdgcn_fdot2(ev2{v[i], v[i + 1]}, one, acc, false);
  return acc;
}

#else

typedef __bf16 elem_t;
typedef bf16x8 ev8;
#define ES_VSA_API(name) name

__device__ __forceinline__ f32x16 emfma(ev8 a, ev8 b, f32x16 c) { return mfma32(a, b, c); }
__device__ __forceinline__ float e2f(e16_t b) { return bf2f(b); }
__device__ __forceinline__ e16_t f2e(float f) { return f2bf(f); }
__device__ __forceinline__ float esum8(ev8 v, float acc) { return sum8_bf16(v, acc); }

#endif

// a * b rounded to float32 as a separate step: the fp16 build would otherwise fuse the product and a following
// conversion into one v_fma_mix (one rounding instead of the reference's two). The empty asm makes the product
// opaque to that combine and costs no instruction.
__device__ __forceinline__ float mul_rn(float a, float b) {
  float r = a * b;
  asm volatile("" : "+v"(r));
  return r;
}

__device__ __forceinline__ ev8 epack8(const float* p) {
  ev8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (elem_t)p[i];
  return r;
}

__device__ __forceinline__ ev8 elds16(const char* base, int off) {
  return *reinterpret_cast<const __attribute__((address_space(3))) ev8*>(LDS_PTR(const char, base) + off);
}

__device__ __forceinline__ ev8 ecat_tr(s16x4 a, s16x4 b) {
  ev8 r;
  s16x4 x[2] = {a, b};
  __builtin_memcpy(&r, x, 16);
  return r;
}

}  // namespace es
