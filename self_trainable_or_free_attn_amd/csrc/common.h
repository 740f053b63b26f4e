// Shared device helpers for the gfx950 (CDNA4) kernels of the EchoSparse / VSA hot path.
//
// Conventions used by every kernel in this directory:
//  * bf16 MFMA tiles are v_mfma_f32_32x32x16_bf16 (wave64). Operand layouts (checked on the GPU):
//      A (32x16): lane l holds A[l % 32][8 * (l / 32) + 0..7]
//      B (16x32): lane l holds B[8 * (l / 32) + 0..7][l % 32]
//      C (32x32): lane l, register r holds C[8 * (r / 4) + 4 * (l / 32) + r % 4][l % 32]
//  * Attention computes S^T = K Q^T (keys in registers, queries across lanes) so that the exponentiated tile is
//    already the B operand of O^T += V^T P^T; V^T comes out of LDS with ds_read_b64_tr_b16, whose semantics (also
//    checked on the GPU) are: in each 16-lane group, lane i receives element (i % 4) of the 8-byte chunks that
//    source lanes 4j + i / 4 addressed, j = 0..3.
//  * 64-row x 256-byte K / V tiles live in LDS with a 16-byte-chunk XOR swizzle, chunk' = chunk ^ sw(row),
//    sw(row) = ((row & 3) << 2) | ((row >> 2) & 3): conflict-free for the row-per-lane K reads and for the
//    4-rows-per-16-lanes transposed V reads.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef unsigned short bf16_t;  // raw bf16 bits in global memory

#define LDS_PTR(T, p) ((__attribute__((address_space(3))) T*)(p))

namespace es {

constexpr int BM = 128;   // query rows per tile (EchoSparse)
constexpr int BK = 64;    // tokens per kv block
constexpr int HD = 128;   // head dimension supported by the MFMA kernels
constexpr float LOG2E = 1.4426950408889634f;

__device__ __forceinline__ int lane_id() { return __lane_id(); }

__device__ __forceinline__ int swz(int row) { return ((row & 3) << 2) | ((row >> 2) & 3); }

// byte offset of logical 16-byte chunk c of row `row` in a swizzled 256-byte-row tile
__device__ __forceinline__ int tile_off(int row, int c) { return row * 256 + ((c ^ swz(row)) << 4); }

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 lds_read16(const char* base, int off) {
  return *reinterpret_cast<const __attribute__((address_space(3))) bf16x8*>(LDS_PTR(const char, base) + off);
}

__device__ __forceinline__ s16x4 lds_read_tr(const char* base, int off) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(s16x4, const_cast<char*>(base) + off));
}

__device__ __forceinline__ bf16x8 cat_tr(s16x4 a, s16x4 b) {
  bf16x8 r;
  s16x4 x[2] = {a, b};
  __builtin_memcpy(&r, x, 16);
  return r;
}

// one wave instruction: every lane moves 16 bytes from its own global address to lds_base + 16 * lane
__device__ __forceinline__ void g2lds16(const void* gsrc, char* lds_base) {
  __builtin_amdgcn_global_load_lds(gsrc, LDS_PTR(void, lds_base), 16, 0, 0);
}

// s_waitcnt vmcnt(0) (expcnt / lgkmcnt left at their maxima)
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m, 64);
  return x;
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x = fmaxf(x, __shfl_xor(x, m, 64));
  return x;
}

__device__ __forceinline__ int wave_sum_i(int x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m, 64);
  return x;
}

__device__ __forceinline__ float exp2f_fast(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float bf2f(bf16_t b) { return __uint_as_float(((unsigned)b) << 16); }

// round-to-nearest-even float -> bf16 bits (NaN kept quiet)
__device__ __forceinline__ bf16_t f2bf(float f) {
  unsigned u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (bf16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (bf16_t)(u >> 16);
}

__device__ __forceinline__ bf16x8 pack8(const float* p) {
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (__bf16)p[i];
  return r;
}

}  // namespace es

// --------------------------------------------------------------------------------------------- host side
#include <string>
namespace es {
void set_error(const std::string& msg);
int check_launch(const char* what);
}  // namespace es

#define ES_REQUIRE(cond, code, msg)          \
  do {                                       \
    if (!(cond)) {                           \
      es::set_error(msg);                    \
      return code;                           \
    }                                        \
  } while (0)
