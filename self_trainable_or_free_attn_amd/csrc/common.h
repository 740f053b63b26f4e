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
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
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

// The same global -> LDS transfer written as inline assembly: the compiler does not see these LDS writes, so it
// adds no conservative vmcnt waits before LDS reads of the other buffer (it would otherwise drain the prefetch).
// Visibility is the caller's job: dma_wait() then a barrier before any wave reads what was transferred.
//
// Wait states. The hardware does not interlock two producers of these transfers' operands (CDNA3 / CDNA4 ISA,
// "manually inserted wait states"): an SALU write of M0 needs 1 wait state before an LDS-DMA instruction reads M0,
// and a VALU write of an SGPR (v_readfirstlane, which uni() compiles to) needs 5 before a vector memory
// instruction reads that SGPR (here the buffer resource and the scalar offset). The compiler's hazard recognizer
// inserts them for its own instructions but treats inline assembly as opaque, and its scheduler is free to put
// `s_mov_b32 m0, ...` or the v_readfirstlane of the resource right in front of the asm (the default build did
// both: 80 transfers issued straight after their M0 write, 20 within 1-4 instructions of the readfirstlane of
// their resource). The transfer then reads the previous M0 (and lands in the previous destination) or a stale
// resource (and reads from another address, or faults). So every transfer starts with `s_nop 4`: five wait states
// after whatever the compiler placed before it, whatever the schedule.
typedef int srd_t __attribute__((ext_vector_type(4)));

// raw buffer descriptor over `bytes` bytes from `base` (offsets past it read as zero); must be wave-uniform
__device__ __forceinline__ srd_t make_srd(const void* base, unsigned bytes) {
  const unsigned long long p = (unsigned long long)base;
  srd_t r;
  r.x = (int)(unsigned)p;
  r.y = (int)(unsigned)((p >> 32) & 0xffffu);
  r.z = (int)bytes;
  r.w = 0x00020000;
  return r;
}

__device__ __forceinline__ unsigned lds_addr(const void* p) {
  return (unsigned)(unsigned long long)(const __attribute__((address_space(3))) char*)(p);
}

// the operands of the asm below must sit in SGPRs: make wave-uniformity explicit (free when already uniform)
__device__ __forceinline__ unsigned uni(unsigned x) { return (unsigned)__builtin_amdgcn_readfirstlane((int)x); }
__device__ __forceinline__ srd_t uni(srd_t r) {
  srd_t o;
  o.x = __builtin_amdgcn_readfirstlane(r.x);
  o.y = __builtin_amdgcn_readfirstlane(r.y);
  o.z = __builtin_amdgcn_readfirstlane(r.z);
  o.w = __builtin_amdgcn_readfirstlane(r.w);
  return o;
}

// every lane moves 16 bytes at srd + voff + soff to lds_base + 16 * lane
__device__ __forceinline__ void dma16(srd_t r, const void* lds_base, unsigned voff, unsigned soff) {
  asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               :
               : "v"(voff), "s"(uni(r)), "s"(uni(soff)), "{m0}"(uni(lds_addr(lds_base)))
               : "memory");
}

// dma16 with the LDS destination given as a 32-bit LDS address (no pointer conversion)
__device__ __forceinline__ void dma16_at(srd_t r, unsigned lds, unsigned voff, unsigned soff) {
  asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               :
               : "v"(voff), "s"(uni(r)), "s"(uni(soff)), "{m0}"(uni(lds))
               : "memory");
}

// every lane moves 4 bytes at srd + voff + soff to lds_base + 4 * lane
__device__ __forceinline__ void dma4(srd_t r, const void* lds_base, unsigned voff, unsigned soff) {
  asm volatile("s_nop 4\n\tbuffer_load_dword %0, %1, %2 offen lds"
               :
               : "v"(voff), "s"(uni(r)), "s"(uni(soff)), "{m0}"(uni(lds_addr(lds_base)))
               : "memory");
}

// every vector memory operation of this wave (dma16 / dma4 included) has completed; also a compiler memory barrier.
// The wait is the builtin, not inline assembly: the compiler then knows that its own earlier loads (the query rows
// loaded ahead of a loop, say) have completed too. Behind an assembly wait it still counts them as outstanding and
// places partial vmcnt waits for them in the loop body, where they also wait for the transfers issued by the
// assembly above, which it does not count.
__device__ __forceinline__ void dma_wait() {
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), expcnt / lgkmcnt at their maxima
  asm volatile("" ::: "memory");
}

// uniform load through the scalar cache (the value must not change during the kernel)
template <typename T>
__device__ __forceinline__ T sload(const T* p) {
  return *(const __attribute__((address_space(4))) T*)(p);
}

// s_waitcnt vmcnt(0) (expcnt / lgkmcnt left at their maxima)
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// this lane's value and lane (l ^ 32)'s, the lower half's first, on both lanes (v_permlane32_swap_b32: one VALU
// instruction, where a shuffle across the two 32-lane halves is an LDS round trip). A commutative x op x' is then
// op(.x, .y), the same on both lanes of the pair.
__device__ __forceinline__ float2 lane_pair32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
  const float2 h = lane_pair32(x);
  return fmaxf(h.x, h.y);
}
__device__ __forceinline__ float sum_xor32(float x) {
  const float2 h = lane_pair32(x);
  return h.x + h.y;
}

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

// DPP lane shuffle with zero fill (bound_ctrl) and a row mask; lanes outside the mask read 0
template <int CTRL, int ROWMASK = 0xF>
__device__ __forceinline__ float dpp_f(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROWMASK, 0xF, true));
}

// sum over the 64 lanes with DPP row shifts / broadcasts (no LDS traffic); the result is wave-uniform
__device__ __forceinline__ float wave_sum_dpp(float x) {
  x += dpp_f<0x111>(x);        // row_shr:1
  x += dpp_f<0x112>(x);        // row_shr:2
  x += dpp_f<0x114>(x);        // row_shr:4
  x += dpp_f<0x118>(x);        // row_shr:8   -> lane 16r + 15 holds row r's sum
  x += dpp_f<0x142, 0xA>(x);   // row_bcast:15 -> lanes 31, 63 hold rows 0+1, 2+3
  x += dpp_f<0x143, 0xC>(x);   // row_bcast:31 -> lane 63 holds the total
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 63));
}

// max over the 64 lanes (DPP; lanes without a source keep their own value)
template <int CTRL, int ROWMASK = 0xF>
__device__ __forceinline__ float dpp_keep(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(x), __float_as_int(x), CTRL, ROWMASK, 0xF, false));
}
__device__ __forceinline__ float wave_max_dpp(float x) {
  x = fmaxf(x, dpp_keep<0x111>(x));
  x = fmaxf(x, dpp_keep<0x112>(x));
  x = fmaxf(x, dpp_keep<0x114>(x));
  x = fmaxf(x, dpp_keep<0x118>(x));
  x = fmaxf(x, dpp_keep<0x142, 0xA>(x));
  x = fmaxf(x, dpp_keep<0x143, 0xC>(x));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 63));
}

// sum of the 8 bf16 values of a packed MFMA operand, fp32 accumulate (v_dot2_f32_bf16 against 1.0)
__device__ __forceinline__ float sum8_bf16(bf16x8 v, float acc) {
  const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
  acc = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{v[0], v[1]}, one, acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{v[2], v[3]}, one, acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{v[4], v[5]}, one, acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{v[6], v[7]}, one, acc, false);
  return acc;
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
