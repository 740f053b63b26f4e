// VSA / VSA2 elementwise passes: pooling, gate fusion (forward / backward) and the coarse-unpool finalize.
//
// Token tensors are [BH, L, D] bf16 with L = NB * 64 in block-major order; blk_cnt [NB] holds the valid tokens of
// each 64-token block (valid-first: rows >= blk_cnt of a block are padding). D = 128. Pooled tensors are
// [BH, rows_pad, D] with rows_pad a multiple of 64; their padding rows are left untouched (callers zero them).
//
// Every kernel here moves each token row once and is HBM-bound. A 16-lane DPP row of a wave covers one 256-byte
// token row with 16-byte accesses, so row reductions stay inside one DPP row, and a workgroup takes four
// consecutive 64-token blocks of one head.
//
//   pool_kernel      reference csrc/vsa/router/pool.cu:16-51 (router group means of R tokens, whole-block means)
//   fuse_fwd_kernel  reference csrc/vsa/fuse.cu:3 (O = O_f + act(gate) * O_c[blk] on valid rows, 0 elsewhere)
//   fuse_bwd_kernel  reference csrc/vsa/fuse.cu:4-8 (dO_f, delta_f, dO_c, delta_c, dgate)
//   finalize_kernel  reference csrc/vsa/fuse.cu:9 (dX = acc + add[blk] / cnt on valid rows, 0 elsewhere)
#include "../../include/vsa_hip.h"
#include "common.h"
#include "elem.h"

namespace es {

namespace {

__device__ __forceinline__ void ld8(const e16_t* p, float* x) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  const unsigned w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = e2f((e16_t)(w[i] & 0xffffu));
    x[2 * i + 1] = e2f((e16_t)(w[i] >> 16));
  }
}

__device__ __forceinline__ void st8(e16_t* p, const float* x) {
  uint4 u;
  u.x = (unsigned)f2e(x[0]) | ((unsigned)f2e(x[1]) << 16);
  u.y = (unsigned)f2e(x[2]) | ((unsigned)f2e(x[3]) << 16);
  u.z = (unsigned)f2e(x[4]) | ((unsigned)f2e(x[5]) << 16);
  u.w = (unsigned)f2e(x[6]) | ((unsigned)f2e(x[7]) << 16);
  *reinterpret_cast<uint4*>(p) = u;
}

// gate activations: 0 = tanh, 1 = identity; the derivative is written in terms of a = act(g)
__device__ __forceinline__ float gact(float g, int act) { return act == 0 ? tanhf(g) : g; }
__device__ __forceinline__ float gdact(float a, int act) { return act == 0 ? 1.f - a * a : 1.f; }

// sum over the 16 lanes of one DPP row
__device__ __forceinline__ float row16_sum(float x) {
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) x += __shfl_xor(x, m, 16);
  return x;
}

struct PoolArgs {
  const e16_t* src[3];  // q, k, v
  e16_t* grp[3];        // qr, kr, vr (any may be null)
  e16_t* blk[3];        // qc, kc, vc
  const int* blk_cnt;
  int NB, L, R, G, Lr_pad, NBc_pad;
};

constexpr int POOL_BLOCKS = 4;  // 64-token blocks per workgroup

// grid (cdiv(NB, 4), BH), 192 threads: 48 per block = 3 tensors x 16 chunks of 8 columns. Each column sums its
// group's rows in order, then the group sums in order, so the float result is that of a sequential loop.
__global__ __launch_bounds__(192) void pool_kernel(PoolArgs a) {
  const int sub = threadIdx.x / 48, t = threadIdx.x % 48;
  const int blk = blockIdx.x * POOL_BLOCKS + sub;
  const int which = t / 16, c8 = (t % 16) * 8;
  if (blk >= a.NB || a.src[which] == nullptr) return;  // a null source: that tensor is not pooled
  const size_t bh = blockIdx.y;
  const int n = a.blk_cnt[blk];
  const e16_t* src = a.src[which] + (bh * a.L + (size_t)blk * BK) * HD + c8;
  e16_t* grp = a.grp[which];
  float tot[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int g = 0; g < a.G; ++g) {
    const int r0 = g * a.R, r1 = min(r0 + a.R, n);
    float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int r = r0; r < r1; ++r) {
      float x[8];
      ld8(src + (size_t)r * HD, x);
#pragma unroll
      for (int e = 0; e < 8; ++e) s[e] += x[e];
    }
    if (grp != nullptr) {
      const float inv = r1 > r0 ? 1.f / (float)(r1 - r0) : 0.f;
      float m[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) m[e] = mul_rn(s[e], inv);
      st8(grp + (bh * a.Lr_pad + (size_t)blk * a.G + g) * HD + c8, m);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) tot[e] += s[e];
  }
  const float inv = 1.f / (float)n;
#pragma unroll
  for (int e = 0; e < 8; ++e) tot[e] = mul_rn(tot[e], inv);
  st8(a.blk[which] + (bh * a.NBc_pad + blk) * HD + c8, tot);
}

// lane -> (row slot s = lane / 16, column chunk c8 = 8 * (lane % 16)); the slot walks rows s, s + 4, ..., s + 60
struct FuseArgs {
  const e16_t *dout, *of, *oc, *gate;
  e16_t *o, *dout_f, *dout_c, *dgate;
  float *delta_f, *delta_c;
  const int* blk_cnt;
  int NB, L, NBc_pad, gate_mode, gate_act;
};

// grid (cdiv(NB, 4), BH), 256 threads: one wave per 64-token block
__global__ __launch_bounds__(256) void fuse_fwd_kernel(FuseArgs a) {
  const int blk = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (blk >= a.NB) return;
  const int l = threadIdx.x & 63, s = l >> 4, c8 = (l & 15) * 8;
  const size_t bh = blockIdx.y;
  const int n = a.blk_cnt[blk];
  float c[8];
  ld8(a.oc + (bh * a.NBc_pad + blk) * HD + c8, c);
  const size_t tok0 = bh * a.L + (size_t)blk * BK;
#pragma unroll 4
  for (int r = s; r < BK; r += 4) {
    const size_t tok = tok0 + r;
    float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (r < n) {
      ld8(a.of + tok * HD + c8, x);
      if (a.gate_mode == 1) {
        const float g = gact(e2f(a.gate[tok]), a.gate_act);
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] += g * c[e];
      } else if (a.gate_mode == 2) {
        float g[8];
        ld8(a.gate + tok * HD + c8, g);
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] += gact(g[e], a.gate_act) * c[e];
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] += c[e];
      }
    }
    st8(a.o + tok * HD + c8, x);
  }
}

__global__ __launch_bounds__(256) void fuse_bwd_kernel(FuseArgs a) {
  const int blk = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (blk >= a.NB) return;
  const int l = threadIdx.x & 63, s = l >> 4, c8 = (l & 15) * 8;
  const size_t bh = blockIdx.y;
  const int n = a.blk_cnt[blk];
  const size_t crow = (bh * a.NBc_pad + blk) * HD;
  float c[8], dc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  ld8(a.oc + crow + c8, c);
  const size_t tok0 = bh * a.L + (size_t)blk * BK;
  for (int r = s; r < BK; r += 4) {
    const size_t tok = tok0 + r;
    const bool valid = r < n;
    float d[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, f[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (valid) {
      ld8(a.dout + tok * HD + c8, d);
      ld8(a.of + tok * HD + c8, f);
    }
    if (a.dout_f != nullptr) st8(a.dout_f + tok * HD + c8, d);
    float dot_f = 0.f, dot_c = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) dot_f += d[e] * f[e];
    if (a.gate_mode == 1) {
      const float g = valid ? gact(e2f(a.gate[tok]), a.gate_act) : 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        dot_c += d[e] * c[e];
        dc[e] += g * d[e];
      }
      dot_c *= gdact(g, a.gate_act);
    } else if (a.gate_mode == 2) {
      float g[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, dg[8];
      if (valid) ld8(a.gate + tok * HD + c8, g);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float ge = valid ? gact(g[e], a.gate_act) : 0.f;
        dg[e] = valid ? gdact(ge, a.gate_act) * d[e] * c[e] : 0.f;
        dc[e] += ge * d[e];
      }
      st8(a.dgate + tok * HD + c8, dg);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) dc[e] += d[e];
    }
    dot_f = row16_sum(dot_f);
    dot_c = row16_sum(dot_c);
    if ((l & 15) == 0) {
      a.delta_f[tok] = valid ? dot_f : 0.f;
      if (a.gate_mode == 1) a.dgate[tok] = f2e(valid ? dot_c : 0.f);
    }
  }
  // dO_c = the four row slots' column sums (fixed order), rounded; delta_c = <dO_c (rounded), O_c>
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    dc[e] += __shfl_xor(dc[e], 16);
    dc[e] = sum_xor32(dc[e]);
  }
  float part = 0.f;
  if (s == 0) {
    st8(a.dout_c + crow + c8, dc);
#pragma unroll
    for (int e = 0; e < 8; ++e) part += e2f(f2e(dc[e])) * c[e];
  }
  part = row16_sum(part);
  if (l == 0) a.delta_c[bh * a.NBc_pad + blk] = part;
}

// grid (cdiv(NB, 4), BH), 256 threads: one wave per 64-token block; acc fp32 [BH, L, D] (optional), add fp32
// [BH, add_nb, D] (optional)
__global__ __launch_bounds__(256) void finalize_kernel(const float* __restrict__ acc, const float* __restrict__ add,
                                                       e16_t* __restrict__ out, const int* __restrict__ blk_cnt,
                                                       int NB, int L, int add_nb) {
  const int blk = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (blk >= NB) return;
  const int l = threadIdx.x & 63, s = l >> 4, c8 = (l & 15) * 8;
  const size_t bh = blockIdx.y;
  const int n = blk_cnt[blk];
  float ad[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (add != nullptr) {
    const float inv = 1.f / (float)n;
    const float4* p = reinterpret_cast<const float4*>(add + (bh * add_nb + blk) * HD + c8);
    const float4 u = p[0], w = p[1];
    ad[0] = u.x * inv; ad[1] = u.y * inv; ad[2] = u.z * inv; ad[3] = u.w * inv;
    ad[4] = w.x * inv; ad[5] = w.y * inv; ad[6] = w.z * inv; ad[7] = w.w * inv;
  }
  const size_t tok0 = bh * L + (size_t)blk * BK;
#pragma unroll 4
  for (int r = s; r < BK; r += 4) {
    const size_t tok = tok0 + r;
    float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (r < n) {
      if (acc != nullptr) {
        const float4* p = reinterpret_cast<const float4*>(acc + tok * HD + c8);
        const float4 u = p[0], w = p[1];
        x[0] = u.x; x[1] = u.y; x[2] = u.z; x[3] = u.w; x[4] = w.x; x[5] = w.y; x[6] = w.z; x[7] = w.w;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] += ad[e];
    }
    st8(out + tok * HD + c8, x);
  }
}

// log2 of the valid tokens of every representative group (RM per block) and of every block; -inf when empty
__global__ void rep_counts_kernel(const int* __restrict__ blk_cnt, float* __restrict__ lc_mid,
                                  float* __restrict__ lc_tail, int NB, int RM) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= NB * RM) return;
  const int blk = e / RM, g = e - blk * RM, gs = BK / RM;
  const int cnt = blk_cnt[blk];
  const int n = min(max(cnt - g * gs, 0), gs);
  lc_mid[e] = n > 0 ? log2f((float)n) : -INFINITY;
  if (g == 0) lc_tail[blk] = cnt > 0 ? log2f((float)cnt) : -INFINITY;
}

}  // namespace

}  // namespace es

using namespace es;

static int check_tokens(int BH, int L, int D) {
  ES_REQUIRE(BH > 0 && BH <= 65535 && L > 0 && L % BK == 0, ES_ERR_INVALID,
             "VSA: tokens must be [BH <= 65535, L = NB * 64, D]");
  ES_REQUIRE(D == 64 || D == HD, ES_ERR_UNSUPPORTED, "VSA: head dim must be 64 or 128 (rows stored with 128 columns)");
  return ES_OK;
}

extern "C" int ES_VSA_API(vsa_pool)(const void* q, const void* k, const void* v, const int* blk_cnt, void* qr, void* kr, void* vr,
                        void* qc, void* kc, void* vc, int BH, int L, int D, int R, hipStream_t stream) {
  if (int st = check_tokens(BH, L, D)) return st;
  ES_REQUIRE(q && k && v && blk_cnt && qc && kc && vc, ES_ERR_INVALID, "VSA: null tensor pointer");
  ES_REQUIRE(R == 4 || R == 8 || R == 16 || R == 32, ES_ERR_INVALID, "VSA2: router pool size R must be 4, 8, 16 or 32");
  const int NB = L / BK, G = BK / R;
  PoolArgs a{{(const e16_t*)q, (const e16_t*)k, (const e16_t*)v},
             {(e16_t*)qr, (e16_t*)kr, (e16_t*)vr},
             {(e16_t*)qc, (e16_t*)kc, (e16_t*)vc},
             blk_cnt, NB, L, R, G, (NB * G + 63) / 64 * 64, (NB + 63) / 64 * 64};
  hipLaunchKernelGGL(pool_kernel, dim3((NB + POOL_BLOCKS - 1) / POOL_BLOCKS, BH), dim3(192), 0, stream, a);
  return check_launch("vsa_pool");
}

extern "C" int ES_VSA_API(vsa_fuse_fwd)(const void* of, const void* oc, const void* gate, void* o, const int* blk_cnt, int BH,
                            int L, int D, int NBc_pad, int gate_mode, int gate_act, hipStream_t stream) {
  if (int st = check_tokens(BH, L, D)) return st;
  ES_REQUIRE(of && oc && o && blk_cnt && (gate_mode == 0 || gate), ES_ERR_INVALID, "VSA: null tensor pointer");
  ES_REQUIRE(gate_mode >= 0 && gate_mode <= 2 && (gate_act == 0 || gate_act == 1), ES_ERR_INVALID,
             "VSA: gate_mode must be 0 (none), 1 (per token) or 2 (elementwise), gate_act 0 (tanh) or 1 (identity)");
  const int NB = L / BK;
  ES_REQUIRE(NBc_pad >= NB, ES_ERR_INVALID, "VSA: coarse output has fewer rows than blocks");
  FuseArgs a{nullptr, (const e16_t*)of, (const e16_t*)oc, (const e16_t*)gate, (e16_t*)o, nullptr, nullptr, nullptr,
             nullptr, nullptr, blk_cnt, NB, L, NBc_pad, gate_mode, gate_act};
  hipLaunchKernelGGL(fuse_fwd_kernel, dim3((NB + 3) / 4, BH), dim3(256), 0, stream, a);
  return check_launch("vsa_fuse_fwd");
}

extern "C" int ES_VSA_API(vsa_fuse_bwd)(const void* dout, const void* of, const void* oc, const void* gate, void* dout_f,
                            float* delta_f, void* dout_c, float* delta_c, void* dgate, const int* blk_cnt, int BH,
                            int L, int D, int NBc_pad, int gate_mode, int gate_act, hipStream_t stream) {
  if (int st = check_tokens(BH, L, D)) return st;
  ES_REQUIRE(dout && of && oc && delta_f && dout_c && delta_c && blk_cnt, ES_ERR_INVALID, "VSA: null tensor pointer");
  ES_REQUIRE(gate_mode >= 0 && gate_mode <= 2 && (gate_act == 0 || gate_act == 1), ES_ERR_INVALID,
             "VSA: gate_mode must be 0 (none), 1 (per token) or 2 (elementwise), gate_act 0 (tanh) or 1 (identity)");
  ES_REQUIRE(gate_mode == 0 || (gate && dgate), ES_ERR_INVALID, "VSA: a gated fusion needs gate and dgate");
  const int NB = L / BK;
  ES_REQUIRE(NBc_pad >= NB, ES_ERR_INVALID, "VSA: coarse output has fewer rows than blocks");
  FuseArgs a{(const e16_t*)dout, (const e16_t*)of, (const e16_t*)oc, (const e16_t*)gate, nullptr, (e16_t*)dout_f,
             (e16_t*)dout_c, (e16_t*)dgate, delta_f, delta_c, blk_cnt, NB, L, NBc_pad, gate_mode, gate_act};
  hipLaunchKernelGGL(fuse_bwd_kernel, dim3((NB + 3) / 4, BH), dim3(256), 0, stream, a);
  return check_launch("vsa_fuse_bwd");
}

extern "C" int ES_VSA_API(vsa_finalize)(const float* acc, const float* add, int add_nb, void* out, const int* blk_cnt, int BH,
                            int L, int D, hipStream_t stream) {
  if (int st = check_tokens(BH, L, D)) return st;
  ES_REQUIRE(out && blk_cnt, ES_ERR_INVALID, "VSA: null tensor pointer");
  const int NB = L / BK;
  ES_REQUIRE(add == nullptr || add_nb >= NB, ES_ERR_INVALID, "VSA: finalize add has fewer rows than blocks");
  hipLaunchKernelGGL(finalize_kernel, dim3((NB + 3) / 4, BH), dim3(256), 0, stream, acc, add, (e16_t*)out, blk_cnt,
                     NB, L, add_nb);
  return check_launch("vsa_finalize");
}

extern "C" int ES_VSA_API(vsa_rep_build)(const void* k, const void* v, const int* blk_cnt, void* k_mid, void* v_mid,
                             float* lc_mid, void* k_tail, void* v_tail, float* lc_tail, int BH, int L, int D, int RM,
                             hipStream_t stream) {
  if (int st = check_tokens(BH, L, D)) return st;
  ES_REQUIRE(k && v && blk_cnt && k_mid && v_mid && lc_mid && k_tail && v_tail && lc_tail, ES_ERR_INVALID,
             "VSA2-rep: null tensor pointer");
  ES_REQUIRE(RM == 1 || RM == 2 || RM == 4 || RM == 8 || RM == 16, ES_ERR_INVALID,
             "RepTiers.mid_reps must be one of (1, 2, 4, 8, 16)");
  const int NB = L / BK, R = BK / RM;
  // the mid table is the pooled groups of R = 64 / RM tokens, the tail table the block means
  PoolArgs a{{nullptr, (const e16_t*)k, (const e16_t*)v},
             {nullptr, (e16_t*)k_mid, (e16_t*)v_mid},
             {nullptr, (e16_t*)k_tail, (e16_t*)v_tail},
             blk_cnt, NB, L, R, RM, (NB * RM + 63) / 64 * 64, (NB + 63) / 64 * 64};
  hipLaunchKernelGGL(pool_kernel, dim3((NB + POOL_BLOCKS - 1) / POOL_BLOCKS, BH), dim3(192), 0, stream, a);
  hipLaunchKernelGGL(rep_counts_kernel, dim3((NB * RM + 255) / 256), dim3(256), 0, stream, blk_cnt, lc_mid, lc_tail,
                     NB, RM);
  return check_launch("vsa_rep_build");
}
