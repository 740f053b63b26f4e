// Tier construction for the VSA2 three-tier attention as the HunyuanVideo-shape benchmark states it (gfx950):
//
//   kmeans_tab_kernel  seeded Lloyd k-means of every block's valid keys into RM clusters: the tier-B table rows are
//                      the clusters' key / value means, with per-(b, h) log2 cluster sizes, cluster sizes and each
//                      token's cluster (the reference's tables are contiguous group means, vsa2_rep/reference.py:
//                      23-50; this construction has no reference counterpart). One 64-lane workgroup per (block,
//                      head). Float32 arithmetic in a fixed order with no fused multiply-add, so the tables equal
//                      the numpy restatement bit for bit:
//                        seeds     partial Fisher-Yates of the n valid tokens, swap partner i + h_i mod (n - i),
//                                  h_i = fmix32(seed * 0x9E3779B9 ^ fmix32(bh * 0x85EBCA6B ^ fmix32(blk *
//                                  0xC2B2AE35 ^ i))) (MurmurHash3's finaliser); clusters past n stay empty
//                        assign    lane = token, its key row in registers: squared distance to each centroid
//                                  summed over the 128 columns in order, nearest wins, ties to the smaller cluster
//                        update    lane = two columns: member keys summed in token order, one correctly
//                                  rounded division by the count; an emptied cluster keeps its centroid
//   row_tiers_kernel   per-query-block tier split: for each row of the fp32 router scores, the ka and kab best kv
//                      blocks (score desc, ties to the smaller index, -0 == +0) as ascending CSR lists with bases
//                      (bh * NB + i) * K and as selection bitmaps. One wave per row: 32-round bisection of the K-th
//                      largest order key with wave counts, then ballot prefix counts for the emission.
#include "../../include/vsa_hip.h"
#include "common.h"
#include "elem.h"

namespace es {

namespace {

constexpr int KM_MAX_RM = 16;

__device__ __forceinline__ unsigned fmix32(unsigned h) {
  h ^= h >> 16;
  h *= 0x85EBCA6Bu;
  h ^= h >> 13;
  h *= 0xC2B2AE35u;
  h ^= h >> 16;
  return h;
}

struct KmArgs {
  const e16_t *k, *v;
  const int* blk_cnt;
  e16_t *k_mid, *v_mid;
  float* lc_mid;        // [BH, NB * RM]
  int* counts;          // [BH, NB * RM]
  uint8_t* labels;      // [BH, L], 255 on padding
  int L, NB, mid_rows, iters;
  unsigned seed;
};

template <int RM>
__global__ __launch_bounds__(64) void kmeans_tab_kernel(KmArgs a) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) float cent_s[RM][HD];
  __shared__ __attribute__((aligned(16))) e16_t x_s[BK][HD];
  __shared__ int lab_s[BK];
  __shared__ int perm_s[BK];
  const int blk = blockIdx.x, bh = blockIdx.y, l = threadIdx.x;
  // a block holds 0..64 valid keys; clamping keeps an out-of-range count inside the 64-row LDS arrays and the block
  const int n = min(max(a.blk_cnt[blk], 0), BK);
  const size_t tok0 = (size_t)bh * a.L + (size_t)blk * BK;
  const e16_t* kb = a.k + tok0 * HD;
  const e16_t* vb = a.v + tok0 * HD;

  // the block's keys: row-major in LDS (the update pass reads columns) and this lane's row in registers
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int P = i * 64 + l, r = P >> 4, c = P & 15;
    uint4 u = {0u, 0u, 0u, 0u};
    if (r < n) u = *reinterpret_cast<const uint4*>(kb + (size_t)r * HD + c * 8);
    *reinterpret_cast<uint4*>(&x_s[r][c * 8]) = u;
  }
  float xr[HD];
#pragma unroll
  for (int c = 0; c < 16; ++c) {
    uint4 u = {0u, 0u, 0u, 0u};
    if (l < n) u = *reinterpret_cast<const uint4*>(kb + (size_t)l * HD + c * 8);
    const unsigned w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      xr[c * 8 + 2 * e] = e2f((e16_t)(w[e] & 0xffffu));
      xr[c * 8 + 2 * e + 1] = e2f((e16_t)(w[e] >> 16));
    }
  }
  perm_s[l] = l;
  __syncthreads();
  const int nlive = min(RM, n);
  if (l == 0) {
    for (int i = 0; i < nlive; ++i) {
      const unsigned h = fmix32((a.seed * 0x9E3779B9u) ^ fmix32(((unsigned)bh * 0x85EBCA6Bu) ^
                                                                 fmix32(((unsigned)blk * 0xC2B2AE35u) ^ (unsigned)i)));
      const int j = i + (int)(h % (unsigned)(n - i));
      const int t = perm_s[i];
      perm_s[i] = perm_s[j];
      perm_s[j] = t;
    }
  }
  __syncthreads();
  for (int c = 0; c < nlive; ++c) {
    const int s = perm_s[c];
    cent_s[c][2 * l] = e2f(x_s[s][2 * l]);
    cent_s[c][2 * l + 1] = e2f(x_s[s][2 * l + 1]);
  }
  __syncthreads();

  // A round whose assignment leaves every label as it was would rebuild the same centroids from the same members in
  // the same order, and so would every round after it: the loop stops there with the tables, counts and labels
  // that all a.iters rounds give.
  int cnt[RM];
  for (int it = 0; it < a.iters; ++it) {
    // assignment: lane = token
    int best = 0;
    if (l < n) {
      float bd = 0.0f;
#pragma unroll
      for (int c = 0; c < RM; ++c) {
        if (c >= nlive) break;
        float acc = 0.0f;
#pragma unroll
        for (int d = 0; d < HD; d += 4) {
          const f32x4 cv = *reinterpret_cast<const f32x4*>(&cent_s[c][d]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float diff = xr[d + e] - cv[e];
            const float sq = diff * diff;
            acc = acc + sq;
          }
        }
        if (c == 0 || acc < bd) {
          bd = acc;
          best = c;
        }
      }
    }
    if (it > 0 && __builtin_amdgcn_ballot_w64(l < n && best != lab_s[l]) == 0ull) break;  // (one wave: uniform)
    if (l < n) lab_s[l] = best;
    __syncthreads();
    // update: lane = columns 2l, 2l + 1
    float s0[RM], s1[RM];
#pragma unroll
    for (int c = 0; c < RM; ++c) {
      s0[c] = 0.0f;
      s1[c] = 0.0f;
      cnt[c] = 0;
    }
#pragma unroll 8
    for (int t = 0; t < n; ++t) {
      const int lb = lab_s[t];
      const float x0 = e2f(x_s[t][2 * l]), x1 = e2f(x_s[t][2 * l + 1]);
#pragma unroll
      for (int c = 0; c < RM; ++c) {
        if (lb == c) {
          s0[c] = s0[c] + x0;
          s1[c] = s1[c] + x1;
          cnt[c] += 1;
        }
      }
    }
#pragma unroll
    for (int c = 0; c < RM; ++c) {
      if (cnt[c] > 0) {
        cent_s[c][2 * l] = __fdiv_rn(s0[c], (float)cnt[c]);
        cent_s[c][2 * l + 1] = __fdiv_rn(s1[c], (float)cnt[c]);
      }
    }
    __syncthreads();
  }

  // value means of the final clusters (lane = two columns, rows read straight from global memory)
  float v0[RM], v1[RM];
#pragma unroll
  for (int c = 0; c < RM; ++c) {
    v0[c] = 0.0f;
    v1[c] = 0.0f;
  }
#pragma unroll 8
  for (int t = 0; t < n; ++t) {  // (eight rows' loads in flight together; the sums take the rows in order)
    const int lb = lab_s[t];
    const unsigned u = *reinterpret_cast<const unsigned*>(vb + (size_t)t * HD + 2 * l);
    const float y0 = e2f((e16_t)(u & 0xffffu)), y1 = e2f((e16_t)(u >> 16));
#pragma unroll
    for (int c = 0; c < RM; ++c) {
      if (lb == c) {
        v0[c] = v0[c] + y0;
        v1[c] = v1[c] + y1;
      }
    }
  }
  const size_t row0 = (size_t)bh * a.mid_rows + (size_t)blk * RM;
#pragma unroll
  for (int c = 0; c < RM; ++c) {
    unsigned ku = 0u, vu = 0u;
    if (cnt[c] > 0) {
      const float fc = (float)cnt[c];
      ku = (unsigned)f2e(cent_s[c][2 * l]) | ((unsigned)f2e(cent_s[c][2 * l + 1]) << 16);
      vu = (unsigned)f2e(__fdiv_rn(v0[c], fc)) | ((unsigned)f2e(__fdiv_rn(v1[c], fc)) << 16);
    }
    *reinterpret_cast<unsigned*>(a.k_mid + (row0 + c) * HD + 2 * l) = ku;
    *reinterpret_cast<unsigned*>(a.v_mid + (row0 + c) * HD + 2 * l) = vu;
  }
  const size_t crow = (size_t)bh * a.NB * RM + (size_t)blk * RM;
#pragma unroll
  for (int c = 0; c < RM; ++c) {
    if (l == c) {
      a.counts[crow + c] = cnt[c];
      a.lc_mid[crow + c] = cnt[c] > 0 ? log2f((float)cnt[c]) : -INFINITY;
    }
  }
  a.labels[tok0 + l] = l < n ? (uint8_t)lab_s[l] : (uint8_t)255;
}

}  // namespace

}  // namespace es

using namespace es;

extern "C" int ES_VSA_API(vsa_rep_build_kmeans)(const void* k, const void* v, const int* blk_cnt, void* k_mid,
                                                void* v_mid, float* lc_mid, int* counts, uint8_t* labels, int BH,
                                                int L, int D, int RM, int iters, unsigned seed, hipStream_t stream) {
  ES_REQUIRE(k && v && blk_cnt && k_mid && v_mid && lc_mid && counts && labels, ES_ERR_INVALID,
             "VSA2-rep: null tensor pointer");
  ES_REQUIRE(BH > 0 && BH <= 65535 && L > 0 && L % BK == 0, ES_ERR_INVALID,
             "VSA2-rep: tokens must be [BH, L = NB * 64, D]");
  ES_REQUIRE(D == 64 || D == HD, ES_ERR_UNSUPPORTED, "VSA2-rep: head dim must be 64 or 128 (rows stored with 128 columns)");
  ES_REQUIRE(RM == 1 || RM == 2 || RM == 4 || RM == 8 || RM == KM_MAX_RM, ES_ERR_INVALID,
             "RepTiers.mid_reps must be one of (1, 2, 4, 8, 16)");
  ES_REQUIRE(iters >= 1 && iters <= 1000, ES_ERR_INVALID, "VSA2-rep: k-means needs 1..1000 iterations");
  const int NB = L / BK;
  KmArgs a = {(const e16_t*)k, (const e16_t*)v, blk_cnt, (e16_t*)k_mid, (e16_t*)v_mid, lc_mid, counts, labels,
              L, NB, (NB * RM + 63) / 64 * 64, iters, seed};
  const dim3 grid(NB, BH);
  switch (RM) {
    case 1: hipLaunchKernelGGL(kmeans_tab_kernel<1>, grid, dim3(64), 0, stream, a); break;
    case 2: hipLaunchKernelGGL(kmeans_tab_kernel<2>, grid, dim3(64), 0, stream, a); break;
    case 4: hipLaunchKernelGGL(kmeans_tab_kernel<4>, grid, dim3(64), 0, stream, a); break;
    case 8: hipLaunchKernelGGL(kmeans_tab_kernel<8>, grid, dim3(64), 0, stream, a); break;
    default: hipLaunchKernelGGL(kmeans_tab_kernel<16>, grid, dim3(64), 0, stream, a); break;
  }
  return check_launch("vsa_rep_build_kmeans");
}

#ifndef ES_ELEM_F16  // no token tensors: built once

namespace es {
namespace {

// keys of one row in registers, CH per lane (64 * CH >= NB): CH = 32, 64 or 128, so NB <= 8192
constexpr int TIER_MAX_NB = 8192;

// order-preserving key of a float: larger key = larger value, -0 and +0 share a key
__device__ __forceinline__ unsigned okey(float f) {
  unsigned u = __float_as_uint(f);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

struct TierArgs {
  const float* scores;  // [bh_count, NB, NB]
  int NB, W, bh0, rows;
  int ka, kab;
  int *a_ptr, *a_idx, *ab_ptr, *ab_idx;
  unsigned *bits_a, *bits_ab;
};

// the K-th largest key of the row (K >= 1): the largest T with #(key >= T) >= K, built bit by bit from the top
template <int TIER_CH>
__device__ __forceinline__ unsigned kth_key(const unsigned (&key)[TIER_CH], int nch, int NB, int K) {
  const int l = threadIdx.x & 63;
  unsigned T = 0u;
  for (int b = 31; b >= 0; --b) {
    const unsigned cand = T | (1u << b);
    int c = 0;
#pragma unroll
    for (int ch = 0; ch < TIER_CH; ++ch) c += (ch < nch && ch * 64 + l < NB && key[ch] >= cand) ? 1 : 0;
    c = wave_sum_i(c);
    if (c >= K) T = cand;
  }
  return T;
}

template <int TIER_CH>
__device__ __forceinline__ void emit(const unsigned (&key)[TIER_CH], int nch, int NB, int W, int K, int* ptr,
                                     int* idx, unsigned* bits, size_t bh, int i) {
  const int l = threadIdx.x & 63;
  const size_t base = (bh * NB + i) * (size_t)K;
  if (l == 0) {
    ptr[bh * (NB + 1) + i] = (int)base;
    if (i == NB - 1) ptr[bh * (NB + 1) + NB] = (int)(base + K);
  }
  unsigned* brow = bits + (bh * NB + i) * W;
  if (K <= 0) {
    for (int w = l; w < W; w += 64) brow[w] = 0u;
    return;
  }
  const unsigned T = kth_key(key, nch, NB, K);
  int gt = 0;
#pragma unroll
  for (int ch = 0; ch < TIER_CH; ++ch) gt += (ch < nch && ch * 64 + l < NB && key[ch] > T) ? 1 : 0;
  const int need = K - wave_sum_i(gt);  // T-equal entries to take, smallest indices first
  int eq_before = 0, out = 0;
  const unsigned long long below = (1ull << l) - 1ull;
#pragma unroll
  for (int ch = 0; ch < TIER_CH; ++ch) {
    if (ch >= nch) continue;  // (not a break: the loop must unroll fully so that key[] stays in registers)
    const int j = ch * 64 + l;
    const bool in = j < NB;
    const bool eq = in && key[ch] == T;
    const unsigned long long me = __builtin_amdgcn_ballot_w64(eq);
    const bool sel = in && (key[ch] > T || (eq && eq_before + __popcll(me & below) < need));
    const unsigned long long ms = __builtin_amdgcn_ballot_w64(sel);
    if (sel) idx[base + out + __popcll(ms & below)] = j;
    out += __popcll(ms);
    eq_before += __popcll(me);
    if (l == 0 && 2 * ch < W) brow[2 * ch] = (unsigned)ms;
    if (l == 0 && 2 * ch + 1 < W) brow[2 * ch + 1] = (unsigned)(ms >> 32);
  }
}

template <int TIER_CH>
__global__ __launch_bounds__(256) void row_tiers_kernel(TierArgs a) {
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63;
  if (r >= a.rows) return;
  const int bhl = r / a.NB, i = r - bhl * a.NB;
  const size_t bh = (size_t)a.bh0 + bhl;
  const float* row = a.scores + ((size_t)bhl * a.NB + i) * a.NB;
  const int nch = (a.NB + 63) / 64;
  unsigned key[TIER_CH];
#pragma unroll
  for (int ch = 0; ch < TIER_CH; ++ch) key[ch] = (ch < nch && ch * 64 + l < a.NB) ? okey(row[ch * 64 + l]) : 0u;
  emit(key, nch, a.NB, a.W, a.ka, a.a_ptr, a.a_idx, a.bits_a, bh, i);
  emit(key, nch, a.NB, a.W, a.kab, a.ab_ptr, a.ab_idx, a.bits_ab, bh, i);
}

}  // namespace
}  // namespace es

extern "C" int vsa_row_tiers(const float* scores, int NB, int bh0, int bh_count, int ka, int kab, int* a_ptr,
                             int* a_idx, int* ab_ptr, int* ab_idx, unsigned* bits_a, unsigned* bits_ab,
                             hipStream_t stream) {
  ES_REQUIRE(scores && a_ptr && ab_ptr && bits_a && bits_ab, ES_ERR_INVALID, "VSA2-rep: null tensor pointer");
  ES_REQUIRE(NB >= 1 && NB <= TIER_MAX_NB, ES_ERR_UNSUPPORTED, "VSA2-rep: per-row tiers support 1 <= NB <= 8192");
  ES_REQUIRE(bh0 >= 0 && bh_count >= 1 && (long long)bh_count * NB < (1LL << 31), ES_ERR_INVALID,
             "VSA2-rep: bad (b,h) range");
  ES_REQUIRE(0 <= ka && ka <= kab && kab <= NB, ES_ERR_INVALID, "VSA2-rep: need 0 <= ka <= kab <= NB");
  ES_REQUIRE((ka == 0 || a_idx) && (kab == 0 || ab_idx), ES_ERR_INVALID, "VSA2-rep: null list pointer");
  ES_REQUIRE((long long)(bh0 + bh_count) * NB * kab < (1LL << 31), ES_ERR_UNSUPPORTED,
             "VSA2-rep: selected blocks exceed int32 CSR range");
  TierArgs a = {scores, NB, (NB + 31) / 32, bh0, bh_count * NB, ka, kab, a_ptr, a_idx, ab_ptr, ab_idx, bits_a,
                bits_ab};
  const dim3 grid((unsigned)((a.rows + 3) / 4));
  if (NB <= 2048)
    hipLaunchKernelGGL(row_tiers_kernel<32>, grid, dim3(256), 0, stream, a);
  else if (NB <= 4096)
    hipLaunchKernelGGL(row_tiers_kernel<64>, grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(row_tiers_kernel<128>, grid, dim3(256), 0, stream, a);
  return check_launch("vsa_row_tiers");
}

#endif
