// VSA2 split-KV scheduling: the device-side task plan over a CSR list and the two merges (gfx950).
//
// Plan (reference csrc/vsa/split.cu:1-19, vsa2_kernels.h:48-74; contract of the pure-Python planner in
// tests/test_vsa2_split.py:60-87). For the NR = BH * NB rows of a CSR list (q2k for the forward and the Q-owner
// backward, k2q for the KV-owner backward):
//   thr    = max(chunk + 1, min_len, ceil(tail_frac * W / resident)) and, with rel_mean > 0, per (b, h)
//            max(thr, ceil(rel_mean * nnz_bh / NB)); W = all edges of the list
//   cnt_r  = n_r >= thr ? ceil(n_r / chunk) : 0; E = #rows with n_r >= thr
//   split  = E <= budget && cnt_r > 0 && (inclusive scan of cnt up to r) <= max_slots
//   tasks  : split rows first, chunk j of row r = [beg + j n / c, beg + (j + 1) n / c) with slot = (exclusive scan
//            of cnt) + j; then one direct task (slot -1) per other row, in row order
//   merges : one {r, first slot, c, 0} per split row; info = {tasks, split rows, split slots, NR, E, E <= budget,
//            thr without the per-(b, h) term, W}
// One workgroup of 1024 threads plans the whole list: each thread owns a contiguous run of rows, and three
// workgroup scans give every thread its slot, task and merge bases. Nothing is read back to the host.
//
// Merges (one workgroup per split row, in chunk order: deterministic):
//   forward : o = sum_i 2^(lse_i - M) o_i / sum_i 2^(lse_i - M), lse = (M + log2 sum) ln 2 (reference
//             split.cu:117-155); padded query rows get o = 0, lse = -inf when mask_rows
//   sum     : out = valid ? sum_i part_i + add[blk] / cnt : 0 (reference split.cu:157-200)
#include "../../include/vsa_hip.h"
#include "common.h"
#include "elem.h"

#include <cmath>

namespace es {

namespace {

constexpr int PLAN_THREADS = 1024;

struct PlanArgs {
  const int* ptr;
  int BH, NB, chunk, max_slots, min_len, resident, budget;
  double rel_mean, tail_frac;
  int4* tasks;
  int4* merges;
  int* info;
};

// exclusive scan of x over the 1024 threads (16 waves); returns the prefix, total in *tot
__device__ long long plan_scan(long long x, long long* red, long long* tot) {
  const int l = threadIdx.x & 63, wv = threadIdx.x >> 6;
  long long inc = x;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const long long y = __shfl_up(inc, d, 64);
    if (l >= d) inc += y;
  }
  __syncthreads();
  if (l == 63) red[wv] = inc;
  __syncthreads();
  long long before = 0, all = 0;
  for (int i = 0; i < PLAN_THREADS / 64; ++i) {
    before += i < wv ? red[i] : 0;
    all += red[i];
  }
  *tot = all;
  return before + inc - x;
}

__global__ __launch_bounds__(PLAN_THREADS) void plan_kernel(PlanArgs a) {
  __shared__ long long red[PLAN_THREADS / 64];
  const int NR = a.BH * a.NB;
  const int per = (NR + PLAN_THREADS - 1) / PLAN_THREADS;
  const int r0 = min(NR, (int)threadIdx.x * per), r1 = min(NR, r0 + per);
  const long long W = (long long)a.ptr[(size_t)a.BH * (a.NB + 1) - 1] - a.ptr[0];
  int gthr = max(a.chunk + 1, a.min_len);
  if (a.tail_frac > 0.0) gthr = max(gthr, (int)ceil(a.tail_frac * (double)W / (double)a.resident));
  auto row = [&](int r, int& beg, int& n, int& c) {
    const int bh = r / a.NB, i = r - bh * a.NB;
    const int* hp = a.ptr + (size_t)bh * (a.NB + 1);
    beg = hp[i];
    n = hp[i + 1] - beg;
    int thr = gthr;
    if (a.rel_mean > 0.0) thr = max(thr, (int)ceil(a.rel_mean * (double)(hp[a.NB] - hp[0]) / (double)a.NB));
    c = n >= thr ? (n + a.chunk - 1) / a.chunk : 0;
  };
  // 1: chunk counts and eligible rows
  long long cnt_mine = 0, elig_mine = 0;
  for (int r = r0; r < r1; ++r) {
    int beg, n, c;
    row(r, beg, n, c);
    cnt_mine += c;
    elig_mine += c > 0;
  }
  long long cnt_tot, E;
  const long long cnt_before = plan_scan(cnt_mine, red, &cnt_tot);
  plan_scan(elig_mine, red, &E);
  const bool ok = E <= (long long)a.budget;
  // 2: split rows, split chunks, direct rows of this thread
  long long split_mine = 0, chunks_mine = 0, direct_mine = 0;
  {
    long long incl = cnt_before;
    for (int r = r0; r < r1; ++r) {
      int beg, n, c;
      row(r, beg, n, c);
      incl += c;
      const bool split = ok && c > 0 && incl <= a.max_slots;
      split_mine += split;
      chunks_mine += split ? c : 0;
      direct_mine += split ? 0 : 1;
    }
  }
  long long nsplit, t_split, ndirect;
  const long long split_before = plan_scan(split_mine, red, &nsplit);
  plan_scan(chunks_mine, red, &t_split);
  const long long direct_before = plan_scan(direct_mine, red, &ndirect);
  // 3: write
  long long incl = cnt_before, ms = split_before, dt = direct_before;
  for (int r = r0; r < r1; ++r) {
    int beg, n, c;
    row(r, beg, n, c);
    const long long slot0 = incl;
    incl += c;
    if (ok && c > 0 && incl <= a.max_slots) {
      for (int j = 0; j < c; ++j)
        a.tasks[slot0 + j] = make_int4(r, beg + (int)((long long)j * n / c), beg + (int)((long long)(j + 1) * n / c),
                                       (int)(slot0 + j));
      a.merges[ms++] = make_int4(r, (int)slot0, c, 0);
    } else {
      a.tasks[t_split + dt++] = make_int4(r, beg, beg + n, -1);
    }
  }
  if (threadIdx.x == 0) {
    a.info[0] = (int)(t_split + ndirect);
    a.info[1] = (int)nsplit;
    a.info[2] = (int)t_split;
    a.info[3] = NR;
    a.info[4] = (int)E;
    a.info[5] = ok ? 1 : 0;
    a.info[6] = gthr;
    a.info[7] = (int)W;
  }
}

// thread -> (row = tid / 4, 32 columns (tid % 4) * 32 ..)
__global__ __launch_bounds__(256) void merge_fwd_kernel(const float* __restrict__ part_o,
                                                        const float* __restrict__ part_lse,
                                                        const int4* __restrict__ merges, const int* __restrict__ info,
                                                        const int* __restrict__ blk_cnt, e16_t* __restrict__ o,
                                                        float* __restrict__ lse, int L, int NB, int mask_rows) {
  if ((int)blockIdx.x >= info[1]) return;
  const int4 mg = merges[blockIdx.x];
  const int bh = mg.x / NB, qb = mg.x - bh * NB, slot0 = mg.y, c = mg.z;
  const int row = threadIdx.x >> 2, c0 = (threadIdx.x & 3) * 32;
  const size_t tok = (size_t)bh * L + (size_t)qb * BK + row;
  float acc[32];
#pragma unroll
  for (int e = 0; e < 32; ++e) acc[e] = 0.0f;
  float out_lse = -INFINITY;
  if (row < blk_cnt[qb] || !mask_rows) {
    float mx = -INFINITY;
    for (int j = 0; j < c; ++j) mx = fmaxf(mx, part_lse[(size_t)(slot0 + j) * BK + row]);
    if (mx != -INFINITY) {
      float sum = 0.0f;
      for (int j = 0; j < c; ++j) {
        const float w = exp2f(part_lse[(size_t)(slot0 + j) * BK + row] - mx);
        const f32x4* src = reinterpret_cast<const f32x4*>(part_o + ((size_t)(slot0 + j) * BK + row) * HD + c0);
        sum += w;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const f32x4 x = src[q];
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[4 * q + e] += w * x[e];
        }
      }
      const float inv = 1.0f / sum;
#pragma unroll
      for (int e = 0; e < 32; ++e) acc[e] *= inv;
      out_lse = (mx + log2f(sum)) * 0.6931471805599453f;
    }
  }
  uint4* dst = reinterpret_cast<uint4*>(o + tok * HD + c0);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    uint4 u;
    u.x = (unsigned)f2e(acc[8 * q + 0]) | ((unsigned)f2e(acc[8 * q + 1]) << 16);
    u.y = (unsigned)f2e(acc[8 * q + 2]) | ((unsigned)f2e(acc[8 * q + 3]) << 16);
    u.z = (unsigned)f2e(acc[8 * q + 4]) | ((unsigned)f2e(acc[8 * q + 5]) << 16);
    u.w = (unsigned)f2e(acc[8 * q + 6]) | ((unsigned)f2e(acc[8 * q + 7]) << 16);
    dst[q] = u;
  }
  if ((threadIdx.x & 3) == 0) lse[tok] = out_lse;
}

__global__ __launch_bounds__(256) void merge_sum_kernel(const float* __restrict__ part, const int4* __restrict__ merges,
                                                        const int* __restrict__ info, const float* __restrict__ add,
                                                        int add_nb, const int* __restrict__ blk_cnt,
                                                        e16_t* __restrict__ out, float* __restrict__ out_f32, int L,
                                                        int NB) {
  if ((int)blockIdx.x >= info[1]) return;
  const int4 mg = merges[blockIdx.x];
  const int bh = mg.x / NB, blk = mg.x - bh * NB, slot0 = mg.y, c = mg.z;
  const int row = threadIdx.x >> 2, c0 = (threadIdx.x & 3) * 32;
  const size_t tok = (size_t)bh * L + (size_t)blk * BK + row;
  const int cnt = blk_cnt[blk];
  float acc[32];
#pragma unroll
  for (int e = 0; e < 32; ++e) acc[e] = 0.0f;
  if (row < cnt) {
    for (int j = 0; j < c; ++j) {
      const f32x4* src = reinterpret_cast<const f32x4*>(part + ((size_t)(slot0 + j) * BK + row) * HD + c0);
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const f32x4 x = src[q];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[4 * q + e] += x[e];
      }
    }
    if (add != nullptr) {
      const float inv = 1.0f / (float)cnt;
      const f32x4* ad = reinterpret_cast<const f32x4*>(add + ((size_t)bh * add_nb + blk) * HD + c0);
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const f32x4 x = ad[q];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[4 * q + e] += x[e] * inv;
      }
    }
  }
  if (out_f32 != nullptr) {
    f32x4* dst = reinterpret_cast<f32x4*>(out_f32 + tok * HD + c0);
#pragma unroll
    for (int q = 0; q < 8; ++q) dst[q] = f32x4{acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
  } else {
    uint4* dst = reinterpret_cast<uint4*>(out + tok * HD + c0);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint4 u;
      u.x = (unsigned)f2e(acc[8 * q + 0]) | ((unsigned)f2e(acc[8 * q + 1]) << 16);
      u.y = (unsigned)f2e(acc[8 * q + 2]) | ((unsigned)f2e(acc[8 * q + 3]) << 16);
      u.z = (unsigned)f2e(acc[8 * q + 4]) | ((unsigned)f2e(acc[8 * q + 5]) << 16);
      u.w = (unsigned)f2e(acc[8 * q + 6]) | ((unsigned)f2e(acc[8 * q + 7]) << 16);
      dst[q] = u;
    }
  }
}

}  // namespace

}  // namespace es

using namespace es;

#ifndef ES_ELEM_F16  // no token tensors: built once
extern "C" int vsa_split_plan(const int* ptr, int BH, int NB, int chunk, int max_slots, int min_len, double rel_mean,
                              double tail_frac, int resident, int budget, int* tasks, int* merges, int* info,
                              hipStream_t stream) {
  ES_REQUIRE(ptr && tasks && merges && info, ES_ERR_INVALID, "VSA2: null tensor pointer");
  ES_REQUIRE(BH >= 1 && NB >= 1, ES_ERR_INVALID, "ptr must be [B, H, NB+1]");
  ES_REQUIRE(chunk >= 1 && chunk <= (1 << 30), ES_ERR_INVALID, "split chunk must be in [1, 2^30]");
  ES_REQUIRE(max_slots >= 0 && max_slots < (1 << 30), ES_ERR_INVALID, "bad max_slots");
  ES_REQUIRE(rel_mean >= 0.0 && tail_frac >= 0.0 && resident >= 1, ES_ERR_INVALID, "bad split policy");
  PlanArgs a = {};
  a.ptr = ptr;
  a.BH = BH;
  a.NB = NB;
  a.chunk = chunk;
  a.max_slots = max_slots;
  a.min_len = min_len;
  a.resident = resident;
  a.budget = budget < 0 ? 0x7fffffff : budget;
  a.rel_mean = rel_mean;
  a.tail_frac = tail_frac;
  a.tasks = (int4*)tasks;
  a.merges = (int4*)merges;
  a.info = info;
  hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(PLAN_THREADS), 0, stream, a);
  return check_launch("vsa_split_plan");
}
#endif

extern "C" int ES_VSA_API(vsa_split_merge_fwd)(const float* part_o, const float* part_lse, const int* merges, const int* info,
                                   int max_merges, const int* blk_cnt, void* o, float* lse, int BH, int L, int D,
                                   int mask_rows, hipStream_t stream) {
  ES_REQUIRE(D == 64 || D == HD, ES_ERR_UNSUPPORTED, "VSA: head dim must be 64 or 128 (rows stored with 128 columns)");
  ES_REQUIRE(BH >= 1 && L > 0 && L % BK == 0, ES_ERR_INVALID, "o must be [B,H,L,D]");
  if (max_merges <= 0) return ES_OK;
  ES_REQUIRE(part_o && part_lse && merges && info && blk_cnt && o && lse, ES_ERR_INVALID, "VSA2: null tensor pointer");
  hipLaunchKernelGGL(merge_fwd_kernel, dim3(max_merges), dim3(256), 0, stream, part_o, part_lse, (const int4*)merges,
                     info, blk_cnt, (e16_t*)o, lse, L, L / BK, mask_rows);
  return check_launch("vsa_split_merge_fwd");
}

extern "C" int ES_VSA_API(vsa_split_merge_sum)(const float* part, const int* merges, const int* info, int max_merges,
                                   const float* add, int add_nb, const int* blk_cnt, void* out, float* out_f32, int BH,
                                   int L, int D, hipStream_t stream) {
  ES_REQUIRE(D == 64 || D == HD, ES_ERR_UNSUPPORTED, "VSA: head dim must be 64 or 128 (rows stored with 128 columns)");
  ES_REQUIRE(BH >= 1 && L > 0 && L % BK == 0, ES_ERR_INVALID, "out must be [B,H,L,D]");
  if (max_merges <= 0) return ES_OK;
  ES_REQUIRE(part && merges && info && blk_cnt && (out || out_f32), ES_ERR_INVALID, "VSA2: null tensor pointer");
  hipLaunchKernelGGL(merge_sum_kernel, dim3(max_merges), dim3(256), 0, stream, part, (const int4*)merges, info, add,
                     add_nb, blk_cnt, (e16_t*)out, out_f32, L, L / BK);
  return check_launch("vsa_split_merge_sum");
}
