// VSA2 three-tier representative attention (gfx950): tier A = the selected 64-token blocks, tier B = RM
// representatives (contiguous 64 / RM-token group means) of the next-ranked blocks, tier C = the block mean of every
// other block. A representative of c tokens is one softmax column with + log2(c) on its logit (reference
// experiments/vsa2_representative/csrc/rep/rep_kernels.h:1-40, vsa2_rep/reference.py:53-96).
//
// Tables (built by vsa_rep_build): k_mid / v_mid [BH, ceil64(NB * RM), D] (row blk * RM + g), k_tail / v_tail
// [BH, ceil64(NB), D] (row blk), lc_mid [NB * RM] and lc_tail [NB] log2 counts (-inf: empty group), shared by
// every head; lc_mid may instead be per head ([BH, NB * RM], lc_mid_stride = NB * RM), as the seeded k-means tables
// of vsa_rep_build_kmeans need. Tier membership of pair (query block i, kv block j) comes from the bitmaps bits_a / bits_ab
// [BH, NB, W], W = ceil(NB / 32): A = a, B = ab & ~a, C = ~ab.
//
//   rep_fwd_kernel      one workgroup per (query block, head), the VSA fine forward's layout (2 row groups x 2 key
//                       halves, chunks staged in LDS) over one column stream: tier-A blocks of the CSR list, then
//                       64-row chunks of tier-B representatives, then 64-row chunks of tier-C means; the B and C
//                       block lists are compacted from the bitmaps into LDS at the start (wave ballots).
//   rep_bwd_q_kernel    dQ over the same stream (S^T, dP^T, dQ^T += K^T dS^T), deterministic.
//   rep_bwd_tab_kernel  dK / dV of the representative tables, KV-owner: a workgroup owns 64 table rows and walks
//                       every query block that has one of its pairs in the tier (pairs outside get P = 0), so the
//                       shared rows need no atomics; a dV pass and a dK pass (two waves per SIMD, 119.8 -> 118.0 ms
//                       per C4 step at B = 1). Tier-A token dK / dV come from the fine KV-owner kernel.
//   rep_unpool_kernel   dX = acc + dk_mid[group] / c_group + dk_tail[blk] / c_blk on valid rows (the adjoint of the
//                       means), tier_b_lists_kernel (A|B lists minus tier A), row_dot_kernel (delta).
#include "../../include/vsa_hip.h"
#include "common.h"
#include "elem.h"
#include "queues.h"

namespace es {

namespace {

constexpr float LN2_F = 0.6931471805599453f;
constexpr float SLACK = 8.0f;
constexpr int REP_LIST = 4096;    // one LDS list of a query block's tier-B and tier-C blocks (disjoint: <= NB)
constexpr int REP_MAX_NB = 8192;  // past REP_LIST blocks the forward / dQ take a list of this size (82 KB of LDS in all:
                                  // one workgroup per CU instead of two)
enum { PH_A = 1, PH_B = 2, PH_C = 4 };

struct RepArgs {
  const e16_t *q, *k, *v, *dout;
  const e16_t *k_mid, *v_mid, *k_tail, *v_tail;
  const float *lc_mid, *lc_tail;
  int lc_mid_stride;  // per-head stride of lc_mid (0: one table for every head)
  const float *lse, *delta;
  e16_t* out;
  float* lse_out;
  const int *row_ptr, *col_idx, *blk_cnt;
  const unsigned *bits_a, *bits_ab;
  const float* add_dq;
  int add_nb;
  float* dq_acc;
  int* queues;  // the eight row-block queue counters of this launch (queues.h)
  int L, NB, RM, W, BH, per_xcd, fixed, phases, mid_rows, tail_rows;
  float scale_log2, scale;
};

// The column stream of one (query block, head): chunk kinds A (one 64-token block each), B (64 representative
// rows), C (64 block means). Built once per workgroup; every lane can then name the 4 rows it stages per chunk.
struct Stream {
  int nA, nBrows, nC;  // tier-A blocks, tier-B representative rows, tier-C blocks
  int cA, cB, cC;      // chunks of each kind
  int beg;             // tier-A list start
};

__device__ __forceinline__ unsigned row_word(const unsigned* bits, size_t row, int W, int w) {
  return bits[row * W + w];
}

// compact tier B (ab & ~a) and tier C (~ab) blocks of bitmap row `row` into LDS lists (wave 0)
// tier-B blocks ascending into lists[0..), tier-C blocks ascending into lists[N - 1], [N - 2], ...
// (the two never meet: a row holds at most NB <= N of them)
template <int N>
__device__ void build_lists(const RepArgs& a, size_t row, unsigned short* lists, int* counts) {
  const int l = threadIdx.x & 63;
  int nb_run = 0, nc_run = 0;
  for (int w0 = 0; w0 < a.W; w0 += 64) {
    const int w = w0 + l;
    unsigned bm = 0, cm = 0;
    if (w < a.W) {
      const unsigned av = row_word(a.bits_a, row, a.W, w), abv = row_word(a.bits_ab, row, a.W, w);
      const int lo = w * 32;
      const unsigned valid = a.NB - lo >= 32 ? 0xffffffffu : ((1u << (a.NB - lo)) - 1u);
      bm = (a.phases & PH_B) ? (abv & ~av & valid) : 0u;
      cm = (a.phases & PH_C) ? (~abv & valid) : 0u;
    }
    int pb = __popc(bm), pc = __popc(cm), ib = pb, ic = pc;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int yb = __shfl_up(ib, d, 64), yc = __shfl_up(ic, d, 64);
      if (l >= d) {
        ib += yb;
        ic += yc;
      }
    }
    int ob = nb_run + ib - pb, oc = nc_run + ic - pc;
    while (bm) {
      const int b = __ffs(bm) - 1;
      lists[ob++] = (unsigned short)(w * 32 + b);
      bm &= bm - 1;
    }
    while (cm) {
      const int b = __ffs(cm) - 1;
      lists[N - 1 - oc++] = (unsigned short)(w * 32 + b);
      cm &= cm - 1;
    }
    nb_run += __shfl(ib, 63, 64);
    nc_run += __shfl(ic, 63, 64);
  }
  if (l == 0) {
    counts[0] = nb_run;
    counts[1] = nc_run;
  }
}

// ------------------------------------------------------------------------------------------------ forward / dQ
template <bool BWD, int LISTN>
__global__ __launch_bounds__(256, 2) void rep_q_kernel(RepArgs a) {
  __shared__ __attribute__((aligned(16))) char kv_s[2][2][BK * 256];
  __shared__ __attribute__((aligned(16))) float bias_s[2][BK];
  __shared__ unsigned short lists[LISTN];
  __shared__ int counts[2];

  int bh, qb;  // XCD-aware, run-time balanced order of (query block, head) (queues.h)
  if (!balanced_item(a.queues, a.fixed, a.per_xcd, a.BH, a.NB, bh, qb)) return;
  const int tid = threadIdx.x, l = tid & 63, hi = l >> 5, lq = l & 31;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rg = wv & 1, kh = wv >> 1;
  const int qrow = 32 * rg + lq;
  const int qcnt = sload(a.blk_cnt + qb);
  const bool qvalid = qrow < qcnt;
  const size_t head = (size_t)bh * a.L;
  const size_t tok = head + (size_t)qb * BK + qrow;
  const size_t brow = (size_t)bh * a.NB + qb;

  if (wv == 0) build_lists<LISTN>(a, brow, lists, counts);
  Stream st;
  st.beg = sload(a.row_ptr + (size_t)bh * (a.NB + 1) + qb);
  st.nA = (a.phases & PH_A) ? sload(a.row_ptr + (size_t)bh * (a.NB + 1) + qb + 1) - st.beg : 0;
  st.beg = __builtin_amdgcn_readfirstlane(st.beg);
  st.nA = __builtin_amdgcn_readfirstlane(st.nA);
  __syncthreads();
  st.nBrows = __builtin_amdgcn_readfirstlane(counts[0] * a.RM);
  st.nC = __builtin_amdgcn_readfirstlane(counts[1]);
  st.cA = st.nA;
  st.cB = (st.nBrows + BK - 1) / BK;
  st.cC = (st.nC + BK - 1) / BK;
  const int nc = st.cA + st.cB + st.cC;

  const unsigned head_bytes = (unsigned)((size_t)a.L * HD * 2);
  const srd_t rk = make_srd(a.k + head * HD, head_bytes);
  const srd_t rv = make_srd(a.v + head * HD, head_bytes);
  const srd_t rkm = make_srd(a.k_mid + (size_t)bh * a.mid_rows * HD, (unsigned)((size_t)a.mid_rows * HD * 2));
  const srd_t rvm = make_srd(a.v_mid + (size_t)bh * a.mid_rows * HD, (unsigned)((size_t)a.mid_rows * HD * 2));
  const srd_t rkt = make_srd(a.k_tail + (size_t)bh * a.tail_rows * HD, (unsigned)((size_t)a.tail_rows * HD * 2));
  const srd_t rvt = make_srd(a.v_tail + (size_t)bh * a.tail_rows * HD, (unsigned)((size_t)a.tail_rows * HD * 2));
  unsigned chb[4];
  int lrow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int P = (wv * 4 + i) * 64 + l, R = P >> 4;
    lrow[i] = R;
    chb[i] = (unsigned)(((P & 15) ^ swz(R)) * 16);
  }
  // stage chunk cj into buffer sb; returns (wave 0) the bias of chunk column l; `plain`: a tier-A block of 64
  // valid tokens (every bias 0)
  auto issue = [&](int cj, int sb, bool& plain) -> float {
    char* kd = kv_s[sb][0] + wv * 4096;
    char* vd = kv_s[sb][1] + wv * 4096;
    plain = false;
    if (cj < st.cA) {
      const int b = __builtin_amdgcn_readfirstlane(a.col_idx[st.beg + cj]);
      const unsigned soff = (unsigned)b * (BK * 256);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        dma16(rk, kd + i * 1024, (unsigned)lrow[i] * 256 + chb[i], soff);
        dma16(rv, vd + i * 1024, (unsigned)lrow[i] * 256 + chb[i], soff);
      }
      const int cnt = sload(a.blk_cnt + b);
      plain = cnt == BK;
      return l < cnt ? 0.0f : -INFINITY;
    }
    const bool tb = cj < st.cA + st.cB;
    const int p0 = (cj - (tb ? st.cA : st.cA + st.cB)) * BK;
    const int n = tb ? st.nBrows : st.nC;
    auto table_row = [&](int p) -> int {
      if (p >= n) return -1;
      return tb ? (int)lists[p / a.RM] * a.RM + p % a.RM : (int)lists[LISTN - 1 - p];
    };
    const srd_t r1 = tb ? rkm : rkt, r2 = tb ? rvm : rvt;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = table_row(p0 + lrow[i]);
      const unsigned off = row < 0 ? 0x80000000u : (unsigned)row * 256 + chb[i];
      dma16(r1, kd + i * 1024, off, 0);
      dma16(r2, vd + i * 1024, off, 0);
    }
    const int row = table_row(p0 + l);
    return row < 0 ? -INFINITY : (tb ? a.lc_mid[(size_t)bh * a.lc_mid_stride + row] : a.lc_tail[row]);
  };

  ev8 qreg[8], dreg[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    qreg[ks] = *reinterpret_cast<const ev8*>(a.q + tok * HD + 16 * ks + 8 * hi);
    if (BWD) dreg[ks] = *reinterpret_cast<const ev8*>(a.dout + tok * HD + 16 * ks + 8 * hi);
  }
  float ls = 0.0f, dl = 0.0f;
  if (BWD) {
    const float lv = a.lse[tok];
    ls = (qvalid && lv != -INFINITY) ? lv * LOG2E : INFINITY;
    dl = a.delta[tok];
  }
  int koff[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) koff[ks] = kh * 8192 + tile_off(lq, 2 * ks + hi);
  int toff[2][4];
  {
    const int g1 = (l >> 4) & 1, sub = (l & 1) * 8, rowA = 4 * hi + ((l & 15) >> 2);
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      toff[0][db] = kh * 8192 + tile_off(rowA, 4 * db + 2 * g1 + ((l & 3) >> 1)) + sub;
      toff[1][db] = kh * 8192 + tile_off(rowA + 8, 4 * db + 2 * g1 + ((l & 3) >> 1)) + sub;
    }
  }
  f32x16 acc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) acc[db] = f32x16{};
  float lsum = 0.0f, mref = -INFINITY;

  bool plain = false;  // chunk j is a tier-A block of 64 valid tokens: no bias, the scale goes into the exponent
  if (nc > 0) {
    const float b0 = issue(0, 0, plain);
    if (wv == 0) bias_s[0][l] = b0;
  }
  dma_wait();
  __syncthreads();
  for (int j = 0; j < nc; ++j) {
    const int sb = j & 1;
    float bn = 0.0f;
    bool plain_next = false;
    if (j + 1 < nc) bn = issue(j + 1, sb ^ 1, plain_next);
    const char* kt = kv_s[sb][0];
    const char* vt = kv_s[sb][1];
    f32x16 s = {};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) s = emfma(elds16(kt, koff[ks]), qreg[ks], s);
    float x[16];
    if (!plain) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 b4 = *reinterpret_cast<const f32x4*>(&bias_s[sb][32 * kh + 8 * g + 4 * hi]);
#pragma unroll
        for (int e = 0; e < 4; ++e) x[4 * g + e] = fmaf(s[4 * g + e], a.scale_log2, b4[e]);
      }
    }
    if (!BWD) {
      // (a plain chunk takes its maximum on the raw products: the scale is positive and rounding monotone)
      float mx;
      if (plain) {
        mx = s[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
        mx = max_xor32(mx) * a.scale_log2;
      } else {
        mx = x[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) mx = fmaxf(mx, x[r]);
        mx = max_xor32(mx);
      }
      if (__builtin_amdgcn_ballot_w64(mx > mref + SLACK) != 0) {
        const float mnew = fmaxf(mref, mx);
        const float alpha = mref == -INFINITY ? 0.0f : exp2f_fast(mref - mnew);
        lsum *= alpha;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[db][r] *= alpha;
        mref = mnew;
      }
      const float msub = mref == -INFINITY ? 0.0f : mref;
      if (plain) {
#pragma unroll
        for (int r = 0; r < 16; ++r) x[r] = exp2f_fast(fmaf(s[r], a.scale_log2, -msub));
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) x[r] = exp2f_fast(x[r] - msub);
      }
      const ev8 pa = epack8(&x[0]), pb = epack8(&x[8]);
      lsum += esum8(pb, esum8(pa, 0.0f));
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        acc[db] = emfma(ecat_tr(lds_read_tr(vt, toff[0][db]), lds_read_tr(vt, toff[1][db])), pa, acc[db]);
        acc[db] = emfma(ecat_tr(lds_read_tr(vt + 4096, toff[0][db]), lds_read_tr(vt + 4096, toff[1][db])), pb, acc[db]);
      }
    } else {
      f32x16 dp = {};
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) dp = emfma(elds16(vt, koff[ks]), dreg[ks], dp);
      float ds[16];
      if (plain) {
#pragma unroll
        for (int r = 0; r < 16; ++r) ds[r] = exp2f_fast(fmaf(s[r], a.scale_log2, -ls)) * (dp[r] - dl) * a.scale;
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) ds[r] = exp2f_fast(x[r] - ls) * (dp[r] - dl) * a.scale;
      }
      const ev8 sa = epack8(&ds[0]), sb8 = epack8(&ds[8]);
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        acc[db] = emfma(ecat_tr(lds_read_tr(kt, toff[0][db]), lds_read_tr(kt, toff[1][db])), sa, acc[db]);
        acc[db] = emfma(ecat_tr(lds_read_tr(kt + 4096, toff[0][db]), lds_read_tr(kt + 4096, toff[1][db])), sb8,
                         acc[db]);
      }
    }
    if (j + 1 < nc && wv == 0) bias_s[sb ^ 1][l] = bn;
    dma_wait();
    __syncthreads();
    plain = plain_next;
  }

  // combine the two key halves of each row group through LDS
  float* xo = reinterpret_cast<float*>(&kv_s[0][0][0]) + rg * (64 * 64);
  float* xm = reinterpret_cast<float*>(&kv_s[1][0][0]) + rg * 128;
  const float ltot = sum_xor32(lsum);
  if (kh == 1) {
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) xo[(db * 16 + r) * 64 + l] = acc[db][r];
    xm[l] = mref;
    xm[64 + l] = ltot;
  }
  __syncthreads();
  if (kh == 1) return;
  float a0 = 1.0f, a1 = 1.0f, inv = 1.0f, lse2 = 0.0f;
  bool live = qvalid;
  if (!BWD) {
    const float m1 = xm[l], l1 = xm[64 + l];
    const float M = fmaxf(mref, m1);
    a0 = mref == -INFINITY ? 0.0f : exp2f_fast(mref - M);
    a1 = m1 == -INFINITY ? 0.0f : exp2f_fast(m1 - M);
    const float lt = a0 * ltot + a1 * l1;
    live = qvalid && lt > 0.0f;
    inv = live ? 1.0f / lt : 0.0f;
    lse2 = live ? M + log2f(lt) : -INFINITY;
  } else {
    inv = qvalid ? 1.0f : 0.0f;
  }
  const float inv_cnt = qvalid ? 1.0f / (float)qcnt : 0.0f;
  const float* adq = a.add_dq ? a.add_dq + ((size_t)bh * a.add_nb + qb) * HD : nullptr;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = 32 * db + 8 * i + 4 * hi;
      f32x4 x;
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = (a0 * acc[db][4 * i + e] + a1 * xo[(db * 16 + 4 * i + e) * 64 + l]) * inv;
      if (BWD && a.dq_acc != nullptr) {
        if (qvalid) x += *reinterpret_cast<const f32x4*>(a.dq_acc + tok * HD + c);
      }
      if (BWD && adq != nullptr) x += *reinterpret_cast<const f32x4*>(adq + c) * inv_cnt;
      ushort4 u;
      u.x = f2e(x[0]); u.y = f2e(x[1]); u.z = f2e(x[2]); u.w = f2e(x[3]);
      *reinterpret_cast<ushort4*>(a.out + tok * HD + c) = u;
    }
  if (!BWD && hi == 0) a.lse_out[tok] = live ? lse2 * LN2_F : -INFINITY;
}

// ------------------------------------------------------------------------------------------------ table dK / dV
struct TabArgs {
  const e16_t *q, *dout;
  const e16_t *k_tab, *v_tab;  // [BH, rows_pad, D]
  const float* lc;              // [rows], or [BH, lc_stride] per head
  int lc_stride;
  const float *lse, *delta;
  const unsigned *bits_a, *bits_ab;
  float *dk_tab, *dv_tab;       // [BH, rows_pad, D] fp32, accumulated
  int* queues;                  // the eight row-group queue counters of this launch (queues.h)
  int L, NB, RM, W, rows, rows_pad, tier, BH, fixed;  // tier: PH_B or PH_C
  float scale_log2, scale;
};

// 64-bit mask of the tier blocks of query-block row `row` among the workgroup's blocks fb .. fb + nblk - 1 (plain
// per-thread loads: each thread of a refill looks at its own query block)
__device__ __forceinline__ unsigned long long tier_mask(const TabArgs& a, size_t row, int fb, int nblk) {
  const int w0 = fb >> 5;
  auto word = [&](int w) -> unsigned long long {
    if (w >= a.W) return 0ull;
    const unsigned abv = a.bits_ab[row * a.W + w];
    unsigned m = a.tier == PH_B ? (abv & ~a.bits_a[row * a.W + w]) : ~abv;
    const int lo = w * 32;
    if (a.NB - lo < 32) m &= (1u << (a.NB - lo)) - 1u;
    return m;
  };
  unsigned long long m = word(w0) | (nblk > 32 - (fb & 31) ? word(w0 + 1) << 32 : 0ull);
  m >>= (fb & 31);
  return nblk >= 64 ? m : (m & ((1ull << nblk) - 1ull));
}

// one 512-thread workgroup per (64 table rows, head) in head-major balanced order (queues.h), one per CU, in the
// fine KV-owner layout (2 key halves x 2 query halves) twice: a dV group of four waves (S, P, dV) and a dK group
// (dP with the table's V rows in registers, dS from the dV group's P handed over through LDS, dK), one accumulator
// set per wave so that two waves share a SIMD; each query block's Q / dO is staged once for both groups.
__global__ __launch_bounds__(512, 1) void rep_bwd_tab_kernel(TabArgs a) {
  __shared__ __attribute__((aligned(16))) char qd_s[2][2][BK * 256];
  __shared__ __attribute__((aligned(16))) float st_s[2][2][BK];
  __shared__ f32x4 p_s[4][4 * 64];  // P of each dV wave, for the dK wave of the same tiles
  // ring of the query blocks with at least one tier pair among this workgroup's blocks, and their masks, filled
  // 256 query blocks at a time by the whole workgroup (one mask per thread, ballot compaction), so the loop reads
  // its next block from LDS instead of scanning the bitmaps block by block
  constexpr int RING = 512;
  __shared__ int act_s[RING];
  __shared__ unsigned long long am_s[RING];
  __shared__ int wcnt_s[8];
  int grp, bh;
  if (!balanced_head_item(a.queues, a.fixed, a.rows_pad / BK, a.BH, bh, grp)) return;
  const int tid = threadIdx.x, l = tid & 63, hi = l >> 5, lq = l & 31;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wl = wv & 3, part = wv >> 2;  // wave within its group; 0: dV, 1: dK (wave-uniform)
  const int kh = wl & 1, qh = wl >> 1;
  const int key = 32 * kh + lq;
  const int trow = grp * BK + key;  // table row of this lane's key
  const int per_blk = a.tier == PH_B ? a.RM : 1;
  const int fb = grp * BK / per_blk, nblk = BK / per_blk;
  const int lblk = key / per_blk;   // block of this key within the workgroup's blocks
  const float kbias = trow < a.rows ? a.lc[(size_t)bh * a.lc_stride + trow] : -INFINITY;
  const size_t head = (size_t)bh * a.L;

  const unsigned head_bytes = (unsigned)((size_t)a.L * HD * 2);
  const srd_t rq = make_srd(a.q + head * HD, head_bytes);
  const srd_t rd = make_srd(a.dout + head * HD, head_bytes);
  unsigned ld_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int P = (wl * 4 + i) * 64 + l, R = P >> 4;
    ld_off[i] = (unsigned)R * 256 + (unsigned)(((P & 15) ^ swz(R)) * 16);
  }
  ev8 kreg[8], vreg[8];
  {
    const size_t off = ((size_t)bh * a.rows_pad + trow) * HD + 8 * hi;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      if (part == 0) kreg[ks] = *reinterpret_cast<const ev8*>(a.k_tab + off + 16 * ks);
      else vreg[ks] = *reinterpret_cast<const ev8*>(a.v_tab + off + 16 * ks);
    }
  }
  // (wave 0 also loads the block's raw LSE and delta; `stats` turns them into what st_s holds once the transfers
  // have been waited for, so that the compiler's wait for these loads does not come first and wait for the
  // transfers as well)
  auto issue = [&](int i, int sb, float& lv, float& dl) {  // (the dV group stages Q, the dK group dO)
    const unsigned soff = (unsigned)i * (BK * 256);
#pragma unroll
    for (int r = 0; r < 4; ++r) dma16(part ? rd : rq, qd_s[sb][part] + wl * 4096 + r * 1024, ld_off[r], soff);
    if (wv == 0) {
      const size_t t = head + (size_t)i * BK + l;
      lv = a.lse[t];
      dl = a.delta[t];
    }
  };
  auto stats = [&](int sb, float lv, float dl) {  // wave 0, after dma_wait()
    asm volatile("" : "+v"(lv), "+v"(dl));
    st_s[sb][0][l] = lv == -INFINITY ? INFINITY : lv * LOG2E;
    st_s[sb][1][l] = dl;
  };
  int produced = 0, chunk = 0;  // ring entries written so far, query-block chunks (of 256) scanned so far
  auto refill = [&]() {         // every thread (the masks from the first 256); ends with a barrier
    const int i = chunk * 256 + tid;
    const unsigned long long m = (tid < 256 && i < a.NB) ? tier_mask(a, (size_t)bh * a.NB + i, fb, nblk) : 0ull;
    const unsigned long long bal = __builtin_amdgcn_ballot_w64(m != 0ull);
    if (l == 0) wcnt_s[wv] = __popcll(bal);
    __syncthreads();
    int before = 0, total = 0;
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      const int c = wcnt_s[w];
      before += w < wv ? c : 0;
      total += c;
    }
    if (m != 0ull) {
      const int slot = (produced + before + __popcll(bal & ((1ull << l) - 1ull))) & (RING - 1);
      act_s[slot] = i;
      am_s[slot] = m;
    }
    produced += total;
    ++chunk;
    __syncthreads();
  };
  // at least `need` entries written, or every query block scanned (wave-uniform)
  auto ensure = [&](int need) {
    while (produced < need && chunk * 256 < a.NB) refill();
  };
  int aoff[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) aoff[ks] = qh * 8192 + tile_off(lq, 2 * ks + hi);
  int toff[2][4];
  {
    const int g1 = (l >> 4) & 1, sub = (l & 1) * 8, rowA = 4 * hi + ((l & 15) >> 2);
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      toff[0][db] = qh * 8192 + tile_off(rowA, 4 * db + 2 * g1 + ((l & 3) >> 1)) + sub;
      toff[1][db] = qh * 8192 + tile_off(rowA + 8, 4 * db + 2 * g1 + ((l & 3) >> 1)) + sub;
    }
  }
  f32x16 acc[4];  // dV (group 0) or dK (group 1)
#pragma unroll
  for (int db = 0; db < 4; ++db) acc[db] = f32x16{};

  float ls = 0.0f, dl = 0.0f;
  ensure(1);
  int icur = produced > 0 ? act_s[0] : a.NB;
  unsigned long long mcur = produced > 0 ? am_s[0] : 0ull;
  if (icur < a.NB) {
    issue(icur, 0, ls, dl);
    dma_wait();
    if (wv == 0) stats(0, ls, dl);
  }
  dma_wait();
  __syncthreads();
  for (int j = 0; icur < a.NB; ++j) {
    const int sb = j & 1;
    ensure(j + 2);  // (entries j and j + 1 stay in the ring: a refill writes at most 256 past the last one)
    const int inext = j + 1 < produced ? act_s[(j + 1) & (RING - 1)] : a.NB;
    const unsigned long long mnext = j + 1 < produced ? am_s[(j + 1) & (RING - 1)] : 0ull;
    if (inext < a.NB) issue(inext, sb ^ 1, ls, dl);
    // this lane's key: bias log2(c) when its block's pair with query block icur is in the tier, else -inf
    const float kb = ((mcur >> lblk) & 1ull) ? kbias : -INFINITY;
    const char* qt = qd_s[sb][0];
    const char* dt = qd_s[sb][1];
    f32x16 s = {}, dp = {};
    float p[16], ds[16];
    ev8 xa8, xb8;  // the B operands of this wave's last product: P (dV) or dS (dK), bf16
    // the dV wave computes S and P and hands P (fp32) to the dK wave of the same tiles, which computes dP meanwhile
    f32x4* pex = p_s[wl];
    if (part == 0) {
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) s = emfma(elds16(qt, aoff[ks]), kreg[ks], s);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 l4 = *reinterpret_cast<const f32x4*>(&st_s[sb][0][32 * qh + 8 * g + 4 * hi]);
#pragma unroll
        for (int e = 0; e < 4; ++e) p[4 * g + e] = exp2f_fast(fmaf(s[4 * g + e], a.scale_log2, kb) - l4[e]);
        pex[g * 64 + l] = f32x4{p[4 * g], p[4 * g + 1], p[4 * g + 2], p[4 * g + 3]};
      }
      xa8 = epack8(&p[0]);
      xb8 = epack8(&p[8]);
    } else {
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) dp = emfma(elds16(dt, aoff[ks]), vreg[ks], dp);
    }
    __syncthreads();  // P is in LDS
    if (part == 1) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 d4 = *reinterpret_cast<const f32x4*>(&st_s[sb][1][32 * qh + 8 * g + 4 * hi]);
        const f32x4 pv = pex[g * 64 + l];
#pragma unroll
        for (int e = 0; e < 4; ++e) ds[4 * g + e] = pv[e] * (dp[4 * g + e] - d4[e]) * a.scale;
      }
      xa8 = epack8(&ds[0]);
      xb8 = epack8(&ds[8]);
    }
    // dV += P^T dO (group 0) or dK += dS^T Q (group 1): the same products on the other tile and operand
    const char* xt = part == 0 ? dt : qt;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      acc[db] = emfma(ecat_tr(lds_read_tr(xt, toff[0][db]), lds_read_tr(xt, toff[1][db])), xa8, acc[db]);
      acc[db] = emfma(ecat_tr(lds_read_tr(xt + 4096, toff[0][db]), lds_read_tr(xt + 4096, toff[1][db])), xb8, acc[db]);
    }
    dma_wait();
    if (inext < a.NB && wv == 0) stats(sb ^ 1, ls, dl);
    __syncthreads();
    icur = inext;
    mcur = mnext;
  }

  // sum the query-half partials (each group in its own half of the staging buffers)
  float* xa = reinterpret_cast<float*>(&qd_s[0][0][0]) + part * (2 * 64 * 64) + kh * (64 * 64);
  if (qh == 1) {
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) xa[(db * 16 + r) * 64 + l] = acc[db][r];
  }
  __syncthreads();
  if (qh == 1) return;
  float* g = (part == 0 ? a.dv_tab : a.dk_tab) + ((size_t)bh * a.rows_pad + trow) * HD;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = 32 * db + 8 * i + 4 * hi;
      f32x4 x4;
#pragma unroll
      for (int e = 0; e < 4; ++e) x4[e] = acc[db][4 * i + e] + xa[(db * 16 + 4 * i + e) * 64 + l];
      *reinterpret_cast<f32x4*>(g + c) = *reinterpret_cast<const f32x4*>(g + c) + x4;
    }
}

// ------------------------------------------------------------------------------------------------ small passes
// grid (cdiv(NB, 4), BH), 256 threads: one wave per block, lane -> (row slot, 8 columns)
__global__ __launch_bounds__(256) void rep_unpool_kernel(const float* __restrict__ acc_k, const float* __restrict__ acc_v,
                                                         const float* __restrict__ dk_mid, const float* __restrict__ dv_mid,
                                                         const float* __restrict__ dk_tail,
                                                         const float* __restrict__ dv_tail, e16_t* __restrict__ dk,
                                                         e16_t* __restrict__ dv, const int* __restrict__ blk_cnt,
                                                         const uint8_t* __restrict__ labels,
                                                         const int* __restrict__ mid_counts, int L, int NB, int RM,
                                                         int mid_rows, int tail_rows) {
  const int blk = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (blk >= NB) return;
  const int l = threadIdx.x & 63, s = l >> 4, c8 = (l & 15) * 8;
  const size_t bh = blockIdx.y;
  const int cnt = blk_cnt[blk], gs = BK / RM;
  const float invc = 1.0f / (float)cnt;
  // the block-mean gradient is the same for every token of the block: loaded once, already divided by the count
  const size_t tail = (bh * tail_rows + blk) * HD + c8;
  f32x4 tk[2], tv[2];
#pragma unroll
  for (int h2 = 0; h2 < 2; ++h2) {
    tk[h2] = *reinterpret_cast<const f32x4*>(dk_tail + tail + 4 * h2) * invc;
    tv[h2] = *reinterpret_cast<const f32x4*>(dv_tail + tail + 4 * h2) * invc;
  }
  const bool has_k = acc_k != nullptr, has_v = acc_v != nullptr;
  auto pack = [](const f32x4& x0, const f32x4& x1) {
    uint4 u;
    u.x = (unsigned)f2e(x0[0]) | ((unsigned)f2e(x0[1]) << 16);
    u.y = (unsigned)f2e(x0[2]) | ((unsigned)f2e(x0[3]) << 16);
    u.z = (unsigned)f2e(x1[0]) | ((unsigned)f2e(x1[1]) << 16);
    u.w = (unsigned)f2e(x1[2]) | ((unsigned)f2e(x1[3]) << 16);
    return u;
  };
#pragma unroll 4
  for (int r = s; r < BK; r += 4) {
    const size_t lrow = bh * L + (size_t)blk * BK + r;
    const size_t tok = lrow * HD + c8;
    f32x4 xk[2] = {f32x4{}, f32x4{}}, xv[2] = {f32x4{}, f32x4{}};
    if (r < cnt) {
      // the token's representative: its contiguous group, or (k-means tables) its cluster
      const int g = labels ? (int)labels[lrow] : r / gs;
      const int n = labels ? mid_counts[(bh * NB + blk) * RM + g] : min(max(cnt - g * gs, 0), gs);
      const float invg = 1.0f / (float)n;
      const size_t mid = (bh * mid_rows + (size_t)blk * RM + g) * HD + c8;
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {  // (acc + mid / n) + tail / c, in that order
        const f32x4 ak = has_k ? *reinterpret_cast<const f32x4*>(acc_k + tok + 4 * h2) : f32x4{};
        const f32x4 av = has_v ? *reinterpret_cast<const f32x4*>(acc_v + tok + 4 * h2) : f32x4{};
        xk[h2] = (ak + *reinterpret_cast<const f32x4*>(dk_mid + mid + 4 * h2) * invg) + tk[h2];
        xv[h2] = (av + *reinterpret_cast<const f32x4*>(dv_mid + mid + 4 * h2) * invg) + tv[h2];
      }
    }
    *reinterpret_cast<uint4*>(dk + tok) = pack(xk[0], xk[1]);
    *reinterpret_cast<uint4*>(dv + tok) = pack(xv[0], xv[1]);
  }
}

// delta[row] = <dO, O> on valid rows, 0 on padding; one wave per block, 16 lanes per token row
__global__ __launch_bounds__(256) void row_dot_kernel(const e16_t* __restrict__ x, const e16_t* __restrict__ y,
                                                      float* __restrict__ out, const int* __restrict__ blk_cnt, int L,
                                                      int NB) {
  const int blk = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (blk >= NB) return;
  const int l = threadIdx.x & 63, s = l >> 4, c8 = (l & 15) * 8;
  const size_t bh = blockIdx.y;
  const int cnt = blk_cnt[blk];
  for (int r = s; r < BK; r += 4) {
    const size_t t = bh * L + (size_t)blk * BK + r;
    float acc = 0.0f;
    if (r < cnt) {
      const uint4 ux = *reinterpret_cast<const uint4*>(x + t * HD + c8);
      const uint4 uy = *reinterpret_cast<const uint4*>(y + t * HD + c8);
      const unsigned wx[4] = {ux.x, ux.y, ux.z, ux.w}, wy[4] = {uy.x, uy.y, uy.z, uy.w};
#pragma unroll
      for (int i = 0; i < 4; ++i)
        acc += e2f((e16_t)(wx[i] & 0xffffu)) * e2f((e16_t)(wy[i] & 0xffffu)) +
               e2f((e16_t)(wx[i] >> 16)) * e2f((e16_t)(wy[i] >> 16));
    }
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) acc += __shfl_xor(acc, m, 16);
    if ((l & 15) == 0) out[t] = acc;
  }
}

// tier-B lists: row i of the A|B lists without its tier-A columns (one wave per row); ptr_B = ptr_AB - ptr_A
__global__ __launch_bounds__(256) void tier_b_lists_kernel(const int* __restrict__ ab_ptr, const int* __restrict__ ab_idx,
                                                           const int* __restrict__ a_ptr,
                                                           const unsigned* __restrict__ bits_a, int* __restrict__ b_ptr,
                                                           int* __restrict__ b_idx, int NB, int W) {
  const int bh = blockIdx.y, row = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63;
  if (row >= NB) return;
  const size_t r = (size_t)bh * (NB + 1) + row;
  const int s0 = ab_ptr[r], s1 = ab_ptr[r + 1];
  const int o0 = s0 - a_ptr[r];
  if (l == 0) {
    b_ptr[r] = o0;
    if (row == NB - 1) b_ptr[r + 1] = s1 - a_ptr[r + 1];
  }
  const unsigned* bits = bits_a + ((size_t)bh * NB + row) * W;
  int out = o0;
  for (int e0 = s0; e0 < s1; e0 += 64) {
    const int e = e0 + l;
    int col = 0;
    bool keep = false;
    if (e < s1) {
      col = ab_idx[e];
      keep = ((bits[col >> 5] >> (col & 31)) & 1u) == 0u;
    }
    const unsigned long long m = __builtin_amdgcn_ballot_w64(keep);
    if (keep) b_idx[out + __popcll(m & ((1ull << l) - 1ull))] = col;
    out += __popcll(m);
  }
}

}  // namespace

}  // namespace es

using namespace es;

static int rep_check(int BH, int L, int D, int RM) {
  ES_REQUIRE(BH > 0 && BH <= 65535 && L > 0 && L % BK == 0, ES_ERR_INVALID, "VSA2-rep: tokens must be [BH, L = NB * 64, D]");
  ES_REQUIRE(D == 64 || D == HD, ES_ERR_UNSUPPORTED, "VSA2-rep: head dim must be 64 or 128 (rows stored with 128 columns)");
  ES_REQUIRE(L / BK <= REP_MAX_NB, ES_ERR_UNSUPPORTED, "VSA2-rep: NB <= 8192 blocks");
  ES_REQUIRE(RM == 1 || RM == 2 || RM == 4 || RM == 8 || RM == 16, ES_ERR_INVALID,
             "RepTiers.mid_reps must be one of (1, 2, 4, 8, 16)");
  ES_REQUIRE((size_t)L * HD * 2 < (1ull << 31), ES_ERR_UNSUPPORTED, "VSA2-rep: one head's tokens exceed 2 GiB");
  return ES_OK;
}

static RepArgs rep_args(const void* q, const void* k, const void* v, const void* k_mid, const void* v_mid,
                        const float* lc_mid, int lc_mid_stride, const void* k_tail, const void* v_tail, const float* lc_tail,
                        const int* q2k_ptr, const int* q2k_idx, const unsigned* bits_a, const unsigned* bits_ab,
                        const int* blk_cnt, int BH, int L, int D, int RM, int phases) {
  RepArgs a = {};
  a.q = (const e16_t*)q;
  a.k = (const e16_t*)k;
  a.v = (const e16_t*)v;
  a.k_mid = (const e16_t*)k_mid;
  a.v_mid = (const e16_t*)v_mid;
  a.lc_mid = lc_mid;
  a.lc_mid_stride = lc_mid_stride;
  a.k_tail = (const e16_t*)k_tail;
  a.v_tail = (const e16_t*)v_tail;
  a.lc_tail = lc_tail;
  a.row_ptr = q2k_ptr;
  a.col_idx = q2k_idx;
  a.bits_a = bits_a;
  a.bits_ab = bits_ab;
  a.blk_cnt = blk_cnt;
  a.L = L;
  a.NB = L / BK;
  a.RM = RM;
  a.W = (a.NB + 31) / 32;
  a.BH = BH;
  a.per_xcd = (a.NB + 7) / 8;
  a.phases = phases;
  a.mid_rows = (a.NB * RM + 63) / 64 * 64;
  a.tail_rows = (a.NB + 63) / 64 * 64;
  a.scale_log2 = LOG2E / sqrtf((float)D);
  a.scale = 1.0f / sqrtf((float)D);
  return a;
}

extern "C" int ES_VSA_API(vsa_rep_attn_fwd)(const void* q, const void* k, const void* v, const void* k_mid, const void* v_mid,
                                const float* lc_mid, int lc_mid_stride, const void* k_tail, const void* v_tail, const float* lc_tail,
                                const int* q2k_ptr, const int* q2k_idx, const unsigned* bits_a,
                                const unsigned* bits_ab, const int* blk_cnt, void* out, float* lse, int BH, int L,
                                int D, int RM, int phases, hipStream_t stream) {
  if (int st = rep_check(BH, L, D, RM)) return st;
  ES_REQUIRE(q && k && v && k_mid && v_mid && lc_mid && k_tail && v_tail && lc_tail && q2k_ptr && bits_a && bits_ab &&
                 blk_cnt && out && lse,
             ES_ERR_INVALID, "VSA2-rep: null tensor pointer");
  ES_REQUIRE(phases >= 0 && phases <= 7, ES_ERR_INVALID, "VSA2-rep: phases must be a mask of 1 | 2 | 4");
  ES_REQUIRE(lc_mid_stride == 0 || lc_mid_stride >= (L / BK) * RM, ES_ERR_INVALID,
             "VSA2-rep: lc_mid_stride must be 0 (shared) or >= NB * RM (per head)");
  RepArgs a = rep_args(q, k, v, k_mid, v_mid, lc_mid, lc_mid_stride, k_tail, v_tail, lc_tail, q2k_ptr, q2k_idx, bits_a, bits_ab,
                       blk_cnt, BH, L, D, RM, phases);
  a.out = (e16_t*)out;
  a.lse_out = lse;
  Queues qs;
  ES_REQUIRE(balanced_launch(BH, a.per_xcd, stream, qs), ES_ERR_LAUNCH, "VSA2-rep: row-block queues unavailable");
  a.queues = qs.counters;
  a.fixed = qs.fixed;
  if (L / BK <= REP_LIST)
    hipLaunchKernelGGL((rep_q_kernel<false, REP_LIST>), dim3((unsigned)qs.grid), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((rep_q_kernel<false, REP_MAX_NB>), dim3((unsigned)qs.grid), dim3(256), 0, stream, a);
  return check_launch("vsa_rep_attn_fwd");
}

extern "C" int ES_VSA_API(vsa_rep_attn_bwd_q)(const void* q, const void* k, const void* v, const void* k_mid, const void* v_mid,
                                  const float* lc_mid, int lc_mid_stride, const void* k_tail, const void* v_tail, const float* lc_tail,
                                  const void* dout, const float* lse, const float* delta, const int* q2k_ptr,
                                  const int* q2k_idx, const unsigned* bits_a, const unsigned* bits_ab,
                                  const int* blk_cnt, const float* add_dq, int add_nb, const float* dq_acc, void* dq,
                                  int BH, int L, int D, int RM, int phases, hipStream_t stream) {
  if (int st = rep_check(BH, L, D, RM)) return st;
  ES_REQUIRE(q && k && v && k_mid && v_mid && lc_mid && k_tail && v_tail && lc_tail && dout && lse && delta &&
                 q2k_ptr && bits_a && bits_ab && blk_cnt && dq,
             ES_ERR_INVALID, "VSA2-rep: null tensor pointer");
  ES_REQUIRE(add_dq == nullptr || add_nb >= L / BK, ES_ERR_INVALID, "VSA2-rep: add_dq has fewer rows than blocks");
  ES_REQUIRE(lc_mid_stride == 0 || lc_mid_stride >= (L / BK) * RM, ES_ERR_INVALID,
             "VSA2-rep: lc_mid_stride must be 0 (shared) or >= NB * RM (per head)");
  RepArgs a = rep_args(q, k, v, k_mid, v_mid, lc_mid, lc_mid_stride, k_tail, v_tail, lc_tail, q2k_ptr, q2k_idx, bits_a, bits_ab,
                       blk_cnt, BH, L, D, RM, phases);
  a.dout = (const e16_t*)dout;
  a.lse = lse;
  a.delta = delta;
  a.add_dq = add_dq;
  a.add_nb = add_nb;
  a.dq_acc = (float*)dq_acc;
  a.out = (e16_t*)dq;
  Queues qs;
  ES_REQUIRE(balanced_launch(BH, a.per_xcd, stream, qs), ES_ERR_LAUNCH, "VSA2-rep: row-block queues unavailable");
  a.queues = qs.counters;
  a.fixed = qs.fixed;
  if (L / BK <= REP_LIST)
    hipLaunchKernelGGL((rep_q_kernel<true, REP_LIST>), dim3((unsigned)qs.grid), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((rep_q_kernel<true, REP_MAX_NB>), dim3((unsigned)qs.grid), dim3(256), 0, stream, a);
  return check_launch("vsa_rep_attn_bwd_q");
}

extern "C" int ES_VSA_API(vsa_rep_bwd_tables)(const void* q, const void* dout, const void* k_tab, const void* v_tab,
                                  const float* lc, int lc_stride, const float* lse, const float* delta,
                                  const unsigned* bits_a, const unsigned* bits_ab, float* dk_tab, float* dv_tab,
                                  int BH, int L, int D, int RM, int tier, hipStream_t stream) {
  if (int st = rep_check(BH, L, D, RM)) return st;
  ES_REQUIRE(q && dout && k_tab && v_tab && lc && lse && delta && bits_a && bits_ab && dk_tab && dv_tab,
             ES_ERR_INVALID, "VSA2-rep: null tensor pointer");
  ES_REQUIRE(tier == 2 || tier == 4, ES_ERR_INVALID, "VSA2-rep: tier must be 2 (B, mid table) or 4 (C, tail table)");
  ES_REQUIRE(lc_stride == 0 || lc_stride >= (L / BK) * (tier == 2 ? RM : 1), ES_ERR_INVALID,
             "VSA2-rep: lc_stride must be 0 (shared) or >= the table's rows (NB * RM for tier 2, NB for tier 4)");
  TabArgs a = {};
  a.q = (const e16_t*)q;
  a.dout = (const e16_t*)dout;
  a.k_tab = (const e16_t*)k_tab;
  a.v_tab = (const e16_t*)v_tab;
  a.lc = lc;
  a.lc_stride = lc_stride;
  a.lse = lse;
  a.delta = delta;
  a.bits_a = bits_a;
  a.bits_ab = bits_ab;
  a.dk_tab = dk_tab;
  a.dv_tab = dv_tab;
  a.L = L;
  a.NB = L / BK;
  a.RM = RM;
  a.W = (a.NB + 31) / 32;
  a.tier = tier;
  a.rows = tier == 2 ? a.NB * RM : a.NB;
  a.rows_pad = (a.rows + 63) / 64 * 64;
  a.scale_log2 = LOG2E / sqrtf((float)D);
  a.scale = 1.0f / sqrtf((float)D);
  a.BH = BH;
  const int per_queue = (BH + 7) / 8 * (a.rows_pad / BK);
  Queues qs;
  ES_REQUIRE(balanced_launch_queues(per_queue, stream, qs), ES_ERR_LAUNCH, "VSA2-rep: row-group queues unavailable");
  a.queues = qs.counters;
  a.fixed = qs.fixed;
  hipLaunchKernelGGL(rep_bwd_tab_kernel, dim3((unsigned)qs.grid), dim3(512), 0, stream, a);
  return check_launch("vsa_rep_bwd_tables");
}

extern "C" int ES_VSA_API(vsa_rep_unpool)(const float* acc_k, const float* acc_v, const float* dk_mid, const float* dv_mid,
                              const float* dk_tail, const float* dv_tail, const int* blk_cnt, const uint8_t* labels,
                              const int* mid_counts, void* dk, void* dv, int BH, int L, int D, int RM,
                              hipStream_t stream) {
  if (int st = rep_check(BH, L, D, RM)) return st;
  ES_REQUIRE(dk_mid && dv_mid && dk_tail && dv_tail && blk_cnt && dk && dv, ES_ERR_INVALID,
             "VSA2-rep: null tensor pointer");
  ES_REQUIRE((labels == nullptr) == (mid_counts == nullptr), ES_ERR_INVALID,
             "VSA2-rep: pass labels and mid_counts together (k-means tables) or neither (contiguous groups)");
  const int NB = L / BK;
  hipLaunchKernelGGL(rep_unpool_kernel, dim3((NB + 3) / 4, BH), dim3(256), 0, stream, acc_k, acc_v, dk_mid, dv_mid,
                     dk_tail, dv_tail, (e16_t*)dk, (e16_t*)dv, blk_cnt, labels, mid_counts, L, NB, RM, (NB * RM + 63) / 64 * 64,
                     (NB + 63) / 64 * 64);
  return check_launch("vsa_rep_unpool");
}

extern "C" int ES_VSA_API(vsa_row_dot)(const void* x, const void* y, const int* blk_cnt, float* out, int BH, int L, int D,
                           hipStream_t stream) {
  ES_REQUIRE(x && y && blk_cnt && out, ES_ERR_INVALID, "VSA: null tensor pointer");
  ES_REQUIRE(BH > 0 && BH <= 65535 && L > 0 && L % BK == 0, ES_ERR_INVALID, "VSA: tokens must be [BH, L = NB * 64, D]");
  ES_REQUIRE(D == 64 || D == HD, ES_ERR_UNSUPPORTED, "VSA: head dim must be 64 or 128 (rows stored with 128 columns)");
  const int NB = L / BK;
  hipLaunchKernelGGL(row_dot_kernel, dim3((NB + 3) / 4, BH), dim3(256), 0, stream, (const e16_t*)x, (const e16_t*)y,
                     out, blk_cnt, L, NB);
  return check_launch("vsa_row_dot");
}

#ifndef ES_ELEM_F16  // no token tensors: built once
extern "C" int vsa_tier_b_lists(const int* ab_ptr, const int* ab_idx, const int* a_ptr, const unsigned* bits_a,
                                int* b_ptr, int* b_idx, int BH, int NB, hipStream_t stream) {
  ES_REQUIRE(ab_ptr && a_ptr && bits_a && b_ptr, ES_ERR_INVALID, "VSA2-rep: null tensor pointer");
  ES_REQUIRE(BH > 0 && BH <= 65535 && NB > 0, ES_ERR_INVALID, "VSA2-rep: bad shape");
  hipLaunchKernelGGL(tier_b_lists_kernel, dim3((NB + 3) / 4, BH), dim3(256), 0, stream, ab_ptr, ab_idx, a_ptr, bits_a,
                     b_ptr, b_idx, NB, (NB + 31) / 32);
  return check_launch("vsa_tier_b_lists");
}
#endif
