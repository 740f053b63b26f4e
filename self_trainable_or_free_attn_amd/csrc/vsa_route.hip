// VSA / VSA2 routers: block scores and exact top-k block selection into CSR lists (gfx950).
//
// Original VSA (reference csrc/vsa/vsa2_api.cpp:284-315 route_rows, scores.cu:1-6, topk.cu:621-685):
//   S[i, j] = rnd(rnd(qc_i . kc_j) / sqrt(D)) with rnd = bf16 rounding, then exactly K = min(topk, NB) blocks per
//   query-block row i: larger score first, equal scores by smaller j, -0 == +0. rows_select_kernel computes a
//   32-row strip of S with MFMA straight into LDS as order-preserving 16-bit keys (or reads given scores), and one
//   wave per row finds the K-th largest key by bisection over the 16-bit key space with wave ballots (16 rounds,
//   keys held in registers), then emits the row's ascending list and its selection bitmask with ballot prefix
//   counts.
// VSA2 (reference csrc/vsa/router/router.cu:1-15, vsa2_api.cpp:120-219, topk.cu:69-578):
//   psp_kernel: PSP scores over the pooled groups (qr / kr): pass 1 lse2 of each pooled query row over every valid
//   pooled key, pass 2 A = 2^(s * log2e / sqrt(D) - lse2) summed into (query block, key block) bins, times the row
//   norm 1 / G^2 ("paper") or 1 / #valid query groups ("valid_groups"). Each bin is produced by one lane in a fixed
//   order (deterministic).
//   Global top-k: exactly k = min(budget, NB^2) entries of each (b, h) score matrix under the total order (score
//   desc, flat index asc): a 4 x 8-bit radix select of the threshold key T and the number of T-equal entries to
//   take, per-row counts, a per-(b, h) scan, then one wave per row emits the ascending list and the bitmask.
// Both routers finish with the kv->q inversion: per 32-row group column counts of the selection bits, a per-(b, h)
// scan into k2q_ptr (base (bh0 + b) * keff), and an emission that lists each column's query blocks ascending.
#include "../../include/vsa_hip.h"
#include "common.h"
#include "elem.h"

#include <algorithm>

namespace es {

namespace {

constexpr int ROWS = 32;        // query-block rows per rows_select / inversion group
constexpr int MAX_NB = 2048;    // rows_select keeps a 32 x ceil64(NB) strip of 16-bit keys in LDS (<= 128 KB)
constexpr int WIDE_ROWS = 8;    // past MAX_NB: an 8 x ceil64(NB) strip (the rows of one S tile split over 4 workgroups)
constexpr int MAX_NB_WIDE = 8192;

// order-preserving keys: larger key = larger value; -0 and +0 share a key
__device__ __forceinline__ unsigned key16(unsigned u) {
  if ((u & 0x7fffu) == 0) u = 0;
  return (u & 0x8000u) ? (~u & 0xffffu) : (u | 0x8000u);
}
__device__ __forceinline__ unsigned key32(float f) {
  unsigned u = __float_as_uint(f);
  if ((u & 0x7fffffffu) == 0) u = 0;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ unsigned long long lanes_below() {
  return (1ull << (threadIdx.x & 63)) - 1ull;
}

// ------------------------------------------------------------------------------------ original-VSA rows
struct RowsArgs {
  const e16_t *qc, *kc;      // [BH, NBc_pad, D]
  const e16_t* scores_in;    // [bh_count, NB, NB] (FROM_SCORES)
  e16_t* scores_out;         // optional [bh_count, NB, NB]
  int *q2k_ptr, *q2k_idx;
  unsigned* selbits;          // [bh_count, ceil32(NB), W]
  int NB, NBc_pad, bh0, K, W;
  float scale;
};

// the selection of one row whose keys stay in LDS (WIDE): the same bisection of the K-th key, count of the keys
// above it and ascending emission with the T-equal entries taken smallest column first, as the register form below
__device__ __forceinline__ void select_row_lds(const unsigned short* keys, int NB, int nchunk, int K, int* out,
                                               unsigned* bits, int W) {
  const int l = threadIdx.x & 63;
  unsigned T = 0x10000u;
  if (K > 0) {
    unsigned lo = 0, hi2 = 0x10000u;
    while (hi2 - lo > 1) {
      const unsigned mid = (lo + hi2) >> 1;
      int cnt = 0;
      for (int c = 0; c < nchunk; ++c) cnt += __popcll(__builtin_amdgcn_ballot_w64(keys[64 * c + l] >= mid));
      if (cnt >= K) lo = mid; else hi2 = mid;
    }
    T = lo;
  }
  int above = 0;
  for (int c = 0; c < nchunk; ++c)
    above += __popcll(__builtin_amdgcn_ballot_w64((unsigned)keys[64 * c + l] > T && 64 * c + l < NB));
  const int take_eq = K - above;
  int eq_run = 0, sel_run = 0;
  for (int c = 0; c < nchunk; ++c) {
    const int j = 64 * c + l;
    const unsigned kv = keys[j];
    const bool in = j < NB;
    const bool eq = in && kv == T;
    const unsigned long long eqb = __builtin_amdgcn_ballot_w64(eq);
    const bool sel = in && (kv > T || (eq && eq_run + __popcll(eqb & lanes_below()) < take_eq));
    const unsigned long long sb = __builtin_amdgcn_ballot_w64(sel);
    if (sel) out[sel_run + __popcll(sb & lanes_below())] = j;
    eq_run += __popcll(eqb);
    sel_run += __popcll(sb);
    if (l < 2 && 2 * c + l < W) bits[2 * c + l] = (unsigned)(sb >> (32 * l));
  }
}

// grid (cdiv(NB, SR), bh_count), 256 threads, SR = 32 rows per workgroup (NB <= 2048, the keys of a row in
// registers) or 8 (WIDE, NB <= 8192: the S tile of 32 rows is computed by each of its four workgroups, which keep
// their 8 rows; the keys are read from LDS in every step). K < 0: scores only.
template <bool FROM_SCORES, bool WIDE>
__global__ __launch_bounds__(256) void rows_select_kernel(RowsArgs a) {
  constexpr int SR = WIDE ? WIDE_ROWS : ROWS;
  extern __shared__ __attribute__((aligned(16))) unsigned short keys_s[];  // [SR][NBp]
  const int strip = blockIdx.x, bhl = blockIdx.y;
  const int NB = a.NB, NBp = (NB + 63) & ~63;
  const int l = threadIdx.x & 63, hi = l >> 5, lq = l & 31;
  const int wv = threadIdx.x >> 6;
  const int r0 = strip * SR;           // first row of this workgroup
  const int t0 = r0 & ~(ROWS - 1);    // first row of its S tile
  const size_t bh = (size_t)(a.bh0 + bhl);

  if (FROM_SCORES) {
    for (int e = threadIdx.x; e < SR * NBp; e += 256) {
      const int r = e / NBp, c = e - r * NBp;
      const int row = r0 + r;
      keys_s[e] = (row < NB && c < NB) ? (unsigned short)key16(a.scores_in[((size_t)bhl * NB + row) * NB + c]) : 0;
    }
  } else {
    // S strip: A = qc rows t0 .. t0 + 31 (registers), B = kc rows of each 32-column tile (L2)
    ev8 qa[8];
    const e16_t* qp = a.qc + (bh * a.NBc_pad + t0 + lq) * HD + 8 * hi;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qa[ks] = *reinterpret_cast<const ev8*>(qp + 16 * ks);
    for (int ct = wv; ct < NBp / 32; ct += 4) {
      const e16_t* kp = a.kc + (bh * a.NBc_pad + ct * 32 + lq) * HD + 8 * hi;
      f32x16 acc = {};
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) acc = emfma(qa[ks], *reinterpret_cast<const ev8*>(kp + 16 * ks), acc);
      const int col = ct * 32 + lq;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int rr = t0 + 8 * (r / 4) + 4 * hi + (r % 4) - r0;  // row within this workgroup's strip
        if (WIDE && (rr < 0 || rr >= SR)) continue;
        const e16_t s = f2e(mul_rn(e2f(f2e(acc[r])), a.scale));
        const bool in = r0 + rr < NB && col < NB;
        keys_s[rr * NBp + col] = in ? (unsigned short)key16(s) : 0;
        if (a.scores_out != nullptr && in) a.scores_out[((size_t)bhl * NB + r0 + rr) * NB + col] = s;
      }
    }
  }
  if (a.K < 0) return;
  __syncthreads();

  const int K = a.K, nchunk = NBp / 64;
  for (int rr = wv; rr < SR; rr += 4) {
    const int row = r0 + rr;
    if (row >= NB) break;
    const long long base = ((long long)bh * NB + row) * K;
    if (l == 0) {
      int* ptr = a.q2k_ptr + bh * (NB + 1);
      ptr[row] = (int)base;
      if (row == NB - 1) ptr[NB] = (int)(base + K);
    }
    if (WIDE) {
      select_row_lds(keys_s + rr * NBp, NB, nchunk, K, a.q2k_idx + base,
                     a.selbits + ((size_t)bhl * (size_t)((NB + 31) & ~31) + row) * a.W, a.W);
      continue;
    }
    unsigned kv[MAX_NB / 64];
#pragma unroll
    for (int c = 0; c < MAX_NB / 64; ++c) kv[c] = c < nchunk ? keys_s[rr * NBp + 64 * c + l] : 0u;
    // T = the largest t with #(key >= t) >= K; keys of padding columns are 0 and never reach t >= 1
    unsigned T = 0x10000u;
    if (K > 0) {
      unsigned lo = 0, hi2 = 0x10000u;
      while (hi2 - lo > 1) {
        const unsigned mid = (lo + hi2) >> 1;
        int cnt = 0;
#pragma unroll
        for (int c = 0; c < MAX_NB / 64; ++c)
          if (c < nchunk) cnt += __popcll(__builtin_amdgcn_ballot_w64(kv[c] >= mid));
        if (cnt >= K) lo = mid; else hi2 = mid;
      }
      T = lo;
    }
    int above = 0;
#pragma unroll
    for (int c = 0; c < MAX_NB / 64; ++c)
      if (c < nchunk) above += __popcll(__builtin_amdgcn_ballot_w64(kv[c] > T && 64 * c + l < NB));
    const int take_eq = K - above;  // T-equal entries to take, smallest column first
    int eq_run = 0, sel_run = 0;
    int* out = a.q2k_idx + base;
    unsigned* bits = a.selbits + ((size_t)bhl * (size_t)((NB + 31) & ~31) + row) * a.W;
#pragma unroll
    for (int c = 0; c < MAX_NB / 64; ++c) {
      if (c >= nchunk) continue;
      const int j = 64 * c + l;
      const bool in = j < NB;
      const bool eq = in && kv[c] == T;
      const unsigned long long eqb = __builtin_amdgcn_ballot_w64(eq);
      const bool sel = in && (kv[c] > T || (eq && eq_run + __popcll(eqb & lanes_below()) < take_eq));
      const unsigned long long sb = __builtin_amdgcn_ballot_w64(sel);
      if (sel) out[sel_run + __popcll(sb & lanes_below())] = j;
      eq_run += __popcll(eqb);
      sel_run += __popcll(sb);
      if (l < 2 && 2 * c + l < a.W) bits[2 * c + l] = (unsigned)(sb >> (32 * l));
    }
  }
}

// ------------------------------------------------------------------------------------ kv->q inversion
// column counts of one 32-row group: gcnt[bhl][g][j]; rows >= NB have no bits set. The group's bits are staged
// in LDS COL_WORDS words (COL_WORDS * 32 columns) of every row at a time, so NB has no bound here.
constexpr int COL_WORDS = 128;
__global__ __launch_bounds__(256) void col_count_kernel(const unsigned* __restrict__ selbits, int* __restrict__ gcnt,
                                                        int NB, int W) {
  __shared__ unsigned bits_s[ROWS * COL_WORDS];
  const int g = blockIdx.x, bhl = blockIdx.y, NG = (NB + ROWS - 1) / ROWS;
  const unsigned* src = selbits + ((size_t)bhl * NG * ROWS + (size_t)g * ROWS) * W;
  const int nrows = min(ROWS, NB - g * ROWS);
  for (int w0 = 0; w0 < W; w0 += COL_WORDS) {
    const int nw = min(COL_WORDS, W - w0);
    __syncthreads();
    for (int e = threadIdx.x; e < nrows * nw; e += 256) {
      const int r = e / nw, w = e - r * nw;
      bits_s[r * COL_WORDS + w] = src[(size_t)r * W + w0 + w];
    }
    __syncthreads();
    for (int j = w0 * 32 + threadIdx.x; j < min(NB, (w0 + nw) * 32); j += 256) {
      const int wj = (j >> 5) - w0;
      int c = 0;
      for (int r = 0; r < nrows; ++r) c += (bits_s[r * COL_WORDS + wj] >> (j & 31)) & 1u;
      gcnt[((size_t)bhl * NG + g) * NB + j] = c;
    }
  }
}

// per (b, h): column j's groups get offsets base + (earlier columns) + (earlier groups of column j); base_of[b]
// is the absolute offset of (b, h)'s first list
__global__ __launch_bounds__(1024) void col_scan_kernel(int* __restrict__ gcnt, int* __restrict__ k2q_ptr, int NB,
                                                        int bh0, const long long* __restrict__ base_of) {
  __shared__ int red[16];
  const int bhl = blockIdx.x, NG = (NB + ROWS - 1) / ROWS;
  int* gc = gcnt + (size_t)bhl * NG * NB;
  const int per = (NB + 1023) / 1024;
  const int c0 = min(NB, (int)threadIdx.x * per), c1 = min(NB, c0 + per);
  int mine = 0;
  for (int j = c0; j < c1; ++j) {
    int run = 0;
    for (int g = 0; g < NG; ++g) run += gc[(size_t)g * NB + j];
    mine += run;
  }
  // exclusive scan of `mine` over the 1024 threads
  const int l = threadIdx.x & 63, wv = threadIdx.x >> 6;
  int inc = mine;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(inc, d, 64);
    if (l >= d) inc += y;
  }
  if (l == 63) red[wv] = inc;
  __syncthreads();
  int before = 0, total = 0;
  for (int i = 0; i < 16; ++i) {
    before += i < wv ? red[i] : 0;
    total += red[i];
  }
  const long long base = base_of[bhl];
  int* ptr = k2q_ptr + (size_t)(bh0 + bhl) * (NB + 1);
  int run = before + inc - mine;
  for (int j = c0; j < c1; ++j) {
    ptr[j] = (int)(base + run);
    for (int g = 0; g < NG; ++g) {
      const int c = gc[(size_t)g * NB + j];
      gc[(size_t)g * NB + j] = (int)(base + run);
      run += c;
    }
  }
  if (threadIdx.x == 1023) ptr[NB] = (int)(base + total);
}

__global__ __launch_bounds__(256) void col_emit_kernel(const unsigned* __restrict__ selbits,
                                                       const int* __restrict__ goff, int* __restrict__ k2q_idx, int NB,
                                                       int W) {
  __shared__ unsigned bits_s[ROWS * COL_WORDS];
  const int g = blockIdx.x, bhl = blockIdx.y, NG = (NB + ROWS - 1) / ROWS;
  const unsigned* src = selbits + ((size_t)bhl * NG * ROWS + (size_t)g * ROWS) * W;
  const int nrows = min(ROWS, NB - g * ROWS);
  for (int w0 = 0; w0 < W; w0 += COL_WORDS) {
    const int nw = min(COL_WORDS, W - w0);
    __syncthreads();
    for (int e = threadIdx.x; e < nrows * nw; e += 256) {
      const int r = e / nw, w = e - r * nw;
      bits_s[r * COL_WORDS + w] = src[(size_t)r * W + w0 + w];
    }
    __syncthreads();
    for (int j = w0 * 32 + threadIdx.x; j < min(NB, (w0 + nw) * 32); j += 256) {
      const int wj = (j >> 5) - w0;
      int n = goff[((size_t)bhl * NG + g) * NB + j];
      for (int r = 0; r < nrows; ++r)
        if ((bits_s[r * COL_WORDS + wj] >> (j & 31)) & 1u) k2q_idx[n++] = g * ROWS + r;
    }
  }
}

// ------------------------------------------------------------------------------------ global top-k
struct TopkState {
  unsigned prefix;  // high digits of T found so far (then T itself)
  int krem;         // entries still to take among those matching prefix
  long long keff;   // min(budget, NB^2)
  int pad[2];
};

__global__ void gk_init_kernel(TopkState* st, unsigned* hist, int bh_count, long long nn, long long budget) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < bh_count) {
    const long long keff = budget < 0 ? 0 : (budget < nn ? budget : nn);
    st[i].prefix = 0;
    st[i].krem = (int)keff;
    st[i].keff = keff;
  }
  for (int e = i; e < bh_count * 256; e += gridDim.x * blockDim.x) hist[e] = 0;
}

// pass p: histogram of digit (3 - p) of the keys whose higher digits equal the prefix
__global__ __launch_bounds__(256) void gk_hist_kernel(const float* __restrict__ scores, long long nn,
                                                      const TopkState* __restrict__ st, unsigned* __restrict__ hist,
                                                      int pass) {
  __shared__ unsigned h_s[256];
  const int bhl = blockIdx.y;
  h_s[threadIdx.x] = 0;
  __syncthreads();
  const int shift = 24 - 8 * pass;
  const unsigned himask = pass == 0 ? 0u : (0xffffffffu << (shift + 8));
  const unsigned prefix = st[bhl].prefix;
  if (st[bhl].keff > 0) {
    const float* s = scores + (size_t)bhl * nn;
    for (long long e = (long long)blockIdx.x * 256 + threadIdx.x; e < nn; e += (long long)gridDim.x * 256) {
      const unsigned k = key32(s[e]);
      if ((k & himask) == prefix) atomicAdd(&h_s[(k >> shift) & 255u], 1u);
    }
  }
  __syncthreads();
  if (h_s[threadIdx.x] != 0) atomicAdd(&hist[(size_t)bhl * 256 + threadIdx.x], h_s[threadIdx.x]);
}

// one wave per (b, h): the digit holding the krem-th largest remaining key; clears the histogram for the next pass
__global__ __launch_bounds__(64) void gk_find_kernel(TopkState* st, unsigned* hist, int pass) {
  const int bhl = blockIdx.x, l = threadIdx.x;
  unsigned* h = hist + (size_t)bhl * 256;
  const int krem = st[bhl].krem;
  unsigned c4[4];
  int mine = 0;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    c4[b] = h[4 * l + b];
    mine += (int)c4[b];
    h[4 * l + b] = 0;
  }
  if (st[bhl].keff <= 0) return;
  // inclusive suffix sums over lanes: entries in bins >= 4 l
  int suf = mine;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_down(suf, d, 64);
    if (l + d < 64) suf += y;
  }
  const unsigned long long ok = __builtin_amdgcn_ballot_w64(suf >= krem);
  const int top = 63 - __builtin_clzll(ok);
  if (l == top) {
    int cum = suf - mine;
    for (int b = 3; b >= 0; --b) {
      if (cum + (int)c4[b] >= krem) {
        const int shift = 24 - 8 * pass;
        st[bhl].prefix |= (unsigned)(4 * l + b) << shift;
        st[bhl].krem = krem - cum;
        break;
      }
      cum += (int)c4[b];
    }
  }
}

// one wave per row: #(key > T) and #(key == T)
__global__ __launch_bounds__(256) void gk_rowcount_kernel(const float* __restrict__ scores, int NB,
                                                          const TopkState* __restrict__ st, int* __restrict__ cnt) {
  const int bhl = blockIdx.y, row = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63;
  if (row >= NB) return;
  const unsigned T = st[bhl].prefix;
  const bool none = st[bhl].keff <= 0;
  const float* s = scores + ((size_t)bhl * NB + row) * NB;
  int gt = 0, eq = 0;
  for (int j = l; j < NB; j += 64) {
    const unsigned k = key32(s[j]);
    gt += k > T;
    eq += k == T;
  }
  gt = wave_sum_i(gt);
  eq = wave_sum_i(eq);
  if (l == 0) {
    cnt[((size_t)bhl * NB + row) * 2] = none ? 0 : gt;
    cnt[((size_t)bhl * NB + row) * 2 + 1] = none ? 0 : eq;
  }
}

// per (b, h): T-equal entries before each row (flat order), the row's take, q2k_ptr; cnt -> (eq_before, take)
__global__ __launch_bounds__(1024) void gk_scan_kernel(int* __restrict__ cnt, int* __restrict__ q2k_ptr, int NB,
                                                       int bh0, const TopkState* __restrict__ st) {
  __shared__ int red[2][16];
  const int bhl = blockIdx.x;
  int* c = cnt + (size_t)bhl * NB * 2;
  const int krem = st[bhl].krem;
  const long long keff = st[bhl].keff;
  const int per = (NB + 1023) / 1024;
  const int r0 = min(NB, (int)threadIdx.x * per), r1 = min(NB, r0 + per);
  int eq_mine = 0;
  for (int r = r0; r < r1; ++r) eq_mine += c[2 * r + 1];
  const int l = threadIdx.x & 63, wv = threadIdx.x >> 6;
  auto scan = [&](int x, int which, int& before_out) {
    int inc = x;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(inc, d, 64);
      if (l >= d) inc += y;
    }
    if (l == 63) red[which][wv] = inc;
    __syncthreads();
    int before = 0;
    for (int i = 0; i < wv; ++i) before += red[which][i];
    before_out = before + inc - x;
  };
  int eq_before;
  scan(eq_mine, 0, eq_before);
  int take_mine = 0;
  {
    int e = eq_before;
    for (int r = r0; r < r1; ++r) {
      const int gt = c[2 * r], eq = c[2 * r + 1];
      take_mine += gt + min(eq, max(0, krem - e));
      e += eq;
    }
  }
  int take_before;
  scan(take_mine, 1, take_before);
  const long long base = (long long)(bh0 + bhl) * keff;
  int* ptr = q2k_ptr + (size_t)(bh0 + bhl) * (NB + 1);
  int e = eq_before, t = take_before;
  for (int r = r0; r < r1; ++r) {
    const int gt = c[2 * r], eq = c[2 * r + 1];
    ptr[r] = (int)(base + t);
    c[2 * r] = e;  // T-equal entries before this row
    t += gt + min(eq, max(0, krem - e));
    e += eq;
  }
  if (threadIdx.x == 1023) ptr[NB] = (int)(base + (keff > 0 ? keff : 0));
}

// one wave per row: ascending list and selection bits
__global__ __launch_bounds__(256) void gk_emit_kernel(const float* __restrict__ scores, int NB, int bh0, int W,
                                                      const TopkState* __restrict__ st, const int* __restrict__ cnt,
                                                      const int* __restrict__ q2k_ptr, int* __restrict__ q2k_idx,
                                                      unsigned* __restrict__ selbits) {
  const int bhl = blockIdx.y, row = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63;
  if (row >= NB) return;
  const unsigned T = st[bhl].prefix;
  const int krem = st[bhl].keff > 0 ? st[bhl].krem : 0;
  const bool none = st[bhl].keff <= 0;
  const float* s = scores + ((size_t)bhl * NB + row) * NB;
  int eq_run = cnt[((size_t)bhl * NB + row) * 2];
  int sel_run = 0;
  int* out = q2k_idx + q2k_ptr[(size_t)(bh0 + bhl) * (NB + 1) + row];
  unsigned* bits = selbits + ((size_t)bhl * (size_t)((NB + 31) & ~31) + row) * W;
  for (int j0 = 0; j0 < NB; j0 += 64) {
    const int j = j0 + l;
    const bool in = j < NB && !none;
    const unsigned k = in ? key32(s[j]) : 0u;
    const bool eq = in && k == T;
    const unsigned long long eqb = __builtin_amdgcn_ballot_w64(eq);
    const bool sel = in && (k > T || (eq && eq_run + __popcll(eqb & lanes_below()) < krem));
    const unsigned long long sb = __builtin_amdgcn_ballot_w64(sel);
    if (sel) out[sel_run + __popcll(sb & lanes_below())] = j;
    eq_run += __popcll(eqb);
    sel_run += __popcll(sb);
    const int w0 = j0 >> 5;
    if (l < 2 && w0 + l < W) bits[w0 + l] = (unsigned)(sb >> (32 * l));
  }
}

// rows of the selection-bit buffer past NB (the last group's padding) must read as empty
__global__ void clear_pad_rows_kernel(unsigned* selbits, int NB, int W, int bh_count) {
  const int NBr = (NB + 31) & ~31, pad = NBr - NB;
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= bh_count * pad * W) return;
  const int bhl = e / (pad * W), rem = e - bhl * pad * W;
  selbits[((size_t)bhl * NBr + NB) * W + rem] = 0;
}

// absolute list base of each (b, h): (bh0 + b) * keff (routers) or the first entry of a given ptr (transpose)
__global__ void fill_base_kernel(long long* base, const TopkState* st, long long keff, const int* src_ptr, int NB,
                                 int bh0, int bh_count) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= bh_count) return;
  if (src_ptr != nullptr) base[i] = src_ptr[(size_t)(bh0 + i) * (NB + 1)];
  else base[i] = (long long)(bh0 + i) * (st ? st[i].keff : keff);
}

// the selection bitmap rows of (b, h) bh0 + b into bits_out [BH, NB, W] (the workspace pads rows to ceil32(NB))
__global__ void export_bits_kernel(const unsigned* __restrict__ selbits, unsigned* __restrict__ bits_out, int NB, int W,
                                   int bh0, int bh_count) {
  const long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (long long)bh_count * NB * W) return;
  const int bhl = (int)(e / ((long long)NB * W));
  const long long rem = e - (long long)bhl * NB * W;
  bits_out[(size_t)(bh0 + bhl) * NB * W + rem] = selbits[((size_t)bhl * ((NB + 31) & ~31)) * W + rem];
}

// selection bits of given CSR rows (one wave per row): bit j of row i set for every listed j
__global__ __launch_bounds__(256) void csr_bits_kernel(const int* __restrict__ ptr, const int* __restrict__ idx,
                                                       unsigned* __restrict__ selbits, int NB, int W, int bh0) {
  const int bhl = blockIdx.y, row = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63;
  if (row >= NB) return;
  const int* hp = ptr + (size_t)(bh0 + bhl) * (NB + 1);
  unsigned* bits = selbits + ((size_t)bhl * (size_t)((NB + 31) & ~31) + row) * W;
  for (int w = l; w < W; w += 64) bits[w] = 0;
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
  for (int e = hp[row] + l; e < hp[row + 1]; e += 64) {
    const int j = idx[e];
    atomicOr(&bits[j >> 5], 1u << (j & 31));
  }
}

// ------------------------------------------------------------------------------------ VSA2 PSP router
struct PspArgs {
  const e16_t *qr, *kr;  // [BH, Lr_pad, D]
  const int* blk_cnt;
  float* lse2;            // [BH, Lr_pad]
  float* scores;          // [bh_count, NB, NB]
  int NB, R, Lr, Lr_pad, bh0, row_norm;
  float scale_log2;
};

// pooled row r is valid iff its group holds >= 1 valid token
__device__ __forceinline__ bool group_valid(const PspArgs& a, int r) {
  return r < a.Lr && (r % (BK / a.R)) * a.R < a.blk_cnt[r / (BK / a.R)];
}

// grid (Lr_pad / 64, bh_count), 256 threads: 4 waves = 2 row groups of 32 pooled queries x 2 key halves of each
// 64-key chunk (the fine forward's layout: S^T = K Q^T with pooled keys on the rows, one query per lane column).
template <int G, bool SCORES>
__global__ __launch_bounds__(256) void psp_kernel(PspArgs a) {
  __shared__ __attribute__((aligned(16))) char k_s[2][BK * 256];
  __shared__ float bias_s[2][BK];
  __shared__ float xch_s[2][2][64];
  const int qt = blockIdx.x, bhl = blockIdx.y;
  const size_t bh = (size_t)(a.bh0 + bhl);
  const int tid = threadIdx.x, l = tid & 63, hi = l >> 5, lq = l & 31;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rg = wv & 1, kh = wv >> 1;
  const int qrow = qt * 64 + 32 * rg + lq;
  const bool qvalid = group_valid(a, qrow);
  const e16_t* kbase = a.kr + bh * a.Lr_pad * HD;
  const srd_t rk = make_srd(kbase, (unsigned)((size_t)a.Lr_pad * HD * 2));
  unsigned ld_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int P = (wv * 4 + i) * 64 + l, R = P >> 4;
    ld_off[i] = (unsigned)R * 256 + (unsigned)(((P & 15) ^ swz(R)) * 16);
  }
  auto issue = [&](int c, int sb) -> float {
#pragma unroll
    for (int i = 0; i < 4; ++i) dma16(rk, k_s[sb] + wv * 4096 + i * 1024, ld_off[i], (unsigned)c * (BK * 256));
    return group_valid(a, c * 64 + l) ? 0.0f : -INFINITY;
  };
  ev8 qreg[8];
  {
    const e16_t* qp = a.qr + (bh * a.Lr_pad + qrow) * HD + 8 * hi;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qreg[ks] = *reinterpret_cast<const ev8*>(qp + 16 * ks);
  }
  int koff[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) koff[ks] = kh * 8192 + tile_off(lq, 2 * ks + hi);

  const int nchunk = a.Lr_pad / 64;
  float m = -INFINITY, sum = 0.0f;     // pass 1: running max / sum (log2 domain)
  const float lse = SCORES ? (qvalid ? a.lse2[bh * a.Lr_pad + qrow] : INFINITY) : 0.0f;
  // pass 2 bins: a lane's 16 keys 32 kh + 8 (r / 4) + 4 hi + r % 4 fall into NBIN key blocks of G keys
  constexpr int NBIN = G == 2 ? 8 : G == 16 ? 2 : 4;
  auto bin_of = [](int r) { return G == 2 ? 2 * (r / 4) + (r % 4) / 2 : G == 16 ? r / 8 : r / 4; };
  auto block_of = [&](int b) {  // key block inside the 64-key chunk
    return G == 2 ? 16 * kh + 2 * hi + (b / 2) * 4 + b % 2 : G == 4 ? 8 * kh + 2 * b + hi : G == 8 ? 4 * kh + b : 2 * kh + b;
  };

  float b0 = issue(0, 0);
  if (wv == 0) bias_s[0][l] = b0;
  dma_wait();
  __syncthreads();
  for (int c = 0; c < nchunk; ++c) {
    const int sb = c & 1;
    float bn = 0.0f;
    if (c + 1 < nchunk) bn = issue(c + 1, sb ^ 1);
    f32x16 s = {};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) s = emfma(elds16(k_s[sb], koff[ks]), qreg[ks], s);
    float x[16];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 b4 = *reinterpret_cast<const f32x4*>(&bias_s[sb][32 * kh + 8 * g + 4 * hi]);
#pragma unroll
      for (int e = 0; e < 4; ++e) x[4 * g + e] = fmaf(s[4 * g + e], a.scale_log2, b4[e]);
    }
    if (!SCORES) {
      float mx = x[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mx = fmaxf(mx, x[r]);
      const float mn = fmaxf(m, mx);
      if (mn != -INFINITY) {
        float acc = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc += exp2f_fast(x[r] - mn);
        sum = sum * exp2f_fast(m - mn) + acc;
        m = mn;
      }
    } else {
      float p[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) p[r] = exp2f_fast(x[r] - lse);
      // this lane's keys into its key blocks, then over the query block's G lanes (and, G >= 8, the half-waves)
      float bin[NBIN];
#pragma unroll
      for (int b = 0; b < NBIN; ++b) bin[b] = 0.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) bin[bin_of(r)] += p[r];
#pragma unroll
      for (int b = 0; b < NBIN; ++b) {
        float v = bin[b];
        if (G >= 8) v += __shfl_xor(v, 32, 64);
#pragma unroll
        for (int d = 1; d < G; d <<= 1) v += __shfl_xor(v, d, 64);
        bin[b] = v;
      }
      const int qblk = qrow / G;
      if ((lq % G) == 0 && (G < 8 || hi == 0) && qblk < a.NB) {
        const int cnt = a.blk_cnt[qblk];
        const float norm = a.row_norm == 1 ? 1.0f / (float)(G * G) : 1.0f / (float)((cnt + a.R - 1) / a.R);
        float* out = a.scores + ((size_t)bhl * a.NB + qblk) * a.NB;
#pragma unroll
        for (int b = 0; b < NBIN; ++b) {
          const int kblk = c * (64 / G) + block_of(b);
          if (kblk < a.NB) out[kblk] = bin[b] * norm;
        }
      }
    }
    if (c + 1 < nchunk && wv == 0) bias_s[sb ^ 1][l] = bn;
    dma_wait();
    __syncthreads();
  }
  if (!SCORES) {
    // combine the half-waves, then the two key halves (kh) through LDS
    const float mo = __shfl_xor(m, 32, 64), so = __shfl_xor(sum, 32, 64);
    float M = fmaxf(m, mo);
    float S = M == -INFINITY ? 0.0f : sum * exp2f_fast(m - M) + so * exp2f_fast(mo - M);
    if (kh == 1 && hi == 0) {
      xch_s[rg][0][lq] = M;
      xch_s[rg][1][lq] = S;
    }
    __syncthreads();
    if (kh == 0 && hi == 0) {
      const float m2 = xch_s[rg][0][lq], s2 = xch_s[rg][1][lq];
      const float MM = fmaxf(M, m2);
      const float SS = MM == -INFINITY ? 0.0f
                                       : (M == -INFINITY ? 0.0f : S * exp2f_fast(M - MM)) +
                                             (m2 == -INFINITY ? 0.0f : s2 * exp2f_fast(m2 - MM));
      a.lse2[bh * a.Lr_pad + qrow] = SS > 0.0f ? MM + log2f(SS) : -INFINITY;
    }
  }
}

}  // namespace

}  // namespace es

using namespace es;

// ------------------------------------------------------------------------------------------- host side
static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct TopkCarve {
  unsigned* selbits;
  int* gcnt;
  int* rowcnt;
  TopkState* st;
  unsigned* hist;
  long long* base;
};

static size_t carve(void* base, int bh_count, int NB, TopkCarve* c) {
  const size_t W = (NB + 31) / 32, NBr = (NB + 31) & ~31, NG = (NB + ROWS - 1) / ROWS;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* p = (char*)base + off;
    off += align256(bytes);
    return p;
  };
  char* p0 = take((size_t)bh_count * NBr * W * 4);
  char* p1 = take((size_t)bh_count * NG * NB * 4);
  char* p2 = take((size_t)bh_count * NB * 2 * 4);
  char* p3 = take((size_t)bh_count * sizeof(TopkState));
  char* p4 = take((size_t)bh_count * 256 * 4);
  char* p5 = take((size_t)bh_count * 8);
  if (c) {
    c->selbits = (unsigned*)p0;
    c->gcnt = (int*)p1;
    c->rowcnt = (int*)p2;
    c->st = (TopkState*)p3;
    c->hist = (unsigned*)p4;
    c->base = (long long*)p5;
  }
  return off;
}

#ifndef ES_ELEM_F16  // no token tensors: built once
extern "C" size_t vsa_topk_workspace(int bh_count, int NB) {
  if (bh_count <= 0 || NB <= 0) return 0;
  return carve(nullptr, bh_count, NB, nullptr);
}
#endif

static int invert(const TopkCarve& c, int* k2q_ptr, int* k2q_idx, int NB, int bh0, int bh_count, hipStream_t stream) {
  const int W = (NB + 31) / 32, NG = (NB + ROWS - 1) / ROWS;
  hipLaunchKernelGGL(col_count_kernel, dim3(NG, bh_count), dim3(256), 0, stream, c.selbits, c.gcnt, NB, W);
  hipLaunchKernelGGL(col_scan_kernel, dim3(bh_count), dim3(1024), 0, stream, c.gcnt, k2q_ptr, NB, bh0, c.base);
  hipLaunchKernelGGL(col_emit_kernel, dim3(NG, bh_count), dim3(256), 0, stream, c.selbits, c.gcnt, k2q_idx, NB, W);
  return ES_OK;
}

static int rows_common(const void* qc, const void* kc, const void* scores_in, void* scores_out, int NB, int NBc_pad,
                       int bh0, int bh_count, int K, int* q2k_ptr, int* q2k_idx, int* k2q_ptr, int* k2q_idx,
                       void* workspace, size_t workspace_bytes, int D, hipStream_t stream, const char* what) {
  ES_REQUIRE(NB >= 1 && NB <= MAX_NB_WIDE, ES_ERR_UNSUPPORTED, "VSA: route_rows supports 1 <= NB <= 8192 blocks");
  ES_REQUIRE(bh0 >= 0 && bh_count >= 1 && bh_count <= 65535, ES_ERR_INVALID, "VSA: bad (b,h) range");
  RowsArgs a = {};
  a.qc = (const e16_t*)qc;
  a.kc = (const e16_t*)kc;
  a.scores_in = (const e16_t*)scores_in;
  a.scores_out = (e16_t*)scores_out;
  a.NB = NB;
  a.NBc_pad = NBc_pad;
  a.bh0 = bh0;
  a.W = (NB + 31) / 32;
  a.scale = 1.0f / sqrtf((float)D);  // D: the logical head dimension (64 or 128)
  const bool wide = NB > MAX_NB;
  const int SR = wide ? WIDE_ROWS : ROWS;
  const size_t lds = (size_t)SR * ((NB + 63) & ~63) * 2;  // <= 128 KB either way
  const dim3 grid((NB + SR - 1) / SR, bh_count);
  if (K < 0) {  // scores only
    a.K = -1;
    if (wide)
      hipLaunchKernelGGL((rows_select_kernel<false, true>), grid, dim3(256), lds, stream, a);
    else
      hipLaunchKernelGGL((rows_select_kernel<false, false>), grid, dim3(256), lds, stream, a);
    return check_launch(what);
  }
  ES_REQUIRE(q2k_ptr && k2q_ptr && workspace, ES_ERR_INVALID, "VSA: null tensor pointer");
  ES_REQUIRE(K == 0 || (q2k_idx && k2q_idx), ES_ERR_INVALID, "VSA: null list pointer");
  ES_REQUIRE(workspace_bytes >= vsa_topk_workspace(bh_count, NB), ES_ERR_INVALID, "VSA: top-k workspace too small");
  ES_REQUIRE((long long)(bh0 + bh_count) * NB * K < (1LL << 31), ES_ERR_UNSUPPORTED,
             "VSA: total selected blocks exceed int32 CSR range");
  TopkCarve c;
  carve(workspace, bh_count, NB, &c);
  a.K = K;
  a.q2k_ptr = q2k_ptr;
  a.q2k_idx = q2k_idx;
  a.selbits = c.selbits;
  const int W = a.W, pad = ((NB + 31) & ~31) - NB;
  if (pad > 0)
    hipLaunchKernelGGL(clear_pad_rows_kernel, dim3((bh_count * pad * W + 255) / 256), dim3(256), 0, stream, c.selbits,
                       NB, W, bh_count);
  hipLaunchKernelGGL(fill_base_kernel, dim3((bh_count + 255) / 256), dim3(256), 0, stream, c.base,
                     (const TopkState*)nullptr, (long long)NB * K, (const int*)nullptr, NB, bh0, bh_count);
  if (scores_in != nullptr && wide)
    hipLaunchKernelGGL((rows_select_kernel<true, true>), grid, dim3(256), lds, stream, a);
  else if (scores_in != nullptr)
    hipLaunchKernelGGL((rows_select_kernel<true, false>), grid, dim3(256), lds, stream, a);
  else if (wide)
    hipLaunchKernelGGL((rows_select_kernel<false, true>), grid, dim3(256), lds, stream, a);
  else
    hipLaunchKernelGGL((rows_select_kernel<false, false>), grid, dim3(256), lds, stream, a);
  invert(c, k2q_ptr, k2q_idx, NB, bh0, bh_count, stream);
  return check_launch(what);
}

extern "C" int ES_VSA_API(vsa_block_scores)(const void* qc, const void* kc, void* scores, int NB, int NBc_pad, int bh0,
                                int bh_count, int D, hipStream_t stream) {
  ES_REQUIRE(qc && kc && scores, ES_ERR_INVALID, "VSA: null tensor pointer");
  ES_REQUIRE(D == 64 || D == HD, ES_ERR_UNSUPPORTED, "VSA: head dim must be 64 or 128 (rows stored with 128 columns)");
  ES_REQUIRE(NBc_pad == (NB + 63) / 64 * 64, ES_ERR_INVALID, "qc must hold ceil(nb/64)*64 pooled rows");
  return rows_common(qc, kc, nullptr, scores, NB, NBc_pad, bh0, bh_count, -1, nullptr, nullptr, nullptr, nullptr,
                     nullptr, 0, D, stream, "vsa_block_scores");
}

extern "C" int ES_VSA_API(vsa_route_rows)(const void* qc, const void* kc, int NB, int NBc_pad, int bh0, int bh_count, int K,
                              int D, int* q2k_ptr, int* q2k_idx, int* k2q_ptr, int* k2q_idx, void* workspace,
                              size_t workspace_bytes, hipStream_t stream) {
  ES_REQUIRE(qc && kc, ES_ERR_INVALID, "VSA: null tensor pointer");
  ES_REQUIRE(D == 64 || D == HD, ES_ERR_UNSUPPORTED, "VSA: head dim must be 64 or 128 (rows stored with 128 columns)");
  ES_REQUIRE(NBc_pad == (NB + 63) / 64 * 64, ES_ERR_INVALID, "qc must hold ceil(nb/64)*64 pooled rows");
  ES_REQUIRE(K >= 0 && K <= NB, ES_ERR_INVALID, "VSA: K must be in [0, NB]");
  return rows_common(qc, kc, nullptr, nullptr, NB, NBc_pad, bh0, bh_count, K, q2k_ptr, q2k_idx, k2q_ptr, k2q_idx,
                     workspace, workspace_bytes, D, stream, "vsa_route_rows");
}

extern "C" int ES_VSA_API(vsa_row_topk)(const void* scores, int NB, int bh0, int bh_count, int K, int* q2k_ptr, int* q2k_idx,
                            int* k2q_ptr, int* k2q_idx, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  ES_REQUIRE(scores, ES_ERR_INVALID, "VSA: null tensor pointer");
  ES_REQUIRE(K >= 0 && K <= NB, ES_ERR_INVALID, "VSA: K must be in [0, NB]");
  return rows_common(nullptr, nullptr, scores, nullptr, NB, 0, bh0, bh_count, K, q2k_ptr, q2k_idx, k2q_ptr, k2q_idx,
                     workspace, workspace_bytes, HD, stream, "vsa_row_topk");
}

#ifndef ES_ELEM_F16  // no token tensors: built once
extern "C" int vsa_global_topk(const float* scores, int NB, int bh0, int bh_count, long long budget, int* q2k_ptr,
                               int* q2k_idx, int* k2q_ptr, int* k2q_idx, unsigned* bits_out, void* workspace,
                               size_t workspace_bytes, hipStream_t stream) {
  ES_REQUIRE(scores && q2k_ptr && k2q_ptr && workspace, ES_ERR_INVALID, "VSA: null tensor pointer");
  ES_REQUIRE(NB >= 1 && NB <= 46340 && bh0 >= 0 && bh_count >= 1 && bh_count <= 65535, ES_ERR_INVALID,
             "VSA: bad top-k shape");
  ES_REQUIRE(workspace_bytes >= vsa_topk_workspace(bh_count, NB), ES_ERR_INVALID, "VSA: top-k workspace too small");
  const long long nn = (long long)NB * NB;
  const long long keff = budget < 0 ? 0 : (budget < nn ? budget : nn);
  ES_REQUIRE(keff == 0 || (q2k_idx && k2q_idx), ES_ERR_INVALID, "VSA: null list pointer");
  ES_REQUIRE((long long)(bh0 + bh_count) * keff < (1LL << 31), ES_ERR_UNSUPPORTED,
             "VSA2: total selected blocks exceed int32 CSR range");
  TopkCarve c;
  carve(workspace, bh_count, NB, &c);
  const int W = (NB + 31) / 32, pad = ((NB + 31) & ~31) - NB;
  hipLaunchKernelGGL(gk_init_kernel, dim3((bh_count * 256 + 255) / 256), dim3(256), 0, stream, c.st, c.hist, bh_count,
                     nn, budget);
  const int chunks = (int)std::max<long long>(1, std::min<long long>((nn + 4095) / 4096, 1024));
  for (int pass = 0; pass < 4; ++pass) {
    hipLaunchKernelGGL(gk_hist_kernel, dim3(chunks, bh_count), dim3(256), 0, stream, scores, nn, c.st, c.hist, pass);
    hipLaunchKernelGGL(gk_find_kernel, dim3(bh_count), dim3(64), 0, stream, c.st, c.hist, pass);
  }
  const dim3 rgrid((NB + 3) / 4, bh_count);
  hipLaunchKernelGGL(gk_rowcount_kernel, rgrid, dim3(256), 0, stream, scores, NB, c.st, c.rowcnt);
  hipLaunchKernelGGL(gk_scan_kernel, dim3(bh_count), dim3(1024), 0, stream, c.rowcnt, q2k_ptr, NB, bh0, c.st);
  if (pad > 0)
    hipLaunchKernelGGL(clear_pad_rows_kernel, dim3((bh_count * pad * W + 255) / 256), dim3(256), 0, stream, c.selbits,
                       NB, W, bh_count);
  hipLaunchKernelGGL(gk_emit_kernel, rgrid, dim3(256), 0, stream, scores, NB, bh0, W, c.st, c.rowcnt, q2k_ptr,
                     q2k_idx, c.selbits);
  hipLaunchKernelGGL(fill_base_kernel, dim3((bh_count + 255) / 256), dim3(256), 0, stream, c.base, c.st, 0LL,
                     (const int*)nullptr, NB, bh0, bh_count);
  invert(c, k2q_ptr, k2q_idx, NB, bh0, bh_count, stream);
  if (bits_out != nullptr)
    hipLaunchKernelGGL(export_bits_kernel, dim3((bh_count * NB * W + 255) / 256), dim3(256), 0, stream, c.selbits,
                       bits_out, NB, W, bh0, bh_count);
  return check_launch("vsa_global_topk");
}
#endif

template <int G>
static void launch_psp(const PspArgs& a, bool scores, int bh_count, hipStream_t stream) {
  const dim3 grid(a.Lr_pad / 64, bh_count);
  if (scores)
    hipLaunchKernelGGL((psp_kernel<G, true>), grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((psp_kernel<G, false>), grid, dim3(256), 0, stream, a);
}

static int psp(const void* qr, const void* kr, const int* blk_cnt, float* lse2, float* scores, int NB, int R,
               int row_norm, int bh0, int bh_count, int D, bool do_scores, hipStream_t stream, const char* what) {
  ES_REQUIRE(qr && kr && blk_cnt && lse2 && (!do_scores || scores), ES_ERR_INVALID, "VSA: null tensor pointer");
  ES_REQUIRE(D == 64 || D == HD, ES_ERR_UNSUPPORTED, "VSA: head dim must be 64 or 128 (rows stored with 128 columns)");
  ES_REQUIRE(R == 4 || R == 8 || R == 16 || R == 32, ES_ERR_INVALID, "VSA2: router pool size R must be 4, 8, 16 or 32");
  ES_REQUIRE(row_norm == 0 || row_norm == 1, ES_ERR_INVALID, "VSA2: row_norm must be 0 (valid_groups) or 1 (paper)");
  ES_REQUIRE(NB >= 1 && bh0 >= 0 && bh_count >= 1 && bh_count <= 65535, ES_ERR_INVALID, "VSA: bad (b,h) range");
  const int G = BK / R;
  PspArgs a = {};
  a.qr = (const e16_t*)qr;
  a.kr = (const e16_t*)kr;
  a.blk_cnt = blk_cnt;
  a.lse2 = lse2;
  a.scores = scores;
  a.NB = NB;
  a.R = R;
  a.Lr = NB * G;
  a.Lr_pad = (NB * G + 63) / 64 * 64;
  a.bh0 = bh0;
  a.row_norm = row_norm;
  a.scale_log2 = LOG2E / sqrtf((float)D);
  ES_REQUIRE((size_t)a.Lr_pad * HD * 2 < (1ull << 31), ES_ERR_UNSUPPORTED, "VSA2: pooled rows exceed 2 GiB");
  switch (G) {
    case 2: launch_psp<2>(a, do_scores, bh_count, stream); break;
    case 4: launch_psp<4>(a, do_scores, bh_count, stream); break;
    case 8: launch_psp<8>(a, do_scores, bh_count, stream); break;
    default: launch_psp<16>(a, do_scores, bh_count, stream); break;
  }
  return check_launch(what);
}

extern "C" int ES_VSA_API(vsa_router_lse)(const void* qr, const void* kr, const int* blk_cnt, float* lse2, int NB, int R, int BH,
                              int D, hipStream_t stream) {
  return psp(qr, kr, blk_cnt, lse2, nullptr, NB, R, 0, 0, BH, D, false, stream, "vsa_router_lse");
}

extern "C" int ES_VSA_API(vsa_router_scores)(const void* qr, const void* kr, const float* lse2, const int* blk_cnt, float* scores,
                                 int NB, int R, int row_norm, int bh0, int bh_count, int D, hipStream_t stream) {
  return psp(qr, kr, blk_cnt, (float*)lse2, scores, NB, R, row_norm, bh0, bh_count, D, true, stream,
             "vsa_router_scores");
}

#ifndef ES_ELEM_F16  // no token tensors: built once
extern "C" int vsa_csr_transpose(const int* ptr, const int* idx, int NB, int bh0, int bh_count, int* out_ptr,
                                 int* out_idx, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  ES_REQUIRE(ptr && out_ptr && workspace, ES_ERR_INVALID, "VSA: null tensor pointer");
  ES_REQUIRE(NB >= 1 && NB <= 46340 && bh0 >= 0 && bh_count >= 1 && bh_count <= 65535, ES_ERR_INVALID,
             "VSA: bad CSR shape (1 <= NB <= 46340)");
  ES_REQUIRE(workspace_bytes >= vsa_topk_workspace(bh_count, NB), ES_ERR_INVALID, "VSA: workspace too small");
  TopkCarve c;
  carve(workspace, bh_count, NB, &c);
  const int W = (NB + 31) / 32, pad = ((NB + 31) & ~31) - NB;
  if (pad > 0)
    hipLaunchKernelGGL(clear_pad_rows_kernel, dim3((bh_count * pad * W + 255) / 256), dim3(256), 0, stream, c.selbits,
                       NB, W, bh_count);
  hipLaunchKernelGGL(csr_bits_kernel, dim3((NB + 3) / 4, bh_count), dim3(256), 0, stream, ptr, idx, c.selbits, NB, W,
                     bh0);
  hipLaunchKernelGGL(fill_base_kernel, dim3((bh_count + 255) / 256), dim3(256), 0, stream, c.base,
                     (const TopkState*)nullptr, 0LL, ptr, NB, bh0, bh_count);
  invert(c, out_ptr, out_idx, NB, bh0, bh_count, stream);
  return check_launch("vsa_csr_transpose");
}
#endif
