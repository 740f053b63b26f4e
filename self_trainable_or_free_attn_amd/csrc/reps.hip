// Four representatives per 64-token kv block, clustered in the query metric (reference
// echosparse/kernels/representatives.py:1-166).
//
//   gram_kernel    partial Gram matrices sum_rows q q^T per (head, row split), bf16 MFMA, fp32; written to the
//                  workspace and reduced in a fixed order (deterministic, unlike the reference's atomics)
//   chol_kernel    G = Gram * scale^2 / L + 1e-3 * mean(diag) * I; right-looking Cholesky in LDS with the pivot
//                  clamped at trace/D * 1e-12; writes the factor transposed (metric_t[e][d] = Lchol[d][e]), bf16
//   probe_kernel   64 probe queries: scale * mean of the valid q rows of block round(i * (nb - 1) / 63)
//   kmeans_kernel  one wave per (block, head): probe softmax weights (MFMA), the token Gram matrix X X^T of
//                  X = K Lchol (MFMA), weighted Lloyd on it from the four contiguous 16-token groups with early
//                  exit, plain K / V means per cluster (MFMA over one-hot labels) and log2 cluster sizes (-inf if
//                  empty); optionally the block means
#include "../../include/echosparse_hip.h"
#include "common.h"

#include <atomic>
#include <mutex>

namespace es {

constexpr int NPROBE = 64;
constexpr int MAX_SPLITS = 16;

struct RepWorkspace {
  float* gram;       // (H, S, D, D)
  bf16_t* metric_t;  // (H, D, D)
  bf16_t* probes;    // (H, 64, D)
  int splits, rows_per_split;
};

static RepWorkspace carve(void* ws, int L, int H) {
  RepWorkspace w;
  w.rows_per_split = (((L + MAX_SPLITS - 1) / MAX_SPLITS + 63) / 64) * 64;
  w.splits = (L + w.rows_per_split - 1) / w.rows_per_split;
  char* p = (char*)ws;
  w.gram = (float*)p;
  p += (size_t)H * w.splits * HD * HD * 4;
  w.metric_t = (bf16_t*)p;
  p += (size_t)H * HD * HD * 2;
  w.probes = (bf16_t*)p;
  return w;
}

static size_t ws_bytes(int L, int H) {
  RepWorkspace w = carve(nullptr, L, H);
  return (size_t)H * w.splits * HD * HD * 4 + (size_t)H * HD * HD * 2 + (size_t)H * NPROBE * HD * 2;
}

// stage rows [r0, r0 + 64) of one head of an (L, H, D) tensor into a swizzled LDS tile; rows >= L are clamped
// to L - 1 (callers mask them)
__device__ __forceinline__ void stage_rows(const bf16_t* x, int r0, int L, int H, int h, char* tile) {
  const int wv = threadIdx.x >> 6, l = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int P = (wv * 4 + i) * 64 + l;
    const int R = P >> 4, c = (P & 15) ^ swz(R);
    const int row = min(r0 + R, L - 1);
    g2lds16(x + ((size_t)row * H + h) * HD + c * 8, tile + (wv * 4 + i) * 1024);
  }
}

// transposed read of rows base + 0..3 at channel block (32 * db + lane % 32) of a swizzled tile
__device__ __forceinline__ s16x4 tr4(const char* tile, int base, int db) {
  const int l = threadIdx.x & 63;
  const int row = base + ((l & 15) >> 2);
  const int c = 4 * db + 2 * ((l >> 4) & 1) + ((l & 3) >> 1);
  return lds_read_tr(tile, tile_off(row, c) + (l & 1) * 8);
}

// stage_rows through the compiler-invisible transfer (dma16), one buffer resource per block: the caller waits
// (dma_wait) and synchronises before reading, and LDS reads of the other buffer are not held back behind it
__device__ __forceinline__ void stage_rows_dma(const bf16_t* x, int r0, int L, int H, int h, char* tile) {
  const int wv = threadIdx.x >> 6, l = threadIdx.x & 63, rows = min(BK, L - r0);
  const srd_t rs = make_srd(x + ((size_t)r0 * H + h) * HD, (unsigned)((rows - 1) * H * HD * 2 + 256));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int P = (wv * 4 + i) * 64 + l;
    const int R = P >> 4, c = (P & 15) ^ swz(R);
    dma16(rs, tile + (wv * 4 + i) * 1024, (unsigned)(min(R, rows - 1) * H * HD * 2 + c * 16), 0u);
  }
}

// partial Gram matrix of one (row split, head): 64-row chunks double-buffered in LDS, the next chunk's transfer
// in flight under the current chunk's products
__global__ __launch_bounds__(256) void gram_kernel(const bf16_t* __restrict__ q, float* __restrict__ gram, int L,
                                                   int H, int rps, int splits) {
  __shared__ __attribute__((aligned(16))) char tiles[2][BK * 256];
  const int s = blockIdx.x, h = blockIdx.y;
  const int wv = threadIdx.x >> 6, l = threadIdx.x & 63, hi = l >> 5, lq = l & 31;
  f32x16 acc[4] = {f32x16{}, f32x16{}, f32x16{}, f32x16{}};
  const int r_end = min(L, (s + 1) * rps);
  if (s * rps < r_end) stage_rows_dma(q, s * rps, L, H, h, tiles[0]);
  for (int r0 = s * rps, buf = 0; r0 < r_end; r0 += BK, buf ^= 1) {
    dma_wait();
    __syncthreads();  // chunk r0 has landed for every wave, and every wave is done with the other buffer
    if (r0 + BK < r_end) stage_rows_dma(q, r0 + BK, L, H, h, tiles[buf ^ 1]);
    const char* tile = tiles[buf];
    // rows >= r_end hold clamped copies: they are not part of this split, so zero their contribution by
    // restricting the k steps; the last chunk of a split may be partial only at L (rps is a multiple of 64)
    const int valid_rows = min(BK, r_end - r0);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      // slots 0..7 of half hi are rows 16 ks + 8 hi + 0..7
      const int base = 16 * ks + 8 * hi;
      bf16x8 a = cat_tr(tr4(tile, base, wv), tr4(tile, base + 4, wv));
      if (base + 8 > valid_rows) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (base + e >= valid_rows) a[e] = (__bf16)0.0f;
      }
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        bf16x8 b = cat_tr(tr4(tile, base, nb), tr4(tile, base + 4, nb));
        acc[nb] = mfma32(a, b, acc[nb]);
      }
    }
  }
  float* g = gram + ((size_t)h * splits + s) * HD * HD;
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d1 = 32 * wv + 8 * (r / 4) + 4 * hi + (r % 4), d2 = 32 * nb + lq;
      g[d1 * HD + d2] = acc[nb][r];
    }
}

// sum of the split partials of one head's Gram matrix, in split order, into the split-0 slot
__global__ __launch_bounds__(256) void gram_reduce_kernel(float* __restrict__ gram, int splits) {
  const int h = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
  float* g = gram + (size_t)h * splits * HD * HD + i;
  float s = 0.0f;
#pragma unroll 8
  for (int sp = 0; sp < splits; ++sp) s += g[(size_t)sp * HD * HD];  // (loads in flight together, sums in order)
  g[0] = s;
}

constexpr int CHOL_T = 1024;                 // threads of the Cholesky workgroup
constexpr int CHOL_R = HD * HD / CHOL_T;     // rows of one column per thread

__global__ __launch_bounds__(CHOL_T) void chol_kernel(const float* __restrict__ gram, bf16_t* __restrict__ metric_t,
                                                      int splits, float gscale) {
  __shared__ float A[HD][HD + 1];
  __shared__ float red[CHOL_T / 64];
  const int h = blockIdx.x, tid = threadIdx.x;
  // the split partials were summed into split 0 by gram_reduce_kernel
  for (int i = tid; i < HD * HD; i += CHOL_T) A[i / HD][i % HD] = gram[(size_t)h * splits * HD * HD + i] * gscale;
  __syncthreads();
  float dsum = tid < HD ? A[tid][tid] : 0.0f;
  dsum = wave_sum(dsum);
  if ((tid & 63) == 0) red[tid >> 6] = dsum;
  __syncthreads();
  const float ridge = 1e-3f * (red[0] + red[1]) / (float)HD;
  __syncthreads();
  if (tid < HD) A[tid][tid] += ridge;
  __syncthreads();
  float tr = tid < HD ? A[tid][tid] : 0.0f;
  tr = wave_sum(tr);
  if ((tid & 63) == 0) red[tid >> 6] = tr;
  __syncthreads();
  const float eps = (red[0] + red[1]) / (float)HD * 1e-12f;
  bf16_t* mt = metric_t + (size_t)h * HD * HD;
  // Register-resident right-looking factorisation: thread (cc = tid % 128, part = tid / 128) holds column cc at
  // rows 16 part .. 16 part + 15 (1024 threads, so a step's own arithmetic is short against its barrier and LDS
  // round trip). Step j: the owners of column j publish it into column buffer j % 2 (16-byte LDS writes) with its
  // rows above j as zeros, one barrier, then every thread reads the pivot column with 16-byte
  // broadcast reads and subtracts the rank-1 update col * (col[cc] / pivot) from its own entries: the zeros leave
  // the finished rows alone, and the columns left of j (already published) are never read again, so no entry
  // needs a mask. (Two buffers: step j+1 writes the other one while step j's readers may still be reading.)
  const int cc = tid & (HD - 1), rb = CHOL_R * (tid >> 7);
  float a[CHOL_R];
#pragma unroll
  for (int i = 0; i < CHOL_R; ++i) a[i] = A[rb + i][cc];
  __syncthreads();
  float* colbuf = &A[0][0];  // the matrix now lives in registers; reuse the LDS as two column buffers
  for (int j = 0; j < HD; ++j) {
    float* cb = colbuf + (j & 1) * HD;
    if (cc == j) {
#pragma unroll
      for (int q4 = 0; q4 < CHOL_R / 4; ++q4) {
        f32x4 c4;
#pragma unroll
        for (int k = 0; k < 4; ++k) c4[k] = rb + 4 * q4 + k >= j ? a[4 * q4 + k] : 0.0f;
        *reinterpret_cast<f32x4*>(cb + rb + 4 * q4) = c4;
      }
    }
    __syncthreads();
    const float inv = __builtin_amdgcn_rsqf(fmaxf(cb[j], eps));  // 1 / sqrt(pivot), hardware rsq (1 ulp)
    const float sc = cb[cc] * (inv * inv);
    if (tid < HD) mt[j * HD + tid] = f2bf(cb[tid] * inv);  // metric_t[j][d] = Lchol[d][j] (zero above j)
#pragma unroll
    for (int q4 = 0; q4 < CHOL_R / 4; ++q4) {
      const f32x4 c4 = *reinterpret_cast<const f32x4*>(cb + rb + 4 * q4);
#pragma unroll
      for (int k = 0; k < 4; ++k) a[4 * q4 + k] = fmaf(-c4[k], sc, a[4 * q4 + k]);
    }
  }
}

__global__ __launch_bounds__(64) void probe_kernel(const bf16_t* __restrict__ q, bf16_t* __restrict__ probes, int L,
                                                   int H, int NB, float scale) {
  const int i = blockIdx.x, h = blockIdx.y, l = threadIdx.x;
  const int blk = (int)((float)(i * (NB - 1)) / (float)(NPROBE - 1) + 0.5f);
  const int r0 = blk * BK, n = max(min(L - r0, BK), 0);
  float a = 0.f, b = 0.f;
#pragma unroll 8
  for (int r = 0; r < n; ++r) {  // (eight rows' loads in flight together; the sums take the rows in order)
    const unsigned w = *reinterpret_cast<const unsigned*>(q + ((size_t)(r0 + r) * H + h) * HD + 2 * l);
    a += __uint_as_float(w << 16);
    b += __uint_as_float(w & 0xffff0000u);
  }
  const float d = fmaxf((float)n, 1.0f);
  bf16_t* p = probes + ((size_t)h * NPROBE + i) * HD + 2 * l;
  p[0] = f2bf(a * scale / d);
  p[1] = f2bf(b * scale / d);
}

// stage rows [r0, r0 + 64) of one head of an (L, H, D) tensor into a swizzled LDS tile with one wave (16 transfers
// of 1 KB); rows >= L are clamped to L - 1 (callers mask them)
__device__ __forceinline__ void stage_rows_wave(const bf16_t* x, int r0, int L, int H, int h, char* tile) {
  const int l = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int P = i * 64 + l;
    const int R = P >> 4, c = (P & 15) ^ swz(R);
    const int row = min(r0 + R, L - 1);
    g2lds16(x + ((size_t)row * H + h) * HD + c * 8, tile + i * 1024);
  }
}

// x + the value of lane (lane ^ M) within each 32-lane half (ds_swizzle bit mode, no LDS traffic)
// the same staging through the compiler-invisible transfer (dma16): the caller waits (dma_wait) before reading, and
// LDS accesses in between are not held back behind it. A buffer resource per block keeps the offsets 32-bit.
__device__ __forceinline__ void stage_rows_wave_dma(const bf16_t* x, int r0, int L, int H, int h, char* tile) {
  const int l = threadIdx.x & 63, rows = min(BK, L - r0);
  const srd_t rs = make_srd(x + ((size_t)r0 * H + h) * HD, (unsigned)((rows - 1) * H * HD * 2 + 256));
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int P = i * 64 + l;
    const int R = P >> 4, c = (P & 15) ^ swz(R);
    dma16(rs, tile + i * 1024, (unsigned)(min(R, rows - 1) * H * HD * 2 + c * 16), 0u);
  }
}

// orders this wave's LDS accesses against each other across lanes (the wave runs in lockstep and the LDS serves a
// wave's instructions in order: only the compiler has to be kept from moving them)
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

template <int M>
__device__ __forceinline__ float swz_xor(float x) {
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), (M << 10) | 0x1F));
}

// kmeans_kernel: one wave (64-thread workgroup) per (block, head), no cross-wave synchronisation; 17.3 KB of LDS
// (the K tile, later the V tile, and per-token weights).
//
// The clustering works on the token Gram matrix P = X X^T (64 x 64, X = K Lchol) instead of X: a weighted centroid
// is a combination of tokens, mu_c = S_c / m_c with S_c = sum_s a_sc x_s, a_sc = w_s [lab_s == c] and
// m_c = max(sum_s a_sc, 1e-6), so with U[t][c] = sum_s a_sc P[s][t] = x_t . S_c
//   x_t . mu_c = U[t][c] / m_c   and   |mu_c|^2 = sum_t a_tc U[t][c] / m_c^2,
// the same distances |mu_c|^2 - 2 x_t . mu_c as the reference's Lloyd step (representatives.py:103-118) for 64 x 4
// x 64 multiply-adds per round instead of two 64 x 4 x 128 products. A cluster left without weight gets distance
// +inf in the next round, so the centroid it keeps in the reference is never used; the representatives are plain
// means over the final labels.
//   1. probe logits S^T = K probes^T (MFMA, tokens in registers, probes across lanes), the softmax over tokens in
//      registers, the sum over probes by a 32-lane reduce-scatter: token weights w (LDS)
//   2. X^T = Lchol^T K^T per 32-channel slice (MFMA, tokens across lanes), split into bf16 high + low parts, and
//      P += Xh Xh^T + Xh Xl^T + Xl Xh^T (relative error ~2^-16); P stays in registers (lane: token t, registers:
//      tokens s)
//   3. Lloyd from the four contiguous 16-token groups with early exit: each lane sums U over its registers' tokens
//      (the per-token cluster weights come from LDS), the two lane halves are added, |mu|^2 and m by wave sums
//   4. cluster sums of K and V: one-hot labels times the transposed tile on MFMA; the block means (MEANS) as the
//      same sequential fp32 sums as means_kernel
constexpr int KM_WAVES = 4;  // independent waves (blocks) per workgroup

template <bool MEANS>
__global__ __launch_bounds__(64 * KM_WAVES, 2) void kmeans_kernel(const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
                                                    const bf16_t* __restrict__ metric_t,
                                                    const bf16_t* __restrict__ probes, bf16_t* __restrict__ k4,
                                                    bf16_t* __restrict__ v4, float* __restrict__ lc4,
                                                    bf16_t* __restrict__ km, bf16_t* __restrict__ vm, int L, int H,
                                                    int NB, int iters) {
  __shared__ __attribute__((aligned(16))) char tiles[KM_WAVES][BK * 256];
  __shared__ __attribute__((aligned(16))) float wtoks[KM_WAVES][BK];
  __shared__ __attribute__((aligned(16))) f32x4 atoks[KM_WAVES][BK];

  const int wv = threadIdx.x >> 6;
  const int j = blockIdx.x * KM_WAVES + wv, h = blockIdx.y;
  if (j >= NB) return;  // (no workgroup barrier below: the waves are independent)
  char* tile = tiles[wv];
  float* wtok = wtoks[wv];
  f32x4* atok = atoks[wv];
  const int l = threadIdx.x & 63, hi = l >> 5, lq = l & 31;
  const int nvalid = min(L - j * BK, BK);
  const bf16_t* mt = metric_t + (size_t)h * HD * HD;
  const bf16_t* pr = probes + (size_t)h * NPROBE * HD;
  // token of register r of a 32 x 32 C tile whose rows are tokens (tile tb)
  auto row_tok = [&](int tb, int r) { return 32 * tb + 8 * (r >> 2) + 4 * hi + (r & 3); };

  stage_rows_wave(k, j * BK, L, H, h, tile);
  bf16x8 pop[8][2];  // probe operands (B: probe 32 pb + lq, channels 16 ks + 8 hi ..), loaded under the staging
#pragma unroll
  for (int ks = 0; ks < 8; ++ks)
#pragma unroll
    for (int pb = 0; pb < 2; ++pb)
      pop[ks][pb] = *reinterpret_cast<const bf16x8*>(pr + (size_t)(32 * pb + lq) * HD + 16 * ks + 8 * hi);
  wait_vmem();
  wave_lds_sync();

  bf16x8 mop[8];  // metric operands of the first 32-channel slice (A: metric_t row 32 eb + lq, channels 16 ks + 8 hi ..)
  // 1. probe logits: sp[tb][pb][r] = K[row_tok(tb, r)] . probe[32 pb + lq]
  {
    f32x16 sp[2][2] = {{f32x16{}, f32x16{}}, {f32x16{}, f32x16{}}};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
#pragma unroll
      for (int tb = 0; tb < 2; ++tb) {
        const bf16x8 kf = lds_read16(tile, tile_off(32 * tb + lq, 2 * ks + hi));
#pragma unroll
        for (int pb = 0; pb < 2; ++pb) sp[tb][pb] = mfma32(kf, pop[ks][pb], sp[tb][pb]);
      }
    if (nvalid < BK) {  // the last block: tokens past L get logit -inf, i.e. weight 0
#pragma unroll
      for (int tb = 0; tb < 2; ++tb)
#pragma unroll
        for (int pb = 0; pb < 2; ++pb)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (row_tok(tb, r) >= nvalid) sp[tb][pb][r] = -INFINITY;
    }
    float ew[32];  // [16 tb + r]: sum over this lane's probes of the normalised exponentials
#pragma unroll
    for (int i = 0; i < 32; ++i) ew[i] = 0.0f;
#pragma unroll
    for (int pb = 0; pb < 2; ++pb) {
      // max(x, m) as med3(x, m, +inf): one instruction, no operand canonicalisation
      float mx = -INFINITY;
#pragma unroll
      for (int tb = 0; tb < 2; ++tb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = __builtin_amdgcn_fmed3f(sp[tb][pb][r], mx, INFINITY);
      {
        const float2 hm = lane_pair32(mx);
        mx = __builtin_amdgcn_fmed3f(hm.x, hm.y, INFINITY);
      }
      const float nmx = -mx * LOG2E;
      float e[32], sm = 0.0f;
#pragma unroll
      for (int tb = 0; tb < 2; ++tb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          e[16 * tb + r] = exp2f_fast(fmaf(sp[tb][pb][r], LOG2E, nmx));
          sm += e[16 * tb + r];
        }
      sm = sum_xor32(sm);
      const float inv = 1.0f / sm;
#pragma unroll
      for (int i = 0; i < 32; ++i) ew[i] = fmaf(e[i], inv, ew[i]);
    }
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)  // (loaded under the reduction)
      mop[ks] = *reinterpret_cast<const bf16x8*>(mt + (size_t)lq * HD + 16 * ks + 8 * hi);
    // reduce-scatter over the 32 lanes of each half: lane lq ends with the total of value index lq
    float r16[16], r8[8], r4[4], r2[2];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const bool up = lq & 16;
      r16[i] = (up ? ew[i + 16] : ew[i]) + swz_xor<16>(up ? ew[i] : ew[i + 16]);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const bool up = lq & 8;
      r8[i] = (up ? r16[i + 8] : r16[i]) + swz_xor<8>(up ? r16[i] : r16[i + 8]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool up = lq & 4;
      r4[i] = (up ? r8[i + 4] : r8[i]) + swz_xor<4>(up ? r8[i] : r8[i + 4]);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const bool up = lq & 2;
      r2[i] = (up ? r4[i + 2] : r4[i]) + swz_xor<2>(up ? r4[i] : r4[i + 2]);
    }
    const bool up = lq & 1;
    const float tot = (up ? r2[1] : r2[0]) + swz_xor<1>(up ? r2[0] : r2[1]);
    const int t = row_tok(lq >> 4, lq & 15);
    wtok[t] = t < nvalid ? tot * ((float)nvalid / (float)NPROBE) : 0.0f;
  }

  // 2. P = X X^T, X^T built 32 channels at a time
  f32x16 P[2][2] = {{f32x16{}, f32x16{}}, {f32x16{}, f32x16{}}};  // [sb][tb]: P[row_tok(sb, r)][32 tb + lq]
#pragma unroll 1
  for (int eb = 0; eb < 4; ++eb) {
    f32x16 xt[2] = {f32x16{}, f32x16{}};  // X^T[32 eb + row][32 tb + lq]
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
#pragma unroll
      for (int tb = 0; tb < 2; ++tb)
        xt[tb] = mfma32(mop[ks], lds_read16(tile, tile_off(32 * tb + lq, 2 * ks + hi)), xt[tb]);
    bf16x8 xh[2][2], xl[2][2];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float x = xt[tb][8 * q + i];
          const __bf16 b = (__bf16)x;
          xh[tb][q][i] = b;
          xl[tb][q][i] = (__bf16)(x - (float)b);
        }
    if (eb < 3) {  // the next slice's metric operands load under this slice's P products
#pragma unroll
      for (int ks = 0; ks < 8; ++ks)
        mop[ks] = *reinterpret_cast<const bf16x8*>(mt + (size_t)(32 * (eb + 1) + lq) * HD + 16 * ks + 8 * hi);
    }
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
          P[sb][tb] = mfma32(xh[sb][q], xh[tb][q], P[sb][tb]);
          P[sb][tb] = mfma32(xh[sb][q], xl[tb][q], P[sb][tb]);
          P[sb][tb] = mfma32(xl[sb][q], xh[tb][q], P[sb][tb]);
        }
  }
  wave_lds_sync();  // wtok is written

  // the K tile's last uses: its transposed operands for the cluster sums (kept in registers) and the block mean;
  // then the V tile streams into the same LDS under the clustering
  auto block_mean = [&](bf16_t* dst) {  // the same sequential fp32 sum and division as means_kernel
    const int e = 2 * l;
    float a = 0.f, b = 0.f;
    if (nvalid == BK) {  // reads issued 16 rows ahead of the sums
#pragma unroll
      for (int r0 = 0; r0 < BK; r0 += 16) {
        unsigned w[16];
#pragma unroll
        for (int r = 0; r < 16; ++r)
          w[r] = *reinterpret_cast<const unsigned*>(tile + tile_off(r0 + r, e / 8) + (e % 8) * 2);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          a += __uint_as_float(w[r] << 16);
          b += __uint_as_float(w[r] & 0xffff0000u);
        }
      }
    } else {
#pragma unroll 4
      for (int r = 0; r < nvalid; ++r) {
        const unsigned w = *reinterpret_cast<const unsigned*>(tile + tile_off(r, e / 8) + (e % 8) * 2);
        a += __uint_as_float(w << 16);
        b += __uint_as_float(w & 0xffff0000u);
      }
    }
    const float n = (float)nvalid;
    const size_t o = ((size_t)j * H + h) * HD + e;
    dst[o] = f2bf(a / n);
    dst[o + 1] = f2bf(b / n);
  };
  if (MEANS) block_mean(km);
  bf16x8 kT[4][4];  // [db][ks]: K[16 ks + 8 hi + i][32 db + lq]
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int base = 16 * ks + 8 * hi;
      kT[db][ks] = cat_tr(tr4(tile, base, db), tr4(tile, base + 4, db));
    }
  wave_lds_sync();  // the K tile is consumed
  stage_rows_wave_dma(v, j * BK, L, H, h, tile);

  // 3. weighted Lloyd
  const bool tv[2] = {lq < nvalid, 32 + lq < nvalid};
  const float wt[2] = {wtok[lq], wtok[32 + lq]};
  int lab[2] = {lq >> 4, 2 + (lq >> 4)};  // the four contiguous 16-token groups
  // U summed over all four clusters does not depend on the labels; each round sums only the tokens whose label
  // has bit 0, bit 1, or both set, and the four cluster sums follow from those and the total
  float uall[2] = {0.0f, 0.0f};
#pragma unroll
  for (int sb = 0; sb < 2; ++sb)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 w4 = *reinterpret_cast<const f32x4*>(wtok + 32 * sb + 8 * g + 4 * hi);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) uall[tb] = fmaf(w4[i], P[sb][tb][4 * g + i], uall[tb]);
    }
#pragma unroll
  for (int tb = 0; tb < 2; ++tb) uall[tb] = sum_xor32(uall[tb]);
  float u[2][4], cw[4], r2m[4], nn[4];
  auto update = [&]() {  // u, cw, r2m, nn of the labels `lab`
    if (hi == 0) {
#pragma unroll
      for (int tb = 0; tb < 2; ++tb) {
        const float w = wt[tb];
        atok[32 * tb + lq] = f32x4{lab[tb] & 1 ? w : 0.0f, lab[tb] & 2 ? w : 0.0f, lab[tb] == 3 ? w : 0.0f, 0.0f};
      }
    }
    wave_lds_sync();
    float ub[2][3] = {{0.f, 0.f, 0.f}, {0.f, 0.f, 0.f}};  // sums over the tokens with label bit 0 / bit 1 / both
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const f32x4 a = atok[row_tok(sb, r)];
#pragma unroll
        for (int tb = 0; tb < 2; ++tb)
#pragma unroll
          for (int c = 0; c < 3; ++c) ub[tb][c] = fmaf(a[c], P[sb][tb][r], ub[tb][c]);
      }
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
#pragma unroll
      for (int c = 0; c < 3; ++c) ub[tb][c] = sum_xor32(ub[tb][c]);
      u[tb][3] = ub[tb][2];
      u[tb][1] = ub[tb][0] - ub[tb][2];
      u[tb][2] = ub[tb][1] - ub[tb][2];
      u[tb][0] = uall[tb] - ub[tb][0] - ub[tb][1] + ub[tb][2];
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float wsum = 0.0f, usum = 0.0f;
      if (hi == 0) {
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
          const float a = lab[tb] == c ? wt[tb] : 0.0f;
          wsum += a;
          usum = fmaf(a, u[tb][c], usum);
        }
      }
      cw[c] = wave_sum_dpp(wsum);
      const float rm = __builtin_amdgcn_rcpf(fmaxf(cw[c], 1e-6f));
      nn[c] = wave_sum_dpp(usum) * rm * rm;
      r2m[c] = 2.0f * rm;
    }
    wave_lds_sync();  // every lane has read atok before the next update rewrites it
  };
  update();
  for (int it = 0; it < iters; ++it) {
    int changed = 0;
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
      int best = 0;
      float bd = INFINITY;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float dc = cw[c] > 0.0f ? fmaf(-u[tb][c], r2m[c], nn[c]) : INFINITY;
        if (c == 0 || dc < bd) {  // first minimum, like argmin
          bd = dc;
          best = c;
        }
      }
      changed += __popcll(__builtin_amdgcn_ballot_w64(tv[tb] && best != lab[tb]) & 0xffffffffull);
      lab[tb] = best;
    }
    // converged, or the last round: the labels are final and the centroids of these labels are not needed
    if (changed == 0 || it == iters - 1) break;
    update();
  }

  // 4. cluster sums: S[c][d] = sum_t [lab_t == c] x[t][d] with one-hot bf16 (exact) times the tile on MFMA
  const unsigned long long vmask = nvalid >= 64 ? ~0ull : ((1ull << nvalid) - 1);
  const unsigned long long b0 = (__builtin_amdgcn_ballot_w64(lab[0] & 1) & 0xffffffffull) |
                                (__builtin_amdgcn_ballot_w64(lab[1] & 1) << 32);
  const unsigned long long b1 = (__builtin_amdgcn_ballot_w64(lab[0] & 2) & 0xffffffffull) |
                                (__builtin_amdgcn_ballot_w64(lab[1] & 2) << 32);
  unsigned long long member[4];
  member[0] = ~b0 & ~b1 & vmask;
  member[1] = b0 & ~b1 & vmask;
  member[2] = ~b0 & b1 & vmask;
  member[3] = b0 & b1 & vmask;
  float inv[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) inv[c] = 1.0f / fmaxf((float)__popcll(member[c]), 1.0f);
  // one-hot operand: lane (hi, lq) holds [lab_t == lq] for t = 16 ks + 8 hi + i (zero for lanes lq >= 4)
  bf16x8 oh[4];
  {
    const unsigned long long mine =
        (lq == 0 ? member[0] : lq == 1 ? member[1] : lq == 2 ? member[2] : lq == 3 ? member[3] : 0ull) >> (8 * hi);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int i = 0; i < 8; ++i) oh[ks][i] = ((mine >> (16 * ks + i)) & 1ull) ? (__bf16)1.0f : (__bf16)0.0f;
  }
  const size_t rep0 = (size_t)h * (NB + 1) * 4 + (size_t)j * 4;
  auto cluster_means = [&](bf16_t* out, const bf16x8 (*xt)[4]) {  // xt: transposed operands, or null: the tile
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      f32x16 s = {};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int base = 16 * ks + 8 * hi;
        s = mfma32(oh[ks], xt ? xt[db][ks] : cat_tr(tr4(tile, base, db), tr4(tile, base + 4, db)), s);
      }
      if (hi == 0) {  // rows 0..3 of the C tile are the four clusters
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const __bf16 b = (__bf16)(s[c] * inv[c]);
          out[(rep0 + c) * HD + 32 * db + lq] = __builtin_bit_cast(bf16_t, b);
        }
      }
    }
  };
  cluster_means(k4, kT);
  if (l < 4) {
    const int n = __popcll(member[l == 0 ? 0 : l == 1 ? 1 : l == 2 ? 2 : 3]);
    lc4[rep0 + l] = n > 0 ? log2f((float)n) : -INFINITY;
  }
  dma_wait();  // the V tile has arrived
  wave_lds_sync();
  cluster_means(v4, nullptr);
  if (MEANS) block_mean(vm);
}

static void run_representatives(const void* q, const void* k, const void* v, void* k_rep, void* v_rep,
                                float* log_counts, void* k_mean, void* v_mean, const RepWorkspace& w, int iters,
                                int L, int H, hipStream_t stream) {
  const int nb = (L + BK - 1) / BK;
  const float scale = 1.0f / sqrtf((float)HD);
  hipLaunchKernelGGL(gram_kernel, dim3(w.splits, H), dim3(256), 0, stream, (const bf16_t*)q, w.gram, L, H,
                     w.rows_per_split, w.splits);
  hipLaunchKernelGGL(gram_reduce_kernel, dim3(HD * HD / 256, H), dim3(256), 0, stream, w.gram, w.splits);
  hipLaunchKernelGGL(chol_kernel, dim3(H), dim3(CHOL_T), 0, stream, w.gram, w.metric_t, w.splits,
                     scale * scale / (float)L);
  hipLaunchKernelGGL(probe_kernel, dim3(NPROBE, H), dim3(64), 0, stream, (const bf16_t*)q, w.probes, L, H, nb,
                     scale);
  if (k_mean)
    hipLaunchKernelGGL(kmeans_kernel<true>, dim3((nb + KM_WAVES - 1) / KM_WAVES, H), dim3(64 * KM_WAVES), 0, stream, (const bf16_t*)k, (const bf16_t*)v,
                       w.metric_t, w.probes, (bf16_t*)k_rep, (bf16_t*)v_rep, log_counts, (bf16_t*)k_mean,
                       (bf16_t*)v_mean, L, H, nb, iters);
  else
    hipLaunchKernelGGL(kmeans_kernel<false>, dim3((nb + KM_WAVES - 1) / KM_WAVES, H), dim3(64 * KM_WAVES), 0, stream, (const bf16_t*)k,
                       (const bf16_t*)v, w.metric_t, w.probes, (bf16_t*)k_rep, (bf16_t*)v_rep, log_counts,
                       nullptr, nullptr, L, H, nb, iters);
}

static int check_representatives(const void* q, const void* k, const void* v, void* k_rep, void* v_rep,
                                 float* log_counts, void* k_mean, void* v_mean, int L, int H, int D) {
  ES_REQUIRE(q && k && v && k_rep && v_rep && log_counts, ES_ERR_INVALID, "null tensor pointer");
  ES_REQUIRE(L > 0 && H > 0, ES_ERR_INVALID, "L and H must be positive");
  ES_REQUIRE(D == HD, ES_ERR_UNSUPPORTED, "head dimension must be 128");
  ES_REQUIRE((k_mean == nullptr) == (v_mean == nullptr), ES_ERR_INVALID, "pass both k_mean and v_mean or neither");
  ES_REQUIRE((L + BK - 1) / BK >= NPROBE, ES_ERR_INVALID, "needs at least 64 kv blocks (4096 tokens)");
  return ES_OK;
}

// The allocation-free variant's workspace: one file-scope array, of which each GPU holds its own copy at its own
// address until the process ends. Host code never passes the array's name as a device address: the address is
// looked up once per device (with that device current) by hipGetSymbolAddress and kept in noalloc_base. Nothing
// in it has to start at zero (every kernel writes what it later reads), and calls that overlap on one GPU race on
// it.
constexpr size_t NOALLOC_SCRATCH_BYTES = size_t(48) << 20;
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

static void* noalloc_base() {
  static std::atomic<void*> base[64];
  static std::mutex init;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  void* p = base[dev].load();
  if (p) return p;
  std::lock_guard<std::mutex> g(init);
  if ((p = base[dev].load())) return p;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
  base[dev].store(p);
  return p;
}

}  // namespace es

using namespace es;

extern "C" size_t es_representatives_workspace(int L, int H, int D) {
  if (L <= 0 || H <= 0 || D != HD) return 0;
  return ws_bytes(L, H);
}

extern "C" int es_representatives(const void* q, const void* k, const void* v, void* k_rep, void* v_rep,
                                  float* log_counts, void* k_mean, void* v_mean, void* workspace,
                                  size_t workspace_bytes, int iters, int L, int H, int D, hipStream_t stream) {
  if (int st = check_representatives(q, k, v, k_rep, v_rep, log_counts, k_mean, v_mean, L, H, D)) return st;
  ES_REQUIRE(workspace, ES_ERR_INVALID, "null tensor pointer");
  ES_REQUIRE(workspace_bytes >= ws_bytes(L, H), ES_ERR_INVALID, "workspace too small");
  run_representatives(q, k, v, k_rep, v_rep, log_counts, k_mean, v_mean, carve(workspace, L, H), iters, L, H,
                      stream);
  return check_launch("es_representatives");
}

extern "C" size_t es_representatives_noalloc_limit(void) { return NOALLOC_SCRATCH_BYTES; }

extern "C" int es_representatives_noalloc(const void* q, const void* k, const void* v, void* k_rep, void* v_rep,
                                          float* log_counts, void* k_mean, void* v_mean, int iters, int L, int H,
                                          int D, hipStream_t stream) {
  if (int st = check_representatives(q, k, v, k_rep, v_rep, log_counts, k_mean, v_mean, L, H, D)) return st;
  ES_REQUIRE(ws_bytes(L, H) <= NOALLOC_SCRATCH_BYTES, ES_ERR_UNSUPPORTED,
             "es_representatives_noalloc: these L and H need more than the 48 MiB device scratch "
             "(es_representatives_workspace(L, H, D) bytes); use es_representatives with a caller workspace");
  void* base = noalloc_base();
  ES_REQUIRE(base, ES_ERR_LAUNCH, "es_representatives_noalloc: device scratch unavailable on this device");
  run_representatives(q, k, v, k_rep, v_rep, log_counts, k_mean, v_mean, carve(base, L, H), iters, L, H, stream);
  return check_launch("es_representatives_noalloc");
}
