// Four representatives per 64-token kv block, clustered in the query metric (reference
// echosparse/kernels/representatives.py:1-166).
//
//   gram_kernel    partial Gram matrices sum_rows q q^T per (head, row split), bf16 MFMA, fp32; written to the
//                  workspace and reduced in a fixed order (deterministic, unlike the reference's atomics)
//   chol_kernel    G = Gram * scale^2 / L + 1e-3 * mean(diag) * I; right-looking Cholesky in LDS with the pivot
//                  clamped at trace/D * 1e-12; writes the factor transposed (metric_t[e][d] = Lchol[d][e]), bf16
//   probe_kernel   64 probe queries: scale * mean of the valid q rows of block round(i * (nb - 1) / 63)
//   kmeans_kernel  per (block, head): X = K Lchol (MFMA), probe softmax weights (MFMA + LDS), weighted Lloyd from
//                  the four contiguous 16-token groups with early exit, plain K / V means per cluster and log2
//                  cluster sizes (-inf if empty); optionally the block means
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

__global__ __launch_bounds__(256) void gram_kernel(const bf16_t* __restrict__ q, float* __restrict__ gram, int L,
                                                   int H, int rps, int splits) {
  __shared__ __attribute__((aligned(16))) char tile[BK * 256];
  const int s = blockIdx.x, h = blockIdx.y;
  const int wv = threadIdx.x >> 6, l = threadIdx.x & 63, hi = l >> 5, lq = l & 31;
  f32x16 acc[4] = {f32x16{}, f32x16{}, f32x16{}, f32x16{}};
  const int r_end = min(L, (s + 1) * rps);
  for (int r0 = s * rps; r0 < r_end; r0 += BK) {
    __syncthreads();
    stage_rows(q, r0, L, H, h, tile);
    wait_vmem();
    __syncthreads();
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
  for (int sp = 0; sp < splits; ++sp) s += g[(size_t)sp * HD * HD];
  g[0] = s;
}

__global__ __launch_bounds__(256) void chol_kernel(const float* __restrict__ gram, bf16_t* __restrict__ metric_t,
                                                   int splits, float gscale) {
  __shared__ float A[HD][HD + 1];
  __shared__ float red[4];
  const int h = blockIdx.x, tid = threadIdx.x;
  // the split partials were summed into split 0 by gram_reduce_kernel
  for (int i = tid; i < HD * HD; i += 256) A[i / HD][i % HD] = gram[(size_t)h * splits * HD * HD + i] * gscale;
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
  // Register-resident right-looking factorisation: thread (cc = tid % 128, half = tid / 128) holds column cc at
  // rows 64 half .. 64 half + 63. Step j: the owners of column j publish it into column buffer j % 2 (16-byte
  // LDS writes), one barrier, then every thread reads the pivot column with 16-byte broadcast reads and subtracts
  // the rank-1 update from its own entries. (Two buffers: step j+1 writes the other one while step j's readers
  // may still be reading.)
  const int cc = tid & (HD - 1), rb = 64 * (tid >> 7);
  float a[64];
#pragma unroll
  for (int i = 0; i < 64; ++i) a[i] = A[rb + i][cc];
  __syncthreads();
  float* colbuf = &A[0][0];  // the matrix now lives in registers; reuse the LDS as two column buffers
  for (int j = 0; j < HD; ++j) {
    float* cb = colbuf + (j & 1) * HD;
    if (cc == j) {
#pragma unroll
      for (int q4 = 0; q4 < 16; ++q4)
        *reinterpret_cast<f32x4*>(cb + rb + 4 * q4) = f32x4{a[4 * q4], a[4 * q4 + 1], a[4 * q4 + 2], a[4 * q4 + 3]};
    }
    __syncthreads();
    const float inv = 1.0f / sqrtf(fmaxf(cb[j], eps));
    const float cv = cc >= j ? cb[cc] * inv : 0.0f;
    if (tid < HD) mt[j * HD + tid] = f2bf(tid >= j ? cb[tid] * inv : 0.0f);  // metric_t[j][d] = Lchol[d][j]
#pragma unroll
    for (int q4 = 0; q4 < 16; ++q4) {
      const f32x4 c4 = *reinterpret_cast<const f32x4*>(cb + rb + 4 * q4);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int r = rb + 4 * q4 + k;
        const float cr = r >= j ? c4[k] * inv : 0.0f;
        a[4 * q4 + k] = fmaf(-cr, cv, a[4 * q4 + k]);
      }
    }
  }
}

__global__ __launch_bounds__(64) void probe_kernel(const bf16_t* __restrict__ q, bf16_t* __restrict__ probes, int L,
                                                   int H, int NB, float scale) {
  const int i = blockIdx.x, h = blockIdx.y, l = threadIdx.x;
  const int blk = (int)((float)(i * (NB - 1)) / (float)(NPROBE - 1) + 0.5f);
  const int r0 = blk * BK, n = max(min(L - r0, BK), 0);
  float a = 0.f, b = 0.f;
  for (int r = 0; r < n; ++r) {
    const unsigned w = *reinterpret_cast<const unsigned*>(q + ((size_t)(r0 + r) * H + h) * HD + 2 * l);
    a += __uint_as_float(w << 16);
    b += __uint_as_float(w & 0xffff0000u);
  }
  const float d = fmaxf((float)n, 1.0f);
  bf16_t* p = probes + ((size_t)h * NPROBE + i) * HD + 2 * l;
  p[0] = f2bf(a * scale / d);
  p[1] = f2bf(b * scale / d);
}

// kmeans_kernel: one (block, head) per 256-thread workgroup; under 40 KB of LDS so four workgroups share a CU.
//   LDS region A (33 KB): the K tile, then the probe logits, then X (fp32, padded rows), then the K and V tiles
//                         for the final means (X waits in registers while the probe softmax reads the logits)
//   LDS region B (7 KB):  the softmax partials, then the dot partials / centroids / weights
// Thread (wave w, lane l) keeps X[l][32 w ..] in registers for the distances; the centroid sums (threads 0..127,
// channel = tid) read X's columns from LDS.
template <bool MEANS>
__global__ __launch_bounds__(256, 4) void kmeans_kernel(const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
                                                        const bf16_t* __restrict__ metric_t,
                                                        const bf16_t* __restrict__ probes, bf16_t* __restrict__ k4,
                                                        bf16_t* __restrict__ v4, float* __restrict__ lc4,
                                                        bf16_t* __restrict__ km, bf16_t* __restrict__ vm, int L,
                                                        int H, int NB, int iters) {
  __shared__ __attribute__((aligned(16))) float regA[BK * (HD + 1)];
  __shared__ __attribute__((aligned(16))) float regB[(4 * BK + HD + BK) * 4];
  __shared__ float wgt[BK];
  __shared__ int lab[BK];
  __shared__ float cw[4];
  __shared__ float nnp[2][4];
  __shared__ int red_i[1];
  float(*X)[HD + 1] = reinterpret_cast<float(*)[HD + 1]>(regA);
  char* kt2 = reinterpret_cast<char*>(regA);  // K tile for the means (after the clustering)
  char* vt2 = kt2 + BK * 256;                 // V tile for the means
  char* kt = reinterpret_cast<char*>(regA);   // K tile for X and the probe logits
  float(*sp)[BK + 1] = reinterpret_cast<float(*)[BK + 1]>(regA);
  float(*wpart)[BK] = reinterpret_cast<float(*)[BK]>(regB);  // softmax partials [4][BK]
  float* pmax = regB + 4 * BK;
  float* pinv = pmax + NPROBE;
  f32x4* part = reinterpret_cast<f32x4*>(regB);            // [4 waves][BK] partial dots
  f32x4* cen = reinterpret_cast<f32x4*>(regB) + 4 * BK;    // [HD] centroids, (channel, cluster)
  f32x4* aw = reinterpret_cast<f32x4*>(regB) + 4 * BK + HD;  // [BK] token weight per cluster

  const int j = blockIdx.x, h = blockIdx.y;
  const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, hi = l >> 5, lq = l & 31;
  const int nvalid = min(L - j * BK, BK);
  // the metric operands do not depend on the K tile: their loads are issued first, so that their latency
  // overlaps the tile's staging instead of following it (the first half of them: registers)
  const int tb = wv & 1, e0 = (wv >> 1) * 2, pb = wv & 1, tk = wv >> 1;
  const bf16_t* mt = metric_t + (size_t)h * HD * HD;
  bf16x8 mop[4][2];
  {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int eb = 0; eb < 2; ++eb)
        mop[ks][eb] = *reinterpret_cast<const bf16x8*>(mt + (size_t)(32 * (e0 + eb) + lq) * HD + 16 * ks + 8 * hi);
  }
  stage_rows(k, j * BK, L, H, h, kt);
  wait_vmem();
  __syncthreads();

  // X = K Lchol: wave wv -> tokens 32 (wv & 1) .., channels 64 (wv >> 1) .. (two 32-wide C tiles); probe logits:
  // wave wv -> probes 32 (wv & 1) .., tokens 32 (wv >> 1) ..
  f32x16 ax[2] = {f32x16{}, f32x16{}}, ap = {};
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    const bf16x8 a = lds_read16(kt, tile_off(32 * tb + lq, 2 * ks + hi));
#pragma unroll
    for (int eb = 0; eb < 2; ++eb)
      ax[eb] = mfma32(a, ks < 4 ? mop[ks & 3][eb]
                                : *reinterpret_cast<const bf16x8*>(mt + (size_t)(32 * (e0 + eb) + lq) * HD + 16 * ks + 8 * hi),
                      ax[eb]);
  }
  const bf16_t* pr = probes + ((size_t)h * NPROBE + 32 * pb + lq) * HD;
#pragma unroll
  for (int ks = 0; ks < 8; ++ks)
    ap = mfma32(*reinterpret_cast<const bf16x8*>(pr + 16 * ks + 8 * hi), lds_read16(kt, tile_off(32 * tk + lq, 2 * ks + hi)),
                ap);
  __syncthreads();  // every wave is done with the K tile: region A takes the probe logits
  {
    const int pb = wv & 1, tk = wv >> 1;
#pragma unroll
    for (int r = 0; r < 16; ++r) sp[32 * pb + 8 * (r / 4) + 4 * hi + (r % 4)][32 * tk + lq] = ap[r];
  }
  __syncthreads();

  // probe softmax weights w_t = sum_p softmax_p(t). (a) thread (probe tid % 64, token quarter tid / 64): row max
  // and row sum over its 16 tokens, combined through LDS; (b) wave wv, lane = token: its 16 probes. Plain loops
  // and LDS instead of one cross-lane reduction per probe.
  {
    const int pp = tid & 63, q4 = tid >> 6;
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int tk = 16 * q4 + i;
      mx = fmaxf(mx, tk < nvalid ? sp[pp][tk] : -INFINITY);
    }
    wpart[q4][pp] = mx;
    __syncthreads();
    const float m = fmaxf(fmaxf(wpart[0][pp], wpart[1][pp]), fmaxf(wpart[2][pp], wpart[3][pp]));
    float sm = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int tk = 16 * q4 + i;
      sm += tk < nvalid ? exp2f_fast((sp[pp][tk] - m) * LOG2E) : 0.0f;
    }
    __syncthreads();  // the maxima are read
    wpart[q4][pp] = sm;
    __syncthreads();
    if (tid < NPROBE) {
      pmax[tid] = m;
      pinv[tid] = 1.0f / (wpart[0][tid] + wpart[1][tid] + wpart[2][tid] + wpart[3][tid]);
    }
    __syncthreads();
    float wsum = 0.0f;
    if (l < nvalid) {
#pragma unroll 4
      for (int p = 16 * wv; p < 16 * wv + 16; ++p) wsum = fmaf(exp2f_fast((sp[p][l] - pmax[p]) * LOG2E), pinv[p], wsum);
    }
    wpart[wv][l] = wsum;  // (every read of wpart above precedes the last barrier)
  }
  __syncthreads();  // the probe logits are consumed: region A takes X
  {
    const int tb = wv & 1, e0 = (wv >> 1) * 2;
#pragma unroll
    for (int eb = 0; eb < 2; ++eb)
#pragma unroll
      for (int r = 0; r < 16; ++r) X[32 * tb + 8 * (r / 4) + 4 * hi + (r % 4)][32 * (e0 + eb) + lq] = ax[eb][r];
  }
  // token weights and the initial labels (four contiguous 16-token groups); the per-cluster weights cw are
  // summed by the centroid pass
  auto set_weights = [&](int lb) {  // wave 0, lane = token: aw and lab of the labels lb
    const float w = wgt[l];
    f32x4 a4;
#pragma unroll
    for (int c = 0; c < 4; ++c) a4[c] = lb == c ? w : 0.0f;
    aw[l] = a4;
    lab[l] = lb;
  };
  if (wv == 0) {
    const float s = wpart[0][l] + wpart[1][l] + wpart[2][l] + wpart[3][l];
    wgt[l] = l < nvalid ? s * ((float)nvalid / (float)NPROBE) : 0.0f;
    set_weights(l / (BK / 4));
  }
  __syncthreads();
  float xd[32];  // X[l][32 wv + i]
#pragma unroll
  for (int i = 0; i < 32; ++i) xd[i] = X[l][32 * wv + i];

  // weighted centroids of the current labels and the cluster weights cw: thread (channel tid % 128, token half
  // tid / 128) sums its 32 tokens, the second halves are added through LDS (`part`, free at this point); a cluster
  // with zero weight keeps its previous centroid unless `init`; also the squared centroid norms (per wave, nnp).
  // Every thread of the workgroup calls it (it holds a barrier).
  auto centroids = [&](bool init) {
    const int ch = tid & (HD - 1), hh = tid >> 7;
    float s[4] = {0.f, 0.f, 0.f, 0.f}, ws[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
    for (int t = 32 * hh; t < 32 * hh + 32; ++t) {
      const f32x4 a4 = aw[t];
      const float x = X[t][ch];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        s[c] = fmaf(a4[c], x, s[c]);
        ws[c] += a4[c];
      }
    }
    if (hh == 1) {
      part[ch] = f32x4{s[0], s[1], s[2], s[3]};
      part[HD + ch] = f32x4{ws[0], ws[1], ws[2], ws[3]};
    }
    __syncthreads();
    if (hh == 1) return;
    const f32x4 s1 = part[ch], w1 = part[HD + ch];
    f32x4 c4 = init ? f32x4{} : cen[ch];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float w = ws[c] + w1[c];
      if (init || w > 0.0f) c4[c] = (s[c] + s1[c]) / fmaxf(w, 1e-6f);
      if (ch == 0) cw[c] = w;
    }
    cen[ch] = c4;
    float q[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) q[c] = wave_sum_dpp(c4[c] * c4[c]);
    if (l == 0) {
#pragma unroll
      for (int c = 0; c < 4; ++c) nnp[wv][c] = q[c];
    }
  };
  centroids(true);
  __syncthreads();
  for (int it = 0; it < iters; ++it) {
    {  // partial dots over channels 32 wv .. 32 wv + 31 for token l
      float d[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        const f32x4 c4 = cen[32 * wv + i];
#pragma unroll
        for (int c = 0; c < 4; ++c) d[c] = fmaf(xd[i], c4[c], d[c]);
      }
      part[wv * BK + l] = f32x4{d[0], d[1], d[2], d[3]};
    }
    __syncthreads();
    if (wv == 0) {
      const f32x4 p0 = part[l], p1 = part[BK + l], p2 = part[2 * BK + l], p3 = part[3 * BK + l];
      int best = 0;
      float bd = INFINITY;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float xcd = p0[c] + p1[c] + p2[c] + p3[c];
        const float nn = nnp[0][c] + nnp[1][c];
        const float dc = cw[c] > 0.0f ? nn - 2.0f * xcd : INFINITY;
        if (c == 0 || dc < bd) {  // first minimum, like argmin
          bd = dc;
          best = c;
        }
      }
      const int changed = __popcll(__builtin_amdgcn_ballot_w64((l < nvalid) && best != lab[l]));
      set_weights(best);
      if (l == 0) red_i[0] = changed;
    }
    __syncthreads();
    // converged, or the last round: the labels are final and the representatives are plain means over them, so
    // the centroids of these labels are not needed
    if (red_i[0] == 0 || it == iters - 1) break;
    centroids(false);
    __syncthreads();
  }

  // representatives: plain means of K and V over each cluster's valid tokens (both tiles in LDS, region A)
  stage_rows(k, j * BK, L, H, h, kt2);
  stage_rows(v, j * BK, L, H, h, vt2);
  wait_vmem();
  __syncthreads();
  {
    const int c = tid >> 6, e = 2 * (tid & 63);
    float k0 = 0.f, k1 = 0.f, v0 = 0.f, v1 = 0.f;
    int n = 0;
#pragma unroll 4
    for (int t = 0; t < nvalid; ++t) {
      const int off = tile_off(t, e / 8) + (e % 8) * 2;
      const unsigned kw = *reinterpret_cast<const unsigned*>(kt2 + off);
      const unsigned vw = *reinterpret_cast<const unsigned*>(vt2 + off);
      const float m = lab[t] == c ? 1.0f : 0.0f;
      n += lab[t] == c;
      k0 = fmaf(m, __uint_as_float(kw << 16), k0);
      k1 = fmaf(m, __uint_as_float(kw & 0xffff0000u), k1);
      v0 = fmaf(m, __uint_as_float(vw << 16), v0);
      v1 = fmaf(m, __uint_as_float(vw & 0xffff0000u), v1);
    }
    const float inv = 1.0f / fmaxf((float)n, 1.0f);
    const size_t o = ((size_t)h * (NB + 1) * 4 + (size_t)j * 4 + c) * HD + e;
    k4[o] = f2bf(k0 * inv);
    k4[o + 1] = f2bf(k1 * inv);
    v4[o] = f2bf(v0 * inv);
    v4[o + 1] = f2bf(v1 * inv);
    if ((tid & 63) == 0) lc4[(size_t)h * (NB + 1) * 4 + (size_t)j * 4 + c] = n > 0 ? log2f((float)n) : -INFINITY;
  }
  if (MEANS && tid < 128) {  // block means: the same sequential fp32 sum and division as means_kernel
    const char* src = tid < 64 ? kt2 : vt2;
    bf16_t* dst = tid < 64 ? km : vm;
    const int e = 2 * (tid & 63);
    float a = 0.f, b = 0.f;
#pragma unroll 4
    for (int r = 0; r < nvalid; ++r) {
      const unsigned w = *reinterpret_cast<const unsigned*>(src + tile_off(r, e / 8) + (e % 8) * 2);
      a += __uint_as_float(w << 16);
      b += __uint_as_float(w & 0xffff0000u);
    }
    const float n = (float)nvalid;
    const size_t o = ((size_t)j * H + h) * HD + e;
    dst[o] = f2bf(a / n);
    dst[o + 1] = f2bf(b / n);
  }
}

static void run_representatives(const void* q, const void* k, const void* v, void* k_rep, void* v_rep,
                                float* log_counts, void* k_mean, void* v_mean, const RepWorkspace& w, int iters,
                                int L, int H, hipStream_t stream) {
  const int nb = (L + BK - 1) / BK;
  const float scale = 1.0f / sqrtf((float)HD);
  hipLaunchKernelGGL(gram_kernel, dim3(w.splits, H), dim3(256), 0, stream, (const bf16_t*)q, w.gram, L, H,
                     w.rows_per_split, w.splits);
  hipLaunchKernelGGL(gram_reduce_kernel, dim3(HD * HD / 256, H), dim3(256), 0, stream, w.gram, w.splits);
  hipLaunchKernelGGL(chol_kernel, dim3(H), dim3(256), 0, stream, w.gram, w.metric_t, w.splits,
                     scale * scale / (float)L);
  hipLaunchKernelGGL(probe_kernel, dim3(NPROBE, H), dim3(64), 0, stream, (const bf16_t*)q, w.probes, L, H, nb,
                     scale);
  if (k_mean)
    hipLaunchKernelGGL(kmeans_kernel<true>, dim3(nb, H), dim3(256), 0, stream, (const bf16_t*)k, (const bf16_t*)v,
                       w.metric_t, w.probes, (bf16_t*)k_rep, (bf16_t*)v_rep, log_counts, (bf16_t*)k_mean,
                       (bf16_t*)v_mean, L, H, nb, iters);
  else
    hipLaunchKernelGGL(kmeans_kernel<false>, dim3(nb, H), dim3(256), 0, stream, (const bf16_t*)k,
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
