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

__global__ __launch_bounds__(256) void chol_kernel(const float* __restrict__ gram, bf16_t* __restrict__ metric_t,
                                                   int splits, float gscale) {
  __shared__ float A[HD][HD + 1];
  __shared__ float col[HD];
  __shared__ float red[4];
  const int h = blockIdx.x, tid = threadIdx.x;
  for (int i = tid; i < HD * HD; i += 256) {
    float s = 0.0f;
    for (int sp = 0; sp < splits; ++sp) s += gram[((size_t)h * splits + sp) * HD * HD + i];
    A[i / HD][i % HD] = s * gscale;
  }
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
  for (int j = 0; j < HD; ++j) {
    if (tid < HD) {
      const float piv = fmaxf(A[j][j], eps);
      const float c = tid >= j ? A[tid][j] / sqrtf(piv) : 0.0f;
      col[tid] = c;
      mt[j * HD + tid] = f2bf(c);  // metric_t[e = j][d = tid] = Lchol[tid][j]
    }
    __syncthreads();
    for (int i = tid; i < HD * HD; i += 256) {
      const int r = i / HD, c = i % HD;
      if (r >= j && c >= j) A[r][c] -= col[r] * col[c];
    }
    __syncthreads();
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

template <bool MEANS>
__global__ __launch_bounds__(256) void kmeans_kernel(const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
                                                     const bf16_t* __restrict__ metric_t,
                                                     const bf16_t* __restrict__ probes, bf16_t* __restrict__ k4,
                                                     bf16_t* __restrict__ v4, float* __restrict__ lc4,
                                                     bf16_t* __restrict__ km, bf16_t* __restrict__ vm, int L, int H,
                                                     int NB, int iters) {
  __shared__ __attribute__((aligned(16))) char kt[BK * 256];
  __shared__ float X[BK][HD + 1];
  __shared__ float sp[NPROBE][BK + 1];
  __shared__ float wgt[BK];
  __shared__ float cen[4][HD];
  __shared__ float cw[4];
  __shared__ float dist[BK][4];
  __shared__ int lab[BK];
  __shared__ int red_i[4];
  __shared__ float cnt_s[4];

  const int j = blockIdx.x, h = blockIdx.y;
  const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, hi = l >> 5, lq = l & 31;
  const int nvalid = min(L - j * BK, BK);
  stage_rows(k, j * BK, L, H, h, kt);
  wait_vmem();
  __syncthreads();

  // X = K Lchol: wave wv -> tokens 32 (wv & 1) .., channels 64 (wv >> 1) .. (two 32-wide C tiles)
  {
    const int tb = wv & 1, e0 = (wv >> 1) * 2;
    f32x16 acc[2] = {f32x16{}, f32x16{}};
    const bf16_t* mt = metric_t + (size_t)h * HD * HD;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      const bf16x8 a = lds_read16(kt, tile_off(32 * tb + lq, 2 * ks + hi));
#pragma unroll
      for (int eb = 0; eb < 2; ++eb) {
        const bf16x8 b = *reinterpret_cast<const bf16x8*>(mt + (size_t)(32 * (e0 + eb) + lq) * HD + 16 * ks + 8 * hi);
        acc[eb] = mfma32(a, b, acc[eb]);
      }
    }
#pragma unroll
    for (int eb = 0; eb < 2; ++eb)
#pragma unroll
      for (int r = 0; r < 16; ++r) X[32 * tb + 8 * (r / 4) + 4 * hi + (r % 4)][32 * (e0 + eb) + lq] = acc[eb][r];
  }
  // probe logits: wave wv -> probes 32 (wv & 1) .., tokens 32 (wv >> 1) ..
  {
    const int pb = wv & 1, tb = wv >> 1;
    f32x16 acc = {};
    const bf16_t* pr = probes + ((size_t)h * NPROBE + 32 * pb + lq) * HD;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      const bf16x8 a = *reinterpret_cast<const bf16x8*>(pr + 16 * ks + 8 * hi);
      const bf16x8 b = lds_read16(kt, tile_off(32 * tb + lq, 2 * ks + hi));
      acc = mfma32(a, b, acc);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) sp[32 * pb + 8 * (r / 4) + 4 * hi + (r % 4)][32 * tb + lq] = acc[r];
  }
  __syncthreads();
  if (tid < NPROBE) {  // softmax of probe tid over the valid tokens (natural exponent)
    float m = -INFINITY;
    for (int t = 0; t < nvalid; ++t) m = fmaxf(m, sp[tid][t]);
    float s = 0.0f;
    for (int t = 0; t < nvalid; ++t) {
      const float e = expf(sp[tid][t] - m);
      sp[tid][t] = e;
      s += e;
    }
    const float inv = 1.0f / s;
    for (int t = 0; t < nvalid; ++t) sp[tid][t] *= inv;
  }
  __syncthreads();
  if (tid < BK) {
    float s = 0.0f;
    for (int p = 0; p < NPROBE; ++p) s += tid < nvalid ? sp[p][tid] : 0.0f;
    wgt[tid] = tid < nvalid ? s * ((float)nvalid / (float)NPROBE) : 0.0f;
    lab[tid] = tid / (BK / 4);
  }
  __syncthreads();

  // centroids of the current labels; cen keeps its old value for an empty (zero-weight) cluster unless `init`
  auto centroids = [&](bool init) {
    const int c = tid >> 6, e = 2 * (tid & 63);
    float s0 = 0.f, s1 = 0.f, ws = 0.f;
    for (int t = 0; t < nvalid; ++t) {
      if (lab[t] == c) {
        const float w = wgt[t];
        ws += w;
        s0 += w * X[t][e];
        s1 += w * X[t][e + 1];
      }
    }
    __syncthreads();
    const float d = fmaxf(ws, 1e-6f);
    if (init || ws > 0.0f) {
      cen[c][e] = s0 / d;
      cen[c][e + 1] = s1 / d;
    }
    if ((tid & 63) == 0) cw[c] = ws;
    __syncthreads();
  };
  centroids(true);
  for (int it = 0; it < iters; ++it) {
    {  // distances: thread (token tid & 63, cluster tid >> 6)
      const int t = tid & 63, c = tid >> 6;
      float cc = 0.f, xc = 0.f;
      for (int e = 0; e < HD; ++e) {
        const float z = cen[c][e];
        cc += z * z;
        xc += X[t][e] * z;
      }
      dist[t][c] = cw[c] > 0.0f ? cc - 2.0f * xc : INFINITY;
    }
    __syncthreads();
    int changed = 0;
    if (tid < BK) {
      int best = 0;
      float bd = dist[tid][0];
      for (int c = 1; c < 4; ++c)
        if (dist[tid][c] < bd) {
          bd = dist[tid][c];
          best = c;
        }
      changed = (tid < nvalid) && best != lab[tid];
      lab[tid] = best;
    }
    changed = wave_sum_i(changed);
    if (l == 0) red_i[wv] = changed;
    __syncthreads();
    const int total = red_i[0];
    centroids(false);
    if (total == 0) break;
  }

  // representatives: plain means of K and V over each cluster's valid tokens
  {
    const int c = tid >> 6, e = 2 * (tid & 63);
    float k0 = 0.f, k1 = 0.f, v0 = 0.f, v1 = 0.f;
    int n = 0;
    for (int t = 0; t < nvalid; ++t) {
      if (lab[t] != c) continue;
      ++n;
      const unsigned kw = *reinterpret_cast<const unsigned*>(kt + tile_off(t, e / 8) + (e % 8) * 2);
      const unsigned vw = *reinterpret_cast<const unsigned*>(v + ((size_t)(j * BK + t) * H + h) * HD + e);
      k0 += __uint_as_float(kw << 16);
      k1 += __uint_as_float(kw & 0xffff0000u);
      v0 += __uint_as_float(vw << 16);
      v1 += __uint_as_float(vw & 0xffff0000u);
    }
    const float inv = 1.0f / fmaxf((float)n, 1.0f);
    const size_t o = ((size_t)h * (NB + 1) * 4 + (size_t)j * 4 + c) * HD + e;
    k4[o] = f2bf(k0 * inv);
    k4[o + 1] = f2bf(k1 * inv);
    v4[o] = f2bf(v0 * inv);
    v4[o + 1] = f2bf(v1 * inv);
    if ((tid & 63) == 0) lc4[(size_t)h * (NB + 1) * 4 + (size_t)j * 4 + c] = n > 0 ? log2f((float)n) : -INFINITY;
  }
  if (MEANS && tid < 128) {  // block means, same arithmetic as means_kernel
    const bf16_t* src = tid < 64 ? k : v;
    bf16_t* dst = tid < 64 ? km : vm;
    const int e = 2 * (tid & 63);
    float a = 0.f, b = 0.f;
    for (int r = 0; r < nvalid; ++r) {
      const unsigned w = *reinterpret_cast<const unsigned*>(src + ((size_t)(j * BK + r) * H + h) * HD + e);
      a += __uint_as_float(w << 16);
      b += __uint_as_float(w & 0xffff0000u);
    }
    const float n = (float)nvalid;
    const size_t o = ((size_t)j * H + h) * HD + e;
    dst[o] = f2bf(a / n);
    dst[o + 1] = f2bf(b / n);
  }
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
  ES_REQUIRE(q && k && v && k_rep && v_rep && log_counts && workspace, ES_ERR_INVALID, "null tensor pointer");
  ES_REQUIRE(L > 0 && H > 0, ES_ERR_INVALID, "L and H must be positive");
  ES_REQUIRE(D == HD, ES_ERR_UNSUPPORTED, "head dimension must be 128");
  ES_REQUIRE((k_mean == nullptr) == (v_mean == nullptr), ES_ERR_INVALID, "pass both k_mean and v_mean or neither");
  const int nb = (L + BK - 1) / BK;
  ES_REQUIRE(nb >= NPROBE, ES_ERR_INVALID, "needs at least 64 kv blocks (4096 tokens)");
  ES_REQUIRE(workspace_bytes >= ws_bytes(L, H), ES_ERR_INVALID, "workspace too small");
  RepWorkspace w = carve(workspace, L, H);
  const float scale = 1.0f / sqrtf((float)HD);
  hipLaunchKernelGGL(gram_kernel, dim3(w.splits, H), dim3(256), 0, stream, (const bf16_t*)q, w.gram, L, H,
                     w.rows_per_split, w.splits);
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
  return check_launch("es_representatives");
}
