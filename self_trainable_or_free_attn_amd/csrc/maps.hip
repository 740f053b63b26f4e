// Block means and the block-mass estimates of skipped blocks.
//
//   means_kernel     reference echosparse/kernels/triton_ops.py:21-40 (block_means)
//   estimate_kernel  reference echosparse/kernels/triton_ops.py:122-177 (estimate_skipped; sm120.py:183-250 is the
//                    same computation four tiles per program, as here)
#include "../../include/echosparse_hip.h"
#include "common.h"

namespace es {

// one wave per (block, head); lane owns two channels; fp32 sum over the block's valid tokens, one rounding
__global__ __launch_bounds__(64) void means_kernel(const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
                                                   bf16_t* __restrict__ km, bf16_t* __restrict__ vm, int L, int H) {
  const int j = blockIdx.x, h = blockIdx.y, l = threadIdx.x;
  const int n = min(L - j * BK, BK);
  float k0 = 0.f, k1 = 0.f, v0 = 0.f, v1 = 0.f;
#pragma unroll 8
  for (int r = 0; r < n; ++r) {  // (eight rows' loads in flight together; the sums take the rows in order)
    const size_t o = ((size_t)(j * BK + r) * H + h) * HD + 2 * l;
    const unsigned kw = *reinterpret_cast<const unsigned*>(k + o);
    const unsigned vw = *reinterpret_cast<const unsigned*>(v + o);
    k0 += __uint_as_float(kw << 16);
    k1 += __uint_as_float(kw & 0xffff0000u);
    v0 += __uint_as_float(vw << 16);
    v1 += __uint_as_float(vw & 0xffff0000u);
  }
  const float inv = (float)n;
  const size_t o = ((size_t)j * H + h) * HD + 2 * l;
  km[o] = f2bf(k0 / inv);
  km[o + 1] = f2bf(k1 / inv);
  vm[o] = f2bf(v0 / inv);
  vm[o + 1] = f2bf(v1 / inv);
}

// Sixteen query tiles per workgroup, one head; each wave owns four of them: 4 x 16 sampled rows (rows t*128 + 8i)
// = 64 queries, and walks every 32-key chunk of the block means: S = Q Kmean^T with Q as the A operand (two 32-row
// M tiles) and the key chunk as the B operand read straight from global memory, one chunk ahead. The waves are
// independent (no barrier): a wave's four tiles get their sums, their map entries and their scales from it alone.
__global__ __launch_bounds__(256) void estimate_kernel(const bf16_t* __restrict__ q, const bf16_t* __restrict__ km,
                                                       const uint8_t* __restrict__ keep,
                                                       const float* __restrict__ m_prev,
                                                       const float* __restrict__ m_new, float* __restrict__ map,
                                                       float* __restrict__ scale_exact,
                                                       float* __restrict__ scale_skip, int L, int H, int nq, int NB,
                                                       float scale, float lb_last) {
  const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, hi = l >> 5, lq = l & 31;
  const int t0 = blockIdx.x * 16 + wv * 4, h = blockIdx.y;
  if (t0 >= nq) return;

  // A operands: query qi = 32*mb + lq, tile t0 + qi/16, sample qi%16
  bf16x8 qa[2][8];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
    const int qi = 32 * mb + lq;
    const int tt = t0 + qi / 16, row = tt * BM + (qi % 16) * (BM / 16);
    const bool ok = tt < nq && row < L;
    const bf16_t* qr = q + ((size_t)(ok ? row : 0) * H + h) * HD;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      bf16x8 z = {};
      qa[mb][ks] = ok ? *reinterpret_cast<const bf16x8*>(qr + 16 * ks + 8 * hi) : z;
    }
  }
  // -prior of the C rows this lane holds (row index 8i + 4hi + jj of M tile mb); -inf for invalid rows
  float nms[2][16];
  int nsv[4];
#pragma unroll
  for (int tl = 0; tl < 4; ++tl) {
    const int tt = t0 + tl;
    int c = 0;
    for (int s = 0; s < 16; ++s) c += (tt < nq && tt * BM + s * 8 < L);
    nsv[tl] = c;
  }
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qi = 32 * mb + 8 * (r / 4) + 4 * hi + (r % 4);
      const int tt = t0 + qi / 16, row = tt * BM + (qi % 16) * (BM / 16);
      nms[mb][r] = (tt < nq && row < L) ? -m_prev[(size_t)row * H + h] : -INFINITY;
    }

  float num[4] = {0.f, 0.f, 0.f, 0.f}, den[4] = {0.f, 0.f, 0.f, 0.f};
  const int nchunks = (NB + 31) / 32;
  // B operands (the chunk's 32 block means) are fetched one chunk ahead of the MFMAs that use them
  auto load_b = [&](int c, bf16x8 (&b)[8]) {
    const int key = c * 32 + lq;
    const bf16_t* kr = km + ((size_t)(key < NB ? key : 0) * H + h) * HD;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) b[ks] = *reinterpret_cast<const bf16x8*>(kr + 16 * ks + 8 * hi);
  };
  bf16x8 bn[8];
  load_b(0, bn);
  for (int c = 0; c < nchunks; ++c) {
    const int key = c * 32 + lq;
    const bool kvalid = key < NB;
    bf16x8 bc[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) bc[ks] = bn[ks];
    // this chunk's keep flags and current map values, loaded before the products so that their latency is spent
    // under them (the map holds the exact blocks' masses from the attention, read for the kept blocks), and before
    // the next chunk's operands, so that waiting for them leaves those in flight
    uint8_t kp[4] = {1, 1, 1, 1};
    float mv[4] = {0.f, 0.f, 0.f, 0.f};
    if (hi == 0 && kvalid) {
#pragma unroll
      for (int tl = 0; tl < 4; ++tl) {
        if (t0 + tl >= nq) continue;
        const size_t o = ((size_t)h * nq + t0 + tl) * NB + key;
        kp[tl] = keep[o];
        mv[tl] = map[o];
      }
    }
    if (c + 1 < nchunks) load_b(c + 1, bn);
    f32x16 acc[2] = {f32x16{}, f32x16{}};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      acc[0] = mfma32(qa[0][ks], bc[ks], acc[0]);
      acc[1] = mfma32(qa[1][ks], bc[ks], acc[1]);
    }
    const float lb = key == NB - 1 ? lb_last : 6.0f;
    float est[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float x = fminf(acc[mb][r] * scale + nms[mb][r] + lb, 100.0f);
        est[2 * mb + (r / 8)] += exp2f_fast(x);
      }
#pragma unroll
    for (int tl = 0; tl < 4; ++tl) est[tl] = sum_xor32(est[tl]);
    if (hi == 0 && kvalid) {
#pragma unroll
      for (int tl = 0; tl < 4; ++tl) {
        const int tt = t0 + tl;
        if (tt >= nq) continue;
        const float e = est[tl] / fmaxf((float)nsv[tl], 1.0f);
        const size_t o = ((size_t)h * nq + tt) * NB + key;
        if (kp[tl] == 0) {
          map[o] = e;
        } else {
          num[tl] += mv[tl];
          den[tl] += e;
        }
      }
    }
  }
  // the wave's four tiles: f over each tile's rows, then the scales
#pragma unroll
  for (int tl = 0; tl < 4; ++tl) {
    const float sn = wave_sum(num[tl]), sd = wave_sum(den[tl]);
    const int tt = t0 + tl;
    if (tt >= nq) break;
    const int nrows = min(L - tt * BM, BM);
    float f = 0.0f;
    for (int r = l; r < BM; r += 64) {
      const int row = tt * BM + r;
      if (row < L) {
        const size_t o = (size_t)row * H + h;
        f += exp2f(fminf(fmaxf(m_prev[o] - m_new[o], -100.0f), 100.0f));
      }
    }
    f = wave_sum(f) / (float)nrows;
    if (l == 0) {
      const float nn = sn / (float)nrows;
      const float c = sd > 0.0f ? fminf(fmaxf(nn / fmaxf(sd, 1e-30f), 1.0f), 64.0f) : 1.0f;
      scale_exact[h * nq + tt] = f / (float)nrows;
      scale_skip[h * nq + tt] = f * c;
    }
  }
}

}  // namespace es

using namespace es;

extern "C" int es_block_means(const void* k, const void* v, void* k_mean, void* v_mean, int L, int H, int D,
                              hipStream_t stream) {
  ES_REQUIRE(k && v && k_mean && v_mean, ES_ERR_INVALID, "null tensor pointer");
  ES_REQUIRE(L > 0 && H > 0, ES_ERR_INVALID, "L and H must be positive");
  ES_REQUIRE(D == HD, ES_ERR_UNSUPPORTED, "head dimension must be 128");
  const int nb = (L + BK - 1) / BK;
  hipLaunchKernelGGL(means_kernel, dim3(nb, H), dim3(64), 0, stream, (const bf16_t*)k, (const bf16_t*)v,
                     (bf16_t*)k_mean, (bf16_t*)v_mean, L, H);
  return check_launch("es_block_means");
}

extern "C" int es_estimate_skipped(const void* q, const void* k_mean, const uint8_t* keep, const float* offset,
                                   const float* lse, float* mass, float* scale_exact, float* scale_skip, int L,
                                   int H, int D, hipStream_t stream) {
  ES_REQUIRE(q && k_mean && keep && offset && lse && mass && scale_exact && scale_skip, ES_ERR_INVALID,
             "null tensor pointer");
  ES_REQUIRE(L > 0 && H > 0, ES_ERR_INVALID, "L and H must be positive");
  ES_REQUIRE(D == HD, ES_ERR_UNSUPPORTED, "head dimension must be 128");
  const int nq = (L + BM - 1) / BM, nb = (L + BK - 1) / BK;
  const float scale = LOG2E / sqrtf((float)HD);
  const float lb_last = log2f((float)(L - (nb - 1) * BK));
  hipLaunchKernelGGL(estimate_kernel, dim3((nq + 15) / 16, H), dim3(256), 0, stream, (const bf16_t*)q,
                     (const bf16_t*)k_mean, keep, offset, lse, mass, scale_exact, scale_skip, L, H, nq, nb, scale,
                     lb_last);
  return check_launch("es_estimate_skipped");
}
