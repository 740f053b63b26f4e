// Block selection and the bit plans (bit-exact integer work on float32 bit patterns).
//
//   select_kernel   reference echosparse/kernels/triton_ops.py:43-119 (select_blocks, _kth_largest)
//   pack_kernel     reference echosparse/kernels/sm120.py:258-273 (pack_plan)
//   rebuild_kernel  reference echosparse/kernels/sm120.py:276-305 (rebuild_plan)
//   scales_kernel   reference echosparse/kernels/triton_ops.py:180-199 (full_step_scales)
//
// The K-th largest value is the one the reference's bisection returns: the largest int32 x in [0, 0x7F800001)
// with count(bits >= x) >= K. Values are non-negative floats (padding -1.0), which order like their bit
// patterns. Here the count runs over the workgroup with wave-level popcounts and one LDS exchange per step.
#include "../../include/echosparse_hip.h"
#include "common.h"

namespace es {

constexpr int SEL_THREADS = 256;
constexpr int SEL_MAXE = 16;  // elements per thread: next_pow2(nb) <= 4096

// exclusive prefix over the workgroup of one int per thread; returns (prefix, total)
__device__ __forceinline__ int2 block_scan(int x, int* scan_s) {
  const int l = threadIdx.x & 63, wv = threadIdx.x >> 6;
  int inc = x;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    int y = __shfl_up(inc, d, 64);
    if (l >= d) inc += y;
  }
  if (l == 63) scan_s[wv] = inc;
  __syncthreads();
  int before = 0, total = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int v = scan_s[i];
    before += i < wv ? v : 0;
    total += v;
  }
  __syncthreads();
  return make_int2(before + inc - x, total);
}

// The K-th largest of a (tile, head)'s values: the search runs bit by bit from bit 30 down (bit 31, the sign, is clear in every value that can count): x takes
// bit b when at least K elements are >= x | (1 << b). The count falls as x grows, so this ends at the largest x
// whose count reaches K, which is 0 when no x >= 0 does, the bisection's answer; K <= 0 gives its upper end, +inf.
// Values are at most +inf (no NaN patterns), so the result never passes it. One threshold per round: the cost is
// the comparisons per element (31 here; 48 for four-way steps, 77 and 120 for eight- and sixteen-way ones, which
// measured slower in that order), not the barriers. Waves with no valid element (`live` false) count nothing.
template <int E>
__device__ int kth_largest(const int (&bits)[E], int K, bool live, int* red, int& parity) {
  if (K <= 0) return 0x7F800000;
  const int wv = threadIdx.x >> 6;
  int x = 0;
  for (int b = 30; b >= 0; --b) {
    const int t = x | (1 << b);
    int c = 0;
    if (live) {
#pragma unroll
      for (int e = 0; e < E; ++e) c += __builtin_popcountll(__builtin_amdgcn_ballot_w64(bits[e] >= t));
    }
    int* r = red + parity * 4;
    if ((threadIdx.x & 63) == 0) r[wv] = c;
    __syncthreads();
    const int tot = r[0] + r[1] + r[2] + r[3];
    parity ^= 1;
    if (tot >= K) x = t;
  }
  return x;
}

template <int E>
__global__ __launch_bounds__(SEL_THREADS) void select_kernel(const float* __restrict__ map,
                                                              const uint8_t* __restrict__ keep_prev,
                                                              const float* __restrict__ scale_exact,
                                                              const float* __restrict__ scale_skip,
                                                              uint8_t* __restrict__ keep, int* __restrict__ cnt,
                                                              int* __restrict__ idx, const int* __restrict__ flags,
                                                              int* __restrict__ bits_out, int nw, int* __restrict__ ridx,
                                                              int rw, int K, int R, int NB, int L, int H, int nq,
                                                              int sink, int nwords) {
  __shared__ int red[8];  // two rounds' per-wave counts (kth_largest)
  __shared__ int scan_s[4];
  const int t = blockIdx.x, h = blockIdx.y;
  const int tid = threadIdx.x;
  const int j0 = tid * E;  // this thread's E consecutive block ids
  const size_t base = ((size_t)h * nq + t) * NB;
  const int lo_f = (t * BM) / BK - 1;
  const int hi_f = (min((t + 1) * BM, L) - 1) / BK + 1;
  const float se = scale_exact[h * nq + t], ss = scale_skip[h * nq + t];
  const int fell_back = flags[t * H + h];

  int vb[E], rb[E];
  float raw[E];
  bool forced[E], valid[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int j = j0 + e;
    valid[e] = j < NB;
    const bool kb = valid[e] && keep_prev[base + j] != 0;
    raw[e] = valid[e] ? map[base + j] : 0.0f;
    forced[e] = valid[e] && ((j >= lo_f && j <= hi_f) || j >= sink);
    float val = kb ? (fell_back != 0 ? INFINITY : raw[e] * se) : raw[e] * ss;
    val = val == val ? val : 0.0f;
    val = j >= sink ? INFINITY : val;
    val = valid[e] ? val : -1.0f;
    vb[e] = __float_as_int(val);
  }
  int parity = 0;
  const bool live = (int)(threadIdx.x & ~63u) * E < NB;  // (wave-uniform: the wave's first block)
  const float thr = __int_as_float(kth_largest<E>(vb, K, live, red, parity));
  bool kp[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    kp[e] = valid[e] && (__int_as_float(vb[e]) >= thr || forced[e]);
    float r2 = raw[e] == raw[e] ? raw[e] : 0.0f;
    r2 = (valid[e] && !kp[e]) ? r2 : -1.0f;
    rb[e] = __float_as_int(r2);
  }
  const int rthr = kth_largest<E>(rb, R, live, red, parity);
  bool ref[E];
  int ncand_local = 0, nkeep_local = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    ref[e] = rb[e] >= rthr && __int_as_float(rb[e]) >= 0.0f;  // candidates, before the index tie cut
    ncand_local += ref[e];
    nkeep_local += kp[e];
  }
  // index tie cut: only the first R candidates in block order; candidate number c goes to refine[c]
  const int2 rs = block_scan(ncand_local, scan_s);
  const int nref = min(rs.y, max(R, 0));
  const size_t rbase = ((size_t)t * H + h) * rw;
  int rpos = rs.x;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    if (ref[e]) {
      ref[e] = rpos < R;
      if (ref[e]) ridx[rbase + rpos] = j0 + e;
      ++rpos;
    }
  }
  for (int p = nref + tid; p < rw; p += SEL_THREADS) ridx[rbase + p] = NB;

  const int2 ks = block_scan(nkeep_local, scan_s);
  int pos = ks.x;
  const size_t ibase = ((size_t)t * H + h) * NB;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int j = j0 + e;
    if (kp[e]) idx[ibase + pos++] = j;
    if (valid[e]) keep[base + j] = kp[e] ? 1 : 0;
  }
  if (tid == 0) cnt[t * H + h] = ks.y;

  // skip bits: kept, past nb, or refined; E consecutive bits per thread
  unsigned word_bits = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const bool s = kp[e] || (j0 + e >= NB) || ref[e];
    word_bits |= (s ? 1u : 0u) << e;
  }
  // gather 32 / E threads into one word
  constexpr int TPW = 32 / E;  // threads per word
  unsigned w = word_bits << ((tid % TPW) * E);
#pragma unroll
  for (int m = 1; m < TPW; m <<= 1) w |= __shfl_xor(w, m, 64);
  if (tid % TPW == 0) {
    const int word = tid / TPW;
    if (word < nwords && word < nw) bits_out[((size_t)h * nq + t) * nw + word] = (int)w;
  }
}

__global__ void pack_kernel(const uint8_t* __restrict__ keep, int* __restrict__ out, int nw, int nwords, int nq,
                            int NB) {
  const int t = blockIdx.x, h = blockIdx.y;
  const size_t base = ((size_t)h * nq + t);
  for (int word = threadIdx.x; word < nwords; word += blockDim.x) {
    unsigned b = 0;
    for (int i = 0; i < 32; ++i) {
      const int j = word * 32 + i;
      const bool s = j >= NB || keep[base * NB + j] != 0;
      b |= (s ? 1u : 0u) << i;
    }
    out[base * nw + word] = (int)b;
  }
}

// one wave per (tile, head); each lane owns one 32-block word per round
__global__ __launch_bounds__(64) void rebuild_kernel(const int* __restrict__ exact_bits,
                                                     const int* __restrict__ skip_bits, int nw, int nwords,
                                                     uint8_t* __restrict__ keep, int* __restrict__ cnt,
                                                     int* __restrict__ idx, int* __restrict__ ridx,
                                                     int* __restrict__ rcnt, int rw, int* __restrict__ midx,
                                                     int* __restrict__ mcnt, int H, int nq, int NB) {
  const int t = blockIdx.x, h = blockIdx.y, l = threadIdx.x;
  const size_t pb = ((size_t)h * nq + t) * nw;
  const size_t lb = ((size_t)t * H + h) * NB;
  const size_t rbase = ((size_t)t * H + h) * rw;
  // lane l takes block j0 + l: one ballot per list gives every set bit its position among the lanes below it, so
  // the three lists come out in ascending block order with coalesced stores, 64 blocks per step
  (void)nwords;
  int off_e = 0, off_m = 0, off_r = 0;
  for (int j0 = 0; j0 < NB; j0 += 64) {
    const int j = j0 + l;
    const bool valid = j < NB;
    const unsigned ex = valid ? (unsigned)exact_bits[pb + (j >> 5)] : 0u;
    const unsigned sk = valid ? (unsigned)skip_bits[pb + (j >> 5)] : 0u;
    const bool e = valid && ((ex >> (j & 31)) & 1u);
    const bool sbit = (sk >> (j & 31)) & 1u;
    const bool r = valid && sbit && !e, m = valid && !sbit;
    const unsigned long long be = __builtin_amdgcn_ballot_w64(e), br = __builtin_amdgcn_ballot_w64(r),
                             bm = __builtin_amdgcn_ballot_w64(m);
    auto below = [&](unsigned long long b) {
      return (int)__builtin_amdgcn_mbcnt_hi((unsigned)(b >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)b, 0u));
    };
    if (e) idx[lb + off_e + below(be)] = j;
    if (m) midx[lb + off_m + below(bm)] = j;
    if (r) {
      const int pr = off_r + below(br);
      if (pr < rw) ridx[rbase + pr] = j;
    }
    if (valid) keep[((size_t)h * nq + t) * NB + j] = e ? 1 : 0;
    off_e += __builtin_popcountll(be);
    off_r += __builtin_popcountll(br);
    off_m += __builtin_popcountll(bm);
  }
  for (int p = off_r + l; p < rw; p += 64) ridx[rbase + p] = NB;
  if (l == 0) {
    cnt[t * H + h] = off_e;
    mcnt[t * H + h] = off_m;
    rcnt[t * H + h] = min(off_r, rw);
  }
}

__global__ __launch_bounds__(64) void scales_kernel(const float* __restrict__ m_in, float* __restrict__ lse,
                                                    float* __restrict__ scale_exact, float* __restrict__ scale_skip,
                                                    int L, int H, int nq) {
  const int t = blockIdx.x, h = blockIdx.y, l = threadIdx.x;
  const int nrows = min(L - t * BM, BM);
  float f = 0.0f;
  for (int r = l; r < BM; r += 64) {
    const int row = t * BM + r;
    const size_t o = (size_t)row * H + h;
    const float ls = lse[o];
    if (row < L) {
      f += exp2f(fminf(fmaxf(m_in[o] - ls, -100.0f), 100.0f));
    } else {
      lse[o] = 1e30f;
    }
  }
  f = wave_sum(f);
  if (l == 0) {
    scale_exact[h * nq + t] = f / (float)nrows / (float)nrows;
    scale_skip[h * nq + t] = 1.0f;
  }
}

static int next_pow2(int n) {
  int p = 1;
  while (p < n) p <<= 1;
  return p;
}

}  // namespace es

using namespace es;

extern "C" int es_select_blocks(const float* mass, const uint8_t* keep_prev, const float* scale_exact,
                                const float* scale_skip, uint8_t* keep, int* counts, int* blocks, const int* flags,
                                int* skip_bits, int nw, int* refine, int rw, int k, int r, int L, int H, int sink,
                                hipStream_t stream) {
  ES_REQUIRE(mass && keep_prev && scale_exact && scale_skip && keep && counts && blocks && flags && skip_bits &&
                 (refine || rw == 0),
             ES_ERR_INVALID, "null tensor pointer");
  ES_REQUIRE(L > 0 && H > 0, ES_ERR_INVALID, "L and H must be positive");
  const int nq = (L + BM - 1) / BM, nb = (L + BK - 1) / BK, nbp = next_pow2(nb);
  ES_REQUIRE(rw >= r && rw <= nbp, ES_ERR_INVALID, "refine width must satisfy r <= rw <= next_pow2(nb)");
  ES_REQUIRE(nw >= nbp / 32 || nbp < 32, ES_ERR_INVALID, "skip_bits has too few words per tile");
  ES_REQUIRE(nbp <= SEL_THREADS * SEL_MAXE, ES_ERR_UNSUPPORTED, "more than 4096 kv blocks");
  dim3 grid(nq, H);
#define SEL(E)                                                                                                   \
  hipLaunchKernelGGL(select_kernel<E>, grid, dim3(SEL_THREADS), 0, stream, mass, keep_prev, scale_exact,          \
                     scale_skip, keep, counts, blocks, flags, skip_bits, nw, refine, rw, k, r, nb, L, H, nq, sink, \
                     max(1, nbp / 32))
  const int E = nbp <= 256 * 1 ? 1 : nbp / 256;
  switch (E) {
    case 1: SEL(1); break;
    case 2: SEL(2); break;
    case 4: SEL(4); break;
    case 8: SEL(8); break;
    case 16: SEL(16); break;
    default: ES_REQUIRE(false, ES_ERR_UNSUPPORTED, "unsupported block count");
  }
#undef SEL
  return check_launch("es_select_blocks");
}

extern "C" int es_pack_plan(const uint8_t* keep, int* exact_bits, int nw, int H, int nq, int nb,
                            hipStream_t stream) {
  ES_REQUIRE(keep && exact_bits, ES_ERR_INVALID, "null tensor pointer");
  const int nwords = max(1, next_pow2(nb) / 32);
  ES_REQUIRE(nw >= nwords, ES_ERR_INVALID, "exact_bits has too few words per tile");
  hipLaunchKernelGGL(pack_kernel, dim3(nq, H), dim3(64), 0, stream, keep, exact_bits, nw, nwords, nq, nb);
  return check_launch("es_pack_plan");
}

extern "C" int es_rebuild_plan(const int* exact_bits, const int* skip_bits, int nw, uint8_t* keep, int* counts,
                               int* blocks, int* refine, int* refine_counts, int rw, int* means, int* mean_counts,
                               int H, int nq, int nb, hipStream_t stream) {
  ES_REQUIRE(exact_bits && skip_bits && keep && counts && blocks && (refine || rw == 0) && refine_counts && means &&
                 mean_counts,
             ES_ERR_INVALID, "null tensor pointer");
  const int nwords = max(1, next_pow2(nb) / 32);
  ES_REQUIRE(nw >= nwords, ES_ERR_INVALID, "bit plans have too few words per tile");
  hipLaunchKernelGGL(rebuild_kernel, dim3(nq, H), dim3(64), 0, stream, exact_bits, skip_bits, nw, nwords, keep,
                     counts, blocks, refine, refine_counts, rw, means, mean_counts, H, nq, nb);
  return check_launch("es_rebuild_plan");
}

extern "C" int es_full_step_scales(const float* offset, float* lse, float* scale_exact, float* scale_skip, int L,
                                   int H, hipStream_t stream) {
  ES_REQUIRE(offset && lse && scale_exact && scale_skip, ES_ERR_INVALID, "null tensor pointer");
  const int nq = (L + BM - 1) / BM;
  hipLaunchKernelGGL(scales_kernel, dim3(nq, H), dim3(64), 0, stream, offset, lse, scale_exact, scale_skip, L, H,
                     nq);
  return check_launch("es_full_step_scales");
}
