// Column-stream attention kernels for 128-row query tiles (gfx950, bf16 MFMA 32x32x16).
//
// One workgroup = one (query tile, head), 4 waves x 32 query rows. The keys the tile attends to arrive as a
// stream of 64-column chunks, each staged in LDS (double-buffered, direct global->LDS 16-byte loads, swizzled
// 256-byte rows) while the previous chunk is computed:
//   FIXED       the fixed-softmax-offset pass (reference echosparse/kernels/sm90.py:54-115): exact 64-token
//               blocks from the tile's block list, then (COMP) one column per listed mean block and four per
//               listed refined block, p = 2^(s*log2e/sqrt(D) + bias - prior); per-block mass (MASS), O, LSE,
//               flag.
//   ONLINE      online softmax over the block list (reference sm120.py:143-180 exact_fallback, flagged tiles
//               only); with no list and no flags it is dense attention with a log2 LSE.
//   COMPENSATE  block-mean columns of the skipped blocks appended at the new LSE (reference
//               triton_ops.py:251-295, flagged tiles only).
// Row sources per chunk kind: exact block b -> token rows b*64 + r of k / v (rows >= L clamped, bias -inf);
// mean block b -> row (b*H + h) of k_mean / v_mean; refined block b, rep c -> row h*(nb+1)*4 + 4b + c of
// k_rep / v_rep.
#include "../../include/echosparse_hip.h"
#include "common.h"
#include "queues.h"

#include <type_traits>

namespace es {

enum { FIXED = 0, ONLINE = 1, COMPENSATE = 2 };

constexpr float ONLINE_SLACK = 8.0f;  // log2 growth of a row's maximum that triggers a rescale (ONLINE)



struct AttnArgs {
  const bf16_t* q;
  const bf16_t* k;
  const bf16_t* v;
  const bf16_t* k_mean;
  const bf16_t* v_mean;
  const int* means;
  const int* mean_counts;
  const int* counts;
  const int* blocks;  // nullptr: every block (dense)
  const int* refine;
  const int* refine_counts;
  const bf16_t* k_rep;
  const bf16_t* v_rep;
  const float* log_counts;
  const uint8_t* keep;
  const float* prior;  // FIXED: offset; COMPENSATE: LSE after the fallback
  bf16_t* out;
  float* lse;
  int* flags;  // FIXED: written; ONLINE / COMPENSATE: read (nullptr = every tile)
  float* mass;
  int* queues;  // FIXED: the eight tile-queue counters of this launch (queues.h)
  int fixed;    // items per queue bound to dispatch slots; FIXED launches claim the rest
  int L, Lk, H, nq, nb, NK, RW, tiles, per_xcd;  // L query rows, Lk key rows (Lk == L but in dense_kv)
  float threshold, tail_log2, scale;
};

// Sources of one chunk for this lane: the ids of its four load rows and (wave 0) of its bias row.
struct ChunkIds {
  int row[4];  // exact: token block id (uniform); mean: mean block id; rep: rep row h-relative; -1 = padding
  int brow;    // the same for bias row = lane (wave 0)
};


// one (query tile t, head h)
template <int MODE, bool COMP, bool MASS>
__device__ __forceinline__ void attn_tile(const AttnArgs& a, const int h, const int t) {
  __shared__ __attribute__((aligned(16))) char kv_s[2][2][BK * 256];
  __shared__ __attribute__((aligned(16))) float bias_s[2][BK];
  __shared__ float mass_s[16][129];  // [wave * 4 + row of 16 lanes][chunk % 128], rows padded against bank conflicts
  // list entries of chunks j .. j+3 (ring slot j % 4), staged from global memory straight into LDS three chunks
  // ahead, so the loop holds no global->register or scalar loads whose waits would also drain the K / V loads
  __shared__ int ids_s[4][64];
  __shared__ float lc_s[BK];  // log2 counts of the next representative chunk's columns (wave 0, global -> LDS)

  const int th = t * a.H + h;
  if (MODE != FIXED && a.flags != nullptr && sload(a.flags + th) == 0) return;

  const int L = a.L, H = a.H, nb = a.nb;
  const int tid = threadIdx.x, l = tid & 63, hi = l >> 5, lq = l & 31;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, made scalar
  const int row = t * BM + wv * 32 + lq;
  const bool rvalid = row < L;
  const size_t nb4 = (size_t)(nb + 1) * 4;

  // ---------------------------------------------------------------- the column stream
  int n = 0, nm = 0, nr = 0;
  const int* g_ex = nullptr;
  const int* g_me = nullptr;
  const int* g_rf = nullptr;
  if (MODE == COMPENSATE) {
    n = 0;
  } else if (a.blocks == nullptr) {
    n = nb;
  } else {
    n = sload(a.counts + th);
    g_ex = a.blocks + (size_t)th * a.NK;
  }
  if (COMP) {
    nm = sload(a.mean_counts + th);
    nr = sload(a.refine_counts + th);
    g_me = a.means + (size_t)th * a.NK;
    g_rf = a.refine + (size_t)th * a.RW;
  }
  const int cm = (nm + BK - 1) / BK, cr = (4 * nr + BK - 1) / BK;
  const int nc = MODE == COMPENSATE ? (nb + BK - 1) / BK : n + (COMP ? cm + cr : 0);
  const bool tail_block = (a.Lk & (BK - 1)) != 0;

  // Loads go through buffer resources (32-bit offsets; offsets past the end read as zero). Token tensors and the
  // mean table are row-strided by H * 256 bytes from this head's first row; representatives are contiguous rows.
  // A token block gets a resource of its own based at its first row (64-bit address arithmetic), so q / k / v may
  // exceed 4 GiB; its range ends after the last valid key row, so rows past Lk read as zero.
  const unsigned hstride = (unsigned)H * HD * 2;
  auto block_srd = [&](const bf16_t* x, int b0) -> srd_t {
    const int rows = min(BK, a.Lk - b0);
    return make_srd(x + ((size_t)b0 * H + h) * HD, (unsigned)(rows - 1) * hstride + HD * 2);
  };
  srd_t rkm = {}, rvm = {}, rkr = {}, rvr = {};
  if (COMP || MODE == COMPENSATE) {
    rkm = make_srd(a.k_mean + (size_t)h * HD, (unsigned)(((size_t)nb * H - h) * HD * 2));
    rvm = make_srd(a.v_mean + (size_t)h * HD, (unsigned)(((size_t)nb * H - h) * HD * 2));
  }
  if (COMP) {
    rkr = make_srd(a.k_rep + (size_t)h * nb4 * HD, (unsigned)(nb4 * HD * 2));
    rvr = make_srd(a.v_rep + (size_t)h * nb4 * HD, (unsigned)(nb4 * HD * 2));
  }
  // this lane's four load rows R_i = 16 wv + 4 i + l / 16 and its swizzled 16-byte chunk within them
  const int rbase = wv * 16 + (l >> 4);
  unsigned chb[4], tok_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int P = (wv * 4 + i) * 64 + l, R = P >> 4;
    chb[i] = (unsigned)(((P & 15) ^ swz(R)) * 16);
    tok_off[i] = (unsigned)R * hstride + chb[i];
  }

  // wave 3 stages the list entries chunk cj needs into ids_s[cj % 4] (wave 0 writes the bias rows and wave 1 flushes
  // the mass partials, so the per-chunk duties are spread over the waves): exact -> its block id (every lane, same
  // word); mean -> the ids of its 64 columns; rep -> the refined block of each of its 64 columns
  auto stage_ids = [&](int cj) {
    if (MODE == COMPENSATE || wv != 3 || cj >= nc || (cj < n && g_ex == nullptr)) return;
    int* dst = ids_s[cj & 3];
    if (cj < n) {
      dma4(make_srd(g_ex, (unsigned)n * 4u), dst, 0, (unsigned)cj * 4u);
    } else if (cj < n + cm) {
      dma4(make_srd(g_me, (unsigned)nm * 4u), dst, (unsigned)((cj - n) * BK + l) * 4u, 0);
    } else {
      dma4(make_srd(g_rf, (unsigned)nr * 4u), dst, (unsigned)(((cj - n - cm) * BK + l) >> 2) * 4u, 0);
    }
  };
  // this lane's sources of chunk cj from ids_s (staged before the last barrier)
  auto read_ids = [&](int cj) -> ChunkIds {
    ChunkIds c = {};
    if (MODE == COMPENSATE || cj >= nc) return c;
    const int* src = ids_s[cj & 3];
    if (cj < n) {
      c.row[0] = g_ex == nullptr ? cj : __builtin_amdgcn_readfirstlane(src[0]);
    } else if (cj < n + cm) {
      const int c0 = (cj - n) * BK;
#pragma unroll
      for (int i = 0; i < 4; ++i) c.row[i] = c0 + rbase + 4 * i < nm ? src[rbase + 4 * i] : -1;
      c.brow = (wv == 0 && c0 + l < nm) ? src[l] : -1;
    } else {
      const int c0 = (cj - n - cm) * BK;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int col = c0 + rbase + 4 * i;
        c.row[i] = col < 4 * nr ? src[rbase + 4 * i] * 4 + (col & 3) : -1;
      }
      c.brow = (wv == 0 && c0 + l < 4 * nr) ? src[l] * 4 + ((c0 + l) & 3) : -1;
    }
    return c;
  };
  // the loads that stage one chunk (16 + 16 one-KB instructions, 4 + 4 per wave): sources and this lane's offsets
  struct Dma {
    srd_t rk, rv;
    unsigned off[4];
    unsigned soff;
  };
  auto dma_k = [&](const Dma& d, int sb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) dma16(d.rk, kv_s[sb][0] + wv * 4096 + i * 1024, d.off[i], d.soff);
  };
  auto dma_v = [&](const Dma& d, int sb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) dma16(d.rv, kv_s[sb][1] + wv * 4096 + i * 1024, d.off[i], d.soff);
  };
  // the loads of chunk cj into d; returns wave 0's bias value
  auto plan = [&](int cj, const ChunkIds& c, Dma& d) -> float {
    float bias = 0.0f;
    if (MODE == COMPENSATE || cj < n) {
      // 64 consecutive rows: token block b (exact) or mean blocks 64 cj .. (compensation)
      const int b0 = MODE == COMPENSATE ? cj * BK : __builtin_amdgcn_readfirstlane(c.row[0]) * BK;
      if (MODE == COMPENSATE) {
        d.rk = rkm;
        d.rv = rvm;
        d.soff = (unsigned)b0 * hstride;
      } else {
        d.rk = block_srd(a.k, b0);
        d.rv = block_srd(a.v, b0);
        d.soff = 0;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) d.off[i] = tok_off[i];
      if (wv == 0) {
        if (MODE == COMPENSATE) {
          const int b = b0 + l;
          bias = (b < nb && a.keep[((size_t)h * a.nq + t) * nb + b] == 0) ? (b == nb - 1 ? a.tail_log2 : 6.0f)
                                                                           : -INFINITY;
        } else {
          bias = b0 + l < a.Lk ? 0.0f : -INFINITY;
        }
      }
    } else {
      const bool mean = cj < n + cm;
      d.rk = mean ? rkm : rkr;
      d.rv = mean ? rvm : rvr;
      const unsigned stride = mean ? hstride : (unsigned)HD * 2;
#pragma unroll
      for (int i = 0; i < 4; ++i) d.off[i] = c.row[i] < 0 ? 0x80000000u : (unsigned)c.row[i] * stride + chb[i];
      d.soff = 0;
      if (wv == 0) {
        if (mean) {
          bias = c.brow < 0 ? -INFINITY : c.brow == nb - 1 ? a.tail_log2 : 6.0f;
        } else {
          // the log2 count goes to lc_s; the bias is read back once this chunk's loads have landed
          dma4(make_srd(a.log_counts + (size_t)h * nb4, (unsigned)nb4 * 4u), lc_s, c.brow < 0 ? 0x80000000u : (unsigned)c.brow * 4u, 0);
          bias = -INFINITY;
        }
      }
    }
    return bias;
  };

  // ---------------------------------------------------------------- per-lane query state
  bf16x8 qreg[8];
  {
    const bf16_t* qr = a.q + ((size_t)(rvalid ? row : 0) * H + h) * HD;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      bf16x8 z = {};
      qreg[ks] = rvalid ? *reinterpret_cast<const bf16x8*>(qr + 16 * ks + 8 * hi) : z;
    }
  }
  const float pr = (MODE != ONLINE && rvalid) ? a.prior[(size_t)row * H + h] : 0.0f;
  const float nprior = rvalid ? -pr : -INFINITY;
  const float scale = a.scale;

  // loop-invariant LDS offsets. K (A operand of S^T): row 32 mb + lq, chunk 2 ks + hi; the swizzle only sees the
  // low 4 row bits, so the mb = 1 rows sit 8 KB further. V^T (transposed reads): row block kk adds 4 KB.
  int koff[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) koff[ks] = tile_off(lq, 2 * ks + hi);
  int voff[2][4];  // [first / second four keys of the slot group][channel block]; rows 8 apart differ in swizzle
  {
    const int g1 = (l >> 4) & 1, sub = (l & 1) * 8;
    const int rowA = 4 * hi + ((l & 15) >> 2);
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      voff[0][db] = tile_off(rowA, 4 * db + 2 * g1 + ((l & 3) >> 1)) + sub;
      voff[1][db] = tile_off(rowA + 8, 4 * db + 2 * g1 + ((l & 3) >> 1)) + sub;
    }
  }

  f32x16 o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) o[db] = f32x16{};
  float lsum = 0.0f;        // this lane's share of the row sum (its 32 keys of every chunk)
  float mrun = -INFINITY;   // ONLINE running max (same in both half-waves)
  bool online_biased = true;  // ONLINE: the chunk has masked columns (the tail block)

  // exponentials of one 32-key half (C tile sh of the chunk) packed into two B operands of O^T += V^T P^T;
  // returns this lane's share of the half's sum. FIXED / COMPENSATE only (fixed offset, no running max).
  auto half = [&](const f32x16& sh, int boff, bf16x8& pa, bf16x8& pb, auto biased_tag) -> float {
    constexpr bool BIASED = decltype(biased_tag)::value;
    float p[16];
    if (BIASED) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4 b4 = *reinterpret_cast<const f32x4*>(&bias_s[0][0] + boff + 8 * i + 4 * hi);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) p[4 * i + jj] = fmaf(sh[4 * i + jj], scale, b4[jj]) + nprior;
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) p[r] = fmaf(sh[r], scale, nprior);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] = exp2f_fast(MODE == COMPENSATE ? fminf(p[r], 100.0f) : p[r]);
    pa = pack8(&p[0]);
    pb = pack8(&p[8]);
    return sum8_bf16(pb, sum8_bf16(pa, 0.0f));
  };
  // ONLINE: the same for a running maximum that is raised only when a half's maximum exceeds it by more than
  // 2^ONLINE_SLACK (then O and the row sum are rescaled first); otherwise the exponentials use the stale maximum,
  // so p <= 2^ONLINE_SLACK and most halves skip the rescale. The result is the same softmax: the final O / sum
  // and LSE = max + log2(sum) do not depend on which maximum the terms were taken against.
  // (the half's row sum goes straight into lsum: a later half's rescale must scale it too)
  // (one instantiation for both chunk kinds, within 256 VGPRs: `biased` is a wave-uniform run-time flag)
  // (an unbiased half takes its maximum on the raw products, max(s) * scale + prior being the maximum of the
  // logits, and folds the subtraction of the running maximum into the exponent's multiply-add)
  auto half_online = [&](const f32x16& sh, int boff, bf16x8& pa, bf16x8& pb, bool biased) {
    float p[16];
    float mh;
    if (biased) {
#pragma unroll
      for (int r = 0; r < 16; ++r) p[r] = fmaf(sh[r], scale, nprior);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4 b4 = *reinterpret_cast<const f32x4*>(&bias_s[0][0] + boff + 8 * i + 4 * hi);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) p[4 * i + jj] += b4[jj];
      }
      mh = p[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mh = fmaxf(mh, p[r]);
    } else {
      float mr = sh[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mr = fmaxf(mr, sh[r]);
      mh = fmaf(mr, scale, nprior);
    }
    mh = max_xor32(mh);
    if (mh > mrun + ONLINE_SLACK) {
      const float alpha = exp2f_fast(mrun - mh);
      lsum *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
      mrun = mh;
    }
    const float msub = mrun == -INFINITY ? 0.0f : mrun;
    if (biased) {
#pragma unroll
      for (int r = 0; r < 16; ++r) p[r] = exp2f_fast(p[r] - msub);
    } else {
      const float c = nprior - msub;
#pragma unroll
      for (int r = 0; r < 16; ++r) p[r] = exp2f_fast(fmaf(sh[r], scale, c));
    }
    pa = pack8(&p[0]);
    pb = pack8(&p[8]);
    lsum += sum8_bf16(pb, sum8_bf16(pa, 0.0f));
  };
  auto pv = [&](const char* vb, int kk, const bf16x8& pk) {
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const s16x4 ta = lds_read_tr(vb + 4096 * kk, voff[0][db]);
      const s16x4 tb = lds_read_tr(vb + 4096 * kk, voff[1][db]);
      o[db] = mfma32(cat_tr(ta, tb), pk, o[db]);
    }
  };

  // K fragments (A operands) of the chunk's first 32 keys, read into registers right after the barrier that made
  // the chunk visible and before the next chunk's transfers are issued: the eight reads then run under the
  // transfer issue, and the first S^T chain finds all its operands ready instead of waiting for one LDS read per
  // MFMA (the compiler, short of registers inside the compute section, reused one register quad for them)
  auto load_k0 = [&](int sb, bf16x8 (&kf)[8]) {
    const char* kb = kv_s[sb][0];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) kf[ks] = lds_read16(kb, koff[ks]);
  };

  // one chunk as two 32-key halves, so the matrix cores compute S^T of the second half while the VALU
  // exponentiates the first, and O^T += V^T P^T of the first half while the VALU does the second.
  auto compute = [&](int j, int sb, auto biased_tag, const bf16x8 (&kf0)[8]) {
    const char* kb = kv_s[sb][0];
    const char* vb = kv_s[sb][1];
    f32x16 s0 = {}, s1 = {};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) s0 = mfma32(kf0[ks], qreg[ks], s0);
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) s1 = mfma32(lds_read16(kb + 8192, koff[ks]), qreg[ks], s1);
    if (MODE != ONLINE) {
      bf16x8 pk0, pk1, pk2, pk3;
      float csum = half(s0, sb * BK, pk0, pk1, biased_tag);
      pv(vb, 0, pk0);
      pv(vb, 1, pk1);
      csum += half(s1, sb * BK + 32, pk2, pk3, biased_tag);
      pv(vb, 2, pk2);
      pv(vb, 3, pk3);
      lsum += csum;
      if (MODE == FIXED && MASS && j < n) {
        float bs = csum;
        bs += dpp_f<0x111>(bs);
        bs += dpp_f<0x112>(bs);
        bs += dpp_f<0x114>(bs);
        bs += dpp_f<0x118>(bs);
        if ((l & 15) == 15) mass_s[wv * 4 + (l >> 4)][j & 127] = bs;
      }
      return;
    }
    bf16x8 pk0, pk1, pk2, pk3;
    half_online(s0, sb * BK, pk0, pk1, online_biased);
    pv(vb, 0, pk0);
    pv(vb, 1, pk1);
    half_online(s1, sb * BK + 32, pk2, pk3, online_biased);
    pv(vb, 2, pk2);
    pv(vb, 3, pk3);
  };

  stage_ids(0);
  stage_ids(1);
  stage_ids(2);
  dma_wait();
  __syncthreads();
  int cur_row = 0;  // exact block id of the chunk being computed
  if (nc > 0) {
    const ChunkIds c = read_ids(0);
    cur_row = c.row[0];
    Dma d;
    const float b0 = plan(0, c, d);
    dma_k(d, 0);
    dma_v(d, 0);
    dma_wait();
    if (wv == 0) bias_s[0][l] = (COMP && n + cm == 0 && c.brow >= 0) ? lc_s[l] : b0;
  }
  dma_wait();
  __syncthreads();

  // exact block id of chunk j + 1, read from the ring one chunk early so that the LDS latency of the read is
  // spent under the previous chunk's compute rather than in front of the next transfers
  int pre_v = (nc > 1 && 1 < n && g_ex != nullptr) ? ids_s[1][0] : 1;
  int j = 0;
  // the exact-block stretch of a listed stream (chunks j .. j + 3 all exact blocks, chunk j not the partial last
  // token block, which a sorted list holds last if at all): the same steps as the general loop below with the chunk
  // kinds known, so none of its kind tests and list-source selections run per chunk, and one compute variant
  // (also the dense and full-block launches, whose block of chunk j is j itself)
  if (MODE != COMPENSATE && (MODE == ONLINE || g_ex != nullptr)) {
    const bool listed = MODE == FIXED || g_ex != nullptr;  // (a constant for the FIXED variants)
    const srd_t rex = make_srd(g_ex, listed ? (unsigned)n * 4u : 0u);
    cur_row = __builtin_amdgcn_readfirstlane(cur_row);  // (wave-uniform: keeps the loop test scalar)
    const unsigned kv_lds = uni(lds_addr(kv_s[0][0]) + (unsigned)wv * 4096u);
    for (; j + 3 < n && !(tail_block && cur_row == nb - 1); ++j) {
      const int sb = j & 1;
      bf16x8 kf0[8];
      load_k0(sb, kf0);
      const int next_row = listed ? __builtin_amdgcn_readfirstlane(pre_v) : j + 1;
      const int b0 = next_row * BK;
      Dma dn;
      dn.rk = block_srd(a.k, b0);
      dn.rv = block_srd(a.v, b0);
      dn.soff = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) dn.off[i] = tok_off[i];
      {
        const unsigned kd = kv_lds + (unsigned)(sb ^ 1) * (2u * BK * 256u);
#pragma unroll
        for (int i = 0; i < 4; ++i) dma16_at(dn.rk, kd + i * 1024, dn.off[i], 0u);
#pragma unroll
        for (int i = 0; i < 4; ++i) dma16_at(dn.rv, kd + BK * 256 + i * 1024, dn.off[i], 0u);
      }
      if (listed && wv == 3) dma4(rex, ids_s[(j + 3) & 3], 0, (unsigned)(j + 3) * 4u);
      pre_v = listed ? ids_s[(j + 2) & 3][0] : j + 2;  // (the general loop below starts from it)
      online_biased = false;
      if (!COMP)
        compute(j, sb, std::true_type{}, kf0);
      else
        compute(j, sb, std::false_type{}, kf0);
      dma_wait();
      // (the compensated and online variants read the bias of an exact chunk only for the partial last block)
      if (wv == 0 && ((MODE == FIXED && !COMP) || (tail_block && next_row == nb - 1)))
        bias_s[sb ^ 1][l] = b0 + l < a.Lk ? 0.0f : -INFINITY;
      __syncthreads();
      if (MASS && ((j & 63) == 63) && wv == 1) {
        const int idx = (j & ~63) + l;
        float m = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) m += mass_s[r][idx & 127];
        a.mass[((size_t)h * a.nq + t) * nb + (listed ? g_ex[idx] : idx)] = m;
      }
      cur_row = next_row;
    }
  }
  // one chunk of any kind (the general step)
  auto general_step = [&](int j) {
    const int sb = j & 1;
    bf16x8 kf0[8];
    load_k0(sb, kf0);
    float bnext = 0.0f;
    int next_row = 0;
    bool next_lc = false;  // the next chunk's bias comes from lc_s
    if (j + 1 < nc) {
      ChunkIds c;
      if (j + 1 < n) { c = ChunkIds{}; c.row[0] = __builtin_amdgcn_readfirstlane(pre_v); }
      else c = read_ids(j + 1);
      next_row = c.row[0];
      next_lc = COMP && j + 1 >= n + cm && c.brow >= 0;
      Dma dn;
      bnext = plan(j + 1, c, dn);
      dma_k(dn, sb ^ 1);
      dma_v(dn, sb ^ 1);
    }
    stage_ids(j + 3);
    pre_v = (j + 2 < n && g_ex != nullptr) ? ids_s[(j + 2) & 3][0] : j + 2;
    const bool biased = MODE == COMPENSATE || j >= n || (tail_block && cur_row == nb - 1);
    online_biased = biased;
    if (!COMP || biased)   // (non-COMP variants: one instantiation keeps them within 256 VGPRs)
      compute(j, sb, std::true_type{}, kf0);
    else
      compute(j, sb, std::false_type{}, kf0);
    dma_wait();
    if (j + 1 < nc && wv == 0) bias_s[sb ^ 1][l] = next_lc ? lc_s[l] : bnext;
    __syncthreads();
    if (MODE == FIXED && MASS && j < n && ((j & 63) == 63 || j == n - 1) && wv == 1) {
      const int idx = (j & ~63) + l;
      if (idx <= j) {
        float m = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) m += mass_s[r][idx & 127];
        const int b = g_ex == nullptr ? idx : g_ex[idx];
        a.mass[((size_t)h * a.nq + t) * nb + b] = m;
      }
    }
    cur_row = next_row;
    };
  if (MODE == FIXED && COMP) {
    for (; j < nc && j < n; ++j) general_step(j);
    // the block-mean stretch (chunk j and chunk j + 1 both mean columns): the same steps with the kind known
    {
      const unsigned kv_lds = uni(lds_addr(kv_s[0][0]) + (unsigned)wv * 4096u);
      for (; j + 1 < n + cm; ++j) {
        const int sb = j & 1;
        bf16x8 kf0[8];
        load_k0(sb, kf0);
        const int* src = ids_s[(j + 1) & 3];
        const int c0 = (j + 1 - n) * BK;
        unsigned off[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int col = c0 + rbase + 4 * i;
          off[i] = col < nm ? (unsigned)src[rbase + 4 * i] * hstride + chb[i] : 0x80000000u;
        }
        int brow = -1;
        if (wv == 0) brow = c0 + l < nm ? src[l] : -1;
        {
          const unsigned kd = kv_lds + (unsigned)(sb ^ 1) * (2u * BK * 256u);
#pragma unroll
          for (int i = 0; i < 4; ++i) dma16_at(rkm, kd + i * 1024, off[i], 0u);
#pragma unroll
          for (int i = 0; i < 4; ++i) dma16_at(rvm, kd + BK * 256 + i * 1024, off[i], 0u);
        }
        stage_ids(j + 3);
        compute(j, sb, std::true_type{}, kf0);
        dma_wait();
        if (wv == 0) bias_s[sb ^ 1][l] = brow < 0 ? -INFINITY : brow == nb - 1 ? a.tail_log2 : 6.0f;
        __syncthreads();
      }
    }
    for (; j < nc && !(j >= n + cm && j + 3 < nc); ++j) general_step(j);
    // the representative stretch (chunks j .. j + 3 all representative columns): the same steps with the kind known
    const srd_t rlc = make_srd(a.log_counts + (size_t)h * nb4, (unsigned)nb4 * 4u);
    const srd_t rrf = make_srd(g_rf, (unsigned)nr * 4u);
    const unsigned kv_lds = uni(lds_addr(kv_s[0][0]) + (unsigned)wv * 4096u);
    for (; j + 3 < nc; ++j) {
      const int sb = j & 1;
      bf16x8 kf0[8];
      load_k0(sb, kf0);
      const int* src = ids_s[(j + 1) & 3];
      const int c0 = (j + 1 - n - cm) * BK;
      unsigned off[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int col = c0 + rbase + 4 * i;
        off[i] = col < 4 * nr ? (unsigned)(src[rbase + 4 * i] * 4 + (col & 3)) * (HD * 2) + chb[i] : 0x80000000u;
      }
      int brow = -1;
      if (wv == 0) {
        brow = c0 + l < 4 * nr ? src[l] * 4 + ((c0 + l) & 3) : -1;
        dma4(rlc, lc_s, brow < 0 ? 0x80000000u : (unsigned)brow * 4u, 0u);
      }
      {
        const unsigned kd = kv_lds + (unsigned)(sb ^ 1) * (2u * BK * 256u);
#pragma unroll
        for (int i = 0; i < 4; ++i) dma16_at(rkr, kd + i * 1024, off[i], 0u);
#pragma unroll
        for (int i = 0; i < 4; ++i) dma16_at(rvr, kd + BK * 256 + i * 1024, off[i], 0u);
      }
      if (wv == 3) dma4(rrf, ids_s[(j + 3) & 3], (unsigned)((((j + 3 - n - cm) * BK + l) >> 2) * 4), 0u);
      compute(j, sb, std::true_type{}, kf0);
      dma_wait();
      if (wv == 0) bias_s[sb ^ 1][l] = brow >= 0 ? lc_s[l] : -INFINITY;
      __syncthreads();
    }
  }
  for (; j < nc; ++j) general_step(j);

  // ---------------------------------------------------------------- epilogue
  const float tot = sum_xor32(lsum);
  bf16_t* orow = a.out + ((size_t)(rvalid ? row : 0) * H + h) * HD;
  float* lrow = a.lse + (size_t)row * H + h;
  auto store_rows = [&](float inv) {
    if (!rvalid) return;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ushort4 v4;
        v4.x = f2bf(o[db][4 * i + 0] * inv);
        v4.y = f2bf(o[db][4 * i + 1] * inv);
        v4.z = f2bf(o[db][4 * i + 2] * inv);
        v4.w = f2bf(o[db][4 * i + 3] * inv);
        *reinterpret_cast<ushort4*>(orow + 32 * db + 8 * i + 4 * hi) = v4;
      }
  };
  if (MODE == FIXED) {
    const float lg = log2f(tot);
    const bool bad = rvalid && !(lg >= -a.threshold && lg <= a.threshold);
    const int any = __syncthreads_or(bad);
    store_rows(1.0f / tot);
    if (hi == 0) *lrow = rvalid ? pr + lg : 1e30f;
    if (tid == 0) a.flags[th] = any;
  } else if (MODE == ONLINE) {
    const bool empty = n == 0;
    store_rows(empty ? 0.0f : 1.0f / tot);
    if (hi == 0) *lrow = !rvalid ? 1e30f : empty ? -1e30f : mrun + log2f(tot);
  } else {
    const float den = 1.0f + tot;
    const float inv = 1.0f / den;
    if (rvalid) {
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          ushort4* dst = reinterpret_cast<ushort4*>(orow + 32 * db + 8 * i + 4 * hi);
          ushort4 old = *dst, v4;
          v4.x = f2bf((bf2f(old.x) + o[db][4 * i + 0]) * inv);
          v4.y = f2bf((bf2f(old.y) + o[db][4 * i + 1]) * inv);
          v4.z = f2bf((bf2f(old.z) + o[db][4 * i + 2]) * inv);
          v4.w = f2bf((bf2f(old.w) + o[db][4 * i + 3]) * inv);
          *dst = v4;
        }
    }
    if (hi == 0) *lrow = rvalid ? pr + log2f(den) : 1e30f;
  }
}

// XCD-aware, run-time balanced tile order (queues.h); the fallback launches (ONLINE with flags, COMPENSATE), which
// skip unflagged tiles, bind every item to its dispatch slot
template <int MODE, bool COMP, bool MASS>
__global__ __launch_bounds__(256, 2) void attn_kernel(AttnArgs a) {
  const int w = blockIdx.x, per_queue = a.H * a.per_xcd;
  int x = w & 7, k = w >> 3;
  if (MODE != COMPENSATE && k >= a.fixed) {
    __shared__ int item_s;
    if (threadIdx.x < 64) {
      const int it = claim_item(a.queues, x, a.fixed, per_queue);
      if (threadIdx.x == 0) item_s = it;
    }
    __syncthreads();
    const int it = __builtin_amdgcn_readfirstlane(item_s);
    if (it < 0) return;
    x = it / per_queue;
    k = it - x * per_queue;
  }
  const int h = k / a.per_xcd;
  const int t = ((x + h) & 7) * a.per_xcd + k % a.per_xcd;
  if (h >= a.H || t >= a.tiles) return;
  attn_tile<MODE, COMP, MASS>(a, h, t);
}

template <int MODE, bool COMP, bool MASS>
static int launch(const AttnArgs& a0, hipStream_t stream, const char* what) {
  AttnArgs a = a0;
  a.per_xcd = (a.tiles + 7) / 8;
  long long grid = 8LL * a.H * a.per_xcd;
  if (grid <= 0) return ES_OK;
  a.fixed = a.H * a.per_xcd;
  Queues qs;  // (released after the launch below is enqueued)
  if (MODE == FIXED || (MODE == ONLINE && a.flags == nullptr)) {
    ES_REQUIRE(balanced_launch(a.H, a.per_xcd, stream, qs), ES_ERR_LAUNCH, "tile queues unavailable on this device");
    a.queues = qs.counters;
    a.fixed = qs.fixed;
    grid = qs.grid;
  }
  hipLaunchKernelGGL((attn_kernel<MODE, COMP, MASS>), dim3((unsigned)grid), dim3(256), 0, stream, a);
  return check_launch(what);
}

static int check_common(const void* q, const void* k, const void* v, int L, int H, int D) {
  ES_REQUIRE(q && k && v, ES_ERR_INVALID, "q, k and v must be non-null");
  ES_REQUIRE(L > 0 && H > 0, ES_ERR_INVALID, "L and H must be positive");
  ES_REQUIRE(D == HD, ES_ERR_UNSUPPORTED, "head dimension must be 128");
  ES_REQUIRE((size_t)BK * H * D * 2 < (1ull << 31), ES_ERR_UNSUPPORTED, "too many heads (one token block's rows "
             "must span under 2 GiB)");
  return ES_OK;
}

static AttnArgs base_args(const void* q, const void* k, const void* v, int L, int H) {
  AttnArgs a = {};
  a.q = (const bf16_t*)q;
  a.k = (const bf16_t*)k;
  a.v = (const bf16_t*)v;
  a.L = L;
  a.Lk = L;
  a.H = H;
  a.nq = (L + BM - 1) / BM;
  a.nb = (L + BK - 1) / BK;
  a.tiles = a.nq;
  a.tail_log2 = log2f((float)(L - (a.nb - 1) * BK));
  a.scale = LOG2E / sqrtf((float)HD);
  a.threshold = 60.0f;
  return a;
}

}  // namespace es

using namespace es;

extern "C" int es_block_attention(const void* q, const void* k, const void* v, void* out, const int* counts,
                                  const int* blocks, int nk, const float* offset, float* lse, int* flags,
                                  float* mass, float threshold, int L, int H, int D, hipStream_t stream) {
  int st = check_common(q, k, v, L, H, D);
  if (st) return st;
  ES_REQUIRE(out && counts && blocks && offset && lse && flags, ES_ERR_INVALID, "null output or list pointer");
  AttnArgs a = base_args(q, k, v, L, H);
  ES_REQUIRE(nk >= 1, ES_ERR_INVALID, "block list width must be positive");
  a.out = (bf16_t*)out;
  a.counts = counts;
  a.blocks = blocks;
  a.NK = nk;
  a.prior = offset;
  a.lse = lse;
  a.flags = flags;
  a.mass = mass;
  a.threshold = threshold;
  if (mass) return launch<FIXED, false, true>(a, stream, "es_block_attention");
  return launch<FIXED, false, false>(a, stream, "es_block_attention");
}

extern "C" int es_sparse_attention(const void* q, const void* k, const void* v, const void* k_mean,
                                   const void* v_mean, const int* means, const int* mean_counts, void* out,
                                   const int* counts, const int* blocks, int nk, const float* offset, float* lse,
                                   int* flags, const int* refine, const int* refine_counts, int rw,
                                   const void* k_rep, const void* v_rep, const float* log_counts, float* mass,
                                   float threshold, int tiles, int L, int H, int D, hipStream_t stream) {
  int st = check_common(q, k, v, L, H, D);
  if (st) return st;
  ES_REQUIRE(out && counts && blocks && offset && lse && flags && k_mean && v_mean && means && mean_counts &&
                 (refine || rw == 0) && refine_counts && k_rep && v_rep && log_counts,
             ES_ERR_INVALID, "null tensor pointer");
  AttnArgs a = base_args(q, k, v, L, H);
  ES_REQUIRE(nk >= 1 && rw >= 0, ES_ERR_INVALID, "bad list widths");
  ES_REQUIRE(tiles >= 0 && tiles <= a.nq, ES_ERR_INVALID, "tiles out of range");
  a.k_mean = (const bf16_t*)k_mean;
  a.v_mean = (const bf16_t*)v_mean;
  a.means = means;
  a.mean_counts = mean_counts;
  a.out = (bf16_t*)out;
  a.counts = counts;
  a.blocks = blocks;
  a.NK = nk;
  a.prior = offset;
  a.lse = lse;
  a.flags = flags;
  a.refine = refine;
  a.refine_counts = refine_counts;
  a.RW = rw;
  a.k_rep = (const bf16_t*)k_rep;
  a.v_rep = (const bf16_t*)v_rep;
  a.log_counts = log_counts;
  a.mass = mass;
  a.threshold = threshold;
  a.tiles = tiles;
  if (mass) return launch<FIXED, true, true>(a, stream, "es_sparse_attention");
  return launch<FIXED, true, false>(a, stream, "es_sparse_attention");
}

extern "C" int es_exact_fallback(const void* q, const void* k, const void* v, void* out, const int* counts,
                                 const int* blocks, int nk, float* lse, const int* flags, int L, int H, int D,
                                 hipStream_t stream) {
  int st = check_common(q, k, v, L, H, D);
  if (st) return st;
  ES_REQUIRE(out && counts && blocks && lse && flags, ES_ERR_INVALID, "null tensor pointer");
  AttnArgs a = base_args(q, k, v, L, H);
  a.out = (bf16_t*)out;
  a.counts = counts;
  a.blocks = blocks;
  a.NK = nk;
  a.lse = lse;
  a.flags = (int*)flags;
  return launch<ONLINE, false, false>(a, stream, "es_exact_fallback");
}

extern "C" int es_dense_attention(const void* q, const void* k, const void* v, void* out, float* lse2, int L,
                                  int H, int D, hipStream_t stream) {
  int st = check_common(q, k, v, L, H, D);
  if (st) return st;
  ES_REQUIRE(out && lse2, ES_ERR_INVALID, "null tensor pointer");
  AttnArgs a = base_args(q, k, v, L, H);
  a.out = (bf16_t*)out;
  a.lse = lse2;
  return launch<ONLINE, false, false>(a, stream, "es_dense_attention");
}

extern "C" int es_compensate_fallback(const void* q, const void* k_mean, const void* v_mean, const uint8_t* keep,
                                      float* lse, void* out, const int* flags, int L, int H, int D,
                                      hipStream_t stream) {
  int st = check_common(q, k_mean, v_mean, L, H, D);
  if (st) return st;
  ES_REQUIRE(keep && lse && out && flags, ES_ERR_INVALID, "null tensor pointer");
  AttnArgs a = base_args(q, k_mean, v_mean, L, H);
  a.k_mean = (const bf16_t*)k_mean;
  a.v_mean = (const bf16_t*)v_mean;
  a.keep = keep;
  a.prior = lse;
  a.lse = lse;
  a.out = (bf16_t*)out;
  a.flags = (int*)flags;
  return launch<COMPENSATE, false, false>(a, stream, "es_compensate_fallback");
}

extern "C" int es_dense_attention_kv(const void* q, const void* k, const void* v, void* out, float* lse2, int Lq,
                                     int Lk, int H, int D, hipStream_t stream) {
  int st = check_common(q, k, v, Lq, H, D);
  if (st) return st;
  ES_REQUIRE(Lk > 0, ES_ERR_INVALID, "Lk must be positive");
  ES_REQUIRE(Lk > 0, ES_ERR_INVALID, "Lk must be positive");
  ES_REQUIRE(out && lse2, ES_ERR_INVALID, "null tensor pointer");
  AttnArgs a = base_args(q, k, v, Lq, H);
  a.Lk = Lk;
  a.nb = (Lk + BK - 1) / BK;
  a.out = (bf16_t*)out;
  a.lse = lse2;
  return launch<ONLINE, false, false>(a, stream, "es_dense_attention_kv");
}
