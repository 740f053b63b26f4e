// VSA fine block-sparse attention over a CSR block selection (gfx950, bf16 MFMA 32x32x16).
//
// Tokens are [BH, L, 128] bf16 rows, L = NB * 64 in 64-token blocks. Every kernel is instantiated for the logical
// head dim DH = 128 and DH = 64: at DH = 64 (columns 64..127 zero by contract) it stages only the first 128 bytes
// of each row, runs half the QK^T k-steps and half the 32-column output blocks, and writes zeros past column 64
// (C2 shape at D = 64: forward 2.21 -> 1.76 ms, forward + backward 10.2 -> 7.6 ms). blk_cnt[NB] gives each block's valid
// tokens (valid-first). Query block i of head bh attends to the kv blocks row_ptr / col_idx list for row
// (bh, i), with key columns >= blk_cnt[kv] masked; query rows >= blk_cnt[i] and rows with an empty list get
// O = 0 and lse = -inf. lse is the natural-log row sum. Semantics: reference csrc/vsa/generic/attn_fwd.cu:16-24,
// tests/vsa_reference.py:90-107.
//
// Forward: one workgroup per (query block, head), 4 waves = 2 row groups of 32 queries x 2 key halves of each
// 64-key chunk. Every chunk is staged once in LDS (double-buffered direct global->LDS loads, swizzled 256-byte
// rows) and each wave runs its own online softmax over its 32-key halves (S^T = K Q^T so that exp(S^T) is directly
// the B operand of O^T += V^T P^T); the two key-half states of a row group are merged once at the end through
// LDS. The running max is only moved when a row's new maximum exceeds it by more than 8 (log2 units), which
// keeps the O rescale off the common path without changing the result beyond rounding.
// Task mode (split-KV, reference attn_fwd.cu:216-237): the grid walks (row, beg, end, slot) tasks; slot >= 0
// writes an fp32 normalized partial O and its log2 lse to part_o / part_lse, slot < 0 the final O / lse.
#include "../../include/vsa_hip.h"
#include "common.h"
#include "elem.h"
#include "queues.h"

namespace es {

namespace {

constexpr float LN2 = 0.6931471805599453f;
constexpr float RESCALE_SLACK = 8.0f;

struct VsaFwdArgs {
  const e16_t *q, *k, *v;
  e16_t* out;
  float* lse;
  const int *row_ptr, *col_idx, *blk_cnt;
  const int4* tasks;
  const int* info;  // device task count (task mode)
  float *part_o, *part_lse;
  int* queues;  // the eight row-block queue counters of this launch (queues.h)
  int L, NB, BH, per_xcd, fixed;
  float scale;  // log2(e) / sqrt(D)
};

// (K / V are staged with the inline-assembly transfer dma16. With the compiler-visible buffer-to-LDS builtin the
// compiler cannot tell the next chunk's buffer from this one's and waits for the next chunk's transfers before
// this chunk's V^T reads.)
template <bool TASKS, int DH>
__global__ __launch_bounds__(256, 2) void vsa_fwd_kernel(VsaFwdArgs a) {
  constexpr int NKS = DH / 16, NDB = DH / 32;  // MFMA k-steps of QK^T, 32-column blocks of O (D = 64: the first half)
  __shared__ __attribute__((aligned(16))) char kv_s[2][2][BK * 256];

  int qb, bh, beg, end, slot = -1;
  if (TASKS) {
    if ((int)blockIdx.x >= sload(a.info)) return;
    const int4 tk = a.tasks[blockIdx.x];
    bh = tk.x / a.NB;
    qb = tk.x - bh * a.NB;
    beg = tk.y;
    end = tk.z;
    slot = tk.w;
  } else {
    // XCD-aware, run-time balanced order of (query block, head) (queues.h)
    if (!balanced_item(a.queues, a.fixed, a.per_xcd, a.BH, a.NB, bh, qb)) return;
    const int* rp = a.row_ptr + (size_t)bh * (a.NB + 1) + qb;
    beg = sload(rp);
    end = sload(rp + 1);
  }
  beg = __builtin_amdgcn_readfirstlane(beg);
  end = __builtin_amdgcn_readfirstlane(end);
  const int nc = end - beg;

  const int tid = threadIdx.x, l = tid & 63, hi = l >> 5, lq = l & 31;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rg = wv & 1, kh = wv >> 1;
  const int qrow = 32 * rg + lq;  // row inside the query block
  const int qcnt = sload(a.blk_cnt + qb);
  const bool qvalid = qrow < qcnt;
  const size_t head = (size_t)bh * a.L;

  const unsigned head_bytes = (unsigned)((size_t)a.L * HD * 2);
  const srd_t rk = make_srd(a.k + head * HD, head_bytes);
  const srd_t rv = make_srd(a.v + head * HD, head_bytes);
  // this lane's four load rows R = 16 wv + 4 i + l / 16 of a chunk and its swizzled 16-byte chunk in them
  unsigned ld_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int P = (wv * 4 + i) * 64 + l, R = P >> 4, g = (P & 15) ^ swz(R);
    ld_off[i] = g < DH / 8 ? (unsigned)R * 256 + (unsigned)(g * 16) : 0x80000000u;
  }
  auto issue = [&](int b, int sb) {
    const unsigned soff = (unsigned)b * (BK * 256);
    char* kd = kv_s[sb][0] + wv * 4096;
    char* vd = kv_s[sb][1] + wv * 4096;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      dma16(rk, kd + i * 1024, ld_off[i], soff);
      dma16(rv, vd + i * 1024, ld_off[i], soff);
    }
  };

  ev8 qreg[8];
  {
    const e16_t* qp = a.q + (head + (size_t)qb * BK + qrow) * HD;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) qreg[ks] = *reinterpret_cast<const ev8*>(qp + 16 * ks + 8 * hi);
  }
  int koff[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) koff[ks] = kh * 8192 + tile_off(lq, 2 * ks + hi);
  int voff[2][4];
  {
    const int g1 = (l >> 4) & 1, sub = (l & 1) * 8, rowA = 4 * hi + ((l & 15) >> 2);
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      voff[0][db] = tile_off(rowA, 4 * db + 2 * g1 + ((l & 3) >> 1)) + sub;
      voff[1][db] = tile_off(rowA + 8, 4 * db + 2 * g1 + ((l & 3) >> 1)) + sub;
    }
  }

  f32x16 o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) o[db] = f32x16{};
  float lsum = 0.0f, mref = -INFINITY;
  const float scale = a.scale;

  int bcur = nc > 0 ? sload(a.col_idx + beg) : 0;
  int ccur = nc > 0 ? sload(a.blk_cnt + bcur) : 0;
  int bnext = nc > 1 ? sload(a.col_idx + beg + 1) : 0;
  if (nc > 0) issue(bcur, 0);
  wait_vmem();
  __syncthreads();

  for (int j = 0; j < nc; ++j) {
    const int sb = j & 1;
    int cnext = 0, bnn = 0;
    if (j + 1 < nc) {
      issue(bnext, sb ^ 1);
      cnext = sload(a.blk_cnt + bnext);
      if (j + 2 < nc) bnn = sload(a.col_idx + beg + j + 2);
    }
    const char* kb = kv_s[sb][0];
    const char* vb = kv_s[sb][1] + kh * 8192;
    f32x16 s = {};
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) s = emfma(elds16(kb, koff[ks]), qreg[ks], s);
    // the maximum is taken on the raw products (scale > 0: max(s) * scale is the maximum of the scaled logits, the
    // rounding being monotone), and the scaling is folded into the multiply-add in front of each exponential
    if (ccur < BK) {  // key columns past the block's valid tokens
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (32 * kh + 8 * (r / 4) + 4 * hi + (r % 4) >= ccur) s[r] = -INFINITY;
    }
    float mx = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
    mx = max_xor32(mx) * scale;
    if (__builtin_amdgcn_ballot_w64(mx > mref + RESCALE_SLACK) != 0) {
      const float mnew = fmaxf(mref, mx);
      const float alpha = mref == -INFINITY ? 0.0f : exp2f_fast(mref - mnew);
      lsum *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
      mref = mnew;
    }
    const float msub = mref == -INFINITY ? 0.0f : mref;
    float p[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] = exp2f_fast(fmaf(s[r], scale, -msub));
    const ev8 pa = epack8(&p[0]), pb = epack8(&p[8]);
    lsum += esum8(pb, esum8(pa, 0.0f));
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      o[db] = emfma(ecat_tr(lds_read_tr(vb, voff[0][db]), lds_read_tr(vb, voff[1][db])), pa, o[db]);
      o[db] = emfma(ecat_tr(lds_read_tr(vb + 4096, voff[0][db]), lds_read_tr(vb + 4096, voff[1][db])), pb, o[db]);
    }
    wait_vmem();
    __syncthreads();
    bcur = bnext;
    ccur = cnext;
    bnext = bnn;
  }

  // merge the two key halves of each row group: kh = 1 waves hand (m, l, O) to the kh = 0 waves through LDS
  float* xo = reinterpret_cast<float*>(&kv_s[0][0][0]) + rg * (64 * 64);        // [64 regs][64 lanes]
  float* xm = reinterpret_cast<float*>(&kv_s[1][0][0]) + rg * 128;              // [m | l][64 lanes]
  const float ltot = sum_xor32(lsum);
  if (kh == 1) {
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) xo[(db * 16 + r) * 64 + l] = o[db][r];
    xm[l] = mref;
    xm[64 + l] = ltot;
  }
  __syncthreads();
  if (kh == 1) return;
  const float m1 = xm[l], l1 = xm[64 + l];
  const float M = fmaxf(mref, m1);
  const float a0 = mref == -INFINITY ? 0.0f : exp2f_fast(mref - M);
  const float a1 = m1 == -INFINITY ? 0.0f : exp2f_fast(m1 - M);
  const float lt = a0 * ltot + a1 * l1;
  const bool live = qvalid && lt > 0.0f;
  const float inv = live ? 1.0f / lt : 0.0f;
  const size_t tok = head + (size_t)qb * BK + qrow;
  const float lse2 = live ? M + log2f(lt) : -INFINITY;
  if (!TASKS || slot < 0) {
    e16_t* orow = a.out + tok * HD;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ushort4 v4;
        v4 = ushort4{0, 0, 0, 0};
        if (db < NDB) {
          v4.x = f2e((a0 * o[db][4 * i + 0] + a1 * xo[(db * 16 + 4 * i + 0) * 64 + l]) * inv);
          v4.y = f2e((a0 * o[db][4 * i + 1] + a1 * xo[(db * 16 + 4 * i + 1) * 64 + l]) * inv);
          v4.z = f2e((a0 * o[db][4 * i + 2] + a1 * xo[(db * 16 + 4 * i + 2) * 64 + l]) * inv);
          v4.w = f2e((a0 * o[db][4 * i + 3] + a1 * xo[(db * 16 + 4 * i + 3) * 64 + l]) * inv);
        }
        *reinterpret_cast<ushort4*>(orow + 32 * db + 8 * i + 4 * hi) = v4;
      }
    if (hi == 0) a.lse[tok] = live ? lse2 * LN2 : -INFINITY;
  } else {
    float* prow = a.part_o + ((size_t)slot * BK + qrow) * HD;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float4 v4 = make_float4(0.f, 0.f, 0.f, 0.f);
        if (db < NDB) {
          v4.x = (a0 * o[db][4 * i + 0] + a1 * xo[(db * 16 + 4 * i + 0) * 64 + l]) * inv;
          v4.y = (a0 * o[db][4 * i + 1] + a1 * xo[(db * 16 + 4 * i + 1) * 64 + l]) * inv;
          v4.z = (a0 * o[db][4 * i + 2] + a1 * xo[(db * 16 + 4 * i + 2) * 64 + l]) * inv;
          v4.w = (a0 * o[db][4 * i + 3] + a1 * xo[(db * 16 + 4 * i + 3) * 64 + l]) * inv;
        }
        *reinterpret_cast<float4*>(prow + 32 * db + 8 * i + 4 * hi) = v4;
      }
    if (hi == 0) a.part_lse[(size_t)slot * BK + qrow] = lse2;
  }
}


// ------------------------------------------------------------------------------------------------ backward
// Per selected pair (query block i, kv block j), with P = exp(S / sqrt(D) - lse) and dS = P (dP - delta) / sqrt(D)
// (reference csrc/vsa/generic/attn_bwd.cu:1-34; rows with lse = -inf and key columns >= blk_cnt get P = 0):
//   KV owner (dK, dV; k2q lists): one workgroup per (kv block, head), 4 waves = 2 key halves x 2 query halves of
//     each staged query block. S = Q K^T and dP = dO V^T come out with keys on lanes, so P and dS are directly the
//     B operands of dV^T += dO^T P and dK^T += Q^T dS (dO^T / Q^T through transposed LDS reads). K and V stay in
//     registers; Q, dO, lse and delta of each listed query block stream through LDS. It runs as two passes, dV
//     (S, dV) then dK (S, dP, dK): 5 products per pair instead of 4, but each pass holds one 128-register
//     accumulator set instead of two, so two waves share a SIMD (one pass with both: 5.68 ms at C2, the two
//     passes 5.14 ms, bit-identical outputs).
//   Q owner (dQ; q2k lists): the forward's layout. S^T = K Q^T, dP^T = V dO^T, dQ^T += K^T dS^T with K^T through
//     transposed LDS reads. 3 products per pair; dQ is deterministic (no atomics).
// The two partial accumulators of a workgroup (query halves, or key halves) are summed once at the end in LDS.
struct VsaBwdArgs {
  const e16_t *q, *k, *v, *dout;
  const float *lse, *delta;
  const int *row_ptr, *col_idx, *blk_cnt;
  const int4* tasks;
  const int* info;
  const float *add_a, *add_b;  // per-block gradients distributed as add / cnt (KV owner: dK, dV; Q owner: dQ)
  int add_nb;
  e16_t *out_a, *out_b;       // bf16 outputs
  float *out_a32, *out_b32;    // fp32 outputs (KV owner) / accumulator dq_acc += dQ (Q owner)
  float *part_a, *part_b;      // split partials [slot, 64, D]
  int* queues;                 // the eight row-block queue counters of this launch (queues.h)
  int L, NB, BH, per_xcd, fixed;
  float scale_log2, scale;
};

// decode the workgroup's (owner block, head, list range, slot); false = nothing to do
template <bool TASKS>
__device__ __forceinline__ bool owner_of(const VsaBwdArgs& a, int& blk, int& bh, int& beg, int& end, int& slot) {
  slot = -1;
  if (TASKS) {
    if ((int)blockIdx.x >= sload(a.info)) return false;
    const int4 tk = a.tasks[blockIdx.x];
    bh = tk.x / a.NB;
    blk = tk.x - bh * a.NB;
    beg = tk.y;
    end = tk.z;
    slot = tk.w;
  } else {
    if (!balanced_item(a.queues, a.fixed, a.per_xcd, a.BH, a.NB, bh, blk)) return false;
    const int* rp = a.row_ptr + (size_t)bh * (a.NB + 1) + blk;
    beg = sload(rp);
    end = sload(rp + 1);
  }
  beg = __builtin_amdgcn_readfirstlane(beg);
  end = __builtin_amdgcn_readfirstlane(end);
  return true;
}

// lse (natural) -> log2 domain, +inf for rows that must get P = 0
__device__ __forceinline__ float lse_to_log2(float lse) { return lse == -INFINITY ? INFINITY : lse * LOG2E; }

// The KV-owner backward: one 256-thread workgroup per (kv block, head), two per CU. Wave (role, key half): a dV
// wave computes S and P of its 32 keys against the chunk's 64 query rows and dV += P^T dO; a dK wave of the same
// keys computes dP = dO V^T (V in registers), dS from the dV wave's P (handed over as bf16 / fp16 operands through
// LDS) and dK += dS^T Q. Each query block's Q / dO is staged once for both roles: four products per pair, 32
// matrix instructions per wave and chunk, and every wave's accumulators hold the full sums of its keys.
template <bool TASKS, int DH>
__global__ __launch_bounds__(256, 2) void vsa_bwd_kv_kernel(VsaBwdArgs a) {
  constexpr int NKS = DH / 16, NDB = DH / 32;
  __shared__ __attribute__((aligned(16))) char qd_s[2][2][BK * 256];  // [buffer][Q | dO]
  __shared__ __attribute__((aligned(16))) float st_s[2][2][BK];       // [buffer][lse2 (+inf: P = 0) | delta]
  __shared__ ev8 p_s[2][4][64];  // [key half][query half x (first | second 8 rows of a lane)][lane]: the dV waves' P
  int kb, bh, beg, end, slot;
  if (!owner_of<TASKS>(a, kb, bh, beg, end, slot)) return;
  const int nc = end - beg;
  const int tid = threadIdx.x, l = tid & 63, hi = l >> 5, lq = l & 31;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int role = wv >> 1, kh = wv & 1;  // role 0: dV, 1: dK (wave-uniform)
  const int key = 32 * kh + lq;
  const int kcnt = sload(a.blk_cnt + kb);
  const bool kvalid = key < kcnt;
  const size_t head = (size_t)bh * a.L;

  const unsigned head_bytes = (unsigned)((size_t)a.L * HD * 2);
  const srd_t rq = make_srd(a.q + head * HD, head_bytes);
  const srd_t rd = make_srd(a.dout + head * HD, head_bytes);
  unsigned ld_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int P = (wv * 4 + i) * 64 + l, R = P >> 4, g = (P & 15) ^ swz(R);
    ld_off[i] = g < DH / 8 ? (unsigned)R * 256 + (unsigned)(g * 16) : 0x80000000u;
  }
  ev8 kvreg[8];  // this lane's key row: K (dV wave, for S) or V (dK wave, for dP)
  {
    const size_t off = (head + (size_t)kb * BK + key) * HD + 8 * hi;
    const e16_t* src = (role ? a.v : a.k) + off;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) kvreg[ks] = *reinterpret_cast<const ev8*>(src + 16 * ks);
  }
  // stage query block i (Q, dO: 16 rows of each per wave); wave 0 returns lane l's lse2 / delta of row i * 64 + l
  auto issue = [&](int i, int sb, float& ls, float& dl) {
    const unsigned soff = (unsigned)i * (BK * 256);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      dma16(rq, qd_s[sb][0] + wv * 4096 + r * 1024, ld_off[r], soff);
      dma16(rd, qd_s[sb][1] + wv * 4096 + r * 1024, ld_off[r], soff);
    }
    if (wv == 0) {
      const size_t t = head + (size_t)i * BK + l;
      ls = lse_to_log2(a.lse[t]);
      dl = a.delta[t];
    }
  };
  // LDS offsets within a query half (32 rows, 8 KB); the second half adds 8192
  int aoff[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) aoff[ks] = tile_off(lq, 2 * ks + hi);
  int toff[2][4];
  {
    const int g1 = (l >> 4) & 1, sub = (l & 1) * 8, rowA = 4 * hi + ((l & 15) >> 2);
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      toff[0][db] = tile_off(rowA, 4 * db + 2 * g1 + ((l & 3) >> 1)) + sub;
      toff[1][db] = tile_off(rowA + 8, 4 * db + 2 * g1 + ((l & 3) >> 1)) + sub;
    }
  }
  f32x16 acc[4];  // dV (role 0) or dK (role 1) of this lane's key
#pragma unroll
  for (int db = 0; db < 4; ++db) acc[db] = f32x16{};

  float ls = 0.0f, dl = 0.0f;
  int inext = nc > 1 ? sload(a.col_idx + beg + 1) : 0;
  if (nc > 0) {
    issue(sload(a.col_idx + beg), 0, ls, dl);
    dma_wait();
    if (wv == 0) {
      st_s[0][0][l] = ls;
      st_s[0][1][l] = dl;
    }
  }
  dma_wait();
  __syncthreads();
  // masked key columns: every row's lse2 becomes +inf for this lane, so P = 2^(s - inf) = 0 without a branch
  const float kmask = kvalid ? 0.0f : INFINITY;
  ev8* pex = p_s[kh][0];
  for (int j = 0; j < nc; ++j) {
    const int sb = j & 1;
    int inn = 0;
    if (j + 1 < nc) {
      issue(inext, sb ^ 1, ls, dl);
      if (j + 2 < nc) inn = sload(a.col_idx + beg + j + 2);
    }
    const char* qt = qd_s[sb][0];
    const char* dt = qd_s[sb][1];
    f32x16 dp[2];  // dK wave: dP of each query half
    if (role == 0) {
#pragma unroll
      for (int qh = 0; qh < 2; ++qh) {
        f32x16 s = {};
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) s = emfma(elds16(qt, qh * 8192 + aoff[ks]), kvreg[ks], s);
        float p[16];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 l4 = *reinterpret_cast<const f32x4*>(&st_s[sb][0][32 * qh + 8 * g + 4 * hi]);
#pragma unroll
          for (int e = 0; e < 4; ++e) p[4 * g + e] = exp2f_fast(fmaf(s[4 * g + e], a.scale_log2, -(l4[e] + kmask)));
        }
        const ev8 pa = epack8(&p[0]), pb = epack8(&p[8]);
        pex[(2 * qh) * 64 + l] = pa;
        pex[(2 * qh + 1) * 64 + l] = pb;
        // dV += P^T dO (needs nothing from the dK wave, so it runs before the hand-over barrier)
        const char* xt = dt + qh * 8192;
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          acc[db] = emfma(ecat_tr(lds_read_tr(xt, toff[0][db]), lds_read_tr(xt, toff[1][db])), pa, acc[db]);
          acc[db] = emfma(ecat_tr(lds_read_tr(xt + 4096, toff[0][db]), lds_read_tr(xt + 4096, toff[1][db])), pb, acc[db]);
        }
      }
    } else {
#pragma unroll
      for (int qh = 0; qh < 2; ++qh) {
        dp[qh] = f32x16{};
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) dp[qh] = emfma(elds16(dt, qh * 8192 + aoff[ks]), kvreg[ks], dp[qh]);
      }
    }
    __syncthreads();  // P is in LDS
    if (role == 1) {  // dS = P (dP - delta) / sqrt(D), dK += dS^T Q
#pragma unroll
      for (int qh = 0; qh < 2; ++qh) {
        const ev8 pa = pex[(2 * qh) * 64 + l], pb = pex[(2 * qh + 1) * 64 + l];
        float ds[16];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 d4 = *reinterpret_cast<const f32x4*>(&st_s[sb][1][32 * qh + 8 * g + 4 * hi]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = 4 * g + e;
            const float pv = r < 8 ? (float)pa[r] : (float)pb[r - 8];
            ds[r] = pv * (dp[qh][r] - d4[e]) * a.scale;
          }
        }
        const ev8 sa = epack8(&ds[0]), sb8 = epack8(&ds[8]);
        const char* xt = qt + qh * 8192;
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          acc[db] = emfma(ecat_tr(lds_read_tr(xt, toff[0][db]), lds_read_tr(xt, toff[1][db])), sa, acc[db]);
          acc[db] = emfma(ecat_tr(lds_read_tr(xt + 4096, toff[0][db]), lds_read_tr(xt + 4096, toff[1][db])), sb8, acc[db]);
        }
      }
    }
    dma_wait();
    if (j + 1 < nc && wv == 0) {
      st_s[sb ^ 1][0][l] = ls;
      st_s[sb ^ 1][1][l] = dl;
    }
    __syncthreads();
    inext = inn;
  }

#pragma unroll
  for (int db = NDB; db < 4; ++db) acc[db] = f32x16{};  // columns past D: zero
  const size_t tok = head + (size_t)kb * BK + key;
  if (TASKS && slot >= 0) {
    float* pa_out = (role == 0 ? a.part_b : a.part_a) + ((size_t)slot * BK + key) * HD;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<float4*>(pa_out + 32 * db + 8 * i + 4 * hi) =
            make_float4(acc[db][4 * i], acc[db][4 * i + 1], acc[db][4 * i + 2], acc[db][4 * i + 3]);
    return;
  }
  // valid keys: dK or dV + add / cnt; padding keys: 0
  const float inv = kvalid ? 1.0f / (float)kcnt : 0.0f;
  const float keep = kvalid ? 1.0f : 0.0f;
  const float* add = role == 0 ? a.add_b : a.add_a;
  const float* adp = add + ((size_t)bh * a.add_nb + kb) * HD;
  float* out32 = role == 0 ? a.out_b32 : a.out_a32;
  e16_t* out16 = role == 0 ? a.out_b : a.out_a;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = 32 * db + 8 * i + 4 * hi;
      f32x4 x4;
#pragma unroll
      for (int e = 0; e < 4; ++e) x4[e] = acc[db][4 * i + e] * keep;
      if (add != nullptr) x4 += *reinterpret_cast<const f32x4*>(adp + c) * inv;
      if (out32 != nullptr) {
        *reinterpret_cast<f32x4*>(out32 + tok * HD + c) = x4;
      } else {
        ushort4 o4;
        o4.x = f2e(x4[0]); o4.y = f2e(x4[1]); o4.z = f2e(x4[2]); o4.w = f2e(x4[3]);
        *reinterpret_cast<ushort4*>(out16 + tok * HD + c) = o4;
      }
    }
}


template <bool TASKS, int DH>
__global__ __launch_bounds__(256, 2) void vsa_bwd_q_kernel(VsaBwdArgs a) {
  constexpr int NKS = DH / 16, NDB = DH / 32;
  __shared__ __attribute__((aligned(16))) char kv_s[2][2][BK * 256];
  int qb, bh, beg, end, slot;
  if (!owner_of<TASKS>(a, qb, bh, beg, end, slot)) return;
  const int nc = end - beg;
  const int tid = threadIdx.x, l = tid & 63, hi = l >> 5, lq = l & 31;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rg = wv & 1, kh = wv >> 1;
  const int qrow = 32 * rg + lq;
  const int qcnt = sload(a.blk_cnt + qb);
  const bool qvalid = qrow < qcnt;
  const size_t head = (size_t)bh * a.L;
  const size_t tok = head + (size_t)qb * BK + qrow;

  ev8 qreg[8], dreg[8];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
    qreg[ks] = *reinterpret_cast<const ev8*>(a.q + tok * HD + 16 * ks + 8 * hi);
    dreg[ks] = *reinterpret_cast<const ev8*>(a.dout + tok * HD + 16 * ks + 8 * hi);
  }
  const float ls = qvalid ? lse_to_log2(a.lse[tok]) : INFINITY;
  const float dl = a.delta[tok];

  const unsigned head_bytes = (unsigned)((size_t)a.L * HD * 2);
  const srd_t rk = make_srd(a.k + head * HD, head_bytes);
  const srd_t rv = make_srd(a.v + head * HD, head_bytes);
  unsigned ld_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int P = (wv * 4 + i) * 64 + l, R = P >> 4, g = (P & 15) ^ swz(R);
    ld_off[i] = g < DH / 8 ? (unsigned)R * 256 + (unsigned)(g * 16) : 0x80000000u;
  }
  auto issue = [&](int b, int sb) {
    const unsigned soff = (unsigned)b * (BK * 256);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      dma16(rk, kv_s[sb][0] + wv * 4096 + i * 1024, ld_off[i], soff);
      dma16(rv, kv_s[sb][1] + wv * 4096 + i * 1024, ld_off[i], soff);
    }
  };
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
  f32x16 dq[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) dq[db] = f32x16{};

  int bcur = nc > 0 ? sload(a.col_idx + beg) : 0;
  int ccur = nc > 0 ? sload(a.blk_cnt + bcur) : 0;
  int bnext = nc > 1 ? sload(a.col_idx + beg + 1) : 0;
  if (nc > 0) issue(bcur, 0);
  dma_wait();
  __syncthreads();
  for (int j = 0; j < nc; ++j) {
    const int sb = j & 1;
    int cnext = 0, bnn = 0;
    if (j + 1 < nc) {
      issue(bnext, sb ^ 1);
      cnext = sload(a.blk_cnt + bnext);
      if (j + 2 < nc) bnn = sload(a.col_idx + beg + j + 2);
    }
    const char* kt = kv_s[sb][0];
    const char* vt = kv_s[sb][1];
    f32x16 s = {}, dp = {};
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) s = emfma(elds16(kt, koff[ks]), qreg[ks], s);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) dp = emfma(elds16(vt, koff[ks]), dreg[ks], dp);
    float ds[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float kill = 32 * kh + 8 * (r / 4) + 4 * hi + (r % 4) < ccur ? 0.0f : INFINITY;
      const float p = exp2f_fast(fmaf(s[r], a.scale_log2, -(ls + kill)));
      ds[r] = p * (dp[r] - dl) * a.scale;
    }
    const ev8 sa = epack8(&ds[0]), sb8 = epack8(&ds[8]);
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      dq[db] = emfma(ecat_tr(lds_read_tr(kt, toff[0][db]), lds_read_tr(kt, toff[1][db])), sa, dq[db]);
      dq[db] = emfma(ecat_tr(lds_read_tr(kt + 4096, toff[0][db]), lds_read_tr(kt + 4096, toff[1][db])), sb8, dq[db]);
    }
    dma_wait();
    __syncthreads();
    bcur = bnext;
    ccur = cnext;
    bnext = bnn;
  }

  float* xq = reinterpret_cast<float*>(&kv_s[0][0][0]) + rg * (64 * 64);
  if (kh == 1) {
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) xq[(db * 16 + r) * 64 + l] = dq[db][r];
  }
  __syncthreads();
  if (kh == 1) return;
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[db][r] += xq[(db * 16 + r) * 64 + l];
#pragma unroll
  for (int db = NDB; db < 4; ++db) dq[db] = f32x16{};  // columns past D: zero
  if (TASKS && slot >= 0) {
    float* pq = a.part_a + ((size_t)slot * BK + qrow) * HD;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<float4*>(pq + 32 * db + 8 * i + 4 * hi) =
            make_float4(dq[db][4 * i], dq[db][4 * i + 1], dq[db][4 * i + 2], dq[db][4 * i + 3]);
    return;
  }
  const float inv = qvalid ? 1.0f / (float)qcnt : 0.0f;
  const float keep = qvalid ? 1.0f : 0.0f;
  const float* adq = a.add_a + ((size_t)bh * a.add_nb + qb) * HD;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = 32 * db + 8 * i + 4 * hi;
      f32x4 x;
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = dq[db][4 * i + e] * keep;
      if (a.out_a32 != nullptr) {  // dq_acc += dQ (padding rows keep their value)
        f32x4* dst = reinterpret_cast<f32x4*>(a.out_a32 + tok * HD + c);
        *dst = *dst + x;
      } else {
        if (a.add_a != nullptr) x += *reinterpret_cast<const f32x4*>(adq + c) * inv;
        ushort4 q4;
        q4.x = f2e(x[0]); q4.y = f2e(x[1]); q4.z = f2e(x[2]); q4.w = f2e(x[3]);
        *reinterpret_cast<ushort4*>(a.out_a + tok * HD + c) = q4;
      }
    }
}

}  // namespace

}  // namespace es

using namespace es;

static int vsa_check_qkv(const void* q, const void* k, const void* v, int BH, int L, int D) {
  ES_REQUIRE(q && k && v, ES_ERR_INVALID, "VSA: null q / k / v");
  ES_REQUIRE(BH > 0 && L > 0 && L % BK == 0, ES_ERR_INVALID, "VSA: tokens must be [BH, L = NB * 64, D]");
  ES_REQUIRE(D == 64 || D == HD, ES_ERR_UNSUPPORTED, "VSA: head dim must be 64 or 128 (rows stored with 128 columns)");
  ES_REQUIRE((size_t)L * HD * 2 < (1ull << 31), ES_ERR_UNSUPPORTED, "VSA: one head's tokens exceed 2 GiB");
  return ES_OK;
}

static VsaFwdArgs fwd_args(const void* q, const void* k, const void* v, const int* blk_cnt, int BH, int L, int D) {
  VsaFwdArgs a = {};
  a.q = (const e16_t*)q;
  a.k = (const e16_t*)k;
  a.v = (const e16_t*)v;
  a.blk_cnt = blk_cnt;
  a.L = L;
  a.NB = L / BK;
  a.BH = BH;
  a.scale = LOG2E / sqrtf((float)D);  // D: the logical head dimension (64 or 128)
  return a;
}

extern "C" int ES_VSA_API(vsa_attn_fwd)(const void* q, const void* k, const void* v, const int* row_ptr, const int* col_idx,
                            const int* blk_cnt, void* out, float* lse, int BH, int L, int D, hipStream_t stream) {
  if (int st = vsa_check_qkv(q, k, v, BH, L, D)) return st;
  ES_REQUIRE(row_ptr && blk_cnt && out && lse, ES_ERR_INVALID, "VSA: null tensor pointer");
  VsaFwdArgs a = fwd_args(q, k, v, blk_cnt, BH, L, D);
  a.row_ptr = row_ptr;
  a.col_idx = col_idx;
  a.out = (e16_t*)out;
  a.lse = lse;
  a.per_xcd = (a.NB + 7) / 8;
  ES_REQUIRE(8LL * BH * a.per_xcd < (1LL << 30), ES_ERR_UNSUPPORTED, "VSA: grid too large");
  Queues qs;
  ES_REQUIRE(balanced_launch(BH, a.per_xcd, stream, qs), ES_ERR_LAUNCH, "VSA: row-block queues unavailable");
  a.queues = qs.counters;
  a.fixed = qs.fixed;
  if (D == 64) hipLaunchKernelGGL((vsa_fwd_kernel<false, 64>), dim3((unsigned)qs.grid), dim3(256), 0, stream, a);
  else hipLaunchKernelGGL((vsa_fwd_kernel<false, 128>), dim3((unsigned)qs.grid), dim3(256), 0, stream, a);
  return check_launch("vsa_attn_fwd");
}

extern "C" int ES_VSA_API(vsa_attn_fwd_tasks)(const void* q, const void* k, const void* v, const int* col_idx,
                                  const int* blk_cnt, const int* tasks, const int* info, int max_tasks, void* out,
                                  float* lse, float* part_o, float* part_lse, int BH, int L, int D,
                                  hipStream_t stream) {
  if (int st = vsa_check_qkv(q, k, v, BH, L, D)) return st;
  // part_o / part_lse may be null when the plan has no split slots (no task then writes a partial)
  ES_REQUIRE(blk_cnt && tasks && info && out && lse, ES_ERR_INVALID, "VSA: null tensor pointer");
  ES_REQUIRE(max_tasks >= 0, ES_ERR_INVALID, "VSA: negative task capacity");
  if (max_tasks == 0) return ES_OK;
  VsaFwdArgs a = fwd_args(q, k, v, blk_cnt, BH, L, D);
  a.col_idx = col_idx;
  a.tasks = (const int4*)tasks;
  a.info = info;
  a.out = (e16_t*)out;
  a.lse = lse;
  a.part_o = part_o;
  a.part_lse = part_lse;
  if (D == 64) hipLaunchKernelGGL((vsa_fwd_kernel<true, 64>), dim3((unsigned)max_tasks), dim3(256), 0, stream, a);
  else hipLaunchKernelGGL((vsa_fwd_kernel<true, 128>), dim3((unsigned)max_tasks), dim3(256), 0, stream, a);
  return check_launch("vsa_attn_fwd_tasks");
}


static VsaBwdArgs bwd_args(const void* q, const void* k, const void* v, const void* dout, const float* lse,
                           const float* delta, const int* blk_cnt, int BH, int L, int D) {
  VsaBwdArgs a = {};
  a.q = (const e16_t*)q;
  a.k = (const e16_t*)k;
  a.v = (const e16_t*)v;
  a.dout = (const e16_t*)dout;
  a.lse = lse;
  a.delta = delta;
  a.blk_cnt = blk_cnt;
  a.L = L;
  a.NB = L / BK;
  a.BH = BH;
  a.per_xcd = (a.NB + 7) / 8;
  a.scale = 1.0f / sqrtf((float)D);
  a.scale_log2 = LOG2E / sqrtf((float)D);
  return a;
}

extern "C" int ES_VSA_API(vsa_attn_bwd_kv)(const void* q, const void* k, const void* v, const void* dout, const float* lse,
                               const float* delta, const int* k2q_ptr, const int* k2q_idx, const int* blk_cnt,
                               const float* add_dk, const float* add_dv, int add_nb, void* dk, void* dv,
                               int out_fp32, int BH, int L, int D, hipStream_t stream) {
  if (int st = vsa_check_qkv(q, k, v, BH, L, D)) return st;
  ES_REQUIRE(dout && lse && delta && k2q_ptr && blk_cnt && dk && dv, ES_ERR_INVALID, "VSA: null tensor pointer");
  ES_REQUIRE((add_dk == nullptr && add_dv == nullptr) || add_nb >= L / BK, ES_ERR_INVALID,
             "VSA: per-block gradient has fewer rows than blocks");
  VsaBwdArgs a = bwd_args(q, k, v, dout, lse, delta, blk_cnt, BH, L, D);
  a.row_ptr = k2q_ptr;
  a.col_idx = k2q_idx;
  a.add_a = add_dk;
  a.add_b = add_dv;
  a.add_nb = add_nb;
  if (out_fp32) {
    a.out_a32 = (float*)dk;
    a.out_b32 = (float*)dv;
  } else {
    a.out_a = (e16_t*)dk;
    a.out_b = (e16_t*)dv;
  }
  ES_REQUIRE(8LL * BH * a.per_xcd < (1LL << 30), ES_ERR_UNSUPPORTED, "VSA: grid too large");
  Queues qs;
  ES_REQUIRE(balanced_launch(BH, a.per_xcd, stream, qs), ES_ERR_LAUNCH, "VSA: row-block queues unavailable");
  a.queues = qs.counters;
  a.fixed = qs.fixed;
  if (D == 64) hipLaunchKernelGGL((vsa_bwd_kv_kernel<false, 64>), dim3((unsigned)qs.grid), dim3(256), 0, stream, a);
  else hipLaunchKernelGGL((vsa_bwd_kv_kernel<false, 128>), dim3((unsigned)qs.grid), dim3(256), 0, stream, a);
  return check_launch("vsa_attn_bwd_kv");
}

extern "C" int ES_VSA_API(vsa_attn_bwd_kv_tasks)(const void* q, const void* k, const void* v, const void* dout, const float* lse,
                                     const float* delta, const int* k2q_idx, const int* blk_cnt, const int* tasks,
                                     const int* info, int max_tasks, const float* add_dk, const float* add_dv,
                                     int add_nb, void* dk, void* dv, float* part_dk, float* part_dv, int BH, int L,
                                     int D, hipStream_t stream) {
  if (int st = vsa_check_qkv(q, k, v, BH, L, D)) return st;
  ES_REQUIRE(dout && lse && delta && blk_cnt && tasks && info && dk && dv, ES_ERR_INVALID, "VSA: null tensor pointer");
  ES_REQUIRE(max_tasks >= 0, ES_ERR_INVALID, "VSA: negative task capacity");
  if (max_tasks == 0) return ES_OK;
  VsaBwdArgs a = bwd_args(q, k, v, dout, lse, delta, blk_cnt, BH, L, D);
  a.col_idx = k2q_idx;
  a.tasks = (const int4*)tasks;
  a.info = info;
  a.add_a = add_dk;
  a.add_b = add_dv;
  a.add_nb = add_nb;
  a.out_a = (e16_t*)dk;
  a.out_b = (e16_t*)dv;
  a.part_a = part_dk;
  a.part_b = part_dv;
  if (D == 64) hipLaunchKernelGGL((vsa_bwd_kv_kernel<true, 64>), dim3((unsigned)max_tasks), dim3(256), 0, stream, a);
  else hipLaunchKernelGGL((vsa_bwd_kv_kernel<true, 128>), dim3((unsigned)max_tasks), dim3(256), 0, stream, a);
  return check_launch("vsa_attn_bwd_kv_tasks");
}

extern "C" int ES_VSA_API(vsa_attn_bwd_q)(const void* q, const void* k, const void* v, const void* dout, const float* lse,
                              const float* delta, const int* q2k_ptr, const int* q2k_idx, const int* blk_cnt,
                              const float* add_dq, int add_nb, void* dq, float* dq_acc, int BH, int L, int D,
                              hipStream_t stream) {
  if (int st = vsa_check_qkv(q, k, v, BH, L, D)) return st;
  ES_REQUIRE(dout && lse && delta && q2k_ptr && blk_cnt && (dq || dq_acc), ES_ERR_INVALID, "VSA: null tensor pointer");
  ES_REQUIRE(add_dq == nullptr || add_nb >= L / BK, ES_ERR_INVALID, "VSA: per-block gradient has fewer rows than blocks");
  VsaBwdArgs a = bwd_args(q, k, v, dout, lse, delta, blk_cnt, BH, L, D);
  a.row_ptr = q2k_ptr;
  a.col_idx = q2k_idx;
  a.add_a = add_dq;
  a.add_nb = add_nb;
  a.out_a = (e16_t*)dq;
  a.out_a32 = dq_acc;
  ES_REQUIRE(8LL * BH * a.per_xcd < (1LL << 30), ES_ERR_UNSUPPORTED, "VSA: grid too large");
  Queues qs;
  ES_REQUIRE(balanced_launch(BH, a.per_xcd, stream, qs), ES_ERR_LAUNCH, "VSA: row-block queues unavailable");
  a.queues = qs.counters;
  a.fixed = qs.fixed;
  if (D == 64) hipLaunchKernelGGL((vsa_bwd_q_kernel<false, 64>), dim3((unsigned)qs.grid), dim3(256), 0, stream, a);
  else hipLaunchKernelGGL((vsa_bwd_q_kernel<false, 128>), dim3((unsigned)qs.grid), dim3(256), 0, stream, a);
  return check_launch("vsa_attn_bwd_q");
}

extern "C" int ES_VSA_API(vsa_attn_bwd_q_tasks)(const void* q, const void* k, const void* v, const void* dout, const float* lse,
                                    const float* delta, const int* q2k_idx, const int* blk_cnt, const int* tasks,
                                    const int* info, int max_tasks, const float* add_dq, int add_nb, void* dq,
                                    float* part_dq, int BH, int L, int D, hipStream_t stream) {
  if (int st = vsa_check_qkv(q, k, v, BH, L, D)) return st;
  ES_REQUIRE(dout && lse && delta && blk_cnt && tasks && info && dq, ES_ERR_INVALID, "VSA: null tensor pointer");
  ES_REQUIRE(max_tasks >= 0, ES_ERR_INVALID, "VSA: negative task capacity");
  if (max_tasks == 0) return ES_OK;
  VsaBwdArgs a = bwd_args(q, k, v, dout, lse, delta, blk_cnt, BH, L, D);
  a.col_idx = q2k_idx;
  a.tasks = (const int4*)tasks;
  a.info = info;
  a.add_a = add_dq;
  a.add_nb = add_nb;
  a.out_a = (e16_t*)dq;
  a.part_a = part_dq;
  if (D == 64) hipLaunchKernelGGL((vsa_bwd_q_kernel<true, 64>), dim3((unsigned)max_tasks), dim3(256), 0, stream, a);
  else hipLaunchKernelGGL((vsa_bwd_q_kernel<true, 128>), dim3((unsigned)max_tasks), dim3(256), 0, stream, a);
  return check_launch("vsa_attn_bwd_q_tasks");
}
