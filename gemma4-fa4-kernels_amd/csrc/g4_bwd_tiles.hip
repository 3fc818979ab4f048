// Backward MFMA kernels for gfx950: dK/dV (key-tile major) and dQ (query-tile major).
//
// Both recompute P = exp2(S log2e - LSE log2e) from the saved fp32 LSE and use
// delta = rowsum(O dO) - dLSE from the pre-pass: dS = P (dP - delta), with
// S = Q K^T and dP = dO V^T (softmax scale 1.0).  P and dS are rounded to bf16
// before they feed the dV / dK / dQ products.  No atomics: each output element
// is owned by one wave, so results repeat bitwise.
//
// dK/dV: a workgroup owns NKB * 32 keys of one KV head and loops over the
// query heads of its GQA group and the query tiles (32 rows) the mask admits
// (key_tile_query_range).  Lanes own keys: S and dP come out of the MFMA with
// keys along lanes, so P and dS feed dV^T += dO^T P and dK^T += Q^T dS directly
// from registers, with dO^T / Q^T read from the natural-layout tiles by
// transposing LDS reads.  K and V fragments stay in VGPRs for the whole loop.
//
// dQ: a workgroup owns 32 * NQG queries of one query head and walks the key
// tiles of its range like the forward: S^T = K Q^T and dP^T = V dO^T with
// lanes owning queries, dQ^T += K^T dS^T with K^T from transposing reads.
//
// With DSPLIT = 2 (head dim 512) the two waves of a pair own the two halves of
// the head dimension and exchange their partial S / dP through LDS.
#include "g4_kernels.h"

namespace g4 {

namespace {

__device__ __forceinline__ void xchg_write(char G4_LDS* xb, int slot, int lane, const f32x16& v) {
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4) {
    f32x4 w = {v[q4 * 4], v[q4 * 4 + 1], v[q4 * 4 + 2], v[q4 * 4 + 3]};
    *(f32x4 G4_LDS*)(xb + ((slot * 4 + q4) * 64 + lane) * 16) = w;
  }
}

// acc = (slice 0 partial) + (slice 1 partial), summed in the same order by both
// slices so they hold bit-identical values.
__device__ __forceinline__ void xchg_add(const char G4_LDS* xb, int slot, int lane, int dh,
                                         f32x16& acc) {
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4) {
    f32x4 w = *(const f32x4 G4_LDS*)(xb + ((slot * 4 + q4) * 64 + lane) * 16);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float mine = acc[q4 * 4 + e];
      acc[q4 * 4 + e] = dh == 0 ? mine + w[e] : w[e] + mine;
    }
  }
}

}  // namespace

// ===========================================================================
// dK / dV
// ===========================================================================

template <int D, int DSPLIT, int NKB, bool DV, bool DK, int KPW>
struct DkdvCfg {
  static constexpr int kNW = NKB * DSPLIT;
  static constexpr int kNT = kNW * 64;
  static constexpr int kBN = NKB * KPW * 32;  // keys per workgroup
  static constexpr int kBM = 32;              // queries per step
  static constexpr int kDH = D / DSPLIT;
  static constexpr int kCPR = D / 8;
  static constexpr int kTile = kBM * D * 2;  // Q or dO tile bytes
  // Partial score tiles each wave of a head-dim pair exports per key block:
  // S, and dP when the launch computes dK.
  static constexpr int kXPer = DSPLIT > 1 ? (DK ? 2 : 1) : 0;
  static constexpr int kXBytes = kNW * KPW * kXPer * 4096;
  // With a head-dim pair exchange, a tile no MFMA reads after the exchange
  // (Q without dK, dO without dV) is single-buffered and refilled as soon as
  // the exchange barrier retires its reads; otherwise tiles are double-buffered
  // and refilled at the top of the step.
  static constexpr bool kQDouble = DSPLIT == 1 || DK;
  static constexpr bool kDoDouble = DSPLIT == 1 || DV;
  static constexpr int kLdsQ = 0;
  static constexpr int kLdsDo = kLdsQ + (kQDouble ? 2 : 1) * kTile;
  static constexpr int kLdsX = kLdsDo + (kDoDouble ? 2 : 1) * kTile;
  static constexpr int kLdsLd = kLdsX + kXBytes;    // [buf][lse x 32 | delta x 32] fp32
  static constexpr int kLdsMeta = kLdsLd + 2 * 256;  // [buf][vid x 32 | doc x 32] int32
  static constexpr int kLdsRed = kLdsMeta + 2 * 256;
  static constexpr int kLdsBytes = kLdsRed + 64;
  static_assert(kLdsBytes <= 160 * 1024, "LDS budget");
};

// DV / DK select the outputs of a launch: both in one pass, or (when the
// combined live state does not fit the register file) a dV-only pass (S, P,
// dV) and a dK-only pass (S, dP, dS, dK).
// KPW key blocks of 32 per wave: each Q / dO fragment read from LDS feeds KPW
// MFMAs (one per key block), at KPW times the accumulator registers.
template <int D, int DSPLIT, int NKB, bool META, bool DV, bool DK, int KPW>
struct DkdvKernel {
  using C = DkdvCfg<D, DSPLIT, NKB, DV, DK, KPW>;
  static constexpr int kNB = C::kDH / 32;
  static constexpr int kNC = C::kDH / 16;

  char G4_LDS* smem;
  const BwdParams* a;
  Seq sq;
  int s, lane, wave, dh, h32, kb;
  int off, j0;
  int my_j[KPW];
  bool has_vid, has_doc, has_meta;
  int my_vid[KPW], my_doc[KPW];
  int grp, kvh, qt_lo, nqt;
  int64_t tq;
  RowReader<C::kCPR> rrd;
  TrReader<C::kCPR> trd;
  using Copier = TileCopier<C::kCPR, 32, C::kNW>;
  Copier qcp, docp;
  bf16x8 kf[KPW][kNC];
  bf16x8 vf[KPW][DK ? kNC : 1];
  f32x16 dk_acc[KPW][DK ? kNB : 1], dv_acc[KPW][DV ? kNB : 1];

  // Step `it` enumerates (query tile, query head) pairs, query tiles from the
  // last one down and the GQA group's heads innermost: every workgroup starts
  // at the top query tile, so concurrently running workgroups of one KV head
  // stream the same Q / dO tiles at about the same time and share them in L2.
  __device__ __forceinline__ void coords(int it, int& qh, int& i0) const {
    // grp is 1, 2, 4 or 8 (validated GQA ratios): shifts, no integer division
    const int sh = __builtin_ctz(grp);
    qh = kvh * grp + (it & (grp - 1));
    i0 = (qt_lo + nqt - 1 - (it >> sh)) * C::kBM;
  }

  __device__ __forceinline__ void issue_q(int it, int buf) {
    int qh, i0;
    coords(it, qh, i0);
    const __bf16* base = a->q + tok_off(sq, s, sq.qtok, i0, a->ql) + (int64_t)qh * a->ql.head_stride;
    char G4_LDS* dst = smem + C::kLdsQ + (C::kQDouble ? buf : 0) * C::kTile;
    if (i0 + C::kBM <= sq.lq)
      qcp.issue(base, dst);
    else
      qcp.issue_clamped(base, a->ql.token_stride, sq.lq - i0, dst, wave, lane);
  }
  __device__ __forceinline__ void issue_do(int it, int buf) {
    int qh, i0;
    coords(it, qh, i0);
    const __bf16* base =
        a->dout + tok_off(sq, s, sq.qtok, i0, a->dol) + (int64_t)qh * a->dol.head_stride;
    char G4_LDS* dst = smem + C::kLdsDo + (C::kDoDouble ? buf : 0) * C::kTile;
    if (i0 + C::kBM <= sq.lq)
      docp.issue(base, dst);
    else
      docp.issue_clamped(base, a->dol.token_stride, sq.lq - i0, dst, wave, lane);
  }
  // LSE (lanes 0-31) and delta (lanes 32-63) of the tile's 32 rows, and with
  // metadata the vision / document IDs of the rows' K positions.
  __device__ __forceinline__ void issue_rows(int it, int buf) {
    int qh, i0;
    coords(it, qh, i0);
    // Each half-wave copies from one array (uniform base pointer, exec-masked
    // issue); lane l lands in LDS slot l either way.
    const int i = min(i0 + (lane & 31), sq.lq - 1);
    if (wave == 0) {
      char G4_LDS* dst = smem + C::kLdsLd + buf * 256;
      if (lane < 32)
        g2l4(a->lse + lse_off(a->p, sq, s, qh, i), dst);
      else
        g2l4(a->delta + (int64_t)qh * tq + sq.qtok + i, dst);
    } else if (wave == 1 && has_meta) {
      char G4_LDS* dst = smem + C::kLdsMeta + buf * 256;
      const int64_t kidx = sq.ktok + i + off;
      if (lane < 32) {
        if (has_vid) g2l4(a->p.vision_ids + kidx, dst);
      } else {
        if (has_doc) g2l4(a->p.document_ids + kidx, dst);
      }
    }
  }

  template <int CP>
  __device__ __forceinline__ void sdp_step(const char G4_LDS* qt, const char G4_LDS* dot,
                                           f32x16 (&sacc)[KPW], f32x16 (&pacc)[KPW]) const {
    if constexpr (CP < kNC) {
      bf16x8 qa = rrd.template read<0, 0, CP>(qt);
#pragma unroll
      for (int kp = 0; kp < KPW; ++kp) sacc[kp] = mfma32(qa, kf[kp][CP], sacc[kp]);
      if constexpr (DK) {
        bf16x8 da = rrd.template read<0, 0, CP>(dot);
#pragma unroll
        for (int kp = 0; kp < KPW; ++kp) pacc[kp] = mfma32(da, vf[kp][CP], pacc[kp]);
      }
      sdp_step<CP + 1>(qt, dot, sacc, pacc);
    }
  }

  template <int M, int B>
  __device__ __forceinline__ void acc_step(const char G4_LDS* t, const bf16x8 (&b)[KPW][2],
                                           f32x16 (&acc)[KPW][kNB]) const {
    if constexpr (B < kNB) {
      bf16x8 x = trd.template read<16 * M, 0, B>(t);
#pragma unroll
      for (int kp = 0; kp < KPW; ++kp) acc[kp][B] = mfma32(x, b[kp][M], acc[kp][B]);
      acc_step<M, B + 1>(t, b, acc);
    }
  }

  // P (and dS) of the lane's 16 * KPW scores; rows (queries) of the
  // accumulators are 8 (r >> 2) + 4 h32 + (r & 3).  MASKED applies the Gemma
  // predicate (tiles the mask does not fully admit).
  // Row LSE / delta come from `lse_r` / `del_r` (read ahead) with a head-dim
  // pair exchange, else straight from the LDS row buffer `ld`.  MODE 0: no
  // mask; 1: mask; 2: mask unless `full` (one code path, fewer registers).
  template <int MODE>
  __device__ __forceinline__ void probs(int cur, int i0, bool full, const float* ld,
                                        const f32x4 (&lse_r)[4], const f32x4 (&del_r)[4],
                                        const f32x16 (&sacc)[KPW], const f32x16 (&pacc)[KPW],
                                        bf16x8 (&pb)[KPW][2], bf16x8 (&db)[KPW][2]) const {
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const int il0 = 8 * r4 + 4 * h32;
      f32x4 lse4, del4;
      if constexpr (DSPLIT > 1) {
        lse4 = lse_r[r4];
        del4 = del_r[r4];
      } else {
        lse4 = *(const f32x4*)(ld + il0);
        del4 = *(const f32x4*)(ld + 32 + il0);
      }
      i32x4 vq4 = {-1, -1, -1, -1}, dq4 = {0, 0, 0, 0};
      if (MODE != 0 && has_meta && !(MODE == 2 && full)) {
        const int* mt = (const int*)(smem + C::kLdsMeta + cur * 256);
        vq4 = *(const i32x4*)(mt + il0);
        dq4 = *(const i32x4*)(mt + 32 + il0);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = r4 * 4 + e;
#pragma unroll
        for (int kp = 0; kp < KPW; ++kp) {
          float p = fast_exp2(sacc[kp][r] * kLog2e - lse4[e] * kLog2e);
          if (MODE == 1 || (MODE == 2 && !full)) {
            const int i = i0 + il0 + e;
            const int aq = i + off;
            const int j = my_j[kp];
            const bool in_w = a->p.window <= 0 || j > aq - a->p.window;
            const bool causal = j <= aq;
            const bool vis = has_vid & (vq4[e] >= 0) & (vq4[e] == my_vid[kp]);
            const bool doc_ok = !has_doc | (dq4[e] == my_doc[kp]);
            const bool ok = (i < sq.lq) & (j < sq.lk) & in_w & (causal | vis) & doc_ok;
            p = ok ? p : 0.f;
          }
          if constexpr (DV) pb[kp][r >> 3][r & 7] = (__bf16)p;
          if constexpr (DK) db[kp][r >> 3][r & 7] = (__bf16)(p * (pacc[kp][r] - del4[e]));
        }
      }
    }
  }

  __device__ __forceinline__ void step(int cur, int it, int nsteps) {
    int qh, i0;
    coords(it, qh, i0);
    // Every copy for this step (Q, row data, dO) has landed in every wave;
    // every wave is done with the buffers refilled below.
    vm_wait<0>();
    barrier_lds();
    if (it + 1 < nsteps) {
      if constexpr (C::kQDouble) issue_q(it + 1, cur ^ 1);
      issue_rows(it + 1, cur ^ 1);
      if constexpr (C::kDoDouble) issue_do(it + 1, cur ^ 1);
    }
    const char G4_LDS* qt = smem + C::kLdsQ + (C::kQDouble ? cur : 0) * C::kTile;
    const char G4_LDS* dot = smem + C::kLdsDo + (C::kDoDouble ? cur : 0) * C::kTile;

    __builtin_amdgcn_sched_barrier(0);
    f32x16 sacc[KPW], pacc[KPW];
#pragma unroll
    for (int kp = 0; kp < KPW; ++kp) sacc[kp] = pacc[kp] = f32x16{};
    sdp_step<0>(qt, dot, sacc, pacc);
    mfma_read_hint<(DK ? 2 : 1) * kNC, KPW, 1, 3>();
    __builtin_amdgcn_sched_barrier(0);

    // Row LSE (pre-scaled to log2) and delta, read with the partner partials
    // so one LDS wait covers both.
    const float* ld = (const float*)(smem + C::kLdsLd + cur * 256);
    f32x4 lse_r[4], del_r[4];
    if constexpr (DSPLIT > 1) {
      char G4_LDS* xb = smem + C::kLdsX;
#pragma unroll
      for (int kp = 0; kp < KPW; ++kp) {
        xchg_write(xb, (wave * KPW + kp) * C::kXPer, lane, sacc[kp]);
        if constexpr (DK) xchg_write(xb, (wave * KPW + kp) * C::kXPer + 1, lane, pacc[kp]);
      }
      barrier_lds();
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        lse_r[r4] = *(const f32x4*)(ld + 8 * r4 + 4 * h32);
        if constexpr (DK) del_r[r4] = *(const f32x4*)(ld + 32 + 8 * r4 + 4 * h32);
      }
      // Single-buffered tiles: every wave's reads of them are retired.
      if (it + 1 < nsteps) {
        if constexpr (!C::kQDouble) issue_q(it + 1, 0);
        if constexpr (!C::kDoDouble) issue_do(it + 1, 0);
      }
#pragma unroll
      for (int kp = 0; kp < KPW; ++kp) {
        xchg_add(xb, ((wave ^ 1) * KPW + kp) * C::kXPer, lane, dh, sacc[kp]);
        if constexpr (DK) xchg_add(xb, ((wave ^ 1) * KPW + kp) * C::kXPer + 1, lane, dh, pacc[kp]);
      }
    }

    const bool full = !has_doc && (i0 + C::kBM <= sq.lq) && (j0 + C::kBN <= sq.lk) &&
                      (j0 + C::kBN - 1 <= i0 + off) &&
                      (a->p.window <= 0 || j0 > i0 + C::kBM - 1 + off - a->p.window);
    bf16x8 pb[KPW][2], db[KPW][2];
    if constexpr (DSPLIT == 1)
      probs<2>(cur, i0, full, ld, lse_r, del_r, sacc, pacc, pb, db);
    else if (full)
      probs<0>(cur, i0, full, ld, lse_r, del_r, sacc, pacc, pb, db);
    else
      probs<1>(cur, i0, full, ld, lse_r, del_r, sacc, pacc, pb, db);

    __builtin_amdgcn_sched_barrier(0);
    if constexpr (DV) {
      acc_step<0, 0>(dot, pb, dv_acc);
      acc_step<1, 0>(dot, pb, dv_acc);
      mfma_read_hint<2 * kNB, KPW, 2, 6>();
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (DK) {
      acc_step<0, 0>(qt, db, dk_acc);
      acc_step<1, 0>(qt, db, dk_acc);
      mfma_read_hint<2 * kNB, KPW, 2, 6>();
    }
    __builtin_amdgcn_sched_barrier(0);
  }
};

template <int D, int DSPLIT, int NKB, bool META, bool DV, bool DK, int KPW>
__global__ void __launch_bounds__(NKB * DSPLIT * 64, 1) dkdv_kernel(BwdParams a) {
  using K = DkdvKernel<D, DSPLIT, NKB, META, DV, DK, KPW>;
  using C = typename K::C;
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  K ker;
  ker.smem = (char G4_LDS*)smem_raw;
  ker.a = &a;
  const g4_problem& p = a.p;
  const int tid = threadIdx.x;
  ker.lane = tid & 63;
  ker.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  ker.kb = ker.wave / DSPLIT;
  ker.dh = ker.wave % DSPLIT;
  ker.h32 = ker.lane >> 5;
  const int l32 = ker.lane & 31;

  // ---- work item: (sequence, key tile, KV head) ------------------------------
  ker.grp = p.num_q_heads / p.num_kv_heads;
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int per_kvh = a.num_seqs * a.ntiles;
  ker.kvh = L / per_kvh;
  const int rank = L % per_kvh;
  ker.s = rank / a.ntiles;
  const int kt = zigzag(rank % a.ntiles, a.ntiles);
  ker.sq = resolve_seq(p, ker.s);
  const Seq& sq = ker.sq;
  ker.j0 = kt * C::kBN;
  if (ker.j0 >= sq.lk) return;
  ker.off = sq.lk - sq.lq;
  ker.tq = q_stream_tokens_dev(p);
  ker.has_vid = META && p.vision_ids != nullptr && p.bidirectional_vision;
  ker.has_doc = META && p.document_ids != nullptr;
  ker.has_meta = ker.has_vid || ker.has_doc;
  const int j_last = min(ker.j0 + C::kBN, sq.lk) - 1;
#pragma unroll
  for (int kp = 0; kp < KPW; ++kp) ker.my_j[kp] = ker.j0 + (ker.kb * KPW + kp) * 32 + l32;

  // ---- query range of this key tile ---------------------------------------
  int span_min = 0x7fffffff;
  if (ker.has_vid) {
    int* red = (int*)(smem_raw + C::kLdsRed);
    int v = 0x7fffffff;
    for (int t = tid; t < C::kBN; t += C::kNT) {
      int j = ker.j0 + t;
      if (j < sq.lk) v = min(v, a.span_lo[sq.ktok + j]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
    if (ker.lane == 0) red[ker.wave] = v;
    barrier_lds();
#pragma unroll
    for (int w = 0; w < C::kNW; ++w) span_min = min(span_min, red[w]);
  }
  int ilo, ihi;
  key_tile_query_range(ker.j0, j_last, sq.lq, ker.off, p.window, span_min, ilo, ihi);
  ker.qt_lo = ilo / C::kBM;
  ker.nqt = ihi > ilo ? (ihi + C::kBM - 1) / C::kBM - ker.qt_lo : 0;
  if (ker.has_doc && ker.nqt > 0 &&
      doc_uniform<C::kNW>(p.document_ids, sq.ktok, sq.lk,
                          min(ker.j0, ker.qt_lo * C::kBM + ker.off),
                          max(j_last + 1, (ker.qt_lo + ker.nqt) * C::kBM + ker.off), tid,
                          ker.lane, ker.wave, (int*)(smem_raw + C::kLdsRed))) {
    ker.has_doc = false;
    ker.has_meta = ker.has_vid;
  }
  const int nsteps = ker.nqt * ker.grp;

  ker.rrd.init(ker.lane, ker.dh * C::kDH * 2);
  ker.trd.init(ker.lane, ker.dh * C::kDH * 2);
  ker.qcp.init(a.ql.token_stride, ker.wave, ker.lane);
  ker.docp.init(a.dol.token_stride, ker.wave, ker.lane);

  // ---- K / V fragments of this wave's KPW * 32 keys (B operands) ----------
#pragma unroll
  for (int kp = 0; kp < KPW; ++kp) {
    const int jc = min(ker.my_j[kp], sq.lk - 1);
    const __bf16* krow = a.k + tok_off(sq, ker.s, sq.ktok, jc, a.kl) +
                         (int64_t)ker.kvh * a.kl.head_stride + ker.dh * C::kDH + ker.h32 * 8;
    const __bf16* vrow = a.v + tok_off(sq, ker.s, sq.ktok, jc, a.vl) +
                         (int64_t)ker.kvh * a.vl.head_stride + ker.dh * C::kDH + ker.h32 * 8;
#pragma unroll
    for (int c = 0; c < K::kNC; ++c) {
      ker.kf[kp][c] = ld_global16(krow + c * 16);
      if constexpr (DK) ker.vf[kp][c] = ld_global16(vrow + c * 16);
    }
    ker.my_vid[kp] = ker.has_vid ? p.vision_ids[sq.ktok + jc] : -1;
    ker.my_doc[kp] = ker.has_doc ? p.document_ids[sq.ktok + jc] : 0;
#pragma unroll
    for (int b = 0; b < K::kNB; ++b) {
      if constexpr (DK) ker.dk_acc[kp][b] = f32x16{};
      if constexpr (DV) ker.dv_acc[kp][b] = f32x16{};
    }
  }

  if (nsteps > 0) {
    ker.issue_q(0, 0);
    ker.issue_rows(0, 0);
    ker.issue_do(0, 0);
  }
  for (int it = 0; it < nsteps; ++it) {
    ker.step(it & 1, it, nsteps);
  }

  // ---- write dK, dV (bf16), 4 consecutive head-dim elements per store --------
#pragma unroll
  for (int kp = 0; kp < KPW; ++kp) {
    const int j = ker.my_j[kp];
    if (j >= sq.lk) continue;
    __bf16* dkrow = a.dk + tok_off(sq, ker.s, sq.ktok, j, a.dkl) +
                    (int64_t)ker.kvh * a.dkl.head_stride;
    __bf16* dvrow = a.dv + tok_off(sq, ker.s, sq.ktok, j, a.dvl) +
                    (int64_t)ker.kvh * a.dvl.head_stride;
#pragma unroll
    for (int b = 0; b < K::kNB; ++b)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d = ker.dh * C::kDH + b * 32 + 8 * r4 + 4 * ker.h32;
        if constexpr (DK) {
          const f32x16& x = ker.dk_acc[kp][b];
          *(bf16x4*)(dkrow + d) = bf16x4{(__bf16)x[r4 * 4], (__bf16)x[r4 * 4 + 1],
                                         (__bf16)x[r4 * 4 + 2], (__bf16)x[r4 * 4 + 3]};
        }
        if constexpr (DV) {
          const f32x16& y = ker.dv_acc[kp][b];
          *(bf16x4*)(dvrow + d) = bf16x4{(__bf16)y[r4 * 4], (__bf16)y[r4 * 4 + 1],
                                         (__bf16)y[r4 * 4 + 2], (__bf16)y[r4 * 4 + 3]};
        }
      }
  }
}

// ===========================================================================
// dQ
// ===========================================================================

template <int D, int BN, int DSPLIT, int NQG, bool VDOUBLE>
struct DqCfg {
  static constexpr int kNW = NQG * DSPLIT;
  static constexpr int kNT = kNW * 64;
  static constexpr int kBM = NQG * 32;
  static constexpr int kDH = D / DSPLIT;
  static constexpr int kCPR = D / 8;
  static constexpr int kTile = BN * D * 2;
  static constexpr int kKB = BN / 32;
  static constexpr int kXBytes = DSPLIT > 1 ? kNW * kKB * 2 * 4096 : 0;
  static constexpr int kLdsK = 0;
  static constexpr int kLdsV = kLdsK + 2 * kTile;
  static constexpr int kLdsX = kLdsV + (VDOUBLE ? 2 : 1) * kTile;
  static constexpr int kLdsMeta = kLdsX + kXBytes;  // [buf][vid x 64 | doc x 64] int32
  static constexpr int kLdsRed = kLdsMeta + 2 * 512;
  static constexpr int kLdsBytes = kLdsRed + 64;
  static_assert(kLdsBytes <= 160 * 1024, "LDS budget");
};

template <int D, int BN, int DSPLIT, int NQG, bool VDOUBLE, bool META>
struct DqKernel {
  using C = DqCfg<D, BN, DSPLIT, NQG, VDOUBLE>;
  static constexpr int kNB = C::kDH / 32;
  static constexpr int kNC = C::kDH / 16;

  char G4_LDS* smem;
  const BwdParams* a;
  Seq sq;
  int lane, wave, dh, h32;
  int my_a, my_vid, my_doc, a0;
  bool has_vid, has_doc, has_meta, q_valid;
  float my_lse2, my_delta;
  const __bf16* kbase;
  const __bf16* vbase;
  int64_t kstride, vstride;
  RowReader<C::kCPR> rrd;
  TrReader<C::kCPR> trd;
  TileCopier<C::kCPR, BN, C::kNW> kcp, vcp;
  bf16x8 qf[kNC], gf[kNC];
  f32x16 dq_acc[kNB];

  __device__ __forceinline__ void issue_k(int row0, int buf) {
    char G4_LDS* dst = smem + C::kLdsK + buf * C::kTile;
    if (row0 + BN <= sq.lk)
      kcp.issue(kbase + row0 * kstride, dst);
    else
      kcp.issue_clamped(kbase + row0 * kstride, kstride, sq.lk - row0, dst, wave, lane);
  }
  __device__ __forceinline__ void issue_v(int row0, int buf) {
    char G4_LDS* dst = smem + C::kLdsV + buf * C::kTile;
    if (row0 + BN <= sq.lk)
      vcp.issue(vbase + row0 * vstride, dst);
    else
      vcp.issue_clamped(vbase + row0 * vstride, vstride, sq.lk - row0, dst, wave, lane);
  }

  template <int KB, int CP>
  __device__ __forceinline__ void sdp_step(const char G4_LDS* kt, const char G4_LDS* vt,
                                           f32x16& sacc, f32x16& pacc) const {
    if constexpr (CP < kNC) {
      bf16x8 ka = rrd.template read<KB * 32, 0, CP>(kt);
      sacc = mfma32(ka, qf[CP], sacc);
      bf16x8 va = rrd.template read<KB * 32, 0, CP>(vt);
      pacc = mfma32(va, gf[CP], pacc);
      sdp_step<KB, CP + 1>(kt, vt, sacc, pacc);
    }
  }

  template <int KB, int HK, int B>
  __device__ __forceinline__ void dq_step(const char G4_LDS* kt, const bf16x8& ds) {
    if constexpr (B < kNB) {
      bf16x8 x = trd.template read<KB * 32 + 16 * HK, 0, B>(kt);
      dq_acc[B] = mfma32(x, ds, dq_acc[B]);
      dq_step<KB, HK, B + 1>(kt, ds);
    }
  }

  __device__ __forceinline__ void step(int cur, int it, int ntiles, int t_first) {
    const int kb0 = (t_first + it) * BN;
    constexpr int kPer = decltype(kcp)::kPer;
    if constexpr (VDOUBLE)
      vm_wait<0>();
    else
      vm_wait<kPer>();
    barrier_lds();
    if (it + 1 < ntiles) {
      issue_k(kb0 + BN, cur ^ 1);
      if (has_meta && wave == 0)
        issue_key_meta(a->p, sq, kb0 + BN, smem + C::kLdsMeta + (cur ^ 1) * 512, lane,
                       has_vid, has_doc);
      if constexpr (VDOUBLE) issue_v(kb0 + BN, cur ^ 1);
    }
    const char G4_LDS* kt = smem + C::kLdsK + cur * C::kTile;
    const char G4_LDS* vt = smem + C::kLdsV + (VDOUBLE ? cur : 0) * C::kTile;
    if constexpr (!VDOUBLE) {
      // This tile's V copies were issued after the previous step's exchange.
      vm_wait<kPer>();
      barrier_lds();
    }

    __builtin_amdgcn_sched_barrier(0);
    f32x16 sacc[C::kKB], pacc[C::kKB];
    sacc[0] = f32x16{};
    pacc[0] = f32x16{};
    sdp_step<0, 0>(kt, vt, sacc[0], pacc[0]);
    if constexpr (C::kKB > 1) {
      sacc[1] = f32x16{};
      pacc[1] = f32x16{};
      sdp_step<1, 0>(kt, vt, sacc[1], pacc[1]);
    }
    mfma_pipeline_hint<2 * C::kKB * kNC, 3, 1>();
    __builtin_amdgcn_sched_barrier(0);

    if constexpr (DSPLIT > 1) {
      char G4_LDS* xb = smem + C::kLdsX;
#pragma unroll
      for (int kb = 0; kb < C::kKB; ++kb) {
        xchg_write(xb, (wave * C::kKB + kb) * 2, lane, sacc[kb]);
        xchg_write(xb, (wave * C::kKB + kb) * 2 + 1, lane, pacc[kb]);
      }
      barrier_lds();
#pragma unroll
      for (int kb = 0; kb < C::kKB; ++kb) {
        xchg_add(xb, ((wave ^ 1) * C::kKB + kb) * 2, lane, dh, sacc[kb]);
        xchg_add(xb, ((wave ^ 1) * C::kKB + kb) * 2 + 1, lane, dh, pacc[kb]);
      }
    }
    if constexpr (!VDOUBLE) {
      // Every wave is past its V reads (the exchange barrier, or the one
      // below without an exchange): refill the single V buffer.
      if constexpr (DSPLIT == 1) barrier_lds();
      if (it + 1 < ntiles) issue_v(kb0 + BN, 0);
    }

    const bool full = !has_doc && (kb0 + BN <= sq.lk) && (kb0 + BN - 1 <= a0) &&
                      (a->p.window <= 0 || kb0 > a0 + C::kBM - 1 - a->p.window);
    const int lo_w = a->p.window > 0 ? my_a - a->p.window + 1 : -0x40000000;
    const int hi_c = min(my_a, sq.lk - 1);
    const int* km = (const int*)(smem + C::kLdsMeta + cur * 512);
    bf16x8 dsb[C::kKB][2];
#pragma unroll
    for (int kb = 0; kb < C::kKB; ++kb)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int jl0 = kb * 32 + 8 * r4 + 4 * h32;
        i32x4 vk = {-1, -1, -1, -1}, dk = {0, 0, 0, 0};
        if (has_meta && !full) {
          vk = *(const i32x4*)(km + jl0);
          dk = *(const i32x4*)(km + 64 + jl0);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = r4 * 4 + e;
          float p = fast_exp2(sacc[kb][r] * kLog2e - my_lse2);
          if (!full) {
            const int j = kb0 + jl0 + e;
            const bool in_w = j >= lo_w;
            const bool causal = in_w & (j <= hi_c);
            const bool vis = has_vid & (my_vid >= 0) & (vk[e] == my_vid) & in_w & (j < sq.lk);
            const bool doc_ok = !has_doc | (dk[e] == my_doc);
            p = ((causal | vis) & doc_ok & q_valid) ? p : 0.f;
          }
          dsb[kb][r >> 3][r & 7] = (__bf16)(p * (pacc[kb][r] - my_delta));
        }
      }

    __builtin_amdgcn_sched_barrier(0);
    dq_step<0, 0, 0>(kt, dsb[0][0]);
    dq_step<0, 1, 0>(kt, dsb[0][1]);
    if constexpr (C::kKB > 1) {
      dq_step<1, 0, 0>(kt, dsb[1][0]);
      dq_step<1, 1, 0>(kt, dsb[1][1]);
    }
    mfma_pipeline_hint<C::kKB * 2 * kNB, 6, 2>();
    __builtin_amdgcn_sched_barrier(0);
  }
};

template <int D, int BN, int DSPLIT, int NQG, bool VDOUBLE, bool META>
__global__ void __launch_bounds__(NQG * DSPLIT * 64, 1) dq_kernel(BwdParams a) {
  using K = DqKernel<D, BN, DSPLIT, NQG, VDOUBLE, META>;
  using C = typename K::C;
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  K ker;
  ker.smem = (char G4_LDS*)smem_raw;
  ker.a = &a;
  const g4_problem& p = a.p;
  const int tid = threadIdx.x;
  ker.lane = tid & 63;
  ker.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qg = ker.wave / DSPLIT;
  ker.dh = ker.wave % DSPLIT;
  ker.h32 = ker.lane >> 5;
  const int l32 = ker.lane & 31;

  const int grp = p.num_q_heads / p.num_kv_heads;
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int per_kvh = a.num_seqs * a.ntiles * grp;
  const int kvh = L / per_kvh;
  const int rem = L % per_kvh;
  const int rank = rem / grp;
  const int qh = kvh * grp + rem % grp;
  const int s = rank / a.ntiles;
  const int qt = zigzag(rank % a.ntiles, a.ntiles);
  ker.sq = resolve_seq(p, s);
  const Seq& sq = ker.sq;
  const int i0 = qt * C::kBM;
  if (i0 >= sq.lq) return;
  const int off = sq.lk - sq.lq;
  ker.a0 = i0 + off;
  const int a_last_valid = min(i0 + C::kBM, sq.lq) - 1 + off;
  ker.has_vid = META && p.vision_ids != nullptr && p.bidirectional_vision;
  ker.has_doc = META && p.document_ids != nullptr;
  ker.has_meta = ker.has_vid || ker.has_doc;

  int span_max = -1;
  if (ker.has_vid) {
    int* red = (int*)(smem_raw + C::kLdsRed);
    int v = -1;
    for (int t = tid; t < C::kBM; t += C::kNT) {
      int i = i0 + t;
      if (i < sq.lq) v = max(v, a.span_hi[sq.ktok + i + off]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
    if (ker.lane == 0) red[ker.wave] = v;
    barrier_lds();
#pragma unroll
    for (int w = 0; w < C::kNW; ++w) span_max = max(span_max, red[w]);
  }
  int klo, khi;
  query_tile_key_range(ker.a0, a_last_valid, sq.lk, p.window, span_max, klo, khi);
  const int t_first = klo / BN;
  const int ntiles = (khi + BN - 1) / BN - t_first;
  if (ker.has_doc &&
      doc_uniform<C::kNW>(p.document_ids, sq.ktok, sq.lk, min(t_first * BN, ker.a0),
                          max((t_first + ntiles) * BN, a_last_valid + 1), tid, ker.lane,
                          ker.wave, (int*)(smem_raw + C::kLdsRed))) {
    ker.has_doc = false;
    ker.has_meta = ker.has_vid;
  }

  ker.kbase = a.k + tok_off(sq, s, sq.ktok, 0, a.kl) + (int64_t)kvh * a.kl.head_stride;
  ker.vbase = a.v + tok_off(sq, s, sq.ktok, 0, a.vl) + (int64_t)kvh * a.vl.head_stride;
  ker.kstride = a.kl.token_stride;
  ker.vstride = a.vl.token_stride;
  ker.rrd.init(ker.lane, ker.dh * C::kDH * 2);
  ker.trd.init(ker.lane, ker.dh * C::kDH * 2);
  ker.kcp.init(ker.kstride, ker.wave, ker.lane);
  ker.vcp.init(ker.vstride, ker.wave, ker.lane);

  const int my_i = i0 + qg * 32 + l32;
  ker.my_a = my_i + off;
  ker.q_valid = my_i < sq.lq;
  const int ic = min(my_i, sq.lq - 1);
  {
    const __bf16* qrow = a.q + tok_off(sq, s, sq.qtok, ic, a.ql) + (int64_t)qh * a.ql.head_stride +
                         ker.dh * C::kDH + ker.h32 * 8;
    const __bf16* grow = a.dout + tok_off(sq, s, sq.qtok, ic, a.dol) +
                         (int64_t)qh * a.dol.head_stride + ker.dh * C::kDH + ker.h32 * 8;
#pragma unroll
    for (int c = 0; c < K::kNC; ++c) {
      ker.qf[c] = ld_global16(qrow + c * 16);
      ker.gf[c] = ld_global16(grow + c * 16);
    }
  }
  ker.my_lse2 = a.lse[lse_off(p, sq, s, qh, ic)] * kLog2e;
  ker.my_delta = a.delta[(int64_t)qh * q_stream_tokens_dev(p) + sq.qtok + ic];
  ker.my_vid = ker.has_vid ? p.vision_ids[sq.ktok + ic + off] : -1;
  ker.my_doc = ker.has_doc ? p.document_ids[sq.ktok + ic + off] : 0;

#pragma unroll
  for (int b = 0; b < K::kNB; ++b) ker.dq_acc[b] = f32x16{};

  if (ntiles > 0) {
    ker.issue_k(t_first * BN, 0);
    if (ker.has_meta && ker.wave == 0)
      issue_key_meta(p, sq, t_first * BN, ker.smem + C::kLdsMeta, ker.lane, ker.has_vid,
                     ker.has_doc);
    ker.issue_v(t_first * BN, 0);
  }
  for (int it = 0; it < ntiles; ++it) {
    ker.step(it & 1, it, ntiles, t_first);
  }

  if (ker.q_valid) {
    __bf16* row = a.dq + tok_off(sq, s, sq.qtok, my_i, a.dql) + (int64_t)qh * a.dql.head_stride;
#pragma unroll
    for (int b = 0; b < K::kNB; ++b)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d = ker.dh * C::kDH + b * 32 + 8 * r4 + 4 * ker.h32;
        const f32x16& x = ker.dq_acc[b];
        *(bf16x4*)(row + d) = bf16x4{(__bf16)x[r4 * 4], (__bf16)x[r4 * 4 + 1],
                                     (__bf16)x[r4 * 4 + 2], (__bf16)x[r4 * 4 + 3]};
      }
  }
}

// ===========================================================================
// launchers
// ===========================================================================

namespace {

bool has_meta(const g4_problem& p) {
  return (p.vision_ids != nullptr && p.bidirectional_vision) || p.document_ids != nullptr;
}

template <typename Kern>
hipError_t set_lds(Kern kern, int bytes, bool& done) {
  if (done) return hipSuccess;
  hipError_t e =
      hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess) done = true;
  return e;
}

template <int D, int DSPLIT, int NKB, bool DV, bool DK, int KPW>
hipError_t launch_dkdv_cfg(const BwdParams& a, hipStream_t stream) {
  using C = DkdvCfg<D, DSPLIT, NKB, DV, DK, KPW>;
  const bool meta = has_meta(a.p);
  auto kern = meta ? dkdv_kernel<D, DSPLIT, NKB, true, DV, DK, KPW>
                   : dkdv_kernel<D, DSPLIT, NKB, false, DV, DK, KPW>;
  static bool done[2] = {false, false};
  hipError_t e = set_lds(kern, C::kLdsBytes, done[meta]);
  if (e != hipSuccess) return e;
  BwdParams b = a;
  b.ntiles = (a.p.seqlen_k + C::kBN - 1) / C::kBN;
  const int64_t nblocks = (int64_t)b.num_seqs * b.ntiles * a.p.num_kv_heads;
  if (nblocks <= 0) return hipSuccess;
  hipLaunchKernelGGL(kern, dim3((unsigned)nblocks), dim3(C::kNT), C::kLdsBytes, stream, b);
  return hipGetLastError();
}

template <int D, int BN, int DSPLIT, int NQG, bool VDOUBLE>
hipError_t launch_dq_cfg(const BwdParams& a, hipStream_t stream) {
  using C = DqCfg<D, BN, DSPLIT, NQG, VDOUBLE>;
  const bool meta = has_meta(a.p);
  auto kern = meta ? dq_kernel<D, BN, DSPLIT, NQG, VDOUBLE, true>
                   : dq_kernel<D, BN, DSPLIT, NQG, VDOUBLE, false>;
  static bool done[2] = {false, false};
  hipError_t e = set_lds(kern, C::kLdsBytes, done[meta]);
  if (e != hipSuccess) return e;
  BwdParams b = a;
  b.ntiles = (a.p.seqlen_q + C::kBM - 1) / C::kBM;
  const int64_t nblocks = (int64_t)b.num_seqs * b.ntiles * a.p.num_q_heads;
  if (nblocks <= 0) return hipSuccess;
  hipLaunchKernelGGL(kern, dim3((unsigned)nblocks), dim3(C::kNT), C::kLdsBytes, stream, b);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_bwd_dkdv(const BwdParams& a, hipStream_t stream) {
  // Role-specialised waves (a dV role and a dK role per SIMD).
  if (a.p.head_dim == 256 || a.p.head_dim == 512) return launch_dkdv_roles(a, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_bwd_dq(const BwdParams& a, hipStream_t stream) {
  // Role-specialised waves (S waves and dP waves per SIMD).
  if (a.p.head_dim == 256 || a.p.head_dim == 512) return launch_dq_roles(a, stream);
  return hipErrorInvalidValue;
}

}  // namespace g4
