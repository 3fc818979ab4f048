// Backward tile kernels for gfx950 (dK/dV and dQ, head dims 256 and 512), all
// with role-specialised waves: eight waves per workgroup, two per SIMD, each
// wave holding one operand fragment set and one accumulator, so a SIMD always
// has a second wave whose MFMAs overlap the first one's VALU and LDS work.
// Both recompute P = exp2(S log2e - LSE log2e) from the saved fp32 LSE and use
// delta = rowsum(O dO) - dLSE from the pre-pass (g4_bwd.hip): dS = P (dP -
// delta), S = Q K^T, dP = dO V^T, softmax scale 1.0.  P and dS are rounded to
// bf16 before they feed the dV / dK / dQ products.  No atomics: each output
// element is written by one wave, so results repeat bitwise.  dK/dV is
// key-tile major (the GQA group's query heads are reduced on chip); dQ is
// query-tile major.
//
// ---------------------------------------------------------------------------
// dK / dV for head dim 512.
//
// A workgroup owns 64 keys (two blocks of 32) of one KV head and runs eight
// waves, two per SIMD.  Four P waves (one per key block and head-dim half)
// form S = Q K^T, P = exp(S - LSE) and accumulate dV^T += dO^T P; four dS
// waves form dP = dO V^T, dS = P (dP - delta) and accumulate dK^T += Q^T dS.
// Each wave holds one 32-key x 256 fp32 accumulator and one fragment set (K or
// V) in registers, so the two roles together keep the state one wave of head
// dim 512 cannot; S and dP are formed once per step and the Q / dO tiles are
// copied once for both outputs.  On each SIMD a P wave and a dS wave share the
// matrix core, so one's VALU and LDS work overlaps the other's MFMAs.
//
// A step is 32 query rows of one query head (steps walk the query tiles from
// the last one down, or up for the second key tile of a pair, the GQA group's
// heads innermost) with three workgroup barriers:
//   B1  the step's Q, dO, LSE / delta (and metadata) copies have landed in
//       every wave.  P waves: copy the next Q tile (and row data) into the
//       other buffer, partial S over their head-dim half, then write the eight
//       rows per lane the partner finishes.  dS waves: partial dP, write all 16.
//   B2  P waves: add the partner's partial to their eight rows, form P (masked)
//       and publish it in fp32 over the partial they just read.  dS waves: add
//       the partner's dP partial, then copy the next dO tile (they would
//       otherwise wait for P here; the copy still lands a phase ahead of B1).
//   B3  P waves: dV MFMAs with both halves of P in bf16.  dS waves: dS from the
//       fp32 P, dK MFMAs.
// P in fp32 and the fixed-order dP sum keep the numerics of a single-wave
// formulation: dS = bf16(P (dP - delta)), dV from bf16(P).  No atomics; every
// output element is written by one wave.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "g4_kernels.h"

namespace g4 {

namespace {


// Head dim 256 with stored dS: the last key tile each 32-query row of the
// 128-query tile at i0 reaches (its causal end, extended by the vision spans
// of its queries; -1 for rows past the sequence), and whether some row reaches
// past its stored band (such tiles are recomputed by dq_roles256_kernel).
// `red` is four ints of LDS, free on entry.
template <int NW>
__device__ __forceinline__ bool dq_row_key_ends(const BwdParams& a, const Seq& sq, int i0,
                                                int off, int tid, int* red, int (&kt_hi)[4]) {
  const bool vis = a.p.vision_ids != nullptr && a.p.bidirectional_vision;
  if (vis) {
    // Waves 0 and 1 hold the tile's 128 queries: row = tid / 32.
    int v = -1;
    if (tid < 128 && i0 + tid < sq.lq) v = a.span_hi[sq.ktok + i0 + tid + off];
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
    barrier_lds();  // earlier readers of red are done
    if (tid < 128 && (tid & 31) == 0) red[tid >> 5] = v;
    barrier_lds();
  }
  bool need = false;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int r0 = i0 + 32 * g;
    if (r0 >= sq.lq) {
      kt_hi[g] = -1;
      continue;
    }
    int last = min(r0 + 32, sq.lq) - 1 + off;
    if (vis) last = max(last, red[g]);
    kt_hi[g] = last / 64;
    need |= kt_hi[g] - ds_band_first(r0 + off, a.p.window) >= a.ds_cols;
  }
  if (vis) barrier_lds();  // red may be overwritten after this
  return need;
}

struct RolesCfg {
  static constexpr int D = 512;
  static constexpr int kNW = 8;
  static constexpr int kNT = kNW * 64;
  static constexpr int kBN = 64;   // keys per workgroup
  static constexpr int kBM = 32;   // queries per step
  static constexpr int kDH = 256;  // head-dim half per wave
  static constexpr int kCPR = D / 8;
  static constexpr int kNC = kDH / 16;  // 16-deep MFMA steps over a half
  static constexpr int kNB = kDH / 32;  // 32-wide accumulator blocks over a half
  static constexpr int kTile = kBM * D * 2;  // Q or dO tile bytes
  static constexpr int kLdsQ = 0;                      // [2 buf] Q tiles
  static constexpr int kLdsDo = kLdsQ + 2 * kTile;     // [2 buf] dO tiles
  // P-wave exchange: [slot = 2 kb + dh][2][64 lanes][4 f32]: the partner's
  // partial S for the slot owner's rows, then the owner's P for those rows.
  static constexpr int kLdsXs = kLdsDo + 2 * kTile;
  // dS-wave exchange: [slot][4][64 lanes][4 f32] partial dP.
  static constexpr int kLdsXp = kLdsXs + 4 * 2 * 1024;
  static constexpr int kLdsLd = kLdsXp + 4 * 4 * 1024;  // [buf][lse x 32 | delta x 32] fp32
  static constexpr int kLdsMeta = kLdsLd + 2 * 256;     // [buf][vid x 32 | doc x 32] int32
  static constexpr int kLdsRed = kLdsMeta + 2 * 256;
  static constexpr int kLdsSeq = kLdsRed + 64;  // SeqUnitsByLength table (work queue)
  static constexpr int kLdsBytes = kLdsSeq + 512;
  static_assert(kLdsBytes <= 160 * 1024, "LDS budget");
};

// First dS row of sequence s (see BwdParams::ds), and whether a launch of
// sequence stripes handles the sequence (BwdParams::ds_seq_rows).
__device__ __forceinline__ int64_t ds_first_row(const BwdParams& a, const Seq& sq, int s) {
  return sq.packed ? sq.qtok / 32 + s : (int64_t)s * ((a.p.seqlen_q + 31) / 32);
}
__device__ __forceinline__ bool ds_seq_skipped(const BwdParams& a, int64_t first_row) {
  return a.ds_seq_rows > 0 &&
         (first_row < a.ds_row_lo || first_row >= (int64_t)a.ds_row_lo + a.ds_seq_rows);
}

// ROT: the dh = 1 P waves read the Q tile rotated by 16 rows (see step_p).
// STRIPED: one stripe of the striped stored-dS backward (BwdParams::ds_row_lo).
template <bool META, bool ROT, bool STRIPED>
struct RolesKernel {
  using C = RolesCfg;
  char G4_LDS* smem;
  const BwdParams* a;
  Seq sq;
  int s, lane, wave, dh, h32, kb, slot;
  int off, j0, my_j;
  bool has_vid, has_doc, has_meta;
  int my_vid, my_doc;
  int grp, kvh, qt_lo, nqt;
  bool up;  // query tiles walked upward (else from the last one down)
  int64_t tq;
  int64_t ds_row0;  // dS tile row of this sequence's first query tile
  uint32_t ds_lane;  // byte offset of this lane's dS run inside a tile
  RowReader<C::kCPR> rrd;
  TrReader<C::kCPR> trd;
  TileCopier<C::kCPR, C::kBM, 8> qcp;  // Q: half by the P waves, half by the dS waves
  TileCopier<C::kCPR, C::kBM, 4> docp;  // dO by the dS waves
  bf16x8 frag[C::kNC];   // K (P waves) or V (dS waves), B operands
  f32x16 acc[C::kNB];    // dV^T (P waves) or dK^T (dS waves)

  __device__ __forceinline__ void coords(int it, int& qh, int& i0) const {
    const int sh = __builtin_ctz(grp);  // grp is 1, 2, 4 or 8
    qh = kvh * grp + (it & (grp - 1));
    i0 = (up ? qt_lo + (it >> sh) : qt_lo + nqt - 1 - (it >> sh)) * C::kBM;
  }

  // One copy path for full and tail tiles (32-bit buffer offsets, rows
  // clamped to the sequence): fewer instructions than the full-tile path.
  __device__ __forceinline__ void issue_do(int it, int buf) {
    int qh, i0;
    coords(it, qh, i0);
    const __bf16* db =
        a->dout + tok_off(sq, s, sq.qtok, i0, a->dol) + (int64_t)qh * a->dol.head_stride;
    docp.issue_clamped(db, a->dol.token_stride, min(C::kBM, sq.lq - i0),
                       smem + C::kLdsDo + buf * C::kTile);
  }
  // This wave's half of the Q tile's rows (every wave issues one).
  __device__ __forceinline__ void issue_q_rows(int it, int buf) {
    int qh, i0;
    coords(it, qh, i0);
    const __bf16* qb = a->q + tok_off(sq, s, sq.qtok, i0, a->ql) + (int64_t)qh * a->ql.head_stride;
    qcp.issue_clamped(qb, a->ql.token_stride, min(C::kBM, sq.lq - i0),
                      smem + C::kLdsQ + buf * C::kTile);
  }
  // The P waves' rows of the Q tile and, by waves 0 and 1, the row data: LSE
  // and delta of the 32 rows; with metadata the vision / document IDs of the
  // rows' K positions.
  // Work-queue launch (!ROT): the row data goes first, lanes 0-31 issuing both
  // copies of a wave (uniform bases: no loop over per-lane buffer
  // descriptors, fewer live registers; config 4 dK/dV -4%).  One item per
  // workgroup (ROT): the Q rows first, lanes 0-31 copying LSE and lanes 32-63
  // delta (config 2 measured 2.5% slower with the other form).
  __device__ __forceinline__ void issue_q(int it, int buf) {
    int qh, i0;
    coords(it, qh, i0);
    if constexpr (ROT) issue_q_rows(it, buf);
    const int i = min(i0 + (lane & 31), sq.lq - 1);
    // uniform bases at the tile's first (clamped) row, per-lane offsets of
    // at most 31 rows
    const int i0c = min(i0, sq.lq - 1);
    const uint32_t ioff = (uint32_t)(i - i0c) * 4u;
    if (wave == 0) {
      char G4_LDS* dst = smem + C::kLdsLd + buf * 256;
      const float* lse = a->lse + lse_off(a->p, sq, s, qh, i0c);
      const float* del = a->delta + (int64_t)qh * tq + sq.qtok + i0c;
      if constexpr (ROT) {
        if (lane < 32)
          b2l4(lse, ioff, dst);
        else
          b2l4(del, ioff, dst);
      } else if (lane < 32) {
        b2l4(lse, ioff, dst);
        b2l4(del, ioff, dst + 128);
      }
    } else if (wave == 1 && has_meta) {
      char G4_LDS* dst = smem + C::kLdsMeta + buf * 256;
      const int64_t k0 = sq.ktok + i0c + off;
      if constexpr (ROT) {
        if (lane < 32) {
          if (has_vid) b2l4(a->p.vision_ids + k0, ioff, dst);
        } else {
          if (has_doc) b2l4(a->p.document_ids + k0, ioff, dst);
        }
      } else if (lane < 32) {
        if (has_vid) b2l4(a->p.vision_ids + k0, ioff, dst);
        if (has_doc) b2l4(a->p.document_ids + k0, ioff, dst + 128);
      }
    }
    if constexpr (!ROT) issue_q_rows(it, buf);
  }

  // acc^T[32 d x 32 keys] += (tile^T half dh)[32 d x 32 rows] . b[32 rows x 32 keys]
  // (acc_steps); part[32 rows x 32 keys] = tile rows (head-dim half dh) . frag
  // (row_steps).

  // Rows of the accumulators: value r of a lane is query row 8 (r >> 2) +
  // 4 h32 + (r & 3); P waves finish rows r in [8 dh, 8 dh + 8).
  __device__ __forceinline__ char G4_LDS* xs(int sl, int q4) const {
    return smem + C::kLdsXs + ((sl * 2 + q4) * 64 + lane) * 16;
  }

  __device__ __forceinline__ void step_p(int cur, int it, int nsteps) {
    int qh, i0;
    coords(it, qh, i0);
    vm_wait<0>();
    barrier_lds();  // B1
    const char G4_LDS* qt = smem + C::kLdsQ + cur * C::kTile;
    const char G4_LDS* dot = smem + C::kLdsDo + cur * C::kTile;

    __builtin_amdgcn_sched_barrier(0);
    f32x16 sp = f32x16{};
    if (it + 1 < nsteps) issue_q(it + 1, cur ^ 1);
    row_steps(rrd, qt, sp, frag);
    __builtin_amdgcn_sched_barrier(0);
    // the partner's rows of this partial.  With ROT, registers 8-15 in both
    // waves (the dh = 1 wave reads the Q tile rotated by 16 rows, so its own
    // rows, like the dh = 0 wave's, are in registers 0-7); without, the
    // register index depends on dh, a runtime index (s_set_gpr_idx moves).
    const int po = ROT ? 8 : 8 * (dh ^ 1);
    const int mo = ROT ? 0 : 8 * dh;
#pragma unroll
    for (int q4 = 0; q4 < 2; ++q4)
      *(f32x4 G4_LDS*)xs(slot ^ 1, q4) =
          f32x4{sp[po + 4 * q4], sp[po + 4 * q4 + 1], sp[po + 4 * q4 + 2], sp[po + 4 * q4 + 3]};
    barrier_lds();  // B2

    const float* ld = (const float*)(smem + C::kLdsLd + cur * 256);
    const bool full = !has_doc && (i0 + C::kBM <= sq.lq) && (j0 + C::kBN <= sq.lk) &&
                      (j0 + C::kBN - 1 <= i0 + off) &&
                      (a->p.window <= 0 || j0 > i0 + C::kBM - 1 + off - a->p.window);
#pragma unroll
    for (int q4 = 0; q4 < 2; ++q4) {
      const f32x4 theirs = *(const f32x4 G4_LDS*)xs(slot, q4);
      const int r4 = 2 * dh + q4;
      const int il0 = 8 * r4 + 4 * h32;
      const f32x4 lse4 = *(const f32x4*)(ld + il0);
      i32x4 vq4 = {-1, -1, -1, -1}, dq4 = {0, 0, 0, 0};
      if (has_meta && !full) {
        const int* mt = (const int*)(smem + C::kLdsMeta + cur * 256);
        vq4 = *(const i32x4*)(mt + il0);
        dq4 = *(const i32x4*)(mt + 32 + il0);
      }
      f32x4 pv;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float sv = sp[mo + 4 * q4 + e] + theirs[e];
        float p = fast_exp2(sv * kLog2e - lse4[e] * kLog2e);
        if (!full) {
          const int i = i0 + il0 + e;
          const int aq = i + off;
          const bool in_w = a->p.window <= 0 || my_j > aq - a->p.window;
          const bool causal = my_j <= aq;
          const bool vis = has_vid & (vq4[e] >= 0) & (vq4[e] == my_vid);
          const bool doc_ok = !has_doc | (dq4[e] == my_doc);
          const bool ok = (i < sq.lq) & (my_j < sq.lk) & in_w & (causal | vis) & doc_ok;
          p = ok ? p : 0.f;
        }
        pv[e] = p;
      }
      // Same address as `theirs` (read first in this wave's LDS order).
      *(f32x4 G4_LDS*)xs(slot, q4) = pv;
    }
    barrier_lds();  // B3

    bf16x8 pb[2];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int q4 = 0; q4 < 2; ++q4) {
        const f32x4 v = *(const f32x4 G4_LDS*)xs((slot & ~1) | m, q4);
#pragma unroll
        for (int e = 0; e < 4; ++e) pb[m][4 * q4 + e] = (__bf16)v[e];
      }
    __builtin_amdgcn_sched_barrier(0);
    acc_steps(trd, dot, pb, acc);
    __builtin_amdgcn_sched_barrier(0);
  }

  __device__ __forceinline__ void step_ds(int cur, int it, int nsteps) {
    int qh, i0;
    coords(it, qh, i0);
    vm_wait<0>();
    barrier_lds();  // B1
    const char G4_LDS* qt = smem + C::kLdsQ + cur * C::kTile;
    const char G4_LDS* dot = smem + C::kLdsDo + cur * C::kTile;
    char G4_LDS* xp = smem + C::kLdsXp;

    __builtin_amdgcn_sched_barrier(0);
    f32x16 dp = f32x16{};
    row_steps(rrd, dot, dp, frag);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4)
      *(f32x4 G4_LDS*)(xp + ((slot * 4 + q4) * 64 + lane) * 16) =
          f32x4{dp[4 * q4], dp[4 * q4 + 1], dp[4 * q4 + 2], dp[4 * q4 + 3]};
    // Half of the next Q tile (these waves wait at B2 for the P waves' S
    // partial, which the other half's issue delays).
    if (it + 1 < nsteps) issue_q_rows(it + 1, cur ^ 1);
    barrier_lds();  // B2

    // dP = (slice 0 partial) + (slice 1 partial) in both waves of the pair.
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const f32x4 w = *(const f32x4 G4_LDS*)(xp + (((slot ^ 1) * 4 + q4) * 64 + lane) * 16);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float mine = dp[4 * q4 + e];
        dp[4 * q4 + e] = dh == 0 ? mine + w[e] : w[e] + mine;
      }
    }
    if (it + 1 < nsteps) issue_do(it + 1, cur ^ 1);
    barrier_lds();  // B3

    const float* ld = (const float*)(smem + C::kLdsLd + cur * 256);
    bf16x8 db[2];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int q4 = 0; q4 < 2; ++q4) {
        const f32x4 pv = *(const f32x4 G4_LDS*)xs((slot & ~1) | m, q4);
        const f32x4 del4 = *(const f32x4*)(ld + 32 + 8 * (2 * m + q4) + 4 * h32);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 8 * m + 4 * q4 + e;
          db[m][4 * q4 + e] = (__bf16)(pv[e] * (dp[r] - del4[e]));
        }
      }
    if (a->ds != nullptr) {
      // dS tile [64 keys][32 queries] in query order: this lane's key row
      // holds four runs of four queries (rows 8 (r >> 2) + 4 h32 + (r & 3) of
      // the accumulator layout); both waves of the pair hold all of them, wave
      // dh stores the two runs of db[dh].  (Accumulator order, one 16-byte
      // store per lane, measured 5.60 vs 5.41 ms here: the two waves' stores
      // then interleave within every 64-byte key row.)
      G4_GLOBAL char* tile =
          (G4_GLOBAL char*)a->ds +
          (((int64_t)qh * a->ds_cols + j0 / C::kBN) * a->ds_rows + ds_row0 + i0 / 32) * 4096;
      const bf16x8 x = dh == 0 ? db[0] : db[1];
      *(G4_GLOBAL bf16x4*)(tile + ds_lane) = bf16x4{x[0], x[1], x[2], x[3]};
      *(G4_GLOBAL bf16x4*)(tile + ds_lane + 16) = bf16x4{x[4], x[5], x[6], x[7]};
    }
    __builtin_amdgcn_sched_barrier(0);
    acc_steps(trd, qt, db, acc);
    __builtin_amdgcn_sched_barrier(0);
  }

  // Load this wave's K or V fragments, run the steps, store dV or dK (bf16).
  template <bool PWAVE>
  __device__ __forceinline__ void run(int nsteps) {
    const int jc = min(my_j, sq.lk - 1);
    const __bf16* src = PWAVE ? a->k + tok_off(sq, s, sq.ktok, jc, a->kl) +
                                    (int64_t)kvh * a->kl.head_stride
                              : a->v + tok_off(sq, s, sq.ktok, jc, a->vl) +
                                    (int64_t)kvh * a->vl.head_stride;
    src += dh * C::kDH + h32 * 8;
#pragma unroll
    for (int c = 0; c < C::kNC; ++c) frag[c] = ld_global16(src + c * 16);
#pragma unroll
    for (int b = 0; b < C::kNB; ++b) acc[b] = f32x16{};

    for (int it = 0; it < nsteps; ++it) {
      if constexpr (PWAVE)
        step_p(it & 1, it, nsteps);
      else
        step_ds(it & 1, it, nsteps);
    }

    if (my_j >= sq.lk) return;
    __bf16* dst = PWAVE ? a->dv + tok_off(sq, s, sq.ktok, my_j, a->dvl) +
                              (int64_t)kvh * a->dvl.head_stride
                        : a->dk + tok_off(sq, s, sq.ktok, my_j, a->dkl) +
                              (int64_t)kvh * a->dkl.head_stride;
    // Striped: add to / write the fp32 sums over the stripes; the last stripe
    // writes bf16 dK / dV (see BwdParams::acc_mode).  A middle stripe without
    // steps for this tile leaves its sums as they are.
    float* sum = nullptr;
    if constexpr (STRIPED) {
      if (nsteps == 0 && a->acc_mode == 1) return;
      sum = (PWAVE ? a->dv_acc : a->dk_acc) +
            ((sq.ktok + my_j) * a->p.num_kv_heads + kvh) * (int64_t)C::D;
    }
#pragma unroll
    for (int b = 0; b < C::kNB; ++b)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d = dh * C::kDH + b * 32 + 8 * r4 + 4 * h32;
        f32x4 x = f32x4{acc[b][r4 * 4], acc[b][r4 * 4 + 1], acc[b][r4 * 4 + 2], acc[b][r4 * 4 + 3]};
        if (STRIPED) {
          if (a->acc_mode & 1) x += *(const f32x4*)(sum + d);
          if (!(a->acc_mode & 2)) {
            *(f32x4*)(sum + d) = x;
            continue;
          }
        }
        *(bf16x4*)(dst + d) = bf16x4{(__bf16)x[0], (__bf16)x[1], (__bf16)x[2], (__bf16)x[3]};
      }
  }
};

// One key tile kt of sequence s and KV head kvh; its query tiles are walked
// upward with `up`, else from the last one down.
template <bool META, bool QUEUE, bool STRIPED>
__device__ __forceinline__ void dkdv_roles_tile(const BwdParams& a, char* smem_raw, int kvh,
                                                int s, int kt, bool up) {
  // Rotation only in the one-item-per-workgroup launch: measured on config 2
  // (one 8192-token sequence) dK/dV 5.32 -> 5.17 ms, but 5.21 -> 5.89 ms in the
  // work-queue launch of config 4 (packed, 1-2048-token segments).
  using K = RolesKernel<META, !QUEUE, STRIPED>;
  using C = RolesCfg;
  K ker;
  ker.smem = (char G4_LDS*)smem_raw;
  ker.a = &a;
  const g4_problem& p = a.p;
  const int tid = item_thread_id<QUEUE>();
  ker.lane = tid & 63;
  ker.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool pwave = ker.wave < 4;
  ker.slot = ker.wave & 3;  // 2 kb + dh
  ker.kb = ker.slot >> 1;
  ker.dh = ker.slot & 1;
  ker.h32 = ker.lane >> 5;

  ker.grp = p.num_q_heads / p.num_kv_heads;
  ker.kvh = kvh;
  ker.up = up;
  ker.s = s;
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
  ker.my_j = ker.j0 + ker.kb * 32 + (ker.lane & 31);

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
  if constexpr (STRIPED) {
    // Striped (one sequence): only the stripe's rows, query tiles (one 32-query
    // row each) [ds_row_lo, ds_row_lo + ds_rows) of the sequence, stored from
    // the buffer's first row.
    const int lo = max(ker.qt_lo, a.ds_row_lo);
    const int hi = min(ker.qt_lo + ker.nqt, a.ds_row_lo + a.ds_rows);
    ker.qt_lo = lo;
    ker.nqt = max(hi - lo, 0);
    ker.ds_row0 = -a.ds_row_lo;
  } else {
    // (sequence stripes: rows from the stripe's first, ds_row_lo; else 0)
    ker.ds_row0 = ds_first_row(a, sq, ker.s) - a.ds_row_lo;
  }
  const int nsteps = ker.nqt * ker.grp;
  ker.ds_lane = (ker.kb * 32 + (ker.lane & 31)) * 64 + 32 * ker.dh + 8 * ker.h32;
  const int jc = min(ker.my_j, sq.lk - 1);
  ker.my_vid = ker.has_vid ? p.vision_ids[sq.ktok + jc] : -1;
  ker.my_doc = ker.has_doc ? p.document_ids[sq.ktok + jc] : 0;

  ker.rrd.init(ker.lane, ker.dh * C::kDH * 2);
  // P waves with dh = 1: Q rows rotated by 16 (row r ^ 16; the swizzle depends
  // on r mod 16 only), so both waves of a pair hold their own rows of the S
  // partial in accumulator registers 0-7.
  if (!QUEUE && pwave && ker.dh) ker.rrd.base ^= 16 * C::kCPR * 16;
  ker.trd.init(ker.lane, ker.dh * C::kDH * 2);
  ker.qcp.init(a.ql.token_stride, ker.wave, ker.lane);
  ker.docp.init(a.dol.token_stride, ker.wave & 3, ker.lane);
  if (nsteps > 0) {
    if (pwave) {
      ker.issue_q(0, 0);
    } else {
      ker.issue_do(0, 0);
      ker.issue_q_rows(0, 0);
    }
  }
  // Both roles run nsteps steps of three barriers each.
  if (pwave)
    ker.template run<true>(nsteps);
  else
    ker.template run<false>(nsteps);
}

// Work item L: (KV head, pair r, sequence) = key tiles r and nt - 1 - r of
// the sequence (nt = its key tiles), the largest r (present only in the
// longest sequences) first within a KV head.  Under the causal mask a key
// tile's query count falls linearly with its index, so a pair carries about
// the same number of steps whatever r is.  KV head slowest keeps the
// workgroups of one XCD on one head group's Q and dO, and the step order
// keeps them on the same query tiles at the same time: the first tile walks
// its query tiles from the last one down, the second from its first one up.
// On one causal sequence of Q query tiles (two per key tile), after t query
// tiles of steps a workgroup in its first pass is at query tile Q - 1 - t and
// one in its second pass at t - 2, whatever its r, so the workgroups of an XCD
// read two streams of Q and dO tiles between them (was: one per workgroup
// once they restarted at the last tile at different times).
// With `by_length` (the queue launch of a packed batch of up to 64
// sequences): only the pairs that exist, sequence by sequence from the longest
// (a pair's cost grows with its sequence's length, and a longer sequence has
// more pairs: the heaviest items go first), then KV head, then pair.
template <bool META, bool QUEUE, bool STRIPED>
__device__ __forceinline__ void dkdv_roles_pair(const BwdParams& a, char* smem_raw, int L,
                                                bool by_length = false) {
  using C = RolesCfg;
  int kvh, r, s;
  if (by_length) {
    int local, n;
    SeqUnitsByLength::find_lds((const int G4_LDS*)(smem_raw + C::kLdsSeq), L, s, local, n);
    const int np = n / a.p.num_kv_heads;
    kvh = local / np;
    r = local % np;
  } else {
    const int npairs = (a.ntiles + 1) / 2;
    const int per_kvh = npairs * a.num_seqs;
    kvh = L / per_kvh;
    const int rem = L % per_kvh;
    r = npairs - 1 - rem / a.num_seqs;
    s = rem % a.num_seqs;
  }
  const Seq sq = resolve_seq(a.p, s);
  const int nt = (sq.lk + C::kBN - 1) / C::kBN;
  if (r >= (nt + 1) / 2 || ds_seq_skipped(a, ds_first_row(a, sq, s))) return;
#pragma nounroll
  for (int pass = 0; pass < 2; ++pass) {
    const int kt = pass == 0 ? r : nt - 1 - r;
    if (pass == 1) {
      if (kt == r) break;
      barrier_lds();  // every wave is done with the first tile's LDS
    }
    dkdv_roles_tile<META, QUEUE, STRIPED>(a, smem_raw, kvh, s, kt, pass == 1);
  }
}

// Persistent: a few workgroups per CU take pair tickets from the dK/dV work
// queue.  (With one workgroup per key tile, per-CU busy time on an 8192-token
// causal sequence ranged from 8% to 100% of the launch.)
template <bool META, bool QUEUE, bool STRIPED>
__global__ void __launch_bounds__(RolesCfg::kNT, 1) dkdv_roles_kernel(BwdParams a) {
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  if constexpr (QUEUE) {
    using C = RolesCfg;
    const int hkv = a.p.num_kv_heads;
    int n = (a.ntiles + 1) / 2 * a.num_seqs * hkv;
    const bool by_length = a.p.cu_seqlens_q != nullptr && a.p.cu_seqlens_k != nullptr &&
                           a.num_seqs <= 64;
    if (by_length) {
      // ordered by query length; units: pairs of key tiles over all KV heads
      SeqUnitsByLength order;
      // (sequence stripes: only the stripe's sequences)
      order.init(a.p.cu_seqlens_q, a.p.cu_seqlens_k, a.num_seqs, [&](int seq, int lk) {
        const int64_t first_row = a.p.cu_seqlens_q[seq] / 32 + seq;
        return ds_seq_skipped(a, first_row) ? 0 : ((lk + C::kBN - 1) / C::kBN + 1) / 2 * hkv;
      });
      n = order.total;
      if (threadIdx.x < 64) order.store((int G4_LDS*)(smem_raw + C::kLdsSeq));
      barrier_lds();
    }
    WorkQueue wq{a.sched, n, 0};
    for (;;) {
      const int t = wq.next((int G4_LDS*)smem_raw);
      if (t >= n) break;
      dkdv_roles_pair<META, true, STRIPED>(a, smem_raw, t, by_length);
    }
  } else {
    dkdv_roles_pair<META, false, STRIPED>(a, smem_raw, xcd_remap(blockIdx.x, gridDim.x));
  }
}

// ===========================================================================
// dK / dV for head dim 256 with role-specialised waves.
//
// The same split with the whole head dim in every wave, so no partials are
// exchanged: a workgroup owns 128 keys (four blocks of 32); P wave kb forms S
// and P for key block kb, publishes P in fp32 and accumulates dV^T; dS wave kb
// forms dP, reads P, forms dS and accumulates dK^T.  Two barriers per step:
//   B1  the step's Q, dO, row data (and metadata) have landed.  P waves copy
//       the next Q tile (and row data), form S, P and publish P; dS waves form
//       dP and copy the next dO tile.
//   B2  P published.  P waves: dV MFMAs; dS waves: dS, dK MFMAs.
// ===========================================================================

struct Roles256Cfg {
  static constexpr int D = 256;
  static constexpr int kNW = 8;
  static constexpr int kNT = kNW * 64;
  static constexpr int kBN = 128;  // keys per workgroup
  static constexpr int kBM = 32;   // queries per step
  static constexpr int kCPR = D / 8;
  static constexpr int kNC = D / 16;
  static constexpr int kNB = D / 32;
  // LDS operand reads in flight per MFMA chain (config 3 dK/dV 1.11 -> 1.07 ms
  // against two; config 5 unchanged).
  static constexpr int kReads = 3;
  static constexpr int kTile = kBM * D * 2;
  static constexpr int kLdsQ = 0;                   // [2 buf]
  static constexpr int kLdsDo = kLdsQ + 2 * kTile;  // [2 buf]
  static constexpr int kLdsP = kLdsDo + 2 * kTile;  // [kb][4][64 lanes][4 f32]
  static constexpr int kLdsLd = kLdsP + 4 * 4096;   // [buf][lse x 32 | delta x 32] fp32
  static constexpr int kLdsMeta = kLdsLd + 2 * 256; // [buf][vid x 32 | doc x 32] int32
  static constexpr int kLdsRed = kLdsMeta + 2 * 256;
  static constexpr int kLdsSeq = kLdsRed + 64;       // SeqTiles table (work queue)
  static constexpr int kLdsBytes = kLdsSeq + 512;
  static_assert(kLdsBytes <= 160 * 1024, "LDS budget");
};

template <bool META>
struct Roles256Kernel {
  using C = Roles256Cfg;
  char G4_LDS* smem;
  const BwdParams* a;
  Seq sq;
  int s, lane, wave, h32, kb;
  int off, j0, my_j;
  bool has_vid, has_doc, has_meta;
  int my_vid, my_doc;
  int grp, kvh, qt_lo, nqt;
  int64_t tq;
  int64_t ds_row0;  // dS tile row of this sequence's first query tile
  RowReader<C::kCPR> rrd;
  TrReader<C::kCPR> trd;
  TileCopier<C::kCPR, C::kBM, 4> qcp, docp;  // Q by the P waves, dO by the dS waves
  bf16x8 frag[C::kNC];  // K (P waves) or V (dS waves)
  f32x16 acc[C::kNB];   // dV^T (P waves) or dK^T (dS waves)

  __device__ __forceinline__ void coords(int it, int& qh, int& i0) const {
    const int sh = __builtin_ctz(grp);
    qh = kvh * grp + (it & (grp - 1));
    i0 = (qt_lo + nqt - 1 - (it >> sh)) * C::kBM;
  }
  __device__ __forceinline__ void issue_do(int it, int buf) {
    int qh, i0;
    coords(it, qh, i0);
    const __bf16* db =
        a->dout + tok_off(sq, s, sq.qtok, i0, a->dol) + (int64_t)qh * a->dol.head_stride;
    docp.issue_clamped(db, a->dol.token_stride, min(C::kBM, sq.lq - i0),
                       smem + C::kLdsDo + buf * C::kTile);
  }
  __device__ __forceinline__ void issue_q(int it, int buf) {
    int qh, i0;
    coords(it, qh, i0);
    const __bf16* qb = a->q + tok_off(sq, s, sq.qtok, i0, a->ql) + (int64_t)qh * a->ql.head_stride;
    qcp.issue_clamped(qb, a->ql.token_stride, min(C::kBM, sq.lq - i0),
                      smem + C::kLdsQ + buf * C::kTile);
    const int i = min(i0 + (lane & 31), sq.lq - 1);
    // (row data by the first two waves of the issuing role)
    // uniform bases at the tile's first (clamped) row, per-lane offsets of
    // at most 31 rows
    const int i0c = min(i0, sq.lq - 1);
    const uint32_t ioff = (uint32_t)(i - i0c) * 4u;
    // Lanes 0-31 issue both copies of a wave (uniform bases, so no loop over
    // per-lane buffer descriptors): the first 128 bytes, then the next 128.
    if ((wave & 3) == 0) {
      char G4_LDS* dst = smem + C::kLdsLd + buf * 256;
      if (lane < 32) {
        b2l4(a->lse + lse_off(a->p, sq, s, qh, i0c), ioff, dst);
        b2l4(a->delta + (int64_t)qh * tq + sq.qtok + i0c, ioff, dst + 128);
      }
    } else if ((wave & 3) == 1 && has_meta) {
      char G4_LDS* dst = smem + C::kLdsMeta + buf * 256;
      const int64_t k0 = sq.ktok + i0c + off;
      if (lane < 32) {
        if (has_vid) b2l4(a->p.vision_ids + k0, ioff, dst);
        if (has_doc) b2l4(a->p.document_ids + k0, ioff, dst + 128);
      }
    }
  }
  __device__ __forceinline__ char G4_LDS* pslot(int q4) const {
    return smem + C::kLdsP + ((kb * 4 + q4) * 64 + lane) * 16;
  }

  // Values r of a lane are query rows 8 (r >> 2) + 4 h32 + (r & 3); lanes own keys.
  __device__ __forceinline__ void step_p(int cur, int it, int nsteps) {
    int qh, i0;
    coords(it, qh, i0);
    vm_wait<0>();
    barrier_lds();  // B1
    const char G4_LDS* qt = smem + C::kLdsQ + cur * C::kTile;
    const char G4_LDS* dot = smem + C::kLdsDo + cur * C::kTile;
    __builtin_amdgcn_sched_barrier(0);
    f32x16 sv = f32x16{};
    row_steps<C::kNC, C::kReads>(rrd, qt, sv, frag);
    __builtin_amdgcn_sched_barrier(0);

    const float* ld = (const float*)(smem + C::kLdsLd + cur * 256);
    const bool full = !has_doc && (i0 + C::kBM <= sq.lq) && (j0 + C::kBN <= sq.lk) &&
                      (j0 + C::kBN - 1 <= i0 + off) &&
                      (a->p.window <= 0 || j0 > i0 + C::kBM - 1 + off - a->p.window);
    bf16x8 pb[2];
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const int il0 = 8 * r4 + 4 * h32;
      const f32x4 lse4 = *(const f32x4*)(ld + il0);
      i32x4 vq4 = {-1, -1, -1, -1}, dq4 = {0, 0, 0, 0};
      if (has_meta && !full) {
        const int* mt = (const int*)(smem + C::kLdsMeta + cur * 256);
        vq4 = *(const i32x4*)(mt + il0);
        dq4 = *(const i32x4*)(mt + 32 + il0);
      }
      f32x4 pv;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float p = fast_exp2(sv[4 * r4 + e] * kLog2e - lse4[e] * kLog2e);
        if (!full) {
          const int i = i0 + il0 + e;
          const int aq = i + off;
          const bool in_w = a->p.window <= 0 || my_j > aq - a->p.window;
          const bool causal = my_j <= aq;
          const bool vis = has_vid & (vq4[e] >= 0) & (vq4[e] == my_vid);
          const bool doc_ok = !has_doc | (dq4[e] == my_doc);
          const bool ok = (i < sq.lq) & (my_j < sq.lk) & in_w & (causal | vis) & doc_ok;
          p = ok ? p : 0.f;
        }
        pv[e] = p;
        pb[r4 >> 1][4 * (r4 & 1) + e] = (__bf16)p;
      }
      *(f32x4 G4_LDS*)pslot(r4) = pv;
    }
    barrier_lds();  // B2

    // The next step's Q after the softmax (on the step's critical path) and
    // before the dV MFMAs (these waves then wait at B1 for the dS waves).
    if (it + 1 < nsteps) issue_q(it + 1, cur ^ 1);
    __builtin_amdgcn_sched_barrier(0);
    acc_steps<C::kNB, C::kReads>(trd, dot, pb, acc);
    __builtin_amdgcn_sched_barrier(0);
  }

  __device__ __forceinline__ void step_ds(int cur, int it, int nsteps) {
    vm_wait<0>();
    barrier_lds();  // B1
    const char G4_LDS* qt = smem + C::kLdsQ + cur * C::kTile;
    const char G4_LDS* dot = smem + C::kLdsDo + cur * C::kTile;
    __builtin_amdgcn_sched_barrier(0);
    f32x16 dp = f32x16{};
    row_steps<C::kNC, C::kReads>(rrd, dot, dp, frag);
    __builtin_amdgcn_sched_barrier(0);
    if (it + 1 < nsteps) issue_do(it + 1, cur ^ 1);
    barrier_lds();  // B2

    const float* ld = (const float*)(smem + C::kLdsLd + cur * 256);
    bf16x8 db[2];
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const f32x4 pv = *(const f32x4 G4_LDS*)pslot(r4);
      const f32x4 del4 = *(const f32x4*)(ld + 32 + 8 * r4 + 4 * h32);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        db[r4 >> 1][4 * (r4 & 1) + e] = (__bf16)(pv[e] * (dp[4 * r4 + e] - del4[e]));
    }
    if (a->ds != nullptr) {
      // This wave's 32 keys are one half of a 64-key dS tile of the step's
      // query row; stored when the tile lies in the row's band.  Tile key rows
      // keep queries in accumulator order (ds_query_at), so the lane's 16
      // values are one 32-byte run.
      int qh, i0;
      coords(it, qh, i0);
      const int c = (j0 + kb * 32) / 64 - ds_band_first(i0 + off, a->p.window);
      if (c >= 0 && c < a->ds_cols) {
        char* row = (char*)a->ds +
                    (((int64_t)qh * a->ds_rows + ds_row0 + i0 / 32) * a->ds_cols + c) * 4096 +
                    ((kb & 1) * 32 + (lane & 31)) * 64;
#pragma unroll
        for (int m = 0; m < 2; ++m) *(bf16x8*)(row + (16 * h32 + 8 * m) * 2) = db[m];
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    acc_steps<C::kNB, C::kReads>(trd, qt, db, acc);
    __builtin_amdgcn_sched_barrier(0);
  }

  template <bool PWAVE>
  __device__ __forceinline__ void run(int nsteps) {
    const int jc = min(my_j, sq.lk - 1);
    const __bf16* src = PWAVE ? a->k + tok_off(sq, s, sq.ktok, jc, a->kl) +
                                    (int64_t)kvh * a->kl.head_stride
                              : a->v + tok_off(sq, s, sq.ktok, jc, a->vl) +
                                    (int64_t)kvh * a->vl.head_stride;
    src += h32 * 8;
#pragma unroll
    for (int c = 0; c < C::kNC; ++c) frag[c] = ld_global16(src + c * 16);
#pragma unroll
    for (int b = 0; b < C::kNB; ++b) acc[b] = f32x16{};
    for (int it = 0; it < nsteps; ++it) {
      if constexpr (PWAVE)
        step_p(it & 1, it, nsteps);
      else
        step_ds(it & 1, it, nsteps);
    }
    if (my_j >= sq.lk) return;
    __bf16* dst = PWAVE ? a->dv + tok_off(sq, s, sq.ktok, my_j, a->dvl) +
                              (int64_t)kvh * a->dvl.head_stride
                        : a->dk + tok_off(sq, s, sq.ktok, my_j, a->dkl) +
                              (int64_t)kvh * a->dkl.head_stride;
#pragma unroll
    for (int b = 0; b < C::kNB; ++b)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d = b * 32 + 8 * r4 + 4 * h32;
        const f32x16& x = acc[b];
        *(bf16x4*)(dst + d) = bf16x4{(__bf16)x[r4 * 4], (__bf16)x[r4 * 4 + 1],
                                     (__bf16)x[r4 * 4 + 2], (__bf16)x[r4 * 4 + 3]};
      }
  }
};

// Work item L: (KV head, sequence, key tile); with total > 0, only the key
// tiles that exist (total of them per KV head; the SeqTiles table is in LDS).
template <bool META, bool QUEUE>
__device__ __forceinline__ void dkdv_roles256_item(const BwdParams& a, char* smem_raw, int L,
                                                   int total = 0) {
  using K = Roles256Kernel<META>;
  using C = Roles256Cfg;
  K ker;
  ker.smem = (char G4_LDS*)smem_raw;
  ker.a = &a;
  const g4_problem& p = a.p;
  const int tid = item_thread_id<QUEUE>();
  ker.lane = tid & 63;
  ker.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool pwave = ker.wave < 4;
  ker.kb = ker.wave & 3;
  ker.h32 = ker.lane >> 5;

  ker.grp = p.num_q_heads / p.num_kv_heads;
  int kt;
  if (total > 0) {
    ker.kvh = L / total;
    int local, nt;
    SeqTiles::find_lds((const int G4_LDS*)(smem_raw + C::kLdsSeq), L % total, ker.s, local, nt);
    kt = zigzag(local, nt);
  } else {
    const int per_kvh = a.num_seqs * a.ntiles;
    ker.kvh = L / per_kvh;
    const int rank = L % per_kvh;
    ker.s = rank / a.ntiles;
    kt = zigzag(rank % a.ntiles, a.ntiles);
  }
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
  ker.my_j = ker.j0 + ker.kb * 32 + (ker.lane & 31);

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
  ker.ds_row0 = sq.packed ? sq.qtok / 32 + ker.s : (int64_t)ker.s * ((p.seqlen_q + 31) / 32);
  const int jc = min(ker.my_j, sq.lk - 1);
  ker.my_vid = ker.has_vid ? p.vision_ids[sq.ktok + jc] : -1;
  ker.my_doc = ker.has_doc ? p.document_ids[sq.ktok + jc] : 0;

  ker.rrd.init(ker.lane, 0);
  ker.trd.init(ker.lane, 0);
  ker.qcp.init(a.ql.token_stride, ker.wave & 3, ker.lane);
  ker.docp.init(a.dol.token_stride, ker.wave & 3, ker.lane);
  if (nsteps > 0) {
    if (pwave)
      ker.issue_q(0, 0);
    else
      ker.issue_do(0, 0);
  }
  // Both roles run nsteps steps of two barriers each.
  if (pwave)
    ker.template run<true>(nsteps);
  else
    ker.template run<false>(nsteps);
}

// Persistent: a few workgroups per CU take (KV head, sequence, key tile)
// tickets from the dK/dV work queue.  (Per-XCD runs of the same order, as
// the head-dim 256 dQ kernel takes them, measured 12.7 -> 13.0 ms on config 5.)
template <bool META, bool QUEUE>
__global__ void __launch_bounds__(Roles256Cfg::kNT, 1) dkdv_roles256_kernel(BwdParams a) {
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  if constexpr (QUEUE) {
    int n = a.num_seqs * a.ntiles * a.p.num_kv_heads, total = 0;
    {
      SeqTiles tiles;
      tiles.init(a.p.cu_seqlens_k, a.num_seqs, Roles256Cfg::kBN);
      if (tiles.ok) {
        total = tiles.total;
        n = total * a.p.num_kv_heads;
        if (threadIdx.x < 64) tiles.store((int G4_LDS*)(smem_raw + Roles256Cfg::kLdsSeq));
      }
      barrier_lds();
    }
    WorkQueue wq{a.sched, n, 0};
    for (;;) {
      const int t = wq.next((int G4_LDS*)smem_raw);
      if (t >= n) break;
      dkdv_roles256_item<META, true>(a, smem_raw, t, total);
    }
  } else {
    dkdv_roles256_item<META, false>(a, smem_raw, xcd_remap(blockIdx.x, gridDim.x));
  }
}

// ===========================================================================
// dQ for head dim 512 with role-specialised waves.
//
// A workgroup owns 64 queries (two groups of 32) of one query head and walks
// the 32-key tiles its range admits with eight waves, two per SIMD.  Per query
// group and head-dim half an S wave holds Q fragments and forms the partial
// S^T = K Q^T, a dP wave holds dO fragments and forms the partial
// dP^T = V dO^T.  After one exchange every wave of a query group holds the same
// full S and dP (partials summed half 0 + half 1), forms P and dS and
// accumulates dQ^T += K^T dS^T over its quarter of the head dim.  Per key tile
// two barriers:
//   B1  K(t), V(t) and key metadata have landed; K(t+1) goes out.
//   B2  partials written; V(t+1) goes out (V is read only before B2).
// ===========================================================================

struct DqRolesCfg {
  static constexpr int D = 512;
  static constexpr int kNW = 8;
  static constexpr int kNT = kNW * 64;
  static constexpr int kBM = 64;   // queries per workgroup
  static constexpr int kBN = 32;   // keys per tile
  static constexpr int kDH = 256;  // head-dim half of an S / dP partial
  static constexpr int kDQ = 128;  // head-dim quarter of a dQ accumulator
  static constexpr int kCPR = D / 8;
  static constexpr int kNC = kDH / 16;
  static constexpr int kNB = kDQ / 32;
  static constexpr int kTile = kBN * D * 2;
  static constexpr int kLdsK = 0;                  // [2 buf] K tiles
  static constexpr int kLdsV = kLdsK + 2 * kTile;  // one V tile
  // Partials: [slot = 4 qg + 2 role + dh][4][64 lanes][4 f32].
  static constexpr int kLdsX = kLdsV + kTile;
  static constexpr int kLdsMeta = kLdsX + 8 * 4096;  // [buf][vid x 64 | doc x 64] int32
  static constexpr int kLdsRed = kLdsMeta + 2 * 512;
  static constexpr int kLdsBytes = kLdsRed + 64;
  static_assert(kLdsBytes <= 160 * 1024, "LDS budget");
};

template <bool META>
struct DqRolesKernel {
  using C = DqRolesCfg;
  char G4_LDS* smem;
  const BwdParams* a;
  Seq sq;
  int lane, wave, role, qg, dh, h32;
  int my_a, my_vid, my_doc, a0;
  bool has_vid, has_doc, has_meta, q_valid;
  float my_lse2, my_delta;
  const __bf16* kbase;
  const __bf16* vbase;
  int64_t kstride, vstride;
  RowReader<C::kCPR> rrd;
  TrReader<C::kCPR> trd;
  TileCopier<C::kCPR, C::kBN, C::kNW> kcp, vcp;
  bf16x8 frag[C::kNC];  // Q (S waves) or dO (dP waves) fragments, B operands
  f32x16 acc[C::kNB];   // dQ^T over this wave's head-dim quarter

  __device__ __forceinline__ void issue_k(int row0, int buf) {
    kcp.issue_clamped(kbase + row0 * kstride, kstride, min(C::kBN, sq.lk - row0),
                      smem + C::kLdsK + buf * C::kTile);
    if (has_meta && wave == 0)
      issue_key_meta(a->p, sq, row0, smem + C::kLdsMeta + buf * 512, lane, has_vid, has_doc);
  }
  __device__ __forceinline__ void issue_v(int row0) {
    vcp.issue_clamped(vbase + row0 * vstride, vstride, min(C::kBN, sq.lk - row0),
                      smem + C::kLdsV);
  }
  __device__ __forceinline__ char G4_LDS* xslot(int sl, int q4) const {
    return smem + C::kLdsX + ((sl * 4 + q4) * 64 + lane) * 16;
  }


  __device__ __forceinline__ void step(int cur, int it, int ntiles, int t_first) {
    const int kb0 = (t_first + it) * C::kBN;
    vm_wait<0>();
    barrier_lds();  // B1
    const char G4_LDS* kt = smem + C::kLdsK + cur * C::kTile;
    const char G4_LDS* vt = smem + C::kLdsV;

    __builtin_amdgcn_sched_barrier(0);
    f32x16 part = f32x16{};
    if (it + 1 < ntiles) issue_k(kb0 + C::kBN, cur ^ 1);
    row_steps(rrd, role == 0 ? kt : vt, part, frag);
    __builtin_amdgcn_sched_barrier(0);
    const int own = 4 * qg + 2 * role + dh;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4)
      *(f32x4 G4_LDS*)xslot(own, q4) =
          f32x4{part[4 * q4], part[4 * q4 + 1], part[4 * q4 + 2], part[4 * q4 + 3]};
    barrier_lds();  // B2
    if (it + 1 < ntiles) issue_v(kb0 + C::kBN);

    // Full S and dP: half 0 + half 1, the same bits in every wave of the group.
    f32x16 sv, pv;
    const int s0 = 4 * qg, p0 = 4 * qg + 2;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      f32x4 a0v, a1v, b0v, b1v;
      if (role == 0) {
        const f32x4 mine = f32x4{part[4 * q4], part[4 * q4 + 1], part[4 * q4 + 2], part[4 * q4 + 3]};
        const f32x4 other = *(const f32x4 G4_LDS*)xslot(s0 + (dh ^ 1), q4);
        a0v = dh == 0 ? mine : other;
        a1v = dh == 0 ? other : mine;
        b0v = *(const f32x4 G4_LDS*)xslot(p0, q4);
        b1v = *(const f32x4 G4_LDS*)xslot(p0 + 1, q4);
      } else {
        const f32x4 mine = f32x4{part[4 * q4], part[4 * q4 + 1], part[4 * q4 + 2], part[4 * q4 + 3]};
        const f32x4 other = *(const f32x4 G4_LDS*)xslot(p0 + (dh ^ 1), q4);
        b0v = dh == 0 ? mine : other;
        b1v = dh == 0 ? other : mine;
        a0v = *(const f32x4 G4_LDS*)xslot(s0, q4);
        a1v = *(const f32x4 G4_LDS*)xslot(s0 + 1, q4);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sv[4 * q4 + e] = a0v[e] + a1v[e];
        pv[4 * q4 + e] = b0v[e] + b1v[e];
      }
    }

    // Rows of the partials are keys 8 (r >> 2) + 4 h32 + (r & 3) of the tile;
    // lanes own queries.
    const bool full = !has_doc && (kb0 + C::kBN <= sq.lk) && (kb0 + C::kBN - 1 <= a0) &&
                      (a->p.window <= 0 || kb0 > a0 + C::kBM - 1 - a->p.window);
    const int lo_w = a->p.window > 0 ? my_a - a->p.window + 1 : -0x40000000;
    const int hi_c = min(my_a, sq.lk - 1);
    const int* km = (const int*)(smem + C::kLdsMeta + cur * 512);
    bf16x8 dsb[2];
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const int jl0 = 8 * r4 + 4 * h32;
      i32x4 vk = {-1, -1, -1, -1}, dk = {0, 0, 0, 0};
      if (has_meta && !full) {
        vk = *(const i32x4*)(km + jl0);
        dk = *(const i32x4*)(km + 64 + jl0);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = r4 * 4 + e;
        float p = fast_exp2(sv[r] * kLog2e - my_lse2);
        if (!full) {
          const int j = kb0 + jl0 + e;
          const bool in_w = j >= lo_w;
          const bool causal = in_w & (j <= hi_c);
          const bool vis = has_vid & (my_vid >= 0) & (vk[e] == my_vid) & in_w & (j < sq.lk);
          const bool doc_ok = !has_doc | (dk[e] == my_doc);
          p = ((causal | vis) & doc_ok & q_valid) ? p : 0.f;
        }
        dsb[r >> 3][r & 7] = (__bf16)(p * (pv[r] - my_delta));
      }
    }

    __builtin_amdgcn_sched_barrier(0);
    acc_steps(trd, kt, dsb, acc);
    __builtin_amdgcn_sched_barrier(0);
  }
};

template <bool META>
__global__ void __launch_bounds__(DqRolesCfg::kNT, 1) dq_roles_kernel(BwdParams a) {
  using K = DqRolesKernel<META>;
  using C = DqRolesCfg;
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  K ker;
  ker.smem = (char G4_LDS*)smem_raw;
  ker.a = &a;
  const g4_problem& p = a.p;
  const int tid = threadIdx.x;
  ker.lane = tid & 63;
  ker.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  ker.role = ker.wave >> 2;
  ker.qg = (ker.wave >> 1) & 1;
  ker.dh = ker.wave & 1;
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
  const int t_first = klo / C::kBN;
  const int ntiles = (khi + C::kBN - 1) / C::kBN - t_first;
  if (ker.has_doc &&
      doc_uniform<C::kNW>(p.document_ids, sq.ktok, sq.lk, min(klo / 64 * 64, ker.a0),
                          max((khi + 63) / 64 * 64, a_last_valid + 1), tid, ker.lane,
                          ker.wave, (int*)(smem_raw + C::kLdsRed))) {
    ker.has_doc = false;
    ker.has_meta = ker.has_vid;
  }

  ker.kbase = a.k + tok_off(sq, s, sq.ktok, 0, a.kl) + (int64_t)kvh * a.kl.head_stride;
  ker.vbase = a.v + tok_off(sq, s, sq.ktok, 0, a.vl) + (int64_t)kvh * a.vl.head_stride;
  ker.kstride = a.kl.token_stride;
  ker.vstride = a.vl.token_stride;
  ker.rrd.init(ker.lane, ker.dh * C::kDH * 2);
  ker.trd.init(ker.lane, (ker.dh * C::kDH + ker.role * C::kDQ) * 2);
  ker.kcp.init(ker.kstride, ker.wave, ker.lane);
  ker.vcp.init(ker.vstride, ker.wave, ker.lane);

  const int my_i = i0 + ker.qg * 32 + l32;
  ker.my_a = my_i + off;
  ker.q_valid = my_i < sq.lq;
  const int ic = min(my_i, sq.lq - 1);
  {
    const __bf16* row =
        ker.role == 0
            ? a.q + tok_off(sq, s, sq.qtok, ic, a.ql) + (int64_t)qh * a.ql.head_stride
            : a.dout + tok_off(sq, s, sq.qtok, ic, a.dol) + (int64_t)qh * a.dol.head_stride;
    row += ker.dh * C::kDH + ker.h32 * 8;
#pragma unroll
    for (int c = 0; c < C::kNC; ++c) ker.frag[c] = ld_global16(row + c * 16);
  }
  ker.my_lse2 = a.lse[lse_off(p, sq, s, qh, ic)] * kLog2e;
  ker.my_delta = a.delta[(int64_t)qh * q_stream_tokens_dev(p) + sq.qtok + ic];
  ker.my_vid = ker.has_vid ? p.vision_ids[sq.ktok + ic + off] : -1;
  ker.my_doc = ker.has_doc ? p.document_ids[sq.ktok + ic + off] : 0;
#pragma unroll
  for (int b = 0; b < C::kNB; ++b) ker.acc[b] = f32x16{};

  if (ntiles > 0) {
    ker.issue_k(t_first * C::kBN, 0);
    ker.issue_v(t_first * C::kBN);
  }
  for (int it = 0; it < ntiles; ++it) ker.step(it & 1, it, ntiles, t_first);

  if (ker.q_valid) {
    __bf16* row = a.dq + tok_off(sq, s, sq.qtok, my_i, a.dql) + (int64_t)qh * a.dql.head_stride;
#pragma unroll
    for (int b = 0; b < C::kNB; ++b)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d = ker.dh * C::kDH + ker.role * C::kDQ + b * 32 + 8 * r4 + 4 * ker.h32;
        const f32x16& x = ker.acc[b];
        *(bf16x4*)(row + d) = bf16x4{(__bf16)x[r4 * 4], (__bf16)x[r4 * 4 + 1],
                                     (__bf16)x[r4 * 4 + 2], (__bf16)x[r4 * 4 + 3]};
      }
  }
}

// ===========================================================================
// dQ for head dim 256 with role-specialised waves.
//
// A workgroup owns 128 queries (four groups of 32) of one query head and walks
// the 32-key tiles its range admits.  Per query group an S wave (Q fragments)
// forms S^T and P, a dP wave (dO fragments) forms dP^T; each publishes its
// tile in fp32, reads the other's and forms the same dS, and accumulates dQ^T
// over one head-dim half.  Per key tile two barriers:
//   B1  K(t), V(t) and key metadata have landed; K(t+1) goes out.
//   B2  P and dP published; V(t+1) goes out (V is read only before B2).
// ===========================================================================

struct DqRoles256Cfg {
  static constexpr int D = 256;
  static constexpr int kNW = 8;
  static constexpr int kNT = kNW * 64;
  static constexpr int kBM = 128;  // queries per workgroup
  static constexpr int kBN = 32;   // keys per tile
  static constexpr int kDQ = 128;  // head-dim half of a dQ accumulator
  static constexpr int kCPR = D / 8;
  static constexpr int kNC = D / 16;
  static constexpr int kNB = kDQ / 32;
  static constexpr int kTile = kBN * D * 2;
  static constexpr int kLdsK = 0;                  // [2 buf] K tiles
  static constexpr int kLdsV = kLdsK + 2 * kTile;  // one V tile
  // Published tiles: [slot = 2 qg + role][4][64 lanes][4 f32] (P, dP).
  static constexpr int kLdsX = kLdsV + kTile;
  static constexpr int kLdsMeta = kLdsX + 8 * 4096;  // [buf][vid x 64 | doc x 64] int32
  static constexpr int kLdsRed = kLdsMeta + 2 * 512;
  static constexpr int kLdsBytes = kLdsRed + 64;
  static_assert(kLdsBytes <= 160 * 1024, "LDS budget");
};

template <bool META>
struct DqRoles256Kernel {
  using C = DqRoles256Cfg;
  char G4_LDS* smem;
  const BwdParams* a;
  Seq sq;
  int lane, wave, role, qg, h32;
  int my_a, my_vid, my_doc, a0;
  bool has_vid, has_doc, has_meta, q_valid;
  float my_lse2, my_delta;
  const __bf16* kbase;
  const __bf16* vbase;
  int64_t kstride, vstride;
  RowReader<C::kCPR> rrd;
  TrReader<C::kCPR> trd;
  TileCopier<C::kCPR, C::kBN, C::kNW> kcp, vcp;
  bf16x8 frag[C::kNC];  // Q (S waves) or dO (dP waves) fragments
  f32x16 acc[C::kNB];   // dQ^T over this wave's head-dim half

  __device__ __forceinline__ void issue_k(int row0, int buf) {
    kcp.issue_clamped(kbase + row0 * kstride, kstride, min(C::kBN, sq.lk - row0),
                      smem + C::kLdsK + buf * C::kTile);
    if (has_meta && wave == 0)
      issue_key_meta(a->p, sq, row0, smem + C::kLdsMeta + buf * 512, lane, has_vid, has_doc);
  }
  __device__ __forceinline__ void issue_v(int row0) {
    vcp.issue_clamped(vbase + row0 * vstride, vstride, min(C::kBN, sq.lk - row0),
                      smem + C::kLdsV);
  }
  __device__ __forceinline__ char G4_LDS* xslot(int sl, int q4) const {
    return smem + C::kLdsX + ((sl * 4 + q4) * 64 + lane) * 16;
  }

  // Rows of the tiles are keys 8 (r >> 2) + 4 h32 + (r & 3); lanes own queries.
  __device__ __forceinline__ void step(int cur, int it, int ntiles, int t_first) {
    const int kb0 = (t_first + it) * C::kBN;
    vm_wait<0>();
    barrier_lds();  // B1
    const char G4_LDS* kt = smem + C::kLdsK + cur * C::kTile;
    const char G4_LDS* vt = smem + C::kLdsV;

    __builtin_amdgcn_sched_barrier(0);
    f32x16 part = f32x16{};
    if (it + 1 < ntiles) issue_k(kb0 + C::kBN, cur ^ 1);
    row_steps(rrd, role == 0 ? kt : vt, part, frag);
    __builtin_amdgcn_sched_barrier(0);

    if (role == 0) {
      // S -> P (masked), in place.
      const bool full = !has_doc && (kb0 + C::kBN <= sq.lk) && (kb0 + C::kBN - 1 <= a0) &&
                        (a->p.window <= 0 || kb0 > a0 + C::kBM - 1 - a->p.window);
      const int lo_w = a->p.window > 0 ? my_a - a->p.window + 1 : -0x40000000;
      const int hi_c = min(my_a, sq.lk - 1);
      const int* km = (const int*)(smem + C::kLdsMeta + cur * 512);
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int jl0 = 8 * r4 + 4 * h32;
        i32x4 vk = {-1, -1, -1, -1}, dk = {0, 0, 0, 0};
        if (has_meta && !full) {
          vk = *(const i32x4*)(km + jl0);
          dk = *(const i32x4*)(km + 64 + jl0);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = r4 * 4 + e;
          float p = fast_exp2(part[r] * kLog2e - my_lse2);
          if (!full) {
            const int j = kb0 + jl0 + e;
            const bool in_w = j >= lo_w;
            const bool causal = in_w & (j <= hi_c);
            const bool vis = has_vid & (my_vid >= 0) & (vk[e] == my_vid) & in_w & (j < sq.lk);
            const bool doc_ok = !has_doc | (dk[e] == my_doc);
            p = ((causal | vis) & doc_ok & q_valid) ? p : 0.f;
          }
          part[r] = p;
        }
      }
    }
    const int own = 2 * qg + role;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4)
      *(f32x4 G4_LDS*)xslot(own, q4) =
          f32x4{part[4 * q4], part[4 * q4 + 1], part[4 * q4 + 2], part[4 * q4 + 3]};
    barrier_lds();  // B2
    if (it + 1 < ntiles) issue_v(kb0 + C::kBN);

    // dS = P (dP - delta) from the same fp32 values in both waves of the group.
    bf16x8 dsb[2];
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const f32x4 other = *(const f32x4 G4_LDS*)xslot(own ^ 1, q4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 4 * q4 + e;
        const float pp = role == 0 ? part[r] : other[e];
        const float dp = role == 0 ? other[e] : part[r];
        dsb[r >> 3][r & 7] = (__bf16)(pp * (dp - my_delta));
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    acc_steps(trd, kt, dsb, acc);
    __builtin_amdgcn_sched_barrier(0);
  }
};

// Work item L: (KV head, sequence, query tile, head of the group).
template <bool META, bool QUEUE>
__device__ __forceinline__ void dq_roles256_item(const BwdParams& a, char* smem_raw, int L) {
  using K = DqRoles256Kernel<META>;
  using C = DqRoles256Cfg;
  K ker;
  ker.smem = (char G4_LDS*)smem_raw;
  ker.a = &a;
  const g4_problem& p = a.p;
  const int tid = item_thread_id<QUEUE>();
  ker.lane = tid & 63;
  ker.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  ker.role = ker.wave >> 2;
  ker.qg = ker.wave & 3;
  ker.h32 = ker.lane >> 5;
  const int l32 = ker.lane & 31;

  const int grp = p.num_q_heads / p.num_kv_heads;
  int kvh, qh, s, qt;
  const bool listed = a.dq_recompute_only && a.dq_list != nullptr;
  if (listed) {
    // Entry L of the stored-dS pass's list: a tile known to need recomputing.
    const int4 e = a.dq_list[L];
    s = __builtin_amdgcn_readfirstlane(e.x);
    qt = __builtin_amdgcn_readfirstlane(e.y);
    qh = __builtin_amdgcn_readfirstlane(e.z);
    kvh = qh / grp;
  } else {
    const int per_kvh = a.num_seqs * a.ntiles * grp;
    kvh = L / per_kvh;
    const int rem = L % per_kvh;
    const int rank = rem / grp;
    qh = kvh * grp + rem % grp;
    s = rank / a.ntiles;
    qt = zigzag(rank % a.ntiles, a.ntiles);
  }
  ker.sq = resolve_seq(p, s);
  const Seq& sq = ker.sq;
  const int i0 = qt * C::kBM;
  if (i0 >= sq.lq) return;
  const int off = sq.lk - sq.lq;
  if (a.dq_recompute_only && !listed) {
    int kt_hi[4];
    if (!dq_row_key_ends<C::kNW>(a, sq, i0, off, tid, (int*)(smem_raw + C::kLdsRed), kt_hi))
      return;
  }
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
  const int t_first = klo / C::kBN;
  const int ntiles = (khi + C::kBN - 1) / C::kBN - t_first;
  if (ker.has_doc &&
      doc_uniform<C::kNW>(p.document_ids, sq.ktok, sq.lk, min(klo / 64 * 64, ker.a0),
                          max((khi + 63) / 64 * 64, a_last_valid + 1), tid, ker.lane,
                          ker.wave, (int*)(smem_raw + C::kLdsRed))) {
    ker.has_doc = false;
    ker.has_meta = ker.has_vid;
  }

  ker.kbase = a.k + tok_off(sq, s, sq.ktok, 0, a.kl) + (int64_t)kvh * a.kl.head_stride;
  ker.vbase = a.v + tok_off(sq, s, sq.ktok, 0, a.vl) + (int64_t)kvh * a.vl.head_stride;
  ker.kstride = a.kl.token_stride;
  ker.vstride = a.vl.token_stride;
  ker.rrd.init(ker.lane, 0);
  ker.trd.init(ker.lane, ker.role * C::kDQ * 2);
  ker.kcp.init(ker.kstride, ker.wave, ker.lane);
  ker.vcp.init(ker.vstride, ker.wave, ker.lane);

  const int my_i = i0 + ker.qg * 32 + l32;
  ker.my_a = my_i + off;
  ker.q_valid = my_i < sq.lq;
  const int ic = min(my_i, sq.lq - 1);
  {
    const __bf16* row =
        ker.role == 0
            ? a.q + tok_off(sq, s, sq.qtok, ic, a.ql) + (int64_t)qh * a.ql.head_stride
            : a.dout + tok_off(sq, s, sq.qtok, ic, a.dol) + (int64_t)qh * a.dol.head_stride;
    row += ker.h32 * 8;
#pragma unroll
    for (int c = 0; c < C::kNC; ++c) ker.frag[c] = ld_global16(row + c * 16);
  }
  ker.my_lse2 = a.lse[lse_off(p, sq, s, qh, ic)] * kLog2e;
  ker.my_delta = a.delta[(int64_t)qh * q_stream_tokens_dev(p) + sq.qtok + ic];
  ker.my_vid = ker.has_vid ? p.vision_ids[sq.ktok + ic + off] : -1;
  ker.my_doc = ker.has_doc ? p.document_ids[sq.ktok + ic + off] : 0;
#pragma unroll
  for (int b = 0; b < C::kNB; ++b) ker.acc[b] = f32x16{};

  if (ntiles > 0) {
    ker.issue_k(t_first * C::kBN, 0);
    ker.issue_v(t_first * C::kBN);
  }
  for (int it = 0; it < ntiles; ++it) ker.step(it & 1, it, ntiles, t_first);

  if (ker.q_valid) {
    __bf16* row = a.dq + tok_off(sq, s, sq.qtok, my_i, a.dql) + (int64_t)qh * a.dql.head_stride;
#pragma unroll
    for (int b = 0; b < C::kNB; ++b)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d = ker.role * C::kDQ + b * 32 + 8 * r4 + 4 * ker.h32;
        const f32x16& x = ker.acc[b];
        *(bf16x4*)(row + d) = bf16x4{(__bf16)x[r4 * 4], (__bf16)x[r4 * 4 + 1],
                                     (__bf16)x[r4 * 4 + 2], (__bf16)x[r4 * 4 + 3]};
      }
  }
}

// Persistent: a few workgroups per CU take query-tile tickets from the dQ
// work queue.
template <bool META, bool QUEUE>
__global__ void __launch_bounds__(DqRoles256Cfg::kNT, 1) dq_roles256_kernel(BwdParams a) {
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  // The recompute launch after a stored-dS pass takes its items from that
  // pass's list (at most one entry per query tile and head).
  const int all = a.num_seqs * a.ntiles * a.p.num_q_heads;
  const int n = a.dq_recompute_only && a.dq_list != nullptr
                    ? min(__builtin_amdgcn_readfirstlane((int)a.sched[3]), all)
                    : all;
  if constexpr (QUEUE) {
    WorkQueue wq{a.sched + 2, n, 0};
    for (;;) {
      const int t = wq.next((int G4_LDS*)smem_raw);
      if (t >= n) break;
      dq_roles256_item<META, true>(a, smem_raw, t);
    }
  } else {
    const int t = xcd_remap(blockIdx.x, gridDim.x);
    if (t < n) dq_roles256_item<META, false>(a, smem_raw, t);
  }
}

// ===========================================================================
// dQ for head dim 512 from the dS tiles the dK/dV kernel wrote:
// dQ^T = K^T dS^T, no recomputation of S or dP.
//
// A workgroup owns 128 queries (four 32-query tile rows) of one query head and
// walks the 64-key tiles of their causal range; eight waves, wave w holding
// dQ^T for two rows (2 (w >> 2) + {0, 1}) over head-dim quarter w & 3.  Both
// operands come from transposing LDS reads with the same reduction-dim order:
// K^T from the swizzled K tile, dS^T from the plain [64 keys][32 queries]
// tile.  A row's tiles past its own causal range were never written and are
// skipped.  One barrier per key tile (copies one tile ahead).
// ===========================================================================

template <int D_>
struct DqDsCfg {
  static constexpr int D = D_;
  static constexpr int kNW = 8;
  static constexpr int kNT = kNW * 64;
  static constexpr int kBM = 128;  // queries per workgroup (four tile rows)
  static constexpr int kBN = 64;   // keys per tile
  static constexpr int kCPR = D / 8;
  static constexpr int kKTile = kBN * D * 2;
  // Query heads per item: at head dim 256 the two heads of a GQA pair share
  // the item's K tiles (halving K copies per query); the register file has
  // room for both heads' dQ only there.
  static constexpr int kHeads = D == 256 ? 2 : 1;
  static constexpr int kLdsK = 0;                    // [2 buf] K tiles
  static constexpr int kLdsDs = 2 * kKTile;          // [2 buf][kHeads][4 rows] dS tiles
  static constexpr int kLdsBytes = kLdsDs + 2 * kHeads * 4 * 4096;
  static constexpr int kDW = D / 4;      // head dims per wave
  static constexpr int kNBw = kDW / 32;  // 32-wide head-dim blocks per wave
  static_assert(kLdsBytes <= 160 * 1024, "LDS budget");
};

// Transposing reads of a plain (unswizzled) tile of 64-byte rows (32 bf16
// columns): the MFMA operand [32 columns x 16 rows] with the same row order as
// TrReader's.
struct PlainTrReader {
  int base[2];
  __device__ __forceinline__ void init(int lane) {
    const int g = lane >> 4, sl = lane & 15;
    const int rl = 4 * (g >> 1) + (sl >> 2);
    const int lb = 2 * (g & 1) + ((sl >> 1) & 1);
    const int half = (sl & 1) * 8;
#pragma unroll
    for (int e = 0; e < 2; ++e) base[e] = (rl + 8 * e) * 64 + 16 * lb + half;
  }
  template <int ROW0>
  __device__ __forceinline__ bf16x8 read(const char G4_LDS* tile) const {
    bf16x4 lo = lds_read_tr<true>(tile + base[0] + ROW0 * 64);
    bf16x4 hi = lds_read_tr<true>(tile + base[1] + ROW0 * 64);
    return cat4(lo, hi);
  }
};

// TrReader's transposing reads of NB consecutive 32-column blocks starting at
// block B0 (runtime, wave-uniform): block B sits at chunk group B >> 2 with
// its 4-chunk slot XORed by 64 (B & 3) bytes, so each block keeps its own pair
// of per-lane bases (TrReader's column offset must be a multiple of 256
// bytes, which a quarter of a 256-wide row is not).
template <int CPR, int NB>
struct BlockTrReader {
  int base[NB][2];
  __device__ __forceinline__ void init(int lane, int b0) {
    TrReader<CPR> t;
    t.init(lane, 0);
#pragma unroll
    for (int k = 0; k < NB; ++k)
#pragma unroll
      for (int e = 0; e < 2; ++e)
        base[k][e] = (t.base[e] ^ (64 * ((b0 + k) & 3))) + 256 * ((b0 + k) >> 2);
  }
  template <int ROW0, int K>
  __device__ __forceinline__ bf16x8 read(const char G4_LDS* tile) const {
    constexpr int imm = ROW0 * CPR * 16;
    bf16x4 lo = lds_read_tr<true>(tile + base[K][0] + imm);
    bf16x4 hi = lds_read_tr<true>(tile + base[K][1] + imm);
    return cat4(lo, hi);
  }
};

// dS tile addressing for the two layouts (see BwdParams::ds): the tile of
// workgroup row g (0..3) and key tile c is at base + g * row_stride +
// (c - first[g]) * col_stride.
template <int D>
struct DqDsKernel {
  using C = DqDsCfg<D>;
  char G4_LDS* smem;
  const BwdParams* a;
  Seq sq;
  int lane, wave, h32, dquart, qpair;
  // Key-tile range [lo, hi] (hi = -1: row past the sequence) of this wave's
  // two tile rows and of the row whose dS tiles this wave copies.
  int lo0, hi0, lo1, hi1, lo_copy, hi_copy;
  const __bf16* kbase;
  int64_t kstride;
  const char* ds_copy_row;  // dS tile of key tile lo_copy in the copied row
  int64_t ds_col_stride;
  int64_t ds_head_stride;  // bytes from one query head's dS tiles to the next's
  int nh;                  // query heads of this item (1 or C::kHeads)
  BlockTrReader<C::kCPR, C::kNBw> trk;
  PlainTrReader trs;
  TileCopier<C::kCPR, C::kBN, C::kNW> kcp;
  f32x16 acc[C::kHeads][2][C::kNBw];

  __device__ __forceinline__ void issue(int kt, int buf) {
    const int row0 = kt * C::kBN;
    kcp.issue_clamped(kbase + row0 * kstride, kstride, min(C::kBN, sq.lk - row0),
                      smem + C::kLdsK + buf * C::kKTile);
    // dS: four 4 KB tiles per head, two 1 KB chunks per wave and head, each
    // read once (non-temporal: the K tiles stay in the L2 for the other
    // workgroups of the band; config 5 dQ -3%, config 3 -7%, results the same).
    const int g = wave >> 1;
    if (kt >= lo_copy && kt <= hi_copy) {
      const char* src = ds_copy_row + (int64_t)(kt - lo_copy) * ds_col_stride;
#pragma unroll
      for (int h = 0; h < C::kHeads; ++h) {
        if (h < nh) {
          char G4_LDS* dst = smem + C::kLdsDs + ((buf * C::kHeads + h) * 4 + g) * 4096;
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            const int chunk = (wave & 1) * 2 + c;
            b2l16_nt(src + h * ds_head_stride, (uint32_t)(chunk * 1024 + lane * 16),
                     dst + chunk * 1024);
          }
        }
      }
    }
  }

  template <int KS>
  __device__ __forceinline__ void kstep(const char G4_LDS* kt_tile, const char G4_LDS* dsb,
                                        bool v0, bool v1) {
    bf16x8 ak[C::kNBw];
    ak[0] = trk.template read<16 * KS, 0>(kt_tile);
    ak[1] = trk.template read<16 * KS, 1>(kt_tile);
    if constexpr (C::kNBw == 4) {
      ak[2] = trk.template read<16 * KS, 2>(kt_tile);
      ak[3] = trk.template read<16 * KS, 3>(kt_tile);
    }
#pragma unroll
    for (int h = 0; h < C::kHeads; ++h) {
      if (h >= nh) break;
      const char G4_LDS* ds0 = dsb + h * 4 * 4096;
      if (v0) {
        const bf16x8 bs = trs.template read<16 * KS>(ds0);
#pragma unroll
        for (int b = 0; b < C::kNBw; ++b) acc[h][0][b] = mfma32(ak[b], bs, acc[h][0][b]);
      }
      if (v1) {
        const bf16x8 bs = trs.template read<16 * KS>(ds0 + 4096);
#pragma unroll
        for (int b = 0; b < C::kNBw; ++b) acc[h][1][b] = mfma32(ak[b], bs, acc[h][1][b]);
      }
    }
  }

  // Both tile rows valid (the common case): the operands of step KS + 1 are
  // read while the MFMAs of step KS run, in an order sched_barrier pins.
  template <int KS>
  __device__ __forceinline__ void kread(const char G4_LDS* kt_tile, const char G4_LDS* ds0,
                                        const char G4_LDS* ds1, bf16x8 (&ak)[C::kNBw],
                                        bf16x8 (&bs)[2]) const {
    ak[0] = trk.template read<16 * KS, 0>(kt_tile);
    ak[1] = trk.template read<16 * KS, 1>(kt_tile);
    if constexpr (C::kNBw == 4) {
      ak[2] = trk.template read<16 * KS, 2>(kt_tile);
      ak[3] = trk.template read<16 * KS, 3>(kt_tile);
    }
    bs[0] = trs.template read<16 * KS>(ds0);
    bs[1] = trs.template read<16 * KS>(ds1);
  }
  template <int KS>
  __device__ __forceinline__ void kpipe(const char G4_LDS* kt_tile, const char G4_LDS* ds0,
                                        const char G4_LDS* ds1, bf16x8 (&ak)[2][C::kNBw],
                                        bf16x8 (&bs)[2][2]) {
    if constexpr (KS < 4) {
      if constexpr (KS + 1 < 4)
        kread<KS + 1>(kt_tile, ds0, ds1, ak[(KS + 1) & 1], bs[(KS + 1) & 1]);
#pragma unroll
      for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int b = 0; b < C::kNBw; ++b)
          acc[0][g][b] = mfma32(ak[KS & 1][b], bs[KS & 1][g], acc[0][g][b]);
      __builtin_amdgcn_sched_barrier(0);
      kpipe<KS + 1>(kt_tile, ds0, ds1, ak, bs);
    }
  }
  __device__ __forceinline__ void ktile_both(const char G4_LDS* kt_tile, const char G4_LDS* ds0,
                                             const char G4_LDS* ds1) {
    bf16x8 ak[2][C::kNBw], bs[2][2];
    __builtin_amdgcn_sched_barrier(0);
    kread<0>(kt_tile, ds0, ds1, ak[0], bs[0]);
    __builtin_amdgcn_sched_barrier(0);
    kpipe<0>(kt_tile, ds0, ds1, ak, bs);
  }
};


// Query heads of one dQ-from-dS item: the GQA pair at head dim 256 (both
// share their KV head's K tiles), one otherwise.
template <int D>
__host__ __device__ __forceinline__ int dq_ds_heads(const g4_problem& p) {
  return DqDsCfg<D>::kHeads > 1 && p.num_q_heads / p.num_kv_heads >= DqDsCfg<D>::kHeads
             ? DqDsCfg<D>::kHeads
             : 1;
}

// Work item L.  Head dim 512 (causal): query tile (last, i.e. heaviest, first),
// then sequence, then query head.  Head dim 256 (the band's tiles cost about
// the same): GQA head pair slowest, then sequence, then query tile (last
// first), with `compact` only the tiles that exist; neighbouring items are
// then neighbouring query tiles of one head, whose key bands overlap, and the
// launches hand each XCD a contiguous run of items, so the K tiles they share
// are read once into that XCD's L2 (config 3 dQ 0.257 -> 0.227 ms; the same
// order at head dim 512 measured 0.98 -> 1.03 ms on config 2: there the
// heaviest-first order across heads matters more).
template <int D, bool QUEUE>
__device__ __forceinline__ void dq_ds_item(const BwdParams& a, char* smem_raw, int L,
                                           const SeqTiles& tiles, bool compact) {
  using C = DqDsCfg<D>;
  DqDsKernel<D> ker;
  ker.smem = (char G4_LDS*)smem_raw;
  ker.a = &a;
  const g4_problem& p = a.p;
  const int tid = item_thread_id<QUEUE>();
  ker.lane = tid & 63;
  ker.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  ker.h32 = ker.lane >> 5;
  ker.dquart = ker.wave & 3;
  ker.qpair = ker.wave >> 2;
  const int l32 = ker.lane & 31;

  const int grp = p.num_q_heads / p.num_kv_heads;
  // Heads qh .. qh + nh - 1 (one KV head: nh divides grp).
  ker.nh = dq_ds_heads<D>(p);
  int qt, s, qh;
  if constexpr (D == 512) {
    const int hslots = p.num_q_heads / ker.nh;
    const int per_qt = a.num_seqs * hslots;
    qt = a.dq_qt_lo + a.ntiles - 1 - L / per_qt;
    const int rem = L % per_qt;
    s = rem / hslots;
    qh = rem % hslots * ker.nh;
  } else {
    const int per_slot = compact ? tiles.total : a.num_seqs * a.ntiles;
    qh = L / per_slot * ker.nh;
    const int r = L % per_slot;
    if (compact) {
      int local, nt;
      tiles.find(r, s, local, nt);
      qt = nt - 1 - local;
    } else {
      qt = a.ntiles - 1 - r / a.num_seqs;
      s = r % a.num_seqs;
    }
  }
  const int kvh = qh / grp;
  ker.sq = resolve_seq(p, s);
  const Seq& sq = ker.sq;
  const int i0 = qt * C::kBM;
  if (i0 >= sq.lq) return;
  const int off = sq.lk - sq.lq;
  constexpr bool kBand = D == 256;
  // Key tiles of row g: up to the causal end of its last query (for the band,
  // extended by its queries' vision spans) and, for the band, from the band
  // start of its first query.
  int kt_hi[4];
  if constexpr (kBand) {
    if (dq_row_key_ends<C::kNW>(a, sq, i0, off, tid, (int*)smem_raw, kt_hi)) {
      // A row reaches past the stored band: left to the recompute launch
      // (one entry per query head).
      if (tid == 0 && a.dq_list != nullptr) {
        const unsigned e = atomicAdd(&a.sched[3], (unsigned)ker.nh);
        for (int h = 0; h < ker.nh; ++h) a.dq_list[e + h] = int4{s, qt, qh + h, 0};
      }
      return;
    }
  } else {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int r0 = i0 + 32 * g;
      kt_hi[g] = r0 < sq.lq ? (min(r0 + 32, sq.lq) - 1 + off) / C::kBN : -1;
    }
  }
  auto kt_last = [&](int g) { return kt_hi[g]; };
  auto kt_first = [&](int g) {
    return kBand ? ds_band_first(i0 + 32 * g + off, p.window) : 0;
  };
  const int kt_begin = kt_first(0);
  const int nkt = max(max(kt_last(0), kt_last(1)), max(kt_last(2), kt_last(3))) + 1;
  ker.lo0 = kt_first(2 * ker.qpair);
  ker.hi0 = kt_last(2 * ker.qpair);
  ker.lo1 = kt_first(2 * ker.qpair + 1);
  ker.hi1 = kt_last(2 * ker.qpair + 1);
  const int gc = ker.wave >> 1;
  ker.lo_copy = kt_first(gc);
  ker.hi_copy = kt_last(gc);

  ker.kbase = a.k + tok_off(sq, s, sq.ktok, 0, a.kl) + (int64_t)kvh * a.kl.head_stride;
  ker.kstride = a.kl.token_stride;
  // (row stripes: the one sequence's rows; sequence stripes: rows from the
  // stripe's first, ds_row_lo, and only the stripe's sequences)
  const int64_t first_row = ds_first_row(a, sq, s);
  if (ds_seq_skipped(a, first_row)) return;
  const int64_t row0 = (a.dk_acc != nullptr ? 0 : first_row) + i0 / 32 - a.ds_row_lo;
  ker.ds_head_stride = (int64_t)a.ds_rows * a.ds_cols * 4096;
  if constexpr (kBand) {
    ker.ds_col_stride = 4096;
    ker.ds_copy_row = (const char*)a.ds + (((int64_t)qh * a.ds_rows + row0 + gc) * a.ds_cols) * 4096;
  } else {
    ker.ds_col_stride = (int64_t)a.ds_rows * 4096;
    ker.ds_copy_row = (const char*)a.ds + ((int64_t)qh * a.ds_cols * a.ds_rows + row0 + gc) * 4096;
  }
  ker.trk.init(ker.lane, ker.dquart * C::kNBw);
  ker.trs.init(ker.lane);
  ker.kcp.init(ker.kstride, ker.wave, ker.lane);
#pragma unroll
  for (int h = 0; h < C::kHeads; ++h)
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int b = 0; b < C::kNBw; ++b) ker.acc[h][g][b] = f32x16{};

  const int g0 = 2 * ker.qpair;
  if (kt_begin < nkt) ker.issue(kt_begin, 0);
  for (int kt = kt_begin; kt < nkt; ++kt) {
    const int cur = (kt - kt_begin) & 1;
    vm_wait<0>();
    barrier_lds();  // tile kt landed; every wave is done with buffer cur ^ 1
    if (kt + 1 < nkt) ker.issue(kt + 1, cur ^ 1);
    const char G4_LDS* ktile = ker.smem + C::kLdsK + cur * C::kKTile;
    const char G4_LDS* ds0 = ker.smem + C::kLdsDs + (cur * C::kHeads * 4 + g0) * 4096;
    const char G4_LDS* ds1 = ds0 + 4096;
    const bool v0 = kt >= ker.lo0 && kt <= ker.hi0, v1 = kt >= ker.lo1 && kt <= ker.hi1;
    // (The band kernel measured slower pipelined: 5.52 vs 5.39 ms on config 5;
    // with its dS copies through buffer descriptors, the same: 3.97 ms both.)
    if (!kBand && v0 && v1) {
      ker.ktile_both(ktile, ds0, ds1);
    } else {
      ker.template kstep<0>(ktile, ds0, v0, v1);
      ker.template kstep<1>(ktile, ds0, v0, v1);
      ker.template kstep<2>(ktile, ds0, v0, v1);
      ker.template kstep<3>(ktile, ds0, v0, v1);
    }
  }

  // dQ leaves through LDS: a lane's accumulators hold one query and 8-byte
  // runs of the head dim, so storing them directly writes 8 bytes into each
  // of 32 rows per instruction.  They are staged as bf16 rows of the
  // 128-query tile (chunk c of row r at slot c ^ (r mod kCPR), which keeps the
  // 32-row staging writes and the row reads free of bank conflicts) and
  // written back as whole rows.  Band tiles keep queries in accumulator
  // order, dense tiles in query order.
  char G4_LDS* stage = ker.smem;
  static_assert(C::kBM * C::kCPR * 16 <= C::kLdsBytes, "dQ staging tile");
  constexpr int kRowsPerInst = 64 / C::kCPR;
#pragma unroll
  for (int h = 0; h < C::kHeads; ++h) {
    if (h >= ker.nh) break;
    barrier_lds();  // every wave is done with the operands / the previous head's rows
#pragma unroll
    for (int g2 = 0; g2 < 2; ++g2) {
      const int r = 32 * (g0 + g2) + (kBand ? ds_query_at(l32) : l32);
#pragma unroll
      for (int b = 0; b < C::kNBw; ++b)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const int d = ker.dquart * C::kDW + b * 32 + 8 * r4 + 4 * ker.h32;
          const f32x16& x = ker.acc[h][g2][b];
          *(bf16x4 G4_LDS*)(stage + (r * C::kCPR + ((d >> 3) ^ (r & (C::kCPR - 1)))) * 16 +
                            (d & 4) * 2) =
              bf16x4{(__bf16)x[r4 * 4], (__bf16)x[r4 * 4 + 1], (__bf16)x[r4 * 4 + 2],
                     (__bf16)x[r4 * 4 + 3]};
        }
    }
    barrier_lds();
#pragma unroll
    for (int j = 0; j < C::kBM / (C::kNW * kRowsPerInst); ++j) {
      const int r = (j * C::kNW + ker.wave) * kRowsPerInst + ker.lane / C::kCPR;
      const int c = ker.lane % C::kCPR;
      const int my_i = i0 + r;
      if (my_i < sq.lq) {
        const bf16x8 v =
            *(const bf16x8 G4_LDS*)(stage + (r * C::kCPR + (c ^ (r & (C::kCPR - 1)))) * 16);
        __bf16* row =
            a.dq + tok_off(sq, s, sq.qtok, my_i, a.dql) + (int64_t)(qh + h) * a.dql.head_stride;
        __builtin_nontemporal_store(v, (bf16x8*)(row + c * 8));  // (written once)
      }
    }
  }
}

// Persistent (QUEUE): a few workgroups per CU take items from the dQ work
// queue: head dim 512 the heaviest tiles first from one queue, head dim 256
// each XCD from its own contiguous run (XcdQueue).
template <int D, bool QUEUE>
__global__ void __launch_bounds__(DqDsCfg<D>::kNT, 1) dq_ds_kernel(BwdParams a) {
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  if constexpr (QUEUE) {
    // An item leaves no tile copy in flight, only its dQ stores.
    SeqTiles tiles;
    tiles.init(a.p.cu_seqlens_q, a.num_seqs, DqDsCfg<D>::kBM);
    const bool compact = D == 256 && tiles.ok;
    const int hslots = a.p.num_q_heads / dq_ds_heads<D>(a.p);
    const unsigned n = compact ? (unsigned)(tiles.total * hslots)
                               : (unsigned)(a.num_seqs * a.ntiles * hslots);
    if constexpr (D == 512) {
      PrefetchQueue q{a.sched + 2, n};
      for (int t = q.first(); q.valid(t); t = q.next((int G4_LDS*)smem_raw)) {
        q.draw();
        dq_ds_item<D, true>(a, smem_raw, t, tiles, false);
      }
    } else {
      XcdQueue q{a.sched + kDqXcdQueue, n};
      q.draw();
      for (int t = q.next((int G4_LDS*)smem_raw); t >= 0; t = q.next((int G4_LDS*)smem_raw)) {
        q.draw();
        dq_ds_item<D, true>(a, smem_raw, t, tiles, compact);
      }
    }
  } else {
    dq_ds_item<D, false>(a, smem_raw, xcd_remap(blockIdx.x, gridDim.x), SeqTiles{}, false);
  }
}

}  // namespace


template <int D>
static hipError_t launch_dq_ds(const BwdParams& a, hipStream_t stream) {
  using C = DqDsCfg<D>;
  static LdsAttr attr[2];
  BwdParams b = a;
  // (striped: the stripe's 128-query tiles, from dq_qt_lo)
  b.ntiles = a.dk_acc != nullptr ? (a.ds_rows + 3) / 4 : (a.p.seqlen_q + C::kBM - 1) / C::kBM;
  const int64_t items =
      (int64_t)b.num_seqs * b.ntiles * (a.p.num_q_heads / dq_ds_heads<D>(a.p));
  if (items <= 0) return hipSuccess;
  static PersistentGrid grid;
  bool queue = false;
  const int64_t nblocks =
      grid.size((const void*)dq_ds_kernel<D, true>, C::kNT, C::kLdsBytes, items, &queue);
  if (nblocks <= 0) return hipErrorInvalidValue;
  void (*kern)(BwdParams) = queue ? dq_ds_kernel<D, true> : dq_ds_kernel<D, false>;
  hipError_t e = attr[queue].ensure((const void*)kern, C::kLdsBytes);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3((unsigned)nblocks), dim3(C::kNT), C::kLdsBytes, stream, b);
  return hipGetLastError();
}

template <int D>
hipError_t launch_dq_roles_d(const BwdParams& a, hipStream_t stream) {
  using C = std::conditional_t<D == 512, DqRolesCfg, DqRoles256Cfg>;
  const bool meta = (a.p.vision_ids != nullptr && a.p.bidirectional_vision) ||
                    a.p.document_ids != nullptr;
  BwdParams b = a;
  b.ntiles = (a.p.seqlen_q + C::kBM - 1) / C::kBM;
  const int64_t items = (int64_t)b.num_seqs * b.ntiles * a.p.num_q_heads;
  if (items <= 0) return hipSuccess;
  int64_t nblocks = items;  // head dim 512: one workgroup per query tile
  bool queue = false;
  void (*kern)(BwdParams);
  if constexpr (D == 512) {
    kern = meta ? dq_roles_kernel<true> : dq_roles_kernel<false>;
  } else {
    static PersistentGrid grid;
    nblocks = grid.size((const void*)(meta ? dq_roles256_kernel<true, true>
                                           : dq_roles256_kernel<false, true>),
                        C::kNT, C::kLdsBytes, items, &queue);
    if (nblocks <= 0) return hipErrorInvalidValue;
    kern = meta ? (queue ? dq_roles256_kernel<true, true> : dq_roles256_kernel<true, false>)
                : (queue ? dq_roles256_kernel<false, true> : dq_roles256_kernel<false, false>);
  }
  static LdsAttr attr[4];
  hipError_t e = attr[2 * meta + queue].ensure((const void*)kern, C::kLdsBytes);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3((unsigned)nblocks), dim3(C::kNT), C::kLdsBytes, stream, b);
  return hipGetLastError();
}

static_assert(DqRoles256Cfg::kBM == DqDsCfg<256>::kBM,
              "the recompute list holds stored-dS pass query tiles");

__global__ void clear_counter_kernel(unsigned* c) {
  if (threadIdx.x == 0) *c = 0u;
}

hipError_t launch_bwd_dq(const BwdParams& a, hipStream_t stream) {
  // With the dK/dV kernel's dS tiles in the workspace, dQ is a plain product.
  if (a.p.head_dim == 512) {
    if (a.ds != nullptr) return launch_dq_ds<512>(a, stream);
    return launch_dq_roles_d<512>(a, stream);
  }
  if (a.p.head_dim == 256) {
    if (a.ds == nullptr) return launch_dq_roles_d<256>(a, stream);
    if (a.dq_list != nullptr) {
      // The list is refilled by every stored-dS pass (a fill kernel, not a
      // memset node, so the launch sequence can be captured in a graph).
      hipLaunchKernelGGL(clear_counter_kernel, dim3(1), dim3(64), 0, stream, a.sched + 3);
      hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
    hipError_t e = launch_dq_ds<256>(a, stream);
    if (e != hipSuccess || a.p.vision_ids == nullptr || !a.p.bidirectional_vision) return e;
    // Query tiles with vision spans past the stored band: recomputed.
    BwdParams b = a;
    b.dq_recompute_only = 1;
    return launch_dq_roles_d<256>(b, stream);
  }
  return hipErrorInvalidValue;
}

template <int D>
hipError_t launch_dkdv_roles_d(const BwdParams& a, hipStream_t stream) {
  using C = std::conditional_t<D == 512, RolesCfg, Roles256Cfg>;
  const bool meta = (a.p.vision_ids != nullptr && a.p.bidirectional_vision) ||
                    a.p.document_ids != nullptr;
  BwdParams b = a;
  b.ntiles = (a.p.seqlen_k + C::kBN - 1) / C::kBN;
  // Head dim 512: one item per pair of key tiles (see dkdv_roles_pair).
  const int64_t per_seq = D == 512 ? (b.ntiles + 1) / 2 : b.ntiles;
  const int64_t items = (int64_t)b.num_seqs * per_seq * a.p.num_kv_heads;
  if (items <= 0) return hipSuccess;
  void (*kq[2])(BwdParams);  // [meta] queue variants
  void (*ks[2])(BwdParams);  // [meta] one workgroup per item
  const bool striped = D == 512 && a.dk_acc != nullptr;
  if constexpr (D == 512) {
    if (striped) {
      kq[0] = dkdv_roles_kernel<false, true, true>;
      kq[1] = dkdv_roles_kernel<true, true, true>;
      ks[0] = dkdv_roles_kernel<false, false, true>;
      ks[1] = dkdv_roles_kernel<true, false, true>;
    } else {
      kq[0] = dkdv_roles_kernel<false, true, false>;
      kq[1] = dkdv_roles_kernel<true, true, false>;
      ks[0] = dkdv_roles_kernel<false, false, false>;
      ks[1] = dkdv_roles_kernel<true, false, false>;
    }
  } else {
    kq[0] = dkdv_roles256_kernel<false, true>;
    kq[1] = dkdv_roles256_kernel<true, true>;
    ks[0] = dkdv_roles256_kernel<false, false>;
    ks[1] = dkdv_roles256_kernel<true, false>;
  }
  static PersistentGrid grid;
  bool queue = false;
  const int64_t nblocks = grid.size((const void*)kq[meta], C::kNT, C::kLdsBytes, items, &queue);
  if (nblocks <= 0) return hipErrorInvalidValue;
  void (*kern)(BwdParams) = queue ? kq[meta] : ks[meta];
  static LdsAttr attr[8];
  hipError_t e = attr[4 * striped + 2 * meta + queue].ensure((const void*)kern, C::kLdsBytes);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3((unsigned)nblocks), dim3(C::kNT), C::kLdsBytes, stream, b);
  return hipGetLastError();
}

hipError_t launch_bwd_dkdv(const BwdParams& a, hipStream_t stream) {
  if (a.p.head_dim == 512) return launch_dkdv_roles_d<512>(a, stream);
  if (a.p.head_dim == 256) return launch_dkdv_roles_d<256>(a, stream);
  return hipErrorInvalidValue;
}

}  // namespace g4
