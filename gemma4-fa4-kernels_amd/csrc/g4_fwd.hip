// Forward attention kernel for gfx950: O = softmax(Q K^T + mask) V, fp32 LSE.
//
// One workgroup owns BM = 32 * NQG queries of one query head and walks the key
// tiles its mask-aware range admits (query_tile_key_range).  Each wave owns
// 32 queries and a DH = D / DSPLIT slice of the head dimension:
//   S^T (keys x queries) = K Q^T on MFMA with the query fragments in VGPRs and
//   K read from LDS; with DSPLIT = 2 the two d-slices of a query group
//   exchange their partial S^T through LDS and add them.  Because lanes own
//   queries, the softmax row max / sum are register reductions plus one
//   cross-half shuffle.  P is rounded to bf16 and fed straight from the
//   accumulator registers as the B operand of O^T += V^T P^T, with V^T read
//   from the natural-layout V tile by transposing LDS reads.
// K and V tiles are copied global -> LDS asynchronously (one 16-byte chunk per
// lane) one tile ahead of the compute.
#include "g4_kernels.h"

namespace g4 {

template <int D, int BN, int DSPLIT, int NQG, bool VDOUBLE>
struct FwdCfg {
  static constexpr int kNW = NQG * DSPLIT;
  static constexpr int kNT = kNW * 64;
  static constexpr int kBM = NQG * 32;
  static constexpr int kDH = D / DSPLIT;
  static constexpr int kCPR = D / 8;  // 16-byte chunks per row
  static constexpr int kTileBytes = BN * D * 2;
  static constexpr int kLoadsPerWave = BN * kCPR / (64 * kNW);
  static constexpr int kKB = BN / 32;  // 32-key blocks per tile
  static constexpr int kXBytes = DSPLIT > 1 ? kNW * kKB * 4096 : 0;
  static constexpr int kVBufs = VDOUBLE ? 2 : 1;
  static constexpr int kLdsK = 0;
  static constexpr int kLdsV = kLdsK + 2 * kTileBytes;
  static constexpr int kLdsX = kLdsV + kVBufs * kTileBytes;
  static constexpr int kLdsMeta = kLdsX + kXBytes;  // [buf][vid x 64 | doc x 64] int32
  static constexpr int kLdsRed = kLdsMeta + 2 * 512;
  static constexpr int kLdsBytes = kLdsRed + 16 * 4;
  static_assert(kLdsBytes <= 160 * 1024, "LDS budget");
  static_assert(kDH % 128 == 0, "head-dim slice must be a multiple of 128");
};

// Async copy of the vision / document IDs of keys [j0, j0 + 64) of a sequence
// (clamped to its last key; keys past the end are masked by index).
__device__ __forceinline__ void issue_meta(const g4_problem& p, const Seq& sq, int j0,
                                           char G4_LDS* dst, int lane, bool vid, bool doc) {
  // uniform base at the tile's first (clamped) key, small per-lane offsets
  const int j0c = min(j0, sq.lk - 1);
  const int64_t base = sq.ktok + j0c;
  const uint32_t off = (uint32_t)(min(j0 + lane, sq.lk - 1) - j0c) * 4u;
  if (vid) b2l4(p.vision_ids + base, off, dst);
  if (doc) b2l4(p.document_ids + base, off, dst + 256);
}

// Largest score excess (log2 units) over a row's running maximum that the
// online softmax absorbs without rescaling the O accumulators.
constexpr float kRescaleLog2 = 8.0f;

// META: key metadata kinds compiled in (bit 0 vision IDs, bit 1 document IDs).
template <int D, int BN, int DSPLIT, int NQG, bool VDOUBLE, int META, int OCC = 1>
struct FwdKernel {
  using C = FwdCfg<D, BN, DSPLIT, NQG, VDOUBLE>;
  static constexpr int kNB = C::kDH / 32;  // 32-wide head-dim blocks per wave
  static constexpr int kNC = C::kDH / 16;  // 16-deep head-dim steps per wave

  char G4_LDS* smem;
  const g4_problem* p;
  Seq sq;
  int tid, lane, wave, dh, h32;
  int my_a, my_vid, my_doc;
  bool has_vid, has_doc, has_meta;
  int a0;
  const __bf16* kbase;
  const __bf16* vbase;
  int64_t kstride, vstride;
  RowReader<C::kCPR> krd;
  // Head dim 512 keeps the compiler's wait before the P.V reads: with it the
  // 8192-token causal forward measured 2.81 ms, without it 2.91 ms.
  TrReader<C::kCPR, (D != 512)> vrd;
  TileCopier<C::kCPR, BN, C::kNW, (OCC > 1)> kcp, vcp;
  bf16x8 qf[kNC];
  f32x16 o_acc[kNB];
  float m_run, l_run;

  __device__ __forceinline__ void issue_k(int row0, int buf) {
    char G4_LDS* dst = smem + C::kLdsK + buf * C::kTileBytes;
    if (row0 + BN <= sq.lk)
      kcp.issue(kbase + row0 * kstride, dst);
    else
      kcp.issue_clamped(kbase + row0 * kstride, kstride, sq.lk - row0, dst, wave, lane);
  }
  __device__ __forceinline__ void issue_v(int row0, int buf) {
    char G4_LDS* dst = smem + C::kLdsV + buf * C::kTileBytes;
    if (row0 + BN <= sq.lk)
      vcp.issue(vbase + row0 * vstride, dst);
    else
      vcp.issue_clamped(vbase + row0 * vstride, vstride, sq.lk - row0, dst, wave, lane);
  }

  template <int KB, int CP>
  __device__ __forceinline__ void s_step(const char G4_LDS* kt, f32x16& acc) const {
    if constexpr (CP < kNC) {
      // slice dh starts at chunk dh * kDH / 8 (a multiple of 16)
      bf16x8 kf = krd.template read<KB * 32, 0, CP>(kt);
      acc = mfma32(kf, qf[CP], acc);
      s_step<KB, CP + 1>(kt, acc);
    }
  }

  template <int KB, int HK, int B>
  __device__ __forceinline__ void pv_step(const char G4_LDS* vt, const bf16x8& pb) {
    if constexpr (B < kNB) {
      bf16x8 vf = vrd.template read<KB * 32 + 16 * HK, 0, B>(vt);
      o_acc[B] = mfma32(vf, pb, o_acc[B]);
      pv_step<KB, HK, B + 1>(vt, pb);
    }
  }

  // Branch-free Gemma predicate on the lane's 16 * kKB scores (keys kb0 + ...).
  // Causal part: lo_w <= j <= min(a, Sk - 1); vision part: same non-negative
  // block, j >= lo_w, j < Sk; document part: equal IDs.
  __device__ __forceinline__ void apply_mask(int cur, f32x16 (&sacc)[C::kKB], int kb0) const {
    const int lo_w = p->window > 0 ? my_a - p->window + 1 : -0x40000000;
    const int hi_c = min(my_a, sq.lk - 1);
    const int* km = (const int*)(smem + C::kLdsMeta + cur * 512);
#pragma unroll
    for (int kb = 0; kb < C::kKB; ++kb)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int jl0 = kb * 32 + 8 * r4 + 4 * h32;
        i32x4 vk = {-1, -1, -1, -1}, dk = {0, 0, 0, 0};
        if (has_meta) {
          vk = *(const i32x4*)(km + jl0);
          dk = *(const i32x4*)(km + 64 + jl0);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = kb0 + jl0 + e;
          const bool in_w = j >= lo_w;
          const bool causal = in_w & (j <= hi_c);
          const bool vis = has_vid & (my_vid >= 0) & (vk[e] == my_vid) & in_w & (j < sq.lk);
          const bool doc_ok = !has_doc | (dk[e] == my_doc);
          const bool ok = (causal | vis) & doc_ok;
          sacc[kb][r4 * 4 + e] = ok ? sacc[kb][r4 * 4 + e] : kNegInf;
        }
      }
  }

  // AHEAD (double-buffered V, no key metadata): K runs two tiles ahead
  // instead of one; K(it + 2) is issued into this step's K buffer once every
  // wave is done reading it, so about two tiles of copies stay in flight (the
  // split-key forward, whose steps are short next to a tile's fetch).  The
  // caller issues K(0), V(0) and K(1) first.
  template <bool AHEAD = false>
  __device__ __forceinline__ void step(int cur, int it, int ntiles, int t_first) {
    static_assert(!AHEAD || (VDOUBLE && META == 0), "K-ahead steps");
    const int kb0 = (t_first + it) * BN;
    // This wave's copies of K (and, double-buffered, V) for this tile have
    // landed; the barrier publishes every wave's copies and ends all reads of
    // the buffers refilled below.  (AHEAD: K(it + 1), issued last, may still
    // be in flight.)
    if constexpr (AHEAD) {
      if (it + 1 < ntiles)
        vm_wait<C::kLoadsPerWave>();
      else
        vm_wait<0>();
    } else if constexpr (VDOUBLE) {
      vm_wait<0>();
    } else {
      vm_wait<C::kLoadsPerWave>();
    }
    barrier_lds();
    if constexpr (AHEAD) {
      if (it + 1 < ntiles) issue_v(kb0 + BN, cur ^ 1);
    } else if (it + 1 < ntiles) {
      issue_k(kb0 + BN, cur ^ 1);
      if (has_meta && wave == 0) issue_meta(*p, sq, kb0 + BN, smem + C::kLdsMeta + (cur ^ 1) * 512, lane, has_vid, has_doc);
      if constexpr (VDOUBLE) issue_v(kb0 + BN, cur ^ 1);
    }

    // S^T partial over this wave's head-dim slice.
    f32x16 sacc[C::kKB];
    const char G4_LDS* kt = smem + C::kLdsK + cur * C::kTileBytes;
    __builtin_amdgcn_sched_barrier(0);
    mfma_prio_begin();
    __builtin_amdgcn_sched_barrier(0);
    sacc[0] = f32x16{};
    s_step<0, 0>(kt, sacc[0]);
    if constexpr (C::kKB > 1) {
      sacc[1] = f32x16{};
      s_step<1, 0>(kt, sacc[1]);
    }
    mfma_pipeline_hint<C::kKB * kNC, 3, 1>();

    __builtin_amdgcn_sched_barrier(0);
    mfma_prio_end();
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (DSPLIT > 1) {
      // Publish the partial, then add the partner slice's partial.
      char G4_LDS* xb = smem + C::kLdsX;
#pragma unroll
      for (int kb = 0; kb < C::kKB; ++kb)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          f32x4 v = {sacc[kb][q4 * 4], sacc[kb][q4 * 4 + 1], sacc[kb][q4 * 4 + 2],
                     sacc[kb][q4 * 4 + 3]};
          *(f32x4 G4_LDS*)(xb + (((wave * C::kKB + kb) * 4 + q4) * 64 + lane) * 16) = v;
        }
      // Single V buffer: this tile's V copies were issued after the previous
      // PV phase, before the K copies of the next tile.
      if constexpr (!VDOUBLE) vm_wait<C::kLoadsPerWave>();
      barrier_lds();
      const int pw = wave ^ 1;
#pragma unroll
      for (int kb = 0; kb < C::kKB; ++kb)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          f32x4 v =
              *(const f32x4 G4_LDS*)(xb + (((pw * C::kKB + kb) * 4 + q4) * 64 + lane) * 16);
          // add in slice order so both slices hold bit-identical scores
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float mine = sacc[kb][q4 * 4 + e];
            sacc[kb][q4 * 4 + e] = dh == 0 ? mine + v[e] : v[e] + mine;
          }
        }
    } else if constexpr (!VDOUBLE) {
      vm_wait<C::kLoadsPerWave>();
      barrier_lds();
    }
    if constexpr (AHEAD) {
      // every wave is done reading K(it): after the partial exchange's
      // barrier, or with one wave, once its own S chain has its operands
      if (it + 2 < ntiles) issue_k(kb0 + 2 * BN, cur);
    }

    // Mask (only on tiles the mask does not fully admit), then online softmax
    // in the log2 domain (softmax scale is 1.0; log2 e is folded into the
    // exponent's FMA, and the row maximum is scaled once: rounding is
    // monotonic, so max(s) * log2 e rounds to the maximum of the scaled scores).
    const bool full = !has_doc && (kb0 + BN <= sq.lk) && (kb0 + BN - 1 <= a0) &&
                      (p->window <= 0 || kb0 > a0 + C::kBM - 1 - p->window);
    if (!full) {
      __builtin_amdgcn_sched_barrier(0);
      apply_mask(cur, sacc, kb0);
      __builtin_amdgcn_sched_barrier(0);
    }
    float mx = kNegInf;
#pragma unroll
    for (int kb = 0; kb < C::kKB; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[kb][r]);
    mx = fmaxf(mx, wave_xor32(mx)) * kLog2e;
    // The running maximum only moves when a row's scores exceed it by more
    // than kRescaleLog2 (P <= 2^kRescaleLog2 meanwhile, exact in fp32 and in
    // bf16 range), so the O accumulators are rescaled rarely after the first
    // admitted tile instead of on most tiles.
    const float m_new = mx > m_run + kRescaleLog2 ? mx : m_run;
    const float m_use = m_new == kNegInf ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - m_use);
    float rs = 0.f;
    bf16x8 pb[C::kKB][2];
#pragma unroll
    for (int kb = 0; kb < C::kKB; ++kb)
#pragma unroll
      for (int hk = 0; hk < 2; ++hk)
#pragma unroll
        for (int m = 0; m < 8; ++m) {
          float pv = fast_exp2(__builtin_fmaf(sacc[kb][hk * 8 + m], kLog2e, -m_use));
          rs += pv;
          pb[kb][hk][m] = (__bf16)pv;
        }
    l_run = l_run * alpha + rs;
    m_run = m_new;
    if (__ballot(alpha != 1.f)) {
#pragma unroll
      for (int b = 0; b < kNB; ++b) o_acc[b] *= alpha;
    }

    // O^T += V^T P^T with V^T from transposing reads of the V tile.
    const char G4_LDS* vt = smem + C::kLdsV + (VDOUBLE ? cur : 0) * C::kTileBytes;
    __builtin_amdgcn_sched_barrier(0);
    mfma_prio_begin();
    __builtin_amdgcn_sched_barrier(0);
    pv_step<0, 0, 0>(vt, pb[0][0]);
    pv_step<0, 1, 0>(vt, pb[0][1]);
    if constexpr (C::kKB > 1) {
      pv_step<1, 0, 0>(vt, pb[1][0]);
      pv_step<1, 1, 0>(vt, pb[1][1]);
    }
    mfma_pipeline_hint<C::kKB * 2 * kNB, 6, 2>();

    __builtin_amdgcn_sched_barrier(0);
    mfma_prio_end();
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (!VDOUBLE) {
      // Single V buffer: every wave must finish its PV reads before refill.
      barrier_lds();
      if (it + 1 < ntiles) issue_v(kb0 + BN, 0);
    }
  }
};

// Work item L of a forward grid: heads outermost (KV head, then the grid's
// query tiles, then the query heads of the group), query tiles sequence by
// sequence.  A compact grid (FwdParams::compact) enumerates only the tiles
// that exist; otherwise every sequence has ntq slots, the ones past its end
// empty.
struct FwdItem {
  int kvh, qh, s, local, nt;
  // False for an item past the last tile of a compact grid.
  __device__ __forceinline__ bool decode(const FwdParams& a, int L, int bm) {
    const g4_problem& p = a.p;
    const int grp = p.num_q_heads / p.num_kv_heads;
    SeqTiles tiles;
    if (a.compact) tiles.init(p.cu_seqlens_q, a.num_seqs, bm);
    const int per_kvh = (a.compact ? tiles.total : a.num_seqs * a.ntq) * grp;
    kvh = L / per_kvh;
    if (kvh >= p.num_kv_heads) return false;
    const int rem = L % per_kvh;
    const int rank = rem / grp;
    qh = kvh * grp + rem % grp;
    if (a.compact) {
      tiles.find(rank, s, local, nt);
    } else {
      s = rank / a.ntq;
      local = rank % a.ntq;
      nt = a.ntq;
    }
    return true;
  }
  // The item of this workgroup in a launch of one item per workgroup.
  __device__ static __forceinline__ int of_block(const FwdParams& a) {
    return a.desc_order ? xcd_remap_desc(blockIdx.x, gridDim.x,
                                          a.p.num_q_heads / a.p.num_kv_heads)
                        : xcd_remap(blockIdx.x, gridDim.x);
  }
  // The index in the full (num_seqs x ntq) grid of the item for the same
  // query tile (the two grids order a sequence's tiles over nt and over ntq).
  __device__ __forceinline__ int full_index(const FwdParams& a) const {
    const int grp = a.p.num_q_heads / a.p.num_kv_heads;
    const int r = unzigzag(zigzag(local, nt), a.ntq);
    return (kvh * a.num_seqs * a.ntq + s * a.ntq + r) * grp + qh % grp;
  }
};

// Workgroups of a forward grid of bm-query tiles; sets b->compact.  A packed
// batch of 2..64 sequences enumerates only its tiles: at most
// sum ceil(len / bm) <= (total_q + num_seqs (bm - 1)) / bm per head, against
// num_seqs x ntq for the grid sized by the longest sequence.
static int64_t fwd_grid(FwdParams* b, int bm, bool allow_compact) {
  const g4_problem& p = b->p;
  b->ntq = (p.seqlen_q + bm - 1) / bm;
  b->compact = 0;
  b->desc_order = 0;
  int64_t tiles = (int64_t)b->num_seqs * b->ntq;
  if (allow_compact && p.cu_seqlens_q != nullptr && b->num_seqs > 1 && b->num_seqs <= 64) {
    const int64_t bound = (p.total_q + (int64_t)b->num_seqs * (bm - 1)) / bm;
    if (bound < tiles) {
      tiles = bound;
      b->compact = 1;
    }
  }
  const int64_t n = tiles * p.num_q_heads;
  // Heaviest first within each XCD: the zigzag ranks of a sequence alternate
  // heavy and light only if ntq is even (rank parity = tile-rank parity).
  const int grp = p.num_q_heads / p.num_kv_heads;
  if (allow_compact && !b->compact && b->ntq % 2 == 0 && n % (16 * grp) == 0) b->desc_order = 1;
  return n;
}

// One work item L of the forward (one query tile of one head).
// FIXUP: rerun only the 32-query groups the wide kernel flagged in raise_flags.
// OCC: workgroups per CU the register budget is sized for.
template <int D, int BN, int DSPLIT, int NQG, bool VDOUBLE, int META, bool FIXUP, int OCC>
__device__ __forceinline__ void fwd_item(const FwdParams& a, char* smem_raw, int L) {
  using K = FwdKernel<D, BN, DSPLIT, NQG, VDOUBLE, META, OCC>;
  using C = typename K::C;
  K ker;
  ker.smem = (char G4_LDS*)smem_raw;
  ker.p = &a.p;
  const g4_problem& p = a.p;

  ker.tid = threadIdx.x;
  ker.lane = ker.tid & 63;
  ker.wave = __builtin_amdgcn_readfirstlane(ker.tid >> 6);
  const int qg = ker.wave / DSPLIT;
  ker.dh = ker.wave % DSPLIT;
  ker.h32 = ker.lane >> 5;
  const int l32 = ker.lane & 31;

  // ---- work item -------------------------------------------------------
  FwdItem it;
  if (!it.decode(a, L, C::kBM)) return;
  const int kvh = it.kvh, qh = it.qh, s = it.s;
  const int qt = zigzag(it.local, it.nt);

  ker.sq = resolve_seq(p, s);
  const Seq& sq = ker.sq;
  const int i0 = qt * C::kBM;
  if (i0 >= sq.lq) return;
  if constexpr (FIXUP) {
    const int nq32 = (p.seqlen_q + 31) / 32;
    bool need = false;
#pragma unroll
    for (int g = 0; g < NQG; ++g) {
      const int q32 = i0 / 32 + g;
      if (q32 < nq32) need |= a.raise_flags[((int64_t)s * nq32 + q32) * p.num_q_heads + qh] != 0;
    }
    if (!need) return;
  }
  const int off = sq.lk - sq.lq;  // query i sits at key position i + off
  ker.a0 = i0 + off;
  const int a_last_valid = min(i0 + C::kBM, sq.lq) - 1 + off;
  ker.has_vid = (META & 1) && p.vision_ids != nullptr && p.bidirectional_vision;
  ker.has_doc = (META & 2) && p.document_ids != nullptr;
  ker.has_meta = ker.has_vid || ker.has_doc;

  // ---- key range (mask-aware tile scheduler) -------------------------------
  int span_max = -1;
  if (ker.has_vid) {
    int* red = (int*)(smem_raw + C::kLdsRed);
    int v = -1;
    for (int t = ker.tid; t < C::kBM; t += C::kNT) {
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
  // ---- document uniformity -------------------------------------------------
  // The range spans whole 64-key tiles (a superset of the visited tiles for
  // BN <= 64), so both launches of a split problem evaluate it identically.
  if (p.document_ids != nullptr && (ker.has_doc || a.doc_pass == 1)) {
    const bool uni = doc_uniform<C::kNW>(
        p.document_ids, sq.ktok, sq.lk, min(klo / 64 * 64, ker.a0),
        max((khi + 63) / 64 * 64, a_last_valid + 1), ker.tid, ker.lane, ker.wave,
        (int*)(smem_raw + C::kLdsRed));
    if (a.doc_pass == 1 && !uni) {
      // left to the second pass
      // (its index in the full grid, which pass 2 decodes)
      if (ker.tid == 0 && a.doc_list != nullptr)
        a.doc_list[atomicAdd(a.doc_list_n, 1u)] = it.full_index(a);
      return;
    }
    if (a.doc_pass == 2 && uni) return;
    if (uni) {
      ker.has_doc = false;
      ker.has_meta = ker.has_vid;
    }
  }

  // ---- operand bases, address tables ---------------------------------------
  ker.kbase = a.k + tok_off(sq, s, sq.ktok, 0, a.kl) + (int64_t)kvh * a.kl.head_stride;
  ker.vbase = a.v + tok_off(sq, s, sq.ktok, 0, a.vl) + (int64_t)kvh * a.vl.head_stride;
  ker.kstride = a.kl.token_stride;
  ker.vstride = a.vl.token_stride;
  ker.krd.init(ker.lane, ker.dh * C::kDH * 2);
  ker.vrd.init(ker.lane, ker.dh * C::kDH * 2);
  ker.kcp.init(ker.kstride, ker.wave, ker.lane);
  ker.vcp.init(ker.vstride, ker.wave, ker.lane);

  // ---- query fragments (B operand of S^T = K Q^T) -------------------------
  const int my_i = i0 + qg * 32 + l32;  // this lane's query
  ker.my_a = my_i + off;
  const bool q_valid = my_i < sq.lq;
  {
    const __bf16* qrow = a.q + tok_off(sq, s, sq.qtok, min(my_i, sq.lq - 1), a.ql) +
                         (int64_t)qh * a.ql.head_stride + ker.dh * C::kDH + ker.h32 * 8;
#pragma unroll
    for (int c = 0; c < K::kNC; ++c) {
      bf16x8 x = ld_global16(qrow + c * 16);
      ker.qf[c] = q_valid ? x : bf16x8{};
    }
  }
  ker.my_vid = -1;
  ker.my_doc = 0;
  if (ker.has_vid && q_valid) ker.my_vid = p.vision_ids[sq.ktok + ker.my_a];
  if (ker.has_doc && q_valid) ker.my_doc = p.document_ids[sq.ktok + ker.my_a];

  // ---- prologue: tile 0 (issue order K, key metadata, V) -----------------
  if (ntiles > 0) {
    ker.issue_k(t_first * BN, 0);
    if (ker.has_meta && ker.wave == 0) issue_meta(p, sq, t_first * BN, ker.smem + C::kLdsMeta, ker.lane, ker.has_vid, ker.has_doc);
    ker.issue_v(t_first * BN, 0);
  }

#pragma unroll
  for (int b = 0; b < K::kNB; ++b) ker.o_acc[b] = f32x16{};
  ker.m_run = kNegInf;
  ker.l_run = 0.f;

  // Two tiles per iteration, so each step's buffers are compile-time.
  // (Two tiles per iteration with compile-time buffers measured slower: the
  // unrolled loop spills.)
  for (int it = 0; it < ntiles; ++it) ker.step(it & 1, it, ntiles, t_first);

  // ---- epilogue: normalise, write O and LSE ---------------------------------
  const float l_tot = ker.l_run + wave_xor32(ker.l_run);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (q_valid) {
    __bf16* orow = a.o + tok_off(sq, s, sq.qtok, my_i, a.ol) + (int64_t)qh * a.ol.head_stride;
#pragma unroll
    for (int b = 0; b < K::kNB; ++b) {
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d = ker.dh * C::kDH + b * 32 + 8 * r4 + 4 * ker.h32;
        const f32x16& acc = ker.o_acc[b];
        bf16x4 v = {(__bf16)(acc[r4 * 4] * inv), (__bf16)(acc[r4 * 4 + 1] * inv),
                    (__bf16)(acc[r4 * 4 + 2] * inv), (__bf16)(acc[r4 * 4 + 3] * inv)};
        *(bf16x4*)(orow + d) = v;
      }
    }
    if (ker.dh == 0 && ker.h32 == 0) {
      a.lse[lse_off(p, sq, s, qh, my_i)] =
          l_tot > 0.f ? (ker.m_run + fast_log2(l_tot)) * kLn2 : kNegInf;
    }
  }
}

template <int D, int BN, int DSPLIT, int NQG, bool VDOUBLE, int META, bool FIXUP = false,
          int OCC = 1>
__global__ void __launch_bounds__(NQG * DSPLIT * 64, OCC) fwd_kernel(FwdParams a) {
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  if constexpr (META == 3 && !FIXUP) {
    // Second document pass with the first pass's list: the listed items,
    // strided over a resident grid (an item leaves no tile copy in flight;
    // the barrier retires its LDS reads).  One call site, so the item is
    // inlined once.
    const bool listed = a.doc_pass == 2 && a.doc_list != nullptr;
    const int n = listed ? (int)__builtin_amdgcn_readfirstlane(*a.doc_list_n) : (int)blockIdx.x + 1;
    for (int t = blockIdx.x; t < n; t += gridDim.x) {
      if (t != (int)blockIdx.x) barrier_lds();
      const int L = listed ? __builtin_amdgcn_readfirstlane(a.doc_list[t])
                           : FwdItem::of_block(a);
      fwd_item<D, BN, DSPLIT, NQG, VDOUBLE, META, FIXUP, OCC>(a, smem_raw, L);
    }
  } else {
    fwd_item<D, BN, DSPLIT, NQG, VDOUBLE, META, FIXUP, OCC>(a, smem_raw, FwdItem::of_block(a));
  }
}

// ===========================================================================
// Split-key forward for few queries per KV head (decode).
//
// One workgroup per (sequence, KV head, chunk of split_keys keys): its 32
// rows are the query rows of the KV head's group, row r = query head
// kvh * grp + r / Sq, query r % Sq (grp * Sq <= 32; the rest are zero rows),
// so each K / V tile is read once for the whole group, and the chunks spread a
// long key range over the GPU.  The steps are FwdKernel's (one 32-row group,
// head dim split over D / 256 waves); the workgroup writes its rows' partial
// state (O not normalised, running maximum m in log2 units, row sum l) and
// merge_split_kernel combines the chunks: with M the largest m,
// O = sum 2^(m_c - M) O_c / sum 2^(m_c - M) l_c.
// ===========================================================================

template <int D>
using SplitKernel = FwdKernel<D, 32, D / 256, 1, true, 0, (D == 256 ? 2 : 1)>;

template <int D>
__global__ void __launch_bounds__(D / 4, (D == 256 ? 2 : 1)) fwd_split_kernel(FwdParams a) {
  using K = SplitKernel<D>;
  using C = typename K::C;
  constexpr int BN = 32;
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  K ker;
  ker.smem = (char G4_LDS*)smem_raw;
  ker.p = &a.p;
  const g4_problem& p = a.p;
  ker.tid = threadIdx.x;
  ker.lane = ker.tid & 63;
  ker.wave = __builtin_amdgcn_readfirstlane(ker.tid >> 6);
  ker.dh = ker.wave;
  ker.h32 = ker.lane >> 5;
  const int r = ker.lane & 31;

  // ---- item: (sequence, KV head) group g, chunk c ---------------------------
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int n = a.split_chunks;
  const int g = L / n, c = L % n;
  const int s = g / p.num_kv_heads, kvh = g % p.num_kv_heads;
  const int grp = p.num_q_heads / p.num_kv_heads;
  const int rows = grp * p.seqlen_q;  // row stride of the partial buffers
  ker.sq = resolve_seq(p, s);
  const Seq& sq = ker.sq;
  const int lq = sq.lq;
  if (lq <= 0) return;
  const int off = sq.lk - lq;
  const bool valid = r < grp * lq;
  const int qh = kvh * grp + (valid ? r / lq : 0);
  const int qi = valid ? r % lq : 0;
  ker.my_a = qi + off;
  ker.a0 = off;  // the first query's position (the full-tile test's lower bound)
  ker.has_vid = ker.has_doc = ker.has_meta = false;
  ker.my_vid = -1;
  ker.my_doc = 0;

  // ---- this chunk's key tiles ------------------------------------------------
  int klo, khi;
  query_tile_key_range(off, off + lq - 1, sq.lk, p.window, -1, klo, khi);
  const int per = a.split_keys / BN;
  const int t_first = klo / BN + c * per;
  const int t_end = min((khi + BN - 1) / BN, t_first + per);
  const int ntiles = khi > klo ? max(t_end - t_first, 0) : 0;

  ker.kbase = a.k + tok_off(sq, s, sq.ktok, 0, a.kl) + (int64_t)kvh * a.kl.head_stride;
  ker.vbase = a.v + tok_off(sq, s, sq.ktok, 0, a.vl) + (int64_t)kvh * a.vl.head_stride;
  ker.kstride = a.kl.token_stride;
  ker.vstride = a.vl.token_stride;
  ker.krd.init(ker.lane, ker.dh * C::kDH * 2);
  ker.vrd.init(ker.lane, ker.dh * C::kDH * 2);
  ker.kcp.init(ker.kstride, ker.wave, ker.lane);
  ker.vcp.init(ker.vstride, ker.wave, ker.lane);
  {
    const __bf16* qrow = a.q + tok_off(sq, s, sq.qtok, qi, a.ql) +
                         (int64_t)qh * a.ql.head_stride + ker.dh * C::kDH + ker.h32 * 8;
#pragma unroll
    for (int cc = 0; cc < K::kNC; ++cc) {
      bf16x8 x = ld_global16(qrow + cc * 16);
      ker.qf[cc] = valid ? x : bf16x8{};
    }
  }
  if (ntiles > 0) {
    ker.issue_k(t_first * BN, 0);
    ker.issue_v(t_first * BN, 0);
    if (ntiles > 1) ker.issue_k((t_first + 1) * BN, 1);
  }
#pragma unroll
  for (int b = 0; b < K::kNB; ++b) ker.o_acc[b] = f32x16{};
  ker.m_run = kNegInf;
  ker.l_run = 0.f;
  for (int it = 0; it < ntiles; ++it) ker.template step<true>(it & 1, it, ntiles, t_first);

  // ---- partial rows ---------------------------------------------------------
  const float l_tot = ker.l_run + wave_xor32(ker.l_run);
  if (valid) {
    const int64_t row = ((int64_t)g * n + c) * rows + r;
    float* po = a.part + row * D;
#pragma unroll
    for (int b = 0; b < K::kNB; ++b)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d = ker.dh * C::kDH + b * 32 + 8 * r4 + 4 * ker.h32;
        const f32x16& x = ker.o_acc[b];
        *(f32x4*)(po + d) = f32x4{x[r4 * 4], x[r4 * 4 + 1], x[r4 * 4 + 2], x[r4 * 4 + 3]};
      }
    if (ker.dh == 0 && ker.h32 == 0) {
      float* ml = a.part + (int64_t)p.num_seqs * p.num_kv_heads * n * rows * D + row * 2;
      ml[0] = ker.m_run;
      ml[1] = l_tot;
    }
  }
}

// One workgroup per (sequence, KV head, row): the row's maximum over its
// chunks first, then wave w sums chunks w, w + 4, ... (four chunks' loads in
// flight per lane), and wave 0 adds the four waves' sums in order.  (One
// 64-lane workgroup walking the chunks one by one took 73 us at 128 chunks.)
template <int D>
__global__ void __launch_bounds__(256) merge_split_kernel(FwdParams a) {
  constexpr int E = D / 64;  // elements per lane: 4 (D = 256) or 8 (D = 512)
  constexpr int kW = 4;      // waves
  __shared__ float red_m[kW], red_l[kW];
  __shared__ float stage[kW - 1][E][64];
  const g4_problem& p = a.p;
  const int grp = p.num_q_heads / p.num_kv_heads;
  const int rows = grp * p.seqlen_q;
  const int n = a.split_chunks;
  const int g = blockIdx.x / rows, r = blockIdx.x % rows;
  const int s = g / p.num_kv_heads, kvh = g % p.num_kv_heads;
  const Seq sq = resolve_seq(p, s);
  if (r >= grp * sq.lq) return;
  const int qh = kvh * grp + r / sq.lq, qi = r % sq.lq;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const float* ml = a.part + (int64_t)p.num_seqs * p.num_kv_heads * n * rows * D;
  const int64_t row0 = (int64_t)g * n * rows + r;  // chunk c: row0 + c * rows
  float mx = kNegInf;
  for (int c = threadIdx.x; c < n; c += kW * 64) {
    const float* e = ml + (row0 + (int64_t)c * rows) * 2;
    if (e[1] > 0.f) mx = fmaxf(mx, e[0]);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  if (lane == 0) red_m[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red_m[0], red_m[1]), fmaxf(red_m[2], red_m[3]));
  float acc[E] = {};
  float l = 0.f;
#pragma unroll 4
  for (int c = wave; c < n; c += kW) {
    const int64_t row = row0 + (int64_t)c * rows;
    const float lc = ml[row * 2 + 1];
    // an empty chunk (no keys for this row) wrote l = 0 and O = 0
    const float w = lc > 0.f ? fast_exp2(ml[row * 2] - mx) : 0.f;
    l += w * lc;
    const float* po = a.part + row * D;
#pragma unroll
    for (int h = 0; h < E / 4; ++h) {
      const f32x4 x = *(const f32x4*)(po + h * 256 + 4 * lane);
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[4 * h + u] += w * x[u];
    }
  }
  if (wave > 0) {
#pragma unroll
    for (int e = 0; e < E; ++e) stage[wave - 1][e][lane] = acc[e];
    if (lane == 0) red_l[wave] = l;
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 1; w < kW; ++w) {
    l += red_l[w];
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] += stage[w - 1][e][lane];
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  __bf16* orow = a.o + tok_off(sq, s, sq.qtok, qi, a.ol) + (int64_t)qh * a.ol.head_stride;
#pragma unroll
  for (int h = 0; h < E / 4; ++h)
    *(bf16x4*)(orow + h * 256 + 4 * lane) =
        bf16x4{(__bf16)(acc[4 * h] * inv), (__bf16)(acc[4 * h + 1] * inv),
               (__bf16)(acc[4 * h + 2] * inv), (__bf16)(acc[4 * h + 3] * inv)};
  if (lane == 0)
    a.lse[lse_off(p, sq, s, qh, qi)] = l > 0.f ? (mx + fast_log2(l)) * kLn2 : kNegInf;
}

template <int D>
static hipError_t launch_fwd_split(const FwdParams& a, hipStream_t stream) {
  using C = typename SplitKernel<D>::C;
  static_assert(C::kNT == D / 4, "one wave per 256 of the head dim");
  static LdsAttr attr;
  hipError_t e = attr.ensure((const void*)fwd_split_kernel<D>, C::kLdsBytes);
  if (e != hipSuccess) return e;
  const int64_t groups = (int64_t)a.num_seqs * a.p.num_kv_heads;
  const int64_t rows = (int64_t)(a.p.num_q_heads / a.p.num_kv_heads) * a.p.seqlen_q;
  const int64_t items = groups * a.split_chunks;
  if (items <= 0) return hipSuccess;
  hipLaunchKernelGGL(fwd_split_kernel<D>, dim3((unsigned)items), dim3(C::kNT), C::kLdsBytes,
                     stream, a);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(merge_split_kernel<D>, dim3((unsigned)(groups * rows)), dim3(256), 0, stream,
                     a);
  return hipGetLastError();
}

// ===========================================================================
// Software-pipelined forward for wide heads without key metadata.
//
// Four waves, one per SIMD, each owning 32 queries and the whole head dim, so
// no partial scores are exchanged and one K / V tile serves 128 queries.  Per
// key tile the loop runs two regions:
//   A: S^T(t+1) = K(t+1) Q^T on MFMA, interleaved with the softmax of tile t
//      (VALU) and with the async copies of K(t+2) and V(t+1);
//   B: O^T += V(t)^T P(t)^T on MFMA.
// One barrier per tile: it publishes K(t+1) and V(t) and retires every read
// of the buffers refilled in the next region A.
//
// The O accumulators (256 AGPRs per lane) are never rescaled.  A row's
// running maximum m is set by its first admitted tile; later tiles use the
// same m as long as their maximum stays below m + kRaiseLog2 (log2 units), so
// P = exp2(s - m) <= 2^kRaiseLog2 is exact in fp32 and in bf16 range and O, l
// stay far from fp32 overflow.  A row whose scores jump higher (by more than
// kRaiseLog2 * ln 2 within the row) marks its 32-query group in raise_flags;
// launch_fwd then reruns exactly those groups with the rescaling kernel.
// ===========================================================================

constexpr float kRaiseLog2 = 48.0f;

template <int D>
struct WideCfg {
  static constexpr int kNW = 4;
  static constexpr int kNT = kNW * 64;
  static constexpr int kBM = kNW * 32;
  static constexpr int kBN = 32;
  static constexpr int kCPR = D / 8;
  static constexpr int kTile = kBN * D * 2;
  static constexpr int kNC = D / 16;  // 16-deep steps of S^T
  static constexpr int kNB = D / 32;  // 32-wide head-dim blocks of O^T
  static constexpr int kLdsK = 0;
  static constexpr int kLdsV = 2 * kTile;
  static constexpr int kLdsBytes = 4 * kTile;
  static_assert(kLdsBytes <= 160 * 1024, "LDS budget");
};

template <int D>
struct FwdWide {
  using C = WideCfg<D>;
  static constexpr int kNC = C::kNC;
  static constexpr int kNB = C::kNB;
  static constexpr int BN = C::kBN;
  // Operand reads in flight in the S and P.V chains: one wave per SIMD has no
  // other wave to cover LDS latency (2.79 ms on config 2 with the scheduler's
  // one read per MFMA, 2.66 with two in flight, 2.56-2.59 with three or four).
  static constexpr int kAhead = 4;

  char G4_LDS* smem;
  Seq sq;
  int lane, wave, h32;
  int a0, window, lo_w, hi_c;
  const __bf16* kbase;
  const __bf16* vbase;
  int64_t kstride, vstride;
  RowReader<C::kCPR> krd;
  TrReader<C::kCPR, false> vrd;  // as FwdKernel's at head dim 512
  TileCopier<C::kCPR, BN, C::kNW> kcp, vcp;
  bf16x8 qf[kNC];
  f32x16 o_acc[kNB];
  float m_run, l_run;
  bool raise;  // a later tile exceeded this row's maximum by more than kRaiseLog2

  __device__ __forceinline__ void issue_k(int row0, int buf) {
    char G4_LDS* dst = smem + C::kLdsK + buf * C::kTile;
    if (row0 + BN <= sq.lk)
      kcp.issue(kbase + row0 * kstride, dst);
    else
      kcp.issue_clamped(kbase + row0 * kstride, kstride, sq.lk - row0, dst);
  }
  __device__ __forceinline__ void issue_v(int row0, int buf) {
    char G4_LDS* dst = smem + C::kLdsV + buf * C::kTile;
    if (row0 + BN <= sq.lk)
      vcp.issue(vbase + row0 * vstride, dst);
    else
      vcp.issue_clamped(vbase + row0 * vstride, vstride, sq.lk - row0, dst);
  }

  // Softmax of one tile's raw scores (keys kb0 + ...) into bf16 P.
  __device__ __forceinline__ void softmax(f32x16& s, int kb0, bf16x8 (&pb)[2]) {
    const bool full = (kb0 + BN <= sq.lk) && (kb0 + BN - 1 <= a0) &&
                      (window <= 0 || kb0 > a0 + C::kBM - 1 - window);
    if (!full) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int j = kb0 + 8 * (r >> 2) + 4 * h32 + (r & 3);
        const bool ok = (j >= lo_w) & (j <= hi_c);
        s[r] = ok ? s[r] : kNegInf;
      }
    }
    float mx = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
    mx = fmaxf(mx, wave_xor32(mx)) * kLog2e;
    if (m_run == kNegInf) m_run = mx;  // first admitted tile of the row (or still none)
    raise |= mx > m_run + kRaiseLog2;
    const float m_use = m_run == kNegInf ? 0.f : m_run;
    float rs = 0.f;
#pragma unroll
    for (int hk = 0; hk < 2; ++hk)
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const float pv = fast_exp2(__builtin_fmaf(s[hk * 8 + m], kLog2e, -m_use));
        rs += pv;
        pb[hk][m] = (__bf16)pv;
      }
    l_run += rs;
  }
};

template <int D>
__global__ void __launch_bounds__(256, 1) fwd_wide_kernel(FwdParams a) {
  using K = FwdWide<D>;
  using C = typename K::C;
  constexpr int BN = C::kBN;
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  K ker;
  ker.smem = (char G4_LDS*)smem_raw;
  const g4_problem& p = a.p;
  const int tid = threadIdx.x;
  ker.lane = tid & 63;
  ker.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  ker.h32 = ker.lane >> 5;
  const int l32 = ker.lane & 31;

  const int L = FwdItem::of_block(a);
  FwdItem it;
  if (!it.decode(a, L, C::kBM)) return;
  const int kvh = it.kvh, qh = it.qh, s = it.s;
  const int qt = zigzag(it.local, it.nt);

  ker.sq = resolve_seq(p, s);
  const Seq& sq = ker.sq;
  const int i0 = qt * C::kBM;
  if (i0 >= sq.lq) return;
  const int off = sq.lk - sq.lq;
  ker.a0 = i0 + off;
  const int a_last_valid = min(i0 + C::kBM, sq.lq) - 1 + off;
  ker.window = p.window;

  int klo, khi;
  query_tile_key_range(ker.a0, a_last_valid, sq.lk, p.window, -1, klo, khi);
  const int t_first = klo / BN;
  const int ntiles = (khi + BN - 1) / BN - t_first;

  ker.kbase = a.k + tok_off(sq, s, sq.ktok, 0, a.kl) + (int64_t)kvh * a.kl.head_stride;
  ker.vbase = a.v + tok_off(sq, s, sq.ktok, 0, a.vl) + (int64_t)kvh * a.vl.head_stride;
  ker.kstride = a.kl.token_stride;
  ker.vstride = a.vl.token_stride;
  ker.krd.init(ker.lane, 0);
  ker.vrd.init(ker.lane, 0);
  ker.kcp.init(ker.kstride, ker.wave, ker.lane);
  ker.vcp.init(ker.vstride, ker.wave, ker.lane);

  const int my_i = i0 + ker.wave * 32 + l32;
  const int my_a = my_i + off;
  const bool q_valid = my_i < sq.lq;
  ker.lo_w = p.window > 0 ? my_a - p.window + 1 : -0x40000000;
  ker.hi_c = min(my_a, sq.lk - 1);
  {
    const __bf16* qrow = a.q + tok_off(sq, s, sq.qtok, min(my_i, sq.lq - 1), a.ql) +
                         (int64_t)qh * a.ql.head_stride + ker.h32 * 8;
#pragma unroll
    for (int c = 0; c < K::kNC; ++c) {
      bf16x8 x = ld_global16(qrow + c * 16);
      ker.qf[c] = q_valid ? x : bf16x8{};
    }
  }
  ker.m_run = kNegInf;
  ker.l_run = 0.f;
  ker.raise = false;
#pragma unroll
  for (int b = 0; b < K::kNB; ++b) ker.o_acc[b] = f32x16{};

  f32x16 s_cur = {};
  if (ntiles > 0) {
    // Prologue: K(0), V(0), K(1); S(0).
    ker.issue_k(t_first * BN, 0);
    ker.issue_v(t_first * BN, 0);
    if (ntiles > 1) {
      ker.issue_k((t_first + 1) * BN, 1);
      vm_wait<decltype(ker.kcp)::kPer>();
    } else {
      vm_wait<0>();
    }
    barrier_lds();
    __builtin_amdgcn_sched_barrier(0);
    row_steps<K::kNC, K::kAhead>(ker.krd, ker.smem + C::kLdsK, s_cur, ker.qf);
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int it = 0; it < ntiles; ++it) {
    const int cur = it & 1, nxt = cur ^ 1;
    const int kb0 = (t_first + it) * BN;
    // K(it + 1) and V(it) have landed in every wave; every wave is done with
    // the K buffer of tile it and the V buffer of tile it - 1.
    vm_wait<0>();
    barrier_lds();
    __builtin_amdgcn_sched_barrier(0);

    // ---- region A: S(it + 1) || softmax(it) || copies K(it + 2), V(it + 1)
    if (it + 2 < ntiles) ker.issue_k(kb0 + 2 * BN, cur);
    if (it + 1 < ntiles) ker.issue_v(kb0 + BN, nxt);
    f32x16 s_nxt = {};
    bf16x8 pb[2];
    if (it + 1 < ntiles) {
      row_steps<K::kNC, K::kAhead>(ker.krd, ker.smem + C::kLdsK + nxt * C::kTile, s_nxt,
                                   ker.qf);
      ker.softmax(s_cur, kb0, pb);
    } else {
      ker.softmax(s_cur, kb0, pb);
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- region B: O^T += V(it)^T P(it)^T
    const char G4_LDS* vt = ker.smem + C::kLdsV + cur * C::kTile;
    acc_steps<K::kNB, K::kAhead>(ker.vrd, vt, pb, ker.o_acc);
    __builtin_amdgcn_sched_barrier(0);
    s_cur = s_nxt;
  }

  // Every 32-query group reports whether its rows need the rescaling pass.
  const int q32 = i0 / 32 + ker.wave;
  const int nq32 = (p.seqlen_q + 31) / 32;
  const bool raise_any = __ballot(ker.raise && q_valid) != 0;
  if (ker.lane == 0 && q32 < nq32)
    a.raise_flags[((int64_t)s * nq32 + q32) * p.num_q_heads + qh] = raise_any ? 1 : 0;

  const float l_tot = ker.l_run + wave_xor32(ker.l_run);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (q_valid) {
    __bf16* orow = a.o + tok_off(sq, s, sq.qtok, my_i, a.ol) + (int64_t)qh * a.ol.head_stride;
#pragma unroll
    for (int b = 0; b < K::kNB; ++b) {
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d = b * 32 + 8 * r4 + 4 * ker.h32;
        const f32x16& acc = ker.o_acc[b];
        bf16x4 v = {(__bf16)(acc[r4 * 4] * inv), (__bf16)(acc[r4 * 4 + 1] * inv),
                    (__bf16)(acc[r4 * 4 + 2] * inv), (__bf16)(acc[r4 * 4 + 3] * inv)};
        *(bf16x4*)(orow + d) = v;
      }
    }
    if (ker.h32 == 0) {
      a.lse[lse_off(p, sq, s, qh, my_i)] =
          l_tot > 0.f ? (ker.m_run + fast_log2(l_tot)) * kLn2 : kNegInf;
    }
  }
}

template <int D>
static hipError_t launch_fwd_wide(const FwdParams& a, hipStream_t stream) {
  using C = WideCfg<D>;
  static LdsAttr attr;
  hipError_t e = attr.ensure((const void*)fwd_wide_kernel<D>, C::kLdsBytes);
  if (e != hipSuccess) return e;
  FwdParams b = a;
  const int64_t nblocks = fwd_grid(&b, C::kBM, true);
  if (nblocks <= 0) return hipSuccess;
  hipLaunchKernelGGL(fwd_wide_kernel<D>, dim3((unsigned)nblocks), dim3(C::kNT), C::kLdsBytes,
                     stream, b);
  return hipGetLastError();
}

// Key metadata kinds a problem carries (bit 0 vision IDs, bit 1 document IDs).
static int meta_kind(const g4_problem& p) {
  return ((p.vision_ids != nullptr && p.bidirectional_vision) ? 1 : 0) |
         (p.document_ids != nullptr ? 2 : 0);
}

// meta < 0: the problem's own metadata kinds; doc_pass: see FwdParams.
template <int D, int BN, int DSPLIT, int NQG, bool VDOUBLE, int OCC = 1>
static hipError_t launch_fwd_cfg(const FwdParams& a, hipStream_t stream, bool fixup = false,
                                 int meta_override = -1, int doc_pass = 0) {
  using C = FwdCfg<D, BN, DSPLIT, NQG, VDOUBLE>;
  const int meta = meta_override >= 0 ? meta_override : meta_kind(a.p);
  void (*kern)(FwdParams) =
      meta == 1   ? fwd_kernel<D, BN, DSPLIT, NQG, VDOUBLE, 1, false, OCC>
      : meta == 2 ? fwd_kernel<D, BN, DSPLIT, NQG, VDOUBLE, 2, false, OCC>
      : meta == 3 ? fwd_kernel<D, BN, DSPLIT, NQG, VDOUBLE, 3, false, OCC>
      : fixup     ? fwd_kernel<D, BN, DSPLIT, NQG, VDOUBLE, 0, true, OCC>
                  : fwd_kernel<D, BN, DSPLIT, NQG, VDOUBLE, 0, false, OCC>;
  const int variant = fixup ? 4 : meta;
  static LdsAttr attr[5];
  hipError_t e = attr[variant].ensure((const void*)kern, C::kLdsBytes);
  if (e != hipSuccess) return e;
  FwdParams b = a;
  b.doc_pass = doc_pass;
  // (the fixup pass and the listed second document pass decode full-grid indices)
  int64_t nblocks = fwd_grid(&b, C::kBM, !fixup && doc_pass != 2);
  if (nblocks <= 0) return hipSuccess;
  if (doc_pass == 2 && a.doc_list != nullptr) {
    // the first pass's list, over at most one resident grid
    static PersistentGrid grid;
    bool many = false;
    const int64_t g = grid.size((const void*)kern, C::kNT, C::kLdsBytes, nblocks, &many);
    if (g <= 0) return hipErrorInvalidValue;
    nblocks = many ? g : nblocks;
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)nblocks), dim3(C::kNT), C::kLdsBytes, stream, b);
  return hipGetLastError();
}

__global__ void clear_list_kernel(unsigned* n) {
  if (threadIdx.x == 0) *n = 0u;
}

hipError_t launch_fwd(const FwdParams& a, hipStream_t stream) {
  if (a.split_chunks > 0) {
    if (a.p.head_dim == 256) return launch_fwd_split<256>(a, stream);
    if (a.p.head_dim == 512) return launch_fwd_split<512>(a, stream);
    return hipErrorInvalidValue;
  }
  if (a.p.head_dim == 256) {
    // Two workgroups of 32-key tiles share a CU (the register file holds two
    // waves per SIMD).  With both vision and document IDs the mask state needs
    // one workgroup of 64-key tiles per CU, so such a problem is split: the
    // query tiles that see a single document run in the vision-only kernel,
    // the rest in the full-mask one.
    if (meta_kind(a.p) != 3) return launch_fwd_cfg<256, 32, 1, 4, true, 2>(a, stream);
    static_assert(FwdCfg<256, 32, 1, 4, true>::kBM == FwdCfg<256, 64, 1, 4, true>::kBM,
                  "both passes must tile queries alike");
    if (a.doc_list_n != nullptr) {
      // pass 1 refills the list on every call (a fill kernel, not a memset
      // node, so the launch sequence can be captured in a graph)
      hipLaunchKernelGGL(clear_list_kernel, dim3(1), dim3(64), 0, stream, a.doc_list_n);
      hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
    hipError_t e = launch_fwd_cfg<256, 32, 1, 4, true, 2>(a, stream, false, /*meta=*/1,
                                                          /*doc_pass=*/1);
    if (e != hipSuccess) return e;
    return launch_fwd_cfg<256, 64, 1, 4, true, 1>(a, stream, false, /*meta=*/3,
                                                  /*doc_pass=*/2);
  }
  if (a.p.head_dim == 512) {
    if (meta_kind(a.p) != 0 || a.raise_flags == nullptr)
      return launch_fwd_cfg<512, 32, 2, 2, true>(a, stream);
    // Fast pass, then the rescaling kernel on the 32-query groups it flagged.
    hipError_t e = launch_fwd_wide<512>(a, stream);
    if (e != hipSuccess) return e;
    return launch_fwd_cfg<512, 32, 2, 2, true>(a, stream, /*fixup=*/true);
  }
  return hipErrorInvalidValue;
}

}  // namespace g4
