// Shared device-side building blocks of the gfx950 Gemma 4 attention kernels.
//
// Conventions (all kernels):
//  * MFMA v_mfma_f32_32x32x16_bf16 (64 lanes).  For C[32 x 32] += A[32 x 16] B[16 x 32]:
//      A: lane l holds row (l & 31), k = 8*(l >> 5) + 0..7
//      B: lane l holds col (l & 31), k = 8*(l >> 5) + 0..7
//      C: lane l, register r holds row 8*(r >> 2) + 4*(l >> 5) + (r & 3), col (l & 31)
//  * Reduction-dimension permutation: when an accumulator tile is reused as an
//    MFMA operand, the 16 k-values an MFMA consumes are taken from accumulator
//    registers 8m..8m+7, i.e. rows {16m' + 4h + e, 16m' + 8 + 4h + e : e < 4}
//    for lane half h.  The matching operand is read with two transposing LDS
//    reads (ds_read_b64_tr_b16), one per 4-row group, so no data is permuted
//    in memory.
//  * LDS tiles hold rows of 16-byte chunks; chunk c of row r is stored at slot
//    c ^ swz(r) with swz(r) = 4*(r & 3) + ((r >> 2) & 3), which keeps both the
//    row-wise 16-byte MFMA operand reads and the 4-row transposing reads free of
//    bank conflicts.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemma4_attn.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

#define G4_LDS __attribute__((address_space(3)))
#define G4_GLOBAL __attribute__((address_space(1)))

namespace g4 {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_huge_valf();

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Swizzled 16-byte slot of chunk c in row r.
__device__ __forceinline__ int swz_slot(int r, int c) {
  return c ^ (((r & 3) << 2) | ((r >> 2) & 3));
}

// Byte offset of element (row r, column col) of a bf16 LDS tile whose rows
// hold `row_chunks` 16-byte chunks.  col must be a multiple of 4 (8-byte
// accesses) -- the 8-byte half within the chunk is preserved.
__device__ __forceinline__ int lds_off(int r, int col, int row_chunks) {
  int c = col >> 3;
  return (r * row_chunks + swz_slot(r, c)) * 16 + (col & 7) * 2;
}

__device__ __forceinline__ bf16x8 lds_read16(const char G4_LDS* base, int off) {
  return *(const bf16x8 G4_LDS*)(base + off);
}

// Transposing 8-byte LDS reads (ds_read_b64_tr_b16).  Without alias-scope
// metadata on the read the compiler's wait insertion ties it to every
// outstanding buffer -> LDS copy and waits for them all (vmcnt 0) before it,
// although the copies fill the other buffer.  The restrict-qualified
// parameter of lds_read_tr_scoped gives the read that metadata once inlined,
// so no such wait is inserted; every kernel here orders its copies and reads
// itself (vm_wait before the barrier that publishes a copied buffer).
__device__ __forceinline__ bf16x4 lds_read_tr_scoped(const char G4_LDS* __restrict__ p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((bf16x4 G4_LDS*)p);
}
__device__ __forceinline__ bf16x4 lds_read_tr_waited(const char G4_LDS* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((bf16x4 G4_LDS*)p);
}
template <bool SCOPED>
__device__ __forceinline__ bf16x4 lds_read_tr(const char G4_LDS* p) {
  if constexpr (SCOPED)
    return lds_read_tr_scoped(p);
  else
    return lds_read_tr_waited(p);
}

__device__ __forceinline__ bf16x8 cat4(bf16x4 a, bf16x4 b) {
  return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

__device__ __forceinline__ bf16x8 ld_global16(const void* p) {
  return *(const bf16x8*)p;
}

// Value of lane l ^ 32.  v_permlane32_swap_b32 with both operands x returns
// (x with lanes 32-63 replaced by lanes 0-31, x with lanes 0-31 replaced by
// lanes 32-63): a VALU exchange, so no LDS permute and no LDS-counter wait
// that would drain the wave's in-flight operand reads.
__device__ __forceinline__ float wave_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float((__lane_id() & 32) ? r[0] : r[1]);
}

// Workgroup barrier that orders LDS traffic only.  Unlike __syncthreads() it
// does not drain outstanding global loads, so tile copies issued earlier stay
// in flight across it; callers wait for those with vm_wait<N>() first.
__device__ __forceinline__ void barrier_lds() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Wait until at most N vector-memory operations of this wave are outstanding.
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}



// Async 16-byte buffer -> LDS copy from a wave-uniform base with a 32-bit
// per-lane byte offset (raw buffer, no stride, 2 GiB range): lane l writes LDS
// bytes [lds_wave_base + 16 l, +16).  The offset stays a single 32-bit VGPR.
__device__ __forceinline__ void b2l16(const void* base, uint32_t voff, char G4_LDS* lds_wave_base) {
  __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7fffffff, 0x00020000);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (void G4_LDS*)lds_wave_base, 16, voff, 0, 0, 0);
}

// The same copy with the non-temporal cache policy (nt): for data read once
// (the stored dS tiles), so the stream does not push operands that other
// workgroups re-read out of the L2.
__device__ __forceinline__ void b2l16_nt(const void* base, uint32_t voff,
                                         char G4_LDS* lds_wave_base) {
  __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7fffffff, 0x00020000);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (void G4_LDS*)lds_wave_base, 16, voff, 0, 0,
                                           /*nt=*/2);
}

// Async 4-byte global -> LDS copy: lane l writes LDS bytes [lds_wave_base +
// 4 l, +4) from base + voff (a uniform base, a 32-bit per-lane byte offset).
// Through a buffer descriptor rather than a global address: the compiler
// counts a buffer copy with the vector memory counter only, while after the
// global form the LDS operand reads that follow were all waited for at once.
__device__ __forceinline__ void b2l4(const void* base, uint32_t voff, char G4_LDS* lds_wave_base) {
  __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7fffffff, 0x00020000);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (void G4_LDS*)lds_wave_base, 4, voff, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// Row-wise 16-byte MFMA operand reads of a swizzled tile with CPR chunks per
// row: lane reads row (row0 + (lane & 31)) and chunk (cbase + 2 c' + (lane >> 5)),
// row0 and cbase multiples of 16.  With sw = swz(r), the slot of chunk
// 2w + h (w < 8) is 2 (w ^ (sw >> 1)) + (h ^ (sw & 1)), so the byte offset is
// one per-lane base with the constant 32 w XORed into bits 5-7 (which hold
// sw >> 1): one VGPR and one v_xor per read instead of an offset table.
template <int CPR>
struct RowReader {
  int base;
  // b: byte offset added to every read (e.g. the wave's head-dim slice, a
  // multiple of 256), folded in here.
  __device__ __forceinline__ void init(int lane, int b = 0) {
    const int r = lane & 31, h = lane >> 5;
    const int sw = ((r & 3) << 2) | ((r >> 2) & 3);
    base = b + r * CPR * 16 + 32 * (sw >> 1) + 16 * (h ^ (sw & 1));
  }
  template <int ROW0, int CBASE, int CP>
  __device__ __forceinline__ bf16x8 read(const char G4_LDS* tile) const {
    static_assert(ROW0 % 16 == 0 && CBASE % 16 == 0, "alignment");
    const int off = base ^ (32 * (CP & 7));
    return *(const bf16x8 G4_LDS*)(tile + off + (ROW0 * CPR + CBASE + 16 * (CP >> 3)) * 16);
  }
};

// Transposing reads that build a 32 x 16 MFMA A operand (rows = 32 columns of
// the tile starting at chunk cbase + 4 b, k = 16 tile rows starting at row0)
// from a row-major swizzled tile: lane l gets column 16*((l>>4)&1) + (l&15)
// and rows {4h + e, 8 + 4h + e}.  Chunk 4 bq + lb sits in slot
// 4 (bq ^ (sw >> 2)) + (lb ^ (sw & 3)), so each of the two row groups needs
// one per-lane base with 64 bq XORed into bits 6-7.  SCOPED: see lds_read_tr.
template <int CPR, bool SCOPED = true>
struct TrReader {
  int base[2];
  __device__ __forceinline__ void init(int lane, int b = 0) {
    const int g = lane >> 4, sl = lane & 15;
    const int rl = 4 * (g >> 1) + (sl >> 2);
    const int lb = 2 * (g & 1) + ((sl >> 1) & 1);
    const int half = (sl & 1) * 8;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int r = rl + 8 * e;
      const int sw = ((r & 3) << 2) | ((r >> 2) & 3);
      base[e] = b + r * CPR * 16 + 64 * (sw >> 2) + 16 * (lb ^ (sw & 3)) + half;
    }
  }
  template <int ROW0, int CBASE, int B>
  __device__ __forceinline__ bf16x8 read(const char G4_LDS* tile) const {
    static_assert(ROW0 % 16 == 0 && CBASE % 16 == 0, "alignment");
    constexpr int imm = (ROW0 * CPR + CBASE + 16 * (B >> 2)) * 16;
    bf16x4 lo = lds_read_tr<SCOPED>(tile + (base[0] ^ (64 * (B & 3))) + imm);
    bf16x4 hi = lds_read_tr<SCOPED>(tile + (base[1] ^ (64 * (B & 3))) + imm);
    return cat4(lo, hi);
  }
};

// Async copy of a BN-row tile of a row-major operand (rows of CPR = 32 or 64
// 16-byte chunks) into a swizzled LDS tile by NW waves.  Copy instruction i
// of a wave fills LDS bytes [1 KB * u, +1 KB) with u = i * NW + wave: rows
// u * (64 / CPR) + lane / CPR, chunk slot lane % CPR.  The row is wave-uniform
// up to lane / CPR, so addresses are formed at issue time (scalar row math plus
// a couple of VALU ops) instead of from per-lane offset tables, which keeps
// copies from pinning VGPRs that would otherwise spill.
// FRESH: re-form the per-lane offsets at every issue (see fresh_lane), for
// kernels whose register budget cannot hold them across a loop.
template <int CPR, int BN, int NW, bool FRESH = false>
struct TileCopier {
  static_assert(CPR == 32 || CPR == 64, "rows of 32 or 64 chunks");
  static constexpr int kRows = 64 / CPR;  // rows per copy instruction
  static constexpr int kPer = BN * CPR / (64 * NW);
  static_assert(kPer * 64 * NW == BN * CPR, "tile must split evenly over the waves");
  int wave, lane;
  int64_t stride_bytes;
  __device__ __forceinline__ void init(int64_t row_stride_elems, int wave_, int lane_) {
    wave = wave_;
    lane = lane_;
    stride_bytes = row_stride_elems * 2;
  }
  // rows row0 .. row0 + BN - 1 must all exist.  The scalar base carries the
  // instruction's first row; the per-lane offset (row within the instruction,
  // chunk column) is a 32-bit buffer offset for 32-chunk rows, where a 64-bit
  // per-lane address would be hoisted out of loops and spilled (the C ABI
  // bounds token strides below 2^24 elements, so offsets stay below 2^31).
  // With FRESH the lane id is passed through an empty asm so the per-lane
  // offsets are formed at each issue (a few VALU ops) rather than hoisted out
  // of the caller's loop into registers that would then be spilled.
  __device__ __forceinline__ int fresh_lane() const {
    int l = lane;
    if constexpr (FRESH) asm volatile("" : "+v"(l));
    return l;
  }
  __device__ __forceinline__ void issue(const __bf16* tile_row0, char G4_LDS* tile) const {
    const char* g = (const char*)tile_row0;
    const int ln = fresh_lane();
    if constexpr (CPR == 64) {
      // one row per instruction: the slot is lane ^ swz(row)
      const int lr = ln / CPR, lc = ln % CPR;
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int u = i * NW + wave;
        const int r = u * kRows + lr;
        const uint32_t c = lc ^ (((r & 3) << 2) | ((r >> 2) & 3));
        const char* row = g + (int64_t)(u * kRows) * stride_bytes;
        b2l16(row, c * 16u, tile + u * 1024);
      }
    } else {
      // Two rows per instruction: lane row lr = ln >> 5, row r = 2u + lr.  As 2u
      // is even, swz(r) = swz(2u) ^ (lr << 2), so the slot (ln & 31) ^ swz(r)
      // is a lane constant XOR a wave-uniform value: one v_xad_u32 per copy.
      const int lr = ln >> 5;
      const uint32_t lane16 = (uint32_t)(((ln & 31) ^ (lr << 2)) << 4);
      const uint32_t lane_row = lr ? (uint32_t)stride_bytes : 0u;
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int u = i * NW + wave;
        const int r = 2 * u;
        const uint32_t s16 = (uint32_t)((((r & 3) << 2) | ((r >> 2) & 3)) << 4);
        b2l16(g + (int64_t)r * stride_bytes, (lane16 ^ s16) + lane_row, tile + u * 1024);
      }
    }
  }
  // Tail tile: rows >= nrows are replaced by row nrows - 1 (their scores are
  // masked, so they only need to be finite data).
  __device__ __forceinline__ void issue_clamped(const __bf16* tile_row0, int64_t, int nrows,
                                                char G4_LDS* tile, int = 0, int = 0) const {
    const char* g = (const char*)tile_row0;
    const int ln = fresh_lane();
    const int lr = ln / CPR, lc = ln % CPR;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int u = i * NW + wave;
      const int r = u * kRows + lr;
      const uint32_t c = lc ^ (((r & 3) << 2) | ((r >> 2) & 3));
      b2l16(g, (uint32_t)min(r, nrows - 1) * (uint32_t)stride_bytes + c * 16u, tile + u * 1024);
    }
  }
};

// Scheduling hint for a region of N MFMAs fed by LDS reads: PRE reads first,
// then (1 MFMA, PER reads) repeated, so only a few operand fragments are in
// flight at any time (the default schedule hoists every read to the top of
// the region and runs out of VGPRs).  Place it at the end of the region,
// which must be delimited by sched_barrier(0).
template <int N, int PRE, int PER>
__device__ __forceinline__ void mfma_pipeline_hint() {
  __builtin_amdgcn_sched_group_barrier(0x100, PRE, 0);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, PER, 0);
  }
}

// Sequence geometry resolved from a problem (fixed or packed).
struct Seq {
  int lq, lk;          // lengths
  int64_t qtok, ktok;  // token index of the sequence start in the Q / K stream
  int64_t q_off_b, k_off_b;  // fixed mode: element offsets of the batch
  bool packed;
};

__device__ __forceinline__ Seq resolve_seq(const g4_problem& p, int s) {
  Seq r;
  r.packed = p.cu_seqlens_q != nullptr;
  if (r.packed) {
    int q0 = p.cu_seqlens_q[s], q1 = p.cu_seqlens_q[s + 1];
    int k0 = p.cu_seqlens_k[s], k1 = p.cu_seqlens_k[s + 1];
    r.lq = q1 - q0;
    r.lk = k1 - k0;
    r.qtok = q0;
    r.ktok = k0;
  } else {
    r.lq = p.seqlen_q;
    r.lk = p.seqlen_k;
    r.qtok = (int64_t)s * p.seqlen_q;
    r.ktok = (int64_t)s * p.seqlen_k;
  }
  return r;
}

// Element offset of token t (sequence-local) of sequence s in an operand.
__device__ __forceinline__ int64_t tok_off(const Seq& sq, int s, int64_t seq_tok0, int t,
                                           const g4_layout& L) {
  return sq.packed ? (seq_tok0 + t) * L.token_stride
                   : (int64_t)s * L.batch_stride + (int64_t)t * L.token_stride;
}

// True when every K-stream position [lo, hi) of a sequence (clamped to its
// lk keys) carries one document ID.  A workgroup whose queries and visited
// key tiles all lie in such a range sees the document predicate admit every
// pair it visits, so it drops the predicate (and its per-tile ID copies)
// exactly.  The range must span whole visited tiles, not only the scheduled
// key range: vision spans are per (document, vision ID), so a tile's tail
// past the range can hold keys of the same vision block in another document.  Every thread of the workgroup calls
// this; `red` is one int per wave of LDS, free on entry.
template <int NW>
__device__ __forceinline__ bool doc_uniform(const int* doc, int64_t ktok, int lk, int lo, int hi,
                                            int tid, int lane, int wave, int* red) {
  lo = max(lo, 0);
  hi = min(hi, lk);
  if (lo >= hi) return true;
  const int ref = doc[ktok + lo];
  bool diff = false;
  for (int t = lo + tid; t < hi; t += NW * 64) diff |= doc[ktok + t] != ref;
  const bool wave_diff = __ballot(diff) != 0;  // every lane votes (outside the lane-0 branch)
  barrier_lds();  // earlier readers of red are done
  if (lane == 0) red[wave] = wave_diff;
  barrier_lds();
  int any = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) any |= red[w];
  return any == 0;
}

// Async copy of the vision / document IDs of keys [j0, j0 + 64) of a sequence
// (clamped to its last key; keys past the end are masked by index) into
// [vid x 64 | doc x 64] int32 at dst.  One wave issues it.
__device__ __forceinline__ void issue_key_meta(const g4_problem& p, const Seq& sq, int j0,
                                               char G4_LDS* dst, int lane, bool vid, bool doc) {
  // uniform base at the tile's first (clamped) key, small per-lane offsets
  const int j0c = min(j0, sq.lk - 1);
  const int64_t base = sq.ktok + j0c;
  const uint32_t off = (uint32_t)(min(j0 + lane, sq.lk - 1) - j0c) * 4u;
  if (vid) b2l4(p.vision_ids + base, off, dst);
  if (doc) b2l4(p.document_ids + base, off, dst + 256);
}

// First key tile (64 keys) of the stored-dS band of the 32-query row whose
// first query sits at key position a_first (window W > 0).
__device__ __forceinline__ int ds_band_first(int a_first, int window) {
  return max(a_first - window + 1, 0) / 64;
}

// Tokens in the Q stream (packed total, or num_seqs * seqlen_q).
__device__ __forceinline__ int64_t q_stream_tokens_dev(const g4_problem& p) {
  return p.cu_seqlens_q ? p.total_q : (int64_t)p.num_seqs * p.seqlen_q;
}

// LSE / delta element offset for (s, h, local token i).
__device__ __forceinline__ int64_t lse_off(const g4_problem& p, const Seq& sq, int s, int h,
                                           int i) {
  return (sq.packed ? sq.qtok : (int64_t)s * p.lse_batch_stride) +
         (int64_t)h * p.lse_head_stride + i;
}

// The Gemma predicate for query at K-position a and key j of one sequence.
__device__ __forceinline__ bool allowed(int a, int j, int window, bool bidir, int vq, int vk,
                                        bool use_doc, int dq, int dk) {
  bool keep = (j <= a) || (bidir && vq >= 0 && vq == vk);
  if (window > 0) keep = keep && (j > a - window);
  if (use_doc) keep = keep && (dq == dk);
  return keep;
}

// Key range [lo, hi) (sequence-local key indices) a tile of queries whose
// K-positions are [a0, a1] may attend to, given the maximum span end of its
// vision queries (span_hi_max, -1 if none).
__device__ __forceinline__ void query_tile_key_range(int a0, int a1, int lk, int window,
                                                     int span_hi_max, int& lo, int& hi) {
  lo = window > 0 ? max(0, a0 - window + 1) : 0;
  hi = max(a1, span_hi_max) + 1;
  hi = min(hi, lk);
}

// Query range [lo, hi) (sequence-local query indices) a tile of keys [j0, j1]
// may be attended by, given the minimum span start of its vision keys
// (span_lo_min, large if none).  off = Sk - Sq.
__device__ __forceinline__ void key_tile_query_range(int j0, int j1, int lq, int off, int window,
                                                     int span_lo_min, int& lo, int& hi) {
  int a_lo = min(j0, span_lo_min);
  int a_hi = window > 0 ? j1 + window - 1 : 0x7fffffff - 1;
  lo = max(0, a_lo - off);
  hi = min(lq, a_hi - off + 1);
  if (hi < lo) hi = lo;
}

// Map the hardware block index onto a logical work index so that each XCD
// (blocks are dealt round-robin over 8 XCDs) receives a contiguous run of
// logical work items.  Bijective for any grid size.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
  constexpr int kXcd = 8;
  int xcd = bid % kXcd, pos = bid / kXcd;
  int base = nblocks / kXcd, extra = nblocks % kXcd;
  return xcd * base + min(xcd, extra) + pos;
}

// xcd_remap for a grid whose work items come in zigzag ranks (unit items per
// rank, see zigzag): within each XCD's run the even ranks (heavy tiles,
// heaviest first) come before the odd ranks taken backwards (light tiles,
// heaviest first), so each XCD starts its heaviest items first and ends on
// its lightest.  Needs nblocks to be a multiple of 16 unit (every run then
// holds an even number of whole ranks).
__device__ __forceinline__ int xcd_remap_desc(int bid, int nblocks, int unit) {
  constexpr int kXcd = 8;
  const int xcd = bid % kXcd, pos = bid / kXcd;
  const int len = nblocks / kXcd, m = len / (2 * unit);
  const int q = pos / unit, g = pos % unit;
  const int r = q < m ? 2 * q : 4 * m - 1 - 2 * q;
  return xcd * len + r * unit + g;
}

// Tile rank -> tile index alternating from the heaviest (last) tile:
// n-1, 0, n-2, 1, ...
__device__ __forceinline__ int zigzag(int r, int n) {
  return (r & 1) ? (r >> 1) : (n - 1 - (r >> 1));
}
// Its inverse: the rank of tile t among n.
__device__ __forceinline__ int unzigzag(int t, int n) {
  return 2 * t >= n - 1 ? 2 * (n - 1 - t) : 2 * t + 1;
}

// Thread index as seen by one work item.  In a queue kernel (QUEUE) it passes
// through an empty asm, so the per-lane offsets derived from it are formed in
// each item rather than hoisted out of the ticket loop into registers held
// across all items (which then spill inside the step loops).
template <bool QUEUE>
__device__ __forceinline__ int item_thread_id() {
  int t = threadIdx.x;
  if constexpr (QUEUE) asm volatile("" : "+v"(t));
  return t;
}

// Work queue of a persistent launch (at most as many workgroups as are
// resident at once, each taking tiles until they run out), so every CU stays
// busy to the end however unevenly the tiles' costs or the hardware's
// workgroup placement fall.  Workgroup b first takes item xcd_remap(b) (no
// atomic; each XCD starts on a contiguous range), then tickets
// gridDim.x + atomicAdd(counter, 1).  The n draws of a launch return the old
// values 0 .. n - 1; the workgroup that draws n - 1 is the last to draw and
// zeroes the counter for the next launch on the same workspace (the first
// launch relies on it being zero).  A later ticket passes through an LDS slot
// that lies in the tile area, so no copy may be in flight into it.
struct WorkQueue {
  unsigned* counter;
  int n;      // work items
  int taken;  // items this workgroup has started
  __device__ __forceinline__ int next(int G4_LDS* slot) {
    if (taken++ == 0) return xcd_remap(blockIdx.x, gridDim.x);
    vm_wait<0>();
    barrier_lds();  // every wave is done with the previous item's LDS
    if (threadIdx.x == 0) {
      const unsigned old = atomicAdd(counter, 1u);
      if (old == (unsigned)n - 1u) atomicExch(counter, 0u);
      *slot = (int)(gridDim.x + old);
    }
    barrier_lds();
    const int t = __builtin_amdgcn_readfirstlane(*slot);
    barrier_lds();  // every wave has read the slot before the next item's copies
    return t;
  }
};

// Row tiles of the sequences of a packed problem, so that a launch sized by
// its longest sequence can enumerate only the tiles that exist (in a packed
// batch most of the (sequence, tile) grid is past its sequence's end, and
// each such item still costs a queue draw).  Lane i of every wave holds
// sequence i's tile count and the inclusive prefix over sequences 0..i; up to
// 64 sequences (ok = false otherwise, and for fixed layouts).
struct SeqTiles {
  int cnt, incl, total;
  bool ok;
  __device__ __forceinline__ void init(const int* cu, int nseq, int rows_per_tile) {
    const int lane = __lane_id();
    ok = cu != nullptr && nseq <= 64;
    cnt = 0;
    if (ok && lane < nseq) cnt = (cu[lane + 1] - cu[lane] + rows_per_tile - 1) / rows_per_tile;
    int x = cnt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    incl = x;
    total = __builtin_amdgcn_readfirstlane(__shfl(x, 63, 64));
  }
  // Sequence s, index within it and tile count of the r-th existing tile.
  __device__ __forceinline__ void find(int r, int& s, int& local, int& nt) const {
    s = __builtin_amdgcn_readfirstlane(__popcll(__ballot(incl <= r)));
    local = r - __builtin_amdgcn_readfirstlane(__shfl(incl - cnt, s, 64));
    nt = __builtin_amdgcn_readfirstlane(__shfl(cnt, s, 64));
  }
  // The table in LDS (64 x {incl, cnt}), for kernels that cannot keep it in
  // registers across their items: stored by wave 0, read back by find_lds.
  __device__ __forceinline__ void store(int G4_LDS* tab) const {
    const int lane = __lane_id();
    tab[2 * lane] = incl;
    tab[2 * lane + 1] = cnt;
  }
  __device__ static __forceinline__ void find_lds(const int G4_LDS* tab, int r, int& s,
                                                  int& local, int& nt) {
    SeqTiles t;
    const int lane = __lane_id();
    t.incl = tab[2 * lane];
    t.cnt = tab[2 * lane + 1];
    t.find(r, s, local, nt);
  }
};

// Work units of the sequences of a packed problem (up to 64) in the order of
// their query lengths, longest first (ties by index): for a queue whose items
// all cost about the same within a sequence and whose cost grows with the
// sequence's length, so the heaviest items are drawn first.  Lane i of every
// wave holds sequence i's unit count and the units of the sequences before it
// in that order.
struct SeqUnitsByLength {
  int cnt, lo, total;
  // cu_len orders the sequences; units(sequence, length from cu_cnt) counts
  // their units.
  template <class Units>
  __device__ __forceinline__ void init(const int* cu_len, const int* cu_cnt, int nseq,
                                       Units units) {
    const int lane = __lane_id();
    int len = -1;
    cnt = 0;
    if (lane < nseq) {
      len = cu_len[lane + 1] - cu_len[lane];
      cnt = units(lane, cu_cnt[lane + 1] - cu_cnt[lane]);
    }
    int before = 0;
    for (int j = 0; j < nseq; ++j) {
      const int lj = __builtin_amdgcn_readlane(len, j);
      const int cj = __builtin_amdgcn_readlane(cnt, j);
      if (lj > len || (lj == len && j < lane)) before += cj;
    }
    lo = before;
    int x = cnt;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
    total = __builtin_amdgcn_readfirstlane(x);
  }
  // Sequence s, its unit count n and the index within it of unit u (< total).
  __device__ __forceinline__ void find(int u, int& s, int& local, int& n) const {
    const unsigned long long m = __ballot(lo <= u && u < lo + cnt);
    s = __builtin_amdgcn_readfirstlane(__ffsll((long long)m) - 1);
    local = u - __builtin_amdgcn_readfirstlane(__shfl(lo, s, 64));
    n = __builtin_amdgcn_readfirstlane(__shfl(cnt, s, 64));
  }
  // The table in LDS (64 x {lo, cnt}): stored by wave 0, read back by find_lds.
  __device__ __forceinline__ void store(int G4_LDS* tab) const {
    const int lane = __lane_id();
    tab[2 * lane] = lo;
    tab[2 * lane + 1] = cnt;
  }
  __device__ static __forceinline__ void find_lds(const int G4_LDS* tab, int u, int& s,
                                                  int& local, int& n) {
    SeqUnitsByLength t;
    const int lane = __lane_id();
    t.lo = tab[2 * lane];
    t.cnt = tab[2 * lane + 1];
    t.find(u, s, local, n);
  }
};

// The same protocol with each ticket drawn when the previous item starts, so
// the atomic's latency overlaps that item, and without WorkQueue's wait for
// the item's memory operations: for items that leave no tile copy in flight
// (their global stores do not touch LDS).
//   PrefetchQueue q{counter, n};
//   for (int t = q.first(); q.valid(t); t = q.next(slot)) { q.draw(); item(t); }
struct PrefetchQueue {
  unsigned* counter;
  unsigned n;
  unsigned old = 0;
  __device__ __forceinline__ int first() const { return xcd_remap(blockIdx.x, gridDim.x); }
  __device__ __forceinline__ bool valid(int t) const { return (unsigned)t < n; }
  __device__ __forceinline__ void draw() {
    if (threadIdx.x == 0) old = atomicAdd(counter, 1u);
  }
  __device__ __forceinline__ int next(int G4_LDS* slot) {
    barrier_lds();  // every wave is done with the item's LDS
    if (threadIdx.x == 0) {
      if (old == n - 1u) atomicExch(counter, 0u);
      *slot = (int)(gridDim.x + old);
    }
    barrier_lds();
    const int t = __builtin_amdgcn_readfirstlane(*slot);
    barrier_lds();  // every wave has read the slot before the next item's copies
    return t;
  }
};

// Work queue split over the eight XCDs, for items whose neighbours share
// operands: item range [c n / 8, (c + 1) n / 8) belongs to XCD c, and the
// workgroups of XCD c (blockIdx.x % 8 under the round-robin dispatch that
// xcd_remap also assumes) draw it in order from counter c, so neighbouring
// items run at the same time on the workgroups that share one L2.  A
// workgroup whose range is exhausted draws from the next XCD's (c + 1, ...),
// which only happens at the end of the launch.  Counters: ctr[0..7] per range,
// ctr[8] counts the workgroups that finished; the last one zeroes all nine for
// the next launch on the same workspace (the first relies on them being
// zero).  Thread 0 draws the next ticket while the current item runs:
//   XcdQueue q{ctr, n}; q.draw();
//   for (int t = q.next(slot); t >= 0; t = q.next(slot)) { q.draw(); item(t); }
// (no tile copy may be in flight into the LDS slot at next()).
struct XcdQueue {
  static constexpr int kXcd = 8;
  unsigned* ctr;
  unsigned n;
  int probe = 0;     // thread 0: ranges tried, from this XCD's own
  unsigned old = 0;  // thread 0: the ticket drawn from range (xcd + probe) % 8
  __device__ __forceinline__ int xcd() const { return (int)(blockIdx.x % kXcd); }
  __device__ __forceinline__ unsigned lo(int c) const {
    return (unsigned)(((unsigned long long)c * n) / kXcd);
  }
  __device__ __forceinline__ void draw() {
    if (threadIdx.x == 0 && probe < kXcd) old = atomicAdd(&ctr[(xcd() + probe) % kXcd], 1u);
  }
  // Next item of this workgroup (uniform), or -1 when every range is exhausted.
  __device__ __forceinline__ int next(int G4_LDS* slot) {
    barrier_lds();  // every wave is done with the previous item's LDS
    if (threadIdx.x == 0) {
      int item = -1;
      while (probe < kXcd) {
        const int c = (xcd() + probe) % kXcd;
        if (lo(c) + old < lo(c + 1)) {
          item = (int)(lo(c) + old);
          break;
        }
        if (++probe < kXcd) old = atomicAdd(&ctr[(xcd() + probe) % kXcd], 1u);
      }
      if (item < 0 && atomicAdd(&ctr[kXcd], 1u) == gridDim.x - 1u) {
#pragma unroll
        for (int c = 0; c <= kXcd; ++c) atomicExch(&ctr[c], 0u);
      }
      *slot = item;
    }
    barrier_lds();
    const int t = __builtin_amdgcn_readfirstlane(*slot);
    barrier_lds();  // every wave has read the slot before the next item's copies
    return t;
  }
};

// MFMA chains with A LDS operand reads in flight (kAhead unless a caller
// picks another depth): read n + A is issued right after MFMA n and
// sched_barrier pins that order.  Left to itself the scheduler falls back to
// one read per MFMA, each waited for, whenever registers are tight.
constexpr int kAhead = 2;

// acc[B] += (tile^T rows 16 M ...)[32 x 16] . b[M], over M in {0, 1}, B in [0, NB).
template <int NB, int N, class TR>
__device__ __forceinline__ bf16x8 acc_read(const TR& trd, const char G4_LDS* t) {
  return trd.template read<16 * (N / NB), 0, N % NB>(t);
}
template <int NB, int A, int N, class TR>
__device__ __forceinline__ void acc_pipe(const TR& trd, const char G4_LDS* t,
                                         const bf16x8 (&b)[2], f32x16 (&acc)[NB],
                                         bf16x8 (&x)[A]) {
  if constexpr (N < 2 * NB) {
    acc[N % NB] = mfma32(x[N % A], b[N / NB], acc[N % NB]);
    if constexpr (N + A < 2 * NB) x[N % A] = acc_read<NB, N + A>(trd, t);
    __builtin_amdgcn_sched_barrier(0);
    acc_pipe<NB, A, N + 1>(trd, t, b, acc, x);
  }
}
template <int NB, int A, int N, class TR>
__device__ __forceinline__ void acc_prologue(const TR& trd, const char G4_LDS* t,
                                             bf16x8 (&x)[A]) {
  if constexpr (N < A) {
    x[N] = acc_read<NB, N>(trd, t);
    acc_prologue<NB, A, N + 1>(trd, t, x);
  }
}
// While a wave issues an MFMA chain it runs at raised priority, so that when
// the two waves of a SIMD are both ready the matrix core is fed first.
__device__ __forceinline__ void mfma_prio_begin() { __builtin_amdgcn_s_setprio(1); }
__device__ __forceinline__ void mfma_prio_end() { __builtin_amdgcn_s_setprio(0); }

template <int NB, int A = kAhead, class TR>
__device__ __forceinline__ void acc_steps(const TR& trd, const char G4_LDS* t,
                                          const bf16x8 (&b)[2], f32x16 (&acc)[NB]) {
  static_assert(A >= 1 && A <= 2 * NB, "read depth");
  bf16x8 x[A];
  acc_prologue<NB, A, 0>(trd, t, x);
  __builtin_amdgcn_sched_barrier(0);
  mfma_prio_begin();
  acc_pipe<NB, A, 0>(trd, t, b, acc, x);
  mfma_prio_end();
}

// part += (tile rows)[32 x 16 CP ...] . frag[CP], over CP in [0, NC).
template <int NC, int A, int CP, class RR>
__device__ __forceinline__ void row_pipe(const RR& rrd, const char G4_LDS* t, f32x16& part,
                                         const bf16x8 (&frag)[NC], bf16x8 (&x)[A]) {
  if constexpr (CP < NC) {
    part = mfma32(x[CP % A], frag[CP], part);
    if constexpr (CP + A < NC) x[CP % A] = rrd.template read<0, 0, CP + A>(t);
    __builtin_amdgcn_sched_barrier(0);
    row_pipe<NC, A, CP + 1>(rrd, t, part, frag, x);
  }
}
template <int A, int N, class RR>
__device__ __forceinline__ void row_prologue(const RR& rrd, const char G4_LDS* t,
                                             bf16x8 (&x)[A]) {
  if constexpr (N < A) {
    x[N] = rrd.template read<0, 0, N>(t);
    row_prologue<A, N + 1>(rrd, t, x);
  }
}
template <int NC, int A = kAhead, class RR>
__device__ __forceinline__ void row_steps(const RR& rrd, const char G4_LDS* t, f32x16& part,
                                          const bf16x8 (&frag)[NC]) {
  static_assert(A >= 1 && A <= NC, "read depth");
  bf16x8 x[A];
  row_prologue<A, 0>(rrd, t, x);
  __builtin_amdgcn_sched_barrier(0);
  mfma_prio_begin();
  row_pipe<NC, A, 0>(rrd, t, part, frag, x);
  mfma_prio_end();
}

}  // namespace g4
