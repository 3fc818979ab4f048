/*
 * gemma4_attn.h -- C ABI of the MI355X (gfx950) Gemma 4 attention library.
 *
 * Plain C: pointers, sizes and two small POD structs; no torch types.  Every
 * entry point is stream-ordered on the caller's hipStream_t (passed as void*),
 * allocates no device memory (the caller passes a workspace sized by
 * g4_workspace_bytes), performs no host synchronisation, and returns a
 * G4_* status code; g4_last_error() describes the last failure of the calling
 * thread.
 *
 * The reference has no C FFI: its Python adapters call FlashAttention-4 CuTe
 * kernels directly.  Each entry point below names the reference call it
 * replaces (paths relative to the reference repository).
 *
 * Layouts.  Q/K/V/O are bf16 with unit stride along the head dimension.  A
 * problem is either
 *   - fixed: cu_seqlens_q == cu_seqlens_k == NULL, num_seqs sequences of
 *     seqlen_q queries and seqlen_k keys (BSHD; batch_stride is used), or
 *   - packed: int32 device cu_seqlens_q/k of num_seqs+1 entries (THD;
 *     batch_stride unused), seqlen_q/k are the maxima.
 * Queries are the lower-right suffix of their key sequence (q_abs = i + Sk - Sq).
 * LSE is fp32, token-contiguous: element (seq s, head h, token i) lives at
 *   lse + (packed ? cu_q[s] : s * lse_batch_stride) + h * lse_head_stride + i,
 * i.e. (B, Hq, S) fixed or (Hq, Tq) packed.  Vision/document IDs are int32 over
 * the K stream (num_seqs*seqlen_k fixed, total_k packed), NULL when absent.
 *
 * Mask: allowed(q, k) = (k <= q  OR  (bidirectional AND vid[q] >= 0 AND
 * vid[q] == vid[k]))  AND  (window == 0 OR k > q - window)  AND
 * (doc == NULL OR doc[q] == doc[k]).
 */
#ifndef GEMMA4_ATTN_H
#define GEMMA4_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define G4_ABI_VERSION 2

enum g4_status {
  G4_OK = 0,
  G4_ERR_INVALID = 1,     /* malformed arguments (reference: ValueError) */
  G4_ERR_UNSUPPORTED = 2, /* outside the validated contract (reference: UnsupportedH100Path) */
  G4_ERR_WORKSPACE = 3,   /* workspace too small */
  G4_ERR_LAUNCH = 4       /* HIP launch failure */
};

/* Element strides of a bf16 (B, S, H, D) or (T, H, D) operand; D stride is 1. */
typedef struct g4_layout {
  int64_t batch_stride; /* fixed mode only */
  int64_t token_stride;
  int64_t head_stride;
} g4_layout;

typedef struct g4_problem {
  int32_t num_seqs;
  int32_t seqlen_q; /* fixed: per-sequence length; packed: max_seqlen_q */
  int32_t seqlen_k; /* fixed: per-sequence length; packed: max_seqlen_k */
  int32_t num_q_heads;
  int32_t num_kv_heads;
  int32_t head_dim;  /* 256 (local) or 512 (global); Dqk == Dv */
  int32_t window;    /* strict sliding window W (k > q - W), 0 = none */
  int32_t bidirectional_vision; /* 1: same non-negative vision block is allowed both ways */
  int64_t total_q;   /* tokens in the Q stream (packed) */
  int64_t total_k;   /* tokens in the K stream (packed) */
  const int32_t* cu_seqlens_q; /* device, NULL in fixed mode */
  const int32_t* cu_seqlens_k;
  const int32_t* vision_ids;   /* device, NULL when absent */
  const int32_t* document_ids; /* device, NULL when absent */
  int64_t lse_batch_stride;    /* fixed mode only */
  int64_t lse_head_stride;
  /* Bytes of the backward workspace that may hold dS tiles stored by the
   * dK/dV stage for the dQ stage: 0 = the library default (16 GiB), < 0 =
   * none.  When the tiles a problem needs exceed the budget, g4_attn_bwd
   * stripes head-dim 512 causal problems (see g4_attn_bwd); in every other
   * case none are stored and the dQ stage recomputes S and dP (slower,
   * workspace O(T) instead of O(T * Sk)).  Results are the same on every
   * route up to fp32 summation order.
   * The reference's global backward budget policy is the analogous knob
   * (src/gemma4_fa4/h100.py:713-746). */
  int64_t ds_budget;
} g4_problem;

/* Library ABI version (G4_ABI_VERSION). */
int g4_abi_version(void);

/* Description of the last error raised on this thread ("" if none). */
const char* g4_last_error(void);

/* Bytes of workspace g4_attn_fwd (phase 0) or g4_attn_bwd (phase 1) needs.
 * Returns 0 and sets the error on an invalid problem.  A valid problem that
 * needs no workspace (0 bytes) may pass a NULL workspace. */
size_t g4_workspace_bytes(const g4_problem* p, int phase);

/*
 * Forward: O = softmax(Q K^T (scale 1.0) + mask) V and fp32 LSE.
 * Replaces the FA4 forward launches of the reference adapters:
 *   fa4_local_text_forward     src/gemma4_fa4/h100.py:750-778
 *   fa4_local_forward          src/gemma4_fa4/h100.py:781-815 (+ h100_masks.py:26-59)
 *   fa4_local_varlen_forward   src/gemma4_fa4/h100.py:818-911 (+ h100_masks.py:62-152,
 *                              sparse schedule h100.py:490-601)
 *   global V-slab pairs        src/gemma4_fa4/h100.py:1148-1190, 1320-1387, 1013-1036
 * One launch covers the full Dv (no V slabs).  Problems without key
 * metadata whose query rows per KV head (query heads of a group x Sq) fit 32,
 * over at least 256 keys (a decode step), split the keys into chunks over
 * the GPU and merge the chunks' partial rows (kept in the workspace, which
 * g4_workspace_bytes counts): two launches.
 */
int g4_attn_fwd(const g4_problem* p,
                const void* q, g4_layout q_layout,
                const void* k, g4_layout k_layout,
                const void* v, g4_layout v_layout,
                void* o, g4_layout o_layout,
                float* lse,
                void* workspace, size_t workspace_bytes,
                void* stream);

/*
 * Forward exactly as g4_attn_fwd (same kernels, same results), with the
 * workspace taken from the library's own device memory instead of a caller
 * buffer.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The workspace is a file-scope device
 * array of G4_STATIC_WORKSPACE_BYTES, one per GPU, held until the process
 * ends; its address on the stream's GPU is looked up on the first call there.
 * Problems whose forward workspace (g4_workspace_bytes(p, 0): the vision span
 * tables, 40 bytes per K token with vision IDs, and the head-dim 512 pass
 * flags, 4 bytes per 32 queries per head) exceeds it are rejected with
 * G4_ERR_WORKSPACE.  Every call on a GPU uses the same array: calls that
 * overlap on one GPU (other streams, other threads) race; calls on one stream
 * are ordered and safe.  Allocates nothing, no host synchronisation.
 * Under HIP graph capture: make one call on that GPU outside capture first
 * (it looks up the array's address and sets the kernels' launch attributes);
 * later calls record launches only.
 * Cost: the array is part of the library's code object, so every process
 * that loads the library holds 32 MiB of HBM on each GPU where its kernels
 * are loaded, whether or not it calls this entry point.
 */
#define G4_STATIC_WORKSPACE_BYTES (32u << 20)
int g4_attn_fwd_static(const g4_problem* p,
                       const void* q, g4_layout q_layout,
                       const void* k, g4_layout k_layout,
                       const void* v, g4_layout v_layout,
                       void* o, g4_layout o_layout,
                       float* lse,
                       void* stream);

/*
 * Backward: dQ, dK, dV given O, dO, LSE and optional dLSE (same layout as LSE,
 * NULL = zero).  dK and dV are distinct outputs; no atomics (bitwise
 * repeatable).  Runs g4_attn_bwd_delta, g4_attn_bwd_dkdv and g4_attn_bwd_dq.
 * Striped routes, for head-dim 512 causal problems whose dense dS tiles
 * exceed ds_budget; the dK/dV and dQ launches alternate per stripe, so
 * nothing is recomputed:
 *   - one sequence: stripes of 32-query rows, each stripe's tiles fitting the
 *     budget beside fp32 dK / dV sums (2 x K tokens x KV heads x 512 x 4
 *     bytes, counted in the budget and in g4_workspace_bytes).  dQ is bitwise
 *     that of the dense stored route; dK and dV differ from it by the fp32
 *     additions between stripes.
 *   - several sequences: stripes of whole sequences (those whose first dS row
 *     falls in the stripe), when the budget holds at least two longest
 *     sequences' rows of tiles.  dQ, dK and dV are bitwise those of the dense
 *     stored route.
 * (The three stage entry points on such a problem take the recompute route
 * instead.)
 * Replaces FA4's autograd backward (local) and the patched global d512
 * orchestrator _flash_attn_bwd_gemma4_global_d512
 * (patches/flash-attention/0002-*.patch:1021-1512, called from
 * src/gemma4_fa4/h100.py:1300-1317, 1389-1394).
 */
int g4_attn_bwd(const g4_problem* p,
                const void* q, g4_layout q_layout,
                const void* k, g4_layout k_layout,
                const void* v, g4_layout v_layout,
                const void* o, g4_layout o_layout,
                const void* dout, g4_layout do_layout,
                const float* lse, const float* dlse,
                void* dq, g4_layout dq_layout,
                void* dk, g4_layout dk_layout,
                void* dv, g4_layout dv_layout,
                void* workspace, size_t workspace_bytes,
                void* stream);

/* Stage 1 of the backward: delta[h, t] = rowsum(O * dO) - dLSE into the
 * workspace.  Replaces FA4 _bwd_preprocess (patch 0002:1255-1272). */
int g4_attn_bwd_delta(const g4_problem* p,
                      const void* o, g4_layout o_layout,
                      const void* dout, g4_layout do_layout,
                      const float* dlse,
                      void* workspace, size_t workspace_bytes,
                      void* stream);

/* Stage 2: dK, dV (KV-tile major, reduces the GQA group on chip).  Needs the
 * workspace left by g4_attn_bwd_delta; it also stores dS tiles there for
 * g4_attn_bwd_dq (head dim 512 causal text problems, and head dim 256 with a
 * window).  Replaces the dKV-only FA4 launches (patch 0002:1347-1418) and
 * FA4's fused local backward dK/dV. */
int g4_attn_bwd_dkdv(const g4_problem* p,
                     const void* q, g4_layout q_layout,
                     const void* k, g4_layout k_layout,
                     const void* v, g4_layout v_layout,
                     const void* dout, g4_layout do_layout,
                     const float* lse,
                     void* dk, g4_layout dk_layout,
                     void* dv, g4_layout dv_layout,
                     void* workspace, size_t workspace_bytes,
                     void* stream);

/* Stage 3: dQ (Q-tile major).  Needs the workspace left by
 * g4_attn_bwd_delta and, where g4_attn_bwd_dkdv stored dS tiles there, by
 * that stage (dQ is then one product over them).  Replaces the D256-stream
 * dQ-only FA4 launches (patch 0002:1367-1381, 1430-1449). */
int g4_attn_bwd_dq(const g4_problem* p,
                   const void* q, g4_layout q_layout,
                   const void* k, g4_layout k_layout,
                   const void* v, g4_layout v_layout,
                   const void* dout, g4_layout do_layout,
                   const float* lse,
                   void* dq, g4_layout dq_layout,
                   void* workspace, size_t workspace_bytes,
                   void* stream);

/*
 * Materialise the device mask predicate the kernels evaluate, as bytes
 * (1 = allowed): out[s][i][j] for i < seqlen_q, j < seqlen_k (row-major,
 * num_seqs * seqlen_q * seqlen_k bytes).  Entries past a packed sequence's
 * lengths are 0.  For bit-exact checks of the mask contract of
 * src/gemma4_fa4/masks.py:8-80 / h100_masks.py:26-152.
 */
int g4_mask_materialize(const g4_problem* p, uint8_t* out,
                        void* workspace, size_t workspace_bytes, void* stream);

/*
 * Export the device tile scheduler's ranges.  direction 0: for each
 * (seq, tile of row_tile queries) the half-open range [k_lo, k_hi) of key
 * indices the forward and dQ kernels visit; direction 1: for each
 * (seq, tile of row_tile keys) the range [i_lo, i_hi) of query indices the
 * dK/dV kernel visits: every query whose key range reaches the tile, so it
 * can be wider than the tile's allowed pairs when a vision ID repeats with a
 * gap (the dQ kernel reads the stored dS of all those tiles).  Indices are
 * sequence-local.  Writes int32 pairs for
 * num_seqs * ceil(max_len / row_tile) rows (empty rows give lo == hi).
 * Replaces the host schedule build_gemma4_local_sparse_schedule
 * (src/gemma4_fa4/sparse_schedule.py:291-374) and its D2H/H2D copies
 * (src/gemma4_fa4/h100.py:490-601, 388-422).
 */
int g4_tile_ranges(const g4_problem* p, int direction, int row_tile, int32_t* out,
                   void* workspace, size_t workspace_bytes, void* stream);

/*
 * K/V preparation from a projection source (the reference's
 * prepare_global_kv_from_projection_source, src/gemma4_fa4/reference.py:306-328,
 * with rms_norm 276-281 and partial RoPE 284-303; design note
 * docs/design.md:202-213; the same RMSNorm and RoPE order as the compiled
 * layer ops' _rms_norm / _apply_rotary, src/gemma4_fa4/h100_torch_ops.py:302-326).
 * Per (batch, token, head) row z of head_dim elements:
 *   r = (mean(z^2) + eps)^(-1/2), n = z r               (fp32)
 *   V = bf16(n)                                          (RMSNorm, no weight)
 *   kn = bf16(n w); K = kn with RoPE on its first rotary_dim dims
 *        (K_i = kn_i cos_i + rot(kn)_i sin_i, rot(x) = (-x2, x1) over the
 *        rotary dims), other dims unchanged.
 * K is written as fp32 with k_fp32 = 1 (the dtype the reference returns for a
 * bf16 source and fp32 cos / sin: fp32 products and sum), or as bf16 with
 * k_fp32 = 0 (bf16 source and tables: each product and the sum rounded to
 * bf16, as bf16 tensor operations do).  Z, K, V, dZ use g4_layout element
 * strides (K's in its own dtype); rows are (batch, token, head).  cos / sin
 * are fp32 (batch, seqlen, rotary_dim), rows contiguous, batch stride
 * cs_batch_stride elements (0: shared by every batch); the weight is fp32 of
 * head_dim.  head_dim 512 or 256 (forward; the backward covers 512);
 * rotary_dim a multiple of 16 up to head_dim.
 */
typedef struct g4_kv_prep {
  int32_t num_batches;
  int32_t seqlen;
  int32_t num_heads;
  int32_t head_dim;
  int32_t rotary_dim;
  int32_t k_fp32;
  float eps;
  int64_t cs_batch_stride;
} g4_kv_prep;

/* Forward: K, V from the source; either output may be NULL (not written:
 * queries are prepared as K alone, a separate value projection as V alone).
 * Stream-ordered, no workspace. */
int g4_kv_prep_fwd(const g4_kv_prep* p,
                   const void* z, g4_layout z_layout,
                   const float* weight, const float* cos, const float* sin,
                   void* k, g4_layout k_layout,
                   void* v, g4_layout v_layout,
                   void* stream);

/* Workspace bytes of g4_kv_prep_bwd (per-workgroup partial sums of dweight). */
size_t g4_kv_prep_workspace_bytes(const g4_kv_prep* p);

/* Backward: dZ (bf16) and dweight (fp32, head_dim, overwritten) from dK (in
 * K's dtype) and dV (bf16) through both preparation adjoints; no atomics,
 * bitwise repeatable. */
int g4_kv_prep_bwd(const g4_kv_prep* p,
                   const void* z, g4_layout z_layout,
                   const float* weight, const float* cos, const float* sin,
                   const void* dk, g4_layout dk_layout,
                   const void* dv, g4_layout dv_layout,
                   void* dz, g4_layout dz_layout,
                   float* dweight,
                   void* workspace, size_t workspace_bytes,
                   void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GEMMA4_ATTN_H */
