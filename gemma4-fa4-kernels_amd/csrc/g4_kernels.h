// Kernel parameter blocks and launchers shared by the C ABI layer.
#pragma once

#include <atomic>

#include "g4_common.h"

namespace g4 {

struct FwdParams {
  g4_problem p;
  const __bf16* q;
  const __bf16* k;
  const __bf16* v;
  __bf16* o;
  float* lse;
  g4_layout ql, kl, vl, ol;
  const int* span_lo;  // per K-stream token: first query position reaching it (see g4_meta.hip)
  const int* span_hi;  // per K-stream token: last position of its vision span (or itself)
  int num_seqs;
  int ntq;             // query tiles per sequence (set by the launcher)
  int* raise_flags;    // per (seq, 32-query group, head): rows the fast pass cannot finish
  // Split of a problem with document IDs over two launches (set by the
  // launcher): 0 every workgroup; 1 only workgroups whose queries and visited
  // keys share one document (their document test is dropped); 2 the others.
  int doc_pass;
  // The work items pass 1 leaves to pass 2 (appended by pass 1, in any order;
  // doc_list_n counts them), so pass 2 runs those alone instead of testing
  // every query tile again.  Null: pass 2 tests every tile.
  int* doc_list;
  unsigned* doc_list_n;
  // Packed, 2..64 sequences (set by the launcher): the grid enumerates only
  // the query tiles that exist, sequence by sequence (at most
  // total_q / kBM + num_seqs per head), instead of num_seqs x ntq.
  int compact;
  // Full grid whose XCD runs hold whole rank pairs (set by the launcher):
  // blocks map onto items heaviest first within each XCD (xcd_remap_desc).
  int desc_order;
  // Split-key forward for few queries per KV head (decode; see split_chunks):
  // split_chunks chunks of split_keys keys per (sequence, KV head), whose
  // partial rows (unnormalised O, running maximum and sum) go to `part`
  // before a merge launch.  0: the regular forward.
  int split_chunks, split_keys;
  float* part;
};

// Query (0..31, within its 32-query row) at position p of a dS tile's key row:
// accumulator value r of lane half h sits at p = 16 h + r and holds query
// 8 (r >> 2) + 4 h + (r & 3).
__host__ __device__ inline int ds_query_at(int p) {
  return 8 * ((p & 15) >> 2) + 4 * (p >> 4) + (p & 3);
}

struct BwdParams {
  g4_problem p;
  const __bf16* q;
  const __bf16* k;
  const __bf16* v;
  const __bf16* o;
  const __bf16* dout;
  const float* lse;
  const float* dlse;
  __bf16* dq;
  __bf16* dk;
  __bf16* dv;
  g4_layout ql, kl, vl, ol, dol, dql, dkl, dvl;
  float* delta;        // (Hq, total_q) fp32 workspace, token-contiguous per head
  const int* span_lo;
  const int* span_hi;
  int num_seqs;
  int ntiles;          // row tiles per sequence (set by the launchers)
  // dS tiles written by the dK/dV kernel for the dQ stage (null when not used).
  // Row r of packed sequence s, query tile t is floor(cu_q[s] / 32) + s + t
  // (fixed layouts: s * ceil(Sq / 32) + t).  Head dim 512: tile (query head h,
  // key tile c, row r) at ((h * ds_cols + c) * ds_rows + r) * 4 KB.  Head dim
  // 256 (band): tile (h, r, key tile c) at ((h * ds_rows + r) * ds_cols +
  // c - ds_band_first(r)) * 4 KB for c - ds_band_first(r) < ds_cols.  Each tile
  // is [64 keys][32 positions] bf16: position p holds query p of the row in the
  // dense layout and query ds_query_at(p) in the band (the MFMA accumulator
  // order, so each lane stores one 32-byte run).
  __bf16* ds;
  int ds_rows, ds_cols;
  // Striped stored-dS backward (head dim 512, dense dS past the budget; see
  // DsStripe).  Row stripes (one sequence, dk_acc set): the buffer holds the
  // sequence's rows [ds_row_lo, ds_row_lo + ds_rows), and the dQ launch takes
  // the stripe's 128-query tiles from dq_qt_lo.  Sequence stripes
  // (ds_seq_rows > 0): the launch handles only the sequences whose first row
  // lies in [ds_row_lo, ds_row_lo + ds_seq_rows), whole, and the buffer holds
  // rows from ds_row_lo.  All 0 otherwise.
  int ds_row_lo, dq_qt_lo, ds_seq_rows;
  // fp32 dK / dV sums over the stripes ((Tk, Hkv, D), null unless striped) and
  // what the dK/dV launch's epilogue does with them: bit 0 adds the stored
  // sums (every stripe after the first), bit 1 writes the bf16 dK / dV (the
  // last stripe), else the fp32 sums are written.
  float* dk_acc;
  float* dv_acc;
  int acc_mode;
  // Head dim 256 dQ after the stored-dS pass: only the query tiles whose vision
  // spans reach past the stored band (set by the launcher).
  int dq_recompute_only;
  // Work-queue ticket counters of the persistent tile kernels: [0] dK/dV,
  // [2] dQ; zeroed by the delta pass, and by each launch's last draw.  [3]
  // counts the entries of dq_list.
  unsigned* sched;
  // Head dim 256 with vision IDs: the query tiles the stored-dS dQ pass left
  // for recomputation, appended by that pass ({sequence, query tile, query
  // head, 0}; order not significant: each entry writes its own dQ rows).
  int4* dq_list;
};

// Workspace layout helpers (bytes).
size_t spans_bytes(const g4_problem& p);
size_t delta_bytes(const g4_problem& p);
size_t raise_flags_bytes(const g4_problem& p);
size_t fwd_doc_list_bytes(const g4_problem& p);  // counter (256 B) + entries
constexpr size_t kSchedBytes = 256;  // work-queue counters (backward workspace tail)
// Counter words: [0] dK/dV queue, [2] dQ queue (stored dS at head dim 512,
// recompute), [3] dQ recompute list length, [kDqXcdQueue, +9) the XcdQueue of
// the head-dim 256 stored-dS dQ kernel; words [0, kSchedClear) are zeroed by
// the delta pass of every backward.
constexpr int kDqXcdQueue = 16;
constexpr int kSchedClear = 32;
static_assert(kSchedClear * 4 <= (int)kSchedBytes, "counters fit");
size_t dq_list_bytes(const g4_problem& p);  // after the counters

// Function attributes and occupancy are per device, and one process may drive
// several GPUs: launch-time state is cached per device (the current device,
// which the caller keeps equal to the stream's device, as for any HIP launch).
constexpr int kMaxDevices = 64;

__host__ inline int current_device() {
  int dev = 0;
  return hipGetDevice(&dev) == hipSuccess ? dev : -1;
}

// Dynamic-LDS limit of one kernel, raised once per device.
struct LdsAttr {
  std::atomic<int> set[kMaxDevices] = {};
  hipError_t ensure(const void* kern, int bytes) {
    const int dev = current_device();
    const bool cached = dev >= 0 && dev < kMaxDevices;
    if (cached && set[dev].load(std::memory_order_acquire)) return hipSuccess;
    const hipError_t e =
        hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e == hipSuccess && cached) set[dev].store(1, std::memory_order_release);
    return e;
  }
};

// Launch shape of a tile kernel with a work-queue variant: with more than
// kQueueMin items per resident workgroup (CUs x workgroups per CU from the
// occupancy query of the queue variant) the queue variant on as many
// workgroups as are resident at once; otherwise the plain variant, one
// workgroup per item (with few items per CU the queue's draws and the lost
// XCD locality of later tickets cost more than the balance gains: measured on
// configs 1 and 3).
struct PersistentGrid {
  static constexpr int kQueueMin = 4;
  std::atomic<int> resident[kMaxDevices] = {};  // per device; 0 until queried
  // Workgroups of the launch; *queue says which variant.
  int64_t size(const void* queue_kern, int threads, int lds, int64_t items, bool* queue) {
    const int dev = current_device();
    if (dev < 0) return 0;
    const bool cached = dev < kMaxDevices;
    int n = cached ? resident[dev].load(std::memory_order_relaxed) : 0;
    if (n == 0) {
      int cus = 0, per_cu = 0;
      if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
          hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, queue_kern, threads, lds) !=
              hipSuccess)
        return 0;
      n = cus * (per_cu > 1 ? per_cu : 1);
      if (cached) resident[dev].store(n, std::memory_order_relaxed);
    }
    *queue = items > (int64_t)kQueueMin * n;
    return *queue ? n : items;
  }
};
// dS buffer of the head-dim 512 causal backward (0: the dQ stage recomputes S, dP).
size_t ds_bytes(const g4_problem& p);
void ds_geometry(const g4_problem& p, int* rows, int* cols);
// A stripe of the striped stored-dS backward, buffer geometry rows x cols.
// Row stripe (seq_rows = 0, one sequence): its 32-query rows [row_lo, row_lo +
// rows) (a multiple of 4, so stripes hold whole 128-query dQ tiles) and the
// key tiles they reach (cols).  Sequence stripe (seq_rows > 0, several
// sequences): the sequences whose first row lies in [row_lo, row_lo +
// seq_rows), whose rows all fit in the buffer's rows from row_lo.
struct DsStripe {
  int row_lo, rows, cols, seq_rows;
};
// Stripes of a causal head-dim 512 problem whose dense dS exceeds its budget:
// row stripes of one sequence, sequence stripes of several; writes up to
// max_out of them and returns how many there are (0: not striped).
int ds_stripes(const g4_problem& p, DsStripe* out, int max_out);
// fp32 dK / dV sums of the row-striped backward (0 otherwise).
size_t acc_bytes(const g4_problem& p);
// Split-key forward: the number of key chunks per (sequence, KV head), 0 when
// the problem takes the regular forward; *keys receives the keys per chunk.
int split_chunks(const g4_problem& p, int* keys);
// Workspace bytes of its partial rows (0 when not split).
size_t split_bytes(const g4_problem& p);
int64_t k_stream_tokens(const g4_problem& p);
int64_t q_stream_tokens(const g4_problem& p);

// query_reach: span_lo as the first query reaching each key (backward, tile
// scheduler); without it span_lo keeps each key's own span start (the forward
// reads only span_hi).
hipError_t launch_spans(const g4_problem& p, void* ws, hipStream_t stream, bool query_reach = true);
void span_arrays(const g4_problem& p, void* ws, const int** lo, const int** hi);
hipError_t launch_fwd(const FwdParams& a, hipStream_t stream);
hipError_t launch_bwd_delta(const BwdParams& a, hipStream_t stream);
hipError_t launch_bwd_dkdv(const BwdParams& a, hipStream_t stream);
hipError_t launch_bwd_dq(const BwdParams& a, hipStream_t stream);
hipError_t launch_mask(const g4_problem& p, uint8_t* out, const int* span_lo, const int* span_hi,
                       hipStream_t stream);
hipError_t launch_ranges(const g4_problem& p, int direction, int row_tile, int32_t* out,
                         const int* span_lo, const int* span_hi, hipStream_t stream);

// K/V preparation from the shared projection source (g4_kvprep.hip).
size_t kv_prep_workspace_bytes(const g4_kv_prep& p);
hipError_t launch_kv_prep_fwd(const g4_kv_prep& p, const void* z, g4_layout zl, const float* w,
                              const float* cosv, const float* sinv, void* k, g4_layout kl,
                              void* v, g4_layout vl, hipStream_t stream);
hipError_t launch_kv_prep_bwd(const g4_kv_prep& p, const void* z, g4_layout zl, const float* w,
                              const float* cosv, const float* sinv, const void* dk,
                              g4_layout dkl, const void* dv, g4_layout dvl, void* dz,
                              g4_layout dzl, float* dw, void* ws, hipStream_t stream);

}  // namespace g4
