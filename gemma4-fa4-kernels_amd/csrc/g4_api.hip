// C ABI entry points: argument validation, workspace carving, launches.
// Every entry point is stream-ordered and allocates nothing.
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <string>

#include <algorithm>

#include "g4_kernels.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, const char* detail = "") {
  char buf[512];
  snprintf(buf, sizeof buf, fmt, detail);
  g_last_error = buf;
  return code;
}

int hip_fail(hipError_t e, const char* where) {
  char buf[512];
  snprintf(buf, sizeof buf, "%s: HIP error %d (%s)", where, (int)e, hipGetErrorString(e));
  g_last_error = buf;
  return G4_ERR_LAUNCH;
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

int check_problem(const g4_problem* p) {
  if (p == nullptr) return fail(G4_ERR_INVALID, "problem descriptor is NULL");
  if (p->num_seqs < 1) return fail(G4_ERR_INVALID, "num_seqs must be >= 1");
  if (p->num_q_heads < 1 || p->num_kv_heads < 1 || p->num_q_heads % p->num_kv_heads)
    return fail(G4_ERR_INVALID, "num_q_heads must be a positive multiple of num_kv_heads");
  {
    const int grp = p->num_q_heads / p->num_kv_heads;
    if (grp != 1 && grp != 2 && grp != 4 && grp != 8)
      return fail(G4_ERR_UNSUPPORTED, "GQA ratio (num_q_heads / num_kv_heads) must be 1, 2, 4 or 8");
  }
  if (p->head_dim != 256 && p->head_dim != 512)
    return fail(G4_ERR_UNSUPPORTED, "head_dim must be 256 (local) or 512 (global)");
  if (p->window < 0) return fail(G4_ERR_INVALID, "window must be >= 0");
  if (p->seqlen_q < 1 || p->seqlen_k < 1)
    return fail(G4_ERR_INVALID, "seqlen_q and seqlen_k must be >= 1");
  if ((p->cu_seqlens_q == nullptr) != (p->cu_seqlens_k == nullptr))
    return fail(G4_ERR_INVALID, "cu_seqlens_q and cu_seqlens_k must both be set or both NULL");
  if (p->cu_seqlens_q == nullptr) {
    if (p->seqlen_q > p->seqlen_k)
      return fail(G4_ERR_INVALID, "fixed layout requires seqlen_q <= seqlen_k");
  } else if (p->total_q < 1 || p->total_k < 1) {
    return fail(G4_ERR_INVALID, "packed totals must be positive");
  }
  if ((int64_t)p->num_seqs * p->seqlen_q > 0x7fffffffLL ||
      (int64_t)p->num_seqs * p->seqlen_k > 0x7fffffffLL)
    return fail(G4_ERR_UNSUPPORTED, "token counts must fit int32");
  return G4_OK;
}

int check_operand(const void* ptr, const g4_layout& l, const char* name) {
  if (ptr == nullptr) return fail(G4_ERR_INVALID, "operand %s is NULL", name);
  if (((uintptr_t)ptr) % 16) return fail(G4_ERR_INVALID, "operand %s must be 16-byte aligned", name);
  if (l.token_stride <= 0 || l.head_stride <= 0 || l.token_stride % 8 || l.head_stride % 8 ||
      l.batch_stride < 0 || l.batch_stride % 8)
    return fail(G4_ERR_INVALID, "operand %s strides must be positive multiples of 8 elements",
                name);
  // Tile copies form the in-tile part of their addresses as 32-bit offsets.
  if (l.token_stride >= (int64_t(1) << 24))
    return fail(G4_ERR_INVALID, "operand %s token stride must be below 2^24 elements", name);
  return G4_OK;
}

int check_ws(const g4_problem* p, int phase, void* ws, size_t bytes) {
  size_t need = g4_workspace_bytes(p, phase);
  if (bytes < need) {
    char buf[128];
    snprintf(buf, sizeof buf, "%zu bytes needed, %zu given", need, bytes);
    return fail(G4_ERR_WORKSPACE, "workspace too small: %s", buf);
  }
  if (need > 0 && ws == nullptr) return fail(G4_ERR_WORKSPACE, "workspace is NULL");
  if (((uintptr_t)ws) % 256) return fail(G4_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  return G4_OK;
}

#define G4_TRY(expr)            \
  do {                          \
    int _rc = (expr);           \
    if (_rc != G4_OK) return _rc; \
  } while (0)

// Workspace: [spans][raise flags][document-pass list][split partials] (forward); backward adds
// [delta][dS][queue counters][dQ recompute list][dK / dV sums (striped)]
size_t fwd_ws_bytes(const g4_problem& p) {
  return align256(g4::spans_bytes(p)) + g4::raise_flags_bytes(p) + g4::fwd_doc_list_bytes(p) +
         g4::split_bytes(p);
}
int* raise_flags_ptr(const g4_problem& p, void* ws) {
  return g4::raise_flags_bytes(p) ? (int*)((char*)ws + align256(g4::spans_bytes(p))) : nullptr;
}
unsigned* fwd_doc_list_ptr(const g4_problem& p, void* ws) {
  if (!g4::fwd_doc_list_bytes(p)) return nullptr;
  return (unsigned*)((char*)ws + align256(g4::spans_bytes(p)) + g4::raise_flags_bytes(p));
}
float* split_ptr(const g4_problem& p, void* ws) {
  if (!g4::split_bytes(p)) return nullptr;
  return (float*)((char*)ws + align256(g4::spans_bytes(p)) + g4::raise_flags_bytes(p) +
                  g4::fwd_doc_list_bytes(p));
}
float* delta_ptr(const g4_problem& p, void* ws) {
  return (float*)((char*)ws + fwd_ws_bytes(p));
}
__bf16* ds_ptr(const g4_problem& p, void* ws) {
  if (!g4::ds_bytes(p)) return nullptr;
  return (__bf16*)((char*)ws + fwd_ws_bytes(p) + g4::delta_bytes(p));
}
unsigned* sched_ptr(const g4_problem& p, void* ws) {
  return (unsigned*)((char*)ws + fwd_ws_bytes(p) + g4::delta_bytes(p) + g4::ds_bytes(p));
}
int4* dq_list_ptr(const g4_problem& p, void* ws) {
  if (!g4::dq_list_bytes(p)) return nullptr;
  return (int4*)((char*)sched_ptr(p, ws) + g4::kSchedBytes);
}
float* acc_ptr(const g4_problem& p, void* ws) {
  if (!g4::acc_bytes(p)) return nullptr;
  return (float*)((char*)sched_ptr(p, ws) + g4::kSchedBytes + g4::dq_list_bytes(p));
}

// Forward workspace of g4_attn_fwd_static: a file-scope device array, one
// copy per GPU, held until the process ends.  Host code never passes the
// array's name to a kernel (on the host it is only a stand-in for the symbol);
// it uses the per-device address hipGetSymbolAddress returns.
constexpr size_t kStaticWorkspaceBytes = size_t(32) << 20;
static_assert(kStaticWorkspaceBytes == G4_STATIC_WORKSPACE_BYTES, "header and library agree");
__device__ __align__(256) unsigned char scratch[kStaticWorkspaceBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` on each GPU, once looked up

// Address of `scratch` on the device `stream` belongs to (looked up once per
// device, with that device current).
int scratch_for_stream(hipStream_t stream, void** out) {
  int dev = 0;
  hipError_t e = hipStreamGetDevice(stream, &dev);
  if (e != hipSuccess) return hip_fail(e, "hipStreamGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(G4_ERR_UNSUPPORTED, "device ordinal out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    int cur = 0;
    e = hipGetDevice(&cur);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return hip_fail(e, "hipSetDevice");
    void* ptr = nullptr;
    const hipError_t ge = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (cur != dev && (e = hipSetDevice(cur)) != hipSuccess) return hip_fail(e, "hipSetDevice");
    if (ge != hipSuccess) return hip_fail(ge, "hipGetSymbolAddress(scratch)");
    if (ptr == nullptr || ((uintptr_t)ptr) % 256)
      return fail(G4_ERR_LAUNCH, "static workspace address is not 256-byte aligned");
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return G4_OK;
}

int fwd_impl(const g4_problem* p, const void* q, g4_layout ql, const void* k, g4_layout kl,
             const void* v, g4_layout vl, void* o, g4_layout ol, float* lse, void* ws,
             hipStream_t st) {
  g4::FwdParams a{};
  a.p = *p;
  a.q = (const __bf16*)q;
  a.k = (const __bf16*)k;
  a.v = (const __bf16*)v;
  a.o = (__bf16*)o;
  a.lse = lse;
  a.ql = ql;
  a.kl = kl;
  a.vl = vl;
  a.ol = ol;
  a.num_seqs = p->num_seqs;
  if (g4::spans_bytes(*p)) {
    hipError_t e = g4::launch_spans(*p, ws, st, /*query_reach=*/false);  // (span_hi only)
    if (e != hipSuccess) return hip_fail(e, "span table");
  }
  g4::span_arrays(*p, ws, &a.span_lo, &a.span_hi);
  a.raise_flags = raise_flags_ptr(*p, ws);
  a.part = split_ptr(*p, ws);
  if (a.part != nullptr) a.split_chunks = g4::split_chunks(*p, &a.split_keys);
  if (unsigned* dl = fwd_doc_list_ptr(*p, ws)) {
    a.doc_list_n = dl;
    a.doc_list = (int*)(dl + 64);
  }
  hipError_t e = g4::launch_fwd(a, st);
  if (e != hipSuccess) return hip_fail(e, "forward");
  return G4_OK;
}

int check_fwd_operands(const g4_problem* p, const void* q, g4_layout ql, const void* k,
                       g4_layout kl, const void* v, g4_layout vl, const void* o, g4_layout ol,
                       const float* lse) {
  G4_TRY(check_problem(p));
  G4_TRY(check_operand(q, ql, "q"));
  G4_TRY(check_operand(k, kl, "k"));
  G4_TRY(check_operand(v, vl, "v"));
  G4_TRY(check_operand(o, ol, "o"));
  if (lse == nullptr) return fail(G4_ERR_INVALID, "lse is NULL");
  return G4_OK;
}

}  // namespace

namespace g4 {
size_t delta_bytes(const g4_problem& p) {
  return align256((size_t)q_stream_tokens(p) * p.num_q_heads * 4);
}
// dS tiles written by the dK/dV kernel (bf16, one 4 KB tile [64 keys][32
// queries] per (query head, 32-query row, 64-key tile)) so that the dQ stage
// is a plain product dQ^T = K^T dS^T instead of recomputing S and dP.
// - Head dim 512, text causal (no window, no bidirectional vision): dense over
//   rows x key tiles; every visited pair lies in the causal triangle.
// - Head dim 256 with a window: a band of ds_cols key tiles per row, starting
//   at the tile of the row's first query's window start: (W + 30) / 64 + 2
//   tiles cover every key the row's window and causal part admit, and with
//   bidirectional vision up to 18 more (1152 keys) hold keys of vision spans
//   that reach past the row's causal end, as far as the budget allows.
//   The dQ stage recomputes the query tiles whose spans reach past the band.
// Used while the buffer stays within the problem's ds_budget (0: 16 GiB,
// negative: no stored tiles); otherwise the dQ stage recomputes S and dP.
constexpr size_t kDsCap = size_t(16) << 30;
size_t ds_cap(const g4_problem& p) {
  if (p.ds_budget < 0) return 0;
  return p.ds_budget == 0 ? kDsCap : (size_t)p.ds_budget;
}
void ds_geometry(const g4_problem& p, int* rows, int* cols) {
  const int64_t r = p.cu_seqlens_q ? p.total_q / 32 + p.num_seqs
                                   : (int64_t)p.num_seqs * ((p.seqlen_q + 31) / 32);
  *rows = (int)r;
  if (p.head_dim == 256 && p.window > 0) {
    const int base = (p.window + 30) / 64 + 2;
    const bool vis = p.vision_ids != nullptr && p.bidirectional_vision;
    const int64_t per_col = r * p.num_q_heads * 4096;
    const int64_t fit = per_col > 0 ? (int64_t)(ds_cap(p) / (size_t)per_col) : base;
    *cols = (int)std::max<int64_t>(base, std::min<int64_t>(base + (vis ? 18 : 0), fit));
  } else {
    *cols = (p.seqlen_k + 63) / 64;
  }
}
static bool ds_dense_kind(const g4_problem& p) {
  return p.head_dim == 512 && p.window == 0 && !(p.vision_ids != nullptr && p.bidirectional_vision);
}
static size_t ds_full_bytes(const g4_problem& p) {
  int rows, cols;
  ds_geometry(p, &rows, &cols);
  return (size_t)rows * cols * p.num_q_heads * 4096;
}
// fp32 dK and dV sums of the striped backward, over the K stream's tokens.
static size_t sums_bytes(const g4_problem& p) {
  return align256((size_t)2 * k_stream_tokens(p) * p.num_kv_heads * p.head_dim * 4);
}
// Striped stored dS: when the dense buffer of one causal head-dim 512 sequence
// exceeds the budget, its 32-query rows are cut, from the first, into stripes
// whose tiles (rows x the key tiles their last row reaches) fit the budget
// less the fp32 dK / dV sums, each as many rows (a multiple of four) as fit.
// The dK/dV launch of a stripe stores its dS and adds its dK / dV to the sums;
// the dQ launch of the same stripe then reads those dS tiles.  Every (query,
// key) pair is visited once by each stage, so nothing is recomputed.  Calls
// f(stripe) in order; returns the number of stripes (0: not striped: the dense
// layout fits, or the problem is not a single such sequence, or not even four
// rows reaching every key tile fit).
// Several sequences (packed or fixed): sequence stripes instead.  Stripe k
// takes the sequences whose first row lies in [k H, (k + 1) H), whole: their
// rows fit H + (rows of the longest sequence) - 1 buffer rows of every key
// tile, with H as large as the budget allows and at least the longest
// sequence's rows (fewer would mean many nearly empty launches; such a budget
// leaves the recompute route).  Each sequence's dK / dV come from one stripe,
// so no sums are needed.
template <class F>
static int for_each_seq_stripe(const g4_problem& p, F f) {
  const size_t cap = ds_cap(p);
  if (cap == 0 || ds_full_bytes(p) <= cap) return 0;
  int total_rows, ncols;
  ds_geometry(p, &total_rows, &ncols);
  const int64_t maxrows = (p.seqlen_q + 31) / 32;
  const size_t per_row = (size_t)ncols * p.num_q_heads * 4096;
  const int64_t fit = (int64_t)(cap / per_row);  // buffer rows within the budget
  const int64_t h = fit - maxrows + 1;
  if (h < maxrows) return 0;
  int n = 0;
  for (int64_t r0 = 0; r0 < total_rows; r0 += h, ++n)
    f(DsStripe{(int)r0, (int)std::min<int64_t>(fit, total_rows - r0), ncols, (int)h});
  return n;
}
template <class F>
static int for_each_ds_stripe(const g4_problem& p, F f) {
  if (!ds_dense_kind(p)) return 0;
  if (p.num_seqs > 1) return for_each_seq_stripe(p, f);
  const size_t budget = ds_cap(p);
  if (budget == 0 || ds_full_bytes(p) <= budget || budget <= sums_bytes(p)) return 0;
  const size_t cap = budget - sums_bytes(p);
  const int64_t lq = p.seqlen_q, lk = p.seqlen_k;  // the one sequence's lengths
  const int nrows = (int)((lq + 31) / 32);
  const int ntk = (int)((lk + 63) / 64);
  const int64_t off = lk - lq;
  // key tiles the rows below r1 reach (their last query's causal end)
  auto cols = [&](int r1) {
    const int64_t last_q = std::min<int64_t>((int64_t)32 * r1, lq) - 1;
    return (int)std::min<int64_t>(ntk, (last_q + off) / 64 + 1);
  };
  const size_t per = (size_t)p.num_q_heads * 4096;  // bytes per (row, key tile)
  // Four rows that reach the last key tile must fit; then every stripe of
  // four rows (or the fewer left at the end) does, as cols only grows.  The
  // check comes before any f() call.
  if ((size_t)4 * cols(nrows) * per > cap) return 0;
  int n = 0;
  for (int r0 = 0; r0 < nrows;) {
    int h = std::min(4, nrows - r0);
    while (r0 + h < nrows) {
      const int h2 = std::min(h + 4, nrows - r0);
      if ((size_t)h2 * cols(r0 + h2) * per > cap) break;
      h = h2;
    }
    f(DsStripe{r0, h, cols(r0 + h), 0});
    ++n;
    r0 += h;
  }
  return n;
}
int ds_stripes(const g4_problem& p, DsStripe* out, int max_out) {
  int i = 0;
  return for_each_ds_stripe(p, [&](const DsStripe& s) {
    if (i < max_out) out[i] = s;
    ++i;
  });
}
size_t acc_bytes(const g4_problem& p) {
  return p.num_seqs == 1 && ds_stripes(p, nullptr, 0) ? sums_bytes(p) : 0;
}
size_t ds_bytes(const g4_problem& p) {
  const bool dense = ds_dense_kind(p);
  const bool band = p.head_dim == 256 && p.window > 0;
  if (!dense && !band) return 0;
  const size_t b = ds_full_bytes(p);
  if (b <= ds_cap(p)) return b;
  size_t most = 0;  // the largest stripe, when striped
  for_each_ds_stripe(p, [&](const DsStripe& s) {
    most = std::max(most, (size_t)s.rows * s.cols * p.num_q_heads * 4096);
  });
  return most;
}
// Head dim 256 stored-dS dQ with vision IDs: one 16-byte entry per possible
// (sequence, 128-query tile, query head) for the tiles left to recompute.
size_t dq_list_bytes(const g4_problem& p) {
  if (p.head_dim != 256 || !ds_bytes(p) || p.vision_ids == nullptr || !p.bidirectional_vision)
    return 0;
  return align256((size_t)p.num_seqs * ((p.seqlen_q + 127) / 128) * p.num_q_heads * 16);
}
// Head dim 256 with vision and document IDs: a counter and one int per
// (sequence, 128-query tile, query head) for the forward's second pass.
size_t fwd_doc_list_bytes(const g4_problem& p) {
  if (p.head_dim != 256 || p.vision_ids == nullptr || !p.bidirectional_vision ||
      p.document_ids == nullptr)
    return 0;
  return 256 + align256((size_t)p.num_seqs * ((p.seqlen_q + 127) / 128) * p.num_q_heads * 4);
}
// One int per (sequence, 32-query group, query head) for the head-dim 512
// forward's second pass.
size_t raise_flags_bytes(const g4_problem& p) {
  if (p.head_dim != 512) return 0;
  return align256((size_t)p.num_seqs * ((p.seqlen_q + 31) / 32) * p.num_q_heads * 4);
}
// Split-key forward: problems without key metadata whose query rows of one KV
// head (query heads of the group x queries) fit one 32-row tile, over at least
// 256 keys: one workgroup per (sequence, KV head, chunk of keys) instead of one
// per (query tile, query head), each walking every key (a decode step of one
// query then reads the K/V cache eight times over, in 32 workgroups).  About
// two rounds of resident workgroups in all (head dim 512: one per CU, 256:
// two), each chunk a whole number of 32-key tiles, at least four (head dim
// 512) or two.
int split_chunks(const g4_problem& p, int* keys) {
  if ((p.vision_ids != nullptr && p.bidirectional_vision) || p.document_ids != nullptr) return 0;
  const int64_t rows = (int64_t)(p.num_q_heads / p.num_kv_heads) * p.seqlen_q;
  if (rows > 32) return 0;
  const int64_t range = p.window > 0 ? std::min<int64_t>(p.seqlen_k, (int64_t)p.window + p.seqlen_q)
                                     : p.seqlen_k;
  if (range < 256) return 0;
  const int64_t target = p.head_dim == 512 ? 512 : 1024;
  const int64_t min_tiles = p.head_dim == 512 ? 4 : 2;
  const int64_t groups = (int64_t)p.num_seqs * p.num_kv_heads;
  const int64_t tiles = (range + 31) / 32 + 1;  // (the range may start mid-tile)
  int64_t n = std::max<int64_t>(1, std::min((target + groups - 1) / groups, tiles / min_tiles));
  const int64_t per = (tiles + n - 1) / n;  // tiles per chunk
  n = (tiles + per - 1) / per;
  if (keys != nullptr) *keys = (int)(per * 32);
  return (int)n;
}
size_t split_bytes(const g4_problem& p) {
  const int n = split_chunks(p, nullptr);
  if (n == 0) return 0;
  const size_t rows = (size_t)(p.num_q_heads / p.num_kv_heads) * p.seqlen_q;
  return align256((size_t)p.num_seqs * p.num_kv_heads * n * rows * (p.head_dim + 2) * 4);
}
}  // namespace g4

extern "C" {

int g4_abi_version(void) { return G4_ABI_VERSION; }

const char* g4_last_error(void) { return g_last_error.c_str(); }

size_t g4_workspace_bytes(const g4_problem* p, int phase) {
  g_last_error.clear();
  if (check_problem(p) != G4_OK) return 0;
  size_t b = fwd_ws_bytes(*p);
  if (phase == 1)
    b += g4::delta_bytes(*p) + g4::ds_bytes(*p) + g4::kSchedBytes + g4::dq_list_bytes(*p) +
         g4::acc_bytes(*p);
  return b;
}

int g4_attn_fwd(const g4_problem* p, const void* q, g4_layout ql, const void* k, g4_layout kl,
                const void* v, g4_layout vl, void* o, g4_layout ol, float* lse, void* ws,
                size_t ws_bytes, void* stream) {
  g_last_error.clear();
  G4_TRY(check_fwd_operands(p, q, ql, k, kl, v, vl, o, ol, lse));
  G4_TRY(check_ws(p, 0, ws, ws_bytes));
  return fwd_impl(p, q, ql, k, kl, v, vl, o, ol, lse, ws, (hipStream_t)stream);
}

int g4_attn_fwd_static(const g4_problem* p, const void* q, g4_layout ql, const void* k,
                       g4_layout kl, const void* v, g4_layout vl, void* o, g4_layout ol,
                       float* lse, void* stream) {
  g_last_error.clear();
  G4_TRY(check_fwd_operands(p, q, ql, k, kl, v, vl, o, ol, lse));
  const size_t need = g4_workspace_bytes(p, 0);
  if (need > kStaticWorkspaceBytes) {
    char buf[160];
    snprintf(buf, sizeof buf, "%zu bytes needed, %zu available", need, kStaticWorkspaceBytes);
    return fail(G4_ERR_WORKSPACE, "problem exceeds the static forward workspace: %s", buf);
  }
  void* ws = nullptr;
  G4_TRY(scratch_for_stream((hipStream_t)stream, &ws));
  return fwd_impl(p, q, ql, k, kl, v, vl, o, ol, lse, ws, (hipStream_t)stream);
}

static int fill_bwd(g4::BwdParams& a, const g4_problem* p, const void* q, g4_layout ql,
                    const void* k, g4_layout kl, const void* v, g4_layout vl, void* ws) {
  a.p = *p;
  a.q = (const __bf16*)q;
  a.k = (const __bf16*)k;
  a.v = (const __bf16*)v;
  a.ql = ql;
  a.kl = kl;
  a.vl = vl;
  a.num_seqs = p->num_seqs;
  a.delta = delta_ptr(*p, ws);
  // A striped problem's dS buffer holds one stripe at a time, which only
  // g4_attn_bwd interleaves with the dQ launches; the separate stage entry
  // points run it without stored dS (the dQ stage recomputes S and dP).
  a.ds = g4::ds_stripes(*p, nullptr, 0) ? nullptr : ds_ptr(*p, ws);
  g4::ds_geometry(*p, &a.ds_rows, &a.ds_cols);
  a.sched = sched_ptr(*p, ws);
  a.dq_list = dq_list_ptr(*p, ws);
  g4::span_arrays(*p, ws, &a.span_lo, &a.span_hi);
  return G4_OK;
}

int g4_attn_bwd_delta(const g4_problem* p, const void* o, g4_layout ol, const void* dout,
                      g4_layout dol, const float* dlse, void* ws, size_t ws_bytes, void* stream) {
  g_last_error.clear();
  G4_TRY(check_problem(p));
  G4_TRY(check_operand(o, ol, "o"));
  G4_TRY(check_operand(dout, dol, "dout"));
  G4_TRY(check_ws(p, 1, ws, ws_bytes));
  g4::BwdParams a{};
  a.p = *p;
  a.o = (const __bf16*)o;
  a.dout = (const __bf16*)dout;
  a.ol = ol;
  a.dol = dol;
  a.dlse = dlse;
  a.num_seqs = p->num_seqs;
  a.sched = sched_ptr(*p, ws);
  a.delta = delta_ptr(*p, ws);
  hipStream_t st = (hipStream_t)stream;
  if (g4::spans_bytes(*p)) {
    hipError_t e = g4::launch_spans(*p, ws, st);
    if (e != hipSuccess) return hip_fail(e, "span table");
  }
  hipError_t e = g4::launch_bwd_delta(a, st);
  if (e != hipSuccess) return hip_fail(e, "backward delta");
  return G4_OK;
}

int g4_attn_bwd_dkdv(const g4_problem* p, const void* q, g4_layout ql, const void* k,
                     g4_layout kl, const void* v, g4_layout vl, const void* dout, g4_layout dol,
                     const float* lse, void* dk, g4_layout dkl, void* dv, g4_layout dvl, void* ws,
                     size_t ws_bytes, void* stream) {
  g_last_error.clear();
  G4_TRY(check_problem(p));
  G4_TRY(check_operand(q, ql, "q"));
  G4_TRY(check_operand(k, kl, "k"));
  G4_TRY(check_operand(v, vl, "v"));
  G4_TRY(check_operand(dout, dol, "dout"));
  G4_TRY(check_operand(dk, dkl, "dk"));
  G4_TRY(check_operand(dv, dvl, "dv"));
  if (lse == nullptr) return fail(G4_ERR_INVALID, "lse is NULL");
  G4_TRY(check_ws(p, 1, ws, ws_bytes));
  g4::BwdParams a{};
  fill_bwd(a, p, q, ql, k, kl, v, vl, ws);
  a.dout = (const __bf16*)dout;
  a.dol = dol;
  a.lse = lse;
  a.dk = (__bf16*)dk;
  a.dv = (__bf16*)dv;
  a.dkl = dkl;
  a.dvl = dvl;
  hipError_t e = g4::launch_bwd_dkdv(a, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "backward dK/dV");
  return G4_OK;
}

int g4_attn_bwd_dq(const g4_problem* p, const void* q, g4_layout ql, const void* k, g4_layout kl,
                   const void* v, g4_layout vl, const void* dout, g4_layout dol, const float* lse,
                   void* dq, g4_layout dql, void* ws, size_t ws_bytes, void* stream) {
  g_last_error.clear();
  G4_TRY(check_problem(p));
  G4_TRY(check_operand(q, ql, "q"));
  G4_TRY(check_operand(k, kl, "k"));
  G4_TRY(check_operand(v, vl, "v"));
  G4_TRY(check_operand(dout, dol, "dout"));
  G4_TRY(check_operand(dq, dql, "dq"));
  if (lse == nullptr) return fail(G4_ERR_INVALID, "lse is NULL");
  G4_TRY(check_ws(p, 1, ws, ws_bytes));
  g4::BwdParams a{};
  fill_bwd(a, p, q, ql, k, kl, v, vl, ws);
  a.dout = (const __bf16*)dout;
  a.dol = dol;
  a.lse = lse;
  a.dq = (__bf16*)dq;
  a.dql = dql;
  hipError_t e = g4::launch_bwd_dq(a, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "backward dQ");
  return G4_OK;
}

int g4_attn_bwd(const g4_problem* p, const void* q, g4_layout ql, const void* k, g4_layout kl,
                const void* v, g4_layout vl, const void* o, g4_layout ol, const void* dout,
                g4_layout dol, const float* lse, const float* dlse, void* dq, g4_layout dql,
                void* dk, g4_layout dkl, void* dv, g4_layout dvl, void* ws, size_t ws_bytes,
                void* stream) {
  G4_TRY(g4_attn_bwd_delta(p, o, ol, dout, dol, dlse, ws, ws_bytes, stream));
  const int nstripes = g4::ds_stripes(*p, nullptr, 0);
  if (nstripes == 0) {
    G4_TRY(g4_attn_bwd_dkdv(p, q, ql, k, kl, v, vl, dout, dol, lse, dk, dkl, dv, dvl, ws,
                            ws_bytes, stream));
    G4_TRY(g4_attn_bwd_dq(p, q, ql, k, kl, v, vl, dout, dol, lse, dq, dql, ws, ws_bytes, stream));
    return G4_OK;
  }
  // Striped stored dS (g4::for_each_ds_stripe): per stripe, the dK/dV launch
  // (which stores the stripe's dS; row stripes add to the fp32 dK / dV sums)
  // then the dQ launch that reads them, all on the one stream.
  G4_TRY(check_operand(q, ql, "q"));
  G4_TRY(check_operand(k, kl, "k"));
  G4_TRY(check_operand(v, vl, "v"));
  G4_TRY(check_operand(dout, dol, "dout"));
  G4_TRY(check_operand(dq, dql, "dq"));
  G4_TRY(check_operand(dk, dkl, "dk"));
  G4_TRY(check_operand(dv, dvl, "dv"));
  if (lse == nullptr) return fail(G4_ERR_INVALID, "lse is NULL");
  g4::BwdParams a{};
  fill_bwd(a, p, q, ql, k, kl, v, vl, ws);
  a.ds = ds_ptr(*p, ws);
  a.dout = (const __bf16*)dout;
  a.dol = dol;
  a.lse = lse;
  a.dq = (__bf16*)dq;
  a.dql = dql;
  a.dk = (__bf16*)dk;
  a.dv = (__bf16*)dv;
  a.dkl = dkl;
  a.dvl = dvl;
  a.dk_acc = acc_ptr(*p, ws);
  a.dv_acc = a.dk_acc == nullptr
                 ? nullptr
                 : a.dk_acc + (size_t)g4::k_stream_tokens(*p) * p->num_kv_heads * p->head_dim;
  hipStream_t st = (hipStream_t)stream;
  int i = 0, rc = G4_OK;
  g4::for_each_ds_stripe(*p, [&](const g4::DsStripe& s) {
    if (rc != G4_OK) return;
    a.ds_row_lo = s.row_lo;
    a.ds_rows = s.rows;
    a.ds_cols = s.cols;
    a.ds_seq_rows = s.seq_rows;
    a.dq_qt_lo = s.seq_rows > 0 ? 0 : s.row_lo / 4;
    a.acc_mode = (i > 0 ? 1 : 0) | (i + 1 == nstripes ? 2 : 0);
    hipError_t e = g4::launch_bwd_dkdv(a, st);
    if (e != hipSuccess) {
      rc = hip_fail(e, "backward dK/dV (striped)");
      return;
    }
    e = g4::launch_bwd_dq(a, st);
    if (e != hipSuccess) rc = hip_fail(e, "backward dQ (striped)");
    ++i;
  });
  return rc;
}

int g4_mask_materialize(const g4_problem* p, uint8_t* out, void* ws, size_t ws_bytes,
                        void* stream) {
  g_last_error.clear();
  G4_TRY(check_problem(p));
  if (out == nullptr) return fail(G4_ERR_INVALID, "out is NULL");
  (void)ws;
  (void)ws_bytes;
  hipError_t e = g4::launch_mask(*p, out, nullptr, nullptr, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "mask");
  return G4_OK;
}

static int check_kv_prep(const g4_kv_prep* p) {
  if (p == nullptr) return fail(G4_ERR_INVALID, "K/V preparation descriptor is NULL");
  if (p->num_batches < 1 || p->seqlen < 1 || p->num_heads < 1)
    return fail(G4_ERR_INVALID, "num_batches, seqlen and num_heads must be >= 1");
  if (p->head_dim != 512 && p->head_dim != 256)
    return fail(G4_ERR_UNSUPPORTED, "K/V preparation supports head_dim 512 and 256");
  if (p->rotary_dim < 0 || p->rotary_dim > p->head_dim || p->rotary_dim % 16)
    return fail(G4_ERR_INVALID, "rotary_dim must be a multiple of 16 in [0, head_dim]");
  if (!(p->eps >= 0.f) || p->eps > 1.f) return fail(G4_ERR_INVALID, "eps must be in [0, 1]");
  if (p->cs_batch_stride < 0 || p->cs_batch_stride % 4)
    return fail(G4_ERR_INVALID, "cs_batch_stride must be a non-negative multiple of 4");
  if (p->k_fp32 != 0 && p->k_fp32 != 1) return fail(G4_ERR_INVALID, "k_fp32 must be 0 or 1");
  return G4_OK;
}

static int check_prep_operand(const void* ptr, const g4_layout& l, const char* name) {
  if (ptr == nullptr) return fail(G4_ERR_INVALID, "operand %s is NULL", name);
  if (((uintptr_t)ptr) % 16) return fail(G4_ERR_INVALID, "operand %s must be 16-byte aligned", name);
  if (l.token_stride <= 0 || l.head_stride <= 0 || l.batch_stride < 0 || l.token_stride % 8 ||
      l.head_stride % 8 || l.batch_stride % 8)
    return fail(G4_ERR_INVALID, "operand %s strides must be multiples of 8 elements", name);
  return G4_OK;
}

static int check_prep_tables(const g4_kv_prep* p, const float* w, const float* c, const float* s,
                             bool rope = true) {
  if (w == nullptr || ((uintptr_t)w) % 16)
    return fail(G4_ERR_INVALID, "weight must be a 16-byte aligned fp32 array");
  if (rope && p->rotary_dim > 0 && (c == nullptr || s == nullptr || ((uintptr_t)c) % 16 ||
                            ((uintptr_t)s) % 16))
    return fail(G4_ERR_INVALID, "cos and sin must be 16-byte aligned fp32 arrays");
  return G4_OK;
}

int g4_kv_prep_fwd(const g4_kv_prep* p, const void* z, g4_layout zl, const float* weight,
                   const float* cosv, const float* sinv, void* k, g4_layout kl, void* v,
                   g4_layout vl, void* stream) {
  g_last_error.clear();
  G4_TRY(check_kv_prep(p));
  G4_TRY(check_prep_operand(z, zl, "z"));
  if (k == nullptr && v == nullptr) return fail(G4_ERR_INVALID, "both K and V are NULL");
  if (k != nullptr) G4_TRY(check_prep_operand(k, kl, "k"));
  if (v != nullptr) G4_TRY(check_prep_operand(v, vl, "v"));
  G4_TRY(check_prep_tables(p, weight, k != nullptr ? cosv : nullptr, k != nullptr ? sinv : nullptr,
                           k != nullptr));
  hipError_t e = g4::launch_kv_prep_fwd(*p, z, zl, weight, cosv, sinv, k, kl, v, vl,
                                        (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "K/V preparation forward");
  return G4_OK;
}

size_t g4_kv_prep_workspace_bytes(const g4_kv_prep* p) {
  g_last_error.clear();
  if (check_kv_prep(p) != G4_OK) return 0;
  return g4::kv_prep_workspace_bytes(*p);
}

int g4_kv_prep_bwd(const g4_kv_prep* p, const void* z, g4_layout zl, const float* weight,
                   const float* cosv, const float* sinv, const void* dk, g4_layout dkl,
                   const void* dv, g4_layout dvl, void* dz, g4_layout dzl, float* dweight,
                   void* ws, size_t ws_bytes, void* stream) {
  g_last_error.clear();
  G4_TRY(check_kv_prep(p));
  if (p->head_dim != 512)
    return fail(G4_ERR_UNSUPPORTED, "the K/V preparation backward covers head_dim 512");
  G4_TRY(check_prep_operand(z, zl, "z"));
  G4_TRY(check_prep_operand(dk, dkl, "dk"));
  G4_TRY(check_prep_operand(dv, dvl, "dv"));
  G4_TRY(check_prep_operand(dz, dzl, "dz"));
  G4_TRY(check_prep_tables(p, weight, cosv, sinv));
  if (dweight == nullptr || ((uintptr_t)dweight) % 16)
    return fail(G4_ERR_INVALID, "dweight must be a 16-byte aligned fp32 array");
  const size_t need = g4::kv_prep_workspace_bytes(*p);
  if (ws_bytes < need || ws == nullptr || ((uintptr_t)ws) % 16) {
    char buf[128];
    snprintf(buf, sizeof buf, "%zu aligned bytes needed, %zu given", need, ws_bytes);
    return fail(G4_ERR_WORKSPACE, "K/V preparation workspace: %s", buf);
  }
  hipError_t e = g4::launch_kv_prep_bwd(*p, z, zl, weight, cosv, sinv, dk, dkl, dv, dvl, dz, dzl,
                                        dweight, ws, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "K/V preparation backward");
  return G4_OK;
}

int g4_tile_ranges(const g4_problem* p, int direction, int row_tile, int32_t* out, void* ws,
                   size_t ws_bytes, void* stream) {
  g_last_error.clear();
  G4_TRY(check_problem(p));
  if (out == nullptr) return fail(G4_ERR_INVALID, "out is NULL");
  if (direction != 0 && direction != 1) return fail(G4_ERR_INVALID, "direction must be 0 or 1");
  if (row_tile < 1 || row_tile > 1024) return fail(G4_ERR_INVALID, "row_tile must be in [1, 1024]");
  G4_TRY(check_ws(p, 0, ws, ws_bytes));
  hipStream_t st = (hipStream_t)stream;
  if (g4::spans_bytes(*p)) {
    hipError_t e = g4::launch_spans(*p, ws, st);
    if (e != hipSuccess) return hip_fail(e, "span table");
  }
  const int *lo, *hi;
  g4::span_arrays(*p, ws, &lo, &hi);
  hipError_t e = g4::launch_ranges(*p, direction, row_tile, out, lo, hi, st);
  if (e != hipSuccess) return hip_fail(e, "ranges");
  return G4_OK;
}

}  // extern "C"
