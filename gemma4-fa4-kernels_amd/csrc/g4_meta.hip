// Mask metadata kernels: vision spans, mask materialisation, scheduler ranges.
//
// Vision span of a K-stream token t with vision ID >= 0: the first and last
// position, within t's sequence, of the tokens sharing t's (document, vision)
// pair.  For the local Gemma mask a query at position a may attend future keys
// only inside its span (no right window cap), so the span ends bound the key
// range of a query tile (span_hi, any ID pattern, repeated or non-contiguous
// IDs included).  They are computed on device with one open-addressing hash
// table per sequence (2 * Lk slots), O(tokens), no host round trip.
//
// The query range of a key tile is bounded below by span_lo, which for the
// backward and the tile scheduler (not the forward, which does not read it)
// is the first query position whose reach (its position, or its span end)
// is at or past the key: then a key tile's query range holds every query tile
// whose key range holds the key tile.  The stored-dS dQ pass reads, per query
// row, every band tile up to the row's furthest reach, so the dK/dV pass must
// write each of them (zeros where no query of the row attends the tile: the
// keys between the runs of a vision ID that repeats non-contiguously).
#include "g4_kernels.h"

namespace g4 {

namespace {

constexpr unsigned long long kEmpty = ~0ull;

struct SpanWs {
  int* lo;
  int* hi;
  unsigned long long* keys;
  int* first;
  int* last;
  int* repeats;  // nonzero when some (document, vision ID) key has two runs
};

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

__host__ __device__ inline SpanWs span_ws(void* ws, int64_t tk) {
  char* b = (char*)ws;
  SpanWs w;
  w.lo = (int*)b;
  b += align256(tk * 4);
  w.hi = (int*)b;
  b += align256(tk * 4);
  w.keys = (unsigned long long*)b;
  b += align256(2 * tk * 8);
  w.first = (int*)b;
  b += align256(2 * tk * 4);
  w.last = (int*)b;
  b += align256(2 * tk * 4);
  w.repeats = (int*)b;
  return w;
}

// Sequence holding K-stream token t, with its start and length.
__device__ inline void seq_of_token(const g4_problem& p, int64_t t, int& s, int64_t& ks, int& lk) {
  if (p.cu_seqlens_k == nullptr) {
    s = (int)(t / p.seqlen_k);
    ks = (int64_t)s * p.seqlen_k;
    lk = p.seqlen_k;
    return;
  }
  int lo = 0, hi = p.num_seqs;  // find last s with cu[s] <= t
  while (hi - lo > 1) {
    int mid = (lo + hi) >> 1;
    if (p.cu_seqlens_k[mid] <= t) lo = mid; else hi = mid;
  }
  s = lo;
  ks = p.cu_seqlens_k[lo];
  lk = p.cu_seqlens_k[lo + 1] - p.cu_seqlens_k[lo];
}

__device__ inline unsigned long long span_key(const g4_problem& p, int64_t t, int vid) {
  unsigned doc = p.document_ids ? (unsigned)p.document_ids[t] : 0u;
  return ((unsigned long long)doc << 32) | (unsigned)vid;
}

__device__ inline int64_t probe_slot(SpanWs w, int64_t base, int64_t cap, unsigned long long key,
                                     bool insert) {
  unsigned long long h = key * 0x9E3779B97F4A7C15ull;
  int64_t slot = (int64_t)((h >> 32) % (unsigned long long)cap);
  for (int64_t n = 0; n < cap; ++n) {
    unsigned long long* cell = w.keys + base + slot;
    unsigned long long cur = insert ? atomicCAS(cell, kEmpty, key) : *cell;
    if (cur == key || (insert && cur == kEmpty)) return base + slot;
    slot = slot + 1 == cap ? 0 : slot + 1;
  }
  return -1;  // unreachable: the table holds at most Lk keys in 2 * Lk slots
}

__global__ void span_init_kernel(SpanWs w, int64_t nslots) {
  if (blockIdx.x == 0 && threadIdx.x == 0) *w.repeats = 0;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < nslots;
       i += (int64_t)gridDim.x * blockDim.x) {
    w.keys[i] = kEmpty;
    w.first[i] = 0x7fffffff;
    w.last[i] = -1;
  }
}

__global__ void span_insert_kernel(g4_problem p, SpanWs w, int64_t tk) {
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < tk;
       t += (int64_t)gridDim.x * blockDim.x) {
    int vid = p.vision_ids[t];
    if (vid < 0) continue;
    int s, lk;
    int64_t ks;
    seq_of_token(p, t, s, ks, lk);
    // Only the ends of each run of equal keys (vision ID and document): a
    // run's first position bounds its key's span from below and its last from
    // above, so the other tokens add nothing (and every token of a block
    // updating the same two words serialises on them: config 3's table took
    // 24 us).
    const unsigned long long key = span_key(p, t, vid);
    const bool starts = t == ks || span_key(p, t - 1, p.vision_ids[t - 1]) != key;
    const bool ends = t + 1 == ks + lk || span_key(p, t + 1, p.vision_ids[t + 1]) != key;
    if (!starts && !ends) continue;
    int64_t slot = probe_slot(w, 2 * ks, 2 * (int64_t)lk, key, true);
    if (slot < 0) continue;
    int j = (int)(t - ks);
    if (starts) atomicMin(w.first + slot, j);
    if (ends) atomicMax(w.last + slot, j);
  }
}

__global__ void span_lookup_kernel(g4_problem p, SpanWs w, int64_t tk) {
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < tk;
       t += (int64_t)gridDim.x * blockDim.x) {
    int s, lk;
    int64_t ks;
    seq_of_token(p, t, s, ks, lk);
    int j = (int)(t - ks);
    int vid = p.vision_ids[t];
    int lo = j, hi = j;
    if (vid >= 0) {
      const unsigned long long key = span_key(p, t, vid);
      int64_t slot = probe_slot(w, 2 * ks, 2 * (int64_t)lk, key, false);
      if (slot >= 0) {
        lo = w.first[slot];
        hi = w.last[slot];
        // A run that starts after its key's first position: the key repeats.
        if (lo < j && span_key(p, t - 1, p.vision_ids[t - 1]) != key) atomicOr(w.repeats, 1);
      }
    }
    w.lo[t] = lo;
    w.hi[t] = hi;
  }
}

// span_lo[j] = min{a >= off : M(a) >= j}, with M(a) the largest span end of
// the query positions off..a (each at least the position itself) and off =
// Sk - Sq the first query position.  Never above the key's own span start, so
// it only widens the query ranges of key tiles.  M comes from one prefix
// maximum over the whole K stream of g(t) = ks + span_hi[t] for query
// positions (ks the first token of t's sequence) and -1 for the others:
// every value from an earlier sequence lies below ks, so no reset is needed
// at sequence starts, and M(a) = G(ks + a) - ks.  The scan runs in chunks of
// kReachChunk tokens: one pass writes each chunk's maximum, the next scans
// each chunk from the maxima of the earlier chunks of its first sequence.  M
// is written over the hash table's `first` words and the chunk maxima over
// its `last` words (both free once the spans are looked up); then one binary
// search per key over its sequence's M, which is non-decreasing and ends at
// M(Sk - 1) = Sk - 1.
//
// When every (document, vision ID) key forms a single run (the lookup pass
// sets `repeats` otherwise), a position's span ends inside its own run, so the
// first position whose span reaches key j is j's span start, or Sk - Sq when
// the span starts before the first query position: the span starts are then a
// lower bound as good as the query reach, and the three passes return at once.
constexpr int kReachChunk = 1024;  // tokens per workgroup, one per thread

__device__ __forceinline__ long long reach_end(const g4_problem& p, SpanWs w, int64_t t,
                                               int64_t tk) {
  if (t >= tk) return -1;
  int s, lk;
  int64_t ks;
  seq_of_token(p, t, s, ks, lk);
  const int lq = resolve_seq(p, s).lq;
  return (int)(t - ks) >= lk - lq ? (long long)ks + w.hi[t] : -1;
}

__device__ __forceinline__ long long wave_max(long long v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
  return v;
}

__global__ void __launch_bounds__(kReachChunk) span_chunk_max_kernel(g4_problem p, SpanWs w,
                                                                     int64_t tk) {
  __shared__ long long wmax[kReachChunk / 64];
  if (*w.repeats == 0) return;  // span starts are the query reach (uniform)
  const int tid = threadIdx.x;
  const long long v = wave_max(reach_end(p, w, blockIdx.x * (int64_t)kReachChunk + tid, tk));
  if ((tid & 63) == 0) wmax[tid >> 6] = v;
  __syncthreads();
  if (tid == 0) {
    long long all = -1;
    for (int x = 0; x < kReachChunk / 64; ++x) all = max(all, wmax[x]);
    reinterpret_cast<long long*>(w.last)[blockIdx.x] = all;
  }
}

__global__ void __launch_bounds__(kReachChunk) span_chunk_scan_kernel(g4_problem p, SpanWs w,
                                                                      int64_t tk) {
  __shared__ long long wtot[kReachChunk / 64], wcarry[kReachChunk / 64];
  if (*w.repeats == 0) return;  // (uniform)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t t0 = blockIdx.x * (int64_t)kReachChunk, t = t0 + tid;
  // Earlier chunks that can hold tokens of this chunk's sequences: from the
  // one holding the first token's sequence start.
  int s0, lk0;
  int64_t ks0;
  seq_of_token(p, t0, s0, ks0, lk0);
  const long long* cmax = reinterpret_cast<const long long*>(w.last);
  long long c = -1;
  for (int64_t x = ks0 / kReachChunk + tid; x < (int64_t)blockIdx.x; x += kReachChunk)
    c = max(c, cmax[x]);
  c = wave_max(c);
  long long v = reach_end(p, w, t, tk);
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const long long u = __shfl_up(v, o, 64);
    if (lane >= o) v = max(v, u);
  }
  if (lane == 63) wtot[wave] = v;
  if (lane == 0) wcarry[wave] = c;
  __syncthreads();
#pragma unroll
  for (int x = 0; x < kReachChunk / 64; ++x) {
    v = max(v, wcarry[x]);
    if (x < wave) v = max(v, wtot[x]);
  }
  if (t < tk) {
    int s, lk;
    int64_t ks;
    seq_of_token(p, t, s, ks, lk);
    w.first[t] = v >= ks ? (int)(v - ks) : -1;  // -1: no query position yet
  }
}

__global__ void span_reach_kernel(g4_problem p, SpanWs w, int64_t tk) {
  if (*w.repeats == 0) return;  // span_lo keeps the span starts
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < tk;
       t += (int64_t)gridDim.x * blockDim.x) {
    int s, lk;
    int64_t ks;
    seq_of_token(p, t, s, ks, lk);
    const Seq sq = resolve_seq(p, s);
    if (sq.lq <= 0) {
      w.lo[t] = 0x7fffffff;  // no query attends this sequence's keys
      continue;
    }
    const int j = (int)(t - ks);
    const int* m = w.first + ks;
    int l = max(lk - sq.lq, 0), r = lk - 1;  // the first a in [off, Sk) with M(a) >= j
    while (l < r) {
      const int mid = (l + r) >> 1;
      if (m[mid] >= j)
        r = mid;
      else
        l = mid + 1;
    }
    w.lo[t] = l;
  }
}

__global__ void mask_kernel(g4_problem p, uint8_t* out) {
  const int64_t per_seq = (int64_t)p.seqlen_q * p.seqlen_k;
  const int64_t n = per_seq * p.num_seqs;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n;
       e += (int64_t)gridDim.x * blockDim.x) {
    int s = (int)(e / per_seq);
    int64_t r = e % per_seq;
    int i = (int)(r / p.seqlen_k), j = (int)(r % p.seqlen_k);
    Seq sq = resolve_seq(p, s);
    uint8_t v = 0;
    if (i < sq.lq && j < sq.lk) {
      int a = i + sq.lk - sq.lq;
      bool has_vid = p.vision_ids != nullptr && p.bidirectional_vision;
      bool has_doc = p.document_ids != nullptr;
      int vq = has_vid ? p.vision_ids[sq.ktok + a] : -1;
      int vk = has_vid ? p.vision_ids[sq.ktok + j] : -1;
      int dq = has_doc ? p.document_ids[sq.ktok + a] : 0;
      int dk = has_doc ? p.document_ids[sq.ktok + j] : 0;
      v = allowed(a, j, p.window, has_vid, vq, vk, has_doc, dq, dk) ? 1 : 0;
    }
    out[e] = v;
  }
}

__global__ void ranges_kernel(g4_problem p, int direction, int row_tile, int ntiles, int32_t* out,
                              const int* span_lo, const int* span_hi) {
  int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= p.num_seqs * ntiles) return;
  int s = e / ntiles, t = e % ntiles;
  Seq sq = resolve_seq(p, s);
  int off = sq.lk - sq.lq;
  bool has_vid = p.vision_ids != nullptr && p.bidirectional_vision;
  int lo = 0, hi = 0;
  if (direction == 0) {
    int i0 = t * row_tile;
    if (i0 < sq.lq) {
      int i1 = min(i0 + row_tile, sq.lq) - 1;
      int smax = -1;
      if (has_vid)
        for (int i = i0; i <= i1; ++i) smax = max(smax, span_hi[sq.ktok + i + off]);
      query_tile_key_range(i0 + off, i1 + off, sq.lk, p.window, smax, lo, hi);
    }
  } else {
    int j0 = t * row_tile;
    if (j0 < sq.lk) {
      int j1 = min(j0 + row_tile, sq.lk) - 1;
      int smin = 0x7fffffff;
      if (has_vid)
        for (int j = j0; j <= j1; ++j) smin = min(smin, span_lo[sq.ktok + j]);
      key_tile_query_range(j0, j1, sq.lq, off, p.window, smin, lo, hi);
    }
  }
  out[2 * e] = lo;
  out[2 * e + 1] = hi;
}

int grid_for(int64_t n, int block) {
  int64_t g = (n + block - 1) / block;
  if (g < 1) g = 1;
  if (g > 65536) g = 65536;
  return (int)g;
}

}  // namespace

int64_t k_stream_tokens(const g4_problem& p) {
  return p.cu_seqlens_k ? p.total_k : (int64_t)p.num_seqs * p.seqlen_k;
}

int64_t q_stream_tokens(const g4_problem& p) {
  return p.cu_seqlens_q ? p.total_q : (int64_t)p.num_seqs * p.seqlen_q;
}

size_t spans_bytes(const g4_problem& p) {
  if (p.vision_ids == nullptr || !p.bidirectional_vision) return 0;
  int64_t tk = k_stream_tokens(p);
  return align256(tk * 4) * 2 + align256(2 * tk * 8) + align256(2 * tk * 4) * 2 + 256;
}

hipError_t launch_spans(const g4_problem& p, void* ws, hipStream_t stream, bool query_reach) {
  int64_t tk = k_stream_tokens(p);
  SpanWs w = span_ws(ws, tk);
  span_init_kernel<<<grid_for(2 * tk, 256), 256, 0, stream>>>(w, 2 * tk);
  span_insert_kernel<<<grid_for(tk, 256), 256, 0, stream>>>(p, w, tk);
  span_lookup_kernel<<<grid_for(tk, 256), 256, 0, stream>>>(p, w, tk);
  if (query_reach && tk > 0) {
    const int64_t chunks = (tk + kReachChunk - 1) / kReachChunk;
    span_chunk_max_kernel<<<chunks, kReachChunk, 0, stream>>>(p, w, tk);
    span_chunk_scan_kernel<<<chunks, kReachChunk, 0, stream>>>(p, w, tk);
    span_reach_kernel<<<grid_for(tk, 256), 256, 0, stream>>>(p, w, tk);
  }
  return hipGetLastError();
}

hipError_t launch_mask(const g4_problem& p, uint8_t* out, const int*, const int*,
                       hipStream_t stream) {
  int64_t n = (int64_t)p.seqlen_q * p.seqlen_k * p.num_seqs;
  mask_kernel<<<grid_for(n, 256), 256, 0, stream>>>(p, out);
  return hipGetLastError();
}

hipError_t launch_ranges(const g4_problem& p, int direction, int row_tile, int32_t* out,
                         const int* span_lo, const int* span_hi, hipStream_t stream) {
  int len = direction == 0 ? p.seqlen_q : p.seqlen_k;
  int ntiles = (len + row_tile - 1) / row_tile;
  int n = ntiles * p.num_seqs;
  if (n <= 0) return hipSuccess;
  ranges_kernel<<<(n + 127) / 128, 128, 0, stream>>>(p, direction, row_tile, ntiles, out, span_lo,
                                                     span_hi);
  return hipGetLastError();
}

// Span arrays inside a workspace produced by launch_spans.
void span_arrays(const g4_problem& p, void* ws, const int** lo, const int** hi) {
  if (spans_bytes(p) == 0) {
    *lo = *hi = nullptr;
    return;
  }
  SpanWs w = span_ws(ws, k_stream_tokens(p));
  *lo = w.lo;
  *hi = w.hi;
}

}  // namespace g4
