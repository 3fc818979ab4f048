// Backward pre-pass: delta[h, t] = rowsum(O * dO) - dLSE (fp32).
#include "g4_kernels.h"

namespace g4 {

namespace {

__device__ inline void seq_of_qtoken(const g4_problem& p, int64_t t, int& s, int& i) {
  if (p.cu_seqlens_q == nullptr) {
    s = (int)(t / p.seqlen_q);
    i = (int)(t - (int64_t)s * p.seqlen_q);
    return;
  }
  int lo = 0, hi = p.num_seqs;
  while (hi - lo > 1) {
    int mid = (lo + hi) >> 1;
    if (p.cu_seqlens_q[mid] <= t) lo = mid; else hi = mid;
  }
  s = lo;
  i = (int)(t - p.cu_seqlens_q[lo]);
}

// One wave per (query token, group of kHG query heads): every lane loads its
// 16-byte chunks of the group's O and dO rows before any reduction, so a wave
// keeps 2 * kHG * D * 2 bytes in flight; 64 / CPR heads share each load
// instruction (CPR = D / 8 chunks per row) and each head's dot product is
// reduced over its CPR lanes.
template <int D>
__global__ void __launch_bounds__(256) delta_kernel(BwdParams a, int64_t tq) {
  constexpr int CPR = D / 8;          // 16-byte chunks per head row
  constexpr int HPI = 64 / CPR;       // heads per load instruction
  constexpr int kHG = 8;              // heads per wave item
  constexpr int NI = kHG / HPI;       // load instructions per operand
  const int lane = threadIdx.x & 63;
  const int hq = a.p.num_q_heads;
  const int groups = (hq + kHG - 1) / kHG;
  const int64_t items = tq * groups;
  const int c = lane % CPR, hl = lane / CPR;
  // Every backward call starts its tile kernels' work queues from zero.
  if (blockIdx.x == 0 && threadIdx.x < kSchedClear && a.sched != nullptr) a.sched[threadIdx.x] = 0u;
  for (int64_t r = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) / 64; r < items;
       r += (int64_t)gridDim.x * blockDim.x / 64) {
    const int64_t t = r / groups;
    const int h0 = (int)(r % groups) * kHG;
    int s, i;
    seq_of_qtoken(a.p, t, s, i);
    const Seq sq = resolve_seq(a.p, s);
    const __bf16* obase = a.o + tok_off(sq, s, sq.qtok, i, a.ol) + c * 8;
    const __bf16* gbase = a.dout + tok_off(sq, s, sq.qtok, i, a.dol) + c * 8;
    bf16x8 x[NI], y[NI];
    // O is read here for the last time: non-temporal, so it does not push out
    // of the caches the dO (and Q, K, V) that the dK/dV pass reads next
    // (config 2 backward -2%).
#pragma unroll
    for (int u = 0; u < NI; ++u) {
      const int h = min(h0 + u * HPI + hl, hq - 1);
      x[u] = __builtin_nontemporal_load((const bf16x8*)(obase + (int64_t)h * a.ol.head_stride));
      y[u] = ld_global16(gbase + (int64_t)h * a.dol.head_stride);
    }
#pragma unroll
    for (int u = 0; u < NI; ++u) {
      float acc = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc += (float)x[u][e] * (float)y[u][e];
#pragma unroll
      for (int o = CPR / 2; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
      const int h = h0 + u * HPI + hl;
      if (c == 0 && h < hq) {
        const float dl = a.dlse ? a.dlse[lse_off(a.p, sq, s, h, i)] : 0.f;
        a.delta[(int64_t)h * tq + t] = acc - dl;
      }
    }
  }
}

}  // namespace

hipError_t launch_bwd_delta(const BwdParams& a, hipStream_t stream) {
  const int64_t tq = q_stream_tokens(a.p);
  const int64_t items = tq * ((a.p.num_q_heads + 7) / 8);  // waves of work (kHG = 8)
  int64_t blocks = (items + 3) / 4;
  if (blocks > 8192) blocks = 8192;
  if (a.p.head_dim == 256)
    delta_kernel<256><<<(unsigned)blocks, 256, 0, stream>>>(a, tq);
  else
    delta_kernel<512><<<(unsigned)blocks, 256, 0, stream>>>(a, tq);
  return hipGetLastError();
}

}  // namespace g4
