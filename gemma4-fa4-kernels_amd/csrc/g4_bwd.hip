// Backward pre-pass: delta[h, t] = rowsum(O * dO) - dLSE (fp32), one wave per row.
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

template <int D>
__global__ void __launch_bounds__(256) delta_kernel(BwdParams a, int64_t tq) {
  const int lane = threadIdx.x & 63;
  const int64_t rows = tq * a.p.num_q_heads;
  for (int64_t r = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) / 64; r < rows;
       r += (int64_t)gridDim.x * blockDim.x / 64) {
    const int64_t t = r / a.p.num_q_heads;
    const int h = (int)(r % a.p.num_q_heads);
    int s, i;
    seq_of_qtoken(a.p, t, s, i);
    const Seq sq = resolve_seq(a.p, s);
    const __bf16* orow = a.o + tok_off(sq, s, sq.qtok, i, a.ol) + (int64_t)h * a.ol.head_stride;
    const __bf16* grow =
        a.dout + tok_off(sq, s, sq.qtok, i, a.dol) + (int64_t)h * a.dol.head_stride;
    float acc = 0.f;
#pragma unroll
    for (int c = lane * 8; c < D; c += 512) {
      bf16x8 x = ld_global16(orow + c), y = ld_global16(grow + c);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc += (float)x[e] * (float)y[e];
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
    if (lane == 0) {
      float dl = a.dlse ? a.dlse[lse_off(a.p, sq, s, h, i)] : 0.f;
      a.delta[(int64_t)h * tq + t] = acc - dl;
    }
  }
}

}  // namespace

hipError_t launch_bwd_delta(const BwdParams& a, hipStream_t stream) {
  const int64_t tq = q_stream_tokens(a.p);
  const int64_t rows = tq * a.p.num_q_heads;
  int64_t blocks = (rows + 3) / 4;
  if (blocks > 65536) blocks = 65536;
  if (a.p.head_dim == 256)
    delta_kernel<256><<<(unsigned)blocks, 256, 0, stream>>>(a, tq);
  else
    delta_kernel<512><<<(unsigned)blocks, 256, 0, stream>>>(a, tq);
  return hipGetLastError();
}

}  // namespace g4
