// K/V (and Q) preparation from a projection source, fused.
//
// Per (token, head) row z of head_dim D (512 for the global layer's shared
// K/V source and its queries, 256 for the sliding layers' queries and keys):
//   r  = (mean(z^2) + eps)^(-1/2)            (fp32 over the row)
//   n  = z r                                  (fp32)
//   V  = bf16(n)                              (RMSNorm without a weight)
//   kn = bf16(n w)                            (RMSNorm with the learned weight)
//   K  = kn with RoPE on its first R dims: K_i = kn_i cos_i + rot(kn)_i sin_i,
//        rot(x)_i = -x_{i+R/2} (i < R/2), x_{i-R/2} (R/2 <= i < R); the other
//        dims pass through.  K in fp32 (fp32 tables): fp32 products and sum,
//        no contraction.  K in bf16 (bf16 tables): each product and the sum
//        rounded to bf16, as bf16 tensor operations round them.
// One wave per row, lane l holding dims E l .. E l + E - 1 (E = D / 64: one
// 16- or 8-byte load), so the row reduction is a wave reduction and rot(x) is
// a lane exchange with lane l +- R / (2 E).  HBM-bound: each row reads 2 D
// bytes of z and writes K and V (either may be left out).
//
// Backward (D = 512; fp32 throughout, dz rounded to bf16 once):
//   g_k  = adjoint of the RoPE applied to dK: i < R/2: dK_i cos_i + dK_{i+R/2} sin_{i+R/2};
//          R/2 <= i < R: dK_i cos_i - dK_{i-R/2} sin_{i-R/2}; pass dims dK_i
//   g_n  = g_k w + dV,   dw += g_k n  (summed over every row)
//   dz   = r g_n - (r^3 / D) z sum_j(g_n,j z_j)
// dw is summed per workgroup in a fixed order into workspace rows, then the
// rows are summed in a fixed order by a second kernel: no atomics, bitwise
// repeatable.
#include <algorithm>

#include "g4_kernels.h"

namespace g4 {
namespace {

constexpr int kPrepD = 512;
constexpr int kPrepWaves = 4;      // forward: rows in flight per workgroup
constexpr int kPrepBwdWaves = 16;  // backward: more rows per dweight partial row

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
  return x;
}

struct RowAddr {
  int64_t b, t, h;
};

__device__ __forceinline__ RowAddr row_of(const g4_kv_prep& p, int64_t row) {
  // rows enumerate (batch, token, head) with the head fastest
  const int64_t h = row % p.num_heads;
  const int64_t bt = row / p.num_heads;
  return RowAddr{bt / p.seqlen, bt % p.seqlen, h};
}

__device__ __forceinline__ int64_t elem_off(const g4_layout& l, const RowAddr& a) {
  return a.b * l.batch_stride + a.t * l.token_stride + a.h * l.head_stride;
}

__device__ __forceinline__ void load8(const __bf16* p, float (&x)[8]) {
  const bf16x8 v = *(const bf16x8*)p;
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = (float)v[e];
}

__device__ __forceinline__ void store8(__bf16* p, const float (&x)[8]) {
  bf16x8 v;
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = (__bf16)x[e];
  *(bf16x8*)p = v;
}

// cos / sin of a row's token for this lane's dims (lanes below R / 8 only).
__device__ __forceinline__ void load_rope(const g4_kv_prep& p, const float* cs, const RowAddr& a,
                                          int lane, float (&x)[8]) {
  const float* src = cs + a.b * p.cs_batch_stride + a.t * (int64_t)p.rotary_dim + 8 * lane;
  const f32x4 lo = *(const f32x4*)src;
  const f32x4 hi = *(const f32x4*)(src + 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    x[e] = lo[e];
    x[4 + e] = hi[e];
  }
}

template <int E>
using bf16v = __bf16 __attribute__((ext_vector_type(E)));

// E consecutive bf16 / fp32 elements of this lane.
template <int E>
__device__ __forceinline__ void load_e(const __bf16* p, float (&x)[E]) {
  const bf16v<E> v = *(const bf16v<E>*)p;
#pragma unroll
  for (int e = 0; e < E; ++e) x[e] = (float)v[e];
}

template <int E>
__device__ __forceinline__ void store_e(__bf16* p, const float (&x)[E]) {
  bf16v<E> v;
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = (__bf16)x[e];
  *(bf16v<E>*)p = v;
}

template <int E>
__device__ __forceinline__ void load_e(const float* p, float (&x)[E]) {
#pragma unroll
  for (int j = 0; j < E / 4; ++j) {
    const f32x4 v = *(const f32x4*)(p + 4 * j);
#pragma unroll
    for (int e = 0; e < 4; ++e) x[4 * j + e] = v[e];
  }
}

template <int E>
__global__ void __launch_bounds__(kPrepWaves * 64) kv_prep_fwd_kernel(
    g4_kv_prep p, const __bf16* z, g4_layout zl, const float* w, const float* cosv,
    const float* sinv, void* k, g4_layout kl, __bf16* v, g4_layout vl, int64_t rows) {
  constexpr int D = 64 * E;
  const int lane = threadIdx.x & 63;
  const int64_t first = (int64_t)blockIdx.x * kPrepWaves + (threadIdx.x >> 6);
  const int64_t step = (int64_t)gridDim.x * kPrepWaves;
  const int rl = p.rotary_dim / E;  // lanes holding rotary dims
  const int half = rl / 2;          // lane distance of the rotate-half partner
  float wl[E];
  load_e<E>(w + E * lane, wl);
  for (int64_t row = first; row < rows; row += step) {
    const RowAddr a = row_of(p, row);
    float x[E], c[E], s[E];
    load_e<E>(z + elem_off(zl, a) + E * lane, x);
    if (k != nullptr && lane < rl) {  // issued with z, before the row reduction waits for it
      const int64_t t = a.b * p.cs_batch_stride + a.t * (int64_t)p.rotary_dim + E * lane;
      load_e<E>(cosv + t, c);
      load_e<E>(sinv + t, s);
    }
    float ss = 0.f;
    {
#pragma clang fp contract(off)
#pragma unroll
      for (int e = 0; e < E; ++e) ss += x[e] * x[e];  // rounded squares, then sums
    }
    ss = wave_sum(ss);
    const float r = 1.f / __fsqrt_rn(ss / (float)D + p.eps);
    float n[E], kn[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
      n[e] = x[e] * r;
      kn[e] = (float)(__bf16)(n[e] * wl[e]);
    }
    if (v != nullptr) store_e<E>(v + elem_off(vl, a) + E * lane, n);
    if (k == nullptr) continue;
    // rotate-half partner values (every lane takes part in the exchange)
    const int partner = lane < half ? lane + half : lane - half;
    float pk[E];
#pragma unroll
    for (int e = 0; e < E; ++e) pk[e] = __shfl(kn[e], partner, 64);
    float kout[E];
#pragma unroll
    for (int e = 0; e < E; ++e) kout[e] = kn[e];
    if (lane < rl) {
      // x * cos + rotate_half(x) * sin as two products and a sum, no fused
      // multiply-add; in bf16 each product is rounded before the sum (the
      // products of bf16 values are exact in fp32, so one rounding each)
#pragma clang fp contract(off)
      const float sign = lane < half ? -1.f : 1.f;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        float a0 = kn[e] * c[e];
        float a1 = (sign * pk[e]) * s[e];
        if (!p.k_fp32) {
          a0 = (float)(__bf16)a0;
          a1 = (float)(__bf16)a1;
        }
        kout[e] = a0 + a1;
      }
    }
    if (p.k_fp32) {
      float* kp = (float*)k + elem_off(kl, a) + E * lane;
#pragma unroll
      for (int j = 0; j < E / 4; ++j)
        *(f32x4*)(kp + 4 * j) = f32x4{kout[4 * j], kout[4 * j + 1], kout[4 * j + 2], kout[4 * j + 3]};
    } else {
      store_e<E>((__bf16*)k + elem_off(kl, a) + E * lane, kout);
    }
  }
}

// dK of this lane's dims, from a bf16 or fp32 gradient.
__device__ __forceinline__ void load_dk(const g4_kv_prep& p, const void* dk, int64_t off,
                                        float (&x)[8]) {
  if (p.k_fp32) {
    const float* q = (const float*)dk + off;
    const f32x4 lo = *(const f32x4*)q;
    const f32x4 hi = *(const f32x4*)(q + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = lo[e];
      x[4 + e] = hi[e];
    }
  } else {
    load8((const __bf16*)dk + off, x);
  }
}

__global__ void __launch_bounds__(kPrepBwdWaves * 64) kv_prep_bwd_kernel(
    g4_kv_prep p, const __bf16* z, g4_layout zl, const float* w, const float* cosv,
    const float* sinv, const void* dk, g4_layout dkl, const __bf16* dv, g4_layout dvl,
    __bf16* dz, g4_layout dzl, float* dw_part, int64_t rows) {
  __shared__ f32x4 red[kPrepBwdWaves][64][2];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t first = (int64_t)blockIdx.x * kPrepBwdWaves + wave;
  const int64_t step = (int64_t)gridDim.x * kPrepBwdWaves;
  const int rl = p.rotary_dim / 8;
  const int half = rl / 2;
  float wl[8], dwl[8];
  {
    const f32x4 lo = *(const f32x4*)(w + 8 * lane);
    const f32x4 hi = *(const f32x4*)(w + 8 * lane + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      wl[e] = lo[e];
      wl[4 + e] = hi[e];
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) dwl[e] = 0.f;
  const int partner = lane < half ? lane + half : lane - half;
  for (int64_t row = first; row < rows; row += step) {
    const RowAddr a = row_of(p, row);
    float x[8], gk[8], gv[8], c[8], ps[8];  // cos of this lane's dims, sin of the partner's
    load8(z + elem_off(zl, a) + 8 * lane, x);
    load_dk(p, dk, elem_off(dkl, a) + 8 * lane, gk);
    load8(dv + elem_off(dvl, a) + 8 * lane, gv);
    if (lane < rl) {
      load_rope(p, cosv, a, lane, c);
      load_rope(p, sinv, a, partner, ps);
    }
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
    ss = wave_sum(ss);
    const float r = 1.f / __fsqrt_rn(ss / (float)kPrepD + p.eps);
    // adjoint of the RoPE: the partner lane's dK times its sin
    float pg[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) pg[e] = __shfl(gk[e], partner, 64);
    if (lane < rl) {
      const float sign = lane < half ? 1.f : -1.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) gk[e] = gk[e] * c[e] + sign * pg[e] * ps[e];
    }
    float gn[8], dot = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float n = x[e] * r;
      gn[e] = gk[e] * wl[e] + gv[e];
      dwl[e] += gk[e] * n;
      dot += gn[e] * x[e];
    }
    dot = wave_sum(dot);
    const float coef = r * r * r * dot / (float)kPrepD;
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = r * gn[e] - coef * x[e];
    store8(dz + elem_off(dzl, a) + 8 * lane, o);
  }
  // fixed-order sum of the waves' dw partials, one 512-float row per workgroup
  red[wave][lane][0] = f32x4{dwl[0], dwl[1], dwl[2], dwl[3]};
  red[wave][lane][1] = f32x4{dwl[4], dwl[5], dwl[6], dwl[7]};
  __syncthreads();
  if (wave == 0) {
    f32x4 s0 = red[0][lane][0], s1 = red[0][lane][1];
#pragma unroll
    for (int wv = 1; wv < kPrepBwdWaves; ++wv) {
      s0 += red[wv][lane][0];
      s1 += red[wv][lane][1];
    }
    float* dst = dw_part + (int64_t)blockIdx.x * kPrepD + 8 * lane;
    *(f32x4*)dst = s0;
    *(f32x4*)(dst + 4) = s1;
  }
}

// dw[d] = sum over workgroups of dw_part[b][d] in a fixed order: a block owns
// 8 columns; thread (g, c) sums rows b = g, g + 32, ... of column c in order,
// then thread g = 0 adds the 32 group sums in group order.
__global__ void __launch_bounds__(256) kv_prep_dw_kernel(const float* dw_part, int nparts,
                                                         float* dw) {
  __shared__ float part[32][8];
  const int c = threadIdx.x & 7, g = threadIdx.x >> 3;
  const int d = blockIdx.x * 8 + c;
  float s = 0.f;
  for (int b = g; b < nparts; b += 32) s += dw_part[(int64_t)b * kPrepD + d];
  part[g][c] = s;
  __syncthreads();
  if (g == 0) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) t += part[i][c];
    dw[d] = t;
  }
}

}  // namespace

// Workgroups of the backward (each writes one row of dweight partials):
// enough waves to keep HBM busy, few partial rows to sum.
int kv_prep_blocks(int64_t rows) {
  const int64_t want = (rows + kPrepBwdWaves - 1) / kPrepBwdWaves;
  return (int)std::min<int64_t>(want, 512);
}

size_t kv_prep_workspace_bytes(const g4_kv_prep& p) {
  const int64_t rows = (int64_t)p.num_batches * p.seqlen * p.num_heads;
  return (size_t)kv_prep_blocks(rows) * kPrepD * sizeof(float);
}

hipError_t launch_kv_prep_fwd(const g4_kv_prep& p, const void* z, g4_layout zl, const float* w,
                              const float* cosv, const float* sinv, void* k, g4_layout kl,
                              void* v, g4_layout vl, hipStream_t stream) {
  const int64_t rows = (int64_t)p.num_batches * p.seqlen * p.num_heads;
  if (rows <= 0) return hipSuccess;
  const int fwd_blocks = (int)std::min<int64_t>((rows + kPrepWaves - 1) / kPrepWaves, 4096);
  if (p.head_dim == 256)
    hipLaunchKernelGGL(kv_prep_fwd_kernel<4>, dim3(fwd_blocks), dim3(kPrepWaves * 64), 0,
                       stream, p, (const __bf16*)z, zl, w, cosv, sinv, k, kl, (__bf16*)v, vl,
                       rows);
  else
    hipLaunchKernelGGL(kv_prep_fwd_kernel<8>, dim3(fwd_blocks), dim3(kPrepWaves * 64), 0,
                       stream, p, (const __bf16*)z, zl, w, cosv, sinv, k, kl, (__bf16*)v, vl,
                       rows);
  return hipGetLastError();
}

hipError_t launch_kv_prep_bwd(const g4_kv_prep& p, const void* z, g4_layout zl, const float* w,
                              const float* cosv, const float* sinv, const void* dk,
                              g4_layout dkl, const void* dv, g4_layout dvl, void* dz,
                              g4_layout dzl, float* dw, void* ws, hipStream_t stream) {
  const int64_t rows = (int64_t)p.num_batches * p.seqlen * p.num_heads;
  const int blocks = rows > 0 ? kv_prep_blocks(rows) : 0;
  if (blocks > 0) {
    hipLaunchKernelGGL(kv_prep_bwd_kernel, dim3(blocks), dim3(kPrepBwdWaves * 64), 0, stream, p,
                       (const __bf16*)z, zl, w, cosv, sinv, dk, dkl, (const __bf16*)dv, dvl,
                       (__bf16*)dz, dzl, (float*)ws, rows);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kv_prep_dw_kernel, dim3(kPrepD / 8), dim3(256), 0, stream,
                     (const float*)ws, blocks, dw);
  return hipGetLastError();
}

}  // namespace g4
