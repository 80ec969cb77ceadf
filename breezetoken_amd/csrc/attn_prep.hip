// Per-head RMSNorm + partial rotate-half RoPE for gfx950, and the fused
// decode-step preparation that feeds the split-KV attention.
//
// Semantics follow the reference operators:
//   rms_norm(x, w, eps) = x * rsqrt(mean(x^2) + eps) * w          (backends.py:187-189)
//   rope(x, cos, sin, pos, rope_dim): the first rope_dim dims turn as
//     y[d] = x[d] * cos[pos][d] + sign(d) * x[partner(d)] * sin[pos][d],
//     partner(d) = d + rope_dim/2 (sign -1) below the half, d - rope_dim/2 (sign +1)
//     above it; the remaining dims pass through                   (backends.py:218-226,
//                                                                  kernels/cuda/rope.py:13-43)
// and the decode step of an attention layer (layers.py:56-73, graph.py:35-53):
//   q = rope(rms_norm(q, q_norm)), k = rope(rms_norm(k, k_norm)), cache.k[pos] = k,
//   cache.v[pos] = v, with q, gate, k, v sliced from the fused projection output
//   [H x (q | gate) | Hkv x k | Hkv x v] (layers.py:58-64).
//
// MI355X layout: one 64-lane wave per row (a q head, or a kv head whose wave
// also converts the head's v row), lane l holding D/64 consecutive values, so
// the mean of squares is one wave reduction.  The rotation reads each value's
// partner from a copy of the normalised row in LDS.  The decode position is a device int32 read through
// the scalar cache, so the fused step is one launch that a hipGraph can
// capture in place of the reference's four norm/rope launches and two cache
// copies.  Products and sums of the rotation use explicitly rounded operations
// (no fused multiply-add) so they round like the reference's separate tensor
// operations.
#include "bt_common.h"
#include "bt_kernels.h"

namespace bt {

namespace {

template <typename T>
__device__ __forceinline__ T uniform_load_prep(const T* p) {
  return ((const __attribute__((address_space(4))) T*)(p))[0];
}

__device__ __forceinline__ float wave_sum_prep(float x) { return wave_sum(x); }

// Normalise and rotate the D values a wave holds (lane l: d = l*E .. l*E+E-1).
template <int D>
__device__ __forceinline__ void norm_rope_row(float (&x)[D / 64], const float* w, float eps,
                                              const float* cos_row, const float* sin_row,
                                              int rope_dim, float* lds) {
  constexpr int E = D / 64;
  const int lane = threadIdx.x;
  if (w != nullptr) {
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) ss = fmaf(x[e], x[e], ss);
    ss = wave_sum_prep(ss);
    const float r = 1.0f / sqrtf(ss / (float)D + eps);
#pragma unroll
    for (int e = 0; e < E; ++e) x[e] = __fmul_rn(__fmul_rn(x[e], r), w[lane * E + e]);
  }
  if (cos_row != nullptr) {
#pragma unroll
    for (int e = 0; e < E; ++e) lds[lane * E + e] = x[e];
    __syncthreads();  // one wave per work-group: orders the stores before the partner reads
    const int half = rope_dim >> 1;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int d = lane * E + e;
      if (d < rope_dim) {
        const bool lo = d < half;
        const float partner = lds[lo ? d + half : d - half];
        const float turned = lo ? -partner : partner;
        x[e] = __fadd_rn(__fmul_rn(x[e], cos_row[d]), __fmul_rn(turned, sin_row[d]));
      }
    }
  }
}

template <int D>
__device__ __forceinline__ void load_row(float (&x)[D / 64], const float* src) {
  constexpr int E = D / 64;
#pragma unroll
  for (int e = 0; e < E; ++e) x[e] = src[threadIdx.x * E + e];
}

template <int D>
__device__ __forceinline__ void store_bf16_row(uint16_t* dst, const float (&x)[D / 64]) {
  constexpr int E = D / 64;
#pragma unroll
  for (int e = 0; e < E; ++e) dst[threadIdx.x * E + e] = (uint16_t)f32_to_bf16_bits(x[e]);
}

}  // namespace

// Rows of x (rows, D) -> out (rows, D), both f32: RMSNorm when w is set, then
// RoPE at the device position when cos/sin are set (the reference's
// Backend.rms_norm and Backend.rope on a (rows, D) view).
template <int D>
__global__ __launch_bounds__(64) void row_norm_rope_kernel(RowPrepParams p) {
  __shared__ float lds[D];
  constexpr int E = D / 64;
  const int row = blockIdx.x;
  const float* cos_row = nullptr;
  const float* sin_row = nullptr;
  if (p.cos != nullptr) {
    int pr = uniform_load_prep(p.pos);
    pr = pr < 0 ? 0 : (pr >= p.rope_cap ? p.rope_cap - 1 : pr);
    cos_row = p.cos + (int64_t)pr * p.rope_dim;
    sin_row = p.sin + (int64_t)pr * p.rope_dim;
  }
  float x[E];
  load_row<D>(x, p.x + (int64_t)row * p.x_stride);
  norm_rope_row<D>(x, p.w, p.eps, cos_row, sin_row, p.rope_dim, lds);
  float* dst = p.out + (int64_t)row * p.out_stride;
#pragma unroll
  for (int e = 0; e < E; ++e) dst[threadIdx.x * E + e] = x[e];
}

// Fused decode-step preparation: waves 0..H-1 produce the rotated, normalised
// q heads; wave H+g normalises and rotates k head g into the bf16 cache at the
// device position and converts v head g beside it.
template <int D>
__global__ __launch_bounds__(64) void attn_prep_kernel(RowPrepParams p) {
  __shared__ float lds[D];
  constexpr int E = D / 64;
  const int row = blockIdx.x;
  const int pos = uniform_load_prep(p.pos);
  const float* cos_row = nullptr;
  const float* sin_row = nullptr;
  if (p.cos != nullptr) {
    const int pr = pos < 0 ? 0 : (pos >= p.rope_cap ? p.rope_cap - 1 : pos);
    cos_row = p.cos + (int64_t)pr * p.rope_dim;
    sin_row = p.sin + (int64_t)pr * p.rope_dim;
  }
  float x[E];
  if (row < p.heads) {
    load_row<D>(x, p.x + (int64_t)row * 2 * D);  // q part of head row's (q | gate)
    norm_rope_row<D>(x, p.w, p.eps, cos_row, sin_row, p.rope_dim, lds);
    if (p.q_out_bf16) {
      store_bf16_row<D>(reinterpret_cast<uint16_t*>(p.q_out) + (int64_t)row * D, x);
    } else {
      float* dst = reinterpret_cast<float*>(p.q_out) + (int64_t)row * D;
#pragma unroll
      for (int e = 0; e < E; ++e) dst[threadIdx.x * E + e] = x[e];
    }
    return;
  }
  const int g = row - p.heads;
  const float* kv = p.x + (int64_t)p.heads * 2 * D;
  load_row<D>(x, kv + (int64_t)g * D);
  norm_rope_row<D>(x, p.wk, p.eps, cos_row, sin_row, p.rope_dim, lds);
  // Slots outside the cache are not written (the position is a device value
  // the host cannot check; the attention kernels clamp it the same way).
  if (pos < 0 || pos >= p.cache_cap) return;
  const int64_t slot = (int64_t)pos * p.kv_stride_tok + (int64_t)g * p.kv_stride_head;
  store_bf16_row<D>(p.cache_k + slot, x);
  load_row<D>(x, kv + (int64_t)(p.kv_heads + g) * D);
  store_bf16_row<D>(p.cache_v + slot, x);
}

hipError_t launch_row_norm_rope(const RowPrepParams& p, int head_dim, hipStream_t stream) {
  switch (head_dim) {
    case 64: hipLaunchKernelGGL(row_norm_rope_kernel<64>, dim3(p.rows), dim3(64), 0, stream, p); break;
    case 128: hipLaunchKernelGGL(row_norm_rope_kernel<128>, dim3(p.rows), dim3(64), 0, stream, p); break;
    case 256: hipLaunchKernelGGL(row_norm_rope_kernel<256>, dim3(p.rows), dim3(64), 0, stream, p); break;
    case 512: hipLaunchKernelGGL(row_norm_rope_kernel<512>, dim3(p.rows), dim3(64), 0, stream, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_attn_prep(const RowPrepParams& p, int head_dim, hipStream_t stream) {
  const dim3 grid(p.heads + p.kv_heads);
  switch (head_dim) {
    case 64: hipLaunchKernelGGL(attn_prep_kernel<64>, grid, dim3(64), 0, stream, p); break;
    case 128: hipLaunchKernelGGL(attn_prep_kernel<128>, grid, dim3(64), 0, stream, p); break;
    case 256: hipLaunchKernelGGL(attn_prep_kernel<256>, grid, dim3(64), 0, stream, p); break;
    case 512: hipLaunchKernelGGL(attn_prep_kernel<512>, grid, dim3(64), 0, stream, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace bt
