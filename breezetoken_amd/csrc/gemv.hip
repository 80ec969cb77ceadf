// Decode matvec y = x . W for gfx950: x (K,) f32, W (K, N) bf16 row-major,
// y (N,) f32.
//
// Semantics follow Backend.linear (breezetoken/backends.py:36-37; torch form
// _torch_linear 182-184: x.float() @ w.float()) as served by the reference's
// split-K bf16 GEMV (kernels/cuda/gemv.py:18-40, selected by _CudaGemv,
// backends.py:303-333): partial sums over SK shares of K, then their sum.
// One deliberate difference: x stays f32 (the reference kernel rounds it to
// bf16 first), so the result is closer to the f32 definition.
//
// MI355X layout: a work-group of 4 waves owns a tile of 64*VEC columns (VEC
// consecutive bf16 per lane: one 16- or 8-byte load per row) over one share of
// K; wave w takes rows k0 + w, k0 + w + 4, ... and keeps ROWS rows of loads in
// flight (16 when that covers a whole share of 61..64 rows in one round trip,
// else 8), so every byte of W is streamed once with non-temporal
// buffer loads (rows are contiguous segments of 64*VEC*2 bytes; the buffer
// range check turns loads past the matrix into zeros).  x[k] is wave-uniform
// and read through the scalar cache.  The four waves' accumulators are summed
// through LDS.  With SK > 1 each share writes a partial row and a second,
// small kernel adds the shares in order, so the result is deterministic.  (A
// one-launch variant in which the last share to arrive adds the others needs
// a device-scope release per work-group, which writes back the L2 each time:
// measured 4x slower on the vocabulary head.)
#include "bt_common.h"
#include "bt_kernels.h"

namespace bt {

namespace {

constexpr int kGemvWaves = 4;

template <typename T>
__device__ __forceinline__ T uniform_load_gemv(const T* p, int i) {
  return ((const __attribute__((address_space(4))) T*)(p))[i];
}

template <int VEC>
struct GemvLoad;
template <>
struct GemvLoad<8> {
  typedef u32x4 type;
  static __device__ __forceinline__ type load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 2 /* nt */);
  }
};
template <>
struct GemvLoad<4> {
  typedef u32x2 type;
  static __device__ __forceinline__ type load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 2 /* nt */);
  }
};

template <int VEC>
__device__ __forceinline__ void fma_row(float (&acc)[VEC], const typename GemvLoad<VEC>::type& w, float x) {
#pragma unroll
  for (int i = 0; i < VEC / 2; ++i) {
    const uint32_t pair = w[i];
    acc[2 * i] = fmaf(x, bf16_bits_to_f32(pair & 0xffffu), acc[2 * i]);
    acc[2 * i + 1] = fmaf(x, bf16_bits_to_f32(pair >> 16), acc[2 * i + 1]);
  }
}

}  // namespace

template <int VEC, int ROWS>
__global__ __launch_bounds__(256) void gemv_bf16_kernel(GemvParams p) {
  constexpr int kTile = 64 * VEC;
  __shared__ float red[kGemvWaves][kTile];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tile = blockIdx.x;
  const int s = blockIdx.y;
  const int k_per = (p.K + p.splits - 1) / p.splits;
  const int k0 = s * k_per;
  const int k1 = min(p.K, k0 + k_per);
  const int n0 = tile * kTile + lane * VEC;

  // K * ldw * 2 < 2^31 is checked on the host.
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(p.w), (short)0, (int)(p.K * p.ldw * 2), 0x00020000);
  const uint32_t col_off = (uint32_t)n0 * 2;
  float acc[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) acc[i] = 0.f;

  // Rows k0 + wave + 4*j; ROWS loads in flight per pass.
  int k = k0 + wave;
  for (; k + kGemvWaves * (ROWS - 1) < k1; k += kGemvWaves * ROWS) {
    typename GemvLoad<VEC>::type wv[ROWS];
#pragma unroll
    for (int j = 0; j < ROWS; ++j)
      wv[j] = GemvLoad<VEC>::load(wrs, (uint32_t)((k + kGemvWaves * j) * p.ldw) * 2 + col_off);
#pragma unroll
    for (int j = 0; j < ROWS; ++j) fma_row<VEC>(acc, wv[j], uniform_load_gemv(p.x, k + kGemvWaves * j));
  }
  for (; k < k1; k += kGemvWaves) {
    const typename GemvLoad<VEC>::type wv = GemvLoad<VEC>::load(wrs, (uint32_t)(k * p.ldw) * 2 + col_off);
    fma_row<VEC>(acc, wv, uniform_load_gemv(p.x, k));
  }

#pragma unroll
  for (int i = 0; i < VEC; ++i) red[wave][lane * VEC + i] = acc[i];
  __syncthreads();
  for (int c = threadIdx.x; c < kTile; c += 256) {
    const float v = (red[0][c] + red[1][c]) + (red[2][c] + red[3][c]);
    const int n = tile * kTile + c;
    if (n < p.N) {
      if (p.splits == 1) p.y[n] = v;
      else p.partial[(int64_t)s * p.N + n] = v;
    }
  }
}

// y[n] = sum over shares s = 0 .. SK-1 of partial[s][n], in that order.  The
// loads of BATCH shares are issued before their adds (one memory round trip
// for SK <= BATCH) without a branch per load: they go through a buffer
// descriptor that ends at the last share, so a load past it reads zero, and
// only the adds of the shares that exist are kept.  BATCH is the smallest of
// 8, 16, 32, 64 that holds SK (64 beyond): loads past the last share still
// cost issue time (BATCH 64 at SK = 16: +0.7 us).
template <int BATCH>
__global__ __launch_bounds__(256) void gemv_reduce_kernel(GemvParams p) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= p.N) return;
  // splits * N * 4 < 2^31 (at most ~1.5 MB for the shapes gemv_shape splits).
  const __amdgpu_buffer_rsrc_t prs =
      __builtin_amdgcn_make_buffer_rsrc(p.partial, (short)0, p.splits * p.N * 4, 0x00020000);
  const uint32_t share_bytes = (uint32_t)p.N * 4;
  float v = 0.f;
  for (int sh = 0; sh < p.splits; sh += BATCH) {
    const int cnt = min(BATCH, p.splits - sh);
    float t[BATCH];
#pragma unroll
    for (int j = 0; j < BATCH; ++j)
      t[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                           prs, (int)((uint32_t)(sh + j) * share_bytes + (uint32_t)n * 4), 0, 0));
#pragma unroll
    for (int j = 0; j < BATCH; ++j)
      if (j < cnt) v += t[j];
  }
  p.y[n] = v;
}

hipError_t launch_gemv(const GemvParams& p, int vec, hipStream_t stream) {
  const int tile = 64 * vec;
  const dim3 grid((p.N + tile - 1) / tile, p.splits);
  // A share of exactly 64 rows is one batch of 16 rows per wave (two batches
  // of 8 otherwise).  Other shares keep 8: in a share of 61..63 rows some
  // waves hold 15, miss the 16-row batch and would load them one at a time
  // while the work-group waits for them at the reduction.
  const int k_per = (p.K + p.splits - 1) / p.splits;
  const bool one_pass = k_per == kGemvWaves * 16;
  if (vec == 8 && one_pass) hipLaunchKernelGGL((gemv_bf16_kernel<8, 16>), grid, dim3(256), 0, stream, p);
  else if (vec == 8) hipLaunchKernelGGL((gemv_bf16_kernel<8, 8>), grid, dim3(256), 0, stream, p);
  else if (vec == 4 && one_pass) hipLaunchKernelGGL((gemv_bf16_kernel<4, 16>), grid, dim3(256), 0, stream, p);
  else if (vec == 4) hipLaunchKernelGGL((gemv_bf16_kernel<4, 8>), grid, dim3(256), 0, stream, p);
  else return hipErrorInvalidValue;
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.splits == 1) return e;
  const dim3 rgrid((p.N + 255) / 256);
  if (p.splits <= 8) hipLaunchKernelGGL(gemv_reduce_kernel<8>, rgrid, dim3(256), 0, stream, p);
  else if (p.splits <= 16) hipLaunchKernelGGL(gemv_reduce_kernel<16>, rgrid, dim3(256), 0, stream, p);
  else if (p.splits <= 32) hipLaunchKernelGGL(gemv_reduce_kernel<32>, rgrid, dim3(256), 0, stream, p);
  else hipLaunchKernelGGL(gemv_reduce_kernel<64>, rgrid, dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace bt
