// Single-token Gated DeltaNet decode step for gfx950, f32 state updated in place.
//
// Semantics follow the reference gated-delta-rule step (breezetoken/backends.py:
// 242-271, the contract of Backend.gdn_decode; kernel kernels/cuda/gdn.py:31-139).
// For value head h, reading key/query head kh = h % heads_k:
//   qn = q[kh] * rsqrt(sum(q[kh]^2) + eps) * scale,  kn = k[kh] * rsqrt(sum(k[kh]^2) + eps)
//   decayed[i][j] = state[h][i][j] * exp(g[h])                  (i: key dim, j: value dim)
//   recall[j]     = sum_i decayed[i][j] * kn[i]
//   delta[j]      = (v[h][j] - recall[j]) * sigmoid(beta[h])
//   state[h][i][j] = decayed[i][j] + kn[i] * delta[j]
//   out[h][j]     = sum_i state[h][i][j] * qn[i]
//
// MI355X layout: one 256-thread work-group per (value head, tile of TW value
// columns), so a head's state is spread over D/TW compute units instead of
// streaming through one.  Thread t owns the float4 column group c = t % (TW/4)
// of the tile and the row chunk r = t / (TW/4) of D*TW/1024 consecutive key
// rows, and keeps that part of the state in registers between the recall and
// the update, so the state is read once and written once with 16-byte
// accesses (each row segment of a wave covers TW contiguous floats).  The sums
// over key rows are reduced first inside the wave (lanes of one column group
// in different row chunks) and then across the four waves through LDS.  The
// q/k norms are folded by every wave from an LDS copy of the two rows.
#include "bt_common.h"
#include "bt_kernels.h"

namespace bt {

namespace {

template <int D, int TW>
struct GdnShape {
  static constexpr int kThreads = 256;
  static constexpr int kCols = TW / 4;                   // float4 column groups of the tile
  static constexpr int kRowCols = D / 4;                 // float4 groups of a whole state row
  static constexpr int kChunks = kThreads / kCols;       // row chunks
  static constexpr int kRows = D / kChunks;              // rows per thread
  static_assert(kCols <= 64 && 64 % kCols == 0, "a wave holds whole row chunks");
  static_assert(kRows >= 1 && D % kChunks == 0, "row chunks tile the key rows");
};

__device__ __forceinline__ float wave_sum_gdn(float x) { return wave_sum(x); }

__device__ __forceinline__ float4 add4(float4 a, float4 b) {
  return float4{a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w};
}

// Sum a per-thread float4 over the row chunks of a column group: first across
// the row chunks inside the wave (lane distance kCols, 2*kCols, ...), then
// across the waves through LDS.  Every thread returns the total of its group.
template <typename S>
__device__ __forceinline__ float4 sum_over_rows(float4 v, float4* red) {
  v.x = sum_from<S::kCols>(v.x);
  v.y = sum_from<S::kCols>(v.y);
  v.z = sum_from<S::kCols>(v.z);
  v.w = sum_from<S::kCols>(v.w);
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  if (lane < S::kCols) red[wave * S::kCols + lane] = v;
  __syncthreads();
  const int c = t % S::kCols;
  float4 s = red[c];
#pragma unroll
  for (int w = 1; w < 4; ++w) s = add4(s, red[w * S::kCols + c]);
  __syncthreads();  // red is reused by the next reduction
  return s;
}

}  // namespace

template <int D, int TW>
__global__ __launch_bounds__(256) void gdn_decode_kernel(GdnParams p) {
  using S = GdnShape<D, TW>;
  __shared__ float qs[D];
  __shared__ float ks[D];
  __shared__ float4 red[4 * S::kCols];
  const int h = blockIdx.x / (D / TW);
  const int tile = blockIdx.x % (D / TW);
  const int kh = h % p.heads_k;
  const int t = threadIdx.x;
  const int c = t % S::kCols;              // column group inside the tile
  const int cg = tile * S::kCols + c;      // column group inside the state row
  const int r0 = (t / S::kCols) * S::kRows;

  // q/k rows of the key head, L2-normalised (q also scaled).
  for (int i = t; i < D; i += S::kThreads) {
    qs[i] = p.q[(int64_t)kh * D + i];
    ks[i] = p.k[(int64_t)kh * D + i];
  }
  __syncthreads();
  float qq = 0.f, kk = 0.f;
  for (int i = t & 63; i < D; i += 64) {
    qq = fmaf(qs[i], qs[i], qq);
    kk = fmaf(ks[i], ks[i], kk);
  }
  qq = wave_sum_gdn(qq);
  kk = wave_sum_gdn(kk);
  const float q_gain = (1.0f / sqrtf(qq + p.eps)) * p.scale;
  const float k_gain = 1.0f / sqrtf(kk + p.eps);

  const float decay = expf(p.g[h]);
  const float beta = 1.0f / (1.0f + expf(-p.beta[h]));

  // Recall: decayed state . kn over this thread's rows.
  float4* st = reinterpret_cast<float4*>(p.state + (int64_t)h * D * D);
  float4 s[S::kRows];
#pragma unroll
  for (int i = 0; i < S::kRows; ++i) s[i] = st[(int64_t)(r0 + i) * S::kRowCols + cg];
  float4 recall = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < S::kRows; ++i) {
    const float kn = ks[r0 + i] * k_gain;
    s[i] = float4{s[i].x * decay, s[i].y * decay, s[i].z * decay, s[i].w * decay};
    recall.x = fmaf(s[i].x, kn, recall.x);
    recall.y = fmaf(s[i].y, kn, recall.y);
    recall.z = fmaf(s[i].z, kn, recall.z);
    recall.w = fmaf(s[i].w, kn, recall.w);
  }
  recall = sum_over_rows<S>(recall, red);

  const float4 vv = reinterpret_cast<const float4*>(p.v + (int64_t)h * D)[cg];
  const float4 delta = {(vv.x - recall.x) * beta, (vv.y - recall.y) * beta, (vv.z - recall.z) * beta,
                        (vv.w - recall.w) * beta};

  // Update, write back, and read out with qn.
  float4 out = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < S::kRows; ++i) {
    const float kn = ks[r0 + i] * k_gain;
    const float qn = qs[r0 + i] * q_gain;
    s[i] = float4{fmaf(kn, delta.x, s[i].x), fmaf(kn, delta.y, s[i].y), fmaf(kn, delta.z, s[i].z),
                  fmaf(kn, delta.w, s[i].w)};
    st[(int64_t)(r0 + i) * S::kRowCols + cg] = s[i];
    out.x = fmaf(s[i].x, qn, out.x);
    out.y = fmaf(s[i].y, qn, out.y);
    out.z = fmaf(s[i].z, qn, out.z);
    out.w = fmaf(s[i].w, qn, out.w);
  }
  out = sum_over_rows<S>(out, red);
  if (t < S::kCols) reinterpret_cast<float4*>(p.out + (int64_t)h * D)[tile * S::kCols + t] = out;
}

hipError_t launch_gdn_decode(const GdnParams& p, int dim, hipStream_t stream) {
  switch (dim) {
    case 64:
      hipLaunchKernelGGL((gdn_decode_kernel<64, 16>), dim3(p.heads_v * 4), dim3(256), 0, stream, p);
      break;
    case 128:
      hipLaunchKernelGGL((gdn_decode_kernel<128, 32>), dim3(p.heads_v * 4), dim3(256), 0, stream, p);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace bt
