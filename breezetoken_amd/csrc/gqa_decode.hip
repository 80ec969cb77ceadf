// Split-KV GQA flash-decode for gfx950 (MI355X) over a bf16 token-major KV cache.
//
// Semantics follow the reference split kernel (breezetoken/kernels/cuda/
// attention.py:88-166, fixed-capacity variant 249-326): the valid context of a
// sequence is cut into 32-token tiles, split s of NS owns tiles
// [s*base + min(s, extra), +base + (s < extra)) (attention.py:106-112), and each
// split writes, per query head, a log2-domain LSE
//     lse = log2(l) + m,   l = sum_j exp2(x_j - m),   x_j = q.k_j * scale * log2e
// and the normalised partial output sum_j exp2(x_j - m) v_j / l.  An empty split
// writes lse = -inf and leaves its partial untouched (the combine never reads it).
//
// Work decomposition (MI355X-first, not the reference's):
//  * one work-group (4 waves) per (split, kv head, sequence); the group's G query
//    heads ride in the N dimension of v_mfma_f32_16x16x32_bf16, so every K/V byte
//    fetched from HBM is used by all G heads;
//  * q is pre-scaled by scale*log2e and split into bf16 hi + lo columns (columns
//    h and 2*GMAX-1-h), so Q.K^T keeps ~16 mantissa bits although the MFMA takes
//    bf16; the two halves are summed with one DPP mirror.  P is split the same
//    way for the P.V product;
//  * S^T = K . Q^T puts the K tile in the A operand, so K rows go straight from
//    HBM into registers with 16-byte loads (64 contiguous bytes per token per
//    instruction);
//  * V is staged through an XOR-swizzled LDS tile per wave and read back with
//    ds_read_b64_tr_b16, which yields the V^T operand of O^T = V^T . P^T without
//    any shuffle; the lane that owns score column n for tokens t also owns the
//    P^T operand for exactly those tokens, so P never moves between lanes;
//  * waves of a work-group take tiles round-robin, keep private online-softmax
//    state and merge once through LDS at the end, so one partial per (head, split)
//    reaches HBM;
//  * the valid length comes from a device position tensor (valid = pos + 1) or a
//    device length table, so the launch shape never depends on host data and the
//    whole call can be captured in a hipGraph.
#include "bt_common.h"
#include "bt_kernels.h"

namespace bt {

namespace {

constexpr int kTile = 32;      // tokens per tile (the P.V MFMA's K dimension)
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;

__device__ __forceinline__ int swz(int row, int slots) { return ((row & 7) * 2) & (slots - 1); }

template <int GMAX, int D>
struct DecodeTile {
  static constexpr int kSteps = D / 32;      // K-dimension steps of Q.K^T
  static constexpr int kDTiles = D / 16;     // 16-wide d tiles of O^T
  static constexpr int kSlots = D / 8;       // 16-byte chunks per row
  static constexpr int kVLoads = D / 16;     // 1 KiB wave loads per V tile
  static constexpr int kRowBytes = D * 2;
  static constexpr int kVTileBytes = kTile * kRowBytes;
};

template <int GMAX, int D>
__global__ __launch_bounds__(kThreads, 1) void gqa_decode_split_kernel(DecodeSplitParams p) {
  using T = DecodeTile<GMAX, D>;
  constexpr int kSteps = T::kSteps;
  constexpr int kDTiles = T::kDTiles;
  constexpr int kSlots = T::kSlots;
  constexpr int kVLoads = T::kVLoads;
  constexpr int kRowBytes = T::kRowBytes;

  // LDS: one V tile per wave; reused for the cross-wave merge at the end.
  constexpr int kMergeBytes = kWaves * GMAX * (D + 2) * 4;
  constexpr int kVBytes = kWaves * T::kVTileBytes;
  constexpr int kLdsBytes = kVBytes > kMergeBytes ? kVBytes : kMergeBytes;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[kLdsBytes];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int kvh = blockIdx.y;
  const int G = p.heads / p.kv_heads;

  int b, s, ns, base;
  if (p.work != nullptr) {
    const int4 w = p.work[blockIdx.x];
    b = w.x; s = w.y; ns = w.z; base = w.w;
  } else {
    b = blockIdx.z; s = blockIdx.x; ns = p.num_split; base = b * p.num_split;
  }

  int valid;
  if (p.pos != nullptr) valid = p.pos[b] + 1;
  else if (p.seq_len != nullptr) valid = p.seq_len[b];
  else valid = p.seqlen;
  if (valid < 0) valid = 0;
  const int64_t seq_off = p.seq_offset != nullptr ? p.seq_offset[b] : 0;

  // Split partition (attention.py:106-112).
  const int tiles = (valid + kTile - 1) / kTile;
  const int tbase = tiles / ns, extra = tiles % ns;
  const int n_tiles = tbase + (s < extra ? 1 : 0);
  const int tile0 = s * tbase + (s < extra ? s : extra);

  const int head0 = kvh * G;
  const int split_idx = base + s;

  if (n_tiles == 0) {
    if (threadIdx.x < G) p.lse[(int64_t)(head0 + threadIdx.x) * p.total_splits + split_idx] = -INFINITY;
    return;
  }

  // ---- column roles: hi column h < G, lo column 2*GMAX-1-h ----------------
  const int col = lane & 15;
  const int kg = lane >> 4;
  int col_head = -1;
  bool col_lo = false;
  if (col < G) {
    col_head = col;
  } else if (col >= 2 * GMAX - G && col < 2 * GMAX) {
    col_head = 2 * GMAX - 1 - col;
    col_lo = true;
  }

  // ---- Q^T operand: bf16 hi or lo of q*scale*log2e ------------------------
  bf16x8 qop[kSteps];
  {
    const int64_t qrow = (int64_t)b * p.q_stride_seq + (int64_t)(head0 + (col_head < 0 ? 0 : col_head)) * D;
#pragma unroll
    for (int st = 0; st < kSteps; ++st) {
      const int d0 = (st * 4 + kg) * 8;
      float qv[8];
      if (p.q_bf16) {
        const u32x4 raw = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(p.q) + qrow + d0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          qv[2 * i] = bf16_bits_to_f32(raw[i] & 0xffffu);
          qv[2 * i + 1] = bf16_bits_to_f32(raw[i] >> 16);
        }
      } else {
        const float4 a = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p.q) + qrow + d0);
        const float4 c = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p.q) + qrow + d0 + 4);
        qv[0] = a.x; qv[1] = a.y; qv[2] = a.z; qv[3] = a.w;
        qv[4] = c.x; qv[5] = c.y; qv[6] = c.z; qv[7] = c.w;
      }
      uint32_t h16[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float x = qv[i] * p.scale_log2;
        const uint32_t hi = f32_to_bf16_bits(x);
        const uint32_t lo = f32_to_bf16_bits(x - bf16_bits_to_f32(hi));
        h16[i] = col_head < 0 ? 0u : (col_lo ? lo : hi);
      }
      const u32x4 packed = {pack2(h16[0], h16[1]), pack2(h16[2], h16[3]), pack2(h16[4], h16[5]),
                            pack2(h16[6], h16[7])};
      qop[st] = as_bf16x8(packed);
    }
  }

  // ---- per-wave state -------------------------------------------------------
  floatx4 oacc[kDTiles];
#pragma unroll
  for (int i = 0; i < kDTiles; ++i) oacc[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;
  float l_run = 0.f;

  const uint16_t* kbase = p.k + seq_off * p.kv_stride_tok + (int64_t)kvh * p.kv_stride_head;
  const uint16_t* vbase = p.v + seq_off * p.kv_stride_tok + (int64_t)kvh * p.kv_stride_head;
  unsigned char* vtile = smem + wave * T::kVTileBytes;
  const int last = valid - 1;

  auto load_k = [&](int tile, u32x4 (&kr)[2][kSteps]) {
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      int t = tile * kTile + sub * 16 + col;
      t = t > last ? last : t;
      const uint16_t* row = kbase + (int64_t)t * p.kv_stride_tok + kg * 8;
#pragma unroll
      for (int st = 0; st < kSteps; ++st) kr[sub][st] = *reinterpret_cast<const u32x4*>(row + st * 32);
    }
  };
  auto load_v = [&](int tile, u32x4 (&vr)[kVLoads]) {
#pragma unroll
    for (int j = 0; j < kVLoads; ++j) {
      const int pbyte = j * 1024 + lane * 16;
      const int r = pbyte / kRowBytes;
      const int slot = (pbyte % kRowBytes) / 16;
      const int c = slot ^ swz(r, kSlots);
      int t = tile * kTile + r;
      t = t > last ? last : t;
      vr[j] = *reinterpret_cast<const u32x4*>(vbase + (int64_t)t * p.kv_stride_tok + c * 8);
    }
  };

  auto compute = [&](int tile, bool has_next, u32x4 (&kr)[2][kSteps], u32x4 (&vr)[kVLoads]) {
    // S^T = K . Q^T for two 16-token sub-tiles.
    floatx4 sacc[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int st = 0; st < kSteps; ++st) {
      sacc[0] = mfma16(as_bf16x8(kr[0][st]), qop[st], sacc[0]);
      sacc[1] = mfma16(as_bf16x8(kr[1][st]), qop[st], sacc[1]);
    }
    // K registers are free again: start fetching the next tile's K.
    if (has_next) load_k(tile + kWaves, kr);
    // Stage V into this wave's swizzled LDS tile (same-wave LDS ops stay ordered),
    // then reuse the V registers for the next tile's V.
#pragma unroll
    for (int j = 0; j < kVLoads; ++j)
      *reinterpret_cast<BT_LDS u32x4*>((BT_LDS unsigned char*)vtile + j * 1024 + lane * 16) = vr[j];
    if (has_next) load_v(tile + kWaves, vr);

    // hi + lo columns, mask, online softmax (attention.py:21-51 semantics).
    float x[8];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float v = sacc[sub][j];
        v += (GMAX <= 4) ? dpp_f32<DPP_ROW_HALF_MIRROR>(v) : dpp_f32<DPP_ROW_MIRROR>(v);
        const int t = tile * kTile + sub * 16 + kg * 4 + j;
        x[sub * 4 + j] = t < valid ? v : -INFINITY;
      }
    }
    float tmax = x[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) tmax = fmaxf(tmax, x[i]);
    tmax = wave_max_xor(tmax, 16);
    tmax = wave_max_xor(tmax, 32);
    const float m_new = fmaxf(m_run, tmax);
    float alpha, pr[8];
    if (m_new == -INFINITY) {
      alpha = 1.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) pr[i] = 0.f;
    } else {
      alpha = fast_exp2(m_run - m_new);
#pragma unroll
      for (int i = 0; i < 8; ++i) pr[i] = fast_exp2(x[i] - m_new);
    }
    m_run = m_new;
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) psum += pr[i];
    l_run = l_run * alpha + psum;
#pragma unroll
    for (int i = 0; i < kDTiles; ++i) oacc[i] *= alpha;

    // P^T operand: this lane's own 8 probabilities, as bf16 hi or lo.
    uint32_t p16[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t hi = f32_to_bf16_bits(pr[i]);
      const uint32_t lo = f32_to_bf16_bits(pr[i] - bf16_bits_to_f32(hi));
      p16[i] = col_head < 0 ? 0u : (col_lo ? lo : hi);
    }
    const u32x4 ppk = {pack2(p16[0], p16[1]), pack2(p16[2], p16[3]), pack2(p16[4], p16[5]),
                       pack2(p16[6], p16[7])};
    const bf16x8 pop = as_bf16x8(ppk);

    // O^T += V^T . P^T, V^T read transposed from LDS.
    const int i16 = lane & 15;
    const int row1 = 4 * kg + (i16 >> 2);
    const int row2 = row1 + 16;
#pragma unroll
    for (int dt = 0; dt < kDTiles; ++dt) {
      const int c = dt * 2 + ((i16 & 3) >> 1);
      const int off = (i16 & 1) * 8;
      const BT_LDS uint16_t* p0 = (const BT_LDS uint16_t*)((BT_LDS unsigned char*)vtile + row1 * kRowBytes +
                                                          ((c ^ swz(row1, kSlots)) * 16) + off);
      const BT_LDS uint16_t* p1 = (const BT_LDS uint16_t*)((BT_LDS unsigned char*)vtile + row2 * kRowBytes +
                                                          ((c ^ swz(row2, kSlots)) * 16) + off);
      oacc[dt] = mfma16(lds_read_tr_pair(p0, p1), pop, oacc[dt]);
    }
  };

  // ---- tile loop: wave w takes local tiles w, w+4, ...; the next tile's loads
  // are issued as soon as the current tile's registers have been consumed.
  const int my_tiles = n_tiles > wave ? (n_tiles - wave + kWaves - 1) / kWaves : 0;
  if (my_tiles > 0) {
    u32x4 kr[2][kSteps];
    u32x4 vr[kVLoads];
    load_k(tile0 + wave, kr);
    load_v(tile0 + wave, vr);
    for (int it = 0; it < my_tiles; ++it)
      compute(tile0 + wave + it * kWaves, it + 1 < my_tiles, kr, vr);
  }

  // ---- wave epilogue: full row sums, hi + lo merge ---------------------------
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
#pragma unroll
  for (int dt = 0; dt < kDTiles; ++dt) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float v = oacc[dt][j];
      oacc[dt][j] = v + ((GMAX <= 4) ? dpp_f32<DPP_ROW_HALF_MIRROR>(v) : dpp_f32<DPP_ROW_MIRROR>(v));
    }
  }

  // ---- cross-wave merge through LDS ----------------------------------------
  __syncthreads();  // every wave is done with its V tile
  float* mo = reinterpret_cast<float*>(smem);              // [wave][GMAX][D]
  float* mm = mo + kWaves * GMAX * D;                       // [wave][GMAX]
  float* ml = mm + kWaves * GMAX;                           // [wave][GMAX]
  if (col < G && !col_lo) {
    float* dst = mo + (wave * GMAX + col) * D;
#pragma unroll
    for (int dt = 0; dt < kDTiles; ++dt) {
      float4 v4 = {oacc[dt][0], oacc[dt][1], oacc[dt][2], oacc[dt][3]};
      *reinterpret_cast<float4*>(dst + dt * 16 + kg * 4) = v4;
    }
    if (kg == 0) {
      mm[wave * GMAX + col] = m_run;
      ml[wave * GMAX + col] = l_run;
    }
  }
  __syncthreads();

  // Each thread finishes (head, 4 consecutive d) items.
  for (int item = threadIdx.x; item < G * (D / 4); item += kThreads) {
    const int h = item / (D / 4);
    const int d = (item % (D / 4)) * 4;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mx = fmaxf(mx, mm[w * GMAX + h]);
    float lsum = 0.f;
    float4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float lw = ml[w * GMAX + h];
      if (lw > 0.f) {
        const float sc = fast_exp2(mm[w * GMAX + h] - mx);
        lsum += lw * sc;
        const float4 o = *reinterpret_cast<const float4*>(mo + (w * GMAX + h) * D + d);
        acc.x += o.x * sc; acc.y += o.y * sc; acc.z += o.z * sc; acc.w += o.w * sc;
      }
    }
    const int64_t row = (int64_t)(head0 + h) * p.total_splits + split_idx;
    if (lsum > 0.f) {
      const float inv = 1.f / lsum;
      acc.x *= inv; acc.y *= inv; acc.z *= inv; acc.w *= inv;
      *reinterpret_cast<float4*>(p.part + row * D + d) = acc;
      if (d == 0) p.lse[row] = fast_log2(lsum) + mx;
    } else if (d == 0) {
      p.lse[row] = -INFINITY;
    }
  }
}

// LSE combine (attention.py:168-189): one work-group per (head, sequence).
template <int D>
__global__ __launch_bounds__(256) void gqa_decode_combine_kernel(CombineParams p) {
  __shared__ float wts[kMaxSplitsPerSeq];
  __shared__ float red[256];
  __shared__ float4 accs[256];
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  int base, ns;
  if (p.split_base != nullptr) {
    base = p.split_base[b];
    ns = p.split_count[b];
  } else {
    base = b * p.num_split;
    ns = p.num_split;
  }
  const float* lse = p.lse + (int64_t)h * p.total_splits + base;

  float mx = -INFINITY;
  for (int i = threadIdx.x; i < ns; i += 256) mx = fmaxf(mx, lse[i]);
  red[threadIdx.x] = mx;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (threadIdx.x < o) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + o]);
    __syncthreads();
  }
  mx = red[0];
  __syncthreads();
  float sum = 0.f;
  for (int i = threadIdx.x; i < ns; i += 256) {
    const float v = lse[i];
    const float e = v == -INFINITY ? 0.f : fast_exp2(v - mx);
    wts[i] = e;
    sum += e;
  }
  red[threadIdx.x] = sum;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  sum = red[0];
  const float inv = sum > 0.f ? 1.f / sum : 0.f;

  // out[d] = sum_s w_s part_s[d] / sum: 4 split groups x (D/4) float4 columns.
  constexpr int kCols = D / 4;
  const int grp = threadIdx.x / kCols;
  const int cidx = threadIdx.x % kCols;
  constexpr int kGroups = 256 / kCols;
  float4 acc = {0.f, 0.f, 0.f, 0.f};
  const float* part = p.part + ((int64_t)h * p.total_splits + base) * D + cidx * 4;
  for (int s = grp; s < ns; s += kGroups) {
    const float w = wts[s];
    if (w != 0.f) {
      const float4 v = *reinterpret_cast<const float4*>(part + (int64_t)s * D);
      acc.x += w * v.x; acc.y += w * v.y; acc.z += w * v.z; acc.w += w * v.w;
    }
  }
  if (kGroups > 1) {
    accs[threadIdx.x] = acc;
    __syncthreads();
    if (grp == 0) {
      for (int g2 = 1; g2 < kGroups; ++g2) {
        const float4 o = accs[g2 * kCols + cidx];
        acc.x += o.x; acc.y += o.y; acc.z += o.z; acc.w += o.w;
      }
    }
  }
  if (grp == 0) {
    acc.x *= inv; acc.y *= inv; acc.z *= inv; acc.w *= inv;
    const int64_t orow = (int64_t)b * p.out_stride_seq + (int64_t)h * D + cidx * 4;
    if (p.out_bf16) {
      uint16_t* o = reinterpret_cast<uint16_t*>(p.out) + orow;
      const u32x2 pk = {pack2(f32_to_bf16_bits(acc.x), f32_to_bf16_bits(acc.y)),
                        pack2(f32_to_bf16_bits(acc.z), f32_to_bf16_bits(acc.w))};
      *reinterpret_cast<u32x2*>(o) = pk;
    } else {
      *reinterpret_cast<float4*>(reinterpret_cast<float*>(p.out) + orow) = acc;
    }
  }
}

}  // namespace

template <int GMAX, int D>
static hipError_t launch_split_t(const DecodeSplitParams& p, int grid_x, int batch, hipStream_t stream) {
  dim3 grid(grid_x, p.kv_heads, batch);
  hipLaunchKernelGGL((gqa_decode_split_kernel<GMAX, D>), grid, dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_decode_split(const DecodeSplitParams& p, int head_dim, int grid_x, int batch,
                               hipStream_t stream) {
  const int G = p.heads / p.kv_heads;
  const bool small = G <= 4;
  switch (head_dim) {
    case 64: return small ? launch_split_t<4, 64>(p, grid_x, batch, stream) : launch_split_t<8, 64>(p, grid_x, batch, stream);
    case 128: return small ? launch_split_t<4, 128>(p, grid_x, batch, stream) : launch_split_t<8, 128>(p, grid_x, batch, stream);
    case 256: return small ? launch_split_t<4, 256>(p, grid_x, batch, stream) : launch_split_t<8, 256>(p, grid_x, batch, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_decode_combine(const CombineParams& p, int head_dim, int heads, int batch,
                                 hipStream_t stream) {
  dim3 grid(heads, batch);
  switch (head_dim) {
    case 64: hipLaunchKernelGGL(gqa_decode_combine_kernel<64>, grid, dim3(256), 0, stream, p); break;
    case 128: hipLaunchKernelGGL(gqa_decode_combine_kernel<128>, grid, dim3(256), 0, stream, p); break;
    case 256: hipLaunchKernelGGL(gqa_decode_combine_kernel<256>, grid, dim3(256), 0, stream, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace bt
