// Causal GQA prefill attention for gfx950 (MI355X) on MFMA.
//
// Computes, for every query position i of a prompt that starts at slot 0 and
// every query head h (kv head g = h / G),
//     out[i, h] = softmax_j<=i (q_i . k_j * scale) . V_j
// -- the F.scaled_dot_product_attention(is_causal=True, enable_gqa=True) call
// of _prefill_attn (breezetoken/model/prefill.py:56-68).
//
// Decomposition (MI355X-first):
//  * one work-group (4 waves) per (block of query positions, kv head); wave w
//    owns query head w of the GQA group (and, for G < 4, a different block of
//    positions), so every K/V tile staged in LDS feeds all G heads;
//  * S^T = K . Q^T on v_mfma_f32_32x32x16_bf16: 64 keys x 32 queries per step,
//    K rows from an XOR-swizzled LDS tile, Q^T held in registers;
//  * O^T = V^T . P^T on v_mfma_f32_32x32x16_f16: V is converted to fp16 once
//    when it is staged in LDS (exact for |v| <= 65504, larger values saturate)
//    and read back with ds_read_b64_tr_b16; P (<= 2^8, see below) is rounded
//    to fp16 (11-bit mantissa; bf16's 8 bits would put the first rows of the
//    prompt above a 2e-3 error), and the lane that owns a score column owns the
//    P^T operand for it, so P never moves between lanes;
//  * online softmax in the log2 domain with lazy rescaling: the reference
//    maximum only moves (and O^T is only rescaled) when a score exceeds it by
//    more than 2^8, so most key blocks skip the 128-register rescale;
//  * software pipeline over 64-key blocks: iteration i stages K_{i+1} and V_i
//    into LDS and fetches K_{i+2} / V_{i+1} from HBM while multiplying
//    S_i = K_i . Q^T, then runs the softmax of S_i next to O += V_{i-1} . P_{i-1},
//    so matrix-core work always has independent VALU/LDS work beside it; every
//    buffer is rewritten only after the barrier that ends its last reader;
//  * heavy (late) query blocks are launched first to balance the causal work.
#include "bt_common.h"
#include "bt_kernels.h"

namespace bt {

namespace {

typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float2v __attribute__((ext_vector_type(2)));


constexpr int kQB = 32;      // query positions per wave
constexpr int kKB = 64;      // keys per step
constexpr int kWaves = 4;
constexpr float kLazy = 8.0f;  // log2-domain slack before the reference max moves

__device__ __forceinline__ floatx16 mfma32_f16(const u32x4& a, const u32x4& b, const floatx16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(halfx8, a), __builtin_bit_cast(halfx8, b),
                                                c, 0, 0, 0);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
}

// Two floats -> packed fp16 pair, round toward zero (bf16 values convert exactly;
// out-of-range magnitudes saturate to +-65504 instead of becoming inf).
__device__ __forceinline__ uint32_t pack_f16_rtz(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
}
// Two floats -> packed fp16 pair, round to nearest even (one v_cvt_pk_f16_f32).
__device__ __forceinline__ uint32_t pack_f16_rne(float a, float b) {
  uint32_t r;
  asm("v_cvt_pk_f16_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

__device__ __forceinline__ u32x4 bf16x8_to_f16x8(const u32x4& v) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    r[i] = pack_f16_rtz(__uint_as_float(v[i] << 16), __uint_as_float(v[i] & 0xffff0000u));
  return r;
}

}  // namespace

// D: head dim (128 or 256).  Wave w of a work-group handles query head
// (pass * 4 + w % GW) of the group and positions [q0 + (w / GW) * 32, +32),
// GW = min(G, 4); groups of 8 heads take two passes over the keys.
template <int D>
__global__ __launch_bounds__(kWaves * 64, 1) void gqa_prefill_kernel(PrefillParams p) {
  constexpr int kSteps = D / 16;       // K-dimension steps of Q.K^T (16 per MFMA)
  constexpr int kDTiles = D / 32;      // 32-wide d tiles of O^T
  constexpr int kRowBytes = D * 2;
  constexpr int kChunks = D / 8;       // 16-byte chunks per row
  constexpr int kTileBytes = kKB * kRowBytes;
  constexpr int kLoads = kTileBytes / (16 * kWaves * 64);  // 16-byte loads per thread per tile
  // Padded LDS rows instead of XOR swizzles, so every per-step offset is an
  // immediate: K rows step 16 B past a multiple of 256 B (16 consecutive rows hit
  // 16 different bank groups for 16-byte reads); V rows step 64 B (the 4 rows of
  // a transposed read land in 4 different 64-byte bank windows).
  constexpr int kKStride = kRowBytes + 16;
  constexpr int kVStride = kRowBytes + 64;
  constexpr int kKTile = kKB * kKStride;
  constexpr int kVTile = kKB * kVStride;
  constexpr int kBufBytes = kKTile + kVTile;

  __shared__ __attribute__((aligned(1024))) unsigned char smem[2 * kBufBytes];  // K0 V0 K1 V1

  asm volatile("" ::"s"(p.q), "s"(p.k), "s"(p.v), "s"(p.out), "s"(p.seqlen), "s"(p.group),
               "s"(p.q_stride_tok), "s"(p.q_stride_head), "s"(p.kv_stride_tok), "s"(p.kv_stride_head),
               "s"(p.out_stride_tok), "s"(p.out_stride_head), "s"(p.scale_log2));
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int kvh = blockIdx.y;
  const int G = p.group;
  const int GW = G < kWaves ? G : kWaves;
  const int pos_per_wg = kQB * (kWaves / GW);
  const int nqb = (p.seqlen + pos_per_wg - 1) / pos_per_wg;
  const int qblk = nqb - 1 - (int)blockIdx.x;  // heavy blocks first
  const int S = p.seqlen;
  const int wg_q0 = qblk * pos_per_wg;
  const int q0 = wg_q0 + (wave / GW) * kQB;   // this wave's first position
  const int wg_qend = min(S, wg_q0 + pos_per_wg);
  // keys needed by the work-group: [0, wg_qend)
  const int nkb = (wg_qend + kKB - 1) / kKB;

  const uint32_t row_bytes = (uint32_t)(p.kv_stride_tok * 2);
  const __amdgpu_buffer_rsrc_t krs = make_rsrc(p.k + (int64_t)kvh * p.kv_stride_head, (uint32_t)S * row_bytes);
  const __amdgpu_buffer_rsrc_t vrs = make_rsrc(p.v + (int64_t)kvh * p.kv_stride_head, (uint32_t)S * row_bytes);

  // Staging: at step i thread t moves chunk (t % kChunks) of row i * kRowsPerStep + t / kChunks;
  // the lane part of every address is computed once, the step part is an
  // immediate (LDS) or a scalar offset (global).
  constexpr int kRowsPerStep = kWaves * 64 / kChunks;
  const uint32_t g_lane = (uint32_t)(t / kChunks) * row_bytes + (t % kChunks) * 16;
  const int k_lane = (t / kChunks) * kKStride + (t % kChunks) * 16;
  const int v_lane = (t / kChunks) * kVStride + (t % kChunks) * 16;
  u32x4 kst[kLoads], vst[kLoads];
  auto load_k = [&](int kb) {
    const uint32_t so = (uint32_t)(kb * kKB) * row_bytes;
#pragma unroll
    for (int i = 0; i < kLoads; ++i) kst[i] = buf_load16(krs, g_lane, so + (uint32_t)(i * kRowsPerStep) * row_bytes);
  };
  auto load_v = [&](int kb) {
    const uint32_t so = (uint32_t)(kb * kKB) * row_bytes;
#pragma unroll
    for (int i = 0; i < kLoads; ++i) vst[i] = buf_load16(vrs, g_lane, so + (uint32_t)(i * kRowsPerStep) * row_bytes);
  };
  auto store_k = [&](int buf) {
    unsigned char* dst = smem + buf * kBufBytes + k_lane;
#pragma unroll
    for (int i = 0; i < kLoads; ++i) *reinterpret_cast<u32x4*>(dst + i * kRowsPerStep * kKStride) = kst[i];
  };
  auto store_v = [&](int buf) {
    unsigned char* dst = smem + buf * kBufBytes + kKTile + v_lane;
#pragma unroll
    for (int i = 0; i < kLoads; ++i)
      *reinterpret_cast<u32x4*>(dst + i * kRowsPerStep * kVStride) = bf16x8_to_f16x8(vst[i]);
  };

  const int qcol = lane & 31;       // this lane's query column
  const int kgrp = lane >> 5;       // k-slot group of MFMA operands
  const int i16 = lane & 15;
  const int sub16 = (lane >> 4) & 1;
  const float c_log2 = p.scale_log2;

  const int passes = (G + kWaves - 1) / kWaves;
  for (int pass = 0; pass < passes; ++pass) {
    const int head_local = pass * kWaves + wave % GW;
    // Waves past the group (or past the prompt) run the same instruction stream
    // on clamped indices and store nothing; their keys beyond their queries are
    // masked like any causal key, so no branch is needed inside the key loop.
    const bool wave_active = wave < GW * (kWaves / GW) && head_local < G && q0 < S;
    const int head = kvh * G + min(head_local, G - 1);

    // ---- Q^T operand in registers: lane holds Q[q0 + qcol][d = st*16 + kgrp*8 .. +8]
    u32x4 qop[kSteps];
    {
      const int qrow = min(q0 + qcol, S - 1);
      const uint16_t* qp = p.q + (int64_t)qrow * p.q_stride_tok + (int64_t)head * p.q_stride_head + kgrp * 8;
#pragma unroll
      for (int st = 0; st < kSteps; ++st) qop[st] = *reinterpret_cast<const u32x4*>(qp + st * 16);
    }

    floatx16 oacc[kDTiles];
#pragma unroll
    for (int i = 0; i < kDTiles; ++i)
#pragma unroll
      for (int j = 0; j < 16; ++j) oacc[i][j] = 0.f;
    float m_ref = -INFINITY;  // reference max (log2 domain) of this lane's column
    float l_run = 0.f;        // partial row sum over this lane's keys
    const int my_q = q0 + qcol;
    uint32_t pk[2][8];        // P of the latest key block (fp16 pairs)

    // S^T (64 keys x 32 queries) = K . Q^T from K buffer `buf`.
    auto qk = [&](int buf, floatx16 (&sacc)[2]) {
      const unsigned char* krow = smem + buf * kBufBytes + qcol * kKStride + kgrp * 16;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int j = 0; j < 16; ++j) sacc[mt][j] = 0.f;
#pragma unroll
      for (int st = 0; st < kSteps; ++st) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const u32x4 a = *reinterpret_cast<const u32x4*>(krow + mt * 32 * kKStride + st * 32);
          sacc[mt] = mfma32(as_bf16x8(a), as_bf16x8(qop[st]), sacc[mt]);
        }
      }
    };
    // O^T += V^T . P^T over the 64 keys held in V buffer `buf`.
    auto pv = [&](int buf) {
      const unsigned char* vlane = smem + buf * kBufBytes + kKTile + (kgrp * 4 + (i16 >> 2)) * kVStride +
                                   (sub16 * 16 + (i16 & 3) * 4) * 2;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int mt = ks >> 1, half = ks & 1;
        const u32x4 pop = {pk[mt][half * 4 + 0], pk[mt][half * 4 + 1], pk[mt][half * 4 + 2], pk[mt][half * 4 + 3]};
#pragma unroll
        for (int dt = 0; dt < kDTiles; ++dt) {
          const unsigned char* pa = vlane + ks * 16 * kVStride + dt * 64;
          const bf16x8 vt = lds_read_tr_pair((const BT_LDS uint16_t*)(const BT_LDS unsigned char*)pa,
                                             (const BT_LDS uint16_t*)(const BT_LDS unsigned char*)(pa + 8 * kVStride));
          oacc[dt] = mfma32_f16(__builtin_bit_cast(u32x4, vt), pop, oacc[dt]);
        }
      }
    };
    // Causal mask of block kb (only blocks reaching past q0 need it).
    auto mask = [&](int kb, floatx16(&sacc)[2]) {
      const int key0 = kb * kKB;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int key = key0 + mt * 32 + (j >> 2) * 8 + kgrp * 4 + (j & 3);
          sacc[mt][j] = key <= my_q ? sacc[mt][j] : -INFINITY;
        }
    };
    // Online softmax of one block: fills pk and returns the factor the
    // accumulated O must be scaled by (1 unless the reference max moved).
    // Scores stay unscaled until exp2(s * c - m).
    auto softmax = [&](floatx16(&sacc)[2]) -> float {
      float tmax = -INFINITY;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int j = 0; j < 16; ++j) tmax = fmaxf(tmax, sacc[mt][j]);
      tmax = halves_max(tmax) * c_log2;
      // lazy reference max: move it only when a score exceeds it by > kLazy
      const bool move = tmax > m_ref + kLazy;
      const float m_new = move ? tmax : m_ref;
      const float alpha = move ? fast_exp2(m_ref - m_new) : 1.f;  // 0 when m_ref is -inf
      m_ref = m_new;
      const float neg_m = m_ref == -INFINITY ? 0.f : -m_ref;
      float psum = 0.f;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int j = 0; j < 16; j += 2) {
          const float p0 = fast_exp2(fmaf(sacc[mt][j], c_log2, neg_m));
          const float p1 = fast_exp2(fmaf(sacc[mt][j + 1], c_log2, neg_m));
          psum += p0 + p1;
          pk[mt][j / 2] = pack_f16_rne(p0, p1);
        }
      l_run = l_run * alpha + psum;
      return alpha;
    };
    auto rescale = [&](float alpha) {
      if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {  // rare: the max moved by > 2^8
#pragma unroll
        for (int i = 0; i < kDTiles; ++i) oacc[i] *= alpha;
      }
    };
    // Blocks whose last key is <= q0 need no causal mask.
    const int kb_diag = (q0 + 1) / kKB;
    const int last = nkb - 1;

    // Prologue: K_0 in LDS, K_1 and V_0 in flight.  Fetches past the last
    // block re-read the last block (min(., last)) and are never consumed, so
    // the key loop has no branches around its loads and stores.
    load_k(0);
    load_v(0);
    store_k(0);
    load_k(min(1, last));
    __syncthreads();

    // Block 0: stage K_1 / V_0, S_0, softmax -> P_0.
    {
      store_k(1);
      store_v(0);
      load_k(min(2, last));
      load_v(min(1, last));
      floatx16 sacc[2];
      qk(0, sacc);
      if (0 >= kb_diag) mask(0, sacc);
      rescale(softmax(sacc));
      __syncthreads();
    }
    // Block kb: stage K_{kb+1} and V_kb, fetch K_{kb+2} and V_{kb+1},
    // S_kb = K_kb . Q^T, O += V_{kb-1} . P_{kb-1}, softmax(S_kb) -> P_kb.
    // Buffers written here (K (kb+1)%2, V kb%2) were last read before the
    // previous barrier, so one barrier per block suffices.
    for (int kb = 1; kb < nkb; ++kb) {
      const int buf = kb & 1;
      store_k(buf ^ 1);
      store_v(buf);
      __builtin_amdgcn_sched_barrier(0);  // keep the refetch behind the stores: one set of staging registers
      load_k(min(kb + 2, last));
      load_v(min(kb + 1, last));
      floatx16 sacc[2];
      qk(buf, sacc);
      if (kb >= kb_diag) mask(kb, sacc);
      pv(buf ^ 1);
      rescale(softmax(sacc));
      __syncthreads();
    }
    pv((nkb - 1) & 1);

    // ---- epilogue: full row sums, normalise, store ---------------------------
    l_run = halves_sum(l_run);
    if (wave_active && my_q < S) {
      const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
      const int64_t orow = (int64_t)my_q * p.out_stride_tok + (int64_t)head * p.out_stride_head;
#pragma unroll
      for (int dt = 0; dt < kDTiles; ++dt) {
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
          const int d = dt * 32 + jb * 8 + kgrp * 4;
          const float o0 = oacc[dt][jb * 4 + 0] * inv, o1 = oacc[dt][jb * 4 + 1] * inv;
          const float o2 = oacc[dt][jb * 4 + 2] * inv, o3 = oacc[dt][jb * 4 + 3] * inv;
          if (p.out_bf16) {
            const u32x2 pk2 = {pack2(f32_to_bf16_bits(o0), f32_to_bf16_bits(o1)),
                               pack2(f32_to_bf16_bits(o2), f32_to_bf16_bits(o3))};
            *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(p.out) + orow + d) = pk2;
          } else {
            *reinterpret_cast<float4*>(reinterpret_cast<float*>(p.out) + orow + d) = float4{o0, o1, o2, o3};
          }
        }
      }
    }
    __syncthreads();  // the next pass restages buffer 0
  }
}

hipError_t launch_prefill(const PrefillParams& p, int head_dim, hipStream_t stream) {
  const int G = p.group;
  const int GW = G < kWaves ? G : kWaves;
  const int pos_per_wg = kQB * (kWaves / GW);
  const int nqb = (p.seqlen + pos_per_wg - 1) / pos_per_wg;
  dim3 grid(nqb, p.kv_heads);
  switch (head_dim) {
    case 128: hipLaunchKernelGGL(gqa_prefill_kernel<128>, grid, dim3(kWaves * 64), 0, stream, p); break;
    case 256: hipLaunchKernelGGL(gqa_prefill_kernel<256>, grid, dim3(kWaves * 64), 0, stream, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace bt
