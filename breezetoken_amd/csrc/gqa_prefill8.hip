// Causal GQA prefill on CDNA4 fp16 MFMA with two waves per SIMD.
//
// Computes, for every new query row i (absolute position p0 + i, where p0 =
// q_offset tokens are already in the cache) and every query head h (kv head
// h / group),
//     out[i, h] = softmax_{j <= p0+i} (q_i . k_j * scale) . V_j
// over the p0 + S keys of the cache -- the F.scaled_dot_product_attention
// (is_causal=True, enable_gqa=True) call of _prefill_attn (breezetoken/model/
// prefill.py:56-68, p0 = 0) and the banded-mask chunked prefill of
// Qwen36MoE._attn_batch (breezetoken/model/qwen36_moe.py:394-428) -- with a
// work decomposition that keeps two waves resident on every SIMD:
//  * a work-group of 8 waves shares one K tile and one V^T tile in LDS; wave w
//    owns query head (w % G) of a subset of G heads of the kv group and 16
//    query positions [q0 + (w / G) * 16, +16), G in {1, 2, 4, 8}: the largest
//    power of two that divides the group size (so a group of 6 runs as 3
//    subsets of 2 heads, each subset's work-groups reading the same K/V);
//  * per 64-key block a wave runs 32 v_mfma_f32_16x16x32_f16 for S^T = K.Q^T
//    (K from LDS, Q^T in registers) and 32 for O^T += V^T.P^T (V^T from LDS,
//    P^T built in registers from the S^T accumulators).  Per wave that is 64
//    accumulators of O, 32 registers of Q and 16 of S (64 of Q for f32 q,
//    below), so two waves fit in the register file and hide each other's
//    LDS, copy and barrier waits;
//  * q enters as fp16 with a power-of-two scale per query row: bf16 q
//    converts exactly, f32 q as two fp16 terms (hi + lo, two MFMAs per K
//    fragment) so the scores keep f32 q's precision at any magnitude;
//    K and V come from the pre-pass's fp16 images (gqa_prefill_vt.hip), each
//    scaled per 64-key block; the softmax takes all three factors back
//    exactly in its exp2 argument;
//  * the K image is row-major with 16-byte chunk c of key row r in slot c ^
//    (r & 15), so a tile copy is contiguous and the operand reads of 16
//    consecutive rows hit 16 different bank groups;
//  * the V^T image holds each 64-key block as 8 chunks of 8 keys; chunk c =
//    kh*4 + g holds keys kh*32 + g*4 + {0,1,2,3} and kh*32 + 16 + g*4 +
//    {0,1,2,3}: the order in which lane group g of the 16x16 result registers
//    holds P for the 32-key half kh, so the P^T operand never moves between
//    lanes;
//  * the online softmax (log2 domain, lazy rescaling by 2^8) of block kb runs
//    beside the P.V product of block kb - 1; tiles are double-buffered with
//    two barriers per block and every copy issued as soon as its buffer is
//    free;
//  * a work-group runs one or two segments (key-block ranges of a query
//    block): the whole query block, a chunk of it under the uniform split, or
//    its share of a query-block pair under the paired split (see
//    PrefillParams); a segment that is not its query block's only chunk writes
//    a partial and an LSE per row for prefill_combine_kernel;
//  * work-groups with at most two key blocks can convert them from the bf16
//    cache into their LDS tiles themselves (DIRECT), with the pre-pass's
//    layout, rounding and scales, so a short prompt needs no pre-pass.
#include "bt_common.h"
#include "bt_kernels.h"

namespace bt {

namespace {

typedef _Float16 halfx8_8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v_8 __attribute__((ext_vector_type(2)));
typedef float float2v_8 __attribute__((ext_vector_type(2)));

template <int B>
struct Buf8 {
  static constexpr int value = B;
};
template <bool B>
struct BoolC {
  static constexpr bool value = B;
};

constexpr int kKB8 = kPrefillKeyBlock;  // keys per block (64)
constexpr int kWaves8 = 8;
constexpr int kRows8 = 128;             // (query, head) rows of a work-group: 8 waves x 16 queries
constexpr int kMaxChunks = 64;          // split-key chunks per query block (combine LDS bound)
constexpr int kQ8 = 16;                 // query positions per wave
constexpr float kLazy8 = 8.0f;          // log2-domain slack before the reference max moves

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc8(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 load16_8(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, 0, 0);
}
// HBM -> LDS copy of 16 bytes per lane (lane l's bytes land at lds + 16 * l);
// offsets past the descriptor's range read as zero.
__device__ __forceinline__ void dma16_8(__amdgpu_buffer_rsrc_t r, unsigned char* lds, uint32_t voff,
                                        uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (BT_LDS void*)lds, 16, (int)voff, (int)soff, 0, 0);
}
__device__ __forceinline__ floatx4 mfma16_f16(const u32x4& a, const u32x4& b, const floatx4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(halfx8_8, a), __builtin_bit_cast(halfx8_8, b), c,
                                                0, 0, 0);
}
// Round to nearest even through a builtin (not asm), so the compiler sees the
// VALU write and inserts the wait states an in-flight MFMA operand needs.
__device__ __forceinline__ uint32_t pack_rne8(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((float2v_8){a, b}, half2v_8));
}

// Chunks of query block qb under the paired split (see PrefillParams): the
// ranges of its pair that reach its key blocks.
template <typename NB>
__host__ __device__ inline int pair_chunks(int qb, int nqb, int parts, NB n_blocks) {
  const int r = qb < nqb - 1 - qb ? qb : nqb - 1 - qb;
  const int qhi = nqb - 1 - r;
  const int nhi = n_blocks(qhi), nlo = r != qhi ? n_blocks(r) : 0;
  const int size = (nhi + nlo + parts - 1) / parts;
  return qb == qhi ? (nhi + size - 1) / size : (nhi + nlo - 1) / size - nhi / size + 1;
}

// Query blocks with more than c chunks of kb key blocks under the uniform
// split: the heaviest n of them (query blocks nqb - n .. nqb - 1), since a
// query block's key blocks grow with its index (block qb ends at position
// min(S, (qb + 1) * pos) behind P0 cached keys).
__host__ __device__ inline int split_blocks_past(int c, int kb, int S, int P0, int pos, int nqb) {
  const int R = c * kb * kKB8 - P0;  // positions a query block must pass
  if (R < 0) return nqb;
  if (S <= R) return 0;
  return nqb - R / pos;
}
// Work-groups of the uniform split's compact grid for one (kv head, head
// subset): per chunk c, one per query block with keys there, rounded up to a
// multiple of 8 so that every chunk of query block qb runs on the XCD of
// work-group id (nqb - 1 - qb) mod 8, whose L2 then holds all of its partials
// for the combine (which places its merge the same way).
__host__ __device__ inline int split_pad8(int n) { return (n + 7) & ~7; }
__host__ __device__ inline int split_items(int kb, int S, int P0, int pos, int nqb, int max_chunks) {
  int n = 0;
  for (int c = 0; c < max_chunks; ++c) n += split_pad8(split_blocks_past(c, kb, S, P0, pos, nqb));
  return n;
}

}  // namespace

// Timeline build only (-DBT_TIMELINE, libbt_timeline.so; never the product
// library): waves 0 and 4 of each of the first kTimelineWGs work-groups
// record s_memrealtime (the device's 100 MHz clock) at eight points of a
// segment -- start, q in registers, first tiles published, first block done,
// key loop done, last P.V issued, stores issued, stores complete -- into
// bt_tl_buf[(work-group * 2 + (wave == 4)) * 8 + point], with vector stores
// after the segment's own.  A work-group with two segments keeps the second's.
#ifdef BT_TIMELINE
constexpr int kTimelineWGs = 4096;
constexpr int kTimelineSlots = kTimelineWGs * 16;
__device__ unsigned long long bt_tl_buf[kTimelineSlots];
#define BT_TL(k) (tl[k] = __builtin_amdgcn_s_memrealtime())
#define BT_TL_END()                                                                                   \
  do {                                                                                                \
    tl[6] = __builtin_amdgcn_s_memrealtime();                                                         \
    __builtin_amdgcn_s_waitcnt(0x0f70); /* vmcnt(0): the stores are complete */                     \
    tl[7] = __builtin_amdgcn_s_memrealtime();                                                         \
    const int wg_ = (int)(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z));            \
    if (lane == 0 && (wave == 0 || wave == 4) && wg_ < kTimelineWGs)                                  \
      for (int k_ = 0; k_ < 8; ++k_) bt_tl_buf[(wg_ * 2 + (wave == 4)) * 8 + k_] = tl[k_];            \
  } while (0)
#else
#define BT_TL(k) ((void)0)
#define BT_TL_END() ((void)0)
#endif

// DIRECT: a work-group with at most two key blocks converts them from the bf16
// cache straight into its LDS tiles (the layout and rounding of the images
// of gqa_prefill_vt.hip, same block scales), so a short prompt needs no
// pre-pass launch.
// PAIRED: the paired split (two segments per work-group at most); its own
// instantiation, so the single-segment kernel keeps one copy of the loop.
// LO: f32 q as two fp16 terms (hi + lo, see split_f16x2), each K fragment
// feeding one MFMA per term, so the scores match f32 q at any magnitude.
template <int D, bool DIRECT, bool PAIRED, bool LO>
__global__ __launch_bounds__(kWaves8 * 64, 1) void gqa_prefill8_kernel(PrefillParams p) {
  constexpr int kDSteps = D / 32;      // K-dimension steps of Q.K^T (32 per MFMA)
  constexpr int kDTiles = D / 16;      // 16-row d tiles of O^T
  constexpr int kImg = kKB8 * D * 2;   // bytes of one K or V^T tile
  constexpr int kCopies = kImg / 1024 / kWaves8;  // 1 KiB copies per wave per tile

  // Separate LDS arrays so the compiler can see that copies into one buffer
  // never alias operand reads from another; the key loop is unrolled by two so
  // every buffer choice is a constant.
  __shared__ __attribute__((aligned(1024))) unsigned char k_lds0[kImg];
  __shared__ __attribute__((aligned(1024))) unsigned char k_lds1[kImg];
  __shared__ __attribute__((aligned(1024))) unsigned char v_lds0[kImg];
  __shared__ __attribute__((aligned(1024))) unsigned char v_lds1[kImg];
  __shared__ uint32_t dmax[2][kWaves8];  // DIRECT: per-wave block maxima
  auto k_buf = [&](auto b) -> unsigned char* {
    if constexpr (decltype(b)::value == 0) return k_lds0; else return k_lds1;
  };
  auto v_buf = [&](auto b) -> unsigned char* {
    if constexpr (decltype(b)::value == 0) return v_lds0; else return v_lds1;
  };

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int G = p.sub_group;                // 1, 2, 4 or 8 (checked by the launcher)
  const int pos_per_wg = kQ8 * (kWaves8 / G);
  const int S = p.seqlen;
  const int P0 = p.q_offset;
  const int nkeys = P0 + S;
  const int nqb = (S + pos_per_wg - 1) / pos_per_wg;
  const int nblk = (nkeys + kKB8 - 1) / kKB8;
  // (kv head, head subset): grid y, or under the uniform split part of the
  // compact grid's x, which lists the (chunk, subset, query block) items that
  // have keys, chunk slowest and the heaviest query block first (the order of
  // a full chunks x subsets x query blocks grid without its empty slots).
  int ysub = blockIdx.y, split_qb = 0, split_chunk = 0;
  if (!PAIRED && p.kb_chunk > 0 && p.split_compact) {
    const int ys = p.kv_heads * p.head_subs;
    int L = (int)blockIdx.x;
    bool found = false;
    for (int c = 0; c < p.max_chunks && !found; ++c) {
      const int n = split_blocks_past(c, p.kb_chunk, S, P0, pos_per_wg, nqb);
      const int np = split_pad8(n);
      if (L < np * ys) {
        if (L % np >= n) return;  // a padding slot (whole work-group)
        ysub = L / np;
        split_qb = nqb - 1 - L % np;
        split_chunk = c;
        found = true;
      } else {
        L -= np * ys;
      }
    }
    if (!found) return;  // past the launcher's item count: no work-group is
  }
  const int kvh = ysub / p.head_subs;
  const int head_base = kvh * p.group + (ysub % p.head_subs) * G;
  // One segment: key blocks [kb0, kb1) of query block qblk, chunk `chunk` of
  // its nchunks (nchunks > 1: the segment writes a partial for the combine).
  auto segment = [&](const int qblk, const int kb0, const int kb1, const int chunk, const int nchunks) {
#ifdef BT_TIMELINE
    unsigned long long tl[8] = {};
#endif
    BT_TL(0);
    const int wg_q0 = qblk * pos_per_wg;
    const int q0 = wg_q0 + (wave / G) * kQ8;
    const int last = kb1 - 1;
    const int head = head_base + wave % G;

    const size_t head_img = (size_t)kvh * p.img_blocks * kKB8 * D;  // this kv head's images
    const __amdgpu_buffer_rsrc_t krs = rsrc8(p.kimg + head_img, (uint32_t)nblk * kImg);
    const __amdgpu_buffer_rsrc_t vrs = rsrc8(p.vt + head_img, (uint32_t)nblk * kImg);
    const int* kexp = p.kexp + kvh * p.img_blocks;
    const uint32_t v_voff = (uint32_t)lane * 16;
    // Tile copy i (1 KiB) is bytes [1024 i, +1024) of the block's K or V^T
    // image; the K image is row-major with 16-byte slot s of row r holding chunk
    // s ^ (r & 15), so the tile lands swizzled.  Wave w issues copies w, w + 8, ...
    auto copy_k = [&](auto b, int kb) {
      const uint32_t so = (uint32_t)kb * kImg;
  #pragma unroll
      for (int j = 0; j < kCopies; ++j) {
        const int i = wave + kWaves8 * j;
        dma16_8(krs, k_buf(b) + i * 1024, v_voff, so + (uint32_t)i * 1024);
      }
    };
    auto copy_v = [&](auto b, int kb) {
      const uint32_t so = (uint32_t)kb * kImg;
  #pragma unroll
      for (int j = 0; j < kCopies; ++j) {
        const int i = wave + kWaves8 * j;
        dma16_8(vrs, v_buf(b) + i * 1024, v_voff, so + (uint32_t)i * 1024);
      }
    };
    // Each wave waits for its own copies; the barrier that follows publishes
    // them.  vmcnt counts a wave's loads in issue order, so naming how many
    // tiles (kCopies loads each) were issued after the awaited one waits for
    // exactly that tile and the older ones.
    auto wait_all = [] { __builtin_amdgcn_s_waitcnt(0x0f70); };
    static_assert(2 * kCopies < 64, "vmcnt holds 6 bits");
    auto wait_tiles = [](int younger) {
      if (younger >= 2) __builtin_amdgcn_s_waitcnt(0x0f70 | ((2 * kCopies) & 0xf) | (((2 * kCopies) >> 4) << 14));
      else if (younger == 1) __builtin_amdgcn_s_waitcnt(0x0f70 | (kCopies & 0xf) | ((kCopies >> 4) << 14));
      else __builtin_amdgcn_s_waitcnt(0x0f70);
    };
    // Work-group barrier without __syncthreads' fence (which would wait for
    // every copy in flight); the LDS reads before it were consumed by MFMAs.
    auto barrier = [] { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };

    const int i16 = lane & 15;   // query column of the 16x16 tiles
    const int g4 = lane >> 4;    // lane group: k slice of the operands, rows 4*g4.. of results

    // Q^T operand: lane holds Q[q0 + i16][st*32 + g4*8 .. +8] for each 32-d step
    // as fp16, the row scaled by 2^-eq so its largest |q| lies in [2^14, 2^15);
    // c_col = scale * log2(e) * 2^eq restores it in the exp2 argument.
    // K and V^T scale exponents of a block, read through the scalar cache a
    // block ahead of their use (each read is a dependent round trip to memory
    // the pre-pass just wrote).
    const int* vexp = p.vexp + kvh * p.img_blocks;
    int dek[2] = {0, 0}, deb[2] = {kVExpZero, kVExpZero};  // DIRECT: exponents of blocks kb0, kb0 + 1
    auto scales = [&](int kb, int& ek, int& eb) {
      if constexpr (DIRECT) {
        const bool second = min(kb, last) > kb0;
        ek = second ? dek[1] : dek[0];
        eb = second ? deb[1] : deb[0];
      } else {
        const int b = min(kb, last);
        ek = sload(kexp, b);
        eb = sload(vexp, b);
      }
    };
    // Copy schedule:
    //   start of step kb: V_kb -> V buffer kb % 2; after the mid barrier: K_{kb+2}
    //   -> K buffer kb % 2; the mid barrier publishes V_{kb-1}, the end barrier
    //   K_{kb+1}.  No copy goes past the last block (a short work-group would
    //   otherwise wait for them at its end).
    // Buffers alternate from the work-group's first block kb0.  The first tiles,
    // and V_{kb0+1} (which the generic schedule would issue a step later), go out
    // before the q loads, so their latencies overlap.
    // DIRECT: threads 0..255 hold V items (chunk c, 8-column slice dc: the 8
    // keys of chunk c at those columns), threads 256..511 K units (16-byte slot
    // of a key row), for both blocks; loads go out before the q loads.
    constexpr int kDC = D / 8;                 // 16-byte column chunks per row
    constexpr int kVItems = 8 * kDC;           // V^T items per block
    constexpr int kKPer = kKB8 * kDC / 256;    // K units per K thread per block
    static_assert(kVItems <= 256 && kKPer >= 1, "head_dim 128 or 256");
    u32x4 draw[2][8];
    if constexpr (DIRECT) {
      const uint32_t row_bytes = (uint32_t)(p.kv_stride_tok * 2);
      const uint32_t range = (uint32_t)nkeys * row_bytes;  // keys past the prompt read as zero
      if (t < 256) {
        const __amdgpu_buffer_rsrc_t vsrc = rsrc8(p.v + (int64_t)kvh * p.kv_stride_head, range);
        const int c = t / kDC, dc = t % kDC;
  #pragma unroll
        for (int b = 0; b < 2; ++b)
          if (t < kVItems && kb0 + b <= last)
  #pragma unroll
            for (int j = 0; j < 8; ++j) {
              const int key = (kb0 + b) * kKB8 + (c >> 2) * 32 + (c & 3) * 4 + (j & 3) + (j >> 2) * 16;
              draw[b][j] = load16_8(vsrc, (uint32_t)key * row_bytes + (uint32_t)dc * 16);
            }
      } else {
        const __amdgpu_buffer_rsrc_t ksrc = rsrc8(p.k + (int64_t)kvh * p.kv_stride_head, range);
  #pragma unroll
        for (int b = 0; b < 2; ++b)
          if (kb0 + b <= last)
  #pragma unroll
            for (int j = 0; j < kKPer; ++j) {
              const int x = j * 256 + (t - 256);
              const int r = x / kDC, slot = x % kDC;
              draw[b][j] = load16_8(ksrc, (uint32_t)((kb0 + b) * kKB8 + r) * row_bytes + (uint32_t)(slot ^ (r & 15)) * 16);
            }
      }
    } else {
      copy_k(Buf8<0>{}, kb0);
      if (kb0 + 1 <= last) copy_k(Buf8<1>{}, kb0 + 1);
      copy_v(Buf8<0>{}, kb0);
      if (kb0 + 1 <= last) copy_v(Buf8<1>{}, kb0 + 1);
    }
    int ek_c, eb_c;
    if constexpr (!DIRECT) scales(kb0, ek_c, eb_c);
    u32x4 qop[kDSteps];
    u32x4 qlo[LO ? kDSteps : 1];
    float c_col;
    {
      const int qrow = min(q0 + i16, S - 1);
      const int64_t off = (int64_t)qrow * p.q_stride_tok + (int64_t)head * p.q_stride_head + g4 * 8;
      auto reduce = [](uint32_t mx) { return xor_umax<32>(xor_umax<16>(mx)); };  // the row's four lane groups
      int eq;
      if constexpr (LO) eq = q_row_f16_lo(reinterpret_cast<const float*>(p.q), off, 32, qop, qlo, reduce);
      else eq = q_row_f16(p.q, p.q_f32 != 0, off, 32, qop, reduce);
      c_col = __builtin_ldexpf(p.scale_log2, eq);
      BT_TL(1);
    }
    if constexpr (DIRECT) {
      // Block maxima (bf16 bits of |x|, which order like |x|): V over waves
      // 0..3, K over waves 4..7; then every thread derives the same exponents.
      uint32_t mx[2] = {0u, 0u};
      const int nj = t < 256 ? (t < kVItems ? 8 : 0) : kKPer;
  #pragma unroll
      for (int b = 0; b < 2; ++b)
        if (kb0 + b <= last)
  #pragma unroll
          for (int j = 0; j < 8; ++j)
            if (j < nj)
  #pragma unroll
              for (int i = 0; i < 4; ++i)
                mx[b] = max(mx[b], max(draw[b][j][i] & 0x7fffu, (draw[b][j][i] >> 16) & 0x7fffu));
  #pragma unroll
      for (int b = 0; b < 2; ++b) {
        mx[b] = wave_umax(mx[b]);
        if (lane == 0) dmax[b][wave] = mx[b];
      }
      __syncthreads();
  #pragma unroll
      for (int b = 0; b < 2; ++b) {
        const uint32_t vm = max(max(dmax[b][0], dmax[b][1]), max(dmax[b][2], dmax[b][3]));
        const uint32_t km = max(max(dmax[b][4], dmax[b][5]), max(dmax[b][6], dmax[b][7]));
        if (km != 0) {
          const int ebits = (int)(km >> 7);
          dek[b] = (ebits == 0 ? 1 : ebits) - 127 - 14;
        }
        if (vm != 0) {
          const int ebits = (int)(vm >> 7);
          const int E = (ebits == 0 ? 1 : ebits) - 127;
          deb[b] = E <= 14 ? -4 * ((14 - E) / 4) : 4 * ((E - 14 + 3) / 4);  // 4 * ceil((E - 14) / 4)
        }
      }
      auto to_f16 = [](float a, float b, int e) {
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(
                                                (float2v_8){__builtin_ldexpf(a, -e), __builtin_ldexpf(b, -e)}, half2v_8));
      };
      auto write_tiles = [&](auto bsel) {
        constexpr int b = decltype(bsel)::value;
        if (kb0 + b > last) return;
        if (t < 256) {
          if (t >= kVItems) return;
          const int c = t / kDC, dc = t % kDC;
          const int e = deb[b];
  #pragma unroll
          for (int i = 0; i < 8; ++i) {  // V^T row d = dc*8 + i of chunk c
            u32x4 o;
  #pragma unroll
            for (int m = 0; m < 4; ++m) {
              const uint32_t w0 = draw[b][2 * m][i >> 1], w1 = draw[b][2 * m + 1][i >> 1];
              o[m] = to_f16(__uint_as_float((i & 1) ? (w0 & 0xffff0000u) : (w0 << 16)),
                            __uint_as_float((i & 1) ? (w1 & 0xffff0000u) : (w1 << 16)), e);
            }
            *reinterpret_cast<u32x4*>(v_buf(bsel) + (c * D + dc * 8 + i) * 16) = o;
          }
        } else {
          const int e = dek[b];
  #pragma unroll
          for (int j = 0; j < kKPer; ++j) {  // unit x lands at x * 16: row x / kDC, slot x % kDC
            u32x4 o;
  #pragma unroll
            for (int m = 0; m < 4; ++m)
              o[m] = to_f16(__uint_as_float(draw[b][j][m] << 16), __uint_as_float(draw[b][j][m] & 0xffff0000u), e);
            *reinterpret_cast<u32x4*>(k_buf(bsel) + (j * 256 + (t - 256)) * 16) = o;
          }
        }
      };
      write_tiles(Buf8<0>{});
      write_tiles(Buf8<1>{});
      scales(kb0, ek_c, eb_c);
    }

    floatx4 oacc[kDTiles];
  #pragma unroll
    for (int i = 0; i < kDTiles; ++i) oacc[i] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_ref = -INFINITY;          // reference max (log2 domain) of this lane's query column
    float l_run = 0.f;                // partial row sum over this lane's keys
    int e_run = kVExpZero;            // V scale O is kept in: O_true = O * 2^e_run
    const int my_q = q0 + i16;
    const int my_pos = P0 + my_q;     // keys 0 .. my_pos
    u32x4 pk[2];                      // P of the pending block: 32-key halves, fp16

    // S^T (64 keys x 16 queries) = K . Q^T from K buffer b: A operand of d-step
    // st / key sub-tile sub is chunk st*4 + g4 of key row sub*16 + i16, stored
    // in slot (st*4 + g4) ^ i16 of that row (row & 15 == i16).
    auto kfrag = [&](auto b, int st, int sub) -> u32x4 {
      return *reinterpret_cast<const u32x4*>(k_buf(b) + (sub * 16 + i16) * (D * 2) + (((st * 4 + g4) ^ i16) * 16));
    };
    // The first d-step's K fragments, read right after the barrier that
    // publishes the tile, ahead of the tile copies the step issues.
    auto k_first = [&](auto b, u32x4 (&f0)[4]) {
  #pragma unroll
      for (int sub = 0; sub < 4; ++sub) f0[sub] = kfrag(b, 0, sub);
    };
    auto qk = [&](auto b, floatx4 (&sacc)[4], const u32x4 (&f0)[4]) {
      const floatx4 zero = {0.f, 0.f, 0.f, 0.f};
  #pragma unroll
      for (int st = 0; st < kDSteps; ++st) {
  #pragma unroll
        for (int sub = 0; sub < 4; ++sub) {
          const u32x4 a = st == 0 ? f0[sub] : kfrag(b, st, sub);
          sacc[sub] = mfma16_f16(a, qop[st], st == 0 ? zero : sacc[sub]);
          if constexpr (LO) sacc[sub] = mfma16_f16(a, qlo[st], sacc[sub]);
        }
      }
    };
    // O^T += V^T . P^T over the 64 keys of V^T buffer b: A operand of key half kh
    // / d tile dt is chunk kh*4 + g4 of row dt*16 + i16.
    auto pv = [&](auto b, const u32x4 (&pp)[2]) {
      const unsigned char* vb_ = v_buf(b);
  #pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
  #pragma unroll
        for (int dt = 0; dt < kDTiles; ++dt) {
          const u32x4 a = *reinterpret_cast<const u32x4*>(vb_ + ((kh * 4 + g4) * D + dt * 16 + i16) * 16);
          oacc[dt] = mfma16_f16(a, pp[kh], oacc[dt]);
        }
      }
    };
    // Causal mask of block kb: score of key sub*16 + g4*4 + r for query my_q.
    auto mask = [&](int kb, floatx4 (&sacc)[4]) {
      const int key0 = kb * kKB8 + g4 * 4;
  #pragma unroll
      for (int sub = 0; sub < 4; ++sub)
  #pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = key0 + sub * 16 + r;
          sacc[sub][r] = key <= my_pos ? sacc[sub][r] : -INFINITY;
        }
    };
    // Online softmax of block kb: max over the 64 keys of the column (this
    // lane's 16 and three lane groups' via xor 16 / 32), lazy reference update,
    // P as fp16 in the MFMA key order; returns the factor O must be scaled by.
    // The V^T block's power-of-two scale enters P' = P * 2^shift through the
    // exp2 bias; the row sum takes P.
    auto softmax = [&](floatx4 (&sacc)[4], u32x4 (&out)[2], int ek, int eb) -> float {
      float lmax = -INFINITY;
  #pragma unroll
      for (int sub = 0; sub < 4; ++sub)
  #pragma unroll
        for (int r = 0; r < 4; ++r) lmax = fmaxf(lmax, sacc[sub][r]);
      const float c_log2 = __builtin_ldexpf(c_col, ek);  // with the K block's scale
      // The column's max is one of its lane groups' own maxes (or NaN), so it
      // passes the lazy bound exactly when one group's does (scaling by
      // c_log2 > 0 keeps the order): the cross-lane reduction runs only when
      // some column's reference max may move, rare after a row's first keys.
      float alpha = 1.f;
      if (__builtin_amdgcn_ballot_w64(lmax * c_log2 > m_ref + kLazy8)) {
        float tmax = xor_fmaxf<16>(lmax);
        tmax = halves_max(tmax) * c_log2;
        const bool move = tmax > m_ref + kLazy8;
        const float m_new = move ? tmax : m_ref;
        alpha = move ? fast_exp2(m_ref - m_new) : 1.f;  // 0 when m_ref is -inf
        m_ref = m_new;
      }
      const int e_new = vexp_next(e_run, eb);
      const int shift = vexp_shift(e_new, eb);
      const float neg_m = (m_ref == -INFINITY ? 0.f : -m_ref) + (float)shift;
      float psum = 0.f;
  #pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
  #pragma unroll
        for (int j = 0; j < 4; ++j) {
          const floatx4& s = sacc[2 * kh + (j >> 1)];
          const float e0 = fast_exp2(fmaf(s[(j & 1) * 2], c_log2, neg_m));
          const float e1 = fast_exp2(fmaf(s[(j & 1) * 2 + 1], c_log2, neg_m));
          psum += e0 + e1;
          out[kh][j] = pack_rne8(e0, e1);
        }
      }
      if (shift != 0) psum = __builtin_ldexpf(psum, -shift);  // wave-uniform, rare
      l_run = l_run * alpha + psum;
      const float factor = e_new != e_run ? __builtin_ldexpf(alpha, e_run - e_new) : alpha;
      e_run = e_new;
      return factor;
    };
    auto rescale = [&](float alpha) {
      if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {  // rare: the max moved by > 2^8
  #pragma unroll
        for (int i = 0; i < kDTiles; ++i) oacc[i] *= alpha;
      }
    };
    const int kb_diag = (P0 + q0 + 1) / kKB8;  // earlier blocks need no mask

    // The first d-step's K fragments of each block are read before the
    // barrier that ends the block before it (the barrier in that block's
    // middle published them), so they arrive while the waves meet there; the
    // barrier leaves them in flight: every other LDS read of the block is
    // consumed by its MFMAs, and the K buffer they come from is refilled only
    // after the next block's Q.K^T.  They are read even when no block follows
    // (a stale buffer's values go unused), so f0 is always written and the
    // compiler keeps no older copy of it alive.
    auto end_block = [&](auto b_next, u32x4 (&f0)[4]) {
      k_first(b_next, f0);
      asm volatile("s_barrier" ::: "memory");
    };
    u32x4 f0[4];
    wait_all();
    __syncthreads();
    BT_TL(2);
    {
      floatx4 sacc[4];
      k_first(Buf8<0>{}, f0);
      qk(Buf8<0>{}, sacc, f0);
      barrier();
      if (kb0 + 2 <= last) copy_k(Buf8<0>{}, kb0 + 2);
      if (kb0 >= kb_diag) mask(kb0, sacc);
      int ek_n, eb_n;
      scales(kb0 + 1, ek_n, eb_n);
      softmax(sacc, pk, ek_c, eb_c);  // O is still zero: its factor does not matter
      ek_c = ek_n;
      eb_c = eb_n;
      end_block(Buf8<1>{}, f0);  // K_{kb0+1} arrived with the prologue's copies
    }
    BT_TL(3);
    // Block kb: A: S_kb = K_kb . Q^T; B: O += V_{kb-1} . P_{kb-1} beside the
    // softmax of S_kb.
    auto step = [&](auto b, int kb) {
      constexpr int B = decltype(b)::value;
      const bool second = kb == kb0 + 1;  // its V^T went out in the prologue
      if (!second) copy_v(b, kb);
      int ek_n, eb_n;
      floatx4 sacc[4];
      qk(b, sacc, f0);
      // The next block's scales are requested after the MFMAs: scalar loads
      // share the LDS reads' counter and return out of order, so issued
      // earlier they would hold the first MFMA until they arrive.
      scales(kb + 1, ek_n, eb_n);
      // V_{kb-1} and K_{kb+1} (if any); issued after them: V_kb (except in the
      // second block, whose V^T went out in the prologue).
      wait_tiles(second ? 0 : 1);
      barrier();
      if (kb + 2 <= last) copy_k(b, kb + 2);
      if (kb >= kb_diag) mask(kb, sacc);
      pv(Buf8<B ^ 1>{}, pk);
      u32x4 pk_next[2];
      const float alpha = softmax(sacc, pk_next, ek_c, eb_c);
      ek_c = ek_n;
      eb_c = eb_n;
      rescale(alpha);
      pk[0] = pk_next[0];
      pk[1] = pk_next[1];
      end_block(Buf8<B ^ 1>{}, f0);
    };
    // Every pass of the loop ends with a buffer-0 step, so no path reaches the
    // loop head with a copy into buffer 1 in flight (the compiler would have to
    // wait for every copy before the first buffer-1 read); an odd last block
    // runs after the loop.
    int kb = kb0 + 1;
    for (; kb + 1 < kb1; kb += 2) {
      step(Buf8<1>{}, kb);
      step(Buf8<0>{}, kb + 1);
    }
    if (kb < kb1) step(Buf8<1>{}, kb);
    BT_TL(4);
    wait_all();
    barrier();
    if ((last - kb0) & 1) pv(Buf8<1>{}, pk); else pv(Buf8<0>{}, pk);
    BT_TL(5);

    // ---- epilogue: row sums over the four lane groups, normalise, store -------
    l_run = xor_sum<16>(l_run);
    l_run = halves_sum(l_run);
    const float inv = l_run > 0.f ? __builtin_ldexpf(1.f / l_run, e_run) : 0.f;
    // Rows leave through LDS, so that every store writes whole 16-byte slices
    // of rows (a wave's store covers 2 rows of bf16 at D = 256) instead of 8-
    // or 16-byte pieces of 16 rows: at config 4, S = 128 took 13.5 against
    // 16.0 us per call.  Wave w stages 16 rows of 2D bytes (bf16 rows, or
    // f32 rows in two column halves) in quarter w % 4 of K buffer w / 4 --
    // every wave is past its last Q.K^T and the barrier after the loop --
    // with 16-byte chunk c of row r in slot c ^ r.
    unsigned char* stage = (wave < 4 ? k_lds0 : k_lds1) + (wave & 3) * (kQ8 * D * 2);
    constexpr int kChunks = D / 8;          // 16-byte chunks of a staged row
    constexpr int kRowsPer = 64 / kChunks;  // staged rows per store
    // Store the staged rows: row r to dst(r) + col_bytes (dst(r) null: skipped).
    auto drain = [&](auto&& dst, int col_bytes) {
  #pragma unroll
      for (int j = 0; j < kQ8 / kRowsPer; ++j) {
        const int r = j * kRowsPer + lane / kChunks, c = lane % kChunks;
        const u32x4 x = *reinterpret_cast<const u32x4*>(stage + r * (D * 2) + (c ^ r) * 16);
        if (unsigned char* d = dst(r)) *reinterpret_cast<u32x4*>(d + col_bytes + c * 16) = x;
      }
    };
    // f32 rows in two halves of D / 2 columns (d tiles [h * kDTiles / 2, +kDTiles / 2)).
    auto store_f32 = [&](auto&& dst) {
  #pragma unroll
      for (int h = 0; h < 2; ++h) {
  #pragma unroll
        for (int dt = h * kDTiles / 2; dt < (h + 1) * kDTiles / 2; ++dt) {
          const int c = (dt - h * kDTiles / 2) * 4 + g4;  // chunk of columns dt*16 + g4*4 ..
          *reinterpret_cast<float4*>(stage + i16 * (D * 2) + (c ^ i16) * 16) =
              float4{oacc[dt][0] * inv, oacc[dt][1] * inv, oacc[dt][2] * inv, oacc[dt][3] * inv};
        }
        drain(dst, h * (D * 2));
      }
    };
    if (nchunks > 1) {
      // One chunk of a split query block: normalised partial and LSE of row
      // (wave, query column) for prefill_combine_kernel; the wave's 16 rows
      // are contiguous.
      const int64_t slot = ((int64_t)ysub * nqb + qblk) * p.max_chunks + chunk;
      unsigned char* prows = reinterpret_cast<unsigned char*>(p.part + (slot * kRows8 + wave * kQ8) * D);
      store_f32([&](int r) -> unsigned char* { return prows + r * (D * 4); });
      if (g4 == 0) p.lse[slot * kRows8 + wave * kQ8 + i16] = l_run > 0.f ? fast_log2(l_run) + m_ref : -INFINITY;
      BT_TL_END();
      return;
    }
    auto out_row = [&](int r) -> unsigned char* {
      if (q0 + r >= S) return nullptr;
      const int64_t e = (int64_t)(q0 + r) * p.out_stride_tok + (int64_t)head * p.out_stride_head;
      return reinterpret_cast<unsigned char*>(p.out) + e * (p.out_bf16 ? 2 : 4);
    };
    if (p.out_bf16) {
  #pragma unroll
      for (int dt = 0; dt < kDTiles; ++dt) {
        const u32x2 pk2 = {f32x2_to_bf16x2_bits(oacc[dt][0] * inv, oacc[dt][1] * inv),
                           f32x2_to_bf16x2_bits(oacc[dt][2] * inv, oacc[dt][3] * inv)};
        const int c = dt * 2 + (g4 >> 1);  // chunk of columns dt*16 + g4*4 ..
        *reinterpret_cast<u32x2*>(stage + i16 * (D * 2) + (c ^ i16) * 16 + (g4 & 1) * 8) = pk2;
      }
      drain(out_row, 0);
    } else {
      store_f32(out_row);
    }
    BT_TL_END();
  };
  auto n_blocks = [&](int qb) { return (P0 + min(S, (qb + 1) * pos_per_wg) + kKB8 - 1) / kKB8; };
  if constexpr (PAIRED) {
    // Paired split: query blocks nqb-1-r and r (r = blockIdx.x / parts) form
    // a pair with about the same number of key blocks for every r; the pair's
    // blocks (those of nqb-1-r, then those of r) are cut into `parts` equal
    // ranges, one per work-group, so each covers at most two segments.
    const int parts = p.pair_parts;
    const int r = (int)blockIdx.x / parts, k = (int)blockIdx.x % parts;
    const int qhi = nqb - 1 - r, qlo = r;
    const int nhi = n_blocks(qhi), nlo = qlo != qhi ? n_blocks(qlo) : 0;
    const int size = (nhi + nlo + parts - 1) / parts;
    const int r0 = k * size, r1 = min(nhi + nlo, r0 + size);
    if (r0 >= r1) return;
    if (r0 < nhi) segment(qhi, r0, min(nhi, r1), k, (nhi + size - 1) / size);
    if (r1 > nhi) {
      if (r0 < nhi) __syncthreads();  // every wave is done with the first segment's tiles
      const int kfirst = nhi / size;   // the pair's first part that reaches block qlo
      segment(qlo, max(0, r0 - nhi), r1 - nhi, k - kfirst, (nhi + nlo - 1) / size - kfirst + 1);
    }
  } else {
    // Key blocks of this work-group: all of its query block's (heavy blocks
    // first), or one chunk of them.
    if (p.kb_chunk > 0) {
      if (!p.split_compact) {  // grid (query block, subset, chunk)
        split_qb = nqb - 1 - (int)blockIdx.x;
        split_chunk = blockIdx.z;
      }
      const int nkb = n_blocks(split_qb);
      const int kb0 = split_chunk * p.kb_chunk;
      if (kb0 >= nkb) return;  // this query block has fewer chunks (whole work-group)
      segment(split_qb, kb0, min(nkb, kb0 + p.kb_chunk), split_chunk, (nkb + p.kb_chunk - 1) / p.kb_chunk);
    } else {
      const int qblk = nqb - 1 - (int)blockIdx.x;
      segment(qblk, 0, n_blocks(qblk), 0, 1);
    }
  }
}


// LSE merge of the chunks of split query blocks (the combine of the
// reference's split decode, attention.py:168-189, applied per query row):
// out = sum_c 2^(lse_c - m) part_c / sum_c 2^(lse_c - m).  Work-group
// (query block, kv head, z) merges 256 consecutive (row, 4 columns) items;
// each thread issues the loads of up to 8 chunks before it adds them.  Query
// blocks with a single chunk were written directly by the main kernel.
template <int D>
__global__ __launch_bounds__(256) void prefill_combine_kernel(PrefillParams p) {
  constexpr int kD4 = D / 4;
  constexpr int kRowsPerGroup = 256 / kD4;  // rows whose items one work-group merges
  constexpr int kBatch = 8;                 // chunks whose loads are in flight together
  const int G = p.sub_group;
  const int pos_per_wg = kQ8 * (kWaves8 / G);
  const int S = p.seqlen;
  const int nqb = (S + pos_per_wg - 1) / pos_per_wg;
  const int qblk = nqb - 1 - (int)blockIdx.x;
  const int ysub = blockIdx.y;  // (kv head, head subset), as in the main kernel
  const int wg_q0 = qblk * pos_per_wg;
  auto n_blocks = [&](int qb) { return (p.q_offset + min(S, (qb + 1) * pos_per_wg) + kKB8 - 1) / kKB8; };
  const int nchunks = p.pair_parts > 0 ? pair_chunks(qblk, nqb, p.pair_parts, n_blocks)
                                       : (n_blocks(qblk) + p.kb_chunk - 1) / p.kb_chunk;
  if (nchunks <= 1) return;
  const int64_t slot0 = ((int64_t)ysub * nqb + qblk) * p.max_chunks;
  const int t = threadIdx.x;
  const int row = (int)blockIdx.z * kRowsPerGroup + t / kD4;
  const int d = (t % kD4) * 4;
  const int w = row / kQ8;
  const int q = wg_q0 + (w / G) * kQ8 + (row % kQ8);
  if (q >= S) return;
  const float* lse = p.lse + slot0 * kRows8 + row;
  const float* base = p.part + (slot0 * kRows8 + row) * D + d;
  const int64_t cstride = (int64_t)kRows8 * D;  // floats between chunks of one row
  // Every thread loads its row's LSEs and partial slices of a batch of chunks
  // at once (one memory round trip per batch) and merges online across
  // batches.  A chunk without keys for the row has lse = -inf: its slice is
  // selected away, never multiplied (the slice of a chunk that exited early
  // was never written).
  float m = -INFINITY, sum = 0.f;
  float4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int c0 = 0; c0 < nchunks; c0 += kBatch) {
    float l[kBatch];
    float4 v[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const bool in = c0 + j < nchunks;
      l[j] = in ? lse[(int64_t)(c0 + j) * kRows8] : -INFINITY;
      v[j] = in ? *reinterpret_cast<const float4*>(base + (c0 + j) * cstride) : float4{0.f, 0.f, 0.f, 0.f};
    }
    float mb = m;
#pragma unroll
    for (int j = 0; j < kBatch; ++j) mb = fmaxf(mb, l[j]);
    if (mb == -INFINITY) continue;  // no keys yet for this row
    const float r = fast_exp2(m - mb);  // m = -inf before the first keys: r = 0
    sum *= r;
    acc.x *= r; acc.y *= r; acc.z *= r; acc.w *= r;
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      if (l[j] != -INFINITY) {
        const float wc = fast_exp2(l[j] - mb);
        sum += wc;
        acc.x += wc * v[j].x; acc.y += wc * v[j].y; acc.z += wc * v[j].z; acc.w += wc * v[j].w;
      }
    }
    m = mb;
  }
  const float inv = sum > 0.f ? 1.f / sum : 0.f;
  acc.x *= inv; acc.y *= inv; acc.z *= inv; acc.w *= inv;
  const int head = (ysub / p.head_subs) * p.group + (ysub % p.head_subs) * G + w % G;
  const int64_t orow = (int64_t)q * p.out_stride_tok + (int64_t)head * p.out_stride_head;
  if (p.out_bf16) {
    const u32x2 pk2 = {f32x2_to_bf16x2_bits(acc.x, acc.y), f32x2_to_bf16x2_bits(acc.z, acc.w)};
    *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(p.out) + orow + d) = pk2;
  } else {
    *reinterpret_cast<float4*>(reinterpret_cast<float*>(p.out) + orow + d) = acc;
  }
}

PrefillSplitPlan prefill8_split_plan(int seqlen, int q_offset, int group, int kv_heads, int head_dim, int num_cus) {
  PrefillSplitPlan plan;
  const int pos_per_wg = kQ8 * (kWaves8 / group);
  const int nqb = (seqlen + pos_per_wg - 1) / pos_per_wg;
  plan.query_blocks = nqb;
  if (nqb < 1 || kv_heads < 1 || num_cus < 1) return plan;
  auto n_blocks = [&](int qb) { return (q_offset + min(seqlen, (qb + 1) * pos_per_wg) + kKB8 - 1) / kKB8; };
  int nkb_max = 0;
  for (int qb = 0; qb < nqb; ++qb) nkb_max = max(nkb_max, n_blocks(qb));
  // The uniform split.  Its grid (query blocks x kv heads x max_chunks) must
  // fit the CUs in one round, counting the slots of chunks that start past a
  // query block's keys and exit at once: at config 4, S = 1024, 3-block chunks
  // (384 slots) took 45.5 us against 34.4 us for 4-block chunks (256 slots)
  // and 44.2 us unsplit; at S = 2048, 16-block chunks (256 slots) took 54.7 us
  // against 62.9 us for 11-block chunks (384 slots) and 71.5 us unsplit.
  // A chunk may be a single key block: with the staged epilogue (partials
  // stored as whole row slices) one-block chunks beat two-block ones at
  // config 4, S = 128 / 192 / 256 / 384 / 512: 13.8 / 16.6 / 17.9 / 19.3 /
  // 20.0 -> 13.2 / 14.1 / 14.8 / 16.1 / 18.6 us per call (before it, S = 128
  // measured 24.5 against 22.3 us).  A query block has at most kMaxChunks.  A grid with a work-group per CU or more is not split
  // (the heavy-first launch order balances it as far as it can).
  int uniform = 0;          // its chunk length (0: no uniform split)
  int longest = nkb_max;    // key blocks of the busiest work-group
  bool compact = false;
  if ((int64_t)nqb * kv_heads < num_cus) {
    const int max_chunks = min(num_cus / (nqb * kv_heads), kMaxChunks);
    const int lo = (nkb_max + max_chunks - 1) / max_chunks;
    if (lo < nkb_max) {
      uniform = lo;
      longest = lo;
    }
  }
  // Two-block chunks convert their tiles in the work-group (no pre-pass, see
  // DIRECT); they are taken over longer chunks while their grid stays within
  // 1.6 rounds of the CUs: config 4, S = 768 / 896 24.5 / 27.2 -> 22.6 / 25.9
  // us per call (288 / 392 slots); at S = 1024 (two full rounds, 512 slots)
  // 27.8 -> 38.6 us.
  if (nkb_max > 2 && (uniform == 0 || uniform > 2) && (nkb_max + 1) / 2 <= kMaxChunks &&
      5 * (int64_t)nqb * kv_heads * ((nkb_max + 1) / 2) <= 8 * (int64_t)num_cus) {
    uniform = 2;
    longest = 2;
  }
  // The compact grid drops the slots of chunks past a query block's keys, so
  // shorter chunks fit one round; it is taken where that shortens a work-group
  // by over 15%, counting ~4 key blocks of fixed cost per segment: config 4,
  // S = 1280 / 1536 / 2048 32.1 / 39.4 / 46.9 -> 30.6 / 34.2 / 43.3 us per
  // call (chunks of 7 / 12 / 16 -> 4 / 6 / 12 blocks).  Where it would not,
  // it measured slower (S = 128 / 512 / 1024 +0.5 / +0.6 / +0.6 us).
  if (uniform > 0 && 2 * (int64_t)nqb * kv_heads <= num_cus) {
    for (int kb = 1; kb < uniform; ++kb) {
      const int mc = (nkb_max + kb - 1) / kb;
      if (mc <= kMaxChunks &&
          (int64_t)kv_heads * split_items(kb, seqlen, q_offset, pos_per_wg, nqb, mc) <= num_cus) {
        if (100 * (kb + 4) < 85 * (uniform + 4)) {
          uniform = kb;
          longest = kb;
          compact = true;
        }
        break;
      }
    }
  }
  // The paired split balances the causal triangle: a pair of query blocks
  // has about the same key blocks for every pair.  It pays a second q load
  // and epilogue in work-groups that cover two segments, more partials, and a
  // fuller machine per block; it replaces the unsplit grid when its longest
  // range is under two thirds of the busiest query block's (config 4: S = 3000
  // and 4096 gain 12% and 17%) and at least two blocks long.  Where the
  // uniform split applies it measured no better (S = 2048: 9 against 16
  // blocks, 60.0 vs 59.4 us).
  const int npairs = (nqb + 1) / 2;
  const int parts = max(1, min(num_cus / (npairs * kv_heads), kMaxChunks));
  int pair_longest = 0;
  for (int r = 0; r < npairs; ++r) {
    const int qhi = nqb - 1 - r;
    const int len = n_blocks(qhi) + (r != qhi ? n_blocks(r) : 0);
    pair_longest = max(pair_longest, (len + parts - 1) / parts);
  }
  if (uniform == 0 && pair_longest >= 2 && 3 * pair_longest < 2 * longest) {
    plan.pair_parts = parts;
    int mc = 1;
    for (int qb = 0; qb < nqb; ++qb) mc = max(mc, pair_chunks(qb, nqb, parts, n_blocks));
    plan.max_chunks = mc;
  } else if (uniform > 0) {
    plan.kb_chunk = uniform;
    plan.compact = compact ? 1 : 0;
    plan.max_chunks = (nkb_max + uniform - 1) / uniform;
  } else {
    return plan;
  }
  if (plan.uses_partials()) {
    plan.part_rows = (size_t)kv_heads * nqb * plan.max_chunks * kRows8;
    plan.part_bytes = plan.part_rows * ((size_t)head_dim * 4 + 4);
  }
  return plan;
}

bool prefill8_serves(int group, int head_dim) {
  return group >= 1 && group <= 8 && (head_dim == 128 || head_dim == 256);
}

int prefill8_sub_group(int group) { return group & -group; }  // largest power of two dividing it

hipError_t launch_prefill8(const PrefillParams& p, int head_dim, hipStream_t stream) {
  if (p.sub_group < 1 || p.head_subs < 1 || p.sub_group * p.head_subs != p.group || kWaves8 % p.sub_group)
    return hipErrorInvalidValue;
  const int pos_per_wg = kQ8 * (kWaves8 / p.sub_group);
  const int nqb = (p.seqlen + pos_per_wg - 1) / pos_per_wg;
  const bool paired = p.pair_parts > 0;
  const bool split = p.kb_chunk > 0 || (paired && p.max_chunks > 1);  // partials and the combine
  if (paired && p.kb_chunk > 0) return hipErrorInvalidValue;
  if (split && (p.max_chunks < 1 || p.max_chunks > kMaxChunks || !p.part || !p.lse)) return hipErrorInvalidValue;
  const int ys = p.kv_heads * p.head_subs;  // grid y: (kv head, head subset)
  const dim3 grid = paired ? dim3(((nqb + 1) / 2) * p.pair_parts, ys, 1)
                   : p.kb_chunk > 0 && p.split_compact
                       ? dim3(ys * split_items(p.kb_chunk, p.seqlen, p.q_offset, pos_per_wg, nqb, p.max_chunks), 1, 1)
                       : dim3(nqb, ys, p.kb_chunk > 0 ? p.max_chunks : 1);
  // The combine's work-groups run the query blocks heaviest first; under the
  // uniform split only the heaviest ones have more than one chunk (a query
  // block's key blocks grow with its index), so its grid stops there -- at a
  // multiple of 8 work-groups in x, which keeps each query block's merge on
  // the XCD (work-group id mod 8) whose L2 holds its partials when nqb is a
  // multiple of 8: C4 S = 2048 50.5 -> 48.5 us per call; S = 512 with 12 of
  // its 16 columns took 22.8 against 21.7 us.
  int cx = nqb;
  if (p.kb_chunk > 0) {
    cx = 0;
    for (int qb = nqb - 1; qb >= 0; --qb) {
      const int nkb = (p.q_offset + min(p.seqlen, (qb + 1) * pos_per_wg) + kKB8 - 1) / kKB8;
      if (nkb <= p.kb_chunk) break;
      ++cx;
    }
    cx = min(nqb, (cx + 7) & ~7);
  }
  const dim3 cgrid(cx, ys, kRows8 * head_dim / 4 / 256);
  // Work-groups with at most two key blocks each convert them themselves,
  // unless the caller keeps the images for later chunks.
  const int longest = (p.q_offset + p.seqlen + kKB8 - 1) / kKB8;
  const bool direct = !p.keep_images && !paired && (p.kb_chunk > 0 ? p.kb_chunk : longest) <= 2;
  if (!direct) {
    const hipError_t vt_rc = launch_prefill_vts(p, head_dim, stream);
    if (vt_rc != hipSuccess) return vt_rc;
  }
  auto launch = [&](auto dsel, auto losel) {
    constexpr int Dk = decltype(dsel)::value;
    constexpr bool LOk = decltype(losel)::value;
    if (paired) hipLaunchKernelGGL((gqa_prefill8_kernel<Dk, false, true, LOk>), grid, dim3(kWaves8 * 64), 0, stream, p);
    else if (direct) hipLaunchKernelGGL((gqa_prefill8_kernel<Dk, true, false, LOk>), grid, dim3(kWaves8 * 64), 0, stream, p);
    else hipLaunchKernelGGL((gqa_prefill8_kernel<Dk, false, false, LOk>), grid, dim3(kWaves8 * 64), 0, stream, p);
    if (split && cx > 0) hipLaunchKernelGGL(prefill_combine_kernel<Dk>, cgrid, dim3(256), 0, stream, p);
  };
  // f32 q takes the two-term (hi + lo) Q.K^T; bf16 q converts to fp16 exactly.
  switch (head_dim) {
    case 128:
      if (p.q_f32) launch(Buf8<128>{}, BoolC<true>{}); else launch(Buf8<128>{}, BoolC<false>{});
      break;
    case 256:
      if (p.q_f32) launch(Buf8<256>{}, BoolC<true>{}); else launch(Buf8<256>{}, BoolC<false>{});
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace bt

#ifdef BT_TIMELINE
// Timeline build only (libbt_timeline.so, built beside the product library,
// never loaded by it): copy out or clear the recorded timestamps.
extern "C" int bt_timeline_read(unsigned long long* host, int n) {
  if (n < 0 || n > bt::kTimelineSlots) return -22;
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(bt::bt_tl_buf), (size_t)n * 8, 0, hipMemcpyDeviceToHost) == hipSuccess ? 0 : -1;
}
extern "C" int bt_timeline_clear() {
  static unsigned long long zero[bt::kTimelineSlots];
  return hipMemcpyToSymbol(HIP_SYMBOL(bt::bt_tl_buf), zero, sizeof(zero), 0, hipMemcpyHostToDevice) == hipSuccess ? 0 : -1;
}
#endif
