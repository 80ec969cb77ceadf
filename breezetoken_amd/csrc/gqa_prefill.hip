// Causal GQA prefill attention for gfx950 (MI355X) on MFMA.
//
// Computes, for every new query row i (absolute position p0 + i, where p0 =
// q_offset tokens are already in the cache) and every query head h (kv head
// g = h / G),
//     out[i, h] = softmax_{j <= p0+i} (q_i . k_j * scale) . V_j
// over the p0 + S keys of the cache -- the F.scaled_dot_product_attention
// (is_causal=True, enable_gqa=True) call of _prefill_attn (breezetoken/model/
// prefill.py:56-68, p0 = 0) and the banded-mask chunked prefill of
// Qwen36MoE._attn_batch (breezetoken/model/qwen36_moe.py:394-428).
//
// Decomposition (MI355X-first):
//  * a small pre-pass (gqa_prefill_vt.hip, key order kVtOrder32) writes K and
//    V once per kv head as fp16 images (V transposed), each scaled by a power
//    of two per 64-key block, so the key loop needs neither a conversion nor
//    a transposing LDS read, and every finite bf16 K and V fits fp16;
//  * one work-group (4 waves) per (block of query positions, kv head); wave w
//    owns query head w of the GQA group (and, for G < 4, a different block of
//    positions), so every K/V tile staged in LDS feeds all G heads;
//  * K and V^T tiles go HBM -> LDS by buffer_load ... lds (no staging
//    registers, no LDS write instructions); K lands chunk-major (16-byte chunk
//    c of key row r at c * 1024 + r * 16), which keeps the MFMA operand reads
//    conflict-free and needs only a per-lane row offset into the image;
//  * S^T = K . Q^T on v_mfma_f32_32x32x16_f16 (64 keys x 32 queries per
//    block, Q^T in registers: q, f32 or bf16, scaled per row by a power of two
//    and rounded to fp16; the softmax takes the q and K factors back in its
//    exp2 argument); O^T = V^T . P^T on v_mfma_f32_32x32x16_f16 with
//    P (<= 2^8, see below) rounded to fp16 -- bf16's 8-bit mantissa would put
//    the first rows of the prompt above a 2e-3 error -- and the lane that owns
//    a score column owns the P^T operand for it, so P never moves between lanes;
//  * online softmax in the log2 domain with lazy rescaling: the reference
//    maximum only moves (and O^T is only rescaled) when a score exceeds it by
//    more than 2^8, so almost every key block skips the 128-register rescale;
//    only blocks that reach past a wave's first query apply the causal mask;
//  * double-buffered tiles with two barriers per 64-key step: the step of
//    block kb multiplies S_kb = K_kb . Q^T beside the exponentials of the
//    second half of P_{kb-1}, then O += V_{kb-1} . P_{kb-1} beside the max and
//    first-half exponentials of S_kb, so both matrix-core phases have VALU
//    work interleaved.  Each tile copy is issued as soon as the barrier that
//    ends its buffer's last reader has passed (V_kb at the start of step kb,
//    K_{kb+2} at its middle), so a copy has about one and a half steps to
//    land before the barrier that publishes it;
//  * heavy (late) query blocks are launched first to balance the causal work.
#include "bt_common.h"
#include "bt_kernels.h"

namespace bt {

namespace {

typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float2v __attribute__((ext_vector_type(2)));

template <int B>
struct Buf {
  static constexpr int value = B;
};

constexpr int kQB = 32;                 // query positions per wave
constexpr int kKB = kPrefillKeyBlock;   // keys per block (64)
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
// HBM -> LDS copy of 16 bytes per lane: lane l's bytes at voff + soff land at
// lds + 16 * l (lds is wave-uniform).  Offsets past the descriptor's range
// (soffset included) read as zero.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, unsigned char* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (BT_LDS void*)lds, 16, (int)voff, (int)soff, 0, 0);
}

// Two floats -> packed fp16 pair, round to nearest even (one v_cvt_pk_f16_f32).
// A builtin, not asm: the compiler must see this VALU write to insert the wait
// states a VGPR needs after an in-flight MFMA has read it as an operand.
__device__ __forceinline__ uint32_t pack_f16_rne(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((float2v){a, b}, half2v));
}

// Instruction-group ordering for the scheduler (masks: 0x2 VALU, 0x8 MFMA,
// 0x100 DS read).  With one wave per SIMD the matrix core only overlaps VALU
// and LDS work that sits between MFMAs in program order, so each MFMA is
// followed by a share of the independent work.
template <int kMfma, int kAhead, int kValu, int kVmem>
__device__ __forceinline__ void interleave() {
  __builtin_amdgcn_sched_group_barrier(0x100, kAhead, 0);  // operands of the first MFMAs
#pragma unroll
  for (int i = 0; i < kMfma; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if (i + kAhead < kMfma) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    if (kValu) __builtin_amdgcn_sched_group_barrier(0x002, kValu, 0);
    if (kVmem && i < kVmem) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
  }
}

}  // namespace

// D: head dim (128 or 256).  Wave w of a work-group handles query head
// (pass * 4 + w % GW) of the group and positions [q0 + (w / GW) * 32, +32),
// GW = min(G, 4); groups of 8 heads take two passes over the keys.
template <int D>
__global__ __launch_bounds__(kWaves * 64, 1) void gqa_prefill_kernel(PrefillParams p) {
  constexpr int kSteps = D / 16;       // K-dimension steps of Q.K^T (16 per MFMA)
  constexpr int kDTiles = D / 32;      // 32-wide d tiles of O^T
  constexpr int kImg = kKB * D * 2;    // bytes of one K or V^T tile
  constexpr int kCopies = kImg / 1024 / kWaves;  // 1 KiB copies per wave per tile

  // Four separate LDS arrays (not offsets into one) so the compiler can see
  // that copies into one buffer never alias MFMA operand reads from another:
  // it neither orders them nor waits for the copies before those reads.  The
  // key loop is unrolled by two so every buffer choice is a constant.
  __shared__ __attribute__((aligned(1024))) unsigned char k_lds0[kImg];
  __shared__ __attribute__((aligned(1024))) unsigned char k_lds1[kImg];
  __shared__ __attribute__((aligned(1024))) unsigned char v_lds0[kImg];
  __shared__ __attribute__((aligned(1024))) unsigned char v_lds1[kImg];
  auto k_buf = [&](auto b) -> unsigned char* {
    if constexpr (decltype(b)::value == 0) return k_lds0; else return k_lds1;
  };
  auto v_buf = [&](auto b) -> unsigned char* {
    if constexpr (decltype(b)::value == 0) return v_lds0; else return v_lds1;
  };

  asm volatile("" ::"s"(p.q), "s"(p.k), "s"(p.vt), "s"(p.out), "s"(p.seqlen), "s"(p.group),
               "s"(p.q_stride_tok), "s"(p.q_stride_head), "s"(p.kv_stride_tok), "s"(p.kv_stride_head),
               "s"(p.out_stride_tok), "s"(p.out_stride_head), "s"(p.scale_log2));
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int kvh = blockIdx.y;
  const int G = p.group;
  const int GW = G < kWaves ? G : kWaves;
  const int pos_per_wg = kQB * (kWaves / GW);
  const int S = p.seqlen;                 // new query rows
  const int P0 = p.q_offset;              // absolute position of query row 0
  const int nkeys = P0 + S;
  const int nqb = (S + pos_per_wg - 1) / pos_per_wg;
  const int nblk = (nkeys + kKB - 1) / kKB;
  const int qblk = nqb - 1 - (int)blockIdx.x;  // heavy blocks first
  const int wg_q0 = qblk * pos_per_wg;
  const int q0 = wg_q0 + (wave / GW) * kQB;   // this wave's first position
  const int wg_qend = min(S, wg_q0 + pos_per_wg);
  // keys needed by the work-group: [0, P0 + wg_qend)
  const int nkb = (P0 + wg_qend + kKB - 1) / kKB;
  const int last = nkb - 1;

  // Tile copies.  K copy i (1 KiB) is 16-byte chunk i of the 64 key rows, lane
  // l taking row l, from the pre-pass's row-major fp16 K image (chunk i of row
  // l sits in slot i ^ (l & 15)); V^T copy i is bytes [1024 i, +1024) of the
  // block's image.  Wave w issues copies w, w + 4, ...
  constexpr int kRowBytes = D * 2;
  const size_t head_img = (size_t)kvh * p.img_blocks * kKB * D;  // this kv head's images
  const __amdgpu_buffer_rsrc_t krs = make_rsrc(p.kimg + head_img, (uint32_t)nblk * kImg);
  const __amdgpu_buffer_rsrc_t vrs = make_rsrc(p.vt + head_img, (uint32_t)nblk * kImg);
  const int* vexp = p.vexp + kvh * p.img_blocks;
  const int* kexp = p.kexp + kvh * p.img_blocks;
  const uint32_t v_voff = (uint32_t)lane * 16;
  auto copy_k = [&](auto b, int kb) {
    const uint32_t so = (uint32_t)kb * kImg;
#pragma unroll
    for (int j = 0; j < kCopies; ++j) {
      const int i = wave + kWaves * j;
      dma16(krs, k_buf(b) + i * 1024, (uint32_t)lane * kRowBytes + (uint32_t)((i ^ (lane & 15)) * 16), so);
    }
  };
  auto copy_v = [&](auto b, int kb) {
    const uint32_t so = (uint32_t)kb * kImg;
#pragma unroll
    for (int j = 0; j < kCopies; ++j) {
      const int i = wave + kWaves * j;
      dma16(vrs, v_buf(b) + i * 1024, v_voff, so + (uint32_t)i * 1024);
    }
  };
  // Each wave waits for its own copies; the barrier that follows publishes
  // them to the other waves.  wait_all: vmcnt(0).  wait_older: all but the
  // 2 * kCopies youngest copies of this wave (the two tiles issued since).
  auto wait_all = [] { __builtin_amdgcn_s_waitcnt(0x0f70); };
  constexpr int kYoung = 2 * kCopies;
  constexpr int kWaitOlder = 0x0f70 | (kYoung & 0xf) | ((kYoung >> 4) << 14);
  static_assert(kYoung < 64, "vmcnt holds 6 bits");
  auto wait_older = [] { __builtin_amdgcn_s_waitcnt(kWaitOlder); };
  // Work-group barrier without the release/acquire fence of __syncthreads:
  // that fence would wait for every copy in flight (vmcnt(0)), while the waits
  // above need only the tiles the next phase reads.  The LDS reads before it
  // have all been consumed by MFMAs; lgkmcnt(0) makes that explicit.
  auto barrier = [] { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };

  const int qcol = lane & 31;       // this lane's query column
  const int kgrp = lane >> 5;       // k-slot group of MFMA operands

  const int passes = (G + kWaves - 1) / kWaves;
  for (int pass = 0; pass < passes; ++pass) {
    const int head_local = pass * kWaves + wave % GW;
    // Waves past the group (or past the prompt) run the same instruction stream
    // on clamped indices and store nothing; their keys beyond their queries are
    // masked like any causal key, so no branch is needed inside the key loop.
    const bool wave_active = wave < GW * (kWaves / GW) && head_local < G && q0 < S;
    const int head = kvh * G + min(head_local, G - 1);
    // Block scale exponents (K, V^T) of the block being softmaxed, read
    // through the scalar cache a block ahead of their use.
    auto scales = [&](int kb, int& ek, int& eb) {
      const int b = min(kb, last);
      ek = sload(kexp, b);
      eb = sload(vexp, b);
    };
    int ek_c, eb_c;
    scales(0, ek_c, eb_c);
    // The first tiles go out before the q loads, so the two latencies overlap.
    copy_k(Buf<0>{}, 0);
    copy_k(Buf<1>{}, min(1, last));
    copy_v(Buf<0>{}, 0);

    // ---- Q^T operand in registers: lane holds Q[q0 + qcol][d = st*16 + kgrp*8 .. +8]
    // as fp16, the row scaled by 2^-eq so its largest |q| lies in [2^14,
    // 2^15); c_col = scale * log2(e) * 2^eq restores it in the exp2 argument.
    u32x4 qop[kSteps];
    float c_col;
    {
      const int qrow = min(q0 + qcol, S - 1);
      const int64_t off = (int64_t)qrow * p.q_stride_tok + (int64_t)head * p.q_stride_head + kgrp * 8;
      const int eq = q_row_f16(p.q, p.q_f32 != 0, off, 16, qop, [](uint32_t mx) {
        return xor_umax<32>(mx);  // the row's two lane halves
      });
      c_col = __builtin_ldexpf(p.scale_log2, eq);
    }
    float c_blk = c_col;  // log2-domain factor of the latest block's scaled scores

    floatx16 oacc[kDTiles];
#pragma unroll
    for (int i = 0; i < kDTiles; ++i)
#pragma unroll
      for (int j = 0; j < 16; ++j) oacc[i][j] = 0.f;
    float m_ref = -INFINITY;  // reference max (log2 domain) of this lane's column
    float l_run = 0.f;        // partial row sum over this lane's keys
    int e_run = kVExpZero;    // V scale O is kept in: O_true = O * 2^e_run
    int tail_shift = 0;       // P' = P * 2^tail_shift of the pending keys 32..63
    const int my_q = q0 + qcol;       // this lane's query row
    const int my_pos = P0 + my_q;     // its absolute position: keys 0..my_pos
    // P of a key block as fp16 pairs: pk0 holds keys 0..31 of the block, pk1
    // keys 32..63 (the two 32-key halves of the S^T registers).
    uint32_t pk0[8], pk1[8];
    floatx16 s_tail;          // S^T of the latest block's keys 32..63, pending exp
    float neg_m_tail = 0.f;   // -reference max those scores are exponentiated with

    // S^T (64 keys x 32 queries) = K . Q^T from K buffer b: the A operand of
    // step st / key half mt is chunk 2*st + kgrp of key row mt*32 + qcol.
    auto qk = [&](auto b, floatx16 (&sacc)[2]) {
      const unsigned char* krow = k_buf(b) + kgrp * 1024 + qcol * 16;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int j = 0; j < 16; ++j) sacc[mt][j] = 0.f;
#pragma unroll
      for (int st = 0; st < kSteps; ++st) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const u32x4 a = *reinterpret_cast<const u32x4*>(krow + st * 2048 + mt * 512);
          sacc[mt] = mfma32_f16(a, qop[st], sacc[mt]);
        }
      }
    };
    // O^T += V^T . P^T over the 64 keys of V^T buffer b: the A operand of key
    // step ks / d tile dt is key chunk 2*ks + kgrp of row dt*32 + (lane % 32),
    // whose key order matches the P^T operand built from the S^T registers.
    auto pv = [&](auto b, const uint32_t(&p0)[8], const uint32_t(&p1)[8]) {
      const unsigned char* vrow = v_buf(b) + kgrp * (D * 16) + qcol * 16;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const uint32_t* ph = (ks < 2 ? p0 : p1) + (ks & 1) * 4;
        const u32x4 pop = {ph[0], ph[1], ph[2], ph[3]};
#pragma unroll
        for (int dt = 0; dt < kDTiles; ++dt) {
          const u32x4 a = *reinterpret_cast<const u32x4*>(vrow + ks * 2 * (D * 16) + dt * 512);
          oacc[dt] = mfma32_f16(a, pop, oacc[dt]);
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
          sacc[mt][j] = key <= my_pos ? sacc[mt][j] : -INFINITY;
        }
    };
    // exp2(s * c - m) of one 32-key half into fp16 pairs; returns the sum.
    auto exp_half = [&](const floatx16& s, float neg_m, uint32_t(&out)[8]) -> float {
      float psum = 0.f;
#pragma unroll
      for (int j = 0; j < 16; j += 2) {
        const float p0 = fast_exp2(fmaf(s[j], c_blk, neg_m));
        const float p1 = fast_exp2(fmaf(s[j + 1], c_blk, neg_m));
        psum += p0 + p1;
        out[j / 2] = pack_f16_rne(p0, p1);
      }
      return psum;
    };
    // Online softmax, first part: block max, lazy reference-max update, P of
    // keys 0..31 into out.  Returns the factor the accumulated O must be
    // scaled by (1 unless the reference max or the V scale moved).  Keys
    // 32..63 follow in softmax_tail beside the next block's S = K.Q^T.  The
    // V^T block's power-of-two scale enters P' = P * 2^shift through the exp2
    // bias; the row sum takes P.
    auto softmax_head = [&](floatx16(&sacc)[2], uint32_t(&out)[8], int ek, int eb) -> float {
      float tmax = -INFINITY;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int j = 0; j < 16; ++j) tmax = fmaxf(tmax, sacc[mt][j]);
      c_blk = __builtin_ldexpf(c_col, ek);  // with the K block's scale
      tmax = halves_max(tmax) * c_blk;
      // lazy reference max: move it only when a score exceeds it by > kLazy
      const bool move = tmax > m_ref + kLazy;
      const float m_new = move ? tmax : m_ref;
      const float alpha = move ? fast_exp2(m_ref - m_new) : 1.f;  // 0 when m_ref is -inf
      m_ref = m_new;
      const int e_new = vexp_next(e_run, eb);
      tail_shift = vexp_shift(e_new, eb);
      neg_m_tail = (m_ref == -INFINITY ? 0.f : -m_ref) + (float)tail_shift;
      float psum = exp_half(sacc[0], neg_m_tail, out);
      if (tail_shift != 0) psum = __builtin_ldexpf(psum, -tail_shift);  // wave-uniform, rare
      l_run = l_run * alpha + psum;
      s_tail = sacc[1];
      const float factor = e_new != e_run ? __builtin_ldexpf(alpha, e_run - e_new) : alpha;
      e_run = e_new;
      return factor;
    };
    auto softmax_tail = [&] {
      float psum = exp_half(s_tail, neg_m_tail, pk1);
      if (tail_shift != 0) psum = __builtin_ldexpf(psum, -tail_shift);
      l_run += psum;
    };
    auto rescale = [&](float alpha) {
      if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {  // rare: the max moved by > 2^8
#pragma unroll
        for (int i = 0; i < kDTiles; ++i) oacc[i] *= alpha;
      }
    };
    // Blocks whose last key is <= the wave's first position need no mask.
    const int kb_diag = (P0 + q0 + 1) / kKB;

    // Copy schedule (double-buffered tiles, copies issued as soon as their
    // buffer is free, so each has about one and a half steps to land):
    //   start of step kb:       V_kb      -> V buffer kb % 2 (held V_{kb-2}, read in step kb-1)
    //   after the mid barrier:  K_{kb+2}  -> K buffer kb % 2 (held K_kb, read in phase A)
    //   mid barrier of step kb: V_{kb-1} has landed (all but the 2 youngest tiles)
    //   end barrier of step kb: K_{kb+1} has landed (likewise)
    // Copies past the last block re-read the last block (min(., last)) into a
    // buffer nobody reads, so the key loop has no branches around its copies.
    wait_all();
    __syncthreads();

    // Block 0: S_0, then K_2 into K buffer 0, first softmax part.
    {
      floatx16 sacc[2];
      qk(Buf<0>{}, sacc);
      barrier();  // every wave is done reading K_0
      copy_k(Buf<0>{}, min(2, last));
      if (0 >= kb_diag) mask(0, sacc);
      int ek_n, eb_n;
      scales(1, ek_n, eb_n);
      rescale(softmax_head(sacc, pk0, ek_c, eb_c));
      ek_c = ek_n;
      eb_c = eb_n;
      barrier();  // K_1 landed in the prologue
    }
    // Block kb (buffer b = kb % 2), two matrix-core phases with VALU work
    // beside each:
    //   A: S_kb = K_kb . Q^T       beside  P_{kb-1} of keys 32..63
    //   B: O += V_{kb-1} . P_{kb-1} beside  max of S_kb, P_kb of keys 0..31
    auto step = [&](auto b, int kb) {
      constexpr int B = decltype(b)::value;
      copy_v(b, kb);
      int ek_n, eb_n;
      scales(kb + 1, ek_n, eb_n);
      floatx16 sacc[2];
      qk(b, sacc);
      softmax_tail();
      interleave<kSteps * 2, 4, 2, kCopies>();
      wait_older();  // V_{kb-1}
      barrier();
      copy_k(b, min(kb + 2, last));
      if (kb >= kb_diag) mask(kb, sacc);
      pv(Buf<B ^ 1>{}, pk0, pk1);
      uint32_t pk0_next[8];
      const float alpha = softmax_head(sacc, pk0_next, ek_c, eb_c);
      ek_c = ek_n;
      eb_c = eb_n;
      interleave<kDTiles * 4, 4, 4, kCopies>();
      rescale(alpha);
#pragma unroll
      for (int i = 0; i < 8; ++i) pk0[i] = pk0_next[i];
      wait_older();  // K_{kb+1}
      barrier();
    };
    // Every pass ends with a buffer-0 step, so no path reaches the loop head
    // with a copy into buffer 1 in flight (the compiler would otherwise wait
    // for every copy before the first buffer-1 read); an odd last block runs
    // after the loop.
    int kb = 1;
    for (; kb + 1 < nkb; kb += 2) {
      step(Buf<1>{}, kb);
      step(Buf<0>{}, kb + 1);
    }
    if (kb < nkb) step(Buf<1>{}, kb);
    wait_all();  // V_last (and the last, unread K copy)
    barrier();
    // P of the last block, keys 32..63; V_last arrived in buffer last % 2
    // (the prologue's V_0 when nkb == 1).
    softmax_tail();
    if (last & 1) pv(Buf<1>{}, pk0, pk1); else pv(Buf<0>{}, pk0, pk1);

    // ---- epilogue: full row sums, normalise, store ---------------------------
    l_run = halves_sum(l_run);
    if (wave_active && my_q < S) {
      const float inv = l_run > 0.f ? __builtin_ldexpf(1.f / l_run, e_run) : 0.f;
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
    __syncthreads();  // the next pass recopies all four buffers
  }
}

hipError_t launch_prefill(const PrefillParams& p, int head_dim, hipStream_t stream) {
  const int G = p.group;
  const int GW = G < kWaves ? G : kWaves;
  const int pos_per_wg = kQB * (kWaves / GW);
  const int nqb = (p.seqlen + pos_per_wg - 1) / pos_per_wg;
  const dim3 grid(nqb, p.kv_heads);
  const hipError_t vt_rc = launch_prefill_vts(p, head_dim, kVtOrder32, stream);
  if (vt_rc != hipSuccess) return vt_rc;
  switch (head_dim) {
    case 128:
      hipLaunchKernelGGL(gqa_prefill_kernel<128>, grid, dim3(kWaves * 64), 0, stream, p);
      break;
    case 256:
      hipLaunchKernelGGL(gqa_prefill_kernel<256>, grid, dim3(kWaves * 64), 0, stream, p);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace bt
