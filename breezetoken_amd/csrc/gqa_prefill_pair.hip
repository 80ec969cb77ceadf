// Causal GQA prefill for long prompts on CDNA4 MFMA: two query blocks per
// work-group, 32 query columns per wave.
//
// Same contract as gqa_prefill8.hip (the causal SDPA of prefill.py:56-68 and
// the banded chunked prefill of qwen36_moe.py:394-428: query row i at absolute
// position q_offset + i attends keys 0 .. q_offset + i).  The work
// decomposition is built for the long-prompt regime, where the kernel is
// bound by LDS operand traffic per MFMA and by the causal triangle's uneven
// work:
//  * a wave holds 32 query columns (two 16-column q-tiles, Q^T in registers),
//    so every K or V^T fragment it reads from LDS feeds two MFMAs -- half the
//    LDS bytes per FLOP of one q-tile per wave.  O^T (D x 32 f32) is 128
//    registers, Q^T 64; two waves still fit each SIMD;
//  * 4 waves form a group that shares one K tile and one V^T tile of 32 keys
//    per step (all heads of a GQA group read the same K/V);
//  * a work-group holds two groups, A and B, and the query blocks j and
//    N-1-j of one kv head: together they need N+1 steps whatever j is, so
//    every work-group does the same work.  A runs block j, then the last
//    keys of block N-1-j; B runs the other keys of block N-1-j; both take
//    ceil((N+1)/2) steps in lockstep (two barrier phases per step: one group
//    runs Q.K^T + softmax while the other runs P.V), and the two halves of
//    block N-1-j are merged through LDS at the end.  While A runs block j the
//    two groups read the same key units, and A reads B's tiles;
//  * Q.K^T runs on fp16 MFMAs: q (f32, as the reference keeps it through
//    prefill.py:49-68, or bf16) is rounded to fp16 after scaling each query
//    row by a power of two, and K comes from the pre-pass's fp16 image, scaled
//    per 64-key block (gqa_prefill_vt.hip); both factors return exactly in the
//    exp2 argument.  fp16's 11 bits keep q's rounding error 8x below bf16's;
//  * P and V^T enter the P.V product as fp16 (P <= 2^8 from the lazily
//    rescaled softmax); each 64-key block of V is stored scaled by its own
//    power of two, which the softmax folds into P, so V of any bf16
//    magnitude keeps fp16's 11 bits.
#include "bt_common.h"
#include "bt_kernels.h"

namespace bt {

namespace {

typedef _Float16 halfx8_p __attribute__((ext_vector_type(8)));
typedef _Float16 half2_p __attribute__((ext_vector_type(2)));
typedef float float2_p __attribute__((ext_vector_type(2)));

constexpr int kUnit = 32;        // keys per step (one K tile and one V^T tile)
// LDS fragment reads in flight ahead of their MFMAs: K two d-steps ahead in
// S = K.Q^T, V^T four d-tiles ahead in O^T += V^T.P^T.  C4 at S = 8192, bf16
// q, same run: lead 1/2 -> 325 us, 2/2 -> 314-320, 1/4 -> 312-314, 2/4 ->
// 300-317, 3/4 and 2/8 -> 332-340 (the bf16 kernel then spills in the loop).
constexpr int kKLead = 2;
constexpr int kVLead = 4;
constexpr int kGWaves = 4;       // waves per group
constexpr float kLazyP = 8.0f;   // log2-domain slack before the reference max moves

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_p(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
// HBM -> LDS copy of 16 bytes per lane (lane l's bytes land at lds + 16 * l);
// offsets past the descriptor's range read as zero.
__device__ __forceinline__ void dma16_p(__amdgpu_buffer_rsrc_t r, unsigned char* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (BT_LDS void*)lds, 16, (int)voff, (int)soff, 0, 0);
}
__device__ __forceinline__ floatx4 mfma_f16(const u32x4& a, const u32x4& b, const floatx4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(halfx8_p, a), __builtin_bit_cast(halfx8_p, b), c,
                                                0, 0, 0);
}
// Round to nearest even through a builtin (not asm), so the compiler sees the
// VALU write and inserts the wait states an in-flight MFMA operand needs.
__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((float2_p){a, b}, half2_p));
}

// Shapes of the pair kernel's query blocks: a group covers 4 * NQT q-tiles of
// 16 query positions each, for HG = min(G, 4 * NQT) heads of the kv group and
// P = 16 * 4 * NQT / HG consecutive positions; G / HG head subgroups share a
// kv head.
struct PairShape {
  int nqt, hg, pos, nsub;
};
__host__ __device__ inline PairShape pair_shape(int group, int nqt) {
  PairShape s;
  s.nqt = nqt;
  s.hg = group < 4 * s.nqt ? group : 4 * s.nqt;
  s.pos = 16 * 4 * s.nqt / s.hg;
  s.nsub = group / s.hg;
  return s;
}

// One group's share of a pair work-group.  GRP 0 (A) runs query block qa's
// keys, then the last keys of qb; GRP 1 (B) the rest of qb.  K0/K1/V0/V1 are
// this group's double-buffered tiles (distinct LDS objects, so the compiler
// can tell a copy into one buffer from a read of another); xbuf(i) is tile
// buffer i of the eight, reused for the final merge.
template <bool B>
struct Sel {
  static constexpr bool value = B;
};

// NQT q-tiles per wave; LO: f32 q as two fp16 terms (hi + lo, see
// split_f16x2), each K fragment feeding one MFMA per term.
template <int D, int NQT, bool LO, int GRP, typename XB>
__device__ __forceinline__ void pair_group(const PrefillParams& p, unsigned char* K0, unsigned char* K1,
                                           unsigned char* V0, unsigned char* V1, XB xbuf, float* xs) {
  auto xbuf_c = [&](int i) { return reinterpret_cast<unsigned char*>(xbuf(i)); };
  constexpr int kDSteps = D / 32;
  constexpr int kDTiles = D / 16;
  constexpr int kRowBytes = D * 2;
  constexpr int kTile = kUnit * kRowBytes;           // 16 KiB at D = 256
  constexpr int kCopies = kTile / 1024 / kGWaves;    // 1 KiB copies per wave per tile
  static_assert(kCopies >= 1, "head_dim 128 or 256");

  const int lane = threadIdx.x & 63;
  const int gw = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6) & 3);
  const int i16 = lane & 15;
  const int g4 = lane >> 4;
  const PairShape sh = pair_shape(p.group, NQT);
  const int kvh = (int)blockIdx.y / sh.nsub;
  const int sub = (int)blockIdx.y % sh.nsub;
  const int S = p.seqlen;
  const int P0 = p.q_offset;
  const int nkeys = P0 + S;
  const int nqb = (S + sh.pos - 1) / sh.pos;
  const int qa = (int)blockIdx.x, qb = nqb - 1 - (int)blockIdx.x;
  auto n_units = [&](int blk) { return (P0 + min(S, (blk + 1) * sh.pos) + kUnit - 1) / kUnit; };
  const int na = qa != qb ? n_units(qa) : 0;
  const int nb = n_units(qb);
  // A runs block qa's na units, then the last xa units of block qb; B runs
  // qb's first nb - xa units.  Both groups read key unit s - lead at step s
  // until A's switch to block qb (the units block qa needs are the first
  // units of block qb too): there A reads B's K and V^T tiles and copies none
  // of its own, and the work-groups on an XCD share each tile through L2.
  // When na is odd both groups start one step late, so A's switch falls on an
  // even step; the step count is even too.  Then the key loop is unrolled by
  // two with a constant buffer per step and no branch between its copies.
  // C4 S = 8192 / 12000 in one process, against A copying every tile: 264.1
  // -> 260.9 / 669.9 -> 645.2 us (bf16 q), 398.0 -> 387.3 us (f32 q).  A
  // work-group whose qa is small shares few steps and gains little, so the
  // gain shows where work-groups outnumber the CUs and others take their
  // place.
  const int lead = na & 1;
  const int sw = lead + na;                        // A's first step on block qb (even)
  const int xa = max(0, (nb - na) / 2);
  const int steps_a = sw + xa;
  const int steps_b = lead + nb - xa;
  const int n_steps = (max(steps_a, steps_b) + 1) & ~1;
  const int my_steps = GRP == 0 ? steps_a : steps_b;
  const int first = lead;                          // both groups' first working step
  // Unit of step s: (query block, key unit); shared(s): A reads B's tiles.
  auto unit_blk = [&](int st) { return (GRP == 0 && st < sw) ? qa : qb; };
  auto unit_key = [&](int st) { return GRP == 0 ? (st < sw ? st - lead : nb - xa + st - sw) : st - lead; };
  auto shared = [&](int st) { return st >= lead && st < sw; };

  const int nblk64 = (nkeys + kPrefillKeyBlock - 1) / kPrefillKeyBlock;
  const uint32_t img_bytes = (uint32_t)nblk64 * kPrefillKeyBlock * kRowBytes;
  const size_t head_img = (size_t)kvh * p.img_blocks * kPrefillKeyBlock * D;  // this kv head's images
  const __amdgpu_buffer_rsrc_t krs = rsrc_p(p.kimg + head_img, img_bytes);
  const __amdgpu_buffer_rsrc_t vrs = rsrc_p(p.vt + head_img, img_bytes);
  const int* vexp = p.vexp + kvh * p.img_blocks;
  const int* kexp = p.kexp + kvh * p.img_blocks;

  // Tile copies: the unit's 32 rows of K (row-major, slots XOR-swizzled by
  // the pre-pass, so the operand reads of 16 consecutive rows hit 16 bank
  // groups) and its V^T half-block are each 16 KiB contiguous in the images.
  auto copy_k = [&](unsigned char* kbuf, int u) {
    const int key0 = unit_key(u) * kUnit;
    const uint32_t ksrc = (uint32_t)key0 * kRowBytes;
#pragma unroll
    for (int j = 0; j < kCopies; ++j) {
      const int i = gw * kCopies + j;
      dma16_p(krs, kbuf + i * 1024, (uint32_t)lane * 16, ksrc + (uint32_t)i * 1024);
    }
  };
  auto copy_v = [&](unsigned char* vbuf, int u) {
    const int key0 = unit_key(u) * kUnit;
    // V^T: the 32-key half (key0 / 32) & 1 of 64-key block key0 / 64 is 16 KiB
    // contiguous in the image.
    const uint32_t vsrc = (uint32_t)(key0 / kPrefillKeyBlock) * (kPrefillKeyBlock * kRowBytes) +
                          (uint32_t)((key0 / kUnit) & 1) * kTile;
#pragma unroll
    for (int j = 0; j < kCopies; ++j) {
      const int i = gw * kCopies + j;
      dma16_p(vrs, vbuf + i * 1024, (uint32_t)lane * 16, vsrc + (uint32_t)i * 1024);
    }
  };

  // ---- q-tiles of this wave -------------------------------------------------
  // q-tile t of wave gw is group tile qt = gw * NQT + t: head (qt % HG) of the
  // subgroup, positions [16 * (qt / HG), +16) of the query block.
  int head[NQT], poff[NQT];
#pragma unroll
  for (int t = 0; t < NQT; ++t) {
    const int qt = gw * NQT + t;
    head[t] = kvh * p.group + sub * sh.hg + qt % sh.hg;
    poff[t] = 16 * (qt / sh.hg);
  }
  // Q^T operand: lane (i16, g4) holds q[row][st*32 + g4*8 .. +8] of column i16
  // as fp16, scaled by 2^-eq so the row's largest |q| lies in [2^14, 2^15);
  // c_col = scale * log2(e) * 2^eq restores it in the exp2 argument.  Rows
  // past the prompt read the last row (their output is not stored).
  u32x4 qop[NQT][kDSteps];
  u32x4 qlo[LO ? NQT : 1][kDSteps];
  float c_col[NQT];
  // One pass over q: every load of the block is issued before any is used (the
  // raw values take the registers O frees between blocks), then each row's
  // largest |q| is reduced over its four lane groups and the values converted.
  auto row_scale = [&](int t, uint32_t mx) {
    mx = xor_umax<32>(xor_umax<16>(mx));  // the row's four lane groups
    const int eq = absmax_exp(mx);
    c_col[t] = __builtin_ldexpf(p.scale_log2, eq);
    return eq;
  };
  auto load_q = [&](int blk) {
    int64_t off[NQT];
#pragma unroll
    for (int t = 0; t < NQT; ++t) {
      const int row = min(blk * sh.pos + poff[t] + i16, S - 1);
      off[t] = (int64_t)row * p.q_stride_tok + (int64_t)head[t] * p.q_stride_head + g4 * 8;
    }
    if constexpr (LO) {
      const float* qf = reinterpret_cast<const float*>(p.q);
      float4 raw[NQT][kDSteps][2];
#pragma unroll
      for (int t = 0; t < NQT; ++t)
#pragma unroll
        for (int st = 0; st < kDSteps; ++st) {
          raw[t][st][0] = *reinterpret_cast<const float4*>(qf + off[t] + st * 32);
          raw[t][st][1] = *reinterpret_cast<const float4*>(qf + off[t] + st * 32 + 4);
        }
#pragma unroll
      for (int t = 0; t < NQT; ++t) {
        const int eq = row_scale(t, absmax_bits(raw[t]));
#pragma unroll
        for (int st = 0; st < kDSteps; ++st) {
          const float4 a = raw[t][st][0], b = raw[t][st][1];
          uint32_t h[4], l[4];
          split_f16x2(a.x, a.y, eq, h[0], l[0]);
          split_f16x2(a.z, a.w, eq, h[1], l[1]);
          split_f16x2(b.x, b.y, eq, h[2], l[2]);
          split_f16x2(b.z, b.w, eq, h[3], l[3]);
          qop[t][st] = u32x4{h[0], h[1], h[2], h[3]};
          qlo[t][st] = u32x4{l[0], l[1], l[2], l[3]};
        }
      }
    } else {  // bf16 q (the launcher sends f32 q to the LO instantiation)
#pragma unroll
      for (int t = 0; t < NQT; ++t)
#pragma unroll
        for (int st = 0; st < kDSteps; ++st) qop[t][st] = *reinterpret_cast<const u32x4*>(p.q + off[t] + st * 32);
#pragma unroll
      for (int t = 0; t < NQT; ++t) {
        uint32_t mx = 0;
#pragma unroll
        for (int st = 0; st < kDSteps; ++st)
#pragma unroll
          for (int i = 0; i < 4; ++i) mx = max(mx, max((qop[t][st][i] << 16) & 0x7fffffffu, qop[t][st][i] & 0x7fff0000u));
        const int eq = row_scale(t, mx);
#pragma unroll
        for (int st = 0; st < kDSteps; ++st) {
          const u32x4 w = qop[t][st];
          qop[t][st] = u32x4{pack_f16x2_scaled(__uint_as_float(w[0] << 16), __uint_as_float(w[0] & 0xffff0000u), eq),
                             pack_f16x2_scaled(__uint_as_float(w[1] << 16), __uint_as_float(w[1] & 0xffff0000u), eq),
                             pack_f16x2_scaled(__uint_as_float(w[2] << 16), __uint_as_float(w[2] & 0xffff0000u), eq),
                             pack_f16x2_scaled(__uint_as_float(w[3] << 16), __uint_as_float(w[3] & 0xffff0000u), eq)};
        }
      }
    }
  };
  // ---- running state: per q-tile column (this lane's i16) -------------------
  floatx4 oacc[NQT][kDTiles];
  float m_ref[NQT], l_run[NQT];
  int e_run = kVExpZero;  // scale exponent O is kept in: O_true = O * 2^e_run
  auto reset = [&]() {
#pragma unroll
    for (int t = 0; t < NQT; ++t) {
#pragma unroll
      for (int i = 0; i < kDTiles; ++i) oacc[t][i] = floatx4{0.f, 0.f, 0.f, 0.f};
      m_ref[t] = -INFINITY;
      l_run[t] = 0.f;
    }
    e_run = kVExpZero;
  };

  // Normalise and store a finished block (rows past the prompt are skipped).
  auto store = [&](int blk, const float (&lsum)[NQT]) {
#pragma unroll
    for (int t = 0; t < NQT; ++t) {
      const int row = blk * sh.pos + poff[t] + i16;
      if (row >= S) continue;
      const float inv = lsum[t] > 0.f ? __builtin_ldexpf(1.f / lsum[t], e_run) : 0.f;
      const int64_t orow = (int64_t)row * p.out_stride_tok + (int64_t)head[t] * p.out_stride_head;
#pragma unroll
      for (int dt = 0; dt < kDTiles; ++dt) {
        const int d = dt * 16 + g4 * 4;
        const float o0 = oacc[t][dt][0] * inv, o1 = oacc[t][dt][1] * inv, o2 = oacc[t][dt][2] * inv,
                    o3 = oacc[t][dt][3] * inv;
        if (p.out_bf16) {
          const u32x2 pk2 = {f32x2_to_bf16x2_bits(o0, o1), f32x2_to_bf16x2_bits(o2, o3)};
          *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(p.out) + orow + d) = pk2;
        } else {
          *reinterpret_cast<float4*>(reinterpret_cast<float*>(p.out) + orow + d) = float4{o0, o1, o2, o3};
        }
      }
    }
  };
  // The same through LDS, so that every store writes whole 16-byte slices of
  // rows instead of 8- or 16-byte pieces of 16 rows: q-tile t's 16 rows (2D
  // bytes each: bf16 rows, or f32 rows in two column halves) go to stage(t),
  // this wave's own 16 x 2D bytes, with 16-byte chunk c of row r in slot
  // c ^ r, and are read back a row slice per lane.
  auto store_staged = [&](int blk, const float (&lsum)[NQT], auto&& stage) {
    constexpr int kChunks = D / 8;          // 16-byte chunks of a staged row
    constexpr int kRowsPer = 64 / kChunks;  // staged rows per store
#pragma unroll
    for (int t = 0; t < NQT; ++t) {
      unsigned char* st_ = stage(t);
      const int row0 = blk * sh.pos + poff[t];
      const float inv = lsum[t] > 0.f ? __builtin_ldexpf(1.f / lsum[t], e_run) : 0.f;
      unsigned char* obase = reinterpret_cast<unsigned char*>(p.out) +
                             (int64_t)head[t] * p.out_stride_head * (p.out_bf16 ? 2 : 4);
      const int64_t row_bytes = p.out_stride_tok * (p.out_bf16 ? 2 : 4);
      auto drain = [&](int col_bytes) {
#pragma unroll
        for (int j = 0; j < 16 / kRowsPer; ++j) {
          const int r = j * kRowsPer + lane / kChunks, c = lane % kChunks;
          const u32x4 x = *reinterpret_cast<const u32x4*>(st_ + r * (D * 2) + (c ^ r) * 16);
          if (row0 + r < S) *reinterpret_cast<u32x4*>(obase + (row0 + r) * row_bytes + col_bytes + c * 16) = x;
        }
      };
      if (p.out_bf16) {
#pragma unroll
        for (int dt = 0; dt < kDTiles; ++dt) {
          const u32x2 pk2 = {f32x2_to_bf16x2_bits(oacc[t][dt][0] * inv, oacc[t][dt][1] * inv),
                             f32x2_to_bf16x2_bits(oacc[t][dt][2] * inv, oacc[t][dt][3] * inv)};
          const int c = dt * 2 + (g4 >> 1);  // chunk of columns dt*16 + g4*4 ..
          *reinterpret_cast<u32x2*>(st_ + i16 * (D * 2) + (c ^ i16) * 16 + (g4 & 1) * 8) = pk2;
        }
        drain(0);
      } else {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
          for (int dt = h * kDTiles / 2; dt < (h + 1) * kDTiles / 2; ++dt) {
            const int c = (dt - h * kDTiles / 2) * 4 + g4;
            *reinterpret_cast<float4*>(st_ + i16 * (D * 2) + (c ^ i16) * 16) =
                float4{oacc[t][dt][0] * inv, oacc[t][dt][1] * inv, oacc[t][dt][2] * inv, oacc[t][dt][3] * inv};
          }
          drain(h * (D * 2));
        }
      }
    }
  };
  auto row_sums = [&](float (&lsum)[NQT]) {
#pragma unroll
    for (int t = 0; t < NQT; ++t) {
      float l = xor_sum<16>(l_run[t]);
      lsum[t] = halves_sum(l);
    }
  };

  // K operand of key tile kt, d-step st: chunk st*4 + g4 of row kt*16 + i16,
  // in slot (st*4 + g4) ^ i16 = ((st ^ (i16 >> 2)) * 4) + ((g4 ^ i16) & 3).
  uint32_t kaddr[4];
#pragma unroll
  for (int s4 = 0; s4 < 4; ++s4)
    kaddr[s4] = (uint32_t)i16 * kRowBytes + (uint32_t)(((s4 ^ (i16 >> 2)) * 4 + ((g4 ^ i16) & 3)) * 16);
  const uint32_t vaddr = (uint32_t)g4 * (D * 16) + (uint32_t)i16 * 16;  // V^T: chunk g4, row dt*16 + i16

  // S^T = K.Q^T on the K tile kb, mask, online softmax: P^T of the step in pk.
  // The softmax of q-tiles kNow.. is deferred to sm_tail, which runs in the
  // P.V phase: that phase (MFMAs and V^T reads) has slack, while Q.K^T +
  // softmax is each step's critical path.  Their masked scores wait in xd and
  // the step's scale exponents in the *_d scalars.  Two q-tiles: the second
  // is deferred (deferring both: C4 S = 8192 275.5 -> 281 us).  One q-tile
  // (f32 q, whose Q.K^T issues two MFMAs per K fragment): it is deferred
  // (426 -> 403 us, same results).
  constexpr int kNow = NQT == 1 ? 0 : 1;
  u32x4 pk[NQT];
  float xd[NQT > kNow ? NQT - kNow : 1][8];
  int shift_d = 0, ek_d = 0, eold_d = 0, enew_d = 0;
  // Block scales (V^T and K exponents) of a step's unit, read one step ahead
  // into scalar registers so the softmax never waits for them.  Steps past this
  // group's range read the last block's (their values are unused).
  auto unit_scales = [&](int u, int& eb, int& ek) {
    int b64 = unit_key(u) * kUnit / kPrefillKeyBlock;
    b64 = b64 < 0 ? 0 : (b64 < nblk64 ? b64 : nblk64 - 1);
    eb = sload(vexp, b64);
    ek = sload(kexp, b64);
  };
  // Online softmax of q-tile t's 32 masked scores s (keys kt*16 + g4*4 + r at
  // s[kt*4 + r]): lazy reference max, O and l rescaled when it moves or the V
  // scale exponent changes from e_old to e_new, P^T into pk[t].
  auto softmax_tile = [&](int t, const float (&s)[8], int ek, int shift, int e_old, int e_new) {
    const float c_log2 = __builtin_ldexpf(c_col[t], ek);  // log2-domain factor of the scaled scores
    const float lmax = fmax_nc(fmax_nc(fmax_nc(s[0], s[1]), fmax_nc(s[2], s[3])),
                               fmax_nc(fmax_nc(s[4], s[5]), fmax_nc(s[6], s[7])));
    // The column's max over its four lane groups passes the lazy bound exactly
    // when one group's own max does (scaling by c_log2 > 0 keeps the order),
    // so the cross-lane reduction runs only when some column's reference max
    // may move: rare after a row's first keys.
    float alpha = 1.f;
    if (__builtin_amdgcn_ballot_w64(lmax * c_log2 > m_ref[t] + kLazyP)) {
      float tmax = rows16_max(lmax);
      tmax = halves_max(tmax) * c_log2;
      const bool move = tmax > m_ref[t] + kLazyP;
      const float m_new = move ? tmax : m_ref[t];
      alpha = move ? fast_exp2(m_ref[t] - m_new) : 1.f;  // 0 when m_ref is -inf
      m_ref[t] = m_new;
    }
    const float bias = (m_ref[t] == -INFINITY ? 0.f : -m_ref[t]) + (float)shift;
    float e[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) e[r] = fast_exp2(fmaf(s[r], c_log2, bias));
    float psum = ((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7]));
    if (shift != 0) psum = __builtin_ldexpf(psum, -shift);  // wave-uniform, rare
    l_run[t] = l_run[t] * alpha + psum;
    // Key order of the V^T chunk g4: keys g4*4 + {0..3}, 16 + g4*4 + {0..3}.
    pk[t] = u32x4{pack_h2(e[0], e[1]), pack_h2(e[2], e[3]), pack_h2(e[4], e[5]), pack_h2(e[6], e[7])};
    if (e_new != e_old) alpha = __builtin_ldexpf(alpha, e_old - e_new);
    if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {  // rare: the max or the V scale moved
#pragma unroll
      for (int i = 0; i < kDTiles; ++i) oacc[t][i] *= alpha;
    }
  };
  // K fragment (d-step st, key tile kt) of the K tile kb.
  auto kread_at = [&](const unsigned char* kb, int st, int kt) -> u32x4 {
    return *reinterpret_cast<const u32x4*>(kb + kaddr[st & 3] + (st & 4) * 64 + kt * 16 * kRowBytes);
  };
  // The first kKLead d-steps' K fragments, read right after the barrier that
  // publishes the tile (before the step's tile copies are issued), so their
  // LDS latency overlaps the copies' issue.
  auto k_first = [&](const unsigned char* kb, u32x4 (&kf)[kKLead + 1][2]) {
#pragma unroll
    for (int i = 0; i < kKLead; ++i) {
      kf[i][0] = kread_at(kb, i, 0);
      kf[i][1] = kread_at(kb, i, 1);
    }
  };
  auto qk_sm = [&](const unsigned char* kb, int u, int eb, int ek, u32x4 (&kf)[kKLead + 1][2], auto&& after_mfma) {
    const int blk = unit_blk(u);
    const int key0 = unit_key(u) * kUnit;
    floatx4 sacc[2][NQT];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int t = 0; t < NQT; ++t) sacc[kt][t] = floatx4{0.f, 0.f, 0.f, 0.f};
    // K fragments are read kKLead d-steps ahead of their MFMAs (scheduling
    // barriers keep the compiler from hoisting all of them: the registers are
    // spoken for by O and Q).
    auto kread = [&](int st, int kt) -> u32x4 { return kread_at(kb, st, kt); };
    constexpr int KLA = kKLead;
#pragma unroll
    for (int st = 0; st < kDSteps; ++st) {
      if (st + KLA < kDSteps) {
        kf[(st + KLA) % (KLA + 1)][0] = kread(st + KLA, 0);
        kf[(st + KLA) % (KLA + 1)][1] = kread(st + KLA, 1);
      }
      const u32x4 a0 = kf[st % (KLA + 1)][0], a1 = kf[st % (KLA + 1)][1];
#pragma unroll
      for (int t = 0; t < NQT; ++t) {
        sacc[0][t] = mfma_f16(a0, qop[t][st], sacc[0][t]);
        sacc[1][t] = mfma_f16(a1, qop[t][st], sacc[1][t]);
      }
      if constexpr (LO) {
#pragma unroll
        for (int t = 0; t < NQT; ++t) {
          sacc[0][t] = mfma_f16(a0, qlo[t][st], sacc[0][t]);
          sacc[1][t] = mfma_f16(a1, qlo[t][st], sacc[1][t]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    after_mfma();
    // Causal mask: key key0 + kt*16 + g4*4 + r against this column's position.
    // The lane's column and lane group are re-derived here from the V^T
    // operand address (g4 * D * 16 + i16 * 16), which the loop keeps anyway,
    // through an opaque copy: kept live across the key loop instead, the
    // column index was spilled, and its reload each step -- a scratch load,
    // counted with the tile copies -- made the softmax wait for every copy in
    // flight before reusing the register.
    uint32_t va = vaddr;
    asm volatile("" : "+v"(va));
    const int col = (int)((va >> 4) & 15u);
    const int grp = (int)(va / (uint32_t)(D * 16));
#pragma unroll
    for (int t = 0; t < NQT; ++t) {
      const int qpos = P0 + blk * sh.pos + poff[t];  // first position of the q-tile
      if (key0 + kUnit - 1 > qpos) {
        const int mypos = qpos + col;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (key0 + kt * 16 + grp * 4 + r > mypos) sacc[kt][t][r] = -INFINITY;
      }
    }
    // The V^T tile's scale: e of its 64-key block (wave-uniform).  P enters
    // P.V as P' = P * 2^shift (the shift rides in the exp2 bias); the row sum
    // takes P, i.e. the sum of P' times 2^-shift.
    const int e_new = vexp_next(e_run, eb);
    const int shift = vexp_shift(e_new, eb);
#pragma unroll
    for (int t = kNow; t < NQT; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        xd[t - kNow][r] = sacc[0][t][r];
        xd[t - kNow][4 + r] = sacc[1][t][r];
      }
#pragma unroll
    for (int t = 0; t < kNow; ++t) {
      float s[8];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        s[r] = sacc[0][t][r];
        s[4 + r] = sacc[1][t][r];
      }
      softmax_tile(t, s, ek, shift, e_run, e_new);
    }
    shift_d = shift;
    ek_d = ek;
    eold_d = e_run;
    enew_d = e_new;
    e_run = e_new;
  };
  // The deferred q-tiles' softmax, row sums and P^T.
  auto sm_tail = [&]() {
#pragma unroll
    for (int t = kNow; t < NQT; ++t) softmax_tile(t, xd[t - kNow], ek_d, shift_d, eold_d, enew_d);
  };
  // O^T += V^T.P^T on the V^T tile vb (after the step's deferred softmax).
  auto pv = [&](const unsigned char* vb) {
    auto vread = [&](int dt) -> u32x4 { return *reinterpret_cast<const u32x4*>(vb + vaddr + dt * 256); };
    constexpr int VLA = kVLead;
    u32x4 vf[VLA];
#pragma unroll
    for (int i = 0; i < VLA; ++i) vf[i] = vread(i);
    sm_tail();  // the first V^T reads are in flight meanwhile
#pragma unroll
    for (int dt = 0; dt < kDTiles; ++dt) {
      const u32x4 a = vf[dt % VLA];
      if (dt + VLA < kDTiles) vf[dt % VLA] = vread(dt + VLA);
#pragma unroll
      for (int t = 0; t < NQT; ++t) oacc[t][dt] = mfma_f16(a, pk[t], oacc[t][dt]);
      if (dt % 2 == 1) __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Each wave waits for its own copies; a barrier publishes them (no
  // __syncthreads: its fence would wait for every copy in flight).  vmcnt
  // counts a wave's loads in issue order, so naming how many of the youngest
  // may still be in flight waits for exactly the older ones.
  auto barrier = [] { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };
  constexpr int kWait1 = 0x0f70 | (kCopies & 0xf) | ((kCopies >> 4) << 14);            // vmcnt(kCopies)
  constexpr int kWait2 = 0x0f70 | ((2 * kCopies) & 0xf) | (((2 * kCopies) >> 4) << 14);  // vmcnt(2 kCopies)
  static_assert(2 * kCopies < 64, "vmcnt holds 6 bits");
  // Wait until at most `younger` tiles' copies (kCopies each) are in flight:
  // exactly the copies issued after the awaited tile, so none is under-waited.
  auto wait_tiles = [&](int younger) {
    if (younger >= 2) __builtin_amdgcn_s_waitcnt(kWait2);
    else if (younger == 1) __builtin_amdgcn_s_waitcnt(kWait1);
    else __builtin_amdgcn_s_waitcnt(0x0f70);
  };

  // The first tiles go out before the q loads, so the two latencies overlap.
  if (first < my_steps && !(GRP == 0 && shared(first))) {
    if (first & 1) { copy_k(K1, first); copy_v(V1, first); } else { copy_k(K0, first); copy_v(V0, first); }
  }
  int cur_blk = unit_blk(first);
  load_q(cur_blk);
  reset();
  auto working = [&](int st) { return st >= first && st < my_steps; };
  // Each step has two barrier phases.  The two groups put their MFMA-heavy
  // and VALU-heavy work in opposite phases, so the two waves that share a
  // SIMD (one of each group) overlap one's softmax with the other's MFMAs:
  //   A: | K_st ready  S = Q.K^T, softmax      | V_st ready  O += P.V       |
  //   B: | V_st-1 ready  O += P_{st-1}.V_{st-1} | K_st ready  S = Q.K^T, softmax |
  // Copies go out as soon as their buffer is free: A requests K and V^T of
  // step st + 1 at the first barrier of st (after its switch: before it, it
  // reads B's); B requests K of st + 1 at the first barrier and V^T of st + 1
  // at the second (after its P.V of st - 1), and reads its first K fragments
  // of st before the second.
  auto step = [&](auto bufsel, auto shtag, int st, int& eb, int& ek) {
    constexpr bool kOdd = decltype(bufsel)::value;
    constexpr bool kShared = decltype(shtag)::value;  // A's steps before its switch
    unsigned char* Kc = kOdd ? K1 : K0;   // this step's buffers
    unsigned char* Vc = kOdd ? V1 : V0;
    unsigned char* Kn = kOdd ? K0 : K1;   // the next step's (and the previous step's)
    unsigned char* Vn = kOdd ? V0 : V1;
    const bool w0 = working(st), w1 = working(st + 1);
    // The wave running Q.K^T + softmax gets issue priority, so its MFMAs go
    // first and its softmax overlaps the other wave's P.V.
    u32x4 kf[kKLead + 1][2];
    if constexpr (GRP == 0 && kShared) {
      // B's tiles of this step: B waits for their copies before the
      // barriers that start A's two phases.
      unsigned char* Kb = kOdd ? xbuf_c(5) : xbuf_c(4);
      unsigned char* Vb = kOdd ? xbuf_c(7) : xbuf_c(6);
      barrier();
      if (w0) k_first(Kb, kf);
      int eb_n, ek_n;
      if (w1 && !shared(st + 1)) { copy_k(Kn, st + 1); copy_v(Vn, st + 1); }  // A's first own tiles
      __builtin_amdgcn_s_setprio(1);
      if (w0) qk_sm(Kb, st, eb, ek, kf, [&] { unit_scales(st + 1, eb_n, ek_n); });
      else unit_scales(st + 1, eb_n, ek_n);
      __builtin_amdgcn_s_setprio(0);
      eb = eb_n;
      ek = ek_n;
      barrier();
      if (w0) pv(Vb);
    } else if constexpr (GRP == 0) {
      wait_tiles(1);  // K of st (its V^T was issued after it)
      barrier();
      if (w0) k_first(Kc, kf);
      int eb_n, ek_n;
      if (w1) { copy_k(Kn, st + 1); copy_v(Vn, st + 1); }
      __builtin_amdgcn_s_setprio(1);
      // The next step's block scales are requested after the MFMAs: scalar
      // loads share the LDS reads' counter and return out of order, so issued
      // earlier they would hold the first MFMA until they arrive.
      if (w0) qk_sm(Kc, st, eb, ek, kf, [&] { unit_scales(st + 1, eb_n, ek_n); });
      else unit_scales(st + 1, eb_n, ek_n);
      __builtin_amdgcn_s_setprio(0);
      eb = eb_n;
      ek = ek_n;
      wait_tiles(w1 ? 2 : 0);  // V^T of st (behind it: K and V^T of st + 1)
      barrier();
      if (w0) pv(Vc);
    } else {
      wait_tiles(w0 ? 1 : 0);  // V^T of st - 1 and K of st (behind them: V^T of st)
      barrier();
      int eb_n, ek_n;
      if (w1) copy_k(Kn, st + 1);
      if (working(st - 1)) pv(Vn);
      // K of st is published by the barrier above (its copies were issued a
      // step ago), so the first fragments are read now and arrive while the
      // wave waits at the next barrier, which leaves them in flight: the P.V
      // reads before them are consumed by its MFMAs, and K of st is
      // overwritten only after this step's Q.K^T.  C4 S = 8192 in one process:
      // 267.1 -> 263.5 us (bf16 q), 393.9 -> 387.8 us (f32 q), bit-identical.
      // The same for A gained nothing more, with its K waited for one phase
      // after its copy is issued or with its K copies moved a phase earlier
      // (A's tile-copy issue after its barrier already covers the first
      // reads); B's first V^T fragments read the same way at the end of its
      // Q.K^T phase cost 1.4% with f32 q.
      if (w0) k_first(Kc, kf);
      // In a shared step A reads V^T of st in the phase that starts here (one
      // phase before B does).
      if (shared(st) && w0) wait_tiles(w1 ? 1 : 0);  // V^T of st (behind it: K of st + 1)
      asm volatile("s_barrier" ::: "memory");
      if (w1) copy_v(Vn, st + 1);
      __builtin_amdgcn_s_setprio(1);
      if (w0) qk_sm(Kc, st, eb, ek, kf, [&] { unit_scales(st + 1, eb_n, ek_n); });
      else unit_scales(st + 1, eb_n, ek_n);
      __builtin_amdgcn_s_setprio(0);
      eb = eb_n;
      ek = ek_n;
    }
  };
  auto run = [&](auto shtag, int s0, int s1) {  // s0 and s1 even
    int eb, ek;
    unit_scales(s0, eb, ek);
    for (int st = s0; st < s1; st += 2) {
      step(Sel<false>{}, shtag, st, eb, ek);
      step(Sel<true>{}, shtag, st + 1, eb, ek);
    }
  };
  if constexpr (GRP == 0) {
    // Block qa (on B's tiles), then (after storing it) the last keys of block qb.
    const int s_switch = min(sw, n_steps);
    run(Sel<true>{}, 0, s_switch);
    if (na > 0 && s_switch < my_steps) {
      float lsum[NQT];
      row_sums(lsum);
      // A's K and V buffers 1 are free here: before the switch A reads B's
      // tiles (and its own buffers 0 in a lead step); the first copies into
      // buffers 1 come after the barrier that opens step s_switch.
      store_staged(cur_blk, lsum, [&](int) -> unsigned char* {
        return reinterpret_cast<unsigned char*>(gw < 2 ? xbuf(1) : xbuf(3)) + (gw & 1) * (16 * D * 2);
      });
      asm volatile("" ::: "memory");  // the next block's q loads stay behind these stores
      cur_blk = qb;
      load_q(qb);
      reset();
    }
    run(Sel<false>{}, s_switch, n_steps);
  } else {
    run(Sel<false>{}, 0, n_steps);
  }

  // B's P.V of its last step (both groups pass the barrier that publishes it).
  __builtin_amdgcn_s_waitcnt(0x0f70);
  barrier();
  if constexpr (GRP == 1) {
    if (working(n_steps - 1)) pv(V1);  // n_steps is even: its last step used buffer 1
  }

  // ---- merge the two halves of block qb --------------------------------------
  float lsum[NQT];
  row_sums(lsum);
  barrier();  // every wave is done with every tile buffer
  if constexpr (GRP == 0) {
    if (cur_blk != qb) {  // A never reached qb: its qa result is final, its qb part empty
      store(cur_blk, lsum);
      reset();
#pragma unroll
      for (int t = 0; t < NQT; ++t) lsum[t] = 0.f;
    }
    // Hand A's qb partial (O, m, l, e) to the wave of B with the same q-tiles:
    // q-tile t of wave gw goes through tile buffer gw * NQT + t.
#pragma unroll
    for (int t = 0; t < NQT; ++t) {
      float* dst = xbuf(gw * NQT + t);
#pragma unroll
      for (int dt = 0; dt < kDTiles; ++dt) *reinterpret_cast<floatx4*>(dst + (dt * 64 + lane) * 4) = oacc[t][dt];
    }
#pragma unroll
    for (int t = 0; t < NQT; ++t) {
      xs[((gw * NQT + t) * 3 + 0) * 64 + lane] = m_ref[t];
      xs[((gw * NQT + t) * 3 + 1) * 64 + lane] = lsum[t];
    }
    if (lane == 0) xs[kGWaves * NQT * 3 * 64 + gw] = __int_as_float(e_run);
  }
  barrier();
  if constexpr (GRP == 1) {
    const int ea = __float_as_int(xs[kGWaves * NQT * 3 * 64 + gw]);
    const int e_m = ea > e_run ? ea : e_run;
#pragma unroll
    for (int t = 0; t < NQT; ++t) {
      const float ma = xs[((gw * NQT + t) * 3 + 0) * 64 + lane];
      const float la = xs[((gw * NQT + t) * 3 + 1) * 64 + lane];
      const float m = fmaxf(ma, m_ref[t]);
      const float mu = m == -INFINITY ? 0.f : m;
      const float wa = la > 0.f ? fast_exp2(ma - mu) : 0.f;
      const float wb = lsum[t] > 0.f ? fast_exp2(m_ref[t] - mu) : 0.f;
      const float sa = __builtin_ldexpf(wa, ea - e_m), sb = __builtin_ldexpf(wb, e_run - e_m);
      const float* src = xbuf(gw * NQT + t);
#pragma unroll
      for (int dt = 0; dt < kDTiles; ++dt) {
        const floatx4 oa = *reinterpret_cast<const floatx4*>(src + (dt * 64 + lane) * 4);
        oacc[t][dt] = oacc[t][dt] * sb + oa * sa;
        __builtin_amdgcn_sched_barrier(0);  // one tile of A's partial at a time
      }
      lsum[t] = la * wa + lsum[t] * wb;
    }
    e_run = e_m;
    // Each wave stages q-tile t in the buffer it just read A's partial from.
    store_staged(qb, lsum, [&](int t) -> unsigned char* { return reinterpret_cast<unsigned char*>(xbuf(gw * NQT + t)); });
  }
}

}  // namespace

template <int D, int NQT, bool LO>
__global__ __launch_bounds__(2 * kGWaves * 64, 1) void gqa_prefill_pair_kernel(PrefillParams p) {
  constexpr int kTile = kUnit * D * 2;
  // Eight tile buffers (two per group per stage); after the key loop group A
  // hands its partial to group B through the first ones.
  __shared__ __attribute__((aligned(1024))) unsigned char kA0[kTile], kA1[kTile], vA0[kTile], vA1[kTile];
  __shared__ __attribute__((aligned(1024))) unsigned char kB0[kTile], kB1[kTile], vB0[kTile], vB1[kTile];
  __shared__ float xs[kGWaves * NQT * 3 * 64 + kGWaves];
  static_assert(kGWaves * NQT <= 8 && (D / 16) * 64 * 16 <= kTile, "a q-tile's partial fits one tile buffer");
  auto xbuf = [&](int i) -> float* {
    unsigned char* b;
    switch (i) {
      case 0: b = kA0; break;
      case 1: b = kA1; break;
      case 2: b = vA0; break;
      case 3: b = vA1; break;
      case 4: b = kB0; break;
      case 5: b = kB1; break;
      case 6: b = vB0; break;
      default: b = vB1; break;
    }
    return reinterpret_cast<float*>(b);
  };
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  if (wave < kGWaves) pair_group<D, NQT, LO, 0>(p, kA0, kA1, vA0, vA1, xbuf, xs);
  else pair_group<D, NQT, LO, 1>(p, kB0, kB1, vB0, vB1, xbuf, xs);
}

bool prefill_pair_serves(int group, int head_dim) {
  if (head_dim != 128 && head_dim != 256) return false;
  return group == 1 || group == 2 || group == 4 || group == 8;
}

// Work-groups of the bf16-q launch (two q-tiles per wave); the f32-q launch
// (one q-tile per wave, hi + lo q) has twice as many, each with half the work.
int prefill_pair_grid(int seqlen, int group, int kv_heads) {
  const PairShape sh = pair_shape(group, 2);
  const int nqb = (seqlen + sh.pos - 1) / sh.pos;
  return ((nqb + 1) / 2) * kv_heads * sh.nsub;
}

hipError_t launch_prefill_pair(const PrefillParams& p, int head_dim, hipStream_t stream) {
  // bf16 q converts to fp16 exactly: two q-tiles per wave.  f32 q takes two
  // fp16 terms, whose registers leave room for one q-tile per wave.
  const int nqt = p.q_f32 ? 1 : 2;
  const PairShape sh = pair_shape(p.group, nqt);
  const int nqb = (p.seqlen + sh.pos - 1) / sh.pos;
  const dim3 grid((nqb + 1) / 2, p.kv_heads * sh.nsub);
  const hipError_t vt_rc = launch_prefill_vts(p, head_dim, stream);
  if (vt_rc != hipSuccess) return vt_rc;
  const dim3 block(2 * kGWaves * 64);
  switch (head_dim) {
    case 128:
      if (p.q_f32) hipLaunchKernelGGL((gqa_prefill_pair_kernel<128, 1, true>), grid, block, 0, stream, p);
      else hipLaunchKernelGGL((gqa_prefill_pair_kernel<128, 2, false>), grid, block, 0, stream, p);
      break;
    case 256:
      if (p.q_f32) hipLaunchKernelGGL((gqa_prefill_pair_kernel<256, 1, true>), grid, block, 0, stream, p);
      else hipLaunchKernelGGL((gqa_prefill_pair_kernel<256, 2, false>), grid, block, 0, stream, p);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace bt
