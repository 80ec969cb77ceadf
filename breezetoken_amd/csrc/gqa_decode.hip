// Split-KV GQA flash-decode for gfx950 (MI355X) over a bf16 token-major KV cache.
//
// Semantics follow the reference split kernel (breezetoken/kernels/cuda/
// attention.py:88-166, fixed-capacity variant 249-326): the valid context is cut
// into tiles, every split writes, per query head, a log2-domain LSE
//     lse = log2(l) + m,   l = sum_j exp2(x_j - m),   x_j = q.k_j * scale * log2e
// and the normalised partial output sum_j exp2(x_j - m) v_j / l (attention.py:
// 153-166); an empty split writes lse = -inf and leaves its partial untouched
// (the combine never reads it).  One deliberate difference: tiles are dealt to
// splits round-robin (tile t -> split t mod NS) instead of in contiguous ranges
// (attention.py:106-112).  The LSE combine is invariant to how tokens are
// partitioned, and with round-robin dealing a split's first tile (tile s) is
// known before the position tensor is read, so its loads start at kernel entry.
//
// Work decomposition (MI355X-first, not the reference's):
//  * one work-group (WAVES waves) per (split, kv head, sequence); the group's G
//    query heads ride in the N dimension of the MFMA, so every K/V byte fetched
//    from HBM is used by all G heads;
//  * q is pre-scaled by scale*log2e and split into bf16 hi + lo columns (columns
//    h and 2*GMAX-1-h), so Q.K^T keeps ~16 mantissa bits although the MFMA takes
//    bf16; the two halves are summed with one DPP mirror.  P is split the same
//    way for the P.V product;
//  * S^T = K . Q^T puts the K tile in the A operand, so K rows go straight from
//    HBM into registers with 16-byte buffer loads (64 contiguous bytes per token
//    per instruction); loads past the valid length return zero (buffer bounds);
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

__device__ __forceinline__ int swz(int row, int slots) { return ((row & 7) * 2) & (slots - 1); }

template <int V>
struct IntConst {
  static constexpr int value = V;
};

// Raw buffer resource over [base, base + bytes): loads past the end return 0,
// so tokens past the valid length need no clamping.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
constexpr float kDecodeLazy = 8.0f;  // log2-domain slack before the reference max moves

// K/V are streamed once per call: the non-temporal policy (nt) keeps them from
// displacing reusable lines and measurably raises the stream rate on gfx950.
constexpr int kPolicyStream = 2;  // gfx940+ cache-policy bits: nt
__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, kPolicyStream);
}

typedef short short4_t __attribute__((ext_vector_type(4)));

// Scalar (constant-cache) read of a wave-uniform value written by an earlier
// kernel: issued as s_load, so its wait lands at the first use instead of
// forcing a vector load + readfirstlane right away.
template <typename T>
__device__ __forceinline__ T uniform_load(const T* p, int i) {
  return ((const __attribute__((address_space(4))) T*)(p))[i];
}

__device__ __forceinline__ floatx4 mfma16k16(const u32x2& a, const u32x2& b, const floatx4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(short4_t, a),
                                                  __builtin_bit_cast(short4_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ u32x2 lds_read_tr4(const BT_LDS uint16_t* p) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((BT_LDS bf16x4*)p));
}

template <int GMAX>
__device__ __forceinline__ float mirror(float v) {
  return (GMAX <= 4) ? dpp_f32<DPP_ROW_HALF_MIRROR>(v) : dpp_f32<DPP_ROW_MIRROR>(v);
}

}  // namespace

// Where the valid length of a sequence comes from.  Each mode is its own
// kernel, so the prologue has no argument-dependent branches and all kernel
// arguments arrive in one batch of scalar loads.
enum DecodeMode : int {
  kModeLen = 0,       // explicit length argument (eager decode)
  kModePos = 1,       // device position of one sequence (graph decode)
  kModePosBatch = 2,  // device positions + first slots of a batch in one cache
  kModeRagged = 3,    // work table + device lengths + first slots
  kModeLenBatch = 4,  // device lengths + first slots, uniform split count
};

// Split pass.  GMAX: 4 (groups of <= 4 query heads) or 8; D: head dim; W:
// waves per work-group; MODE: a DecodeMode; QBF16: q is bf16 (else f32).
//
// Tile t (16 tokens) of a sequence belongs to split t % ns_eff and, inside
// it, to wave (t / ns_eff) % W; a wave's successive tiles are ns_eff * W
// apart.  ns_eff = min(ns, ceil(tiles / tiles_per_split)) when the launch
// gives tiles_per_split (single-sequence and uniform-batch modes), else ns: a
// short context in a large grid then spreads over ceil(tiles / 2) splits
// instead of leaving most waves of 128 work-groups idle, and the splits past
// ns_eff write lse = -inf at once.
//
// Per tile and wave, K (16 tokens x D) and V land in registers; K feeds the
// MFMA directly, V is staged through the wave's XOR-swizzled LDS tile and read
// back transposed.  A wave requests its next V as soon as the current V is in
// LDS, and its next K as soon as Q.K^T has consumed the current one -- except
// after the first tile, where the next K goes out with the next V.  A wave's
// first tile is requested after its slice of Q^T is built (wave 0's, at entry).
template <int GMAX, int D, int W, int MODE, bool QBF16>
__global__ __launch_bounds__(W * 64, 1) void gqa_decode_split_kernel(DecodeSplitParams p) {
  constexpr int kThreads = W * 64;
  constexpr int kSteps = D / 32;            // K-dimension steps of Q.K^T
  constexpr int kDTiles = D / 16;           // 16-wide d tiles of O^T
  constexpr int kSlots = D / 8;             // 16-byte chunks per row
  constexpr int kRowBytes = D * 2;          // one kv head of one token
  constexpr int kTileBytes = 16 * kRowBytes;
  constexpr int kVLoads = kTileBytes / 1024;  // 1 KiB wave loads per V tile
  constexpr int kRowsPerLoad = 1024 / kRowBytes;
  static_assert(kVLoads >= 1 && kSlots >= 8, "head_dim 64, 128 or 256");
  static_assert(kSteps <= W, "one wave per d-step builds Q^T");

  // LDS: one V tile per wave (16-byte chunk c of token row r in slot c ^
  // swz(r), so the transposed reads of 16 rows are conflict-free), the
  // cross-wave merge rows [wave][head][d] with a stride of D + 4 floats (the
  // lanes that store one d-tile of different heads fall on distinct banks), a
  // wave deposits its partial as soon as its own loop ends, and the Q^T
  // operand shared by all waves.
  constexpr int kMoStride = D + 4;
  __shared__ __attribute__((aligned(1024))) unsigned char vlds[W * kTileBytes];
  __shared__ __attribute__((aligned(16))) float mlds[W * GMAX * kMoStride];
  __shared__ __attribute__((aligned(16))) u32x4 qlds[kSteps * 64];  // [step][lane]
  __shared__ float mstat[2 * W * GMAX];                              // m and l per (wave, head)
  static_assert(W * kTileBytes + W * GMAX * kMoStride * 4 + kSteps * 1024 + 8 * W * GMAX <= 160 * 1024,
                "LDS budget");

  // Every kernel argument lands in SGPRs in one batch of scalar loads here,
  // instead of lazily inside branches (each lazy batch is a memory round trip).
  asm volatile("" ::"s"(p.q), "s"(p.k), "s"(p.v), "s"(p.pos), "s"(p.seq_len), "s"(p.seq_offset),
               "s"(p.work), "s"(p.seqlen), "s"(p.num_split), "s"(p.total_splits), "s"(p.group),
               "s"(p.kv_stride_tok), "s"(p.kv_stride_head), "s"(p.q_stride_seq), "s"(p.scale_log2),
               "s"(p.lse), "s"(p.part), "s"(p.tiles_per_split));
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // The kv heads of a split (or of a ragged work entry) are neighbours in the
  // grid's x (work-group x = split * Hkv + head): the heads of one token share
  // a cache row, and work-groups dispatched together then read both halves of
  // the same rows at about the same time, which the DRAM serves better (C2 32k
  // -0.2 us per call, C3 32k -0.6 us, C5 -1.0 us against one grid row per head).
  // A power-of-two Hkv (every served model) splits x with a mask and a shift
  // instead of a division, which would sit before the first loads.
  int kvh, xq;
  if ((p.kv_heads & (p.kv_heads - 1)) == 0) {
    kvh = (int)blockIdx.x & (p.kv_heads - 1);
    xq = (int)blockIdx.x >> __builtin_ctz((unsigned)p.kv_heads);
  } else {
    kvh = (int)blockIdx.x % p.kv_heads;
    xq = (int)blockIdx.x / p.kv_heads;
  }
  const int G = p.group;

  int b, s, ns, base;
  if constexpr (MODE == kModeRagged) {
    const int* w = reinterpret_cast<const int*>(p.work) + 4 * xq;
    b = uniform_load(w, 0); s = uniform_load(w, 1); ns = uniform_load(w, 2); base = uniform_load(w, 3);
    if (b < 0) return;  // padding entry of a device-built plan
  } else {
    b = blockIdx.z; s = xq; ns = p.num_split; base = b * p.num_split;
  }
  // The length source is read first so its round trip overlaps the q loads.
  int len_raw;
  if constexpr (MODE == kModePos || MODE == kModePosBatch) len_raw = uniform_load(p.pos, b) + 1;
  else if constexpr (MODE == kModeRagged || MODE == kModeLenBatch) len_raw = uniform_load(p.seq_len, b);
  else len_raw = p.seqlen;
  int64_t seq_off = 0;
  if constexpr (MODE != kModeLen && MODE != kModePos) seq_off = uniform_load(p.seq_offset, b);

  const int head0 = kvh * G;
  const int split_idx = base + s;

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
  // Branch-free operand selection: keep_hi / keep_lo are all-ones or zero.
  const uint32_t keep_hi = (col_head >= 0 && !col_lo) ? 0xffffffffu : 0u;
  const uint32_t keep_lo = col_lo ? 0xffffffffu : 0u;
  // Two values as bf16 hi = rne(x) and lo = rne(x - hi), packed: the hi
  // columns take hi, the lo columns lo, the others zero.
  auto hilo2 = [&](float a, float b) -> uint32_t {
    const uint32_t hi = f32x2_to_bf16x2_bits(a, b);
    const uint32_t lo = f32x2_to_bf16x2_bits(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xffff0000u));
    return (hi & keep_hi) | (lo & keep_lo);
  };

  // ---- q first: wave w < kSteps loads the q slice of d-step w at entry ------
  // (a wave's loads complete in issue order, so q must not queue behind K/V).
  const int64_t qrow = (int64_t)b * p.q_stride_seq + (int64_t)(head0 + (col_head < 0 ? 0 : col_head)) * D;
  u32x4 qraw[2];
  if (wave < kSteps) {
    const int d0 = (wave * 4 + kg) * 8;
    if constexpr (QBF16) {
      qraw[0] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(p.q) + qrow + d0);
    } else {
      qraw[0] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const float*>(p.q) + qrow + d0);
      qraw[1] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const float*>(p.q) + qrow + d0 + 4);
    }
  }

  // ---- K/V addressing -------------------------------------------------------
  // K: lane (col, kg) holds token col's 16 bytes kg of each 64-byte d-step.
  // V: load j of a tile fills LDS bytes [1024 j, +1024) of the wave's tile;
  // lane l fetches the chunk that belongs in its slot (the swizzle is applied
  // on the source side).
  const uint32_t row_bytes = (uint32_t)(p.kv_stride_tok * 2);
  unsigned char* vtile = vlds + wave * kTileBytes;
  const uint32_t koff = (uint32_t)col * row_bytes + kg * 16;
  auto voff = [&](int j) -> uint32_t {
    const int r = j * kRowsPerLoad + lane / kSlots;
    return (uint32_t)(lane / kSlots) * row_bytes + (uint32_t)((lane % kSlots) ^ swz(r, kSlots)) * 16;
  };

  // Speculative path (device position, single sequence): the split's first
  // tile is tile s whatever ns_eff turns out to be, so wave 0 fetches it inside
  // the capacity bound before the position is known; rows past the valid
  // length are zeroed once it arrives.
  constexpr bool kSpec = MODE == kModePos;
  const int64_t head_off0 = (int64_t)kvh * p.kv_stride_head;
  __amdgpu_buffer_rsrc_t krs = make_rsrc(p.k + head_off0, (uint32_t)p.seqlen * row_bytes);
  __amdgpu_buffer_rsrc_t vrs = make_rsrc(p.v + head_off0, (uint32_t)p.seqlen * row_bytes);

  u32x4 kr[kSteps];
  u32x4 vr[kVLoads];
  auto issue_k = [&](int tile) {
    const uint32_t so = (uint32_t)tile * 16 * row_bytes;
#pragma unroll
    for (int st = 0; st < kSteps; ++st) kr[st] = buf_load16(krs, koff + st * 64, so);
  };
  auto issue_v = [&](int tile) {
    const uint32_t so = (uint32_t)tile * 16 * row_bytes;
#pragma unroll
    for (int j = 0; j < kVLoads; ++j) vr[j] = buf_load16(vrs, voff(j), so + (uint32_t)(j * kRowsPerLoad) * row_bytes);
  };
  const bool spec_loaded = kSpec && wave == 0;
  if (spec_loaded) {
    issue_k(s);
    issue_v(s);
  }

  // ---- valid length, effective split count, this wave's tiles --------------
  int valid = len_raw;
  if constexpr (MODE == kModePos || MODE == kModePosBatch) {
    if (valid > p.seqlen) valid = p.seqlen;  // seqlen carries the capacity here
  }
  if (valid < 0) valid = 0;
  // From here on loads stop at the valid length: rows past it read as zeros.
  {
    const int64_t head_off = seq_off * p.kv_stride_tok + head_off0;
    krs = make_rsrc(p.k + head_off, (uint32_t)valid * row_bytes);
    vrs = make_rsrc(p.v + head_off, (uint32_t)valid * row_bytes);
  }
  const int tiles = (valid + 15) / 16;
  int ns_eff = ns;
  if constexpr (MODE != kModeRagged) {
    if (p.tiles_per_split > 0) {
      int want;
      if (p.tiles_per_split == kDecodeTilesPerSplit) want = (tiles + kDecodeTilesPerSplit - 1) / kDecodeTilesPerSplit;
      else want = (tiles + p.tiles_per_split - 1) / p.tiles_per_split;
      ns_eff = want < 1 ? 1 : (want < ns ? want : ns);
    }
  }
  if (s >= ns_eff || s >= tiles) {
    if (threadIdx.x < G) p.lse[(int64_t)(head0 + threadIdx.x) * p.total_splits + split_idx] = -INFINITY;
    return;
  }
  const int tstride = ns_eff * W;                       // tile distance between a wave's steps
  const int tfirst = s + ns_eff * wave;                 // this wave's first tile
  // ---- Q^T operand (bf16 hi or lo of q*scale*log2e): wave w builds d-step w.
  if (wave < kSteps) {
    float qv[8];
    if constexpr (QBF16) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        qv[2 * i] = bf16_bits_to_f32(qraw[0][i] & 0xffffu);
        qv[2 * i + 1] = bf16_bits_to_f32(qraw[0][i] >> 16);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        qv[i] = __uint_as_float(qraw[0][i]);
        qv[4 + i] = __uint_as_float(qraw[1][i]);
      }
    }
    u32x4 qw;
#pragma unroll
    for (int i = 0; i < 4; ++i) qw[i] = hilo2(qv[2 * i] * p.scale_log2, qv[2 * i + 1] * p.scale_log2);
    qlds[wave * 64 + lane] = qw;
  }
  // The first tile's loads go out after the Q^T build: issued before it, they
  // would sit behind q in the wave's load queue on one path and not on the
  // other (a wave without tiles), and the compiler's wait for q would then be
  // for every load -- the wave's first tile, and through the barrier the
  // slowest wave's.  q and pos arrive about together, so this costs little.
  if (tfirst < tiles && !spec_loaded) {
    issue_k(tfirst);
    issue_v(tfirst);
  }
  // Publish Q^T without waiting for the K/V requests in flight (no vmcnt wait).
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

  // ---- per-wave state -------------------------------------------------------
  floatx4 oacc[kDTiles];
#pragma unroll
  for (int i = 0; i < kDTiles; ++i) oacc[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;
  float l_run = 0.f;
  const int i16 = lane & 15;
  const int row1 = 4 * kg + (i16 >> 2);  // V^T read: token row of this lane

  for (int it = 0, tile = tfirst; tile < tiles; ++it, tile += tstride) {
    const bool first = it == 0;
    const bool more = tile + tstride < tiles;
    // S^T = K . Q^T.
    floatx4 sacc = {0.f, 0.f, 0.f, 0.f};
    u32x4 qop[kSteps];
#pragma unroll
    for (int st = 0; st < kSteps; ++st) qop[st] = qlds[st * 64 + lane];
#pragma unroll
    for (int st = 0; st < kSteps; ++st) sacc = mfma16(as_bf16x8(kr[st]), as_bf16x8(qop[st]), sacc);
    // The next K goes out here, except after the first tile: there it waits
    // for the V staging, which keeps the compiler's waits at the first Q.K^T
    // exact (each MFMA waits for its own K load) without the next requests
    // joining the queue while the first V is still arriving (4k -0.2 us,
    // C3 32k -0.18 us, 32k -0.08 us; issued late in every step, 131k +0.9 us).
    if (more && !first) issue_k(tile + tstride);
    // Stage V in this wave's swizzled LDS tile (same-wave LDS ops stay
    // ordered) and request the next V.  Rows past the valid length are zeros
    // (buffer range), except in a speculative tile read inside the capacity:
    // there they are zeroed here, since p = 0 on them but 0 * NaN is not 0.
    const bool spec_tail = kSpec && first && spec_loaded && tile * 16 + 16 > valid;
#pragma unroll
    for (int j = 0; j < kVLoads; ++j) {
      const u32x4 z = {0u, 0u, 0u, 0u};
      const bool dead = spec_tail && tile * 16 + j * kRowsPerLoad + lane / kSlots >= valid;
      *reinterpret_cast<BT_LDS u32x4*>((BT_LDS unsigned char*)vtile + j * 1024 + lane * 16) = dead ? z : vr[j];
    }
    if (more) {
      if (first) issue_k(tile + tstride);
      issue_v(tile + tstride);
    }

    // hi + lo columns, mask, online softmax (attention.py:21-51 semantics).
    float x[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float vv = sacc[j];
      vv += mirror<GMAX>(vv);
      x[j] = tile * 16 + kg * 4 + j < valid ? vv : -INFINITY;
    }
    float tmax = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
    tmax = rows16_fmaxf(tmax);  // the column's four lane groups (VALU lane swaps)
    tmax = halves_fmaxf(tmax);
    // Lazy reference max: m_run moves only when a score exceeds it by more
    // than 2^8 (log2 domain), so p <= 2^8 and O / l are rescaled only then --
    // behind a wave-uniform branch, almost never after the first tile.  The
    // LSE stays exact: lse = log2(l) + m_run for whatever reference m_run is.
    // While every score so far is masked, m_run is -inf and does not move
    // (-inf > -inf + 8 is false); subtracting 0 then makes exp2 see -inf
    // (not NaN), so p = 0 acts on an O and l that are 0.
    const bool move = tmax > m_run + kDecodeLazy;
    const float m_new = move ? tmax : m_run;
    const float alpha = move ? fast_exp2(m_run - m_new) : 1.f;  // 0 when m_run is -inf
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    float pr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) pr[j] = fast_exp2(x[j] - m_use);
    m_run = m_new;
    l_run = l_run * alpha + ((pr[0] + pr[1]) + (pr[2] + pr[3]));
    // O is zero before the first tile, where alpha is always 0 (m_run starts
    // at -inf): no rescale there (C2 1k / 4k / 32k -0.15 / -0.15 / -0.09 us
    // together with the folded mirror adds below, bit-identical).
    if (!first && __builtin_amdgcn_ballot_w64(alpha != 1.f)) {
#pragma unroll
      for (int i = 0; i < kDTiles; ++i) oacc[i] *= alpha;
    }
    // P^T operand: this lane's own probabilities, as bf16 hi or lo.
    const u32x2 pop = {hilo2(pr[0], pr[1]), hilo2(pr[2], pr[3])};

    // O^T += V^T . P^T, V^T read transposed from LDS.
    u32x2 vop[kDTiles];
#pragma unroll
    for (int dt = 0; dt < kDTiles; ++dt) {
      const int c = dt * 2 + ((i16 & 3) >> 1);
      vop[dt] = lds_read_tr4((const BT_LDS uint16_t*)((BT_LDS unsigned char*)vtile + row1 * kRowBytes +
                                                      ((c ^ swz(row1, kSlots)) * 16) + (i16 & 1) * 8));
    }
#pragma unroll
    for (int dt = 0; dt < kDTiles; ++dt) oacc[dt] = mfma16k16(vop[dt], pop, oacc[dt]);
  }

  // ---- wave epilogue: full row sums, hi + lo merge ---------------------------
  l_run = halves_sum(rows16_sum(l_run));
#pragma unroll
  for (int dt = 0; dt < kDTiles; ++dt) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float v = oacc[dt][j];
      oacc[dt][j] = v + mirror<GMAX>(v);
    }
    // Keep the adds here: only the stores below use them, and the compiler
    // would sink them into the store branch, away from the lane moves (which
    // must run with every lane active), so each move could not fold into
    // its add.
    asm volatile("" : "+v"(oacc[dt]));
  }

  // ---- cross-wave merge through LDS ----------------------------------------
  // After the mirror sum the hi lane (col = h) and the lo lane (col =
  // 2*GMAX-1-h) hold the same head-h sums: the hi lane stores the even
  // d-tiles and the lo lane the odd ones, so each store instruction carries
  // twice the lanes and a wave issues kDTiles/2 of them.
  float* mm = mstat;                // [wave][GMAX]
  float* ml = mstat + W * GMAX;     // [wave][GMAX]
  if (col_head >= 0) {
    const int par = col_lo ? 1 : 0;
    float* dst = mlds + (wave * GMAX + col_head) * kMoStride + par * 16 + kg * 4;
#pragma unroll
    for (int q = 0; q < kDTiles / 2; ++q) {
      const floatx4 a = oacc[2 * q], c = oacc[2 * q + 1];
      const float4 v4 = {par ? c[0] : a[0], par ? c[1] : a[1], par ? c[2] : a[2], par ? c[3] : a[3]};
      *reinterpret_cast<float4*>(dst + q * 32) = v4;
    }
    if (kg == 0 && !col_lo) {
      mm[wave * GMAX + col_head] = m_run;
      ml[wave * GMAX + col_head] = l_run;
    }
  }
  __syncthreads();

  // Each thread finishes (head, 4 consecutive d) items, over the first NW
  // waves' partials: the waves dealt a tile of this split (wave w's first tile
  // is s + ns_eff * w), rounded up to 2, 4 or W.  The others' partials are
  // zeros with weight 0 and are not read (C2 1k / 4k -0.15 / -0.19 us).
  auto merge = [&](auto nw) {
    constexpr int NW = decltype(nw)::value;
    for (int item = threadIdx.x; item < G * (D / 4); item += kThreads) {
      const int h = item / (D / 4);
      const int d = (item % (D / 4)) * 4;
      // Every LDS read is issued before the first use and the weights are a
      // select, not a branch (a branch per wave made each l read its own LDS
      // round trip).  A wave without valid tokens has l = 0, m = -inf and a
      // zero partial: its weight is 0 (the exp2 of its NaN difference is
      // discarded).
      float mw[NW], lw[NW];
      float4 ow[NW];
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        mw[w] = mm[w * GMAX + h];
        lw[w] = ml[w * GMAX + h];
        ow[w] = *reinterpret_cast<const float4*>(mlds + (w * GMAX + h) * kMoStride + d);
      }
      float mx = -INFINITY;
#pragma unroll
      for (int w = 0; w < NW; ++w) mx = fmaxf(mx, mw[w]);
      float lsum = 0.f;
      float4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float e = fast_exp2(mw[w] - mx);
        const float sc = lw[w] > 0.f ? e : 0.f;
        lsum += lw[w] * sc;
        acc.x += ow[w].x * sc; acc.y += ow[w].y * sc; acc.z += ow[w].z * sc; acc.w += ow[w].w * sc;
      }
      const int64_t row = (int64_t)(head0 + h) * p.total_splits + split_idx;
      // The partial is stored unconditionally (zeros for a split without
      // valid tokens, whose lse of -inf the combine skips), so the compiler
      // cannot sink its LDS reads behind the weights' into a second round trip.
      const bool has = lsum > 0.f;
      const float inv = has ? 1.f / lsum : 0.f;
      acc.x *= inv; acc.y *= inv; acc.z *= inv; acc.w *= inv;
      *reinterpret_cast<float4*>(p.part + row * D + d) = acc;
      if (d == 0) p.lse[row] = has ? fast_log2(lsum) + mx : -INFINITY;
    }
  };
  if constexpr (W > 4) {
    // Wave w has a tile iff s + ns_eff * w < tiles.
    if (s + 2 * ns_eff >= tiles) merge(IntConst<2>{});
    else if (s + 4 * ns_eff >= tiles) merge(IntConst<4>{});
    else merge(IntConst<W>{});
  } else {
    merge(IntConst<W>{});
  }
}


// LSE combine (attention.py:168-189).  One wave per (head, sequence,
// 8-column chunk): lane = (split group lane >> 1, float4 column lane & 1).
// Each lane fetches the partials and LSEs of its splits in one batch; the max
// and the sums over the 32 split groups are lane shuffles, so the kernel makes
// one memory round trip before its store and has no barrier (splits past the
// first 32*kPre take a slower second pass).  When this layout was chosen, a
// config-2 call at 32k (split kernel of that time included) took 17.05 us
// with it, against 17.17 us with 16 groups x 4 columns, 17.18 us with 64
// groups x 1 column, and 17.68 us for a 256-thread work-group per 64-column
// chunk with LDS reductions.
template <int D, bool RAGGED, int GROUPS>
__global__ __launch_bounds__(64) void gqa_decode_combine_kernel(CombineParams p) {
  static_assert(GROUPS >= 1 && GROUPS <= 64 && (GROUPS & (GROUPS - 1)) == 0,
                "split groups are a power of two that divides the 64 lanes");
  constexpr int kCols = 64 / GROUPS;   // float4 columns per wave
  constexpr int kPre = 128 / GROUPS;   // splits per lane fetched up front (GROUPS x kPre = 128)
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int chunk = blockIdx.z;
  const int t = threadIdx.x;
  int base, ns;
  if constexpr (RAGGED) {
    base = p.split_base[b];
    ns = p.split_count[b];
  } else {
    base = b * p.num_split;
    ns = p.num_split;
  }
  const float* lse = p.lse + (int64_t)h * p.total_splits + base;
  const int c4 = t % kCols;  // float4 column inside the chunk
  const int sg = t / kCols;  // split group
  const float* part = p.part + ((int64_t)h * p.total_splits + base) * D + chunk * 4 * kCols + c4 * 4;

  float4 pv[kPre];
  float pl[kPre];
  if constexpr (!RAGGED) {
    // Buffer loads bounded by the split count: the lanes of splits past it
    // read zeros (their lse is then set to -inf), so every load issues without
    // a branch around it (C2 4k / 32k -0.1 us per call).  A ragged batch's
    // sequences have a few splits each, so its waves skip the loads instead
    // (C5 +0.16 us issuing them all).
    const __amdgpu_buffer_rsrc_t prs = make_rsrc(p.part + ((int64_t)h * p.total_splits + base) * D, (uint32_t)ns * D * 4);
    const __amdgpu_buffer_rsrc_t lrs = make_rsrc(lse, (uint32_t)ns * 4);
    const uint32_t coff = (uint32_t)(chunk * 4 * kCols + c4 * 4) * 4;
#pragma unroll
    for (int i = 0; i < kPre; ++i) {
      const int s = sg + GROUPS * i;
      pv[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(prs, (int)((uint32_t)s * D * 4 + coff), 0, 0));
      const float l = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(lrs, s * 4, 0, 0));
      pl[i] = s < ns ? l : -INFINITY;
    }
  } else {
#pragma unroll
    for (int i = 0; i < kPre; ++i) {
      const int s = sg + GROUPS * i;
      pl[i] = -INFINITY;
      pv[i] = float4{0.f, 0.f, 0.f, 0.f};
      if (s < ns) {
        pv[i] = *reinterpret_cast<const float4*>(part + (int64_t)s * D);
        pl[i] = lse[s];
      }
    }
  }
  // NaN-propagating max (no operand canonicalisation): an LSE is finite or
  // -inf, and a NaN one makes the output NaN either way.
  float mx = pl[0];
#pragma unroll
  for (int i = 1; i < kPre; ++i) mx = fmax_nc(mx, pl[i]);
  for (int s = sg + GROUPS * kPre; s < ns; s += GROUPS) mx = fmax_nc(mx, lse[s]);
  mx = wave_max(mx);
  // Empty splits have lse = -inf: weight 0, and their (never written) partial is skipped.
  const float m_use = mx == -INFINITY ? 0.f : mx;

  float4 acc = {0.f, 0.f, 0.f, 0.f};
  float wsum = 0.f;
#pragma unroll
  for (int i = 0; i < kPre; ++i) {
    if (pl[i] != -INFINITY) {
      const float w = fast_exp2(pl[i] - m_use);
      wsum += w;
      acc.x += w * pv[i].x; acc.y += w * pv[i].y; acc.z += w * pv[i].z; acc.w += w * pv[i].w;
    }
  }
  for (int s = sg + GROUPS * kPre; s < ns; s += GROUPS) {
    const float l = lse[s];
    if (l != -INFINITY) {
      const float w = fast_exp2(l - m_use);
      wsum += w;
      const float4 v = *reinterpret_cast<const float4*>(part + (int64_t)s * D);
      acc.x += w * v.x; acc.y += w * v.y; acc.z += w * v.z; acc.w += w * v.w;
    }
  }
  // Sum over the split groups (the lane bits above the column); every float4 column sees the
  // same splits, so each column's wsum is the full weight sum.
  acc.x = sum_from<kCols>(acc.x);
  acc.y = sum_from<kCols>(acc.y);
  acc.z = sum_from<kCols>(acc.z);
  acc.w = sum_from<kCols>(acc.w);
  wsum = sum_from<kCols>(wsum);
  if (t < kCols) {
    const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
    acc.x *= inv; acc.y *= inv; acc.z *= inv; acc.w *= inv;
    const int64_t orow = (int64_t)b * p.out_stride_seq + (int64_t)h * D + chunk * 4 * kCols + t * 4;
    if (p.out_bf16) {
      uint16_t* o = reinterpret_cast<uint16_t*>(p.out) + orow;
      const u32x2 pk = {f32x2_to_bf16x2_bits(acc.x, acc.y), f32x2_to_bf16x2_bits(acc.z, acc.w)};
      *reinterpret_cast<u32x2*>(o) = pk;
    } else {
      *reinterpret_cast<float4*>(reinterpret_cast<float*>(p.out) + orow) = acc;
    }
  }
}

template <int GMAX, int D, int MODE, bool QBF16>
static hipError_t launch_split_t(const DecodeSplitParams& p, int grid_x, int batch, hipStream_t stream) {
  const dim3 grid(grid_x * p.kv_heads, 1, batch);
  hipLaunchKernelGGL((gqa_decode_split_kernel<GMAX, D, kDecodeWaves, MODE, QBF16>), grid, dim3(kDecodeWaves * 64), 0,
                     stream, p);
  return hipGetLastError();
}

template <int GMAX, int D>
static hipError_t launch_split_mode(const DecodeSplitParams& p, int grid_x, int batch, hipStream_t stream) {
  const int mode = decode_mode(p.work != nullptr, p.pos != nullptr, p.seq_len != nullptr,
                               p.seq_offset != nullptr, batch);
  if (mode < 0) return hipErrorInvalidValue;
#define BT_SPLIT_CASE(M)                                                                      \
  case M:                                                                                     \
    return p.q_bf16 ? launch_split_t<GMAX, D, M, true>(p, grid_x, batch, stream)              \
                    : launch_split_t<GMAX, D, M, false>(p, grid_x, batch, stream);
  switch (mode) {
    BT_SPLIT_CASE(kModeLen)
    BT_SPLIT_CASE(kModePos)
    BT_SPLIT_CASE(kModePosBatch)
    BT_SPLIT_CASE(kModeRagged)
    BT_SPLIT_CASE(kModeLenBatch)
    default: return hipErrorInvalidValue;
  }
#undef BT_SPLIT_CASE
}

hipError_t launch_decode_split(const DecodeSplitParams& p, int head_dim, int grid_x, int batch,
                               hipStream_t stream) {
  const int G = p.heads / p.kv_heads;
  const bool small = G <= 4;
  switch (head_dim) {
    case 64: return small ? launch_split_mode<4, 64>(p, grid_x, batch, stream) : launch_split_mode<8, 64>(p, grid_x, batch, stream);
    case 128: return small ? launch_split_mode<4, 128>(p, grid_x, batch, stream) : launch_split_mode<8, 128>(p, grid_x, batch, stream);
    case 256: return small ? launch_split_mode<4, 256>(p, grid_x, batch, stream) : launch_split_mode<8, 256>(p, grid_x, batch, stream);
    default: return hipErrorInvalidValue;
  }
}

#ifndef BT_COMBINE_RAGGED_GROUPS
#define BT_COMBINE_RAGGED_GROUPS 8
#endif
// Split groups per combine wave: 32 for a uniform split count (up to 128
// splits per sequence); a ragged batch averages a few splits per sequence, so
// its waves take fewer groups and more columns (fewer, fuller waves).
constexpr int kCombineGroups = 32;
constexpr int kCombineRaggedGroups = BT_COMBINE_RAGGED_GROUPS;

template <int D>
static void launch_combine_t(const CombineParams& p, int heads, int batch, hipStream_t stream) {
  if (p.split_base != nullptr) {
    const dim3 grid(heads, batch, D / (4 * (64 / kCombineRaggedGroups)));
    hipLaunchKernelGGL((gqa_decode_combine_kernel<D, true, kCombineRaggedGroups>), grid, dim3(64), 0, stream, p);
  } else {
    const dim3 grid(heads, batch, D / (4 * (64 / kCombineGroups)));
    hipLaunchKernelGGL((gqa_decode_combine_kernel<D, false, kCombineGroups>), grid, dim3(64), 0, stream, p);
  }
}

hipError_t launch_decode_combine(const CombineParams& p, int head_dim, int heads, int batch,
                                 hipStream_t stream) {
  switch (head_dim) {
    case 64: launch_combine_t<64>(p, heads, batch, stream); break;
    case 128: launch_combine_t<128>(p, heads, batch, stream); break;
    case 256: launch_combine_t<256>(p, heads, batch, stream); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace bt
