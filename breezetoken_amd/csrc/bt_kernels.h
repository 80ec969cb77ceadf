// Internal launch interface between the C ABI (capi.hip) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bt {

// Largest number of splits one sequence may use.
constexpr int kMaxSplitsPerSeq = 4096;

// Tokens per decode tile (the unit dealt round-robin to splits).
constexpr int kDecodeTileTokens = 16;

struct DecodeSplitParams {
  const void* q;             // (batch, heads, D) f32 or bf16; head stride = D
  int64_t q_stride_seq;      // elements between sequences in q
  int q_bf16;                // 1: q is bf16, 0: f32
  const uint16_t* k;         // bf16 cache, token-major
  const uint16_t* v;
  int64_t kv_stride_tok;     // elements between consecutive token slots
  int64_t kv_stride_head;    // elements between kv heads of one slot
  const int64_t* seq_offset; // (batch,) first slot of each sequence, or null (0)
  const int32_t* pos;        // (batch,) valid = pos + 1, or null
  const int32_t* seq_len;    // (batch,) valid lengths, or null
  int32_t seqlen;            // valid length when pos and seq_len are null; capacity when pos is set
  const int4* work;          // (num_work,) {b, s, ns_b, base_b}, or null: uniform num_split
  int32_t num_split;
  int32_t total_splits;      // row length of lse / part per head
  int32_t heads;
  int32_t kv_heads;
  int32_t group;             // heads / kv_heads
  float scale_log2;          // softmax scale * log2(e)
  float* lse;                // (heads, total_splits)
  float* part;               // (heads, total_splits, D)
  int32_t tiles_per_split;   // > 0: a sequence of n tiles uses min(num_split, ceil(n / this)) splits
};

// Waves per decode split work-group, and the tiles per split below which
// bt_gqa_decode's single-sequence and uniform-batch modes use fewer splits
// (measured on MI355X, config 2: 8 waves x 2 tiles took 7.8 / 8.8 / 17.6 us
// per call at 1k / 4k / 32k tokens, against 15.1 / 15.6 / 21.1 us for 16
// waves x 16 tiles and 9.0 / 9.7 / 17.2 us for a fixed 128 splits).
constexpr int kDecodeWaves = 8;
constexpr int kDecodeTilesPerSplit = 2;

struct CombineParams {
  const float* lse;
  const float* part;
  int32_t num_split;            // uniform split count (split_base == null)
  int32_t total_splits;
  const int32_t* split_base;    // (batch,) first split of each sequence, or null
  const int32_t* split_count;   // (batch,) splits of each sequence, or null
  void* out;                    // (batch, heads, D)
  int out_bf16;
  int64_t out_stride_seq;
};

struct PrefillParams {
  const uint16_t* q;   // (S, H, D) with strides, f32 or bf16 (q_f32)
  const uint16_t* k;   // bf16 (S, Hkv, D)
  const uint16_t* v;
  int64_t q_stride_tok, q_stride_head;
  int64_t kv_stride_tok, kv_stride_head;
  int32_t seqlen;      // new query rows S
  int32_t q_offset;    // absolute position of query row 0 (keys: q_offset + S)
  int32_t heads;
  int32_t kv_heads;
  int32_t group;       // heads / kv_heads
  // Two-waves-per-SIMD kernel: the group runs as head_subs subsets of
  // sub_group heads (sub_group in {1, 2, 4, 8}, the largest power of two
  // dividing group; grid y = kv_heads x head_subs).
  int32_t sub_group;
  int32_t head_subs;
  float scale_log2;
  void* out;
  int out_bf16;
  int64_t out_stride_tok, out_stride_head;
  uint16_t* vt;        // workspace: fp16 V^T image, prefill_vt_bytes() bytes
  int32_t* vexp;       // workspace: per (kv head, 64-key block) power-of-two scale of the image
  uint16_t* kimg;      // workspace: fp16 K image (row-major, XOR-swizzled slots), prefill_vt_bytes() bytes
  int32_t* kexp;       // workspace: per (kv head, 64-key block) power-of-two scale of the K image
  int32_t img_blocks;  // 64-key blocks per kv head in the image layout (>= those of q_offset + seqlen keys)
  int32_t img_first;   // first block the pre-pass converts (the images already hold the earlier ones)
  int32_t q_f32;       // 1: q is f32, 0: bf16 (either enters Q.K^T as fp16 scaled per row)
  int32_t keep_images; // 1: the images must hold every block afterwards (kept across chunked-prefill calls)
  // Split-key mode of the two-waves-per-SIMD kernel (kb_chunk > 0): work-group
  // (query block, kv head, chunk c) covers key blocks [c*kb_chunk, +kb_chunk);
  // a query block with more than one chunk writes one normalised partial and
  // its log2-domain LSE per (query, head) row and chunk, merged by
  // prefill_combine_kernel.  kb_chunk = 0: one work-group per query block.
  int32_t kb_chunk;
  // split_compact = 1: the uniform split's grid x lists only the (chunk, kv
  // head subset, query block) items that have keys, each chunk's query blocks
  // padded to a multiple of 8 (grid y = z = 1); 0: grid (query blocks, kv
  // heads x subsets, max_chunks), the items past a query block's keys exiting.
  int32_t split_compact;
  // Paired split (pair_parts > 0, kb_chunk = 0): query blocks nqb-1-r and r
  // form pair r; the pair's key blocks (those of nqb-1-r, then those of r) are
  // cut into pair_parts equal ranges, one per work-group (grid x = pairs x
  // pair_parts), each covering at most two segments; a query block covered
  // by more than one range writes partials for prefill_combine_kernel.
  int32_t pair_parts;
  int32_t max_chunks;  // chunks of the longest query block (grid z of the uniform split)
  float* part;         // (kv_heads, query blocks, max_chunks, 128 rows, D) f32
  float* lse;          // (kv_heads, query blocks, max_chunks, 128 rows) f32
};

// Split-key plan of the two-waves-per-SIMD prefill: used when one work-group
// per query block would leave CUs idle (short prompts, long cached prefixes).
struct PrefillSplitPlan {
  int32_t kb_chunk = 0;    // 0: no uniform split
  int32_t compact = 0;     // uniform split on the compact grid (see PrefillParams)
  int32_t pair_parts = 0;  // 0: no paired split
  int32_t max_chunks = 1;
  int32_t query_blocks = 0;
  size_t part_rows = 0;    // kv_heads x query_blocks x max_chunks x rows per work-group
  size_t part_bytes = 0;   // part_rows x (head_dim f32 partials + 1 f32 LSE)
  bool active() const { return kb_chunk > 0 || pair_parts > 0; }
  bool uses_partials() const { return kb_chunk > 0 || (pair_parts > 0 && max_chunks > 1); }
};
PrefillSplitPlan prefill8_split_plan(int seqlen, int q_offset, int group, int kv_heads, int head_dim,
                                     int num_cus);

// Per-row RMSNorm + RoPE (row mode) and the fused decode-step preparation
// (attention mode); see attn_prep.hip.
struct RowPrepParams {
  const float* x;            // row mode: (rows, D) rows; attention mode: the fused projection output
  int64_t x_stride;          // row mode: elements between rows
  int32_t rows;              // row mode
  float* out;                // row mode: (rows, D) f32
  int64_t out_stride;
  const float* w;            // RMSNorm weight (D,) (q weight in attention mode), or null: no norm
  const float* wk;           // attention mode: k RMSNorm weight (D,), or null
  float eps;
  const float* cos;          // (rope_cap, rope_dim) tables, or null: no rotation
  const float* sin;
  const int32_t* pos;        // device position (1,)
  int32_t rope_dim;
  int32_t rope_cap;
  int32_t heads;             // attention mode
  int32_t kv_heads;
  void* q_out;               // (heads, D) f32 or bf16
  int q_out_bf16;
  uint16_t* cache_k;         // bf16 cache, token-major slots
  uint16_t* cache_v;
  int64_t kv_stride_tok;
  int64_t kv_stride_head;
  int32_t cache_cap;
};

// Gated DeltaNet single-token decode step (gdn_decode.hip).
struct GdnParams {
  const float* q;      // (heads_k, D)
  const float* k;      // (heads_k, D)
  const float* v;      // (heads_v, D)
  const float* g;      // (heads_v,) log decay
  const float* beta;   // (heads_v,) logits of the write strength
  float* state;        // (heads_v, D, D), updated in place
  float* out;          // (heads_v, D)
  int32_t heads_k;
  int32_t heads_v;
  float scale;
  float eps;
};

// Decode matvec y = x . W (gemv.hip).
struct GemvParams {
  const float* x;        // (K,) f32
  const uint16_t* w;     // (K, N) bf16, row stride ldw elements
  int64_t ldw;
  int32_t K;
  int32_t N;
  int32_t splits;        // shares of K (SK); 1: no partials
  float* partial;        // (SK, N) f32 when SK > 1
  float* y;              // (N,) f32
};

// Launch shape of the matvec: VEC columns per lane (tile = 64*VEC columns)
// and the number of K shares.  A wide matrix (>= 256 tiles of 512 columns,
// e.g. the vocabulary head) is not split: every CU already streams whole
// columns.  Otherwise K is split so that about 512 work-groups stream W with
// at least 64 rows per share (measured on MI355X against 256/1024/2048/4096
// groups and 16/32/128 rows).
constexpr int kGemvTargetGroups = 512;
constexpr int kGemvMinRows = 64;
inline void gemv_shape(int K, int N, int* vec, int* splits, int* tiles) {
  const int tiles8 = (N + 511) / 512;
  *vec = tiles8 >= 8 ? 8 : 4;
  *tiles = (N + 64 * *vec - 1) / (64 * *vec);
  if (tiles8 >= 256) {
    *splits = 1;
    return;
  }
  const int sk = (kGemvTargetGroups + *tiles - 1) / *tiles;
  const int cap = K / kGemvMinRows > 1 ? K / kGemvMinRows : 1;
  *splits = sk < 1 ? 1 : (sk > cap ? cap : sk);
}

// Workspace of the split-K matvec: the partial rows.
inline size_t gemv_workspace_bytes(int K, int N) {
  int vec, sk, tiles;
  gemv_shape(K, N, &vec, &sk, &tiles);
  return sk == 1 ? 0 : (size_t)sk * N * 4;
}

// Keys per block of the prefill key loop, and the size of the transposed,
// block-scaled fp16 V image the prefill builds in its workspace: per kv head and 64-key block,
// 8 chunks of 8 keys x head_dim rows x 16 bytes, for kv_len keys.
constexpr int kPrefillKeyBlock = 64;
inline size_t prefill_vt_bytes(int kv_len, int kv_heads, int head_dim) {
  const size_t blocks = (size_t)(kv_len + kPrefillKeyBlock - 1) / kPrefillKeyBlock;
  return (size_t)kv_heads * blocks * kPrefillKeyBlock * (size_t)head_dim * 2;
}

// Which kernel variant serves a combination of length sources, or -1 if the
// combination is not served:
//   work table (ragged)              -> needs seq_len and seq_offset, no pos
//   pos, batch 1, no seq_offset      -> single sequence, device position
//   pos + seq_offset                 -> batch of device positions
//   seq_len + seq_offset             -> batch of device lengths
//   none of them, batch 1            -> explicit length argument
inline int decode_mode(bool work, bool pos, bool seq_len, bool seq_offset, int batch) {
  if (work) return (seq_len && seq_offset && !pos) ? 3 : -1;
  if (pos) {
    if (seq_len) return -1;
    if (!seq_offset) return batch == 1 ? 1 : -1;
    return 2;
  }
  if (seq_len) return seq_offset ? 4 : -1;
  return (batch == 1 && !seq_offset) ? 0 : -1;
}

// Device-side ragged plan (ragged_plan.hip): the plan bt_ragged_plan makes on
// the host, from device lengths, padded to work_capacity entries with {-1, ..}.
constexpr int kRaggedPlanMaxBatch = 4096;
struct RaggedPlanParams {
  const int32_t* seq_len;  // (batch,) device lengths
  int32_t batch;
  int32_t target_groups;
  int32_t* work;           // (work_capacity, 4) entries {b, s, ns_b, base_b}
  int32_t work_capacity;   // >= max(batch, target_groups)
  int32_t* split_base;     // (batch,)
  int32_t* split_count;    // (batch,)
  int32_t* total;          // optional: the number of real entries
};
hipError_t launch_ragged_plan(const RaggedPlanParams& p, hipStream_t stream);

hipError_t launch_decode_split(const DecodeSplitParams& p, int head_dim, int grid_x, int batch,
                               hipStream_t stream);
hipError_t launch_decode_combine(const CombineParams& p, int head_dim, int heads, int batch,
                                 hipStream_t stream);
// Two-waves-per-SIMD prefill (gqa_prefill8.hip) for group sizes 1..8: a
// group runs as subsets of prefill8_sub_group(group) heads.
bool prefill8_serves(int group, int head_dim);
int prefill8_sub_group(int group);
// Pair kernel (gqa_prefill_pair.hip): two query blocks per work-group, 32
// query columns per wave; group sizes 1, 2, 4, 8.
bool prefill_pair_serves(int group, int head_dim);
int prefill_pair_grid(int seqlen, int group, int kv_heads);
hipError_t launch_prefill_pair(const PrefillParams& p, int head_dim, hipStream_t stream);
// Scaled fp16 V^T image + per-block exponents (p.vt, p.vexp) in the key order
// of the 16x16 MFMA result layout, and the scaled fp16 K image + exponents
// (p.kimg, p.kexp).
hipError_t launch_prefill_vts(const PrefillParams& p, int head_dim, hipStream_t stream);
hipError_t launch_prefill8(const PrefillParams& p, int head_dim, hipStream_t stream);
hipError_t launch_row_norm_rope(const RowPrepParams& p, int head_dim, hipStream_t stream);
hipError_t launch_attn_prep(const RowPrepParams& p, int head_dim, hipStream_t stream);
hipError_t launch_gdn_decode(const GdnParams& p, int dim, hipStream_t stream);
hipError_t launch_gemv(const GemvParams& p, int vec, hipStream_t stream);

}  // namespace bt
