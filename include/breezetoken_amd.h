/*
 * breezetoken_amd -- MI355X (gfx950) GQA attention behind a plain C ABI.
 *
 * Every entry point takes device pointers, element strides and a hipStream_t
 * (passed as void*), launches asynchronously on that stream, never allocates,
 * never synchronises and never reads device memory from the host, so every
 * call can be captured in a hipGraph.  Return value: BT_OK (0), a negative
 * BT_E* code for an argument the library refuses (nothing is launched), or a
 * positive hipError_t if the launch itself failed.
 *
 * Layouts:
 *   q       (batch, heads, head_dim)          f32 or bf16, head stride = head_dim
 *   k, v    token-major bf16 cache: element (slot, kv_head, d) at
 *           slot*kv_stride_tok + kv_head*kv_stride_head + d
 *           (the reference cache is (max_context, n_kv*head_dim), i.e.
 *           kv_stride_tok = n_kv*head_dim, kv_stride_head = head_dim)
 *   lse     (heads, total_splits) f32, log2 domain
 *   part    (heads, total_splits, head_dim) f32, normalised split outputs
 *   out     (batch, heads, head_dim) f32 or bf16, sequence stride out_stride_seq
 *
 * Query head h reads kv head h / (heads / kv_heads).  Served shapes:
 * head_dim in {64, 128, 256}, heads / kv_heads in 1..8 (decode) and 1..8
 * (prefill); pointers 16-byte aligned, strides multiples of 8 elements.
 */
#ifndef BREEZETOKEN_AMD_H
#define BREEZETOKEN_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BT_OK 0
#define BT_EINVAL (-22)  /* malformed argument: null pointer, bad shape, stride or alignment */
#define BT_ENOTSUP (-95) /* well-formed but not served (head_dim, group size, split count) */
#define BT_ENOSPC (-28)  /* workspace too small */

#define BT_DTYPE_F32 0
#define BT_DTYPE_BF16 1

/* Library version: major*10000 + minor*100 + patch. */
int bt_version(void);

/* Human-readable text for a return code of this library. */
const char* bt_strerror(int code);

/* Bytes of split workspace (lse + partials) for `total_splits` splits of
 * `heads` query heads.  Replaces the per-call torch.empty of Lse/Part in
 * _build_attention / _build_attention_fixed (breezetoken/backends.py:531-533,
 * 554-556); the caller owns it and may reuse it across calls and graph replays. */
int64_t bt_decode_workspace_bytes(int32_t heads, int32_t head_dim, int32_t total_splits);

/* Split count for one sequence of up to `ctx_len` tokens on a GPU with
 * `num_cus` compute units (the reference hard-codes 16, backends.py:526,550). */
int32_t bt_decode_pick_splits(int32_t kv_heads, int32_t ctx_len, int32_t num_cus);

/* Tokens per tile.  The split pass deals tiles to splits round-robin: tile t
 * (tokens [t*T, (t+1)*T)) belongs to split t % num_split.  The reference gives
 * each split a contiguous range instead (attention.py:106-112); the combined
 * output is the same, only the per-split partials differ. */
int32_t bt_decode_tile_tokens(void);

/* Split-KV pass: the first kernel of gqa_decode / gqa_decode_fixed
 * (breezetoken/kernels/cuda/attention.py:88-166 and 249-326).  The valid length
 * of sequence b is pos[b] + 1 when pos != NULL (the device position tensor of
 * the graph path, attention.py:296-301), else seq_len[b] when seq_len != NULL,
 * else `seqlen`.  When pos != NULL, `seqlen` must be the cache capacity in
 * slots (>= 1): no slot at or past it is read and pos[b] + 1 is clamped to it.
 * seq_offset gives each sequence's first slot; it is required when batch > 1
 * (with pos or seq_len) and must be NULL otherwise; pos and seq_len are
 * exclusive.  Writes lse/part rows [b*num_split, (b+1)*num_split) of every
 * head; total_splits = batch*num_split. */
int bt_gqa_decode_split(const void* q, int32_t q_dtype, int64_t q_stride_seq,
                        const void* k, const void* v, int64_t kv_stride_tok,
                        int64_t kv_stride_head, const int64_t* seq_offset, const int32_t* pos,
                        const int32_t* seq_len, int32_t seqlen, int32_t batch, int32_t heads,
                        int32_t kv_heads, int32_t head_dim, int32_t num_split, float scale,
                        float* lse, float* part, void* stream);

/* LSE combine: the second kernel of gqa_decode (attention.py:168-189, 328-349).
 * split_base/split_count (device, nullable) select each sequence's splits for
 * ragged batches; when NULL every sequence owns num_split consecutive splits. */
int bt_gqa_decode_combine(const float* lse, const float* part, int32_t batch, int32_t heads,
                          int32_t head_dim, int32_t num_split, const int32_t* split_base,
                          const int32_t* split_count, int32_t total_splits, void* out,
                          int32_t out_dtype, int64_t out_stride_seq, void* stream);

/* Split + combine in one call: the launch behind Backend.attention and
 * attention_fixed (breezetoken/backends.py:523-568, 657-706).  `workspace` must
 * hold bt_decode_workspace_bytes(heads, head_dim, batch*num_split) bytes. */
int bt_gqa_decode(const void* q, int32_t q_dtype, int64_t q_stride_seq, const void* k,
                  const void* v, int64_t kv_stride_tok, int64_t kv_stride_head,
                  const int64_t* seq_offset, const int32_t* pos, const int32_t* seq_len,
                  int32_t seqlen, int32_t batch, int32_t heads, int32_t kv_heads,
                  int32_t head_dim, int32_t num_split, float scale, void* workspace,
                  int64_t workspace_bytes, void* out, int32_t out_dtype,
                  int64_t out_stride_seq, void* stream);

/* Bytes of the library's own decode scratch (see bt_gqa_decode_noalloc). */
#define BT_NOALLOC_SCRATCH_BYTES (8 << 20)

/* bt_gqa_decode without a caller workspace, for callers that cannot allocate
 * (code under hipGraph capture that must not call hipMalloc, tight serving
 * loops, harnesses that forbid allocation).  No counterpart in the reference.
 * The split workspace is a file-scope device array of
 * BT_NOALLOC_SCRATCH_BYTES bytes, one per GPU, held from the library's load on
 * that GPU until the process ends; nothing is allocated per call.  A shape whose
 * bt_decode_workspace_bytes(heads, head_dim, batch*num_split) exceeds it returns
 * BT_ENOSPC without launching (H = 8, D = 256 fits up to 1,020 splits; the
 * configuration-2 grid uses 128).  All calls on one GPU share the array: calls
 * that overlap on one GPU (two streams, two threads) race and must be
 * serialised by the caller.  Arguments and results are those of bt_gqa_decode. */
int bt_gqa_decode_noalloc(const void* q, int32_t q_dtype, int64_t q_stride_seq, const void* k,
                          const void* v, int64_t kv_stride_tok, int64_t kv_stride_head,
                          const int64_t* seq_offset, const int32_t* pos, const int32_t* seq_len,
                          int32_t seqlen, int32_t batch, int32_t heads, int32_t kv_heads,
                          int32_t head_dim, int32_t num_split, float scale, void* out,
                          int32_t out_dtype, int64_t out_stride_seq, void* stream);

/* Host-side planner for ragged batches (no device access): given host lengths
 * lens[batch], choose per-sequence split counts ns_b = ceil(len_b / T) (at
 * least 1, at most ceil(len_b / 32)) for the smallest token cap T whose total
 * fits `target_groups` work-groups per kv head (one split each when the batch
 * is larger), and fill
 *   work[4*i .. 4*i+3] = {b, s, ns_b, base_b}, one entry per split (capacity
 *   work_capacity entries), longest splits first; split_base[b],
 *   split_count[b], *total_splits.
 * Returns the number of work entries, or a negative BT_E* code. */
int32_t bt_ragged_plan(const int32_t* lens, int32_t batch, int32_t target_groups,
                       int32_t* work, int32_t work_capacity, int32_t* split_base,
                       int32_t* split_count, int32_t* total_splits);

/* Device-side planner for ragged batches: the plan bt_ragged_plan makes, built
 * on `stream` from the device lengths seq_len[batch] (negative lengths count
 * as 0), so a decode step over many growing sequences needs no host
 * synchronisation and can be captured in a graph.  work (16-byte aligned,
 * work_capacity >= max(batch, target_groups) entries of 4 int32) gets the
 * real entries followed by padding entries {-1, 0, 0, 0} up to its capacity;
 * split_base/split_count as bt_ragged_plan; *total_splits (device, optional)
 * the number of real entries.  Pass work_capacity as both num_work and
 * total_splits to bt_gqa_decode_ragged, whose split kernel skips the padding.
 * batch <= 4096.  No reference counterpart (the reference decodes one
 * sequence). */
int bt_ragged_plan_device(const int32_t* seq_len, int32_t batch, int32_t target_groups,
                          int32_t* work, int32_t work_capacity, int32_t* split_base,
                          int32_t* split_count, int32_t* total_splits, void* stream);

/* Ragged multi-sequence decode over one shared cache: sequence b occupies
 * slots [seq_offset[b], seq_offset[b] + seq_len[b]).  `work`, split_base and
 * split_count are the device copies of bt_ragged_plan's output, or
 * bt_ragged_plan_device's tables (then num_work = total_splits = its
 * work_capacity).  No reference
 * counterpart (the reference decodes one sequence); it generalises
 * gqa_decode's split/combine (attention.py:54-205) to a per-sequence table. */
int bt_gqa_decode_ragged(const void* q, int32_t q_dtype, int64_t q_stride_seq, const void* k,
                         const void* v, int64_t kv_stride_tok, int64_t kv_stride_head,
                         const int64_t* seq_offset, const int32_t* seq_len, int32_t batch,
                         int32_t heads, int32_t kv_heads, int32_t head_dim,
                         const int32_t* work, int32_t num_work, const int32_t* split_base,
                         const int32_t* split_count, int32_t total_splits, float scale,
                         void* workspace, int64_t workspace_bytes, void* out, int32_t out_dtype,
                         int64_t out_stride_seq, void* stream);

/* Bytes of prefill workspace (the fp16 K image and transposed fp16 V image
 * the prefill builds once per call, each with one power-of-two scale per
 * 64-key block) for kv_len = q_offset + seqlen keys; 0 for invalid arguments.  Like
 * bt_decode_workspace_bytes it replaces a per-call allocation: the
 * reference's SDPA call (prefill.py:60-68) allocates its scratch internally. */
int64_t bt_prefill_workspace_bytes(int32_t kv_len, int32_t kv_heads, int32_t head_dim);

/* Bytes of prefill workspace that also hold the split-key partials: with at
 * least this much, bt_gqa_prefill splits the key range of long query blocks
 * across work-groups whenever one work-group per query block would leave
 * compute units idle (short prompts, long cached prefixes), and merges the
 * chunks by their LSEs.  Equal to bt_prefill_workspace_bytes(q_offset +
 * seqlen, ...) when the shape needs no split; 0 for invalid arguments.
 * Depends on the current device's CU count.  No counterpart in the reference,
 * whose SDPA call (prefill.py:60-68) sizes its scratch internally. */
int64_t bt_prefill_split_workspace_bytes(int32_t seqlen, int32_t q_offset, int32_t heads,
                                         int32_t kv_heads, int32_t head_dim);

/* Causal GQA prefill attention on fp16 MFMA.  Replaces the
 * F.scaled_dot_product_attention(is_causal=True, enable_gqa=True) call of
 * _prefill_attn (breezetoken/model/prefill.py:56-68; q_offset = 0) and the
 * banded-mask chunked prefill of Qwen36MoE._attn_batch
 * (breezetoken/model/qwen36_moe.py:394-428; q_offset = pos0).  q (seqlen,
 * heads, D): the new tokens, at absolute positions q_offset .. q_offset +
 * seqlen - 1, f32 (as the reference computes it, prefill.py:49-68) or bf16
 * (q_dtype); Q.K^T takes q as fp16 scaled by a power of two per row;
 * k/v (q_offset + seqlen, kv_heads, D) bf16 with the given strides
 * (token-major or head-major caches both fit): the cache including the new
 * tokens.  Query row i attends keys 0 .. q_offset + i.  out (seqlen, heads, D)
 * f32 or bf16.  `workspace` (16-byte aligned) must hold
 * bt_prefill_workspace_bytes(q_offset + seqlen, kv_heads, head_dim) bytes, and
 * bt_prefill_split_workspace_bytes(...) bytes for the split-key schedule; it is
 * scratch for the duration of the call on `stream`. */
int bt_gqa_prefill(const void* q, int32_t q_dtype, const void* k, const void* v, int64_t q_stride_tok,
                   int64_t q_stride_head, int64_t kv_stride_tok, int64_t kv_stride_head,
                   int32_t seqlen, int32_t q_offset, int32_t heads, int32_t kv_heads,
                   int32_t head_dim, float scale, void* workspace, int64_t workspace_bytes,
                   void* out, int32_t out_dtype, int64_t out_stride_tok, int64_t out_stride_head,
                   void* stream);

/* Split-key partials bytes bt_gqa_prefill_cached uses for this shape on the
 * current device (0: the shape runs without a split).  No reference
 * counterpart. */
int64_t bt_prefill_partials_bytes(int32_t seqlen, int32_t q_offset, int32_t heads, int32_t kv_heads,
                                  int32_t head_dim);

/* bt_gqa_prefill for chunked prefill over one cache, with the K / V^T images
 * kept across calls instead of rebuilt from the whole prefix each time (the
 * chunk loop of Qwen36MoE._attn_batch, breezetoken/model/qwen36_moe.py:
 * 394-428, re-reads the cached prefix on every chunk).  `images` (16-byte
 * aligned, persistent, bt_prefill_workspace_bytes(capacity, kv_heads,
 * head_dim) bytes) holds the images laid out for `capacity` keys; the call
 * converts the 64-key blocks from key `cached_keys` on (0 <= cached_keys <=
 * q_offset) and trusts the earlier blocks to hold this same cache's keys from
 * a previous call -- the prefix must not have changed since.  q_offset +
 * seqlen <= capacity.  `partials` (may be NULL) holds the split-key partials
 * when at least bt_prefill_partials_bytes(...) bytes.  Other arguments,
 * results and errors as bt_gqa_prefill; the results equal bt_gqa_prefill's
 * bit for bit. */
int bt_gqa_prefill_cached(const void* q, int32_t q_dtype, const void* k, const void* v, int64_t q_stride_tok,
                          int64_t q_stride_head, int64_t kv_stride_tok, int64_t kv_stride_head, int32_t seqlen,
                          int32_t q_offset, int32_t heads, int32_t kv_heads, int32_t head_dim, float scale,
                          void* images, int64_t images_bytes, int32_t capacity, int32_t cached_keys,
                          void* partials, int64_t partials_bytes, void* out, int32_t out_dtype,
                          int64_t out_stride_tok, int64_t out_stride_head, void* stream);

/* Per-row RMSNorm and/or partial rotate-half RoPE over rows of f32.  Replaces
 * Backend.rms_norm (breezetoken/backends.py:44-45; torch form 187-189:
 * x * rsqrt(mean(x^2) + eps) * w) and Backend.rope (backends.py:54-62; torch
 * form 218-226, kernel kernels/cuda/rope.py:13-43) on a (rows, dim) view:
 * x (rows, dim) with row stride x_stride -> out (rows, dim), row stride
 * out_stride (out may equal x).  w (dim,) or NULL: no norm (applied first).
 * cos/sin (rope_cap, rope_dim) tables or both NULL: no rotation; the first
 * rope_dim (even) dims of each row turn by row *pos of the tables, the rest
 * pass through; a position outside [0, rope_cap) uses the nearest row.
 * dim in {64, 128, 256, 512}. */
int bt_rms_norm_rope(const float* x, int64_t x_stride, int32_t rows, int32_t dim, const float* w,
                     float eps, const float* cos, const float* sin, const int32_t* pos,
                     int32_t rope_dim, int32_t rope_cap, float* out, int64_t out_stride,
                     void* stream);

/* Fused decode-step preparation of one attention layer, in one launch.
 * Replaces the q/k RMSNorm + RoPE calls and the two cache writes of
 * LayerMixin._attn (breezetoken/model/layers.py:58-73) and
 * GraphMixin._graph_attn (breezetoken/model/graph.py:41-53): qkv is the fused
 * projection output laid out as in layers.py:58-64, [heads x (q | gate) of
 * 2*head_dim | kv_heads x k of head_dim | kv_heads x v of head_dim] f32.
 * Writes q_out (heads, head_dim) = rope(rms_norm(q, q_norm)) as f32 or bf16
 * (q_dtype), and at slot *pos of the bf16 cache (element (slot, kv_head, d) at
 * slot*kv_stride_tok + kv_head*kv_stride_head + d, token-major or head-major)
 * k = rope(rms_norm(k, k_norm)) and v, rounded to bf16.  q_norm/k_norm both
 * set or both NULL; cos/sin as in bt_rms_norm_rope.  A position outside
 * [0, cache_cap) writes no cache slot.  The gate half of qkv is not touched. */
int bt_attn_prep(const float* qkv, int32_t heads, int32_t kv_heads, int32_t head_dim,
                 const float* q_norm, const float* k_norm, float eps, const float* cos,
                 const float* sin, const int32_t* pos, int32_t rope_dim, int32_t rope_cap,
                 void* q_out, int32_t q_dtype, void* cache_k, void* cache_v, int64_t kv_stride_tok,
                 int64_t kv_stride_head, int32_t cache_cap, void* stream);

/* One-token Gated DeltaNet decode step with the f32 recurrent state updated
 * in place.  Replaces Backend.gdn_decode (breezetoken/backends.py:79-92;
 * torch form 242-271; kernel kernels/cuda/gdn.py:31-139) as called by
 * LayerMixin._gdn (breezetoken/model/layers.py:104-108).  q, k (heads_k, dim),
 * v (heads_v, dim), g and beta (heads_v,) f32; state (heads_v, dim, dim) f32
 * contiguous, row index = key dim, column = value dim; out (heads_v, dim) f32.
 * Value head h reads key head h % heads_k.  v, state and out 16-byte aligned;
 * dim in {64, 128}; heads_v a multiple of heads_k. */
int bt_gdn_decode(const float* q, const float* k, const float* v, const float* g, const float* beta,
                  float* state, int32_t heads_k, int32_t heads_v, int32_t dim, float scale, float eps,
                  float* out, void* stream);

/* Bytes of split-K partial rows bt_gemv_bf16 needs for a (K, N) weight (0 when
 * it does not split K); like the other workspace sizes it replaces the
 * reference's per-shape partial buffer (backends.py:327). */
int64_t bt_gemv_workspace_bytes(int32_t K, int32_t N);

/* Decode matvec y (N,) f32 = x (K,) f32 . w (K, N) bf16, w row-major with row
 * stride ldw elements.  Replaces Backend.linear (breezetoken/backends.py:36-37;
 * torch form 182-184) as served by the split-K bf16 GEMV of
 * kernels/cuda/gemv.py:18-40 (selected at backends.py:303-333 and 620-630) for
 * every decode projection and the vocabulary head (graph.py:81).  x stays f32
 * (the reference kernel rounds it to bf16).  N and ldw multiples of 8, w 16-byte
 * aligned, K * ldw * 2 < 2^31; `workspace` (16-byte aligned) holds
 * bt_gemv_workspace_bytes(K, N) bytes (may be NULL when that is 0).  When K is
 * split, a second small kernel adds the shares in a fixed order, so the result
 * is deterministic. */
int bt_gemv_bf16(const float* x, const void* w, int64_t ldw, int32_t K, int32_t N, float* y,
                 void* workspace, int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BREEZETOKEN_AMD_H */
