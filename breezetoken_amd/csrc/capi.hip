// The C ABI of libbreezetoken_amd.so: argument validation and launches.
// Declarations and documentation live in include/breezetoken_amd.h.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "../../include/breezetoken_amd.h"
#include "bt_kernels.h"

namespace {

constexpr double kLog2e = 1.4426950408889634;

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool served_dim(int d) { return d == 64 || d == 128 || d == 256; }
inline int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

int check_decode_common(const void* q, int32_t q_dtype, int64_t q_stride_seq, const void* k,
                        const void* v, int64_t kv_stride_tok, int64_t kv_stride_head,
                        int32_t batch, int32_t heads, int32_t kv_heads, int32_t head_dim) {
  if (!q || !k || !v) return BT_EINVAL;
  if (batch < 1 || heads < 1 || kv_heads < 1 || head_dim < 1) return BT_EINVAL;
  if (heads % kv_heads != 0) return BT_EINVAL;
  if (q_dtype != BT_DTYPE_F32 && q_dtype != BT_DTYPE_BF16) return BT_EINVAL;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v)) return BT_EINVAL;
  if (kv_stride_tok <= 0 || kv_stride_head < 0 || kv_stride_tok % 8 || kv_stride_head % 8)
    return BT_EINVAL;
  if (batch > 1 && (q_stride_seq < (int64_t)heads * head_dim || q_stride_seq % 8)) return BT_EINVAL;
  if (!served_dim(head_dim)) return BT_ENOTSUP;
  if (heads / kv_heads > 8) return BT_ENOTSUP;
  if (batch > 65535 || kv_heads > 65535) return BT_ENOTSUP;
  return BT_OK;
}

int check_out(const void* out, int32_t out_dtype, int64_t out_stride_seq, int32_t batch,
              int32_t heads, int32_t head_dim) {
  if (!out) return BT_EINVAL;
  if (out_dtype != BT_DTYPE_F32 && out_dtype != BT_DTYPE_BF16) return BT_EINVAL;
  if (!aligned16(out)) return BT_EINVAL;
  if (batch > 1 && (out_stride_seq < (int64_t)heads * head_dim || out_stride_seq % 8))
    return BT_EINVAL;
  return BT_OK;
}

bt::DecodeSplitParams make_split_params(const void* q, int32_t q_dtype, int64_t q_stride_seq,
                                        const void* k, const void* v, int64_t kv_stride_tok,
                                        int64_t kv_stride_head, const int64_t* seq_offset,
                                        const int32_t* pos, const int32_t* seq_len,
                                        int32_t seqlen, int32_t heads, int32_t kv_heads,
                                        int32_t head_dim, float scale, float* lse, float* part) {
  bt::DecodeSplitParams p{};
  p.q = q;
  p.q_stride_seq = q_stride_seq > 0 ? q_stride_seq : (int64_t)heads * head_dim;
  p.q_bf16 = q_dtype == BT_DTYPE_BF16;
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.kv_stride_tok = kv_stride_tok;
  p.kv_stride_head = kv_stride_head;
  p.seq_offset = seq_offset;
  p.pos = pos;
  p.seq_len = seq_len;
  p.seqlen = seqlen;
  p.heads = heads;
  p.kv_heads = kv_heads;
  p.group = heads / kv_heads;
  p.scale_log2 = (float)((double)scale * kLog2e);
  p.lse = lse;
  p.part = part;
  return p;
}

inline int hip_rc(hipError_t e) { return e == hipSuccess ? BT_OK : (int)e; }

}  // namespace

namespace {

// Compute units of the current device, cached per device.
int device_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  static int cache[64] = {0};
  if (dev >= 0 && dev < 64 && cache[dev] > 0) return cache[dev];
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) n = 256;
  if (dev >= 0 && dev < 64) cache[dev] = n;
  return n;
}

// Prefill workspace, each part 256-byte aligned: the fp16 V^T image, one int32
// scale exponent per kv head and 64-key block, the fp16 K image of the same
// size, and its exponents.
struct PrefillLayout {
  int64_t vexp, kimg, kexp, bytes;
};
PrefillLayout prefill_layout(int32_t kv_len, int32_t kv_heads, int32_t head_dim) {
  const int64_t img = align256((int64_t)bt::prefill_vt_bytes(kv_len, kv_heads, head_dim));
  const int64_t nblk = ((int64_t)kv_len + bt::kPrefillKeyBlock - 1) / bt::kPrefillKeyBlock;
  const int64_t tab = align256(nblk * kv_heads * 4);
  PrefillLayout l;
  l.vexp = img;
  l.kimg = l.vexp + tab;
  l.kexp = l.kimg + img;
  l.bytes = l.kexp + tab;
  return l;
}
int64_t prefill_base_bytes(int32_t kv_len, int32_t kv_heads, int32_t head_dim) {
  return prefill_layout(kv_len, kv_heads, head_dim).bytes;
}

// Long prompts whose pair grid fills the device run the pair kernel (it needs
// no split-key partials).
bool prefill_uses_pair(int32_t seqlen, int32_t heads, int32_t kv_heads, int32_t head_dim) {
  const int group = heads / kv_heads;
  if (!bt::prefill_pair_serves(group, head_dim)) return false;
  return bt::prefill_pair_grid(seqlen, group, kv_heads) >= device_cus();
}

// The split-key plan bt_gqa_prefill uses for this shape on the current device
// (kb_chunk 0: none), and where its partials start in the workspace.
bt::PrefillSplitPlan prefill_plan(int32_t seqlen, int32_t q_offset, int32_t heads, int32_t kv_heads,
                                  int32_t head_dim, int64_t* part_offset) {
  *part_offset = align256(prefill_base_bytes(q_offset + seqlen, kv_heads, head_dim));
  const int group = heads / kv_heads;
  if (!bt::prefill8_serves(group, head_dim)) return bt::PrefillSplitPlan{};
  if (prefill_uses_pair(seqlen, heads, kv_heads, head_dim)) return bt::PrefillSplitPlan{};
  // The kernel runs the group as subsets of sub_group heads, each subset a
  // row of the grid like a kv head of its own.
  const int sub = bt::prefill8_sub_group(group);
  return bt::prefill8_split_plan(seqlen, q_offset, sub, kv_heads * (group / sub), head_dim, device_cus());
}

}  // namespace

extern "C" {

int bt_version(void) { return 100; }

const char* bt_strerror(int code) {
  switch (code) {
    case BT_OK: return "success";
    case BT_EINVAL: return "invalid argument (null pointer, shape, stride or alignment)";
    case BT_ENOTSUP: return "shape not served (head_dim, group size or split count)";
    case BT_ENOSPC: return "workspace too small";
    default: return code > 0 ? hipGetErrorString((hipError_t)code) : "unknown error";
  }
}

int32_t bt_decode_tile_tokens(void) { return bt::kDecodeTileTokens; }

int64_t bt_decode_workspace_bytes(int32_t heads, int32_t head_dim, int32_t total_splits) {
  if (heads < 1 || head_dim < 1 || total_splits < 1) return 0;
  const int64_t lse = align256((int64_t)heads * total_splits * 4);
  return lse + (int64_t)heads * total_splits * head_dim * 4;
}

int32_t bt_decode_pick_splits(int32_t kv_heads, int32_t ctx_len, int32_t num_cus) {
  if (kv_heads < 1) kv_heads = 1;
  if (num_cus < 1) num_cus = 256;
  int32_t ns = (num_cus + kv_heads - 1) / kv_heads;
  const int32_t tiles = ctx_len > 0 ? (ctx_len + 31) / 32 : 1;
  if (ns > tiles) ns = tiles;
  if (ns > bt::kMaxSplitsPerSeq) ns = bt::kMaxSplitsPerSeq;
  return ns < 1 ? 1 : ns;
}

int bt_gqa_decode_split(const void* q, int32_t q_dtype, int64_t q_stride_seq, const void* k,
                        const void* v, int64_t kv_stride_tok, int64_t kv_stride_head,
                        const int64_t* seq_offset, const int32_t* pos, const int32_t* seq_len,
                        int32_t seqlen, int32_t batch, int32_t heads, int32_t kv_heads,
                        int32_t head_dim, int32_t num_split, float scale, float* lse,
                        float* part, void* stream) {
  int rc = check_decode_common(q, q_dtype, q_stride_seq, k, v, kv_stride_tok, kv_stride_head,
                               batch, heads, kv_heads, head_dim);
  if (rc) return rc;
  if (!lse || !part || !aligned16(part)) return BT_EINVAL;
  if (num_split < 1) return BT_EINVAL;
  if (num_split > bt::kMaxSplitsPerSeq) return BT_ENOTSUP;
  if (!pos && !seq_len && seqlen < 0) return BT_EINVAL;
  if (pos && seqlen < 1) return BT_EINVAL;  // capacity bound for the position path
  if (bt::decode_mode(false, pos != nullptr, seq_len != nullptr, seq_offset != nullptr, batch) < 0)
    return BT_EINVAL;
  if ((int64_t)seqlen * kv_stride_tok * 2 > (int64_t)UINT32_MAX) return BT_ENOTSUP;
  if ((int64_t)batch * num_split > INT32_MAX / 2) return BT_ENOTSUP;
  bt::DecodeSplitParams p = make_split_params(q, q_dtype, q_stride_seq, k, v, kv_stride_tok,
                                              kv_stride_head, seq_offset, pos, seq_len, seqlen,
                                              heads, kv_heads, head_dim, scale, lse, part);
  p.work = nullptr;
  p.num_split = num_split;
  p.total_splits = batch * num_split;
  return hip_rc(bt::launch_decode_split(p, head_dim, num_split, batch, (hipStream_t)stream));
}

int bt_gqa_decode_combine(const float* lse, const float* part, int32_t batch, int32_t heads,
                          int32_t head_dim, int32_t num_split, const int32_t* split_base,
                          const int32_t* split_count, int32_t total_splits, void* out,
                          int32_t out_dtype, int64_t out_stride_seq, void* stream) {
  if (!lse || !part || !aligned16(part)) return BT_EINVAL;
  if (batch < 1 || heads < 1 || total_splits < 1) return BT_EINVAL;
  if ((split_base == nullptr) != (split_count == nullptr)) return BT_EINVAL;
  if (!split_base && (num_split < 1 || (int64_t)batch * num_split > total_splits)) return BT_EINVAL;
  if (!split_base && num_split > bt::kMaxSplitsPerSeq) return BT_ENOTSUP;
  if (!served_dim(head_dim)) return BT_ENOTSUP;
  if (heads > 65535 || batch > 65535) return BT_ENOTSUP;
  int rc = check_out(out, out_dtype, out_stride_seq, batch, heads, head_dim);
  if (rc) return rc;
  bt::CombineParams c{};
  c.lse = lse;
  c.part = part;
  c.num_split = num_split;
  c.total_splits = total_splits;
  c.split_base = split_base;
  c.split_count = split_count;
  c.out = out;
  c.out_bf16 = out_dtype == BT_DTYPE_BF16;
  c.out_stride_seq = out_stride_seq > 0 ? out_stride_seq : (int64_t)heads * head_dim;
  return hip_rc(bt::launch_decode_combine(c, head_dim, heads, batch, (hipStream_t)stream));
}

int bt_gqa_decode(const void* q, int32_t q_dtype, int64_t q_stride_seq, const void* k,
                  const void* v, int64_t kv_stride_tok, int64_t kv_stride_head,
                  const int64_t* seq_offset, const int32_t* pos, const int32_t* seq_len,
                  int32_t seqlen, int32_t batch, int32_t heads, int32_t kv_heads,
                  int32_t head_dim, int32_t num_split, float scale, void* workspace,
                  int64_t workspace_bytes, void* out, int32_t out_dtype,
                  int64_t out_stride_seq, void* stream) {
  int rc = check_decode_common(q, q_dtype, q_stride_seq, k, v, kv_stride_tok, kv_stride_head,
                               batch, heads, kv_heads, head_dim);
  if (rc) return rc;
  rc = check_out(out, out_dtype, out_stride_seq, batch, heads, head_dim);
  if (rc) return rc;
  if (num_split < 1) return BT_EINVAL;
  if (num_split > bt::kMaxSplitsPerSeq) return BT_ENOTSUP;
  if ((int64_t)batch * num_split > INT32_MAX / 2) return BT_ENOTSUP;
  if (!workspace || !aligned16(workspace)) return BT_EINVAL;
  const int32_t total = batch * num_split;
  if (workspace_bytes < bt_decode_workspace_bytes(heads, head_dim, total)) return BT_ENOSPC;
  float* lse = static_cast<float*>(workspace);
  float* part = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                         align256((int64_t)heads * total * 4));
  if (!pos && !seq_len && seqlen < 0) return BT_EINVAL;
  if (pos && seqlen < 1) return BT_EINVAL;  // capacity bound for the position path
  if (bt::decode_mode(false, pos != nullptr, seq_len != nullptr, seq_offset != nullptr, batch) < 0)
    return BT_EINVAL;
  if ((int64_t)seqlen * kv_stride_tok * 2 > (int64_t)UINT32_MAX) return BT_ENOTSUP;
  bt::DecodeSplitParams p = make_split_params(q, q_dtype, q_stride_seq, k, v, kv_stride_tok,
                                              kv_stride_head, seq_offset, pos, seq_len, seqlen,
                                              heads, kv_heads, head_dim, scale, lse, part);
  p.work = nullptr;
  p.num_split = num_split;
  p.total_splits = total;
  // A short context in a large grid uses fewer, fuller splits (the split count
  // follows the length on the device; the combine skips the empty splits).
  p.tiles_per_split = bt::kDecodeTilesPerSplit;
  rc = hip_rc(bt::launch_decode_split(p, head_dim, num_split, batch, (hipStream_t)stream));
  if (rc) return rc;
  return bt_gqa_decode_combine(lse, part, batch, heads, head_dim, num_split, nullptr, nullptr,
                               total, out, out_dtype, out_stride_seq, stream);
}

}  // extern "C"

// Split workspace of bt_gqa_decode_noalloc: one copy per GPU, held from the
// library's load on that GPU until the process ends.  Host code never names it
// as a device address: it uses the pointer hipGetSymbolAddress returns for the
// current device.
static __device__ __align__(256) unsigned char scratch[BT_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up once per
// device with that device current.
int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return BT_ENOTSUP;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (ptr == nullptr) return (int)hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return BT_OK;
}

}  // namespace

extern "C" {

int bt_gqa_decode_noalloc(const void* q, int32_t q_dtype, int64_t q_stride_seq, const void* k,
                          const void* v, int64_t kv_stride_tok, int64_t kv_stride_head,
                          const int64_t* seq_offset, const int32_t* pos, const int32_t* seq_len,
                          int32_t seqlen, int32_t batch, int32_t heads, int32_t kv_heads,
                          int32_t head_dim, int32_t num_split, float scale, void* out,
                          int32_t out_dtype, int64_t out_stride_seq, void* stream) {
  int rc = check_decode_common(q, q_dtype, q_stride_seq, k, v, kv_stride_tok, kv_stride_head,
                               batch, heads, kv_heads, head_dim);
  if (rc) return rc;
  if (num_split < 1) return BT_EINVAL;
  if (num_split > bt::kMaxSplitsPerSeq || (int64_t)batch * num_split > INT32_MAX / 2) return BT_ENOTSUP;
  if (bt_decode_workspace_bytes(heads, head_dim, batch * num_split) > (int64_t)BT_NOALLOC_SCRATCH_BYTES)
    return BT_ENOSPC;
  void* ws = nullptr;
  rc = scratch_address(&ws);
  if (rc) return rc;
  // Every split writes its lse (-inf when it has no tokens) before the combine
  // reads it, and the combine reads only the partials of splits with tokens,
  // so nothing left in the scratch by an earlier call is ever used.
  return bt_gqa_decode(q, q_dtype, q_stride_seq, k, v, kv_stride_tok, kv_stride_head, seq_offset, pos,
                       seq_len, seqlen, batch, heads, kv_heads, head_dim, num_split, scale, ws,
                       (int64_t)BT_NOALLOC_SCRATCH_BYTES, out, out_dtype, out_stride_seq, stream);
}

int32_t bt_ragged_plan(const int32_t* lens, int32_t batch, int32_t target_groups, int32_t* work,
                       int32_t work_capacity, int32_t* split_base, int32_t* split_count,
                       int32_t* total_splits) {
  if (!lens || !work || !split_base || !split_count || !total_splits) return BT_EINVAL;
  if (batch < 1 || target_groups < 1) return BT_EINVAL;
  int32_t max_len = 1;
  for (int32_t b = 0; b < batch; ++b) {
    if (lens[b] < 0) return BT_EINVAL;
    max_len = std::max(max_len, lens[b]);
  }
  // Splits of sequence b under a cap of T tokens per split: ceil(len / T),
  // at least 1, at most one per 32 tokens and kMaxSplitsPerSeq.
  auto splits_of = [](int32_t len, int32_t cap) {
    int64_t ns = ((int64_t)len + cap - 1) / cap;
    ns = std::min<int64_t>(ns, (len + 31) / 32);
    ns = std::min<int64_t>(ns, bt::kMaxSplitsPerSeq);
    return (int32_t)std::max<int64_t>(ns, 1);
  };
  auto count_at = [&](int32_t cap) {
    int64_t n = 0;
    for (int32_t b = 0; b < batch; ++b) n += splits_of(lens[b], cap);
    return n;
  };
  // The smallest cap whose split total fits target_groups (the count only
  // falls as the cap grows): every work-group then streams at most that many
  // tokens and the batch runs in one round of target_groups work-groups per kv
  // head.  A batch with more sequences than target_groups gets one split each.
  int32_t lo = 1, hi = max_len;
  while (lo < hi) {
    const int32_t mid = lo + (hi - lo) / 2;
    if (count_at(mid) <= target_groups) hi = mid;
    else lo = mid + 1;
  }
  const int32_t cap = lo;
  int32_t total = 0;
  for (int32_t b = 0; b < batch; ++b) {
    const int32_t ns = splits_of(lens[b], cap);
    if ((int64_t)total + ns > work_capacity) return BT_ENOSPC;
    split_base[b] = total;
    split_count[b] = ns;
    total += ns;
  }
  // Work entries, longest splits first (when the grid takes more than one
  // round, the long ones start early).
  std::vector<int32_t> order(batch);
  for (int32_t b = 0; b < batch; ++b) order[b] = b;
  std::stable_sort(order.begin(), order.end(), [&](int32_t a, int32_t c) {
    return (int64_t)lens[a] * split_count[c] > (int64_t)lens[c] * split_count[a];
  });
  int64_t i = 0;
  for (const int32_t b : order) {
    for (int32_t s = 0; s < split_count[b]; ++s, ++i) {
      int32_t* w = work + 4 * i;
      w[0] = b;
      w[1] = s;
      w[2] = split_count[b];
      w[3] = split_base[b];
    }
  }
  *total_splits = total;
  return total;
}

int bt_ragged_plan_device(const int32_t* seq_len, int32_t batch, int32_t target_groups, int32_t* work,
                          int32_t work_capacity, int32_t* split_base, int32_t* split_count,
                          int32_t* total_splits, void* stream) {
  if (!seq_len || !work || !split_base || !split_count) return BT_EINVAL;
  if (batch < 1 || target_groups < 1 || !aligned16(work)) return BT_EINVAL;
  if (batch > bt::kRaggedPlanMaxBatch) return BT_ENOTSUP;
  if (work_capacity < std::max(batch, target_groups)) return BT_ENOSPC;
  bt::RaggedPlanParams p{};
  p.seq_len = seq_len;
  p.batch = batch;
  p.target_groups = target_groups;
  p.work = work;
  p.work_capacity = work_capacity;
  p.split_base = split_base;
  p.split_count = split_count;
  p.total = total_splits;
  return hip_rc(bt::launch_ragged_plan(p, (hipStream_t)stream));
}

int bt_gqa_decode_ragged(const void* q, int32_t q_dtype, int64_t q_stride_seq, const void* k,
                         const void* v, int64_t kv_stride_tok, int64_t kv_stride_head,
                         const int64_t* seq_offset, const int32_t* seq_len, int32_t batch,
                         int32_t heads, int32_t kv_heads, int32_t head_dim, const int32_t* work,
                         int32_t num_work, const int32_t* split_base, const int32_t* split_count,
                         int32_t total_splits, float scale, void* workspace,
                         int64_t workspace_bytes, void* out, int32_t out_dtype,
                         int64_t out_stride_seq, void* stream) {
  int rc = check_decode_common(q, q_dtype, q_stride_seq, k, v, kv_stride_tok, kv_stride_head,
                               batch, heads, kv_heads, head_dim);
  if (rc) return rc;
  rc = check_out(out, out_dtype, out_stride_seq, batch, heads, head_dim);
  if (rc) return rc;
  if (!seq_offset || !seq_len || !work || !split_base || !split_count) return BT_EINVAL;
  if (num_work < 1 || total_splits < num_work) return BT_EINVAL;
  if (!workspace || !aligned16(workspace)) return BT_EINVAL;
  if (workspace_bytes < bt_decode_workspace_bytes(heads, head_dim, total_splits)) return BT_ENOSPC;
  if (!aligned16(work)) return BT_EINVAL;
  float* lse = static_cast<float*>(workspace);
  float* part = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                         align256((int64_t)heads * total_splits * 4));
  bt::DecodeSplitParams p = make_split_params(q, q_dtype, q_stride_seq, k, v, kv_stride_tok,
                                              kv_stride_head, seq_offset, nullptr, seq_len, 0,
                                              heads, kv_heads, head_dim, scale, lse, part);
  p.work = reinterpret_cast<const int4*>(work);
  p.num_split = 0;
  p.total_splits = total_splits;
  rc = hip_rc(bt::launch_decode_split(p, head_dim, num_work, 1, (hipStream_t)stream));
  if (rc) return rc;
  return bt_gqa_decode_combine(lse, part, batch, heads, head_dim, 0, split_base, split_count,
                               total_splits, out, out_dtype, out_stride_seq, stream);
}

int64_t bt_prefill_workspace_bytes(int32_t kv_len, int32_t kv_heads, int32_t head_dim) {
  if (kv_len < 1 || kv_heads < 1 || head_dim < 1) return 0;
  return prefill_base_bytes(kv_len, kv_heads, head_dim);
}

int64_t bt_prefill_split_workspace_bytes(int32_t seqlen, int32_t q_offset, int32_t heads, int32_t kv_heads,
                                         int32_t head_dim) {
  if (seqlen < 1 || q_offset < 0 || heads < 1 || kv_heads < 1 || heads % kv_heads || head_dim < 1) return 0;
  if ((int64_t)q_offset + seqlen > INT32_MAX) return 0;
  const int64_t vt = prefill_base_bytes(q_offset + seqlen, kv_heads, head_dim);
  int64_t part_offset = 0;
  const bt::PrefillSplitPlan plan = prefill_plan(seqlen, q_offset, heads, kv_heads, head_dim, &part_offset);
  return plan.uses_partials() ? part_offset + (int64_t)plan.part_bytes : vt;
}

// Shared by bt_gqa_prefill and bt_gqa_prefill_cached: validates the call and
// launches the pre-pass and the attention kernel.  `images` holds the K / V^T
// images and their exponents laid out for img_keys keys (prefill_layout); the
// pre-pass converts the blocks from key img_first_key on.  `partials` (may be
// null) holds the split-key partials when it is large enough.
static int prefill_run(const void* q, int32_t q_dtype, const void* k, const void* v, int64_t q_stride_tok,
                       int64_t q_stride_head, int64_t kv_stride_tok, int64_t kv_stride_head, int32_t seqlen,
                       int32_t q_offset, int32_t heads, int32_t kv_heads, int32_t head_dim, float scale,
                       void* images, int32_t img_keys, int32_t img_first_key, bool keep_images,
                       void* partials, int64_t partials_bytes, void* out, int32_t out_dtype,
                       int64_t out_stride_tok, int64_t out_stride_head, void* stream) {
  if (!q || !k || !v || !out || !images) return BT_EINVAL;
  if (seqlen < 1 || q_offset < 0 || heads < 1 || kv_heads < 1 || heads % kv_heads) return BT_EINVAL;
  if ((int64_t)q_offset + seqlen > INT32_MAX) return BT_EINVAL;
  if (out_dtype != BT_DTYPE_F32 && out_dtype != BT_DTYPE_BF16) return BT_EINVAL;
  if (q_dtype != BT_DTYPE_F32 && q_dtype != BT_DTYPE_BF16) return BT_EINVAL;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out)) return BT_EINVAL;
  if (q_stride_tok <= 0 || q_stride_head <= 0 || kv_stride_tok <= 0 || kv_stride_head < 0 ||
      out_stride_tok <= 0 || out_stride_head <= 0)
    return BT_EINVAL;
  if (q_stride_tok % 8 || q_stride_head % 8 || kv_stride_tok % 8 || kv_stride_head % 8 ||
      out_stride_tok % 8 || out_stride_head % 8)
    return BT_EINVAL;
  if (!aligned16(images) || (partials && !aligned16(partials))) return BT_EINVAL;
  if (head_dim != 256 && head_dim != 128) return BT_ENOTSUP;
  if (heads / kv_heads > 8) return BT_ENOTSUP;
  // 32-bit buffer offsets: the K rows of one kv head (plus the last block's
  // tail) and its images
  const int32_t kv_len = q_offset + seqlen;
  if (img_keys < kv_len || img_first_key < 0 || img_first_key > q_offset) return BT_EINVAL;
  const int64_t nblk = ((int64_t)kv_len + bt::kPrefillKeyBlock - 1) / bt::kPrefillKeyBlock;
  const int64_t img_blocks = ((int64_t)img_keys + bt::kPrefillKeyBlock - 1) / bt::kPrefillKeyBlock;
  if ((nblk + 1) * bt::kPrefillKeyBlock * kv_stride_tok * 2 > (int64_t)UINT32_MAX ||
      img_blocks * bt::kPrefillKeyBlock * head_dim * 2 > (int64_t)UINT32_MAX)
    return BT_ENOTSUP;
  bt::PrefillParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.q_stride_tok = q_stride_tok;
  p.q_stride_head = q_stride_head;
  p.kv_stride_tok = kv_stride_tok;
  p.kv_stride_head = kv_stride_head;
  p.seqlen = seqlen;
  p.q_offset = q_offset;
  p.heads = heads;
  p.kv_heads = kv_heads;
  p.group = heads / kv_heads;
  p.scale_log2 = (float)((double)scale * kLog2e);
  p.out = out;
  p.out_bf16 = out_dtype == BT_DTYPE_BF16;
  p.out_stride_tok = out_stride_tok;
  p.out_stride_head = out_stride_head;
  const PrefillLayout lay = prefill_layout(img_keys, kv_heads, head_dim);
  p.vt = static_cast<uint16_t*>(images);
  p.vexp = reinterpret_cast<int32_t*>(static_cast<char*>(images) + lay.vexp);
  p.kimg = reinterpret_cast<uint16_t*>(static_cast<char*>(images) + lay.kimg);
  p.kexp = reinterpret_cast<int32_t*>(static_cast<char*>(images) + lay.kexp);
  p.img_blocks = (int32_t)img_blocks;
  p.img_first = img_first_key / bt::kPrefillKeyBlock;
  p.q_f32 = q_dtype == BT_DTYPE_F32 ? 1 : 0;
  p.keep_images = keep_images ? 1 : 0;
  if (prefill_uses_pair(seqlen, heads, kv_heads, head_dim))
    return hip_rc(bt::launch_prefill_pair(p, head_dim, (hipStream_t)stream));
  // Every other shape runs two waves per SIMD (groups of 3, 5, 6, 7 as
  // subsets of 1 or 2 heads).  When one work-group per query block would
  // leave CUs idle or the causal triangle's work is uneven, and `partials`
  // holds the plan's partials (if it needs any), the key ranges are split.
  if (bt::prefill8_serves(p.group, head_dim)) {
    p.sub_group = bt::prefill8_sub_group(p.group);
    p.head_subs = p.group / p.sub_group;
    int64_t part_offset = 0;
    const bt::PrefillSplitPlan plan = prefill_plan(seqlen, q_offset, heads, kv_heads, head_dim, &part_offset);
    if (plan.active() && (!plan.uses_partials() || (partials && partials_bytes >= (int64_t)plan.part_bytes))) {
      p.kb_chunk = plan.kb_chunk;
      p.split_compact = plan.compact;
      p.pair_parts = plan.pair_parts;
      p.max_chunks = plan.max_chunks;
      if (plan.uses_partials()) {
        p.part = static_cast<float*>(partials);
        p.lse = p.part + plan.part_rows * (size_t)head_dim;
      }
    }
    return hip_rc(bt::launch_prefill8(p, head_dim, (hipStream_t)stream));
  }
  return BT_ENOTSUP;
}

int bt_gqa_prefill(const void* q, int32_t q_dtype, const void* k, const void* v, int64_t q_stride_tok,
                   int64_t q_stride_head, int64_t kv_stride_tok, int64_t kv_stride_head,
                   int32_t seqlen, int32_t q_offset, int32_t heads, int32_t kv_heads,
                   int32_t head_dim, float scale, void* workspace, int64_t workspace_bytes,
                   void* out, int32_t out_dtype, int64_t out_stride_tok, int64_t out_stride_head,
                   void* stream) {
  if (!workspace) return BT_EINVAL;
  if (seqlen < 1 || q_offset < 0 || heads < 1 || kv_heads < 1 || heads % kv_heads) return BT_EINVAL;
  if ((int64_t)q_offset + seqlen > INT32_MAX) return BT_EINVAL;
  const int32_t kv_len = q_offset + seqlen;
  if (workspace_bytes < bt_prefill_workspace_bytes(kv_len, kv_heads, head_dim)) return BT_ENOSPC;
  // the split-key partials follow the images (256-byte aligned)
  const int64_t part_offset = align256(prefill_base_bytes(kv_len, kv_heads, head_dim));
  void* partials = workspace_bytes > part_offset ? static_cast<char*>(workspace) + part_offset : nullptr;
  return prefill_run(q, q_dtype, k, v, q_stride_tok, q_stride_head, kv_stride_tok, kv_stride_head, seqlen,
                     q_offset, heads, kv_heads, head_dim, scale, workspace, kv_len, 0, false, partials,
                     partials ? workspace_bytes - part_offset : 0, out, out_dtype, out_stride_tok,
                     out_stride_head, stream);
}

int64_t bt_prefill_partials_bytes(int32_t seqlen, int32_t q_offset, int32_t heads, int32_t kv_heads,
                                  int32_t head_dim) {
  if (seqlen < 1 || q_offset < 0 || heads < 1 || kv_heads < 1 || heads % kv_heads || head_dim < 1) return 0;
  if ((int64_t)q_offset + seqlen > INT32_MAX) return 0;
  int64_t part_offset = 0;
  const bt::PrefillSplitPlan plan = prefill_plan(seqlen, q_offset, heads, kv_heads, head_dim, &part_offset);
  return plan.uses_partials() ? (int64_t)plan.part_bytes : 0;
}

int bt_gqa_prefill_cached(const void* q, int32_t q_dtype, const void* k, const void* v, int64_t q_stride_tok,
                          int64_t q_stride_head, int64_t kv_stride_tok, int64_t kv_stride_head, int32_t seqlen,
                          int32_t q_offset, int32_t heads, int32_t kv_heads, int32_t head_dim, float scale,
                          void* images, int64_t images_bytes, int32_t capacity, int32_t cached_keys,
                          void* partials, int64_t partials_bytes, void* out, int32_t out_dtype,
                          int64_t out_stride_tok, int64_t out_stride_head, void* stream) {
  if (capacity < 1 || (int64_t)q_offset + seqlen > capacity) return BT_EINVAL;
  if (cached_keys < 0 || cached_keys > q_offset) return BT_EINVAL;
  if (images_bytes < bt_prefill_workspace_bytes(capacity, kv_heads, head_dim)) return BT_ENOSPC;
  return prefill_run(q, q_dtype, k, v, q_stride_tok, q_stride_head, kv_stride_tok, kv_stride_head, seqlen,
                     q_offset, heads, kv_heads, head_dim, scale, images, capacity, cached_keys, true,
                     partials, partials_bytes, out, out_dtype, out_stride_tok, out_stride_head, stream);
}

static bool prep_dim_served(int32_t d) { return d == 64 || d == 128 || d == 256 || d == 512; }

int bt_rms_norm_rope(const float* x, int64_t x_stride, int32_t rows, int32_t dim, const float* w,
                     float eps, const float* cos, const float* sin, const int32_t* pos,
                     int32_t rope_dim, int32_t rope_cap, float* out, int64_t out_stride,
                     void* stream) {
  if (!x || !out || rows < 1 || dim < 1 || x_stride < dim || out_stride < dim) return BT_EINVAL;
  if ((cos == nullptr) != (sin == nullptr)) return BT_EINVAL;
  if (cos && (!pos || rope_dim < 2 || rope_dim % 2 || rope_dim > dim || rope_cap < 1)) return BT_EINVAL;
  if (!w && !cos) return BT_EINVAL;
  if (!(eps >= 0.f)) return BT_EINVAL;
  if (!prep_dim_served(dim)) return BT_ENOTSUP;
  bt::RowPrepParams p{};
  p.x = x;
  p.x_stride = x_stride;
  p.rows = rows;
  p.out = out;
  p.out_stride = out_stride;
  p.w = w;
  p.eps = eps;
  p.cos = cos;
  p.sin = sin;
  p.pos = pos;
  p.rope_dim = cos ? rope_dim : 0;
  p.rope_cap = rope_cap;
  return hip_rc(bt::launch_row_norm_rope(p, dim, (hipStream_t)stream));
}

int bt_attn_prep(const float* qkv, int32_t heads, int32_t kv_heads, int32_t head_dim,
                 const float* q_norm, const float* k_norm, float eps, const float* cos,
                 const float* sin, const int32_t* pos, int32_t rope_dim, int32_t rope_cap,
                 void* q_out, int32_t q_dtype, void* cache_k, void* cache_v, int64_t kv_stride_tok,
                 int64_t kv_stride_head, int32_t cache_cap, void* stream) {
  if (!qkv || !pos || !q_out || !cache_k || !cache_v) return BT_EINVAL;
  if (heads < 1 || kv_heads < 1 || head_dim < 1 || cache_cap < 1) return BT_EINVAL;
  if ((q_norm == nullptr) != (k_norm == nullptr)) return BT_EINVAL;
  if ((cos == nullptr) != (sin == nullptr)) return BT_EINVAL;
  if (cos && (rope_dim < 2 || rope_dim % 2 || rope_dim > head_dim || rope_cap < 1)) return BT_EINVAL;
  if (q_dtype != BT_DTYPE_F32 && q_dtype != BT_DTYPE_BF16) return BT_EINVAL;
  if (kv_stride_tok < 1 || kv_stride_head < 1) return BT_EINVAL;
  if (!(eps >= 0.f)) return BT_EINVAL;
  if (!prep_dim_served(head_dim)) return BT_ENOTSUP;
  bt::RowPrepParams p{};
  p.x = qkv;
  p.w = q_norm;
  p.wk = k_norm;
  p.eps = eps;
  p.cos = cos;
  p.sin = sin;
  p.pos = pos;
  p.rope_dim = cos ? rope_dim : 0;
  p.rope_cap = rope_cap;
  p.heads = heads;
  p.kv_heads = kv_heads;
  p.q_out = q_out;
  p.q_out_bf16 = q_dtype == BT_DTYPE_BF16;
  p.cache_k = static_cast<uint16_t*>(cache_k);
  p.cache_v = static_cast<uint16_t*>(cache_v);
  p.kv_stride_tok = kv_stride_tok;
  p.kv_stride_head = kv_stride_head;
  p.cache_cap = cache_cap;
  return hip_rc(bt::launch_attn_prep(p, head_dim, (hipStream_t)stream));
}

int bt_gdn_decode(const float* q, const float* k, const float* v, const float* g, const float* beta,
                  float* state, int32_t heads_k, int32_t heads_v, int32_t dim, float scale, float eps,
                  float* out, void* stream) {
  if (!q || !k || !v || !g || !beta || !state || !out) return BT_EINVAL;
  if (heads_k < 1 || heads_v < 1 || heads_v % heads_k || dim < 1) return BT_EINVAL;
  if (!aligned16(v) || !aligned16(state) || !aligned16(out)) return BT_EINVAL;
  if (!(eps >= 0.f)) return BT_EINVAL;
  if (dim != 64 && dim != 128) return BT_ENOTSUP;
  bt::GdnParams p{};
  p.q = q;
  p.k = k;
  p.v = v;
  p.g = g;
  p.beta = beta;
  p.state = state;
  p.out = out;
  p.heads_k = heads_k;
  p.heads_v = heads_v;
  p.scale = scale;
  p.eps = eps;
  return hip_rc(bt::launch_gdn_decode(p, dim, (hipStream_t)stream));
}

int64_t bt_gemv_workspace_bytes(int32_t K, int32_t N) {
  if (K < 1 || N < 1) return 0;
  return (int64_t)bt::gemv_workspace_bytes(K, N);
}

int bt_gemv_bf16(const float* x, const void* w, int64_t ldw, int32_t K, int32_t N, float* y,
                 void* workspace, int64_t workspace_bytes, void* stream) {
  if (!x || !w || !y || K < 1 || N < 1 || ldw < N) return BT_EINVAL;
  if (N % 8 || ldw % 8 || !aligned16(w)) return BT_EINVAL;
  if ((int64_t)K * ldw * 2 > (int64_t)INT32_MAX) return BT_ENOTSUP;
  int vec, sk, tiles;
  bt::gemv_shape(K, N, &vec, &sk, &tiles);
  const int64_t need = (int64_t)bt::gemv_workspace_bytes(K, N);
  if (sk > 1 && (!workspace || !aligned16(workspace) || workspace_bytes < need)) return BT_ENOSPC;
  bt::GemvParams p{};
  p.x = x;
  p.w = static_cast<const uint16_t*>(w);
  p.ldw = ldw;
  p.K = K;
  p.N = N;
  p.splits = sk;
  p.partial = static_cast<float*>(workspace);
  p.y = y;
  return hip_rc(bt::launch_gemv(p, vec, (hipStream_t)stream));
}

}  // extern "C"
