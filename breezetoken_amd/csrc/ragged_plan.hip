// Ragged-batch split plan computed on the device from device lengths, so a
// multi-sequence decode step needs no host synchronisation and can be captured
// in a hipGraph.  It makes exactly the plan bt_ragged_plan makes on the host:
//  * ns_b = ceil(len_b / T), at least 1, at most ceil(len_b / 32) and
//    kMaxSplitsPerSeq, for the smallest token cap T whose total fits
//    target_groups (binary search over T; the total only falls as T grows);
//  * split_base[b] = sum of ns over sequences before b, split_count[b] = ns_b;
//  * work entries {b, s, ns_b, base_b}, sequences ordered by tokens per split,
//    largest first (ties by index, as a stable sort);
// and pads the work table to its capacity with entries {-1, 0, 0, 0}, which the
// split kernel skips.  One work-group of 1024 threads; batch <= 4096.
#include "bt_common.h"
#include "bt_kernels.h"

namespace bt {

namespace {

constexpr int kPlanThreads = 1024;

__device__ __forceinline__ int plan_splits(int len, int cap) {
  int64_t ns = ((int64_t)len + cap - 1) / cap;
  const int64_t fine = ((int64_t)len + 31) / 32;
  if (ns > fine) ns = fine;
  if (ns > kMaxSplitsPerSeq) ns = kMaxSplitsPerSeq;
  return ns < 1 ? 1 : (int)ns;
}

// Sum (or max) over the work-group; every thread gets the result.
template <bool MAX>
__device__ int block_reduce(int x, int* red) {
  x = MAX ? (int)wave_op_desc((uint32_t)x, OpIMax{}) : (int)wave_op_desc((uint32_t)x, OpIAdd{});
  const int wave = threadIdx.x >> 6;
  __syncthreads();  // red may still be read from the previous call
  if ((threadIdx.x & 63) == 0) red[wave] = x;
  __syncthreads();
  int r = red[0];
  for (int w = 1; w < kPlanThreads / 64; ++w) r = MAX ? (r > red[w] ? r : red[w]) : r + red[w];
  return r;
}

// Exclusive prefix sum of v[0 .. n) in place (n <= kRaggedPlanMaxBatch): each
// thread sums its run of consecutive items, the run sums are scanned across
// the work-group, then each run is rewritten.
__device__ void block_exclusive_scan(int* v, int n, int* runs) {
  constexpr int kRun = kRaggedPlanMaxBatch / kPlanThreads;
  const int t = threadIdx.x;
  int local = 0;
  for (int i = 0; i < kRun; ++i) {
    const int j = t * kRun + i;
    if (j < n) local += v[j];
  }
  runs[t] = local;
  __syncthreads();
  for (int off = 1; off < kPlanThreads; off <<= 1) {  // Hillis-Steele inclusive scan of the runs
    const int add = t >= off ? runs[t - off] : 0;
    __syncthreads();
    runs[t] += add;
    __syncthreads();
  }
  int acc = runs[t] - local;
  for (int i = 0; i < kRun; ++i) {
    const int j = t * kRun + i;
    if (j < n) {
      const int x = v[j];
      v[j] = acc;
      acc += x;
    }
  }
  __syncthreads();
}

__global__ __launch_bounds__(kPlanThreads) void ragged_plan_kernel(RaggedPlanParams p) {
  __shared__ int s_len[kRaggedPlanMaxBatch];
  __shared__ int s_ns[kRaggedPlanMaxBatch];
  __shared__ int s_base[kRaggedPlanMaxBatch];
  __shared__ int s_start[kRaggedPlanMaxBatch];  // indexed by rank, then scanned
  __shared__ int s_rank[kRaggedPlanMaxBatch];
  __shared__ int s_runs[kPlanThreads];
  __shared__ int s_red[kPlanThreads / 64];
  const int t = threadIdx.x;
  const int B = p.batch;

  int mx = 1;
  for (int b = t; b < B; b += kPlanThreads) {
    const int len = p.seq_len[b] > 0 ? p.seq_len[b] : 0;
    s_len[b] = len;
    mx = mx > len ? mx : len;
  }
  const int max_len = block_reduce<true>(mx, s_red);
  int lo = 1, hi = max_len;
  while (lo < hi) {  // uniform: every thread sees the same reductions
    const int mid = lo + (hi - lo) / 2;
    int part = 0;
    for (int b = t; b < B; b += kPlanThreads) part += plan_splits(s_len[b], mid);
    if (block_reduce<false>(part, s_red) <= p.target_groups) hi = mid;
    else lo = mid + 1;
  }
  const int cap = lo;
  for (int b = t; b < B; b += kPlanThreads) {
    const int ns = plan_splits(s_len[b], cap);
    s_ns[b] = ns;
    s_base[b] = ns;
  }
  __syncthreads();
  block_exclusive_scan(s_base, B, s_runs);
  // rank: sequences ahead of b in the order "more tokens per split first"
  // (len_c / ns_c > len_b / ns_b, cross-multiplied), ties by index.
  for (int b = t; b < B; b += kPlanThreads) {
    const int64_t lb = s_len[b], nb = s_ns[b];
    int r = 0;
    for (int c = 0; c < B; ++c) {
      const int64_t lhs = (int64_t)s_len[c] * nb, rhs = lb * (int64_t)s_ns[c];
      r += (lhs > rhs || (lhs == rhs && c < b)) ? 1 : 0;
    }
    s_rank[b] = r;
    s_start[r] = s_ns[b];
    p.split_base[b] = s_base[b];
    p.split_count[b] = s_ns[b];
  }
  __syncthreads();
  int part = 0;
  for (int b = t; b < B; b += kPlanThreads) part += s_ns[b];
  const int total = block_reduce<false>(part, s_red);
  block_exclusive_scan(s_start, B, s_runs);
  for (int b = t; b < B; b += kPlanThreads) {
    const int first = s_start[s_rank[b]];
    const int ns = s_ns[b], base = s_base[b];
    for (int s = 0; s < ns; ++s) {
      int* w = p.work + 4 * (first + s);
      *reinterpret_cast<int4*>(w) = int4{b, s, ns, base};
    }
  }
  for (int i = total + t; i < p.work_capacity; i += kPlanThreads)
    *reinterpret_cast<int4*>(p.work + 4 * i) = int4{-1, 0, 0, 0};
  if (t == 0 && p.total) *p.total = total;
}

}  // namespace

hipError_t launch_ragged_plan(const RaggedPlanParams& p, hipStream_t stream) {
  if (p.batch < 1 || p.batch > kRaggedPlanMaxBatch || p.target_groups < 1) return hipErrorInvalidValue;
  if (p.work_capacity < (p.batch > p.target_groups ? p.batch : p.target_groups)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(ragged_plan_kernel, dim3(1), dim3(kPlanThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace bt
