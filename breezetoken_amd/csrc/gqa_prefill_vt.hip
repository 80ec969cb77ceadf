// Pre-pass of the prefill kernels: K and V (kv_len, Hkv, D) bf16 -> scaled
// fp16 images, one power-of-two scale per 64-key block of each.
//
// V^T image, block b of kv head g: e = 4 * ceil((E - 14) / 4), E the binary
// exponent of the block's largest |v| (kVExpZero for a block of zeros).  The
// image holds v * 2^-e (round to nearest even), so the block's largest
// magnitude lies in [2^11, 2^15): no bf16 value overflows fp16, and values
// down to 2^-25 times the block's largest stay normal fp16 numbers (11
// significant bits).  e goes to vexp[g * nblk + b]; the attention kernels fold
// it into P (see vexp_next in bt_common.h).  Layout: block b of head g at vt +
// (g * nblk + b) * 64 * D as 8 key chunks; chunk c holds at row d the 8
// values V[b*64 + key][d] (16 bytes) of key = (c/4)*32 + (c%4)*4 + {0, 1, 2,
// 3, 16, 17, 18, 19}: the order in which lane group c%4 of a 16x16 MFMA
// result holds P of the 32-key half c/4.
// Grid z = 0 converts K, z = 1 V (two work-groups per block, so a CU holds
// one's loads in flight while the other converts and stores).  For V, one
// thread per (chunk, 8-column slice) transposes an 8 x 8 tile in registers; the block's image is assembled in LDS and stored linearly (1 KiB
// per wave instruction): 16-byte unit x sits in LDS slot x ^ ((x >> 3) & 7),
// conflict-free both ways.
//
// K image, block b of kv head g: e = E - 14 for the block's largest |k| (0 for
// a block of zeros), the image holds k * 2^-e in [2^14, 2^15) at most, and e
// goes to kexp[g * nblk + b]; the kernels multiply the scores of the block by
// 2^e (with q's own per-row scale) in the softmax's exp2 argument, which is
// exact.  Layout: row-major, block b of head g at kimg + (g * nblk + b) * 64 *
// D; the 16-byte slot s of row r holds the 8 values of chunk s ^ (r & 15)
// (columns 8 * (s ^ (r & 15)) ..), the XOR swizzle the kernels' K tiles use in
// LDS, so a tile copy is a plain contiguous copy.
//
// Keys past kv_len are zero in both images.  nblk is the layout's blocks per kv
// head (p.img_blocks: the blocks of kv_len keys for a per-call workspace, of
// the cache capacity for images kept across chunked-prefill calls); the
// pre-pass converts blocks p.img_first .. of kv_len keys and leaves the
// earlier ones, which a previous call on the same cache prefix wrote.
#include "bt_common.h"
#include "bt_kernels.h"

namespace bt {

namespace {

typedef _Float16 half2_v __attribute__((ext_vector_type(2)));
typedef float float2_v __attribute__((ext_vector_type(2)));

template <int D>
__global__ __launch_bounds__(256) void prefill_vts_kernel(PrefillParams p) {
  constexpr int kDC = D / 8;                 // 16-byte column chunks per row
  constexpr int kItems = 8 * kDC;            // (chunk, column chunk) items per block
  static_assert(kItems <= 256, "one item per thread");
  static_assert(kPrefillKeyBlock * kDC % 256 == 0, "whole K units per thread");
  constexpr int kBlk = kPrefillKeyBlock;
  // The kv heads of a block are neighbours in the grid's x (work-group x =
  // block * Hkv + head): both read the same token-major cache rows, one half
  // each, and dispatched together they do so at about the same time, which the
  // DRAM serves better (C4 S = 8192 about -3 us per call against one grid row
  // per head).
  const int blk = p.img_first + (int)blockIdx.x / p.kv_heads, g = (int)blockIdx.x % p.kv_heads;
  const int nblk = p.img_blocks;  // image layout stride per kv head
  const uint32_t row_bytes = (uint32_t)(p.kv_stride_tok * 2);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(p.v + (int64_t)g * p.kv_stride_head), (short)0,
      (int)((uint32_t)(p.q_offset + p.seqlen) * row_bytes), 0x00020000);
  uint16_t* img = p.vt + ((size_t)g * nblk + blk) * kBlk * D;
  constexpr int kUnits = kBlk * D * 2 / 16;
  __shared__ __attribute__((aligned(16))) u32x4 stage[kUnits];
  __shared__ uint32_t wmax[2][4];
  const int item = threadIdx.x;
  const int c = item / kDC, dc = item % kDC;
  if (blockIdx.z == 0) {
    // K: unit x = j * 256 + thread is slot x % kDC of row x / kDC; it holds
    // source chunk slot ^ (row & 15).
    constexpr int kKUnits = kBlk * kDC / 256;
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(p.k + (int64_t)g * p.kv_stride_head), (short)0,
        (int)((uint32_t)(p.q_offset + p.seqlen) * row_bytes), 0x00020000);
    u32x4 krow[kKUnits];
    uint32_t kmx = 0;  // largest |k| as bf16 bits
#pragma unroll
    for (int j = 0; j < kKUnits; ++j) {
      const int x = j * 256 + item;
      const int r = x / kDC, slot = x % kDC;
      krow[j] = __builtin_amdgcn_raw_buffer_load_b128(
          krs, (int)((uint32_t)(blk * kBlk + r) * row_bytes + (uint32_t)(slot ^ (r & 15)) * 16), 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) kmx = max(kmx, max(krow[j][i] & 0x7fffu, (krow[j][i] >> 16) & 0x7fffu));
    }
    kmx = wave_umax(kmx);
    if ((threadIdx.x & 63) == 0) wmax[1][threadIdx.x >> 6] = kmx;
    __syncthreads();
    kmx = max(max(wmax[1][0], wmax[1][1]), max(wmax[1][2], wmax[1][3]));
    int ek = 0;
    if (kmx != 0) {
      const int ebits = (int)(kmx >> 7);
      ek = (ebits == 0 ? 1 : ebits) - 127 - 14;
    }
    if (threadIdx.x == 0) p.kexp[g * nblk + blk] = ek;
    uint16_t* kimg = p.kimg + ((size_t)g * nblk + blk) * kBlk * D;
#pragma unroll
    for (int j = 0; j < kKUnits; ++j) {
      u32x4 o;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const float f0 = __uint_as_float(krow[j][m] << 16), f1 = __uint_as_float(krow[j][m] & 0xffff0000u);
        o[m] = __builtin_bit_cast(uint32_t, __builtin_convertvector(
                                                (float2_v){__builtin_ldexpf(f0, -ek), __builtin_ldexpf(f1, -ek)}, half2_v));
      }
      reinterpret_cast<u32x4*>(kimg)[j * 256 + item] = o;
    }
    return;
  }
  u32x4 rows[8];
  uint32_t mx = 0;  // largest |v| as bf16 bits (monotonic in |v|)
  if (item < kItems) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int key = blk * kBlk + (c >> 2) * 32 + (c & 3) * 4 + (j & 3) + (j >> 2) * 16;
      rows[j] = __builtin_amdgcn_raw_buffer_load_b128(vrs, (int)((uint32_t)key * row_bytes + (uint32_t)dc * 16), 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) mx = max(mx, max(rows[j][i] & 0x7fffu, (rows[j][i] >> 16) & 0x7fffu));
    }
  }
  mx = wave_umax(mx);
  if ((threadIdx.x & 63) == 0) wmax[0][threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = max(max(wmax[0][0], wmax[0][1]), max(wmax[0][2], wmax[0][3]));
  int e = kVExpZero;
  if (mx != 0) {
    const int ebits = (int)(mx >> 7);                 // biased exponent (0: subnormal)
    const int E = (ebits == 0 ? 1 : ebits) - 127;
    e = E <= 14 ? -4 * ((14 - E) / 4) : 4 * ((E - 14 + 3) / 4);  // 4 * ceil((E - 14) / 4)
  }
  if (threadIdx.x == 0) p.vexp[g * nblk + blk] = e;
  if (item < kItems) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {  // output row d = dc*8 + i
      u32x4 o;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const uint32_t w0 = rows[2 * m][i >> 1], w1 = rows[2 * m + 1][i >> 1];
        const float f0 = __uint_as_float((i & 1) ? (w0 & 0xffff0000u) : (w0 << 16));
        const float f1 = __uint_as_float((i & 1) ? (w1 & 0xffff0000u) : (w1 << 16));
        o[m] = __builtin_bit_cast(uint32_t, __builtin_convertvector(
                                                (float2_v){__builtin_ldexpf(f0, -e), __builtin_ldexpf(f1, -e)}, half2_v));
      }
      const int x = c * D + dc * 8 + i;
      stage[x ^ ((x >> 3) & 7)] = o;
    }
  }
  __syncthreads();
  u32x4* dst = reinterpret_cast<u32x4*>(img);
  for (int x = threadIdx.x; x < kUnits; x += 256) dst[x] = stage[x ^ ((x >> 3) & 7)];
}

}  // namespace

hipError_t launch_prefill_vts(const PrefillParams& p, int head_dim, hipStream_t stream) {
  const int nblk = (p.q_offset + p.seqlen + kPrefillKeyBlock - 1) / kPrefillKeyBlock;
  if (p.img_blocks < nblk || p.img_first < 0 || p.img_first > nblk) return hipErrorInvalidValue;
  if (p.img_first == nblk) return hipSuccess;  // every block is already in the images
  const dim3 grid((nblk - p.img_first) * p.kv_heads, 1, 2);
  switch (head_dim) {
    case 128: hipLaunchKernelGGL((prefill_vts_kernel<128>), grid, dim3(256), 0, stream, p); break;
    case 256: hipLaunchKernelGGL((prefill_vts_kernel<256>), grid, dim3(256), 0, stream, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace bt
