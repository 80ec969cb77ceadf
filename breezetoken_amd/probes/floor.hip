// Machine-floor probes for the decode measurement (not part of the attention
// library's ABI): what one graph node costs with no work in it, and how fast a
// plain kernel can stream the bytes a decode call reads.  bench.py --mode
// floor times them beside the decode kernels in the same process.
//
//  * floor_empty: one wave that does nothing.
//  * floor_read<LPT>: every thread issues LPT 16-byte non-temporal buffer
//    loads (the decode kernel's load form and cache policy) before it uses
//    any, folds them with xor and writes one word per work-group, so nothing
//    is dead code and the writes are negligible (one word per 64 KiB read at
//    LPT 16).  The grid covers the buffer exactly (n16 a multiple of 256 *
//    LPT, checked by the host).
//  * floor_read_lds: the same bytes through buffer_load ... lds (HBM -> LDS).
//  * floor_read_rows: 512 bytes of every 1 KiB token row, 16 rows x 64 bytes
//    per load instruction (the decode kernel's K access: one kv head of a
//    token-major cache with two kv heads).
//  * floor_tiny: one wave that reads the read kernel's first word and writes
//    one word: the dependent second node of a two-kernel call (split, then
//    combine).
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kPolicyStream = 2;  // gfx940+ cache-policy bits: nt

__global__ __launch_bounds__(64) void floor_empty() {}

template <int LPT>
__global__ __launch_bounds__(256) void floor_read(const void* src, uint32_t bytes_per_group, uint32_t* out) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(src), (short)0, (int)0x7fffffff, 0x00020000);
  const uint32_t base = (uint32_t)blockIdx.x * bytes_per_group;
  u32x4 v[LPT];
#pragma unroll
  for (int i = 0; i < LPT; ++i)
    v[i] = __builtin_amdgcn_raw_buffer_load_b128(r, (int)((i * 256 + threadIdx.x) * 16), (int)base, kPolicyStream);
  uint32_t x = 0;
#pragma unroll
  for (int i = 0; i < LPT; ++i) x ^= v[i][0] ^ v[i][1] ^ v[i][2] ^ v[i][3];
  // One word per work-group (lane 0 of wave 0 after a wave-level fold).
  for (int m = 32; m >= 1; m >>= 1) x ^= (uint32_t)__shfl_xor((int)x, m);
  if (threadIdx.x == 0) out[blockIdx.x] = x;
}

// The same bytes through buffer_load ... lds (HBM -> LDS, no registers): each
// wave copies its LPT KiB into its own LDS area, then one word of it is read.
template <int LPT>
__global__ __launch_bounds__(256) void floor_read_lds(const void* src, uint32_t bytes_per_group, uint32_t* out) {
  __shared__ __attribute__((aligned(1024))) unsigned char buf[4 * LPT * 1024];
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(src), (short)0, (int)0x7fffffff, 0x00020000);
  const uint32_t base = (uint32_t)blockIdx.x * bytes_per_group;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  unsigned char* dst = buf + wave * LPT * 1024;
#pragma unroll
  for (int i = 0; i < LPT; ++i)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(dst + i * 1024), 16,
                                             (int)((wave * LPT + i) * 1024 + lane * 16), (int)base, 0, kPolicyStream);
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
  if (lane == 0) out[blockIdx.x * 4 + wave] = *reinterpret_cast<const uint32_t*>(dst + 4);
}

// The decode kernel's K pattern: token rows of `row_bytes` (the cache's token
// stride), each 64-lane load covering 16 rows x 64 bytes (lanes t, t+16, t+32
// and t+48 take 16 bytes each of row t), LPT loads per thread stepping 64 bytes along the
// rows; a work-group covers 64 consecutive rows' first LPT * 64 bytes.
// MODE 0: the first half of each row only, 64 rows per work-group; 1: both
// halves, work-groups 2i and 2i+1 taking the two halves of the same 64 rows
// (the decode grid's kv heads of one split); 2: both halves of 32 rows in one
// work-group (waves 0-1 the first half, 2-3 the second).
template <int LPT, int MODE>
__global__ __launch_bounds__(256) void floor_read_rows(const void* src, uint32_t row_bytes, uint32_t* out) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(src), (short)0, (int)0x7fffffff, 0x00020000);
  const int wave = (int)(threadIdx.x >> 6), lane = threadIdx.x & 63;
  uint32_t row0, half;
  if constexpr (MODE == 0) { row0 = (uint32_t)blockIdx.x * 64 + wave * 16; half = 0; }
  else if constexpr (MODE == 1 || MODE >= 3) { row0 = (uint32_t)(blockIdx.x >> 1) * 64 + wave * 16; half = blockIdx.x & 1; }
  else { row0 = (uint32_t)blockIdx.x * 32 + (wave & 1) * 16; half = wave >> 1; }
  // MODE 3: each load covers two whole half-rows (lanes 0-31 row 2i, 32-63
  // row 2i+1, 16 bytes each), the way the decode kernel copies V.  MODE 4:
  // each load covers 256 contiguous bytes of four rows (lanes 16t..16t+15 row
  // t), loads 2j and 2j+1 the two quarters of rows 4j..4j+3.  MODE 5: as 4
  // with lane l on row l % 4 (16-byte chunk l / 4), the operand layout of the
  // 4x4x4 block MFMA.
  uint32_t voff;
  if constexpr (MODE == 3) voff = (row0 + (lane >> 5)) * row_bytes + half * (row_bytes / 2) + (lane & 31) * 16;
  else if constexpr (MODE == 4) voff = (row0 + (lane >> 4)) * row_bytes + half * (row_bytes / 2) + (lane & 15) * 16;
  else if constexpr (MODE == 5) voff = (row0 + (lane & 3)) * row_bytes + half * (row_bytes / 2) + (lane >> 2) * 16;
  else voff = (row0 + (lane & 15)) * row_bytes + half * (row_bytes / 2) + (lane >> 4) * 16;
  auto step = [&](int i) -> uint32_t {
    if constexpr (MODE == 3) return i * 2 * row_bytes;
    else if constexpr (MODE == 4 || MODE == 5) return (i >> 1) * 4 * row_bytes + (i & 1) * 256;
    else return i * 64;
  };
  u32x4 v[LPT];
#pragma unroll
  for (int i = 0; i < LPT; ++i) v[i] = __builtin_amdgcn_raw_buffer_load_b128(r, (int)(voff + step(i)), 0, kPolicyStream);
  uint32_t x = 0;
#pragma unroll
  for (int i = 0; i < LPT; ++i) x ^= v[i][0] ^ v[i][1] ^ v[i][2] ^ v[i][3];
  for (int m = 32; m >= 1; m >>= 1) x ^= (uint32_t)__shfl_xor((int)x, m);
  if (threadIdx.x == 0) out[blockIdx.x] = x;
}

__global__ __launch_bounds__(64) void floor_tiny(const uint32_t* in, uint32_t* out) {
  if (threadIdx.x == 0) out[0] = in[0] + 1u;
}

}  // namespace

extern "C" {

// Launches on `stream`; returns hipSuccess or the launch error.
int bt_floor_empty(void* stream) {
  hipLaunchKernelGGL(floor_empty, dim3(1), dim3(64), 0, (hipStream_t)stream);
  return (int)hipGetLastError();
}

// Reads `bytes` (a multiple of 256 * 16 * lpt, lpt in {4, 8, 16, 32}, at most
// 2 GiB) from `src`; `out` holds one word per work-group (bytes / (4096 lpt)).
int bt_floor_read(const void* src, int64_t bytes, int32_t lpt, uint32_t* out, void* stream) {
  const int64_t per_group = 256LL * 16 * lpt;
  if (!src || !out || bytes <= 0 || bytes % per_group || bytes > (1LL << 31)) return (int)hipErrorInvalidValue;
  const dim3 grid((unsigned)(bytes / per_group));
  switch (lpt) {
    case 4: hipLaunchKernelGGL(floor_read<4>, grid, dim3(256), 0, (hipStream_t)stream, src, (uint32_t)per_group, out); break;
    case 8: hipLaunchKernelGGL(floor_read<8>, grid, dim3(256), 0, (hipStream_t)stream, src, (uint32_t)per_group, out); break;
    case 16: hipLaunchKernelGGL(floor_read<16>, grid, dim3(256), 0, (hipStream_t)stream, src, (uint32_t)per_group, out); break;
    case 32: hipLaunchKernelGGL(floor_read<32>, grid, dim3(256), 0, (hipStream_t)stream, src, (uint32_t)per_group, out); break;
    default: return (int)hipErrorInvalidValue;
  }
  return (int)hipGetLastError();
}

// As bt_floor_read, through LDS (lpt 8; `out` holds 4 words per work-group).
int bt_floor_read_lds(const void* src, int64_t bytes, uint32_t* out, void* stream) {
  const int64_t per_group = 256LL * 16 * 8;
  if (!src || !out || bytes <= 0 || bytes % per_group || bytes > (1LL << 31)) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(floor_read_lds<8>, dim3((unsigned)(bytes / per_group)), dim3(256), 0, (hipStream_t)stream, src,
                     (uint32_t)per_group, out);
  return (int)hipGetLastError();
}

// Reads the first 512 bytes (lpt 8) of every row of `rows` rows spaced
// `row_bytes` apart (rows a multiple of 64, row_bytes >= 512 and a multiple of
// 16): one kv head's half of a token-major K cache when row_bytes is the token
// stride.  `out` holds one word per work-group (rows / 64).
// mode 1 / 2: both halves of every row of 1,024 bytes (row_bytes must be 1024),
// read by adjacent work-groups (1) or inside one work-group (2); mode 3: as 1,
// each load covering two whole half-rows; mode 4: as 1, each load covering 256
// contiguous bytes of four rows (lanes 16t..16t+15 on row t); mode 5: as 4,
// lane l on row l % 4.  `out` holds one word per work-group (rows /
// 64 for mode 0, rows / 32 otherwise).
int bt_floor_read_rows(const void* src, int64_t rows, int64_t row_bytes, int32_t mode, uint32_t* out, void* stream) {
  if (!src || !out || rows <= 0 || rows % 64 || row_bytes < 512 || row_bytes % 16 ||
      rows * row_bytes > (1LL << 31) || mode < 0 || mode > 5 || (mode > 0 && row_bytes != 1024))
    return (int)hipErrorInvalidValue;
  const hipStream_t st = (hipStream_t)stream;
  const uint32_t rb = (uint32_t)row_bytes;
  if (mode == 0) hipLaunchKernelGGL((floor_read_rows<8, 0>), dim3((unsigned)(rows / 64)), dim3(256), 0, st, src, rb, out);
  if (mode == 1) hipLaunchKernelGGL((floor_read_rows<8, 1>), dim3((unsigned)(rows / 32)), dim3(256), 0, st, src, rb, out);
  if (mode == 2) hipLaunchKernelGGL((floor_read_rows<8, 2>), dim3((unsigned)(rows / 32)), dim3(256), 0, st, src, rb, out);
  if (mode == 3) hipLaunchKernelGGL((floor_read_rows<8, 3>), dim3((unsigned)(rows / 32)), dim3(256), 0, st, src, rb, out);
  if (mode == 4) hipLaunchKernelGGL((floor_read_rows<8, 4>), dim3((unsigned)(rows / 32)), dim3(256), 0, st, src, rb, out);
  if (mode == 5) hipLaunchKernelGGL((floor_read_rows<8, 5>), dim3((unsigned)(rows / 32)), dim3(256), 0, st, src, rb, out);
  return (int)hipGetLastError();
}

int bt_floor_tiny(const uint32_t* in, uint32_t* out, void* stream) {
  if (!in || !out) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(floor_tiny, dim3(1), dim3(64), 0, (hipStream_t)stream, in, out);
  return (int)hipGetLastError();
}

}  // extern "C"
