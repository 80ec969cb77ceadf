// Shared device helpers for the gfx950 GQA attention kernels.
//
// Conventions used across the kernels:
//  * bf16 values travel as raw 16-bit patterns (uint16_t) in memory and are
//    only reinterpreted as __bf16 vectors when handed to an MFMA.  Whole
//    vectors are bit-cast; single bf16 lanes are never extracted from a
//    vector (hipcc 7.2 folds such extracts of ds_read_tr results wrongly).
//  * MFMA operand layouts (verified on gfx950):
//      v_mfma_f32_16x16x32_bf16: lane l holds A[l%16][(l/16)*8 + 0..7],
//        B[(l/16)*8 + 0..7][l%16]; C[(l/16)*4 + j][l%16] in acc[j].
//      v_mfma_f32_32x32x16_bf16: lane l holds A[l%32][(l/32)*8 + 0..7],
//        B[(l/32)*8 + 0..7][l%32]; C[(j/4)*8 + (l/32)*4 + j%4][l%32] in acc[j].
//  * ds_read_b64_tr_b16 (per 16-lane group): input lane i points at row i/4,
//    columns (i%4)*4 .. +3 of a 4x16 block of 16-bit values; output lane j
//    receives column j, rows 0..3.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bt {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define BT_LDS __attribute__((address_space(3)))

// DPP controls (GCN/CDNA encoding).
constexpr int DPP_ROW_MIRROR = 0x140;       // lane i <- lane 15-i within each row of 16
constexpr int DPP_ROW_HALF_MIRROR = 0x141;  // lane i <- lane 7-i within each half-row of 8

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// float -> bf16 bits, round to nearest even (inputs are finite or +-inf).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// Two floats -> two bf16 packed in one word (a in the low half), round to
// nearest even, by the hardware conversion (v_cvt_pk_bf16_f32): with f32
// denormals kept (the kernels' default float mode) the same bits as
// f32_to_bf16_bits for every finite or infinite input.
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_bits(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}

__device__ __forceinline__ uint32_t pack2(uint32_t lo16, uint32_t hi16) {
  return (lo16 & 0xffffu) | (hi16 << 16);
}

// Lane permutation for controls whose every source lane exists (the row
// mirrors): bound_ctrl then changes no value, and with it set the compiler
// folds the move into the VALU instruction that consumes it (v_add_f32_dpp).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, true));
}

__device__ __forceinline__ floatx4 mfma16(const bf16x8& a, const bf16x8& b, const floatx4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ floatx16 mfma32(const bf16x8& a, const bf16x8& b, const floatx16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 as_bf16x8(const u32x4& v) { return __builtin_bit_cast(bf16x8, v); }

// Two transposed 4x16 reads glued into one 8-element MFMA operand.
__device__ __forceinline__ bf16x8 lds_read_tr_pair(const BT_LDS uint16_t* p0, const BT_LDS uint16_t* p1) {
  bf16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((BT_LDS bf16x4*)p0);
  bf16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((BT_LDS bf16x4*)p1);
  u32x2 ua = __builtin_bit_cast(u32x2, a);
  u32x2 ub = __builtin_bit_cast(u32x2, b);
  u32x4 r = {ua[0], ua[1], ub[0], ub[1]};
  return as_bf16x8(r);
}

// max(a, b) that propagates NaN: one v_maximum_f32 on gfx950, with none of the
// operand canonicalisation fmaxf needs in IEEE mode (-inf stays the identity).
__device__ __forceinline__ float fmax_nc(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// Max / sum of x over lanes l and l ^ 32 with one v_permlane32_swap (gfx950):
// swapping the upper half of one copy with the lower half of another leaves
// {x[0..31], x[0..31]} and {x[32..63], x[32..63]}.
__device__ __forceinline__ float halves_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmax_nc(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// Max of x over lanes l and l ^ 16 with one v_permlane16_swap (gfx950): it
// swaps the odd 16-lane rows of one copy with the even rows of another.
__device__ __forceinline__ float rows16_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmax_nc(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// Sum of x over lanes l and l ^ 16 (v_permlane16_swap, as rows16_max).
__device__ __forceinline__ float rows16_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// fmaxf (NaN-ignoring) of x over lanes l and l ^ 16 / l ^ 32, without an LDS round trip.
__device__ __forceinline__ float rows16_fmaxf(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_fmaxf(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// op(x, x[l ^ MASK]) for one butterfly step of a commutative op on 32-bit
// lanes, without an LDS round trip: DPP for MASK 1 and 2 (quad permutes), 4
// (row shifts, the two halves of each pair of banks taking opposite
// directions) and 8 (a row rotation by 8), lane swaps for 16 and 32.  The op
// sees the lane's own value and its partner's, so the result equals op(x,
// __shfl_xor(x, MASK)) bit for bit.  Where one DPP move with every source lane
// present does the permute (MASK 1, 2, 8), bound_ctrl is set: it changes no
// value and lets the compiler fold the move into the op that consumes it.
template <int MASK>
__device__ __forceinline__ uint32_t xor_partner_bits(uint32_t x) {
  const int v = (int)x;
  if constexpr (MASK == 1) return (uint32_t)__builtin_amdgcn_mov_dpp(v, 0xB1, 0xf, 0xf, true);  // quad_perm 1,0,3,2
  if constexpr (MASK == 2) return (uint32_t)__builtin_amdgcn_mov_dpp(v, 0x4E, 0xf, 0xf, true);  // quad_perm 2,3,0,1
  if constexpr (MASK == 4) {  // banks 0, 2 read lane + 4 (row_shl:4), banks 1, 3 lane - 4 (row_shr:4)
    const int lo = __builtin_amdgcn_update_dpp(0, v, 0x104, 0xf, 0x5, false);
    return (uint32_t)__builtin_amdgcn_update_dpp(lo, v, 0x114, 0xf, 0xA, false);
  }
  // row_ror:8: lane l of a row of 16 reads lane (l + 8) mod 16 = l ^ 8.
  if constexpr (MASK == 8) return (uint32_t)__builtin_amdgcn_mov_dpp(v, 0x128, 0xf, 0xf, true);
  static_assert(MASK == 1 || MASK == 2 || MASK == 4 || MASK == 8, "xor_partner_bits: 1, 2, 4 or 8");
  return x;
}
template <int MASK, typename Op>
__device__ __forceinline__ uint32_t xor_op(uint32_t x, Op op) {
  if constexpr (MASK == 16 || MASK == 32) {
    const auto r = MASK == 16 ? __builtin_amdgcn_permlane16_swap(x, x, false, false)
                              : __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return op(r[0], r[1]);  // the lane's own value and its partner's
  } else {
    return op(x, xor_partner_bits<MASK>(x));
  }
}
struct OpFAdd {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return __float_as_uint(__uint_as_float(a) + __uint_as_float(b)); }
};
struct OpFMaxf {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b))); }
};
// NaN-propagating maximum (v_maximum_f32): unlike fmaxf it needs no operand
// canonicalisation, so a butterfly of it is one lane move and one max.
struct OpFMax {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return __float_as_uint(fmax_nc(__uint_as_float(a), __uint_as_float(b))); }
};
struct OpUMax {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a > b ? a : b; }
};
struct OpIAdd {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return (uint32_t)((int)a + (int)b); }
};
struct OpIMax {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return (int)a > (int)b ? a : b; }
};
template <int MASK>
__device__ __forceinline__ float xor_sum(float x) { return __uint_as_float(xor_op<MASK>(__float_as_uint(x), OpFAdd{})); }
template <int MASK>
__device__ __forceinline__ float xor_fmaxf(float x) { return __uint_as_float(xor_op<MASK>(__float_as_uint(x), OpFMaxf{})); }
template <int MASK>
__device__ __forceinline__ uint32_t xor_umax(uint32_t x) { return xor_op<MASK>(x, OpUMax{}); }
// Whole-wave butterflies, masks 32, 16, ..., 1 in that order (every lane gets the result).
template <typename Op>
__device__ __forceinline__ uint32_t wave_op_desc(uint32_t x, Op op) {
  x = xor_op<32>(x, op);
  x = xor_op<16>(x, op);
  x = xor_op<8>(x, op);
  x = xor_op<4>(x, op);
  x = xor_op<2>(x, op);
  return xor_op<1>(x, op);
}
__device__ __forceinline__ float wave_sum(float x) { return __uint_as_float(wave_op_desc(__float_as_uint(x), OpFAdd{})); }
__device__ __forceinline__ float wave_fmaxf(float x) { return __uint_as_float(wave_op_desc(__float_as_uint(x), OpFMaxf{})); }
__device__ __forceinline__ float wave_max(float x) { return __uint_as_float(wave_op_desc(__float_as_uint(x), OpFMax{})); }
__device__ __forceinline__ uint32_t wave_umax(uint32_t x) { return wave_op_desc(x, OpUMax{}); }
// Sum over the lane bits at and above log2(FROM), masks FROM, 2 FROM, ..., 32.
template <int FROM>
__device__ __forceinline__ float sum_from(float x) {
  if constexpr (FROM <= 1) x = xor_sum<1>(x);
  if constexpr (FROM <= 2) x = xor_sum<2>(x);
  if constexpr (FROM <= 4) x = xor_sum<4>(x);
  if constexpr (FROM <= 8) x = xor_sum<8>(x);
  if constexpr (FROM <= 16) x = xor_sum<16>(x);
  if constexpr (FROM <= 32) x = xor_sum<32>(x);
  return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// Scaled fp16 V^T images of the prefill kernels: 64-key block b of a kv head
// holds v * 2^-e_b with e_b = 4 * ceil((E - 14) / 4), E the binary exponent of
// the block's largest |v| (e_b in [-140, 116]), or kVExpZero for a block of
// zeros.
constexpr int kVExpZero = -1024;

// Exponent e of the units the O accumulator is kept in (O_true = O * 2^e)
// after a block with exponent eb: unchanged for a zero block and for a block
// within 4 of it (P then carries the block's factor 2^(eb - e) <= 2^4 exactly
// in fp16), else the block's own -- but at most 64 below the current one, so
// the f32 accumulator cannot overflow; a block more than 2^64 below the
// running scale enters with its P shifted down by the excess.
__device__ __forceinline__ int vexp_next(int e_run, int eb) {
  if (eb == kVExpZero) return e_run;
  if (e_run == kVExpZero) return eb;
  const int d = eb - e_run;
  if (d >= -4 && d <= 4) return e_run;
  return d < -64 ? e_run - 64 : eb;
}
// Scalar (constant-cache) read of a value an earlier kernel wrote.
__device__ __forceinline__ int sload(const int* p, int i) {
  return ((const __attribute__((address_space(4))) int*)(p))[i];
}
// Power-of-two factor of a block's P: P' = P * 2^shift enters P.V.
__device__ __forceinline__ int vexp_shift(int e_new, int eb) { return eb == kVExpZero ? 0 : eb - e_new; }

// Prefill queries enter Q.K^T as fp16 scaled by 2^-e per query row (f32 or
// bf16 q alike), e = E - 14 for the row's largest |q| (0 for a row of zeros).
__device__ __forceinline__ int absmax_exp(uint32_t bits) {
  if (bits == 0) return 0;
  const int ebits = (int)(bits >> 23);
  return (ebits == 0 ? 1 : ebits) - 127 - 14;
}
typedef _Float16 half2_c __attribute__((ext_vector_type(2)));
typedef float float2_c __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_f16x2_scaled(float a, float b, int e) {
  return __builtin_bit_cast(uint32_t,
                            __builtin_convertvector((float2_c){__builtin_ldexpf(a, -e), __builtin_ldexpf(b, -e)}, half2_c));
}
// Largest |x| of N chunks of 8 f32 values, as the f32 bits of |x| (which order like |x|).
template <int N>
__device__ __forceinline__ uint32_t absmax_bits(const float4 (&raw)[N][2]) {
  uint32_t mx = 0;
#pragma unroll
  for (int i = 0; i < N; ++i)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float4 v = raw[i][h];
      mx = max(mx, max(max(__float_as_uint(v.x) & 0x7fffffffu, __float_as_uint(v.y) & 0x7fffffffu),
                       max(__float_as_uint(v.z) & 0x7fffffffu, __float_as_uint(v.w) & 0x7fffffffu)));
    }
  return mx;
}
// Raw bf16 chunks in `out` become fp16 scaled by 2^-e, e from the row's
// largest |q| (`reduce` combines the maxima of the lanes that share the row).
template <int N, typename Reduce>
__device__ __forceinline__ int q_bf16_to_f16(u32x4 (&out)[N], Reduce reduce) {
  uint32_t mx = 0;
#pragma unroll
  for (int i = 0; i < N; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) mx = max(mx, max((out[i][j] << 16) & 0x7fffffffu, out[i][j] & 0x7fff0000u));
  const int e = absmax_exp(reduce(mx));
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const u32x4 w = out[i];
    out[i] = u32x4{pack_f16x2_scaled(__uint_as_float(w[0] << 16), __uint_as_float(w[0] & 0xffff0000u), e),
                   pack_f16x2_scaled(__uint_as_float(w[1] << 16), __uint_as_float(w[1] & 0xffff0000u), e),
                   pack_f16x2_scaled(__uint_as_float(w[2] << 16), __uint_as_float(w[2] & 0xffff0000u), e),
                   pack_f16x2_scaled(__uint_as_float(w[3] << 16), __uint_as_float(w[3] & 0xffff0000u), e)};
  }
  return e;
}
// One query row's N chunks of 8 values (chunk i at q + off + i * step
// elements, f32 or bf16) as fp16 MFMA operands scaled by 2^-e, e from the
// row's largest |q|.  Every load is issued before any is used, so the row
// costs one memory round trip; `reduce` combines the maxima (as f32 bits of
// |q|, which order like |q|) of the lanes that share the row.  Returns e.
template <int N, typename Reduce>
__device__ __forceinline__ int q_row_f16(const void* q, bool f32, int64_t off, int step, u32x4 (&out)[N],
                                         Reduce reduce) {
  if (f32) {
    const float* qf = reinterpret_cast<const float*>(q) + off;
    float4 raw[N][2];
#pragma unroll
    for (int i = 0; i < N; ++i) {
      raw[i][0] = *reinterpret_cast<const float4*>(qf + (int64_t)i * step);
      raw[i][1] = *reinterpret_cast<const float4*>(qf + (int64_t)i * step + 4);
    }
    const int e = absmax_exp(reduce(absmax_bits(raw)));
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const float4 a = raw[i][0], b = raw[i][1];
      out[i] = u32x4{pack_f16x2_scaled(a.x, a.y, e), pack_f16x2_scaled(a.z, a.w, e), pack_f16x2_scaled(b.x, b.y, e),
                     pack_f16x2_scaled(b.z, b.w, e)};
    }
    return e;
  }
  const uint16_t* qb = reinterpret_cast<const uint16_t*>(q) + off;
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = *reinterpret_cast<const u32x4*>(qb + (int64_t)i * step);
  return q_bf16_to_f16(out, reduce);
}

// f32 q split into two fp16 terms per element: hi = fp16(q * 2^-e) and lo =
// fp16(q * 2^-e - hi), so hi + lo carries ~22 significant bits and Q.K^T
// summed over both terms matches f32 q to ~2^-22 relative (hi alone keeps 11
// bits, and its score error grows with |q|.|k|: at a score standard
// deviation of 2 it already reaches the 2e-3 output gate).  q * 2^-e - hi is
// exact in f32.
__device__ __forceinline__ void split_f16x2(float a, float b, int e, uint32_t& hi, uint32_t& lo) {
  const float sa = __builtin_ldexpf(a, -e), sb = __builtin_ldexpf(b, -e);
  const half2_c h = __builtin_convertvector((float2_c){sa, sb}, half2_c);
  const float ha = (float)h[0], hb = (float)h[1];
  hi = __builtin_bit_cast(uint32_t, h);
  lo = __builtin_bit_cast(uint32_t, __builtin_convertvector((float2_c){sa - ha, sb - hb}, half2_c));
}
// One f32 query row's N chunks of 8 values as hi and lo fp16 operands, in the
// layout and with the scale of q_row_f16.  Returns e.
template <int N, typename Reduce>
__device__ __forceinline__ int q_row_f16_lo(const float* q, int64_t off, int step, u32x4 (&hi)[N], u32x4 (&lo)[N],
                                            Reduce reduce) {
  const float* qf = q + off;
  float4 raw[N][2];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    raw[i][0] = *reinterpret_cast<const float4*>(qf + (int64_t)i * step);
    raw[i][1] = *reinterpret_cast<const float4*>(qf + (int64_t)i * step + 4);
  }
  const int e = absmax_exp(reduce(absmax_bits(raw)));
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const float4 a = raw[i][0], b = raw[i][1];
    uint32_t h[4], l[4];
    split_f16x2(a.x, a.y, e, h[0], l[0]);
    split_f16x2(a.z, a.w, e, h[1], l[1]);
    split_f16x2(b.x, b.y, e, h[2], l[2]);
    split_f16x2(b.z, b.w, e, h[3], l[3]);
    hi[i] = u32x4{h[0], h[1], h[2], h[3]};
    lo[i] = u32x4{l[0], l[1], l[2], l[3]};
  }
  return e;
}

}  // namespace bt
