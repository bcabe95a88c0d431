// Operand helpers shared by the feature-split kernels of the two-pass
// backward (bwd_tp.hip) and the fp32-tensor forward (fwd_x3.hip): 16-bit
// MFMA operands, or for fp32 tensors bf16 hi/lo pairs whose products are
// hi*hi + hi*lo + lo*hi -- fp32's exponent range and a ~16-bit significand
// on the bf16 MFMA.
#pragma once
#include "device_common.h"
#include "params.h"

namespace mlpmk {
namespace tp {

// Operand modes: 16-bit tensors (fp16 or bf16, one MFMA per product) or
// fp32 tensors (bf16 hi/lo pairs, three bf16 MFMAs per product).
enum { EM_F16 = 0, EM_BF16 = 1, EM_F32 = 2 };

template <int EM>
constexpr bool kBf = EM != EM_F16;  // the MFMA takes bf16 payloads
template <int EM>
constexpr int kEs = EM == EM_F32 ? 4 : 2;  // bytes per tensor element

// One MFMA operand of a lane: 8 16-bit payloads; with fp32 tensors a pair
// (hi, lo).
struct Opnd {
  f16x8 h, l;
};

__device__ __forceinline__ float bf16_bits_to_f32(f16 v) {
  return __builtin_bit_cast(float, (uint32_t)__builtin_bit_cast(unsigned short, v) << 16);
}

// 8 fp32 values as an operand: rounded to the 16-bit format (RNE), or split
// into bf16 hi + lo.  A non-finite hi keeps lo = 0, so inf stays inf
// instead of becoming inf + NaN.
template <int EM>
__device__ __forceinline__ Opnd make_op(const float (&v)[8]) {
  Opnd o;
  o.h = pack8<kBf<EM>>(v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]);
  if constexpr (EM == EM_F32) {
    float r[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float hv = bf16_bits_to_f32(o.h[j]);
      r[j] = __builtin_fabsf(hv) < __builtin_huge_valf() ? v[j] - hv : 0.0f;
    }
    o.l = pack8<true>(r[0], r[1], r[2], r[3], r[4], r[5], r[6], r[7]);
  } else {
    o.l = f16x8{};
  }
  return o;
}

// bf16 hi + lo of 8 values that are >= 0, +inf or NaN (softplus outputs):
// hi = the upper half of each value's bits (truncation), lo = v - hi >= 0
// rounded to bf16.  The same ~16-bit significand as make_op at four VALU
// operations per value instead of five: max(v - hi, 0) turns the NaN of
// inf - inf into lo = 0 (maxNum), so inf stays inf.
__device__ __forceinline__ Opnd make_op_nonneg(const float (&v)[8]) {
  uint32_t hp[4];
  float r[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t bits = __builtin_bit_cast(uint32_t, v[j]);
    r[j] = __builtin_fmaxf(v[j] - __builtin_bit_cast(float, bits & 0xffff0000u), 0.0f);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j)
    hp[j] = (__builtin_bit_cast(uint32_t, v[2 * j + 1]) & 0xffff0000u) | (__builtin_bit_cast(uint32_t, v[2 * j]) >> 16);
  Opnd o;
  o.h = __builtin_bit_cast(f16x8, (i32x4){(int)hp[0], (int)hp[1], (int)hp[2], (int)hp[3]});
  o.l = pack8<true>(r[0], r[1], r[2], r[3], r[4], r[5], r[6], r[7]);
  return o;
}

template <int EM>
__device__ __forceinline__ f32x16 mma(const Opnd& a, const Opnd& b, f32x16 c) {
  if constexpr (EM == EM_F32) {
    c = mfma32x32x16<true>(a.l, b.h, c);
    c = mfma32x32x16<true>(a.h, b.l, c);
    return mfma32x32x16<true>(a.h, b.h, c);
  } else {
    return mfma32x32x16<EM == EM_BF16>(a.h, b.h, c);
  }
}

// 8 consecutive tensor elements at element offset `e` of resource r, as an
// operand (16-bit tensors: one 16-byte load; fp32: two, then the split).
template <int EM>
__device__ __forceinline__ Opnd load_op(rsrc_t r, uint32_t e) {
  if constexpr (EM == EM_F32) {
    const f32x4 a = buf_load16<f32x4>(r, e * 4), b = buf_load16<f32x4>(r, e * 4 + 16);
    const float v[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    return make_op<EM>(v);
  } else {
    Opnd o;
    o.h = buf_load16<f16x8>(r, e * 2);
    o.l = f16x8{};
    return o;
  }
}

// 8 fp32 values stored as tensor elements at element offset e.
template <int EM>
__device__ __forceinline__ void store8(rsrc_t r, uint32_t e, const float* v) {
  if constexpr (EM == EM_F32) {
    buf_store16((f32x4){v[0], v[1], v[2], v[3]}, r, e * 4);
    buf_store16((f32x4){v[4], v[5], v[6], v[7]}, r, e * 4 + 16);
  } else {
    buf_store16(pack8<kBf<EM>>(v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]), r, e * 2);
  }
}

// Widths: compile-time maxima N::d (exact for fixed networks); a Gen network
// reads the true widths, each at most N::d, from the launch parameters.
template <class N, class P>
__device__ __forceinline__ int dimw(const P& p, int l) {
  return N::gen ? p.dims[l] : N::d[l];
}

__device__ __forceinline__ uint32_t rows_at(int64_t M, int64_t r0, int n) {
  const int64_t left = M - r0;
  return (uint32_t)(left < n ? (left > 0 ? left : 0) : n);
}

// Exchange-tile slot of (row, 16-byte chunk): XOR-swizzled so that the 8
// rows of an 8-lane LDS access group hit 8 distinct chunks (distinct banks).
template <int CH>
__device__ __forceinline__ int slot(int row, int chunk) {
  return row * CH + (chunk ^ (row & (CH - 1)));
}

}  // namespace tp
}  // namespace mlpmk
