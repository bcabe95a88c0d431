// Device-side building blocks shared by the gfx950 megakernels.
//
// Orientation used by every kernel ("transposed" chaining): a layer computes
// H^T = W^T . A^T with v_mfma_f32_32x32x16_f16, so the MFMA M dimension is the
// layer's output features, K its input features and N the batch (rows of x).
// With this orientation the fp32 C/D registers of one layer are, after the
// activation and an fp16 pack, exactly the B operand of the next layer: no LDS
// round trip and no cross-lane shuffle between layers.
//
// Lane layouts of v_mfma_f32_32x32x16_f16 (64 lanes, lane = 32*g + n):
//   A (32 x 16): lane holds row n, k-group g, 8 fp16 values (k = 8g + j)
//   B (16 x 32): lane holds column n, k-group g, 8 fp16 values (k = 8g + j)
//   D (32 x 32): lane holds column n, rows 8a + 4g + b in register 4a + b
// Only the A/B symmetry of the k assignment matters for correctness (the sum
// over k is order free); the D layout fixes which features a lane owns.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mlpmk {

typedef _Float16 f16;
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Raw buffer resource over [base, base + bytes).  Buffer loads past `bytes`
// return zero and buffer stores past it are dropped by the hardware range
// check, which is how every kernel handles ragged row tails without branches.
// 0x00020000 is the gfx9-family word 3 (32-bit data format, no swizzle).
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
// AUX is the buffer instruction's cache-policy field (bit 1 = "nt").
// Measured on MI355X with the forward's access pattern (each wave reads its
// rows as 32-byte segments of 32 rows per load, writes whole 1 KiB runs per
// store), 256 MiB in + 256 MiB out:
//   default loads + default stores   5.2 TB/s
//   default loads + nt stores        6.9 TB/s
//   nt loads      + nt stores        4.6 TB/s
// nt loads lose because a 128-byte line is consumed by four successive loads
// and must stay in the vector cache between them; nt stores stream the
// output past L2 without evicting the input lines still being read.
constexpr int kStreamStore = 2;
// The fp32 activation stash (two 16-byte pieces of each of 32 rows per
// instruction pair, 1 KiB per row for the 3-layer network) keeps the default
// policy so that L2 merges the pieces of a line: with nt the 3-layer training
// forward at M = 131072 took 87 us instead of 35 us.  Output rows wider than
// 64 bytes written the same way (no LDS staging tile) keep it too
// (kDirectOutStore in fwd_kernel.h).
constexpr int kStashStore = 0;
// Output rows of the training forward (the stash kernels) keep the default
// policy as well: the loss reads them right back, and with nt stores it read
// them from HBM instead of the 256 MB memory-side cache (torch's out.sum()
// after the 3-layer training forward at M = 131072: 17.3 -> 14.2 us, the
// weight-norm training step 0.129 -> 0.125 ms as one graph; the forward
// itself 34.2 vs 34.5 us).  Inference outputs stream past L2 (kStreamStore).
template <bool STASH>
constexpr int kOutStore = STASH ? kStashStore : kStreamStore;
template <class T, int AUX = 0>
__device__ __forceinline__ T buf_load16(rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, AUX));
}
template <int AUX = 0, class T>
__device__ __forceinline__ void buf_store16(T v, rsrc_t r, uint32_t byte_off) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, v), r, (int)byte_off, 0, AUX);
}

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.69314718055994531f;

constexpr int kMaxLayers = 8;

// Element format of the 16-bit tensors (x, W, out, dout, dx): fp16, or bf16
// when BF.  Kernels carry either as 16-bit payloads in f16 vectors and
// interpret them only in the helpers taking BF: the MFMA, the conversions
// from fp32 (RNE) and the overflow tracking of packed activations.
template <bool BF = false>
__device__ __forceinline__ f32x16 mfma32x32x16(f16x8 a, f16x8 b, f32x16 c) {
  if constexpr (BF)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
template <bool BF = false>
__device__ __forceinline__ float elem_to_f32(f16 v) {
  if constexpr (BF)
    return (float)__builtin_bit_cast(__bf16, v);
  else
    return (float)v;
}
template <bool BF = false>
__device__ __forceinline__ f16 f32_to_elem(float v) {
  if constexpr (BF)
    return __builtin_bit_cast(f16, (__bf16)v);
  else
    return (f16)v;
}

// Output-feature permutation of an MFMA row block.  Row i = 8a + 4g + b of
// block mb computes feature outfeat(mb, i).  With it, D registers 0..7 of lane
// (n, g) hold features 32mb + 8g + [0..7] and registers 8..15 hold
// 32mb + 16 + 8g + [0..7]: i.e. the 8 consecutive features that the B operand
// of K-step s = 2mb (resp. 2mb+1) wants at lane (n, g) under the k map
// k(s, g, j) = 16s + 8g + j.  Every layer uses that same k map, which is also
// the natural one for loading rows of x with one 16-byte load per K-step.
__host__ __device__ constexpr int outfeat(int mb, int i) {
  return 32 * mb + 16 * ((i >> 3) >> 1) + 8 * ((i >> 2) & 1) + 4 * ((i >> 3) & 1) + (i & 3);
}

// Softplus in base-2 units: sp2(u) = log2(1 + 2^u).  For u = z*log2(e):
// softplus(z) = ln2 * sp2(u) for every z.  Evaluated directly -- one v_exp_f32,
// one add, one v_log_f32 (hardware base-2 transcendentals) -- it is within a
// few fp32 ulp of the exact value wherever 2^u is finite: for u <= 0 the
// rounding of 1 + 2^u costs at most 2^-24 absolute, for u > 0 at most 2^-24
// relative, and for u >= 24 the result is u itself.  For u >= 128, 2^u
// overflows and the result is +inf instead of u; callers detect that with
// sp2_overflow and then substitute u, which is the reference's threshold
// branch (kernel.py:108: z for z > 20, where the two agree to fp32 rounding).
//
// Other evaluations of the same function were built and timed in this
// kernel (all correct, all slower at the power-limited clock, because the
// transcendental unit does not co-issue with other waves' VALU work):
// max(u, 0) + log2(1 + 2^-|u|) (2 transcendentals + 3 VALU), max(u, 0) +
// y P(y) with y = 2^-|u| and P a degree-5 fit of log2(1 + y)/y (1 + 8), and
// the same with 2^-|u| from a range-reduced degree-4 polynomial (0 + 15).
__device__ __forceinline__ float sp2(float u) { return __builtin_amdgcn_logf(1.0f + __builtin_amdgcn_exp2f(u)); }
// Replaces an overflowed sp2 by u (u >= 128); every other value is kept as is.
__device__ __forceinline__ float sp2_fix(float u, float s) { return u >= 128.0f ? u : s; }

// sigma(z) = 1 - exp(-h) from the post-activation h = softplus(z) >= 0 (the
// softplus derivative as the stash contract states it, mlp_fused.md:57-61),
// evaluated as -expm1(-h): 1 - 2^(-h log2 e) for h >= 1/32, where the
// cancellation costs ~2^-23 / sigma < 4e-6 relative at most, and the series
// h (1 - h/2 (1 - h/3 (1 - h/4))) below, whose truncation error is below
// h^5 / 120 (< 8e-9 relative at h = 1/32).  The plain 1 - exp(-h) has no
// correct digit left for saturated units (h < ~1e-7, z < ~-16).
__device__ __forceinline__ float sig_from_h(float h) {
  const float big = 1.0f - __builtin_amdgcn_exp2f(-h * kLog2e);
  const float small = h * (1.0f - 0.5f * h * (1.0f - (1.0f / 3.0f) * h * (1.0f - 0.25f * h)));
  return h < 0.03125f ? small : big;
}

template <bool BF = false>
__device__ __forceinline__ f16x2 cvt2(float a, float b) {
  if constexpr (BF) {
    f16x2 r = __builtin_bit_cast(f16x2, __builtin_convertvector((f32x2){a, b}, bf16x2));  // v_cvt_pk_bf16_f32
    // An empty statement that takes the packed pair as is: without it the
    // compiler re-derived some pairs read as fp16 (the overflow tracking)
    // from two single conversions and a repack, which spilled.  It emits no
    // instruction, and the compiler still spaces the conversion and the
    // MFMA that reads it as for fp16 (at least two instructions apart in
    // every kernel's generated code).
    asm("" : "+v"(r));
    return r;
  } else
    return __builtin_convertvector((f32x2){a, b}, f16x2);  // v_cvt_pk_f16_f32 (RNE)
}

// A staged weight: w * sc rounded to fp32, then to fp16 (RNE both times).  The
// opaque step keeps the compiler from fusing the multiply and the conversion
// into a single-rounding v_fma_mix in some staging paths and not in others:
// the two roundings differ by one fp16 ulp for a few weights, and every
// kernel (any launch shape, inference or training forward) must stage the
// same bits.
template <bool BF = false>
__device__ __forceinline__ f16 scaled_weight(f16 w, float sc) {
  float t = elem_to_f32<BF>(w) * sc;
  asm volatile("" : "+v"(t));
  return f32_to_elem<BF>(t);
}
template <bool BF = false>
__device__ __forceinline__ f16x8 pack8(float a0, float a1, float a2, float a3, float a4, float a5,
                                       float a6, float a7) {
  f16x2 p0 = cvt2<BF>(a0, a1), p1 = cvt2<BF>(a2, a3), p2 = cvt2<BF>(a4, a5), p3 = cvt2<BF>(a6, a7);
  f16x4 q0 = __builtin_shufflevector(p0, p1, 0, 1, 2, 3);
  f16x4 q1 = __builtin_shufflevector(p2, p3, 0, 1, 2, 3);
  return __builtin_shufflevector(q0, q1, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Running maximum of packed sp2 values; the maximum propagates NaN.
// CHAIN: max(max(m, a), b) folds into one v_pk_maximum3_f16 per two packed
// values (4 per call); the pairwise tree costs ~6 per call but leaves the
// scheduler more freedom, which the stash kernels need to stay spill-free.
// The same code tracks bf16 payloads: read as fp16, a non-negative bf16
// pattern orders like its value below 0x7C00 (finite positive fp16), every
// larger pattern reads as fp16 inf or NaN, which the maximum keeps, and a
// negative one (only -0 or a NaN can occur: sp2 >= 0) is a negative fp16 or
// a NaN.  Only the threshold in sp2_overflowed differs.
template <bool CHAIN>
__device__ __forceinline__ f16x2 sp2_track(f16x2 m, f16x8 lo, f16x8 hi) {
  if constexpr (CHAIN) {
    m = __builtin_elementwise_maximum(__builtin_elementwise_maximum(m, lo.s01), lo.s23);
    m = __builtin_elementwise_maximum(__builtin_elementwise_maximum(m, lo.s45), lo.s67);
    m = __builtin_elementwise_maximum(__builtin_elementwise_maximum(m, hi.s01), hi.s23);
    return __builtin_elementwise_maximum(__builtin_elementwise_maximum(m, hi.s45), hi.s67);
  } else {
    m = __builtin_elementwise_maximum(m, __builtin_elementwise_maximum(lo.s01, lo.s23));
    m = __builtin_elementwise_maximum(m, __builtin_elementwise_maximum(lo.s45, lo.s67));
    m = __builtin_elementwise_maximum(m, __builtin_elementwise_maximum(hi.s01, hi.s23));
    return __builtin_elementwise_maximum(m, __builtin_elementwise_maximum(hi.s45, hi.s67));
  }
}
// True on every lane of the wave when some lane's tracked maximum is not below
// 128.  A finite sp2 below 2^7 rounds to at most 128 in fp16, so this catches
// every overflow (+inf) -- and every NaN, which the exact path reproduces
// unchanged.
// bf16 payloads (BF): 128.0 is the pattern 0x4300, which reads as fp16 3.5;
// likewise a finite sp2 below 2^7 rounds to at most that pattern.
template <bool BF = false>
__device__ __forceinline__ bool sp2_overflowed(f16x2 m) {
  const f16 m1 = __builtin_elementwise_maximum(m.x, m.y);
  const f16 thr = BF ? __builtin_bit_cast(f16, (unsigned short)0x4300) : (f16)128.0f;
  return __builtin_amdgcn_ballot_w64(!(m1 < thr)) != 0;
}

// An opaque copy of a wave-uniform offset.  Weight fragments never change
// after staging, so without this the compiler would hoist every fragment read
// out of a persistent row loop (and spill); routing the LDS address through
// a volatile asm statement pins each block's reads inside the loop while
// leaving the scheduler free to interleave everything else.
__device__ __forceinline__ int opaque(int v) {
  asm volatile("; opaque %0" : "+v"(v));
  return v;
}

// Compile-time description of a network: widths d[0] (input) .. d[L] (output).
template <int... Ds>
struct Net {
  static constexpr bool gen = false;  // widths fixed at compile time
  static constexpr bool rc = false;   // backward: h_{L-1} read from the stash (see Recompute in bwd.hip)
  static constexpr bool bf = false;   // 16-bit tensors are fp16 (see BF16)
  static constexpr int L = sizeof...(Ds) - 1;
  static constexpr int d[sizeof...(Ds)] = {Ds...};
  // K-steps (16 input features each) and 32-row output blocks of layer l.
  static constexpr int ks(int l) { return d[l] / 16; }
  static constexpr int mbs(int l) { return (d[l + 1] + 31) / 32; }
  // First LDS fragment (1 KiB = 64 lanes x 16 B) of layer l.
  static constexpr int frag_off(int l) {
    int o = 0;
    for (int i = 0; i < l; ++i) o += mbs(i) * ks(i);
    return o;
  }
  static constexpr int nfrag() { return frag_off(L); }
  // Largest K-step count over all layer inputs (register buffer size).
  static constexpr int ksmax() {
    int m = 0;
    for (int i = 0; i < L; ++i) m = ks(i) > m ? ks(i) : m;
    return m;
  }
  static constexpr bool valid() {
    for (int i = 0; i <= L; ++i)
      if (d[i] <= 0 || d[i] % 16 != 0) return false;
    return L >= 2;
  }
  static constexpr int64_t weight_elems() {
    int64_t s = 0;
    for (int i = 0; i < L; ++i) s += (int64_t)d[i] * d[i + 1];
    return s;
  }
};

// A runtime-width network: the kernel is compiled for Base's widths (all 128)
// and reads the true widths, each at most Base's, from the launch parameters.
// Weights past the true widths stage as zeros, so a padded input feature
// never contributes; a padded hidden feature computes softplus(0) but meets
// zero weights in the next layer; padded output features are not stored.
template <class Base>
struct Gen : Base {
  static constexpr bool gen = true;
};

// The same network with bf16 tensors (x, W, out, dout, dx) and bf16 MFMA
// operands; accumulation, softplus and the stash stay fp32.
template <class Base>
struct BF16 : Base {
  static constexpr bool bf = true;
};
template <bool B, class N>
struct ElemNet {
  typedef N type;
};
template <class N>
struct ElemNet<true, N> {
  typedef BF16<N> type;
};

}  // namespace mlpmk
