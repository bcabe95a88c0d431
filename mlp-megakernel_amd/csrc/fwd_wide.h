#pragma once
// Forward megakernel for hidden widths above 128 (up to 256) on gfx950.
//
// The reference's kernel takes any hidden width as constexpr tile loops
// (/root/reference/kernel.py:60-123, README.md:62,68) and lists larger H as
// the next step (mlp_fused.md:453-454).  At H = 256 the fp16 weights of a
// 3-layer network are 256 KiB, more than a workgroup's 160 KiB of LDS, so
// this kernel does not keep them resident: every workgroup streams them
// through a two-slot LDS ring once per round, and all its waves consume each
// chunk in lockstep.
//
//  * Round: 8 waves, each with its own block of 32 rows (256 rows).  The
//    round runs the whole layer chain for those rows; activations stay in
//    registers (two buffers of up to 16 K-steps, ping-pong between layers).
//  * Chunk: 128 output columns of one layer, all input rows: up to 256 x 128
//    fp16 = 64 KiB, copied raw from the row-major W_l [in, out] into an LDS
//    slot with buffer_load ... lds (16 bytes per lane, no registers), while
//    the waves compute on the other slot.  A barrier per chunk hands the
//    slots over.  A 3-layer 128-256-256-128 round streams 5 chunks (256
//    KiB), i.e. 1 KiB of weight traffic per row, served by L2.
//  * MFMA A fragments come straight from the raw rows with
//    ds_read_b64_tr_b16 (a 4 x 4 transpose of 16-bit elements on the way out
//    of LDS): lane (i, g) of fragment (mb, s) receives W_l[16s + 8g + j]
//    [outfeat(mb, i)], j = 0..7, the same operand the 128-wide kernels stage
//    pre-permuted.  The chunk rows are XOR-swizzled by whole 16-byte pieces
//    (piece p of row r at p ^ piece_swz(r)), which the loads apply by
//    choosing each lane's source piece.
//  * The weights are used as stored, so the activations stay in natural
//    units: u = z log2 e for the base-2 evaluation, h = ln 2 sp2(u).
//  * Softplus in the exact form everywhere (sp2 with u substituted past 2^u's
//    overflow, h rounded to the tensor format as the reference rounds its
//    hidden h, so hidden values up to fp16's 65,504 survive): a wave cannot
//    re-run a block on its own here, since the ring has moved on.
//    (Measured and not kept, at 1M rows: the 128-wide kernels' fast form
//    with a per-round exact re-run decided by a workgroup vote, and chunks
//    run as straight-line code with the MFMA chain of block mb + 1 issued
//    between block mb's softplus instructions: 0.3835 -> 0.371 ms together,
//    at 2.5x the compile time.  The kernel issues VALU or MFMA work in only
//    ~62 % of its cycles: its two waves per SIMD wait on the per-chunk
//    barrier and on each MFMA's transposed fragment reads.)
#include "device_common.h"
#include "host_common.h"
#include "params.h"

namespace mlpmk {

constexpr int kWideMax = 256;                // widest layer
constexpr int kWideKS = kWideMax / 16;       // K-steps of the widest activation
constexpr int kWideCols = 128;               // output columns per weight chunk
constexpr int kWideSlot = kWideMax * kWideCols;  // elements per ring slot (64 KiB)

// Piece (8-element) swizzle of chunk row r: the transposed reads of one
// fragment touch rows 16s + 8g + [0..7] at the same 32 columns; the XOR
// spreads those rows over distinct bank windows (the exchange-tile swizzle
// of the backward, in piece units).
__device__ __forceinline__ int piece_swz(int r) { return 2 * (r & 3) + ((r >> 2) & 1) + 8 * ((r >> 3) & 1); }

template <int L, int KS0, bool BF, bool STASH, int NW>
struct WideWave {
  const FwdParams& p;
  f16* ring;  // 2 slots of kWideSlot elements
  int lane, n, g, wid;
  int d[L + 1];
  int64_t row0;  // first of this wave's 32 rows in the current round
  // Transposed-read lane constants: rows rr[k] of a K-step and the column
  // within a 32-column block, already XORed with the row's swizzle.
  int rr[2], cx[2];
  f16x8 A[kWideKS], B[kWideKS];  // activations (B operands), ping-pong between layers

  __device__ __forceinline__ void init() {
    const int q = lane >> 4, i = lane & 15, c = i & 3;
    // Lane 4j + c of a 16-lane group q addresses row 8 (q >> 1) + j (+4 in
    // the second read) and 4 columns starting at 16 (q & 1) + 8 (c & 1) + 4 (c >> 1),
    // so that result lane 4a + c' receives column outfeat order
    // 16 (q & 1) + 8 (a & 1) + 4 (a >> 1) + c' of those rows.
    rr[0] = 8 * (q >> 1) + (i >> 2);
    rr[1] = rr[0] + 4;
    const int rcol = 16 * (q & 1) + 8 * (c & 1) + 4 * (c >> 1);
    cx[0] = rcol ^ (8 * piece_swz(rr[0]));
    cx[1] = rcol ^ (8 * piece_swz(rr[1]));
  }

  __device__ __forceinline__ uint32_t nrows() const {
    const int64_t left = p.M - row0;
    return (uint32_t)(left < 32 ? (left > 0 ? left : 0) : 32);
  }

  // K-steps a layer's chain runs: its input width padded to 128 (layer 0,
  // KS0 = 8) or 256.  Weight rows and x features past the true widths are
  // zero in the operands, so the padding adds nothing.
  template <int l>
  static constexpr int kks() { return l == 0 ? KS0 : kWideKS; }

  // Chunk (l, cc): W_l rows [0, 16 kks), columns [128 cc, 128 cc + 128), into
  // slot `slot`.  One buffer_load ... lds per wave and 4 rows (1 KiB): lane t
  // of instruction k writes bytes [16t, 16t + 16) of rows 4k .. 4k + 3, i.e.
  // row 4k + (t >> 4), slot piece t & 15, which holds source piece
  // (t & 15) ^ piece_swz(row).  Rows past W_l's height and pieces past its
  // width read as zeros (offsets past the resource; widths are multiples of
  // 8 except the last layer's output, whose partial piece only feeds
  // columns that are not stored).
  template <int l>
  __device__ __forceinline__ void load_chunk(int slot, int cc) const {
    const int K = d[l], N = d[l + 1];
    const rsrc_t wr = make_rsrc(p.w[l], (uint32_t)K * (uint32_t)N * 2u);
    f16* base = ring + slot * kWideSlot;
    if constexpr (l == L - 1) {
      // An odd output width leaves W_L's rows 2-byte aligned, which the
      // 16-byte loads to LDS do not take: assemble those pieces from 2-byte
      // loads instead (input and hidden widths are multiples of 16).
      if (N & 1) {
        // pieces t of rows 0 .. 16 kks - 1 (16 pieces per row): the slot only
        for (int t = threadIdx.x; t < 16 * kks<l>() * 16; t += NW * 64) {
          const int row = t >> 4, pslot = t & 15;
          const int col = kWideCols * cc + 8 * (pslot ^ piece_swz(row));
          f16x8 v;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const uint32_t off = col + j < N ? (uint32_t)(row * N + col + j) * 2u : 0xFFFFFFF0u;
            v[j] = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(wr, (int)off, 0, 0));
          }
          *reinterpret_cast<f16x8*>(base + row * kWideCols + 8 * pslot) = v;
        }
        return;
      }
    }
    const int r_in = lane >> 4, pc = lane & 15;
#pragma unroll
    for (int k0 = 0; k0 < 4 * kks<l>(); k0 += NW) {
      const int k = k0 + wid;
      const int row = 4 * k + r_in;
      const int col = kWideCols * cc + 8 * (pc ^ piece_swz(row));
      const uint32_t off = col < N ? (uint32_t)(row * N + col) * 2u : 0xFFFFFFF0u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          wr, (__attribute__((address_space(3))) void*)(base + k * 4 * kWideCols), 16, off, 0, 0, 0);
    }
  }

  // x rows of this wave's block as B operands (K-step s: row n, features
  // 16s + 8g + [0..7]); rows past M read zeros.
  __device__ __forceinline__ void load_x() {
    const int D = d[0];
    const rsrc_t xr = make_rsrc(p.x + row0 * D, nrows() * (uint32_t)D * 2u);
#pragma unroll
    for (int s = 0; s < KS0; ++s) {
      const uint32_t off = 16 * s < D ? (uint32_t)(n * D + 16 * s + 8 * g) * 2u : 0xFFFFFFF0u;  // past D: zeros
      A[s] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(xr, (int)off, 0, 0));
    }
  }

  // A fragment of local block mbl (32 columns) and K-step s from a slot.
  __device__ __forceinline__ f16x8 frag(const f16* slot_base, int mbl, int s) const {
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    s16x4 h[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const f16* a = slot_base + (16 * s + rr[k]) * kWideCols + ((32 * mbl) ^ cx[k]);
      h[k] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)const_cast<f16*>(a));
    }
    return __builtin_bit_cast(f16x8, __builtin_shufflevector(h[0], h[1], 0, 1, 2, 3, 4, 5, 6, 7));
  }

  // acc = W_l[:, block mb]^T . in over the layer's (padded) K-steps.
  template <int l>
  __device__ __forceinline__ f32x16 chain(const f16* slot_base, int mbl, const f16x8 (&in)[kWideKS]) const {
    f32x16 acc = {};
#pragma unroll
    for (int s = 0; s < kks<l>(); ++s) acc = mfma32x32x16<BF>(frag(slot_base, mbl, s), in[s], acc);
    return acc;
  }

  // Hidden layer l, block mb: softplus into out[2mb], out[2mb + 1]; the
  // fp32 stash if asked.  Natural units, as the reference keeps them:
  // u = acc log2 e, h = ln 2 * sp2(u) with u substituted where 2^u overflows
  // (softplus(z) = z there), handed on as h rounded to the tensor format --
  // the rounding the reference applies to its hidden h (kernel.py:110), so
  // hidden values up to fp16's 65,504 survive as they do there.
  template <int l, int mb>
  __device__ __forceinline__ void hidden(const f32x16& acc, f16x8 (&out)[kWideKS]) {
    float h[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float u = acc[e] * kLog2e;
      h[e] = kLn2 * sp2_fix(u, sp2(u));
    }
    out[2 * mb] = pack8<BF>(h[0], h[1], h[2], h[3], h[4], h[5], h[6], h[7]);
    if (2 * mb + 1 < kWideKS) out[2 * mb + 1] = pack8<BF>(h[8], h[9], h[10], h[11], h[12], h[13], h[14], h[15]);
    if constexpr (STASH) {
      const int HW = d[l + 1], c = 32 * mb + 8 * g;
      if (p.stash[l]) {
        const rsrc_t sr = make_rsrc(p.stash[l] + row0 * HW, nrows() * (uint32_t)HW * 4u);
        const uint32_t e4 = (uint32_t)(n * HW + c) * 4;
        if (c < HW) {
          buf_store16<kStashStore>((f32x4){h[0], h[1], h[2], h[3]}, sr, e4);
          buf_store16<kStashStore>((f32x4){h[4], h[5], h[6], h[7]}, sr, e4 + 16);
        }
        if (c + 16 < HW) {
          buf_store16<kStashStore>((f32x4){h[8], h[9], h[10], h[11]}, sr, e4 + 64);
          buf_store16<kStashStore>((f32x4){h[12], h[13], h[14], h[15]}, sr, e4 + 80);
        }
      }
    }
  }

  // Last layer, block mb: out rows (16-bit), features 32mb + 8g + [0..7] and
  // 32mb + 16 + 8g + [0..7].
  template <int mb>
  __device__ __forceinline__ void store_out(const f32x16& acc) const {
    const int OW = d[L], c = 32 * mb + 8 * g;
    const rsrc_t orr = make_rsrc(p.out + row0 * OW, nrows() * (uint32_t)OW * 2u);
    const uint32_t e = (uint32_t)(n * OW + c);
    const f32x16& v = acc;  // natural units
    constexpr int P = kStashStore;  // rows of up to 512 bytes, written a piece at a time: let L2 merge them
    if (OW % 8 == 0) {
      if (c < OW) buf_store16<P>(pack8<BF>(v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]), orr, e * 2);
      if (c + 16 < OW) buf_store16<P>(pack8<BF>(v[8], v[9], v[10], v[11], v[12], v[13], v[14], v[15]), orr, e * 2 + 32);
    } else {
      // Each element converted on its own (taken out of a packed vector, the
      // 2-byte store builtin was given element 0 every time).
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (c + j < OW)
          __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, f32_to_elem<BF>(v[j])), orr,
                                                (int)((e + j) * 2), 0, P);
        if (c + 16 + j < OW)
          __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, f32_to_elem<BF>(v[8 + j])), orr,
                                                (int)((e + 16 + j) * 2), 0, P);
      }
    }
  }
};

// The chunk sequence of a round: layer 0 chunks 0 .. nc(0)-1, then layer 1, ...
// `q` counts chunks since the kernel started (slot q & 1).  At a chunk's
// start its slot is filled; the chunk after it (in the round, or the first
// of the next round when `more`) is requested into the other slot, the
// waves compute, and a barrier both publishes the new slot and frees the old.
template <int L, int KS0, bool BF, bool STASH, int NW>
struct WideRound {
  using W = WideWave<L, KS0, BF, STASH, NW>;

  template <int l>
  static __device__ __forceinline__ int nchunks(const W& w) {
    return (w.d[l + 1] + kWideCols - 1) / kWideCols;
  }

  // Requests the chunk after (l, cc): (l, cc + 1), (l + 1, 0), or the next
  // round's (0, 0).
  template <int l>
  static __device__ __forceinline__ void request_next(const W& w, int slot, int cc, bool more) {
    if (cc + 1 < nchunks<l>(w)) {
      w.template load_chunk<l>(slot, cc + 1);
    } else if constexpr (l + 1 < L) {
      w.template load_chunk<l + 1>(slot, 0);
    } else {
      if (more) w.template load_chunk<0>(slot, 0);
    }
  }

  static __device__ __forceinline__ void sync() {
    // The buffer ... lds loads count in vmcnt; their LDS writes are visible
    // to the workgroup after the wait and the barrier.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }

  // Block mbl of chunk cc of layer l (global block mb = 4 cc + mbl).
  template <int l, int cc, int mbl>
  static __device__ __forceinline__ void block(W& w, const f16* sb) {
    if constexpr (mbl < kWideCols / 32) {
      constexpr int mb = 4 * cc + mbl;
      if (kWideCols * cc + 32 * mbl < w.d[l + 1]) {
        const f32x16 acc = w.template chain<l>(sb, mbl, (l % 2 == 0) ? w.A : w.B);
        finish<l, mb>(w, acc);
      } else if constexpr (l + 1 < L) {
        // Past the layer's width: zero operands for the next layer's padded K-steps.
        auto& out = (l % 2 == 0) ? w.B : w.A;
        out[2 * mb] = f16x8{};
        out[2 * mb + 1] = f16x8{};
      }
      block<l, cc, mbl + 1>(w, sb);
    }
  }

  // Softplus and hand-off (hidden layers) or output store (last layer) of
  // global block mb.
  template <int l, int mb>
  static __device__ __forceinline__ void finish(W& w, const f32x16& acc) {
    if constexpr (l + 1 < L)
      w.template hidden<l, mb>(acc, (l % 2 == 0) ? w.B : w.A);
    else
      w.template store_out<mb>(acc);
  }

  // Layer l of the round: its chunks in order.  A chunk past the layer's
  // width is not streamed; its blocks only zero their operands.
  template <int l, int cc = 0>
  static __device__ __forceinline__ void layer(W& w, int& q, bool more) {
    if constexpr (cc < kWideMax / kWideCols) {
      if (cc < nchunks<l>(w)) {
        const f16* sb = w.ring + (q & 1) * kWideSlot;
        request_next<l>(w, (q + 1) & 1, cc, more);
        block<l, cc, 0>(w, sb);
        sync();
        ++q;
      } else if constexpr (l + 1 < L) {
        auto& out = (l % 2 == 0) ? w.B : w.A;
#pragma unroll
        for (int s = 8 * cc; s < 8 * cc + 8; ++s) out[s] = f16x8{};
      }
      layer<l, cc + 1>(w, q, more);
    } else if constexpr (l + 1 < L) {
      layer<l + 1, 0>(w, q, more);
    }
  }
};

template <int L, int KS0, bool BF, bool STASH, int NW>
__global__ __launch_bounds__(NW * 64) void fwd_wide_kernel(FwdParams p) {
  constexpr int kRows = 32 * NW;  // rows per round
  __shared__ __attribute__((aligned(16))) f16 ring[2 * kWideSlot];
  WideWave<L, KS0, BF, STASH, NW> w{p, ring};
  w.lane = threadIdx.x & 63;
  w.n = w.lane & 31;
  w.g = w.lane >> 5;
  w.wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
  for (int i = 0; i <= L; ++i) w.d[i] = __builtin_amdgcn_readfirstlane(p.dims[i]);  // wave-uniform: SGPRs
  w.init();
  using Round = WideRound<L, KS0, BF, STASH, NW>;
  const int64_t nrounds = (p.M + kRows - 1) / kRows;
  int64_t rnd = blockIdx.x;
  if (rnd >= nrounds) return;  // whole workgroup: no barrier follows
  w.template load_chunk<0>(0, 0);
  Round::sync();
  int q = 0;
  for (; rnd < nrounds; rnd += gridDim.x) {
    // Opaque copies of the widths: everything derived from them (chunk
    // offsets, block tests) is then recomputed where it is used instead of
    // being hoisted out of the round loop, where it kept hundreds of
    // registers live (and spilled).
#pragma unroll
    for (int i = 0; i <= L; ++i) asm volatile("" : "+s"(w.d[i]));
    w.row0 = rnd * kRows + 32 * w.wid;
    w.load_x();
    Round::template layer<0>(w, q, rnd + gridDim.x < nrounds);
  }
}

template <int L, int KS0, bool BF, bool STASH, int NW>
static int launch_wide(const FwdParams& p, int cus, hipStream_t st, LaunchInfo* info) {
  const int64_t nrounds = (p.M + 32 * NW - 1) / (32 * NW);
  const int grid = (int)(nrounds < cus ? nrounds : cus);  // 128 KiB of LDS: one workgroup per CU
  if (info) {
    *info = LaunchInfo{MLPMK_KERNEL_PERSISTENT, 32, NW, grid, 1};
    return MLPMK_OK;
  }
  (void)hipGetLastError();
  hipLaunchKernelGGL((fwd_wide_kernel<L, KS0, BF, STASH, NW>), dim3(grid), dim3(NW * 64), 0, st, p);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MLPMK_OK : hip_fail(e, "wide fwd kernel launch");
}

// KS0: layer 0's K-steps, its input width padded to 128 or 256.
template <int KS0, bool BF, bool STASH, int NW>
static int wide_by_depth(int L, const FwdParams& p, int cus, hipStream_t st, LaunchInfo* info) {
  switch (L) {
    case 2: return launch_wide<2, KS0, BF, STASH, NW>(p, cus, st, info);
    case 3: return launch_wide<3, KS0, BF, STASH, NW>(p, cus, st, info);
    case 4: return launch_wide<4, KS0, BF, STASH, NW>(p, cus, st, info);
    default: return launch_wide<5, KS0, BF, STASH, NW>(p, cus, st, info);
  }
}
template <bool BF, bool STASH, int NW>
static int wide_by_input(int L, const int* dims, const FwdParams& p, int cus, hipStream_t st, LaunchInfo* info) {
  return dims[0] > 128 ? wide_by_depth<16, BF, STASH, NW>(L, p, cus, st, info)
                       : wide_by_depth<8, BF, STASH, NW>(L, p, cus, st, info);
}

// Every kernel of one workgroup size (NW waves, rounds of 32 NW rows).
template <int NW>
int wide_dispatch_nw(int L, const int* dims, const FwdParams& p, bool stash, bool bf, int cus, hipStream_t st,
                     LaunchInfo* info) {
  if (bf)
    return stash ? wide_by_input<true, true, NW>(L, dims, p, cus, st, info)
                 : wide_by_input<true, false, NW>(L, dims, p, cus, st, info);
  return stash ? wide_by_input<false, true, NW>(L, dims, p, cus, st, info)
               : wide_by_input<false, false, NW>(L, dims, p, cus, st, info);
}


}  // namespace mlpmk
