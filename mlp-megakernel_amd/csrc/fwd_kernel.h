#pragma once
// Forward megakernel for gfx950 (MI355X): kernel templates and their launch
// templates for 16-bit (fp16 / bf16) tensors, dispatched by fwd.hip.
//
// Replaces the reference's Triton `_fused_mlp_recompute` (/root/reference/kernel.py:60-123)
// and its training-forward variant with stored activations
// (/root/reference/mlp_fused.md:52-61).  Same math, different machine mapping:
//
//  * Persistent grid: min(CUs x occupancy, work) workgroups of NW waves.  Each
//    wave walks blocks of 32*NB rows with a grid-wide stride.
//  * Every weight matrix is staged ONCE per workgroup into LDS, already permuted
//    into MFMA A-operand fragments (1 KiB each, 16 B per lane), so the hot loop
//    reads each fragment with one conflict-free ds_read_b128 and reuses it for
//    NB batch blocks.  (The reference reloads weight tiles from L2 for every
//    tile, kernel.py:105,109,113.)
//  * Each layer runs v_mfma_f32_32x32x16_f16 with fp32 accumulation; softplus is
//    applied to the accumulators in VGPRs and packed to fp16, which is directly
//    the next layer's B operand (see device_common.h).  No intermediate goes to
//    LDS or HBM unless the training stash is requested.
//  * x rows are read with 16-byte loads, out rows written with 16-byte stores.
//  * Activations run in base-2 units: W_1 is staged pre-scaled by log2(e) and
//    W_L by ln(2), hidden layers chain with no scaling at all (ln2 and log2e
//    cancel between W^T h' and the next exp2), so the epilogue is exp2, add,
//    log2 per element in fp32 and one pack per pair (see sp2); overflow is
//    detected one layer later by a class test of one accumulator per row
//    (networks of up to 3 layers) or by a running maximum of the packed
//    activations (deeper ones).  The stash stores natural-unit h = ln2 * h'
//    in fp32.
//  * Each layer is software-pipelined by 32-feature output block: the MFMA
//    chain of block mb+1 is issued ahead of block mb's activation, so the
//    matrix core and the VALU work concurrently within one wave.

#include "device_common.h"
#include "params.h"

#ifndef MLPMK_SCHED_FENCE
#define MLPMK_SCHED_FENCE() __builtin_amdgcn_sched_barrier(0)
#endif

namespace mlpmk {

// Stage all layers' A fragments into LDS.  Fragment (mb, s) of layer l, lane
// (i, g) holds W_l[16s + 8g + j][outfeat(mb, i)], j = 0..7 (zero past the
// layer's output width).  Consecutive threads take consecutive lanes of one
// fragment, so for each j the 32 gathers of a half-wave fall in one 64-byte
// segment of a W row.
// Scale folded into the staged copy of W_l: log2(e) on layer 0 (its
// accumulator is then directly in base-2 units), ln(2) on the last layer
// (which converts base-2 activations back); hidden layers need none because
// ln 2 and log2 e cancel between consecutive layers.  The product is rounded
// to fp16 once, a relative change below 2^-11 per weight.
template <class N>
__device__ __forceinline__ float wscale(int l) {
  return (l == 0 ? kLog2e : 1.0f) * (l == N::L - 1 ? kLn2 : 1.0f);
}

// Lane `lane` of fragment (mb, s) of layer l.  For a runtime-width (Gen)
// network, rows and columns past the true widths (p.dims) stage as zeros.
template <class N>
__device__ __forceinline__ f16x8 weight_fragment(const FwdParams& p, int l, int f, int lane) {
  const int KS = N::ks(l);
  const int Nout = N::gen ? p.dims[l + 1] : N::d[l + 1];
  const int mb = f / KS, s = f % KS;
  const int i = lane & 31, g = lane >> 5;
  const int of = outfeat(mb, i);
  f16x8 v;
  if (of < Nout) {
    const int k0 = 16 * s + 8 * g;
    const f16* src = p.w[l] + (int64_t)k0 * Nout + of;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if constexpr (N::gen)
        v[j] = k0 + j < p.dims[l] ? scaled_weight<N::bf>(src[(int64_t)j * Nout], wscale<N>(l)) : (f16)0.0f;
      else
        v[j] = scaled_weight<N::bf>(src[(int64_t)j * Nout], wscale<N>(l));
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (f16)0.0f;
  }
  return v;
}

// Staging tasks: task (l, kb, cb) covers the 8 x 8 tile of W_l at input rows
// 8kb.. and output columns 8cb.. (columns padded to whole 32-feature blocks).
template <class N>
struct StageTasks {
  static constexpr int cbs(int l) { return N::mbs(l) * 4; }
  static constexpr int count(int l) { return (N::d[l] / 8) * cbs(l); }
  static constexpr int first(int l) {
    int o = 0;
    for (int i = 0; i < l; ++i) o += count(i);
    return o;
  }
  static constexpr int total() { return first(N::L); }
};

// Task t of layer l: eight 16-byte row loads of the tile (consecutive tasks
// take consecutive column blocks, so a wave's loads cover whole W rows), an
// 8 x 8 transpose in registers, and eight 16-byte LDS writes.  The tile's
// rows are input features 16s + 8g + [0..7] (s = kb / 2, g = kb % 2) and its
// 8 columns are outfeat(mb, i) for 8 lanes i of one fragment, so column q
// becomes lane (i, g)'s whole 16 bytes of fragment (mb, s).
template <class N, int l>
__device__ __forceinline__ void stage_load(const FwdParams& p, f16x8 (&r)[8], int t) {
  constexpr int Nout = N::d[l + 1], CB = StageTasks<N>::cbs(l);
  const int kb = t / CB, cb = t % CB;
  if (8 * cb < Nout) {
    const f16* src = p.w[l] + (int64_t)(8 * kb) * Nout + 8 * cb;
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = *reinterpret_cast<const f16x8*>(src + (int64_t)j * Nout);
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = f16x8{};
  }
}

template <class N, int l, int RF>
__device__ __forceinline__ void stage_store(f16x8* lds, const f16x8 (&r)[8], int t) {
  constexpr int CB = StageTasks<N>::cbs(l), KS = N::ks(l);
  const int kb = t / CB, cb = t % CB;
  const float sc = wscale<N>(l);
  const int s = kb >> 1, g = kb & 1;
  const int c0 = 8 * cb, mb = c0 >> 5;
  // outfeat(mb, i) = 32mb + 16 i4 + 8 i2 + 4 i3 + (i & 3) for i = 16 i4 + 8 i3 + 4 i2 + (i & 3).
  const int ibase = 16 * ((c0 >> 4) & 1) + 4 * ((c0 >> 3) & 1);
  const int f = N::frag_off(l) + mb * KS + s;
  if (f < RF) return;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int i = ibase + 8 * (q >> 2) + (q & 3);
    f16x8 v;
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = scaled_weight<N::bf>(r[j][q], sc);
    lds[(f - RF) * 64 + 32 * g + i] = v;
  }
}

// Task t (counted over all layers) -> its layer's stage_load / stage_store.
template <class N, int l>
__device__ __forceinline__ void stage_load_any(const FwdParams& p, f16x8 (&r)[8], int t) {
  if constexpr (l < N::L) {
    if (t < StageTasks<N>::first(l + 1)) stage_load<N, l>(p, r, t - StageTasks<N>::first(l));
    else stage_load_any<N, l + 1>(p, r, t);
  }
}
template <class N, int l, int RF>
__device__ __forceinline__ void stage_store_any(f16x8* lds, const f16x8 (&r)[8], int t) {
  if constexpr (l < N::L) {
    if (t < StageTasks<N>::first(l + 1)) stage_store<N, l, RF>(lds, r, t - StageTasks<N>::first(l));
    else stage_store_any<N, l + 1, RF>(lds, r, t);
  }
}

// Stages every fragment from the RF-th on; fragment F lands at LDS slot F - RF.
// When the 8 x 8 tasks give every thread of the workgroup at least one, they
// replace the per-(fragment, lane) column gathers of weight_fragment() (same
// values): 8x fewer load instructions, 3L-128 staging 6.0K -> 4.7K cycles,
// 5L-128 11.0K -> 6.7K.  With fewer tasks than threads (the narrow network:
// 128 tasks for 1024 threads) the gathers spread over all threads are faster
// (2.0K vs 3.2K cycles).  A thread with several tasks issues all their loads
// before its first LDS write, so the staging costs one memory round trip.
template <class N, int NT, int RF>
__device__ __forceinline__ void stage_weights(const FwdParams& p, f16x8* lds) {
  constexpr int TOTAL = StageTasks<N>::total();
  if constexpr (TOTAL >= NT && !N::gen) {
    constexpr int TPT = (TOTAL + NT - 1) / NT;
    f16x8 r[TPT][8];
#pragma unroll
    for (int k = 0; k < TPT; ++k) {
      const int t = threadIdx.x + k * NT;
      if (TOTAL % NT == 0 || t < TOTAL) stage_load_any<N, 0>(p, r[k], t);
    }
#pragma unroll
    for (int k = 0; k < TPT; ++k) {
      const int t = threadIdx.x + k * NT;
      if (TOTAL % NT == 0 || t < TOTAL) stage_store_any<N, 0, RF>(lds, r[k], t);
    }
  } else {
#pragma unroll
    for (int l = 0; l < N::L; ++l) {
      const int items = N::mbs(l) * N::ks(l) * 64;
      for (int item = threadIdx.x; item < items; item += NT) {
        const int f = item >> 6, lane = item & 63;
        if (N::frag_off(l) + f < RF) continue;
        lds[(N::frag_off(l) + f - RF) * 64 + lane] = weight_fragment<N>(p, l, f, lane);
      }
    }
  }
}

// stage_weights in two phases -- every weight load, then (after the caller
// has issued other loads) every LDS write -- for the persistent kernels,
// which request each wave's first x rows in between.  The LDS writes then
// wait for the weight loads only, not for the 24 MB of first x blocks that
// the whole chip requests at kernel start (3L-128 at 1M rows: the
// workgroup barrier after staging passed at ~7 us with the x rows requested
// first, since the weight loads queued behind them).  Same values as
// stage_weights.
template <class N, int NT, int RF>
struct SplitStaging {
  static constexpr int TOTAL = StageTasks<N>::total();
  static constexpr bool kTasks = TOTAL >= NT && !N::gen;
  static constexpr int TPT = kTasks ? (TOTAL + NT - 1) / NT : 1;
  // Column gathers (too few tasks for every thread): per layer, this thread's
  // items item = threadIdx.x + k * NT, k < kSlots(l).
  static constexpr int kSlots(int l) { return (N::mbs(l) * N::ks(l) * 64 + NT - 1) / NT; }
  static constexpr int kSlotOff(int l) {
    int o = 0;
    for (int i = 0; i < l; ++i) o += kSlots(i);
    return o;
  }
  static constexpr int kGather = kTasks ? 1 : kSlotOff(N::L);
  static_assert(!N::gen, "runtime-width networks stage in one phase");
  f16x8 r[TPT][8];   // task rows (kTasks)
  f16x8 g[kGather];  // raw gathered fragment lanes, unscaled (!kTasks)

  __device__ __forceinline__ void load(const FwdParams& p) {
    if constexpr (kTasks) {
#pragma unroll
      for (int k = 0; k < TPT; ++k) {
        const int t = threadIdx.x + k * NT;
        if (TOTAL % NT == 0 || t < TOTAL) stage_load_any<N, 0>(p, r[k], t);
      }
    } else {
      load_layers<0>(p);
    }
  }
  __device__ __forceinline__ void store(f16x8* lds) {
    if constexpr (kTasks) {
#pragma unroll
      for (int k = 0; k < TPT; ++k) {
        const int t = threadIdx.x + k * NT;
        if (TOTAL % NT == 0 || t < TOTAL) stage_store_any<N, 0, RF>(lds, r[k], t);
      }
    } else {
      store_layers<0>(lds);
    }
  }

 private:
  // The lanes weight_fragment() gathers, before its scaling.
  template <int l>
  __device__ __forceinline__ void load_layers(const FwdParams& p) {
    if constexpr (l < N::L) {
      constexpr int KS = N::ks(l), Nout = N::d[l + 1], items = N::mbs(l) * KS * 64;
#pragma unroll
      for (int k = 0; k < kSlots(l); ++k) {
        const int item = threadIdx.x + k * NT;
        f16x8 v = {};
        const int f = item >> 6, lane = item & 63;
        const int mb = f / KS, st = f % KS, of = outfeat(mb, lane & 31);
        if (item < items && of < Nout) {
          const f16* src = p.w[l] + (int64_t)(16 * st + 8 * (lane >> 5)) * Nout + of;
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] = src[(int64_t)j * Nout];
        }
        g[kSlotOff(l) + k] = v;
      }
      load_layers<l + 1>(p);
    }
  }
  template <int l>
  __device__ __forceinline__ void store_layers(f16x8* lds) {
    if constexpr (l < N::L) {
      constexpr int items = N::mbs(l) * N::ks(l) * 64;
#pragma unroll
      for (int k = 0; k < kSlots(l); ++k) {
        const int item = threadIdx.x + k * NT;
        const int f = item >> 6, lane = item & 63;
        if (item < items && N::frag_off(l) + f >= RF) {
          f16x8 v;
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] = scaled_weight<N::bf>(g[kSlotOff(l) + k][j], wscale<N>(l));
          lds[(N::frag_off(l) + f - RF) * 64 + lane] = v;
        }
      }
      store_layers<l + 1>(lds);
    }
  }
};

// Per-block view of the row-major tensors: buffer resources clipped to the
// block's valid rows, so loads of tail rows read zeros and their stores drop.
struct BlockIO {
  rsrc_t x, out;
  rsrc_t stash[kMaxLayers];
  i32x4* stage;  // this wave's LDS staging tile for the output rows (STAGE only)
  unsigned stash_on;  // bit l: stash entry l requested (STASH only)
  int dl[kMaxLayers + 1];  // true widths (Gen networks only)
};

// LDS plan of a workgroup (160 KiB on gfx950), in priority order:
//  * all weight fragments except `reg_frags` leading ones, which each wave
//    keeps in VGPRs instead (4 registers per fragment);
//  * output staging: the last layer's rows go through an LDS tile per wave so
//    that they leave as whole 128-byte cache lines.  A lane of the MFMA result
//    layout holds one row, so direct stores write 32 bytes into each of 32 rows
//    per instruction and complete a row's lines piecemeal, which costs HBM
//    write efficiency once rows are wider than 64 bytes.  The tile holds two
//    32-feature output blocks (128 bytes per row) and is flushed after every
//    second block.  Needs output rows of a multiple of 64 features.  In the
//    training forwards of 8+ waves the same tile also carries each hidden
//    layer's fp32 stash rows, one 32-feature block (128 bytes per row) at a
//    time (flush_stash_stage): 3L-128 at 131072 rows 48.3 -> 42.2 us, at 1M
//    rows 360 -> 325 us;
//  * the 16-byte row-block claim counter.  Without it waves would split the
//    workgroup's blocks statically, and the SIMD arbiter's preference for the
//    older of two waves then lets one wave of each pair finish far ahead of
//    the other (measured: 142 vs 211 us for the 5-layer network at 1M rows).
//    When the weights alone fill the LDS, one fragment moves to VGPRs to make
//    room for it.
template <class N, int NB, int NW>
struct LdsPlan {
  static constexpr int kLds = 163840;
  static constexpr int kRowChunks = 8;  // 16-byte chunks per staged row segment
  static constexpr int kTileChunks = 32 * NB * kRowChunks;
  static constexpr int wbytes = N::nfrag() * 1024;
  static constexpr bool stage =
      !N::gen && N::d[N::L] % 64 == 0 && wbytes + NW * kTileChunks * 16 + 16 <= kLds;
  static constexpr int stage_bytes = stage ? NW * kTileChunks * 16 : 0;
  static constexpr int reg_frags = wbytes + stage_bytes + 16 <= kLds ? 0 : 1;
  static constexpr bool claim = wbytes - reg_frags * 1024 + stage_bytes + 16 <= kLds;
};

// LDS chunk slot of (row, chunk): the chunk index is XORed with the row so that
// the 16-byte writes of 8 consecutive rows (one per lane) and the reads of one
// row's chunks both fall on distinct banks.
__device__ __forceinline__ int stage_slot(int row, int chunk) { return row * 8 + (chunk ^ (row & 7)); }

// The workgroup's claim counter in LDS; the specialisation without one
// allocates nothing.
template <bool E>
struct ClaimSlot {
  __device__ static unsigned int* get() {
    __shared__ unsigned int ctr;
    return &ctr;
  }
};
template <>
struct ClaimSlot<false> {
  __device__ static unsigned int* get() { return nullptr; }
};

template <class N, bool STASH, int ROWS>
__device__ __forceinline__ BlockIO block_io(const FwdParams& p, int64_t row0) {
  const int64_t left = p.M - row0;
  const uint32_t rows = (uint32_t)(left < ROWS ? (left > 0 ? left : 0) : ROWS);
  BlockIO io;
#pragma unroll
  for (int l = 0; l <= N::L; ++l) io.dl[l] = N::gen ? p.dims[l] : N::d[l];
  io.x = make_rsrc(p.x + row0 * io.dl[0], rows * io.dl[0] * 2u);
  io.out = make_rsrc(p.out + row0 * io.dl[N::L], rows * io.dl[N::L] * 2u);
  if constexpr (STASH) {
    io.stash_on = 0;
#pragma unroll
    for (int l = 0; l < N::L - 1; ++l) {
      io.stash[l] = p.stash[l] ? make_rsrc(p.stash[l] + row0 * io.dl[l + 1], rows * io.dl[l + 1] * 4u)
                               : make_rsrc(nullptr, 0u);  // not requested: every store dropped
      if (p.stash[l]) io.stash_on |= 1u << l;
    }
  }
  return io;
}

// Rows of x as raw dwords: kept as i32x4 until the MFMA reads them, because an
// f16x8 destination makes the compiler re-pack the halves right after the load
// (v_bfi copies), which waits for the load at the point of issue.
// For a runtime-width network rows are D wide (a multiple of 16): K-steps
// past D (a wave-uniform test) are zero without a load.
template <int KS, int NB, bool GEN = false>
__device__ __forceinline__ void load_rows(i32x4 (&xa)[KS][NB], rsrc_t xr, int n, int g, int D = KS * 16) {
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      if (GEN && 16 * s >= D)
        xa[s][nb] = i32x4{};
      else
        xa[s][nb] = __builtin_amdgcn_raw_buffer_load_b128(xr, ((nb * 32 + n) * D + 16 * s + 8 * g) * 2, 0, 0);
    }
}
// x rows of the 32*NB-row block starting at row0 (Gen networks: true width).
template <class N, int NB>
__device__ __forceinline__ void load_block_x(i32x4 (&xa)[N::ks(0)][NB], const FwdParams& p,
                                             int64_t row0, int lane) {
  load_rows<N::ks(0), NB, N::gen>(xa, block_io<N, false, 32 * NB>(p, row0).x, lane & 31, lane >> 5,
                                  N::gen ? p.dims[0] : N::d[0]);
}

__device__ __forceinline__ f16x8 as_f16x8(f16x8 v) { return v; }
__device__ __forceinline__ f16x8 as_f16x8(i32x4 v) { return __builtin_bit_cast(f16x8, v); }

// Steps of one row block: step t is output block mb(t) (32 features) of
// layer layer(t), layers in order.
template <class N>
struct Steps {
  static constexpr int count() {
    int s = 0;
    for (int l = 0; l < N::L; ++l) s += N::mbs(l);
    return s;
  }
  static constexpr int layer(int t) {
    int l = 0;
    while (t >= N::mbs(l)) t -= N::mbs(l++);
    return l;
  }
  static constexpr int mb(int t) {
    int l = 0;
    while (t >= N::mbs(l)) t -= N::mbs(l++);
    return t;
  }
  static constexpr int frag(int t) { return N::frag_off(layer(t)) + mb(t) * N::ks(layer(t)); }
};

// Weight fragments (A operands) of one step's MFMA chain.
template <int KSM>
struct Frags {
  f16x8 a[KSM];
};

// This lane's LDS fragment slots, one base per 64 KiB window: ds_read's
// immediate offset has 16 bits, so fragments past the first window would
// otherwise each need their own address add.  The bases go through opaque():
// weights never change after staging, and without it the compiler would
// hoist every fragment read out of the persistent row loop (and spill).
template <class N, int RF>
struct FragBase {
  static constexpr int kWindows = ((N::nfrag() - RF) * 1024 + 65535) / 65536;
  const char* w[kWindows];
  __device__ __forceinline__ FragBase(const char* lds_b, int lane_off) {
#pragma unroll
    for (int i = 0; i < kWindows; ++i) w[i] = lds_b + opaque(lane_off + i * 65536);
  }
};

// Fragment s of step t: from LDS, or the wave's register copy `rf` below RF.
template <class N, int t, int RF>
__device__ __forceinline__ f16x8 frag(int s, const FragBase<N, RF>& fb, f16x8 rf) {
  constexpr int F0 = Steps<N>::frag(t);
  if (F0 + s < RF) return rf;
  const int off = (F0 + s - RF) * 1024;  // a constant after unrolling
  return *reinterpret_cast<const f16x8*>(fb.w[off >> 16] + (off & 0xffff));
}

// Reads fragments [S0, KS) of step t.
template <class N, int t, int KSM, int RF, int S0 = 0>
__device__ __forceinline__ void load_frags(Frags<KSM>& f, const FragBase<N, RF>& fb, f16x8 rf) {
  constexpr int KS = N::ks(Steps<N>::layer(t));
#pragma unroll
  for (int s = S0; s < KS; ++s) f.a[s] = frag<N, t, RF>(s, fb, rf);
}

// MFMA chain of one output block over input K-steps [S0, S1):
// acc[nb] (+)= W_l[K-steps, block]^T . in.  S0 == 0 starts from zero.
// As soon as the MFMAs of K-step s have been issued (they read their A
// operand at issue), register f.a[s] is refilled with fragment s of step TN,
// the chain after next: each LDS read then has a whole activation epilogue
// to complete before its MFMA, and the fragments occupy no more registers
// than one step's set.
template <class N, int TN, int RF, int S0, int S1, int NB, int KSM, class T, int KIN>
__device__ __forceinline__ void chain(f32x16 (&acc)[NB], Frags<KSM>& f, const T (&in)[KIN][NB],
                                      const FragBase<N, RF>& fb, f16x8 rf) {
  static_assert(KIN >= S1, "input K-steps");
  constexpr int KSN = N::ks(Steps<N>::layer(TN));
  if constexpr (S0 == 0) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] = (f32x16){};
  }
#pragma unroll
  for (int s = S0; s < S1; ++s) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] = mfma32x32x16<N::bf>(f.a[s], as_f16x8(in[s][nb]), acc[nb]);
    if (s < KSN) f.a[s] = frag<N, TN, RF>(s, fb, rf);
  }
}

// Activation and hand-off of output block mb: hidden layers apply softplus
// (base-2 units), optionally store the fp32 stash, and pack the next layer's
// B operands; the last layer stores fp16 rows of `out`.  The fast form
// (EXACT false) evaluates sp2 directly; an overflow there (sp2 = +inf for
// u >= 128, or an fp16 operand past 65,504) or a NaN is caught one layer
// later, by `bad` (see below).  The exact form replaces overflowed values by
// u and hands on sp2 / 2: in base-2 units a hidden activation is 1.44x its
// natural value, so values above ~45,400 (natural) would not fit fp16,
// whereas the reference's fp16 h (kernel.py:110) holds them up to 65,504.
// Halving (and doubling every later accumulator, kIn) keeps the whole range;
// both are exact power-of-two scalings.
//
// Overflow detection by propagation (networks of up to 3 layers): every
// accumulator of a row in layer l >= 1 sums that row's whole input vector,
// and a product with an infinite or NaN operand is infinite or NaN whatever
// the weight (inf * 0 = NaN), so one non-finite input makes every
// accumulator of the row non-finite.  A finite input row keeps the fp32
// accumulators finite (at most 128 products of fp16 magnitudes, far below
// the fp32 range).  Testing one accumulator per row and layer -- element 0 of
// output block 0, which every lane holds for its row -- therefore detects
// every overflow and NaN of the layer below: one class test per lane and
// layer instead of folding every packed activation into a running maximum
// (33 v_pk_maximum3_f16 per 32-row block of the 3-layer network; 3L-128 at
// 1M rows 129.4 -> 126.2 us, narrow at 4M 120.1 -> 116.6 us).  Layer 0's
// inputs are the caller's x, and a non-finite x also triggers the exact
// pass, which reproduces it.  The 4- and 5-layer kernels, bound by the
// matrix core rather than by VALU issue, keep the running maximum `m`
// (sp2_track): without it the scheduler spilled in their hot loop.
template <class N>
constexpr bool kPropagate = N::L <= 3;

// Cache policy of output rows stored straight from the MFMA layout (no LDS
// staging tile): each store instruction writes 16 bytes of each of 32 rows.
// Rows of at most 64 bytes (the narrow network's 32) are then covered by
// consecutive lanes and stream past L2 (nt); wider rows are written a piece
// at a time, so they keep the default policy and L2 merges the pieces into
// whole lines before they go to HBM (5-layer 128-wide at 1M rows: WRITE_SIZE
// 1.44x -> 1.00x the output bytes, 201.3 -> 194.5 us, same box).  The
// training forward's outputs keep the default policy at any width
// (kOutStore).
template <int ROW_BYTES, bool STASH>
constexpr int kDirectOutStore = ROW_BYTES > 64 ? kStashStore : kOutStore<STASH>;

// Stores the staged 128-byte segment mb (fp32 features [32 mb, 32 mb + 32))
// of the wave's 32 stash rows of width W: 8 rows x 128 bytes (8 whole cache
// lines) per instruction, against 32 rows x 2 pieces of 16 bytes for stores
// straight from the MFMA layout.  Default cache policy, as those.
template <int W>
__device__ __forceinline__ void flush_stash_stage(const BlockIO& io, const rsrc_t& sr, int mb, int lane) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = 64 * i + lane;
    const int row = q >> 3, c = q & 7;
    const i32x4 v = io.stage[stage_slot(row, c)];
    __builtin_amdgcn_raw_buffer_store_b128(v, sr, row * W * 4 + mb * 128 + c * 16, 0, kStashStore);
  }
  // The next writes into the tile must stay behind these reads.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

template <class N, int l, int NB, bool STASH, int STAGE, bool EXACT, int KSM>
__device__ __forceinline__ void epilogue(const BlockIO& io, const f32x16 (&acc)[NB], int mb,
                                         f16x8 (&nxt)[KSM][NB], bool& bad, f16x2& m, int lane) {
  constexpr int Nout = N::d[l + 1];
  constexpr bool LAST = (l == N::L - 1);
  const int n = lane & 31, g = lane >> 5;
  if constexpr (!EXACT && kPropagate<N> && l > 0) {
    if (mb == 0) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) bad = bad || !__builtin_isfinite(acc[nb][0]);
    }
  }
  // Registers 0..7 -> features 32mb + 8g + [0..7]; 8..15 -> 32mb + 16 + 8g + [0..7].
  const bool lo_ok = (32 * mb + 16 <= Nout);  // folded after unrolling
  const bool hi_ok = (32 * mb + 32 <= Nout);
  constexpr float kIn = (EXACT && l > 0) ? 2.0f : 1.0f;  // the exact form's halved inputs
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const uint32_t elem = (uint32_t)((nb * 32 + n) * Nout + 32 * mb + 8 * g);
    if constexpr (LAST && STAGE) {
      const f32x16 v = acc[nb] * kIn;  // ln 2 is folded into the staged W_L
      const int row = nb * 32 + n;
      const int c = 4 * (mb & 1) + g;  // chunk within the staged 128-byte row segment
      io.stage[stage_slot(row, c)] =
          __builtin_bit_cast(i32x4, pack8<N::bf>(v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]));
      io.stage[stage_slot(row, c + 2)] =
          __builtin_bit_cast(i32x4, pack8<N::bf>(v[8], v[9], v[10], v[11], v[12], v[13], v[14], v[15]));
    } else if constexpr (LAST && N::gen) {
      // Runtime output width OW: whole 8-feature pieces when OW is a multiple
      // of 8, else one 2-byte store per feature; features past OW are dropped.
      const f32x16 v = acc[nb] * kIn;
      const int OW = io.dl[N::L], c = 32 * mb + 8 * g;
      const uint32_t e = (uint32_t)((nb * 32 + n) * OW + c);
      const f16x8 lo = pack8<N::bf>(v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]);
      const f16x8 hi = pack8<N::bf>(v[8], v[9], v[10], v[11], v[12], v[13], v[14], v[15]);
      // The compile-time width (128) bounds the row: wide rows use the
      // merging policy, as below.
      constexpr int P = kDirectOutStore<N::d[N::L] * 2, STASH>;
      if (OW % 8 == 0) {
        if (c < OW) buf_store16<P>(lo, io.out, e * 2);
        if (c + 16 < OW) buf_store16<P>(hi, io.out, e * 2 + 32);
      } else {
        // Each element converted on its own: taken out of the packed lo / hi
        // vectors, the 2-byte store builtin was given element 0 every time.
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (c + j < OW)
            __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, f32_to_elem<N::bf>(v[j])), io.out,
                                                  (int)((e + j) * 2), 0, P);
          if (c + 16 + j < OW)
            __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, f32_to_elem<N::bf>(v[8 + j])), io.out,
                                                  (int)((e + 16 + j) * 2), 0, P);
        }
      }
    } else if constexpr (LAST) {
      const f32x16 v = acc[nb] * kIn;  // ln 2 is folded into the staged W_L
      constexpr int P = kDirectOutStore<Nout * 2, STASH>;
      if (lo_ok) buf_store16<P>(pack8<N::bf>(v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]), io.out, elem * 2);
      if (hi_ok) buf_store16<P>(pack8<N::bf>(v[8], v[9], v[10], v[11], v[12], v[13], v[14], v[15]), io.out, elem * 2 + 32);
    } else {
      // log2 e is folded into the staged W_1, so acc is u in base-2 units.
      const f32x16 u = acc[nb] * kIn;
      float s[16], q[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        s[e] = EXACT ? sp2_fix(u[e], sp2(u[e])) : sp2(u[e]);
        q[e] = EXACT ? 0.5f * s[e] : s[e];
      }
      f16x8 lo = pack8<N::bf>(q[0], q[1], q[2], q[3], q[4], q[5], q[6], q[7]);
      f16x8 hi = pack8<N::bf>(q[8], q[9], q[10], q[11], q[12], q[13], q[14], q[15]);
      if constexpr (!EXACT && !kPropagate<N>) m = sp2_track<!STASH>(m, lo, hi);
      // Ordering anchor (no instruction) where the running maximum is gone:
      // keeps the packed activations of consecutive epilogues in program
      // order, as the maximum's dependence chain did.  Without either, the
      // scheduler interleaved consecutive epilogues far enough that the
      // stash kernels spilled (and the 5-layer inference kernel waited on its
      // fragment reads: 209 -> 312 us at 1M rows).  The exact pass spills
      // with it; the narrow network's two-block kernel (NB = 2) is faster
      // without it (116.6 vs 120.7 us at 4M rows).
      if constexpr (!EXACT && kPropagate<N> && NB == 1) asm volatile("" : "+v"(lo), "+v"(hi));
      if constexpr (STASH && N::gen) {
        // Runtime hidden width HW (a multiple of 16): feature groups past it are dropped.
        const rsrc_t sr = io.stash[l];
        const int HW = io.dl[l + 1], c = 32 * mb + 8 * g;
        const uint32_t e4 = (uint32_t)((nb * 32 + n) * HW + c) * 4;
        float h[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) h[e] = s[e] * kLn2;
        if (c < HW) {
          buf_store16<kStashStore>((f32x4){h[0], h[1], h[2], h[3]}, sr, e4);
          buf_store16<kStashStore>((f32x4){h[4], h[5], h[6], h[7]}, sr, e4 + 16);
        }
        if (c + 16 < HW) {
          buf_store16<kStashStore>((f32x4){h[8], h[9], h[10], h[11]}, sr, e4 + 64);
          buf_store16<kStashStore>((f32x4){h[12], h[13], h[14], h[15]}, sr, e4 + 80);
        }
      } else if constexpr (STASH && STAGE == 2 && NB == 1 && Nout % 32 == 0) {
        // Through the wave's staging tile, so that the stash leaves as whole
        // 128-byte lines (flush_stash_stage); registers 0..7 are chunks 2g,
        // 2g + 1 of the row's 128-byte segment mb, 8..15 chunks 4 + 2g, 5 + 2g.
        if ((io.stash_on >> l) & 1u) {  // (an entry not requested: nothing to stage)
          float h[16];
#pragma unroll
          for (int e = 0; e < 16; ++e) h[e] = s[e] * kLn2;
          io.stage[stage_slot(n, 2 * g)] = __builtin_bit_cast(i32x4, (f32x4){h[0], h[1], h[2], h[3]});
          io.stage[stage_slot(n, 2 * g + 1)] = __builtin_bit_cast(i32x4, (f32x4){h[4], h[5], h[6], h[7]});
          io.stage[stage_slot(n, 2 * g + 4)] = __builtin_bit_cast(i32x4, (f32x4){h[8], h[9], h[10], h[11]});
          io.stage[stage_slot(n, 2 * g + 5)] = __builtin_bit_cast(i32x4, (f32x4){h[12], h[13], h[14], h[15]});
          flush_stash_stage<Nout>(io, io.stash[l], mb, lane);
        }
      } else if constexpr (STASH) {
        const rsrc_t sr = io.stash[l];
        float h[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) h[e] = s[e] * kLn2;
        if (lo_ok) {
          buf_store16<kStashStore>((f32x4){h[0], h[1], h[2], h[3]}, sr, elem * 4);
          buf_store16<kStashStore>((f32x4){h[4], h[5], h[6], h[7]}, sr, elem * 4 + 16);
        }
        if (hi_ok) {
          buf_store16<kStashStore>((f32x4){h[8], h[9], h[10], h[11]}, sr, elem * 4 + 64);
          buf_store16<kStashStore>((f32x4){h[12], h[13], h[14], h[15]}, sr, elem * 4 + 80);
        }
      }
      if (2 * mb < KSM) nxt[2 * mb][nb] = lo;
      if (2 * mb + 1 < KSM) nxt[2 * mb + 1][nb] = hi;
    }
  }
}

// Stores the staged 128-byte row segments of output features
// [64 seg, 64 seg + 64) with 16-byte stores, 8 rows x 128 bytes (8 whole cache
// lines) per instruction, with cache policy POL.
template <class N, int NB, int POL>
__device__ __forceinline__ void flush_stage(const BlockIO& io, int seg, int lane) {
  constexpr int Nout = N::d[N::L];
  constexpr int TC = LdsPlan<N, NB, 1>::kTileChunks;
  // The tile was written by other lanes of this wave; LDS executes one wave's
  // operations in order, so only the compiler needs a fence here.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int i = 0; i < TC / 64; ++i) {
    const int q = 64 * i + lane;  // linear 16-byte chunk of the tile
    const int row = q >> 3, c = q & 7;
    const i32x4 v = io.stage[stage_slot(row, c)];
    __builtin_amdgcn_raw_buffer_store_b128(v, io.out, row * Nout * 2 + seg * 128 + c * 16, 0, POL);
  }
  // The next writes into the tile must stay behind these reads.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// Register state of a wave while it runs one row block.
template <class N, int NB, int KSM>
struct Chain {
  static constexpr int KS0 = N::ks(0);
  i32x4 xa[KS0][NB];             // x rows of the block (refilled with the next block's)
  f16x8 b0[KSM][NB], b1[KSM][NB];  // hidden activations, ping-pong between layers
  f32x16 acc[2][NB];             // accumulators of the current and the next step
  Frags<KSM> fr;                 // fragments of the next chain to issue
  bool bad;                      // some row's accumulator of layer >= 1 was not finite (kPropagate)
  f16x2 ovf;                     // running maximum of the block's packed sp2 values (!kPropagate)
  f16x8 rf;                      // register-resident fragment (LdsPlan::reg_frags)

  // Layer l reads x (l = 0), b0 (odd l) or b1 (even l >= 2) and writes b0
  // (even l) or b1 (odd l).
  template <int l>
  __device__ __forceinline__ auto& in() {
    if constexpr (l == 0) return xa;
    else if constexpr (l % 2 == 1) return b0;
    else return b1;
  }
  template <int l>
  __device__ __forceinline__ auto& out() {
    if constexpr (l % 2 == 0) return b0;
    else return b1;
  }
};

// Step t of a row block.  Issue order: when step t+1 belongs to the same
// layer, its MFMA chain (which runs on the matrix core while this step's
// activation runs on the VALU), then the epilogue of step t, and -- at a layer
// boundary -- the first chain of the next layer, which needs all of this
// layer's outputs.  c.fr holds step t+1's fragments on entry; the chain
// replaces them with those of step t+2 (step 0 of the next row block after
// the last chain of this one).
template <class N, int t, int NB, bool STASH, int STAGE, bool EXACT, int KSM, int RF>
__device__ __forceinline__ void step(const FwdParams& p, const BlockIO& io, Chain<N, NB, KSM>& c,
                                     const FragBase<N, RF>& fb, int64_t next, int lane) {
  using S = Steps<N>;
  constexpr int T = S::count();
  constexpr int l = S::layer(t), mb = S::mb(t);
  constexpr bool same = t + 1 < T && S::layer(t + 1) == l;
  constexpr int ROWS = 32 * NB;
  constexpr int TN = (t + 2) % T;
  constexpr int KS1 = t + 1 < T ? N::ks(S::layer(t + 1)) : 0;
  if constexpr (same) {
    chain<N, TN, RF, 0, KS1, NB>(c.acc[(t + 1) & 1], c.fr, c.template in<l>(), fb, c.rf);
    load_frags<N, TN, KSM, RF, KS1>(c.fr, fb, c.rf);
  }
  // Last block of a layer: the next layer's first chain can already run over
  // the K-steps the earlier blocks produced (2 per block); only the last two
  // wait for this step's epilogue.
  constexpr int EARLY = (t + 1 < T && !same) ? 2 * mb : 0;
  if constexpr (EARLY > 0)
    chain<N, TN, RF, 0, EARLY, NB>(c.acc[(t + 1) & 1], c.fr, c.template in<(l + 1) % N::L>(), fb, c.rf);
  if constexpr (l == 0 && (same ? t + 1 == N::mbs(0) - 1 : t == 0)) {
    // Every MFMA that reads x has been issued: refill xa with the next block's
    // rows (past the end the resource is empty and the refill reads zeros).
    MLPMK_SCHED_FENCE();
    load_block_x<N, NB>(c.xa, p, next * ROWS, lane);
  }
  epilogue<N, l, NB, STASH, STAGE, EXACT, KSM>(io, c.acc[t & 1], mb, c.template out<l>(), c.bad, c.ovf, lane);
  if constexpr (l == N::L - 1 && STAGE) {
    if (mb & 1) flush_stage<N, NB, kOutStore<STASH>>(io, mb >> 1, lane);
  }
  if constexpr (t + 1 < T && !same) {
    chain<N, TN, RF, EARLY, KS1, NB>(c.acc[(t + 1) & 1], c.fr, c.template in<l + 1>(), fb, c.rf);
    load_frags<N, TN, KSM, RF, KS1>(c.fr, fb, c.rf);
  }
  if constexpr (t + 1 < T) step<N, t + 1, NB, STASH, STAGE, EXACT, KSM, RF>(p, io, c, fb, next, lane);
}

// One row block: the whole layer chain, stores, and the x refill for block
// `next`.  On entry c.xa holds the block's x rows and c.fr the fragments of
// step 0; on exit they hold the same for block `next`.  Returns (wave-
// uniform) whether the fast form overflowed or met a NaN somewhere in the
// block (see epilogue).
template <class N, int NB, bool STASH, int STAGE, bool EXACT, int KSM, int RF>
__device__ __forceinline__ bool fwd_block(const FwdParams& p, Chain<N, NB, KSM>& c, const char* lds_b,
                                          int lane_off, i32x4* stage, int64_t b, int64_t next, int lane) {
  constexpr int ROWS = 32 * NB;
  constexpr int T1 = 1 % Steps<N>::count();
  BlockIO io = block_io<N, STASH, ROWS>(p, b * ROWS);
  io.stage = stage;
  const FragBase<N, RF> fb(lds_b, lane_off);
  c.bad = false;
  c.ovf = f16x2{};
  chain<N, T1, RF, 0, N::ks(0), NB>(c.acc[0], c.fr, c.xa, fb, c.rf);
  load_frags<N, T1, KSM, RF, N::ks(0)>(c.fr, fb, c.rf);
  step<N, 0, NB, STASH, STAGE, EXACT, KSM, RF>(p, io, c, fb, next, lane);
  if constexpr (EXACT) return false;
  else if constexpr (kPropagate<N>) return __builtin_amdgcn_ballot_w64(c.bad) != 0;
  else return sp2_overflowed<N::bf>(c.ovf);
}

// Block b with the fast softplus form, then -- only if one of its wave's rows
// overflowed (some u >= 128 or an fp16 activation past 65,504) or met a NaN
// -- again with the exact form, from a fresh read of its x rows and step-0
// fragments.  The second pass rewrites
// every output (and stash) row of the block and leaves c as the first did.
template <class N, int NB, bool STASH, int STAGE, int KSM, int RF>
__device__ __forceinline__ void fwd_block_checked(const FwdParams& p, Chain<N, NB, KSM>& c, const char* lds_b,
                                                  int lane_off, i32x4* stage, int64_t b, int64_t next,
                                                  int lane) {
  constexpr int ROWS = 32 * NB;
  if (__builtin_expect(fwd_block<N, NB, STASH, STAGE, false, KSM, RF>(p, c, lds_b, lane_off, stage, b, next, lane),
                       0)) {
    load_block_x<N, NB>(c.xa, p, b * ROWS, lane);
    load_frags<N, 0, KSM, RF>(c.fr, FragBase<N, RF>(lds_b, lane_off), c.rf);
    fwd_block<N, NB, STASH, STAGE, true, KSM, RF>(p, c, lds_b, lane_off, stage, b, next, lane);
  }
}

// Persistent forward.  Workgroup b owns row blocks b, b + G, b + 2G, ...
// (G = grid size, 32*NB rows per block); its waves claim them one at a time
// from a counter in LDS.  Claiming (rather than a fixed wave-to-block map)
// matters because the SIMD arbiter favours the older of two waves: with a
// static split one wave of each pair finishes early and the other runs the
// tail alone.  Each wave keeps the x rows of its next claimed block in flight
// while it computes the current one.  D is the number of such blocks in
// flight; one is enough (deeper rings measured no faster).

template <class N, int NB, bool STASH, int NW, int D>
__global__ __launch_bounds__(NW * 64) void fwd_kernel(FwdParams p) {
  static_assert(N::valid(), "unsupported widths");
  static_assert(D >= 1 && D <= 4, "prefetch depth");
  using Plan = LdsPlan<N, NB, NW>;
  constexpr int KSM = N::ksmax();
  constexpr int ROWS = 32 * NB;
  // Staging tile use: 0 none, 1 the output rows, 2 the output rows and the
  // stash (workgroups of 8+ waves; with one block per wave, in the 4-wave
  // kernels of small batches, the staging's LDS round trip is not hidden:
  // M = 16384 11.3 -> 11.9 us).
  constexpr int STAGE = Plan::stage ? (STASH && NW >= 8 ? 2 : 1) : 0;
  constexpr int TC = Plan::kTileChunks;
  constexpr int RF = Plan::reg_frags;
  constexpr bool CLAIM = Plan::claim;
  __shared__ f16x8 lds[(N::nfrag() - RF) * 64];
  __shared__ i32x4 stage_tiles[STAGE ? NW * TC : 1];
  unsigned int* const claim_ctr = ClaimSlot<CLAIM>::get();
  const int lane = threadIdx.x & 63;
  // readfirstlane marks the wave index as wave-uniform, so the block index and
  // every buffer resource derived from it live in SGPRs (a per-lane resource
  // would force a readfirstlane/exec waterfall loop around each buffer access).
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t nblk = (p.M + ROWS - 1) / ROWS;
  const int64_t G = gridDim.x;
  // Wave w's first block is the workgroup's w-th (static); later blocks are
  // claimed from the counter, which starts past the first NW.  The persistent
  // kernels (more than 8 waves) request the first block's x rows between the
  // weight loads and the weight LDS writes of the staging (SplitStaging;
  // requesting them after the staging: 5L-128 at 1M rows 315 us against
  // 203 us); the 4- and 8-wave kernels of smaller batches request them
  // after it (M = 65536: 11.7 / 19.3 us against 12.8 / 21.7 us with the
  // early request, 3L / 5L).  Past the end a block's resource is empty:
  // reads zeros.
  static_assert(D == 1, "one block of x rows in flight per wave");
  constexpr bool kEarlyX = NW > 8;
  Chain<N, NB, KSM> c;
  const int64_t b0 = (int64_t)blockIdx.x + (int64_t)wid * G;
  if constexpr (CLAIM) {
    if (threadIdx.x == 0) *claim_ctr = NW;
  }
  if constexpr (kEarlyX) {
    SplitStaging<N, NW * 64, RF> sw;
    sw.load(p);
    load_block_x<N, NB>(c.xa, p, b0 * ROWS, lane);
    sw.store(lds);
  } else {
    stage_weights<N, NW * 64, RF>(p, lds);
  }
  __syncthreads();

  i32x4* stage = stage_tiles + (STAGE ? wid * TC : 0);
  // Next block of this workgroup (>= nblk once its share is exhausted).  Without
  // LDS room for the counter, wave w takes the workgroup's blocks w, w + NW, ...
  unsigned int seq = (unsigned int)wid + NW;
  auto claim = [&]() -> int64_t {
    unsigned int j;
    if constexpr (CLAIM) {
      j = 0;
      if (lane == 0)
        j = __hip_atomic_fetch_add(claim_ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      j = __builtin_amdgcn_readfirstlane(j);
    } else {
      j = seq;
      seq += NW;
    }
    return (int64_t)blockIdx.x + (int64_t)j * G;
  };

  c.rf = RF ? weight_fragment<N>(p, 0, 0, lane) : f16x8{};
  const char* lds_b = reinterpret_cast<const char*>(lds);
  const int lane_off = lane * 16;  // this lane's 16 bytes within a 1 KiB fragment
  int64_t b = b0;
  if (b >= nblk) return;  // no barrier follows
  if constexpr (!kEarlyX) load_block_x<N, NB>(c.xa, p, b * ROWS, lane);
  load_frags<N, 0, KSM, RF>(c.fr, FragBase<N, RF>(lds_b, lane_off), c.rf);
  // The first block is peeled so that the loop header is entered from two
  // paths with the same outstanding memory operations (the x refill, then
  // stores): vmcnt counts loads and stores in issue order.
  int64_t next = claim();
  fwd_block_checked<N, NB, STASH, STAGE, KSM, RF>(p, c, lds_b, lane_off, stage, b, next, lane);
  // Claims are increasing per wave, so once one is past the end all later are.
  for (b = next; b < nblk; b = next) {
    next = claim();
    fwd_block_checked<N, NB, STASH, STAGE, KSM, RF>(p, c, lds_b, lane_off, stage, b, next, lane);
  }
}

}  // namespace mlpmk

// ---------------------------------------------------------------------------
// Launch templates (host)
// ---------------------------------------------------------------------------
#include "host_common.h"

namespace mlpmk {

typedef Net<128, 128, 128, 128> Net3L128;
typedef Net<128, 128, 128, 128, 128, 128> Net5L128;
typedef Net<32, 64, 64, 16> NetNarrow;
// Runtime-width networks of 2..5 layers, compiled at width 128 (fwd_generic_dims).
typedef Gen<Net<128, 128, 128>> GNet2;
typedef Gen<Net<128, 128, 128, 128>> GNet3;
typedef Gen<Net<128, 128, 128, 128, 128>> GNet4;
typedef Gen<Net<128, 128, 128, 128, 128, 128>> GNet5;

template <class N>
static bool dims_match(int L, const int* dims) {
  if (L != N::L) return false;
  for (int i = 0; i <= L; ++i)
    if (dims[i] != N::d[i]) return false;
  return true;
}

template <class N, int NB, bool STASH, int NW, int D>
static int launch_fwd(const FwdParams& p, hipStream_t st, LaunchInfo* info) {
  constexpr int kMaxDev = 64;
  static int occ_cache[kMaxDev];  // 0 = unknown; benign race (idempotent value)
  int cus = 0;
  int rc = current_device_cus(&cus);
  if (rc != MLPMK_OK) return rc;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  const void* kern = reinterpret_cast<const void*>(&fwd_kernel<N, NB, STASH, NW, D>);
  int occ = (dev >= 0 && dev < kMaxDev) ? occ_cache[dev] : 0;
  if (occ <= 0) {
    rc = kernel_occupancy(kern, NW * 64, &occ);
    if (rc != MLPMK_OK) return rc;
    if (dev >= 0 && dev < kMaxDev) occ_cache[dev] = occ;
  }
  const int64_t rows = 32 * NB;
  const int64_t nblk = (p.M + rows - 1) / rows;
  const int64_t wgs = (nblk + NW - 1) / NW;
  const int64_t cap = (int64_t)cus * occ;
  const int grid = (int)(wgs < cap ? wgs : cap);
  if (info) {
    *info = LaunchInfo{MLPMK_KERNEL_PERSISTENT, (int)rows, NW, grid, occ};
    return MLPMK_OK;
  }
  (void)hipGetLastError();
  hipLaunchKernelGGL((fwd_kernel<N, NB, STASH, NW, D>), dim3(grid), dim3(NW * 64), 0, st, p);
  e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "fwd kernel launch");
  return MLPMK_OK;
}

// NB row blocks per fragment read and NW waves per workgroup for inference,
// NBS and NWS with the fp32 stash (whose extra registers would spill at
// NW = 12 for the 128-wide networks, and at NB = 2 for the narrow one).
//
// Small batches take narrower workgroups.  With NW waves per workgroup the
// grid holds ceil(blocks / NW) workgroups, so with few blocks a 12-wave
// workgroup packs three one-block waves onto each SIMD of a handful of CUs
// (M = 4096: 11 CUs, each wave's block 14K cycles because three waves share
// the SIMD) while the rest of the chip idles.  Up to 4 blocks per CU the
// kernel runs 4-wave workgroups (one wave per SIMD), up to 8 blocks per CU
// 8-wave workgroups; the persistent NW-wave kernel takes over beyond that.
template <class N, int NB, int NW, int NBS, int NWS, int D>
static int launch_fwd_any(const FwdParams& p, bool stash, hipStream_t st, LaunchInfo* info) {
  int cus = 0;
  const int rc = current_device_cus(&cus);
  if (rc != MLPMK_OK) return rc;
  const int64_t nblk = (p.M + 32 * (stash ? NBS : NB) - 1) / (32 * (stash ? NBS : NB));
  if (stash) {
    if constexpr (NWS > 4) {
      if (nblk <= 4 * (int64_t)cus) return launch_fwd<N, NBS, true, 4, D>(p, st, info);
    }
    return launch_fwd<N, NBS, true, NWS, D>(p, st, info);
  }
  if constexpr (NW > 4) {
    if (nblk <= 4 * (int64_t)cus) return launch_fwd<N, NB, false, 4, D>(p, st, info);
  }
  if constexpr (NW > 8) {
    if (nblk <= 8 * (int64_t)cus) return launch_fwd<N, NB, false, 8, D>(p, st, info);
  }
  return launch_fwd<N, NB, false, NW, D>(p, st, info);
}

}  // namespace mlpmk
