// Forward megakernel for gfx950 (MI355X).
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
//  * Activations run in base-2 units: layer 0's accumulator is scaled by log2(e),
//    hidden layers then chain with no scaling at all (ln2 and log2e cancel
//    between W^T h' and the next exp2), and the last accumulator is scaled by
//    ln2.  The stash stores natural-unit h = ln2 * h'.
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
template <class N, int NT>
__device__ __forceinline__ void stage_weights(const FwdParams& p, f16x8* lds) {
#pragma unroll
  for (int l = 0; l < N::L; ++l) {
    const int K = N::d[l], Nout = N::d[l + 1];
    const int KS = N::ks(l);
    const int items = N::mbs(l) * KS * 64;
    const f16* __restrict__ w = p.w[l];
    for (int item = threadIdx.x; item < items; item += NT) {
      const int f = item >> 6, lane = item & 63;
      const int mb = f / KS, s = f % KS;
      const int i = lane & 31, g = lane >> 5;
      const int of = outfeat(mb, i);
      f16x8 v;
      if (of < Nout) {
        const f16* src = w + (int64_t)(16 * s + 8 * g) * Nout + of;
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = src[(int64_t)j * Nout];
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = (f16)0.0f;
      }
      (void)K;
      lds[(N::frag_off(l) + f) * 64 + lane] = v;
    }
  }
}

// Per-block view of the row-major tensors: buffer resources clipped to the
// block's valid rows, so loads of tail rows read zeros and their stores drop.
struct BlockIO {
  rsrc_t x, out;
  rsrc_t stash[kMaxLayers];
};

template <class N, bool STASH, int ROWS>
__device__ __forceinline__ BlockIO block_io(const FwdParams& p, int64_t row0) {
  const int64_t left = p.M - row0;
  const uint32_t rows = (uint32_t)(left < ROWS ? (left > 0 ? left : 0) : ROWS);
  BlockIO io;
  io.x = make_rsrc(p.x + row0 * N::d[0], rows * N::d[0] * 2u);
  io.out = make_rsrc(p.out + row0 * N::d[N::L], rows * N::d[N::L] * 2u);
  if constexpr (STASH) {
#pragma unroll
    for (int l = 0; l < N::L - 1; ++l)
      io.stash[l] = make_rsrc(p.stash[l] + row0 * N::d[l + 1], rows * N::d[l + 1] * 4u);
  }
  return io;
}

template <int KS, int NB>
__device__ __forceinline__ void load_rows(f16x8 (&xa)[KS][NB], rsrc_t xr, int n, int g) {
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int s = 0; s < KS; ++s)
      xa[s][nb] = buf_load16<f16x8>(xr, (uint32_t)(((nb * 32 + n) * (KS * 16) + 16 * s + 8 * g) * 2));
}

// One layer l over NB batch blocks.  `in` holds the B operands of the layer's
// KS input K-steps; hidden layers write the next layer's B operands to `nxt`,
// the last layer stores fp16 rows of `out`.
template <class N, int l, int NB, bool STASH, int KSM>
__device__ __forceinline__ void run_layer(const BlockIO& io, const f16x8* __restrict__ lds,
                                          const f16x8 (&in)[KSM][NB], f16x8 (&nxt)[KSM][NB], int lane) {
  constexpr int KS = N::ks(l);
  constexpr int MB = N::mbs(l);
  constexpr int Nout = N::d[l + 1];
  constexpr bool LAST = (l == N::L - 1);
  const int n = lane & 31, g = lane >> 5;
  const f16x8* frag = lds + N::frag_off(l) * 64 + lane;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    // The weight fragments never change after staging; without this fence the
    // compiler hoists every ds_read of the layer out of the row loop and spills.
    asm volatile("" ::: "memory");
    MLPMK_SCHED_FENCE();
    f32x16 acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] = (f32x16){};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const f16x8 a = frag[(mb * KS + s) * 64];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) acc[nb] = mfma32x32x16(a, in[s][nb], acc[nb]);
    }
    // Registers 0..7 -> features 32mb + 8g + [0..7]; 8..15 -> 32mb + 16 + 8g + [0..7].
    const bool lo_ok = (32 * mb + 16 <= Nout);  // folded after unrolling
    const bool hi_ok = (32 * mb + 32 <= Nout);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const uint32_t elem = (uint32_t)((nb * 32 + n) * Nout + 32 * mb + 8 * g);
      float v[16];
      if constexpr (LAST) {
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = acc[nb][e] * kLn2;
        if (lo_ok) buf_store16(pack8(v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]), io.out, elem * 2);
        if (hi_ok)
          buf_store16(pack8(v[8], v[9], v[10], v[11], v[12], v[13], v[14], v[15]), io.out, elem * 2 + 32);
      } else {
        const float scale = (l == 0) ? kLog2e : 1.0f;
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = sp2(acc[nb][e] * scale);
        if constexpr (STASH) {
          const rsrc_t sr = io.stash[l];
          if (lo_ok) {
            buf_store16((f32x4){v[0], v[1], v[2], v[3]} * kLn2, sr, elem * 4);
            buf_store16((f32x4){v[4], v[5], v[6], v[7]} * kLn2, sr, elem * 4 + 16);
          }
          if (hi_ok) {
            buf_store16((f32x4){v[8], v[9], v[10], v[11]} * kLn2, sr, elem * 4 + 64);
            buf_store16((f32x4){v[12], v[13], v[14], v[15]} * kLn2, sr, elem * 4 + 80);
          }
        }
        if (2 * mb < KSM) nxt[2 * mb][nb] = pack8(v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]);
        if (2 * mb + 1 < KSM)
          nxt[2 * mb + 1][nb] = pack8(v[8], v[9], v[10], v[11], v[12], v[13], v[14], v[15]);
      }
    }
  }
}

// Layers l .. L-1, ping-ponging between two register buffers.  The x rows of
// the wave's next block are requested when the last layer starts (the layer-0
// buffer is dead by then), so their latency hides behind the last layer.
template <class N, int l, int NB, bool STASH, int KSM>
__device__ __forceinline__ void run_chain(const BlockIO& io, const f16x8* __restrict__ lds,
                                          f16x8 (&xa)[N::ks(0)][NB], f16x8 (&cur)[KSM][NB],
                                          f16x8 (&oth)[KSM][NB], rsrc_t next_x, int lane) {
  if constexpr (l == N::L - 1) {
    MLPMK_SCHED_FENCE();  // keep the prefetch from being hoisted into layer L-2
    load_rows<N::ks(0), NB>(xa, next_x, lane & 31, lane >> 5);
    run_layer<N, l, NB, STASH, KSM>(io, lds, cur, oth, lane);
  } else {
    run_layer<N, l, NB, STASH, KSM>(io, lds, cur, oth, lane);
    run_chain<N, l + 1, NB, STASH, KSM>(io, lds, xa, oth, cur, next_x, lane);
  }
}

template <class N, int NB, bool STASH, int NW>
__global__ __launch_bounds__(NW * 64) void fwd_kernel(FwdParams p) {
  static_assert(N::valid(), "unsupported widths");
  constexpr int KSM = N::ksmax();
  constexpr int KS0 = N::ks(0);
  constexpr int ROWS = 32 * NB;
  __shared__ f16x8 lds[N::nfrag() * 64];
  stage_weights<N, NW * 64>(p, lds);
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int64_t nblk = (p.M + ROWS - 1) / ROWS;
  const int64_t stride = (int64_t)gridDim.x * NW;
  int64_t blk = (int64_t)blockIdx.x * NW + wid;
  if (blk >= nblk) return;  // no barrier follows

  f16x8 xa[KS0][NB];
  f16x8 b0[KSM][NB], b1[KSM][NB];
  load_rows<KS0, NB>(xa, block_io<N, false, ROWS>(p, blk * ROWS).x, lane & 31, lane >> 5);
  for (; blk < nblk; blk += stride) {
    const BlockIO io = block_io<N, STASH, ROWS>(p, blk * ROWS);
    // Past the end the resource is empty: the prefetch then reads zeros.
    const rsrc_t next_x = block_io<N, false, ROWS>(p, (blk + stride) * ROWS).x;
    if constexpr (KS0 == KSM) {
      run_layer<N, 0, NB, STASH, KSM>(io, lds, xa, b0, lane);
    } else {
      f16x8 xin[KSM][NB];
#pragma unroll
      for (int s = 0; s < KS0; ++s)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) xin[s][nb] = xa[s][nb];
      run_layer<N, 0, NB, STASH, KSM>(io, lds, xin, b0, lane);
    }
    run_chain<N, 1, NB, STASH, KSM>(io, lds, xa, b0, b1, next_x, lane);
  }
}

}  // namespace mlpmk

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------
#include "host_common.h"

namespace mlpmk {

typedef Net<128, 128, 128, 128> Net3L128;
typedef Net<128, 128, 128, 128, 128, 128> Net5L128;
typedef Net<32, 64, 64, 16> NetNarrow;

template <class N>
static bool dims_match(int L, const int* dims) {
  if (L != N::L) return false;
  for (int i = 0; i <= L; ++i)
    if (dims[i] != N::d[i]) return false;
  return true;
}

template <class N, int NB, bool STASH, int NW>
static int launch_fwd(const FwdParams& p, hipStream_t st) {
  constexpr int kMaxDev = 64;
  static int occ_cache[kMaxDev];  // 0 = unknown; benign race (idempotent value)
  int cus = 0;
  int rc = current_device_cus(&cus);
  if (rc != MLPMK_OK) return rc;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  const void* kern = reinterpret_cast<const void*>(&fwd_kernel<N, NB, STASH, NW>);
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
  (void)hipGetLastError();
  hipLaunchKernelGGL((fwd_kernel<N, NB, STASH, NW>), dim3(grid), dim3(NW * 64), 0, st, p);
  e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "fwd kernel launch");
  return MLPMK_OK;
}

template <class N, int NB, int NW>
static int launch_fwd_any(const FwdParams& p, bool stash, hipStream_t st) {
  return stash ? launch_fwd<N, NB, true, NW>(p, st) : launch_fwd<N, NB, false, NW>(p, st);
}

bool fwd_supported_dims(int L, const int* dims) {
  return dims_match<Net3L128>(L, dims) || dims_match<Net5L128>(L, dims) ||
         dims_match<NetNarrow>(L, dims);
}

int fwd_dispatch(int L, const int* dims, const FwdParams& p, bool stash, hipStream_t st) {
  if (dims_match<Net3L128>(L, dims)) return launch_fwd_any<Net3L128, 2, 8>(p, stash, st);
  if (dims_match<Net5L128>(L, dims)) return launch_fwd_any<Net5L128, 2, 8>(p, stash, st);
  if (dims_match<NetNarrow>(L, dims)) return launch_fwd_any<NetNarrow, 2, 8>(p, stash, st);
  return fail(MLPMK_ERR_UNSUPPORTED_SHAPE, "no forward kernel for these widths");
}

}  // namespace mlpmk
