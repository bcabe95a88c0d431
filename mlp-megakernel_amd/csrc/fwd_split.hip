// Feature-split forward megakernel for gfx950 (MI355X): the same math as
// fwd.hip (the reference's _fused_mlp_recompute, /root/reference/kernel.py:60-123,
// and its training-forward variant, /root/reference/mlp_fused.md:52-61), mapped
// for short per-block latency instead of per-wave independence.
//
//  * A workgroup of NWV waves (one per SIMD; NWV = the widest layer's count of
//    32-feature output blocks, 4 for 128-wide layers) computes one 32-row block
//    at a time: wave w owns output features [32w, 32w + 32) of every layer, so
//    each wave runs a quarter of the block's MFMAs and softplus values.
//  * A wave keeps only its own weight fragments (mb = w), in registers for the
//    whole kernel: 8 fragments (32 VGPRs) per 128-wide layer.  They are
//    staged once, with 16-byte row loads transposed through LDS.
//  * Layers exchange activations through two LDS tiles of [32 rows][features]
//    fp16 (8 KiB each at 128 features): a wave writes its 32 features of each
//    row, a workgroup barrier, and every wave reads the whole row as its next
//    B operand.  Output rows leave through a tile as whole 128-byte lines.
//  * Persistent grid: workgroup b walks blocks b, b + G, ... with the next
//    block's x rows in flight; several workgroups share a CU, so one's
//    barrier waits and MFMA chains overlap another's softplus.
//
// Against fwd.hip's one-block-per-wave kernel the per-block latency is ~4x
// shorter (one chain of 8 MFMAs and 16 softplus values per lane per layer),
// which is what small batches (few blocks, launch-latency bound) and the end
// of a large batch (the last blocks of each workgroup) pay for.
//
// Softplus, its base-2 scaling and the overflow handling are those of fwd.hip:
// sp2(u) = log2(1 + 2^u) with W_1 pre-scaled by log2(e) and W_L by ln(2); a
// block whose fast sp2 overflowed anywhere (every wave votes through LDS)
// is recomputed by the whole workgroup in the exact form.
#include "device_common.h"
#include "host_common.h"
#include "params.h"

namespace mlpmk {
namespace fsplit {

template <class N>
struct Geo {
  static constexpr int L = N::L;
  static constexpr int nwv() {
    int m = 0;
    for (int l = 0; l < L; ++l) m = N::mbs(l) > m ? N::mbs(l) : m;
    return m;
  }
  static constexpr int NWV = nwv();
  // Tile width: the widest layer input (every layer reads its input from a tile).
  static constexpr int tw() {
    int m = 0;
    for (int l = 0; l < L; ++l) m = N::d[l] > m ? N::d[l] : m;
    return m;
  }
  static constexpr int TW = tw();
  static constexpr int CH = TW / 8;     // 16-byte chunks per tile row
  static constexpr int TILE = 32 * CH;  // chunks per tile
  static constexpr int KSM = N::ksmax();
  // Output rows go through a tile when each wave's share of them is a whole
  // number of 16-byte stores per lane; otherwise lanes store their features.
  static constexpr bool STAGE_OUT =
      N::d[L] <= TW && N::d[L] % 32 == 0 && 32 % NWV == 0 && ((32 / NWV) * (N::d[L] / 8)) % 64 == 0;
  // Start-up scratch (each wave's transposed fragments of one layer), overlaid on the tiles.
  static constexpr int SCRATCH = NWV * KSM * 64;
  static constexpr int LDS_CHUNKS = 2 * TILE > SCRATCH ? 2 * TILE : SCRATCH;
  static constexpr bool valid() {
    if (!N::valid() || L % 2 != 1 || TW > 128 || (CH & (CH - 1)) != 0) return false;
    if (N::d[0] % 32 != 0) return false;
    for (int l = 1; l < L; ++l)
      if (N::d[l] % 32 != 0) return false;  // hidden widths in whole 32-feature blocks
    return true;
  }
};

// Tile slot of (row, 16-byte chunk): XOR-swizzled so that the 8 rows of an
// 8-lane LDS access group hit 8 distinct chunks (distinct banks).
template <int CH>
__device__ __forceinline__ int slot(int row, int chunk) {
  return row * CH + (chunk ^ (row & (CH - 1)));
}

// Scale folded into the staged W_l (log2 e on the first layer, ln 2 on the
// last), exactly as fwd.hip stages it.
template <class N>
__device__ __forceinline__ float wscale(int l) {
  return (l == 0 ? kLog2e : 1.0f) * (l == N::L - 1 ? kLn2 : 1.0f);
}

// Weight fragments of one wave: fr[l][s] = fragment (mb = w, K-step s) of layer l.
template <class N>
struct Frags {
  f16x8 fr[N::L][N::ksmax()];
};

// Start-up, first half: lane (kb, cb) = (lane / 4, lane % 4) loads rows
// 8kb .. 8kb+7 of W_l, columns 32w + 8cb .. +8 (16 bytes each).
template <class N, int l>
__device__ __forceinline__ void frag_load(const FwdParams& p, f16x8 (&r)[8], int w, int lane) {
  constexpr int Nout = N::d[l + 1], TASKS = (N::d[l] / 8) * 4;
  const int kb = lane >> 2, cb = lane & 3;
  const int col = 32 * w + 8 * cb;
  if (lane < TASKS && col < Nout) {
    const f16* src = p.w[l] + (int64_t)(8 * kb) * Nout + col;
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = *reinterpret_cast<const f16x8*>(src + (int64_t)j * Nout);
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = f16x8{};
  }
}

// Start-up, second half: transpose the 8 x 8 tile in registers and scatter its
// columns into this wave's scratch as fragment lanes, then read back the
// wave's own fragments.  Column q of task (kb, cb) is feature
// 32w + 8cb + q = outfeat(w, i) for i = 16(cb/2) + 8(q/4) + 4(cb%2) + q%4,
// and rows 8kb + j are K = 16s + 8g + j for s = kb/2, g = kb%2.
template <class N, int l>
__device__ __forceinline__ void frag_build(f16x8 (&fr)[N::ksmax()], const f16x8 (&r)[8], f16x8* scratch,
                                           int lane) {
  constexpr int TASKS = (N::d[l] / 8) * 4, KS = N::ks(l);
  const float sc = wscale<N>(l);
  if (lane < TASKS) {
    const int kb = lane >> 2, cb = lane & 3;
    const int s = kb >> 1, g = kb & 1;
    const int ibase = 16 * (cb >> 1) + 4 * (cb & 1);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int i = ibase + 8 * (q >> 2) + (q & 3);
      f16x8 v;
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = scaled_weight<N::bf>(r[j][q], sc);
      scratch[s * 64 + 32 * g + i] = v;
    }
  }
  // The scratch is this wave's own; LDS runs one wave's operations in order,
  // so only the compiler needs fences around the exchange.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int s = 0; s < KS; ++s) fr[s] = scratch[s * 64 + lane];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

template <class N, int l = 0>
__device__ __forceinline__ void frag_load_all(const FwdParams& p, f16x8 (&r)[N::L][8], int w, int lane) {
  if constexpr (l < N::L) {
    if (w < N::mbs(l)) frag_load<N, l>(p, r[l], w, lane);
    frag_load_all<N, l + 1>(p, r, w, lane);
  }
}

template <class N, int l = 0>
__device__ __forceinline__ void frag_build_all(Frags<N>& f, const f16x8 (&r)[N::L][8], f16x8* scratch, int w,
                                               int lane) {
  if constexpr (l < N::L) {
    if (w < N::mbs(l)) frag_build<N, l>(f.fr[l], r[l], scratch, lane);
    frag_build_all<N, l + 1>(f, r, scratch, w, lane);
  }
}

// Every layer's loads are issued before the first transpose: one memory
// round trip for the whole start-up.
template <class N>
__device__ __forceinline__ void stage_frags(const FwdParams& p, Frags<N>& f, f16x8* scratch, int w, int lane) {
  f16x8 r[N::L][8];
  frag_load_all<N>(p, r, w, lane);
  frag_build_all<N>(f, r, scratch, w, lane);
}

// x rows of one block: wave w loads the 32-feature slices xb = w, w + NWV, ...
// (lane (n, g): features 32xb + 8g + [0..7] and 32xb + 16 + 8g + [0..7] of row n).
template <class N>
struct XRegs {
  static constexpr int XB = N::d[0] / 32;
  static constexpr int XBW = (XB + Geo<N>::NWV - 1) / Geo<N>::NWV;
  i32x4 v[XBW][2];
};

template <class N>
__device__ __forceinline__ void load_x(XRegs<N>& x, const FwdParams& p, int64_t b, int w, int n, int g) {
  constexpr int D0 = N::d[0];
  const int64_t row0 = b * 32;
  const int64_t left = p.M - row0;
  const uint32_t rows = (uint32_t)(left < 32 ? (left > 0 ? left : 0) : 32);
  const rsrc_t xr = make_rsrc(p.x + row0 * D0, rows * D0 * 2u);
#pragma unroll
  for (int k = 0; k < XRegs<N>::XBW; ++k) {
    const int xb = w + k * Geo<N>::NWV;
    if (xb < XRegs<N>::XB) {
      const int off = (n * D0 + 32 * xb + 8 * g) * 2;
      x.v[k][0] = __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0);
      x.v[k][1] = __builtin_amdgcn_raw_buffer_load_b128(xr, off + 32, 0, 0);
    }
  }
}

template <class N>
__device__ __forceinline__ void write_x(const XRegs<N>& x, i32x4* tile, int w, int n, int g) {
  constexpr int CH = Geo<N>::CH;
#pragma unroll
  for (int k = 0; k < XRegs<N>::XBW; ++k) {
    const int xb = w + k * Geo<N>::NWV;
    if (xb < XRegs<N>::XB) {
      tile[slot<CH>(n, 4 * xb + g)] = x.v[k][0];
      tile[slot<CH>(n, 4 * xb + 2 + g)] = x.v[k][1];
    }
  }
}

// Layer l of one block for wave w: B operand (all input features of the 32
// rows) from tile `tin`, one chain of K-steps against the wave's fragments,
// then softplus (hidden layers; fp32 stash optional) or the output values,
// written as this wave's 32 features of each row into `tout`, or stored
// straight to `out` when output rows are not staged.  EXACT as in fwd.hip:
// overflowed sp2 replaced by u, hidden values handed on halved, later
// accumulators doubled.
template <class N, int l, bool STASH, bool EXACT>
__device__ __forceinline__ void layer(const FwdParams& p, const Frags<N>& f, const i32x4* tin, i32x4* tout,
                                      int64_t row0, uint32_t rows, int w, int n, int g, f16x2& m) {
  using G = Geo<N>;
  constexpr int CH = G::CH, KS = N::ks(l), Nout = N::d[l + 1];
  constexpr bool LAST = l == N::L - 1;
  if (w >= N::mbs(l)) return;  // wave-uniform: no output block of this layer
  f16x8 bv[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) bv[s] = __builtin_bit_cast(f16x8, tin[slot<CH>(n, 2 * s + g)]);
  f32x16 acc = {};
#pragma unroll
  for (int s = 0; s < KS; ++s) acc = mfma32x32x16<N::bf>(f.fr[l][s], bv[s], acc);
  constexpr float kIn = (EXACT && l > 0) ? 2.0f : 1.0f;
  const bool lo_ok = 32 * w + 16 <= Nout, hi_ok = 32 * w + 32 <= Nout;
  const uint32_t elem = (uint32_t)(n * Nout + 32 * w + 8 * g);
  if constexpr (LAST) {
    const f32x16 v = acc * kIn;  // ln 2 is folded into the staged W_L
    const f16x8 lo = pack8<N::bf>(v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]);
    const f16x8 hi = pack8<N::bf>(v[8], v[9], v[10], v[11], v[12], v[13], v[14], v[15]);
    if constexpr (G::STAGE_OUT) {
      tout[slot<CH>(n, 4 * w + g)] = __builtin_bit_cast(i32x4, lo);
      tout[slot<CH>(n, 4 * w + 2 + g)] = __builtin_bit_cast(i32x4, hi);
    } else {
      const rsrc_t orr = make_rsrc(p.out + row0 * Nout, rows * Nout * 2u);
      if (lo_ok) buf_store16<kOutStore<STASH>>(lo, orr, elem * 2);
      if (hi_ok) buf_store16<kOutStore<STASH>>(hi, orr, elem * 2 + 32);
    }
  } else {
    const f32x16 u = acc * kIn;  // log2 e is folded into the staged W_1: u in base-2 units
    float s[16], q[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      s[e] = EXACT ? sp2_fix(u[e], sp2(u[e])) : sp2(u[e]);
      q[e] = EXACT ? 0.5f * s[e] : s[e];
    }
    const f16x8 lo = pack8<N::bf>(q[0], q[1], q[2], q[3], q[4], q[5], q[6], q[7]);
    const f16x8 hi = pack8<N::bf>(q[8], q[9], q[10], q[11], q[12], q[13], q[14], q[15]);
    if constexpr (!EXACT) m = sp2_track<true>(m, lo, hi);
    if constexpr (STASH) {
      const rsrc_t sr = p.stash[l] ? make_rsrc(p.stash[l] + row0 * Nout, rows * Nout * 4u)
                                   : make_rsrc(nullptr, 0u);  // not requested: every store dropped
      float h[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) h[e] = s[e] * kLn2;
      buf_store16<kStashStore>((f32x4){h[0], h[1], h[2], h[3]}, sr, elem * 4);
      buf_store16<kStashStore>((f32x4){h[4], h[5], h[6], h[7]}, sr, elem * 4 + 16);
      buf_store16<kStashStore>((f32x4){h[8], h[9], h[10], h[11]}, sr, elem * 4 + 64);
      buf_store16<kStashStore>((f32x4){h[12], h[13], h[14], h[15]}, sr, elem * 4 + 80);
    }
    tout[slot<CH>(n, 4 * w + g)] = __builtin_bit_cast(i32x4, lo);
    tout[slot<CH>(n, 4 * w + 2 + g)] = __builtin_bit_cast(i32x4, hi);
  }
}

// All layers of one block, input in tile 0; layer l reads tile l % 2 and
// writes tile (l + 1) % 2, with a workgroup barrier after every layer but the
// last (the caller's barrier follows it).  Returns the running maximum of the
// block's fast-form sp2 values on this wave.
template <class N, bool STASH, bool EXACT, int l = 0>
__device__ __forceinline__ void layers(const FwdParams& p, const Frags<N>& f, i32x4* tiles, int64_t row0,
                                       uint32_t rows, int w, int n, int g, f16x2& m) {
  if constexpr (l < N::L) {
    constexpr int T = Geo<N>::TILE;
    layer<N, l, STASH, EXACT>(p, f, tiles + (l % 2) * T, tiles + ((l + 1) % 2) * T, row0, rows, w, n, g, m);
    if constexpr (l + 1 < N::L) {
      __syncthreads();
      layers<N, STASH, EXACT, l + 1>(p, f, tiles, row0, rows, w, n, g, m);
    }
  }
}

// Output rows of the block from the output tile, whole rows per instruction:
// wave w stores rows [w * 32 / NWV, (w + 1) * 32 / NWV).
template <class N, bool STASH>
__device__ __forceinline__ void store_rows(const FwdParams& p, const i32x4* tile, int64_t row0, uint32_t rows,
                                           int w, int lane) {
  using G = Geo<N>;
  constexpr int OUT = N::d[N::L], OC = OUT / 8, RPW = 32 / G::NWV, PER = RPW * OC / 64;
  const rsrc_t orr = make_rsrc(p.out + row0 * OUT, rows * OUT * 2u);
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int q = 64 * k + lane;
    const int row = w * RPW + q / OC, c = q % OC;
    __builtin_amdgcn_raw_buffer_store_b128(tile[slot<G::CH>(row, c)], orr, (row * OUT + 8 * c) * 2, 0,
                                           kOutStore<STASH>);
  }
}

template <class N, bool STASH>
__global__ __launch_bounds__(Geo<N>::NWV * 64) void fwd_split_kernel(FwdParams p) {
  using G = Geo<N>;
  static_assert(G::valid(), "unsupported widths for the feature-split kernel");
  constexpr int L = N::L;
  __shared__ i32x4 lds[G::LDS_CHUNKS];
  __shared__ unsigned int redo[2];  // per block parity: some wave's fast sp2 overflowed
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 31, g = lane >> 5;
  const int64_t nblk = (p.M + 31) / 32;
  int64_t b = blockIdx.x;
  if (b >= nblk) return;  // the whole workgroup, before any barrier
  if (threadIdx.x == 0) redo[0] = redo[1] = 0;
  XRegs<N> xr;
  load_x<N>(xr, p, b, w, n, g);
  Frags<N> f;
  stage_frags<N>(p, f, reinterpret_cast<f16x8*>(lds) + w * G::KSM * 64, w, lane);
  __syncthreads();  // the scratch is the tiles' memory
  i32x4* const tiles = lds;
  constexpr int OUTT = (L % 2) * G::TILE;  // the last layer writes tile L % 2 (= 1)
  int par = 0;
  for (;;) {
    const int64_t next = b + gridDim.x;
    const int64_t row0 = b * 32;
    const int64_t left = p.M - row0;
    const uint32_t rows = (uint32_t)(left < 32 ? left : 32);
    write_x<N>(xr, tiles, w, n, g);
    load_x<N>(xr, p, next, w, n, g);  // past the end: an empty resource, reads zeros
    __syncthreads();
    // Block b + 1 (parity par ^ 1) votes after this barrier; its flag was last
    // read after the previous block's final barrier, before this one.
    if (threadIdx.x == 0) redo[par ^ 1] = 0;
    f16x2 m = f16x2{};
    layers<N, STASH, false>(p, f, tiles, row0, rows, w, n, g, m);
    if (sp2_overflowed<N::bf>(m) && lane == 0) redo[par] = 1;
    __syncthreads();
    if (__builtin_expect(redo[par] != 0, 0)) {
      // Exact recompute by the whole workgroup (the flag is the same for all
      // waves).  Tile 0 is free: the last layer read it before the barrier.
      XRegs<N> xb;
      load_x<N>(xb, p, b, w, n, g);
      write_x<N>(xb, tiles, w, n, g);
      __syncthreads();
      layers<N, STASH, true>(p, f, tiles, row0, rows, w, n, g, m);
      __syncthreads();
    }
    if constexpr (G::STAGE_OUT) store_rows<N, STASH>(p, tiles + OUTT, row0, rows, w, lane);
    par ^= 1;
    b = next;
    if (b >= nblk) break;
  }
}

}  // namespace fsplit

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------

template <class N, bool STASH>
static int launch_split_t(const FwdParams& p, hipStream_t st, LaunchInfo* info) {
  using G = fsplit::Geo<N>;
  constexpr int kMaxDev = 64;
  static int occ_cache[kMaxDev];  // 0 = unknown; benign race (idempotent value)
  int cus = 0;
  int rc = current_device_cus(&cus);
  if (rc != MLPMK_OK) return rc;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  const void* kern = reinterpret_cast<const void*>(&fsplit::fwd_split_kernel<N, STASH>);
  int occ = (dev >= 0 && dev < kMaxDev) ? occ_cache[dev] : 0;
  if (occ <= 0) {
    rc = kernel_occupancy(kern, G::NWV * 64, &occ);
    if (rc != MLPMK_OK) return rc;
    if (dev >= 0 && dev < kMaxDev) occ_cache[dev] = occ;
  }
  const int64_t nblk = (p.M + 31) / 32;
  const int64_t cap = (int64_t)cus * occ;
  const int grid = (int)(nblk < cap ? nblk : cap);
  if (info) {
    *info = LaunchInfo{MLPMK_KERNEL_FEATURE_SPLIT, 32, G::NWV, grid, occ};
    return MLPMK_OK;
  }
  (void)hipGetLastError();
  hipLaunchKernelGGL((fsplit::fwd_split_kernel<N, STASH>), dim3(grid), dim3(G::NWV * 64), 0, st, p);
  e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "fwd split kernel launch");
  return MLPMK_OK;
}

typedef Net<128, 128, 128, 128> SNet3L128;
typedef Net<128, 128, 128, 128, 128, 128> SNet5L128;
typedef Net<32, 64, 64, 16> SNetNarrow;

template <class N>
static bool split_dims_match(int L, const int* dims) {
  if (L != N::L) return false;
  for (int i = 0; i <= L; ++i)
    if (dims[i] != N::d[i]) return false;
  return true;
}

// Largest batch, in 32-row blocks per CU, that runs the feature-split kernel.
// Its per-block latency is ~4x shorter than that of fwd.hip's
// one-block-per-wave kernel, which wins once each CU has a few blocks to
// overlap (20-launch graph replay, us per launch, split / one-block-per-wave):
//   3L-128  M = 8192 (1 per CU) 6.2 / 7.9,   M = 16384 (2 per CU) 8.6 / 8.0
//   5L-128  M = 8192 9.1 / 12.4,             M = 16384 13.0 / 13.3
//   narrow  M = 8192 4.7 / 6.6,              M = 16384 5.3 / 6.6
#ifndef MLPMK_SPLIT_BLOCKS_PER_CU_3L
#define MLPMK_SPLIT_BLOCKS_PER_CU_3L 1
#endif
#ifndef MLPMK_SPLIT_BLOCKS_PER_CU
#define MLPMK_SPLIT_BLOCKS_PER_CU 2
#endif

template <class N>
static int split_if_small(const FwdParams& p, bool stash, hipStream_t st, int cus, int per_cu, LaunchInfo* info) {
  if ((p.M + 31) / 32 > (int64_t)per_cu * cus) return MLPMK_ERR_UNSUPPORTED_SHAPE;
  return stash ? launch_split_t<N, true>(p, st, info) : launch_split_t<N, false>(p, st, info);
}

// Launches the feature-split kernel when one exists for these widths and the
// batch is small enough; otherwise returns MLPMK_ERR_UNSUPPORTED_SHAPE without
// recording an error, and the caller runs fwd.hip's kernels.  B: bf16 tensors.
template <bool B>
static int fwd_split_dispatch_t(int L, const int* dims, const FwdParams& p, bool stash, hipStream_t st, int cus,
                                LaunchInfo* info) {
  if (split_dims_match<SNet3L128>(L, dims))
    return split_if_small<typename ElemNet<B, SNet3L128>::type>(p, stash, st, cus, MLPMK_SPLIT_BLOCKS_PER_CU_3L, info);
  if (split_dims_match<SNet5L128>(L, dims))
    return split_if_small<typename ElemNet<B, SNet5L128>::type>(p, stash, st, cus, MLPMK_SPLIT_BLOCKS_PER_CU, info);
  if (split_dims_match<SNetNarrow>(L, dims))
    return split_if_small<typename ElemNet<B, SNetNarrow>::type>(p, stash, st, cus, MLPMK_SPLIT_BLOCKS_PER_CU, info);
  return MLPMK_ERR_UNSUPPORTED_SHAPE;
}

int fwd_split_dispatch(int L, const int* dims, const FwdParams& p, bool stash, bool bf, hipStream_t st, int cus,
                       LaunchInfo* info) {
  return bf ? fwd_split_dispatch_t<true>(L, dims, p, stash, st, cus, info)
            : fwd_split_dispatch_t<false>(L, dims, p, stash, st, cus, info);
}

}  // namespace mlpmk
