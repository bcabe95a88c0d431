// Forward megakernel for fp32 tensors on gfx950 (MI355X): the reference's
// INPUT_DTYPE = fp32 kernels (/root/reference/mlp_fused.md:159-166), whose
// launcher passes fp32 x on (/root/reference/kernel.py:130-138) and whose
// tl.dot rounds fp32 operands to TF32 (10-bit significand, fp32 exponent
// range).
//
// Every MFMA operand -- x, the weights and the hidden activations -- is
// split into bf16 hi + lo (hi = bf16(v), lo = bf16(v - hi); the hidden
// activations, all >= 0, with a truncated hi) and each product
// is hi*hi + hi*lo + lo*hi on v_mfma_f32_32x32x16_bf16: fp32's exponent
// range (|x| or h past fp16's 65,504 are ordinary values here) and a ~16-bit
// significand, with fp32 accumulation, softplus and output rows.  The fp32
// backward (bwd_tp.hip) uses the same operands, so a training step keeps
// fp32's range end to end.
//
// Mapping: the feature split of fwd_split.hip, in the transposed
// orientation (MFMA M = features, N = rows, K = input features): 32-row
// blocks, persistent over the batch; wave w of a layer's group computes
// output features [32w, 32w + 32) of that layer, its A fragments (hi and
// lo) resident in AGPRs, which the MFMA reads directly.  Layers hand their
// activations on as B operands through LDS tiles [32 rows][features] (hi,
// lo).
//
// 2 and 3 layers (fwd_x3p_kernel): a layer pipeline.  One group of NWV
// waves per layer (one wave of each group per SIMD): in step t group r runs
// layer r of block t - r, and every hand-over crosses the one barrier of a
// step, so the waves of a SIMD overlap one's softplus with another's MFMA
// chains; x reaches the layer-0 group through an LDS tile that the whole
// workgroup loads and splits once.  A single wave per SIMD running all
// layers waits out every chain, barrier and softplus in turn: 0.511 against
// 0.326 ms at 3 x 128 and 1M rows.
// 4 and 5 layers (fwd_x3_kernel, whose fragments need the whole register
// file): one wave per output block runs every layer of a block in turn.
//
// Softplus in base 2: u = z log2(e), softplus(z) = ln2 * sp2(u) with sp2(u)
// = log2(1 + 2^u), and u itself where 2^u overflows (u >= 128, z > 88.7; the
// reference's threshold branch, kernel.py:108, gives z there too).  The two
// scales are folded into the first and last layers' weights (fscale), so a
// hidden activation is one exp2 and one log2.  The fp32 stash (training)
// holds softplus(z) as the backward reads it.
#include "device_common.h"
#include "host_common.h"
#include "params.h"
#include "tp_common.h"

namespace mlpmk {
namespace tp {

template <class N>
struct FxGeo {
  static constexpr int L = N::L;
  static constexpr int blocks(int l) { return (N::d[l + 1] + 31) / 32; }  // output blocks of layer l
  static constexpr int ks(int l) { return N::d[l] / 16; }                 // K-steps: input features
  static constexpr int nwv() {
    int m = 1;
    for (int l = 0; l < L; ++l) m = blocks(l) > m ? blocks(l) : m;
    return m;
  }
  static constexpr int ksm() {
    int m = 1;
    for (int l = 0; l < L; ++l) m = ks(l) > m ? ks(l) : m;
    return m;
  }
  static constexpr int tw() {  // exchange tile width: hidden widths, a power of two >= 32
    int m = 32;
    for (int l = 1; l < L; ++l)
      while (m < N::d[l]) m *= 2;
    return m;
  }
  static constexpr int pow2_32(int v) {
    int m = 32;
    while (m < v) m *= 2;
    return m;
  }
  static constexpr int NWV = nwv(), KSM = ksm(), TW = tw(), CH = TW / 8;
  static constexpr int CHX = pow2_32(N::d[0]) / 8;  // chunks of 8 features per x-tile row
  static constexpr bool PIPE = L <= 3;  // the layer pipeline: one wave group per layer
  static constexpr int THREADS = (PIPE ? L : 1) * NWV * 64;
  static constexpr bool valid() {
    for (int i = 0; i < L; ++i)
      if (N::d[i] > 128 || N::d[i] % 16 != 0) return false;
    return L >= 2 && N::d[L] <= 128;
  }
};

// Scale folded into W_l: log2 e on the first layer, ln 2 on the last.  The
// first layer's sums then come out as u = z log2 e, hidden layers carry
// g = sp2(u) = softplus(z) / ln 2 into unscaled weights (the ln 2 of one
// layer and the log2 e of the next cancel), and the last layer's ln 2 turns
// its g inputs back into h.
template <class N>
__device__ __forceinline__ float fscale(int l) {
  return (l == 0 ? kLog2e : 1.0f) * (l == N::L - 1 ? kLn2 : 1.0f);
}

// One exchange tile: [hi, lo][32 rows * CH chunks of 8 features].
template <int CH>
using XTile = f16x8[2][32 * CH];

// What a wave of either kernel does with one block of one layer.  w is the
// wave's output block (features [32w, 32w + 32)).
template <class N, bool STASH>
struct FxOps {
  using G = FxGeo<N>;
  static constexpr int L = N::L, CH = G::CH, EM = EM_F32;
  const FwdParams& p;
  int n, g, w;

  // Whether this wave has output features in layer l (always, for fixed
  // networks whose every layer has NWV output blocks).
  template <int l>
  __device__ __forceinline__ bool owns() const {
    if constexpr (!N::gen && G::blocks(l) == G::NWV) return true;
    return 32 * w < dimw<N>(p, l + 1);
  }

  // Fragment (block w, K-step s) of layer l, scaled: lane (i, g) holds
  // fscale(l) * W_l[16s + 8g + j][outfeat(w, i)], j = 0..7 -- for fixed
  // (s, g, j) the 32 lanes of a half-wave read 32 consecutive columns of one
  // row (128 bytes).  Rows past the true input width read zeros through the
  // resource; columns past the true output width are masked.  The fragments
  // are then pinned to AGPRs: left to itself the allocator parks them there
  // and copies them back to VGPRs before every MFMA.
  template <int l>
  __device__ __forceinline__ void load_frags(Opnd (&f)[G::KSM]) const {
    const int K = dimw<N>(p, l), Nout = dimw<N>(p, l + 1);
    const rsrc_t r = make_rsrc(p.w[l], (uint32_t)(K * Nout * 4));
    const int col = outfeat(w, n);
    const bool ok = !N::gen || col < Nout;
#pragma unroll
    for (int s = 0; s < G::ks(l); ++s) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int row = 16 * s + 8 * g + j;
        v[j] = ok ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (row * Nout + col) * 4, 0, 0)) *
                        fscale<N>(l)
                  : 0.0f;
      }
      f[s] = make_op<EM>(v);
      asm volatile("" : "+a"(f[s].h), "+a"(f[s].l));
    }
  }

  // x rows from row0, as loaded (lane (n, g), K-step s: x[row n][16s + 8g +
  // 0..7]).  Past the batch the resource is empty and the rows read as zeros.
  __device__ __forceinline__ void load_x(f32x4 (&xr)[G::ks(0)][2], int64_t row0) const {
    const int D = dimw<N>(p, 0);
    const rsrc_t r = make_rsrc(reinterpret_cast<const float*>(p.x) + row0 * D, rows_at(p.M, row0, 32) * D * 4u);
#pragma unroll
    for (int s = 0; s < G::ks(0); ++s) {
      const uint32_t e = (uint32_t)(n * D + 16 * s + 8 * g) * 4;
      xr[s][0] = buf_load16<f32x4>(r, e);
      xr[s][1] = buf_load16<f32x4>(r, e + 16);
    }
  }
  // Loaded x rows as split B operands of layer 0.
  __device__ __forceinline__ void x_operands(const f32x4 (&xr)[G::ks(0)][2], Opnd (&X)[G::KSM]) const {
    const int D = dimw<N>(p, 0);
#pragma unroll
    for (int s = 0; s < G::ks(0); ++s) {
      const float v[8] = {xr[s][0][0], xr[s][0][1], xr[s][0][2], xr[s][0][3],
                          xr[s][1][0], xr[s][1][1], xr[s][1][2], xr[s][1][3]};
      X[s] = make_op<EM>(v);
      if (N::gen && 16 * s + 8 * g >= D) X[s] = Opnd{f16x8{}, f16x8{}};
    }
  }

  // Layer 0's B operands (row n) from an x tile (CHX chunks per row).
  __device__ __forceinline__ void read_xtile(const XTile<G::CHX>& t, Opnd (&X)[G::KSM]) const {
    const int D = dimw<N>(p, 0);
#pragma unroll
    for (int s = 0; s < G::ks(0); ++s) {
      X[s].h = t[0][slot<G::CHX>(n, 2 * s + g)];
      X[s].l = t[1][slot<G::CHX>(n, 2 * s + g)];
      if (N::gen && 16 * s + 8 * g >= D) X[s] = Opnd{f16x8{}, f16x8{}};
    }
  }

  // Layer l's B operands (row n) from a tile holding layer l's input.
  template <int l>
  __device__ __forceinline__ void read_tile(const XTile<CH>& t, Opnd (&B)[G::KSM]) const {
    const int Wd = dimw<N>(p, l);
#pragma unroll
    for (int s = 0; s < G::ks(l); ++s) {
      B[s].h = t[0][slot<CH>(n, 2 * s + g)];
      B[s].l = t[1][slot<CH>(n, 2 * s + g)];
      // (past the true width the tile holds stale values: zero operands)
      if (N::gen && 16 * s + 8 * g >= Wd) B[s] = Opnd{f16x8{}, f16x8{}};
    }
  }

  // 16 fp32 values of row n (features 32w + 8g + [0..7] and 32w + 16 + 8g +
  // [0..7]) into a [M, W] fp32 tensor; features past W are dropped.
  __device__ __forceinline__ void store_row16(float* base, int W, int64_t row0, const float (&v)[16]) const {
    const rsrc_t r = make_rsrc(base + row0 * W, rows_at(p.M, row0, 32) * W * 4u);
    const int c0 = 32 * w + 8 * g;
    if (!N::gen || W % 8 == 0) {
      const uint32_t e = (uint32_t)(n * W + c0);
      if (!N::gen || c0 < W) store8<EM>(r, e, v);
      if (!N::gen || c0 + 16 < W) store8<EM>(r, e + 16, v + 8);
      return;
    }
    // Output widths that are not a multiple of 8: element by element.
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int c = c0 + 16 * h + j;
        if (c < W) __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, v[8 * h + j]), r, (n * W + c) * 4, 0, 0);
      }
  }

  // Layer l of one 32-row block for an owning wave: the MFMA chain over the
  // layer's K-steps, then either the hidden activation (g = softplus(z) /
  // ln 2 into tile `out`, h into the stash) or the output rows.
  template <int l>
  __device__ __forceinline__ void compute(const Opnd (&f)[G::KSM], const Opnd (&in)[G::KSM], int64_t row0,
                                          XTile<CH>& out) const {
    f32x16 acc = {};
#pragma unroll
    for (int s = 0; s < G::ks(l); ++s) acc = mma<EM>(f[s], in[s], acc);
    float v[16];
    if constexpr (l + 1 < L) {
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = sp2_fix(acc[j], sp2(acc[j]));
      if constexpr (STASH) {
        if (p.stash[l]) {
          float h[16];
#pragma unroll
          for (int j = 0; j < 16; ++j) h[j] = v[j] * kLn2;
          store_row16(p.stash[l], dimw<N>(p, l + 1), row0, h);
        }
      }
      const Opnd lo = make_op_nonneg(*reinterpret_cast<const float(*)[8]>(v));
      const Opnd hi = make_op_nonneg(*reinterpret_cast<const float(*)[8]>(v + 8));
      out[0][slot<CH>(n, 4 * w + g)] = lo.h;
      out[0][slot<CH>(n, 4 * w + 2 + g)] = hi.h;
      out[1][slot<CH>(n, 4 * w + g)] = lo.l;
      out[1][slot<CH>(n, 4 * w + 2 + g)] = hi.l;
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = acc[j];
      store_row16(reinterpret_cast<float*>(p.out), dimw<N>(p, L), row0, v);
    }
  }
};

// ---------------------------------------------------------------------------
// 2 and 3 layers: the layer pipeline.  L groups of NWV waves, group r
// computing layer r (one wave of each group per SIMD); in step t group r
// runs layer r of the WG's block t - r, reading its input from tile
// tl[r - 1][(t - r) & 1] (group 0: the x tile) and writing its hidden
// activation into tl[r][(t - r) & 1].  A tile written in step t is read in
// step t + 1 and written again in step t + 2, so the one barrier ending each
// step orders every hand-over.  Every group runs nb + L - 1 steps (nb = the
// WG's blocks), every wave the same barriers.
//
// x reaches group 0 through LDS as well: in step t the WG's threads split
// their 8-value pieces of block t + 1 (loaded in step t - 1) into the x tile
// xt[(t + 1) & 1] and issue the loads of their pieces of block t + 2.  Each
// row of x is then loaded once and split once per workgroup, where every
// layer-0 wave loading and splitting the whole block itself costs 4x the
// VALU work and L2 reads.
// ---------------------------------------------------------------------------
template <class N>
struct XPiece {
  using G = FxGeo<N>;
  static_assert(G::THREADS >= 32 * 16, "every 8-value x piece of a block has a thread");
  const FwdParams& p;
  int row, chunk;  // this thread's piece of a block: row, 8-value chunk (row >= 32: none)
  f32x4 raw[2];

  // Loads of the piece of block row0 (rows past the batch read zeros;
  // chunks past the true width are never read unmasked).
  __device__ __forceinline__ void load(int64_t row0) {
    const int D = dimw<N>(p, 0);
    const rsrc_t r = make_rsrc(reinterpret_cast<const float*>(p.x) + row0 * D,
                               row < 32 ? rows_at(p.M, row0, 32) * D * 4u : 0u);
    const uint32_t e = (uint32_t)((row & 31) * D + 8 * chunk) * 4;
    raw[0] = buf_load16<f32x4>(r, e);
    raw[1] = buf_load16<f32x4>(r, e + 16);
  }
  // The loaded piece, split, into an x tile.
  __device__ __forceinline__ void store(XTile<G::CHX>& t) const {
    if (row >= 32 || chunk >= G::CHX) return;
    const float v[8] = {raw[0][0], raw[0][1], raw[0][2], raw[0][3], raw[1][0], raw[1][1], raw[1][2], raw[1][3]};
    const Opnd o = make_op<EM_F32>(v);
    t[0][slot<G::CHX>(row, chunk)] = o.h;
    t[1][slot<G::CHX>(row, chunk)] = o.l;
  }
};

// Group r of the layer pipeline (see above).
template <int r, class N, bool STASH>
__device__ __forceinline__ void x3p_group(const FxOps<N, STASH>& op, XPiece<N>& xp, XTile<FxGeo<N>::CH> (*tl)[2],
                                          XTile<FxGeo<N>::CHX>* xt, int64_t b0, int64_t stride, int64_t nb) {
  using G = FxGeo<N>;
  constexpr int L = N::L;
  Opnd f[G::KSM], in[G::KSM];
  const bool own = op.template owns<r>();
  if (own) op.template load_frags<r>(f);
  const int64_t steps = nb + L - 1;
  for (int64_t t = 0; t < steps; ++t) {
    if (t + 1 < nb) {
      xp.store(xt[(t + 1) & 1]);
      xp.load((b0 + (t + 2) * stride) * 32);
    }
    if (t >= r && t - r < nb) {
      const int64_t b = t - r;
      if constexpr (r == 0)
        op.read_xtile(xt[b & 1], in);
      else
        op.template read_tile<r>(tl[r - 1][b & 1], in);
      if (own) op.template compute<r>(f, in, (b0 + b * stride) * 32, tl[r < L - 1 ? r : 0][b & 1]);
    }
    __syncthreads();
  }
}

template <class N, bool STASH>
__global__ __launch_bounds__(FxGeo<N>::THREADS) void fwd_x3p_kernel(FwdParams p) {
  using G = FxGeo<N>;
  constexpr int L = N::L, CH = G::CH;
  static_assert(G::valid() && G::PIPE, "fp32-tensor pipelined forward shape");
  __shared__ XTile<CH> tl[L - 1][2];
  __shared__ XTile<G::CHX> xt[2];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const FxOps<N, STASH> op{p, lane & 31, lane >> 5, wave % G::NWV};
  const int64_t nblk = (p.M + 31) / 32, stride = gridDim.x, b0 = blockIdx.x;
  const int64_t nb = (nblk - b0 + stride - 1) / stride;  // >= 1: the grid never exceeds the block count
  // x piece of this thread: 16 chunks of 8 values per row (x widths <= 128)
  XPiece<N> xp{p, (int)(threadIdx.x >> 4), (int)(threadIdx.x & 15), {}};
  xp.load(b0 * 32);
  xp.store(xt[0]);
  xp.load((b0 + stride) * 32);
  __syncthreads();
  const int r = wave / G::NWV;
  if (r == 0)
    x3p_group<0>(op, xp, tl, xt, b0, stride, nb);
  else if (L == 2 || r == 1)
    x3p_group<1>(op, xp, tl, xt, b0, stride, nb);
  else
    x3p_group<L - 1>(op, xp, tl, xt, b0, stride, nb);
}

// ---------------------------------------------------------------------------
// 4 and 5 layers: one wave per output block runs every layer of a block in
// turn (NWV waves), its fragments of all layers resident.  The x loads of
// block b + 2 are issued once block b + 1's rows have become operands
// (between block b's first two layers), so each has a whole block's time to
// arrive.
// ---------------------------------------------------------------------------
template <class N, bool STASH>
struct FxWave {
  using G = FxGeo<N>;
  static constexpr int L = N::L, CH = G::CH;
  FxOps<N, STASH> op;
  XTile<CH>* tile;  // [2]
  int par = 0;
  Opnd fr[L][G::KSM];  // this wave's A fragments (output block w)
  Opnd X[G::KSM];      // layer 0's B operands: x row n of the current block
  Opnd B[G::KSM];      // B operands of a hidden layer: row n
  f32x4 xr[G::ks(0)][2];

  template <int l = 0>
  __device__ __forceinline__ void load_all_frags() {
    if constexpr (l < L) {
      if (op.template owns<l>()) op.template load_frags<l>(fr[l]);
      load_all_frags<l + 1>();
    }
  }

  template <int l>
  __device__ __forceinline__ void layer(int64_t row0, int64_t ahead) {
    if (op.template owns<l>()) {
      if constexpr (l == 0)
        op.template compute<0>(fr[0], X, row0, tile[par]);
      else
        op.template compute<l>(fr[l], B, row0, tile[par]);
    }
    if constexpr (l + 1 < L) {
      __syncthreads();  // the whole hidden activation of these rows is in the tile
      op.template read_tile<l + 1>(tile[par], B);
      if constexpr (l == 0) {
        op.x_operands(xr, X);
        op.load_x(xr, ahead);
      }
      // The next hand-over writes the other tile: this one is read until
      // every wave has passed the next barrier.
      par ^= 1;
      layer<l + 1>(row0, ahead);
    }
  }
};

template <class N, bool STASH>
__global__ __launch_bounds__(FxGeo<N>::THREADS) void fwd_x3_kernel(FwdParams p) {
  using G = FxGeo<N>;
  static_assert(G::valid() && !G::PIPE, "fp32-tensor forward shape");
  __shared__ XTile<G::CH> tile[2];
  const int lane = threadIdx.x & 63;
  FxWave<N, STASH> wv{{p, lane & 31, lane >> 5, __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6))}, tile};
  const int64_t nblk = (p.M + 31) / 32, stride = gridDim.x;
  // (the grid never exceeds the block count: every workgroup has a block)
  wv.op.load_x(wv.xr, (int64_t)blockIdx.x * 32);
  wv.load_all_frags();
  wv.op.x_operands(wv.xr, wv.X);
  wv.op.load_x(wv.xr, ((int64_t)blockIdx.x + stride) * 32);
  for (int64_t b = blockIdx.x; b < nblk; b += stride) wv.template layer<0>(b * 32, (b + 2 * stride) * 32);
}

}  // namespace tp

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------

namespace {

template <class N, bool STASH>
constexpr const void* x3_kernel() {
  if constexpr (tp::FxGeo<N>::PIPE)
    return reinterpret_cast<const void*>(&tp::fwd_x3p_kernel<N, STASH>);
  else
    return reinterpret_cast<const void*>(&tp::fwd_x3_kernel<N, STASH>);
}

template <class N>
int launch_x3(const FwdParams& p, bool stash, hipStream_t st, LaunchInfo* info) {
  using G = tp::FxGeo<N>;
  constexpr int kMaxDev = 64;
  static int occ_cache[2][kMaxDev];  // [stash][device]; benign race: the value is idempotent
  const void* kern = stash ? x3_kernel<N, true>() : x3_kernel<N, false>();
  int cus = 0;
  int rc = current_device_cus(&cus);
  if (rc != MLPMK_OK) return rc;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  int occ = (dev >= 0 && dev < kMaxDev) ? occ_cache[stash][dev] : 0;
  if (occ <= 0) {
    rc = kernel_occupancy(kern, G::THREADS, &occ);
    if (rc != MLPMK_OK) return rc;
    if (dev >= 0 && dev < kMaxDev) occ_cache[stash][dev] = occ;
  }
  const int64_t nblk = (p.M + 31) / 32;
  const int64_t cap = (int64_t)cus * occ;
  const int grid = (int)(nblk < cap ? nblk : cap);
  if (info) {
    *info = LaunchInfo{MLPMK_KERNEL_FEATURE_SPLIT, 32, G::THREADS / 64, grid, occ};
    return MLPMK_OK;
  }
  (void)hipGetLastError();
  void* args[] = {const_cast<FwdParams*>(&p)};
  e = hipLaunchKernel(kern, dim3(grid), dim3(G::THREADS), args, 0, st);
  if (e == hipSuccess) e = hipGetLastError();
  return e == hipSuccess ? MLPMK_OK : hip_fail(e, "fp32 forward kernel launch");
}

}  // namespace

bool fwd_generic_dims(int L, const int* dims);

// fp32 tensors: every shape of the 128-wide kernels (the three compiled
// ones and the runtime-width networks of 2..5 layers).  With the stash
// flag, non-NULL stash entries are written.
int fwd_dispatch_f32(int L, const int* dims, const FwdParams& p, bool stash, hipStream_t st, LaunchInfo* info) {
  if (L == 3 && dims[0] == 128 && dims[1] == 128 && dims[2] == 128 && dims[3] == 128)
    return launch_x3<Net<128, 128, 128, 128>>(p, stash, st, info);
  if (fwd_generic_dims(L, dims)) {  // (includes 5 x 128 and 32-64-64-16)
    switch (L) {
      case 2: return launch_x3<Gen<Net<128, 128, 128>>>(p, stash, st, info);
      case 3: return launch_x3<Gen<Net<128, 128, 128, 128>>>(p, stash, st, info);
      case 4: return launch_x3<Gen<Net<128, 128, 128, 128, 128>>>(p, stash, st, info);
      default: return launch_x3<Gen<Net<128, 128, 128, 128, 128, 128>>>(p, stash, st, info);
    }
  }
  return fail(MLPMK_ERR_UNSUPPORTED_SHAPE, "no fp32-tensor forward kernel for these widths (all at most 128)");
}

}  // namespace mlpmk
