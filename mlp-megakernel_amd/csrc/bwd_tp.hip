// Two-pass backward for gfx950 (MI355X): the training backward of the
// softplus MLP as a data-gradient pass spread over the whole chip, then a
// weight-gradient pass whose workgroups each own a block of dW.
//
// Replaces the same reference interface as bwd.hip -- the fused backward of
// the FusedMLPSoftplus autograd function (/root/reference/mlp_fused.md:80-112,
// README.md:30-32) -- for the cases the one-pass megakernel does not serve
// well or at all:
//
//  * small batches (a few thousand rows): the one-pass kernel keeps a whole
//    dW per workgroup, so it runs one 128-row round per workgroup on M / 128
//    CUs (32 of 256 at M = 4096) and then reduces 192 KiB of partials per
//    workgroup;
//  * fp32 tensors (the reference's INPUT_DTYPE = fp32 kernels,
//    mlp_fused.md:159-166): every operand is split into bf16 hi + lo
//    (hi = bf16(v), lo = bf16(v - hi)) and each product is hi*hi + hi*lo +
//    lo*hi on the bf16 MFMA -- fp32's exponent range and a ~16-bit
//    significand (the lo*lo term, below 2^-16 relative, is dropped), where
//    the reference's TF32 operands keep 10 bits;
//  * widths above 128 (up to 256; the reference lists larger H as its next
//    step, mlp_fused.md:453-454), whose dgrad weights and exchange tiles do
//    not fit one workgroup's LDS beside a whole dW of accumulators.
//
// Math (mlp_fused.md:88-95), a_0 = x, a_l = h_l from the fp32 stash,
// dz_{L-1} = dL/dout:
//     dz_{l-1} = (dz_l . W_l^T) * (1 - exp(-h_l)),   dx = dz_0 . W_0^T
//     dW_l     = a_l^T . dz_l
//
// Pass 1, tp_dgrad_kernel (persistent over 32-row blocks, one workgroup per
// block at a time): wave w owns output features [32w, 32w + 32) of every
// data-gradient layer, with its A fragments (16 contiguous bytes of a W_l
// row per lane) loaded once into registers for the 3-layer 128-wide network
// -- which then loads the next block's stash rows while the current block
// computes -- and read from L2 per block and layer otherwise; layers hand dz
// between waves through two LDS tiles, and every dz_{l-1}, l >= 1, is also
// written to the workspace.  When dw is to be written (MLPMK_BWD_WRITE_DW)
// this pass also clears it.  At M = 4096 that is 128 workgroups each running
// a chain of 8-MFMA steps, instead of 32 running whole 128-row rounds.
//
// Pass 2, tp_wgrad_kernel: a workgroup owns a TQI x TQO block of 64 x 64
// "quads" of one dW_l and a chunk of rows; it stages a_l (from x or the
// stash) and dz_l (from dL/dout or the workspace), 64 KiB of rows at a time,
// as 16-bit tiles [row][feature] in LDS, and its waves read both MFMA
// operands with the transposing ds_read_b64_tr_b16, as bwd.hip's wgrad does.
// Each wave adds its 32 x 32 tiles to dw with fp32 atomics: about two
// workgroups per CU (with a register budget that lets both stay resident
// when the grid exceeds the CU count), each adding 4096 elements, so the
// atomics are spread over the whole chip (measured at M = 4096 / 16384: 14.2 / 24.1 us per
// backward, against 16.4 / 31.0 us with per-chunk partial sums and a
// combine kernel).  The summation order of dw is therefore not fixed.
//
// Where it runs (bwd.hip, bwd_path): fp32 tensors and widths above 128
// always; the 16-bit networks the one-pass megakernel also serves up to
// MLPMK_TP_MAX_ROWS rows (3L-128, MI355X, per backward call as a replayed
// graph, two-pass vs one-pass: 14.2 vs 23.0 us at 4096 rows, 24.1 vs 26.8 at
// 16384, 42.6 vs 33.3 at 32768).
#include "device_common.h"
#include "host_common.h"
#include "params.h"
#include "tp_common.h"

namespace mlpmk {

namespace tp {

// ---------------------------------------------------------------------------
// Pass 1: data gradients
// ---------------------------------------------------------------------------

template <class N, bool DX>
struct DgGeo {
  static constexpr int L = N::L;
  static constexpr int LO = DX ? 0 : 1;  // lowest layer with a data gradient
  static constexpr int blocks(int l) { return (N::d[l] + 31) / 32; }
  static constexpr int ks(int l) { return N::d[l + 1] / 16; }  // K-steps: features of dz_l
  static constexpr int nwv() {
    int m = 1;
    for (int l = LO; l < L; ++l) m = blocks(l) > m ? blocks(l) : m;
    return m;
  }
  static constexpr int ksm() {
    int m = 1;
    for (int l = LO; l < L; ++l) m = ks(l) > m ? ks(l) : m;
    return m;
  }
  // Exchange tile width (features per row; a power of two for the swizzle):
  // layer l >= LO + 1 hands dz_{l-1} (d[l] features) to layer l - 1.
  static constexpr int tw() {
    int m = 32;
    for (int l = LO + 1; l < L; ++l)
      while (m < N::d[l]) m *= 2;
    return m;
  }
  static constexpr int NWV = nwv(), KSM = ksm(), TW = tw(), CH = TW / 8;
  static constexpr bool valid() {
    for (int i = 0; i <= L; ++i)
      if (N::d[i] > 256 || N::d[i] % 16 != 0) return false;
    return L >= 2 && NWV <= 8;
  }
};

// RES: every layer's fragments stay in registers for the whole kernel
// (loaded once per workgroup); otherwise (widths above 128, whose fragments
// would not fit beside the rest) each layer's are read from L2 right before
// its MFMA chain, every block -- except, in the 16-bit kernels of widths up
// to 256 (STG), those of the data-gradient layer with the most weights: each
// wave copies its own into LDS once (NWV x 16 K-steps x 1 KiB = 128 KiB,
// beside the 32 KiB exchange tiles: the workgroup's whole 160 KiB, which its
// registers already hold to one workgroup per CU) and reads them from there.
// 128-256-256-128 at 131072 rows: L2 reads of fragments per 32-row block
// 192 -> 64 KiB.
template <class N, int EM, bool DX, bool RES>
struct DgWave {
  using G = DgGeo<N, DX>;
  static constexpr int L = N::L, CH = G::CH, NT = EM == EM_F32 ? 2 : 1;
  static constexpr bool STG = !RES && EM != EM_F32 && G::NWV == 8;
  static constexpr int STG_ELEMS = STG ? G::NWV * G::KSM * 64 : 1;  // f16x8 payloads
  const TpParams& p;
  f16x8 (*tile)[NT][32 * CH];  // [2][NT][32 * CH]
  int lane, n, g, w;
  f16x8* stg = nullptr;               // STG: [NWV][KSM][64] fragments of layer stg_l
  int stg_l = -1;
  int par = 0;                        // exchange tile of the next hand-over
  Opnd fr[RES ? L : 1][G::KSM];       // this wave's A fragments (output block w)
  Opnd B[G::KSM];                     // B operands of the current layer: dz_l of row n
  float h[L][16];                     // h_l of this wave's 16 features of row n (l >= 1)
  float hn[RES ? L : 1][16];          // RES: the same for the workgroup's next block, in flight

  __device__ __forceinline__ bool owns(int l) const { return 32 * w < dimw<N>(p, l); }

  // Fragment (block w, K-step s) of layer l: lane (i, g) holds
  // W_l[outfeat(w, i)][16s + 8g + 0..7].  Rows past the true width read
  // zeros through the resource; columns past it are masked (Gen).
  template <int l>
  __device__ __forceinline__ void load_frags(Opnd (&f)[G::KSM]) const {
    const int K = dimw<N>(p, l), Nout = dimw<N>(p, l + 1);
    const rsrc_t r = make_rsrc(p.w[l], (uint32_t)(K * Nout * kEs<EM>));
    const int row = outfeat(w, n);
#pragma unroll
    for (int s = 0; s < G::ks(l); ++s) {
      const int c = 16 * s + 8 * g;
      if (N::gen && 16 * s >= Nout) {  // a whole K-step past the true width: no load
        f[s] = Opnd{f16x8{}, f16x8{}};
        continue;
      }
      f[s] = load_op<EM>(r, (uint32_t)(row * Nout + c));
      if (N::gen && c >= Nout) f[s] = Opnd{f16x8{}, f16x8{}};
    }
  }
  // STG: copies this wave's fragments of the data-gradient layer with the
  // most weights (true widths) into its LDS slots.
  __device__ __forceinline__ void stage_largest() {
    int64_t best = 0;
    for (int l = G::LO; l < L; ++l) {
      const int64_t e = (int64_t)dimw<N>(p, l) * dimw<N>(p, l + 1);
      if (e > best) {
        best = e;
        stg_l = l;
      }
    }
    stage_layer<G::LO>();
  }
  template <int l>
  __device__ __forceinline__ void stage_layer() {
    if constexpr (l < L) {
      if (l == stg_l && owns(l)) {
        Opnd f[G::KSM];
        load_frags<l>(f);
#pragma unroll
        for (int s = 0; s < G::ks(l); ++s) stg[(w * G::KSM + s) * 64 + lane] = f[s].h;
      }
      stage_layer<l + 1>();
    }
  }
  // Layer l's fragments: from the LDS copy if it holds them, else from L2.
  template <int l>
  __device__ __forceinline__ void frags_of(Opnd (&f)[G::KSM]) const {
    if (STG && l == stg_l) {
      const int Nout = dimw<N>(p, l + 1);
#pragma unroll
      for (int s = 0; s < G::ks(l); ++s) {
        f[s].h = (N::gen && 16 * s >= Nout) ? f16x8{} : stg[(w * G::KSM + s) * 64 + lane];
        f[s].l = f16x8{};
      }
      return;
    }
    load_frags<l>(f);
  }

  template <int l = G::LO>
  __device__ __forceinline__ void load_all_frags() {
    if constexpr (l < L) {
      if (owns(l)) load_frags<l>(fr[l]);
      load_all_frags<l + 1>();
    }
  }

  // dL/dout rows from row0 as B operands (K-steps over the output width).
  // Row stride 0 broadcasts row 0; a negative one (MLPMK_DOUT_SCALAR) one
  // element to every row and feature below the output width.
  __device__ __forceinline__ void load_dout(int64_t row0) {
    constexpr int KS = G::ks(L - 1);
    const int OW = dimw<N>(p, L);
    const int64_t st = p.dout_stride;
    const uint32_t nr = rows_at(p.M, row0, 32);
    if (st < 0) {
      float v;
      const rsrc_t r1 = make_rsrc(p.dout, nr ? (uint32_t)kEs<EM> : 0u);
      if constexpr (EM == EM_F32)
        v = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r1, 0, 0, 0));
      else
        v = elem_to_f32<kBf<EM>>(__builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(r1, 0, 0, 0)));
      const float vv[8] = {v, v, v, v, v, v, v, v};
      const Opnd o = make_op<EM>(vv);
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        B[s] = o;
        if (N::gen && 16 * s + 8 * g >= OW) B[s] = Opnd{f16x8{}, f16x8{}};
      }
      return;
    }
    const uint32_t bytes = nr ? (uint32_t)(((int64_t)(nr - 1) * st + OW) * kEs<EM>) : 0u;
    const rsrc_t r = make_rsrc(static_cast<const char*>(p.dout) + row0 * st * kEs<EM>, bytes);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int c = 16 * s + 8 * g;
      B[s] = load_op<EM>(r, (uint32_t)(n * st + c));
      if (N::gen && c >= OW) B[s] = Opnd{f16x8{}, f16x8{}};
    }
  }

  // h_l for this wave's 16 features of row n (features 32w + 8g + [0..7]
  // and 32w + 16 + 8g + [0..7]), fp32.  With RES every stash layer's are
  // issued at once, a block ahead (into hn, which becomes h when that block
  // starts: the loads of block b + grid are in flight while block b
  // computes); otherwise each layer's with its fragments.  Past the batch the
  // resource is empty and the loads return zeros.
  template <int l = 1>
  __device__ __forceinline__ void load_h(int64_t row0, float (&dst)[L][16]) {
    if constexpr (l < L) {
      load_h_one<l>(row0, dst);
      load_h<l + 1>(row0, dst);
    }
  }
  __device__ __forceinline__ void take_next_h() {
    if constexpr (RES) {
#pragma unroll
      for (int l = 1; l < L; ++l)
#pragma unroll
        for (int j = 0; j < 16; ++j) h[l][j] = hn[l][j];
    }
  }
  template <int l>
  __device__ __forceinline__ void load_h_one(int64_t row0, float (&dst)[L][16]) {
    {
      const int HW = dimw<N>(p, l);
      const rsrc_t r = make_rsrc(p.stash[l - 1] + row0 * HW, owns(l) ? rows_at(p.M, row0, 32) * HW * 4u : 0u);
      const uint32_t e = (uint32_t)(n * HW + 32 * w + 8 * g) * 4;
      const f32x4 a = buf_load16<f32x4>(r, e), b = buf_load16<f32x4>(r, e + 16);
      const f32x4 c = buf_load16<f32x4>(r, e + 64), d = buf_load16<f32x4>(r, e + 80);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        dst[l][j] = a[j];
        dst[l][4 + j] = b[j];
        dst[l][8 + j] = c[j];
        dst[l][12 + j] = d[j];
      }
    }
  }

  // Stores 16 values of row n (features 32w + 8g + [0..7], 32w + 16 + 8g +
  // [0..7]) into a [M, W] tensor of the mode's element type; halves past the
  // true width are dropped.
  __device__ __forceinline__ void store_row16(void* base, int W, int64_t row0, const float (&v)[16]) const {
    const rsrc_t r = make_rsrc(static_cast<char*>(base) + row0 * W * kEs<EM>, rows_at(p.M, row0, 32) * W * kEs<EM>);
    const uint32_t e = (uint32_t)(n * W + 32 * w + 8 * g);
    if (!N::gen || 32 * w < W) store8<EM>(r, e, v);
    if (!N::gen || 32 * w + 16 < W) store8<EM>(r, e + 16, v + 8);
  }

  // Layer l of one 32-row block: B holds dz_l of the rows.  Owning waves
  // compute their 32 features of dz_{l-1} = (dz_l W_l^T) * sigma(h_l) (or of
  // dx for l = 0) and store them; the next layer's B operands then come back
  // from the exchange tile (all of dz_{l-1}, the other waves' features too).
  template <int l>
  __device__ __forceinline__ void layer(int64_t row0) {
    if constexpr (l >= G::LO) {
      if (owns(l)) {
        // Two independent accumulator chains (even and odd K-steps) halve
        // the dependent MFMA latency of the step.
        f32x16 acc = {}, acc2 = {};
        if constexpr (RES) {
#pragma unroll
          for (int s = 0; s < G::ks(l); ++s) {
            if (s & 1)
              acc2 = mma<EM>(fr[l][s], B[s], acc2);
            else
              acc = mma<EM>(fr[l][s], B[s], acc);
          }
        } else {
          Opnd f[G::KSM];
          frags_of<l>(f);
          if constexpr (l >= 1) load_h_one<l>(row0, h);
#pragma unroll
          for (int s = 0; s < G::ks(l); ++s) {
            if (s & 1)
              acc2 = mma<EM>(f[s], B[s], acc2);
            else
              acc = mma<EM>(f[s], B[s], acc);
          }
        }
        acc += acc2;
        float v[16];
        if constexpr (l >= 1) {
#pragma unroll
          for (int j = 0; j < 16; ++j) v[j] = acc[j] * sig_from_h(h[l][j]);
          store_row16(p.dz[l - 1], dimw<N>(p, l), row0, v);  // for the weight-gradient pass
          if constexpr (l - 1 >= G::LO) {  // and for the next layer, through the tile
            const Opnd lo = make_op<EM>(*reinterpret_cast<const float(*)[8]>(v));
            const Opnd hi = make_op<EM>(*reinterpret_cast<const float(*)[8]>(v + 8));
            tile[par][0][slot<CH>(n, 4 * w + g)] = lo.h;
            tile[par][0][slot<CH>(n, 4 * w + 2 + g)] = hi.h;
            if constexpr (NT == 2) {
              tile[par][NT - 1][slot<CH>(n, 4 * w + g)] = lo.l;
              tile[par][NT - 1][slot<CH>(n, 4 * w + 2 + g)] = hi.l;
            }
          }
        } else {
#pragma unroll
          for (int j = 0; j < 16; ++j) v[j] = acc[j];
          store_row16(p.dx, dimw<N>(p, 0), row0, v);
        }
      }
      if constexpr (l >= 1 && l - 1 >= G::LO) {
        __syncthreads();  // the whole of dz_{l-1} of these rows is in the tile
        const int Wd = dimw<N>(p, l);  // features of dz_{l-1} the waves wrote
#pragma unroll
        for (int s = 0; s < G::ks(l - 1); ++s) {
          B[s].h = tile[par][0][slot<CH>(n, 2 * s + g)];
          B[s].l = NT == 2 ? tile[par][NT - 1][slot<CH>(n, 2 * s + g)] : f16x8{};
          // Past the true width the tile holds whatever an earlier block
          // left there (or nothing): zero operands, so that it cannot meet
          // the zero fragments as inf * 0 = NaN.
          if (N::gen && 16 * s + 8 * g >= Wd) B[s] = Opnd{f16x8{}, f16x8{}};
        }
        // The next hand-over writes the other tile: this one is read until
        // every wave has passed the next barrier.
        par ^= 1;
        layer<l - 1>(row0);
      }
    }
  }
};

template <class N, int EM, bool DX, bool RES>
__global__ __launch_bounds__((DgGeo<N, DX>::NWV * 64)) void tp_dgrad_kernel(TpParams p) {
  using G = DgGeo<N, DX>;
  using W = DgWave<N, EM, DX, RES>;
  static_assert(G::valid(), "two-pass backward shape");
  __shared__ f16x8 tile[2][W::NT][32 * G::CH];  // two exchange tiles (hi, and lo with fp32 tensors)
  const int lane = threadIdx.x & 63;
  __shared__ f16x8 stage[W::STG_ELEMS];  // STG: one layer's fragments
  W wv{p, tile, lane, lane & 31, lane >> 5, __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6))};
  if constexpr (W::STG) {
    wv.stg = stage;
    wv.stage_largest();  // (each wave reads back only what it wrote: no barrier)
  }
  const int64_t nblk = (p.M + 31) / 32;
  if (p.zero_dw) {
    // Written (=) rather than accumulated dW: cleared here, before the
    // weight-gradient pass adds its tiles (the next launch on the stream).
    // Every layer's d[l] * d[l+1] is a multiple of 128 (widths multiples of
    // 16, the output width of 8) and dw is 16-byte aligned.
    const int64_t nthr = (int64_t)gridDim.x * blockDim.x;
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
#pragma unroll
    for (int l = 0; l < N::L; ++l) {
      const int64_t n4 = (int64_t)dimw<N>(p, l) * dimw<N>(p, l + 1) / 4;
      f32x4* const d = reinterpret_cast<f32x4*>(p.dw[l]);
      for (int64_t i = tid; i < n4; i += nthr) d[i] = f32x4{};
    }
  }
  if constexpr (RES) {
    wv.template load_h<>((int64_t)blockIdx.x * 32, wv.hn);  // (from HBM: the longest wait first)
    wv.template load_all_frags<>();                          // (L2 hits after the first workgroup)
  }
  for (int64_t b = blockIdx.x; b < nblk; b += gridDim.x) {
    const int64_t row0 = b * 32;
    if constexpr (RES) {
      wv.take_next_h();
      wv.template load_h<>(row0 + 32 * (int64_t)gridDim.x, wv.hn);
    }
    wv.load_dout(row0);
    wv.template layer<N::L - 1>(row0);
  }
}

// ---------------------------------------------------------------------------
// Pass 2: weight gradients
// ---------------------------------------------------------------------------

// A workgroup of 4 waves owns TQI x TQO quads (64 x 64 blocks of dW_l): its
// LDS tile rows hold 64 TQI features of a_l and then 64 TQO features of dz_l,
// RP rows per pass (64 KiB of tiles).  With one quad each wave owns one of
// its four 32 x 32 tiles; with four quads, each wave one quad.  Every wave
// runs all the K-rows of the pass for its tiles, so no partial sums meet
// across waves.
template <int EM, int TQI, int TQO>
struct WgGeo {
  static constexpr int QW = TQI * TQO;
  static constexpr int TPW = QW;                     // 32 x 32 tiles per wave
  static constexpr int FA = 64 * TQI, FZ = 64 * TQO, F = FA + FZ;
  static constexpr int NT = EM == EM_F32 ? 2 : 1;    // tiles: hi (and lo)
  static constexpr int RP = 32768 / F / NT;          // rows per pass
  static constexpr int PA = RP * FA / 8 / 256;       // 8-element pieces of a_l per thread per pass
  static constexpr int PZ = RP * FZ / 8 / 256;       // and of dz_l
  static constexpr int KS = RP / 16;                 // K-steps per pass
  static constexpr int LDS_BYTES = NT * RP * F * 2;
  static_assert(QW == 1 || QW == 4, "one quad per workgroup or one per wave");
};

// Tile layout: element (r, f) of a tile with F features per row sits at
// r*F + (f ^ swz(r, F)); the XOR moves whole 8-feature chunks, so 16-byte
// writes and 8-byte transposed reads stay contiguous, and the four rows of
// one transposed read land in four distinct 16-feature windows.
__device__ __forceinline__ int swz(int r, int F) {
  return (16 * (r & 3) + 8 * ((r >> 2) & 1) + 64 * ((r >> 3) & 1)) & (F - 1);
}

// MFMA operand for features fb .. fb+31 over rows 16kk .. 16kk+15 of a tile:
// lane (m, g) gets rows 16kk + 8g + [0..7] of feature fb + m, through two
// transposing reads (per 16-lane group: result lane i, element j is element
// i & 3 of the 8 bytes addressed by lane (i >> 2) + 4j).
template <int F>
__device__ __forceinline__ f16x8 xread(const f16* t, int fb, int kk, const int (&rrow)[2], int rcol) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  s16x4 h[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int r = rrow[k];
    const f16* a = t + (16 * kk + r) * F + ((fb + rcol) ^ swz(r, F));
    h[k] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)const_cast<f16*>(a));
  }
  return __builtin_bit_cast(f16x8, __builtin_shufflevector(h[0], h[1], 0, 1, 2, 3, 4, 5, 6, 7));
}

// Where a workgroup's operands come from: a_l (x for l = 0, else the fp32
// stash) and dz_l (dL/dout for the last layer, else the workspace).
struct WgSrc {
  const char* base;  // element 0 of the first row of the chunk
  int64_t stride;    // elements between rows; 0 = one row for all; -1 = one element for all
  int es;            // 2 (16-bit) or 4 (fp32)
  int width;         // true features
  int f0;            // first feature of the workgroup's block
  uint32_t bytes;    // resource size from base
};

// MINW: waves per SIMD the register allocation must leave room for.  2 when
// the grid has more workgroups than CUs: two workgroups per CU then keep
// twice the rows in flight (fp32 3L-128 at 131072 rows 228 -> 217 us,
// 128-256-256-128 400 -> 373 us per backward; the 128x128 blocks need 222-228
// VGPRs + 64 AGPRs left to themselves, one workgroup per CU).  1 for grids of
// at most one workgroup per CU (128-256-256-128 at 4096 rows: 38.2 us, 40.7
// with the tighter budget).
template <class N, int EM, int TQI, int TQO, int MINW>
__global__ __launch_bounds__(256, MINW) void tp_wgrad_kernel(TpParams p) {
  using G = WgGeo<EM, TQI, TQO>;
  constexpr int F = G::F, RP = G::RP, NT = G::NT;
  __shared__ __attribute__((aligned(16))) char smem[G::LDS_BYTES];
  f16* const tiles = reinterpret_cast<f16*>(smem);
  const int L = N::L;
  // Task: (layer, quad block) from blockIdx.y, row chunk from blockIdx.x.
  int l = 0, bi = 0, bo = 0;
  {
    int t = blockIdx.y;
    for (int i = 0; i < L; ++i) {
      const int ni = (dimw<N>(p, i) + G::FA - 1) / G::FA, no = (dimw<N>(p, i + 1) + G::FZ - 1) / G::FZ;
      if (t < ni * no) {
        l = i;
        bi = t / no;
        bo = t % no;
        break;
      }
      t -= ni * no;
    }
  }
  const int K = dimw<N>(p, l), NO = dimw<N>(p, l + 1);
  const int64_t r_begin = (int64_t)blockIdx.x * p.chunk_rows;
  const int64_t r_end = r_begin + p.chunk_rows < p.M ? r_begin + p.chunk_rows : p.M;
  const int64_t nrows = r_end - r_begin;
  // Sources.  Resources clip to the chunk's rows, so loads past them read 0.
  WgSrc sa, sz;
  {
    const bool x = l == 0;
    sa.es = x ? kEs<EM> : 4;
    sa.stride = K;
    sa.width = K;
    sa.f0 = G::FA * bi;
    sa.base = x ? static_cast<const char*>(p.x) + r_begin * K * kEs<EM>
                : reinterpret_cast<const char*>(p.stash[l - 1] + r_begin * K);
    sa.bytes = (uint32_t)(nrows * K * sa.es);
    const bool top = l == L - 1;
    sz.es = kEs<EM>;
    sz.width = NO;
    sz.f0 = G::FZ * bo;
    if (top) {
      sz.stride = p.dout_stride < 0 ? -1 : p.dout_stride;
      const int64_t st = sz.stride > 0 ? sz.stride : 0;
      sz.base = static_cast<const char*>(p.dout) + r_begin * st * kEs<EM>;
      sz.bytes = sz.stride < 0 ? (uint32_t)kEs<EM> : (uint32_t)(((nrows - 1) * st + NO) * kEs<EM>);
    } else {
      sz.stride = NO;
      sz.base = static_cast<const char*>(p.dz[l]) + r_begin * NO * kEs<EM>;
      sz.bytes = (uint32_t)(nrows * NO * kEs<EM>);
    }
  }
  const rsrc_t ra = make_rsrc(sa.base, sa.bytes), rz = make_rsrc(sz.base, sz.bytes);
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);

  // Loads of one pass.  a_l pieces first (8 features each), then dz_l
  // pieces: piece k of this thread is q = tid + 256 k, row q / (FA / 8)
  // (resp. FZ / 8), chunk q % (FA / 8) -- consecutive threads read
  // consecutive 16-byte pieces of a row.  Raw payloads: up to 32 bytes (8
  // fp32) per piece, kept until the tile is free.
  struct Raw {
    f32x4 a, b;
  };
  Raw raw_a[G::PA], raw_z[G::PZ];
  auto issue_src = [&](auto& raw, const WgSrc& s, rsrc_t rr, int FS, int64_t prow) {
    constexpr int NP = sizeof(raw) / sizeof(raw[0]);
#pragma unroll
    for (int k = 0; k < NP; ++k) {
      const int q = tid + 256 * k, r = q / (FS / 8), c = q % (FS / 8);
      const int f = s.f0 + 8 * c;
      const int64_t row = prow + r;
      const bool ok = f < s.width && row < nrows;
      const int64_t e = s.stride < 0 ? 0 : row * s.stride + f;
      raw[k].a = raw[k].b = f32x4{};
      if (!ok) continue;
      if (s.es == 4) {
        raw[k].a = buf_load16<f32x4>(rr, (uint32_t)(e * 4));
        raw[k].b = buf_load16<f32x4>(rr, (uint32_t)(e * 4 + 16));
      } else if (s.stride < 0) {  // one 16-bit element for every row and feature
        const int v = __builtin_amdgcn_raw_buffer_load_b16(rr, 0, 0, 0);
        const int vv = (v & 0xffff) | (v << 16);
        raw[k].a = __builtin_bit_cast(f32x4, (i32x4){vv, vv, vv, vv});
      } else {
        raw[k].a = buf_load16<f32x4>(rr, (uint32_t)(e * 2));
      }
    }
  };
  auto issue = [&](int64_t prow) {  // rows prow .. prow + RP - 1 of the chunk
    issue_src(raw_a, sa, ra, G::FA, prow);
    issue_src(raw_z, sz, rz, G::FZ, prow);
  };
  // Convert a pass's pieces and write them into the tile(s): a_l at
  // features [0, FA), dz_l at [FA, F) of each tile row.
  auto commit_src = [&](const auto& raw, const WgSrc& s, int FS, int fbase) {
    constexpr int NP = sizeof(raw) / sizeof(raw[0]);
#pragma unroll
    for (int k = 0; k < NP; ++k) {
      const int q = tid + 256 * k, r = q / (FS / 8), c = q % (FS / 8);
      Opnd o;
      if (s.es == 4) {
        float v[8] = {raw[k].a[0], raw[k].a[1], raw[k].a[2], raw[k].a[3],
                      raw[k].b[0], raw[k].b[1], raw[k].b[2], raw[k].b[3]};
        if (s.stride < 0) {  // (fp32 scalar: element 0 everywhere)
#pragma unroll
          for (int j = 1; j < 8; ++j) v[j] = v[0];
        }
        o = make_op<EM>(v);
      } else {
        o.h = __builtin_bit_cast(f16x8, raw[k].a);
        o.l = f16x8{};
      }
      const int off = r * F + ((fbase + 8 * c) ^ swz(r, F));
      *reinterpret_cast<f16x8*>(tiles + off) = o.h;
      if constexpr (NT == 2) *reinterpret_cast<f16x8*>(tiles + RP * F + off) = o.l;
    }
  };
  auto commit = [&]() {
    commit_src(raw_a, sa, G::FA, 0);
    commit_src(raw_z, sz, G::FZ, G::FA);
  };

  // Wave w: with one quad, tile (w >> 1, w & 1) of it; with four, quad
  // (w / TQO, w % TQO).
  const int qi = G::QW == 1 ? 0 : w / TQO, qo = G::QW == 1 ? 0 : w % TQO;
  int rrow[2], rcol;
  {
    const int q = lane >> 4, i = lane & 15;
    rrow[0] = 8 * (q >> 1) + (i >> 2);
    rrow[1] = rrow[0] + 4;
    rcol = 16 * (q & 1) + 4 * (i & 3);
  }
  f32x16 acc[G::TPW] = {};
  auto opnd = [&](int fb, int kk) {
    Opnd o;
    o.h = xread<F>(tiles, fb, kk, rrow, rcol);
    o.l = NT == 2 ? xread<F>(tiles + RP * F, fb, kk, rrow, rcol) : f16x8{};
    return o;
  };
  const int npass = (int)((nrows + RP - 1) / RP);
  issue(0);
  for (int ps = 0; ps < npass; ++ps) {
    __syncthreads();  // the previous pass's reads are done
    commit();
    if (ps + 1 < npass) issue((int64_t)(ps + 1) * RP);
    __syncthreads();  // the tile is written
    // (K-steps past the chunk's last row read zeros: the loads were masked.)
#pragma unroll
    for (int kk = 0; kk < G::KS; ++kk) {
      if constexpr (G::QW == 1) {
        acc[0] = mma<EM>(opnd(32 * (w >> 1), kk), opnd(G::FA + 32 * (w & 1), kk), acc[0]);
      } else {
        const Opnd a0 = opnd(64 * qi, kk), a1 = opnd(64 * qi + 32, kk);
        const Opnd b0 = opnd(G::FA + 64 * qo, kk), b1 = opnd(G::FA + 64 * qo + 32, kk);
        acc[0] = mma<EM>(a0, b0, acc[0]);
        acc[1] = mma<EM>(a0, b1, acc[1]);
        acc[2] = mma<EM>(a1, b0, acc[2]);
        acc[3] = mma<EM>(a1, b1, acc[3]);
      }
    }
  }

  // Output: tile t = 2 ti + to of quad (qi, qo): C lane (o, g), register e
  // holds dW_l[i][o] for i = 8 (e >> 2) + 4 g + (e & 3) within the tile;
  // added to dw with fp32 atomics.
  auto write_tile = [&](const f32x16& a, int t) {
    const int ti = t >> 1, to = t & 1;
    const int i0 = G::FA * bi + 64 * qi + 32 * ti, o = G::FZ * bo + 64 * qo + 32 * to + (lane & 31);
    const int g = lane >> 5;
    float* const dst = p.dw[l];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int i = i0 + 8 * (e >> 2) + 4 * g + (e & 3);
      if (i < K && o < NO) unsafeAtomicAdd(dst + (int64_t)i * NO + o, a[e]);
    }
  };
  if constexpr (G::QW == 1) {
    write_tile(acc[0], w);
  } else {
#pragma unroll
    for (int t = 0; t < 4; ++t) write_tile(acc[t], t);
  }
}

}  // namespace tp

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------

namespace {

// Per-device occupancy of one kernel (benign race: the value is idempotent).
int cached_occupancy(const void* kern, int threads, int* occ_out) {
  constexpr int kMaxDev = 64;
  struct Entry {
    const void* k;
    int occ;
  };
  static Entry cache[kMaxDev][96];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev >= 0 && dev < kMaxDev) {
    for (auto& c : cache[dev]) {
      if (c.k == kern && c.occ > 0) {
        *occ_out = c.occ;
        return MLPMK_OK;
      }
      if (!c.k) break;
    }
  }
  int occ = 0;
  int rc = kernel_occupancy(kern, threads, &occ);
  if (rc != MLPMK_OK) return rc;
  if (dev >= 0 && dev < kMaxDev) {
    for (auto& c : cache[dev])
      if (!c.k || c.k == kern) {
        c.occ = occ;
        c.k = kern;
        break;
      }
  }
  *occ_out = occ;
  return MLPMK_OK;
}

template <class N, int EM, bool DX, bool RES>
int launch_dgrad(const TpParams& p, int cus, hipStream_t st) {
  using G = tp::DgGeo<N, DX>;
  const void* kern = reinterpret_cast<const void*>(&tp::tp_dgrad_kernel<N, EM, DX, RES>);
  int occ = 0;
  int rc = cached_occupancy(kern, G::NWV * 64, &occ);
  if (rc != MLPMK_OK) return rc;
  const int64_t nblk = (p.M + 31) / 32;
  const int64_t cap = (int64_t)cus * occ;
  const int grid = (int)(nblk < cap ? nblk : cap);
  (void)hipGetLastError();
  hipLaunchKernelGGL((tp::tp_dgrad_kernel<N, EM, DX, RES>), dim3(grid), dim3(G::NWV * 64), 0, st, p);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? MLPMK_OK : hip_fail(e, "two-pass dgrad kernel launch");
}

// Weight-gradient tiling: a workgroup owns TQ x TQ quads (64 x 64 blocks of
// dW).  One quad per workgroup (TQ = 1) gives small batches enough
// workgroups; four (TQ = 2) read each a_l and dz_l element fewer times.
int wgrad_tq(int L, const int* dims, int64_t M) {
  int wmax = 0;
  for (int i = 0; i <= L; ++i) wmax = dims[i] > wmax ? dims[i] : wmax;
  return (wmax > 128 || M >= 65536) ? 2 : 1;
}

int quad_blocks(int L, const int* dims, int tq) {
  int nqb = 0;
  for (int l = 0; l < L; ++l) nqb += ((dims[l] + 64 * tq - 1) / (64 * tq)) * ((dims[l + 1] + 64 * tq - 1) / (64 * tq));
  return nqb;
}

// Workgroups per CU the weight-gradient grid aims at.
#ifndef MLPMK_TP_WG_PER_CU
#define MLPMK_TP_WG_PER_CU 2
#endif

// Longest row chunk with fp32 tensors.  A chunk's products of split
// operands accumulate in one MFMA chain per tile, three MFMAs per K-step, and
// over long chains that sum drifts: the last layer's dW of a 40,000,037-row
// batch (broadcast dout, so its exact value is a column sum) was off by
// 1.6e-4 with chunks of 234 K rows and 6.9e-5 with chunks of 117 K rows;
// the 16-bit one-pass kernel, one MFMA per K-step, stays at 1.6e-6 over
// 156 K rows per workgroup.  Past this length the pass takes more chunks
// (more atomics) instead.
constexpr int64_t kF32MaxChunkRows = 8192;

// Row chunks of the weight-gradient pass: enough chunks for about
// MLPMK_TP_WG_PER_CU workgroups per CU, each a whole number of passes (with
// fp32 tensors, at most kF32MaxChunkRows rows).
void wgrad_chunks(int L, const int* dims, int64_t M, bool f32, int cus, int* S_out, int64_t* rows_out) {
  const int tq = wgrad_tq(L, dims, M);
  const int rp = (tq == 1 ? 256 : 128) / (f32 ? 2 : 1);  // rows per pass (WgGeo::RP)
  const int nqb = quad_blocks(L, dims, tq);
  int64_t smax = ((int64_t)MLPMK_TP_WG_PER_CU * cus + nqb - 1) / nqb;
  if (smax < 1) smax = 1;
  int64_t rows = (M + smax - 1) / smax;
  rows = (rows + rp - 1) / rp * rp;
  if (f32 && rows > kF32MaxChunkRows) rows = kF32MaxChunkRows;  // a multiple of every rp
  *rows_out = rows;
  *S_out = (int)((M + rows - 1) / rows);
}

template <class N, int EM, int TQ>
int launch_wgrad(const TpParams& p, int S, int nqb, int cus, hipStream_t st) {
  (void)hipGetLastError();
  if ((int64_t)S * nqb > cus)
    hipLaunchKernelGGL((tp::tp_wgrad_kernel<N, EM, TQ, TQ, 2>), dim3(S, nqb), dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((tp::tp_wgrad_kernel<N, EM, TQ, TQ, 1>), dim3(S, nqb), dim3(256), 0, st, p);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? MLPMK_OK : hip_fail(e, "two-pass wgrad kernel launch");
}

int64_t round256(int64_t b) { return (b + 255) / 256 * 256; }

typedef Net<128, 128, 128, 128> TNet3L128;
template <int L>
struct GenTp;  // runtime widths up to 256 (16-bit tensors) / 128 (fp32)
template <>
struct GenTp<2> {
  typedef Gen<Net<256, 256, 256>> W;
  typedef Gen<Net<128, 128, 128>> F;
};
template <>
struct GenTp<3> {
  typedef Gen<Net<256, 256, 256, 256>> W;
  typedef Gen<Net<128, 128, 128, 128>> F;
};
template <>
struct GenTp<4> {
  typedef Gen<Net<256, 256, 256, 256, 256>> W;
  typedef Gen<Net<128, 128, 128, 128, 128>> F;
};
template <>
struct GenTp<5> {
  typedef Gen<Net<256, 256, 256, 256, 256, 256>> W;
  typedef Gen<Net<128, 128, 128, 128, 128, 128>> F;
};

bool is_3l128(int L, const int* dims) {
  return L == 3 && dims[0] == 128 && dims[1] == 128 && dims[2] == 128 && dims[3] == 128;
}

template <int EM, int L>
int dispatch_l(const TpParams& p, const int* dims, int S, hipStream_t st) {
  int cus = 0;
  int rc = current_device_cus(&cus);
  if (rc != MLPMK_OK) return rc;
  const bool dx = p.dx != nullptr;
  // Pass 1.
  if (L == 3 && is_3l128(L, dims)) {
    rc = dx ? launch_dgrad<TNet3L128, EM, true, true>(p, cus, st) : launch_dgrad<TNet3L128, EM, false, true>(p, cus, st);
  } else if constexpr (EM == tp::EM_F32) {
    typedef typename GenTp<L>::F NG;
    rc = dx ? launch_dgrad<NG, EM, true, false>(p, cus, st) : launch_dgrad<NG, EM, false, false>(p, cus, st);
  } else {
    typedef typename GenTp<L>::W NG;
    rc = dx ? launch_dgrad<NG, EM, true, false>(p, cus, st) : launch_dgrad<NG, EM, false, false>(p, cus, st);
  }
  if (rc != MLPMK_OK) return rc;
  // Pass 2 (the kernel reads only N's layer count and whether its widths are
  // fixed: one runtime-width instance per depth serves every shape).
  const int tq = wgrad_tq(L, dims, p.M);
  const int nqb = quad_blocks(L, dims, tq);
  typedef typename GenTp<L>::W NW;
  if (L == 3 && is_3l128(L, dims))
    rc = tq == 1 ? launch_wgrad<TNet3L128, EM, 1>(p, S, nqb, cus, st)
                 : launch_wgrad<TNet3L128, EM, 2>(p, S, nqb, cus, st);
  else
    rc = tq == 1 ? launch_wgrad<NW, EM, 1>(p, S, nqb, cus, st) : launch_wgrad<NW, EM, 2>(p, S, nqb, cus, st);
  return rc;
}

}  // namespace

// Shapes of the two-pass backward: 2..5 layers, input and hidden widths
// multiples of 16 and the output width a multiple of 8, all in [16, 256]
// for 16-bit tensors ([16, 128] for fp32 tensors).
bool tp_supported(int L, const int* dims, int dtype) {
  if (L < 2 || L > 5) return false;
  const int wmax = dtype == MLPMK_DTYPE_F32 ? 128 : 256;
  for (int i = 0; i < L; ++i)
    if (dims[i] < 16 || dims[i] > wmax || dims[i] % 16 != 0) return false;
  return dims[L] >= 8 && dims[L] <= wmax && dims[L] % 8 == 0;
}

// Workspace of the two-pass backward: dz_0 .. dz_{L-2} ([M, d[l+1]] each,
// 16-bit or fp32 elements, 256-byte aligned).
int tp_workspace_bytes(int L, const int* dims, int dtype, int64_t M, int64_t* bytes) {
  const int es = dtype == MLPMK_DTYPE_F32 ? 4 : 2;
  int64_t b = 0;
  for (int l = 0; l + 1 < L; ++l) b += round256(M * dims[l + 1] * es);
  *bytes = b;
  return MLPMK_OK;
}

// The two-pass backward.  bp carries the tensors as bwd_common validated
// them; ws holds at least tp_workspace_bytes.
int tp_dispatch(int L, const int* dims, int dtype, const BwdParams& bp, void* ws, hipStream_t st) {
  int cus = 0;
  int rc = current_device_cus(&cus);
  if (rc != MLPMK_OK) return rc;
  TpParams p = {};
  p.x = bp.x;
  for (int l = 0; l < L; ++l) {
    p.w[l] = bp.w[l];
    p.dw[l] = bp.dw[l];
  }
  for (int l = 0; l + 1 < L; ++l) p.stash[l] = bp.stash[l];
  p.dout = bp.dout;
  p.dout_stride = bp.dout_stride;
  p.dx = bp.dx;
  p.M = bp.M;
  p.zero_dw = bp.write_dw;
  for (int l = 0; l <= L; ++l) p.dims[l] = dims[l];
  const int es = dtype == MLPMK_DTYPE_F32 ? 4 : 2;
  char* c = static_cast<char*>(ws);
  for (int l = 0; l + 1 < L; ++l) {
    p.dz[l] = c;
    c += round256(bp.M * dims[l + 1] * es);
  }
  int S = 0;
  wgrad_chunks(L, dims, bp.M, dtype == MLPMK_DTYPE_F32, cus, &S, &p.chunk_rows);
  const int em = dtype == MLPMK_DTYPE_F32 ? tp::EM_F32 : dtype == MLPMK_DTYPE_BF16 ? tp::EM_BF16 : tp::EM_F16;
  switch (em * 8 + L) {
#define MLPMK_TP_CASE(E, LL) \
  case E * 8 + LL: return dispatch_l<E, LL>(p, dims, S, st);
    MLPMK_TP_CASE(tp::EM_F16, 2) MLPMK_TP_CASE(tp::EM_F16, 3) MLPMK_TP_CASE(tp::EM_F16, 4) MLPMK_TP_CASE(tp::EM_F16, 5)
    MLPMK_TP_CASE(tp::EM_BF16, 2) MLPMK_TP_CASE(tp::EM_BF16, 3) MLPMK_TP_CASE(tp::EM_BF16, 4)
    MLPMK_TP_CASE(tp::EM_BF16, 5) MLPMK_TP_CASE(tp::EM_F32, 2) MLPMK_TP_CASE(tp::EM_F32, 3)
    MLPMK_TP_CASE(tp::EM_F32, 4) MLPMK_TP_CASE(tp::EM_F32, 5)
#undef MLPMK_TP_CASE
    default: return fail(MLPMK_ERR_UNSUPPORTED_SHAPE, "two-pass backward: %d layers", L);
  }
}

}  // namespace mlpmk
