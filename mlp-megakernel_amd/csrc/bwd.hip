// Backward megakernel for gfx950 (MI355X): data gradients and weight
// gradients of the softplus MLP in one persistent launch.
//
// Replaces the fused backward of the reference's FusedMLPSoftplus autograd
// function (/root/reference/mlp_fused.md:80-112; README.md:30-32 -- the file
// that held it, fused_mlp.py, is not in the reference snapshot).  Math, with
// a_0 = x, a_l = h_l = softplus(z_{l-1}) read from the fp32 stash and
// dz_{L-1} = dL/dout:
//
//     dW_l     = a_l^T . dz_l                      (every layer)
//     dz_{l-1} = (dz_l . W_l^T) * (1 - exp(-h_l))  (l >= 1; sigmoid(z) = 1 - exp(-h))
//     dx       = dz_0 . W_0^T                      (optional)
//
// Machine mapping (one workgroup of NW waves per CU, R rows per round: 32
// per wave with 4 waves; with the 8-wave feature split below, 32 per wave
// pair):
//
//  * dgrad runs in registers exactly like the forward chain, in the
//    transposed orientation (MFMA M = features of a_l, N = 32 rows, K =
//    features of dz_l): W_l is staged once per workgroup into LDS as A
//    fragments (16 contiguous bytes of a W_l row per lane), dz_l is the B
//    operand, and the fp32 accumulator times (1 - exp(-h_l)), packed to fp16,
//    is directly the next layer's B operand.
//  * wgrad reduces over rows, so it needs rows in the MFMA K dimension while
//    the dgrad layout holds one row per lane.  Every layer, each wave writes
//    its 32 rows of a_l and dz_l (fp16) into LDS exchange tiles laid out
//    [row][feature], one 16-byte write per lane and K-step straight from the
//    row-per-lane registers.  After a workgroup barrier each wave reads the
//    A/B fragments of the 32x32 dW_l tiles it owns with ds_read_b64_tr_b16,
//    which transposes 4x4 blocks of 16-bit elements on the way out of LDS, so
//    a lane receives 8 rows of one feature, and accumulates them over all R
//    rows of the round in MFMA accumulators.
//  * The owned dW tiles stay in registers (AGPRs) across all rounds of the
//    workgroup.  At the end each wave either adds them to the fp32 dW with
//    hardware float atomics (small grids) or writes them to its workgroup's
//    slot of a partial-sum workspace, which bwd_combine_kernel then reduces
//    in a fixed order (no atomics, bitwise-reproducible).
//  * dz through LDS (3-layer and smaller networks, DZL): the dgrad reads its
//    B operands from the exchange tile the wave wrote and writes dz_{l-1}
//    into a second tile, so no dz stays in registers between layers, and the
//    registers that frees let every layer's rows of the next round be
//    requested as soon as this round has consumed them: HBM always has the
//    next rows in flight.
//  * Feature split (FS, 8 waves, the 128-wide networks): wave pairs share a
//    32-row block and split every activation, gradient and dgrad output
//    block in feature halves, each wave owning 2 of each layer's 16 dW
//    tiles: 96 accumulator registers instead of 192, so two waves share a
//    SIMD and hide each other's waits.  The dgrad reads all of dz_l (the
//    partner's half too) from the exchange tile.  With recompute, the pair
//    publishes its halves of h_{L-2} through the second dz tile.
//
// Segment mode (SEG) runs the upper layers of a deeper network on their own:
// layer 0 of the segment then takes its activation from the fp32 stash of
// the layer below (p.h0) instead of x, and its data gradient leaves through
// p.dx already multiplied by 1 - exp(-h) -- exactly the fp16 dz operand the
// in-register chain would have handed to the next layer.  The 5-layer
// backward is two launches this way (layers 4..3, then 2..0), because its
// four dgrad weight blocks and the exchange tiles do not fit the 160 KiB LDS
// of one workgroup together.
//
// The exchange tiles are swizzled by whole 8-feature chunks (Bwd::swz): the
// 16-byte writes of 8 consecutive rows land in 8 distinct chunk slots and the
// four rows of one transposed read fall in four distinct 16-feature windows,
// so both directions are free of bank conflicts.
#include <atomic>

#include "device_common.h"
#include "host_common.h"
#include "params.h"

namespace mlpmk {

template <class N, int NW, bool DX, bool SEG = false>
struct BwdGeom {
  static_assert(!SEG || DX, "a segment always hands on the gradient below it");
  static constexpr int L = N::L;
  // Feature split (FS, 8 waves): wave w takes 32-row block w mod 4 of the
  // round and feature half w / 4 of everything it loads, packs and produces
  // (its share of the dgrad: half the output blocks), and 2 of each layer's
  // 16 dW tiles; half the accumulators per wave let two waves share a SIMD.
  static constexpr bool FS = NW == 8;
  static constexpr int RB = FS ? NW / 2 : NW;  // 32-row blocks per round
  static constexpr int NFH = FS ? 2 : 1;       // feature parts
  static constexpr int R = 32 * RB;            // rows per round
  static constexpr bool has_dgrad(int l) { return l >= 1 || DX; }
  // dgrad of layer l: 32-feature output blocks over d[l], K-steps over d[l+1].
  static constexpr int dmb(int l) { return N::d[l] / 32; }
  static constexpr int dks(int l) { return N::d[l + 1] / 16; }
  static constexpr int dfrag_off(int l) {
    int o = 0;
    for (int i = 0; i < l; ++i)
      if (has_dgrad(i)) o += dmb(i) * dks(i);
    return o;
  }
  static constexpr int ndfrag() { return dfrag_off(L); }
  // wgrad: 32x32 tiles of dW_l.  When 2x2 blocks of tiles divide evenly
  // among the waves, each wave owns whole blocks (2 A + 2 B fragment reads
  // feed 4 MFMAs); otherwise single tiles are dealt round-robin.
  static constexpr int wib(int l) { return (N::d[l] + 31) / 32; }
  static constexpr int wob(int l) { return (N::d[l + 1] + 31) / 32; }
  static constexpr int tiles(int l) { return wib(l) * wob(l); }
  static constexpr int quads(int l) { return (wib(l) / 2) * (wob(l) / 2); }
  static constexpr bool quad(int l) {
    return wib(l) % 2 == 0 && wob(l) % 2 == 0 && quads(l) % NW == 0;
  }
  static constexpr int tpw(int l) { return quad(l) ? 4 * (quads(l) / NW) : (tiles(l) + NW - 1) / NW; }
  static constexpr int tpw_off(int l) {
    int o = 0;
    for (int i = 0; i < l; ++i) o += tpw(i);
    return o;
  }
  static constexpr int ntpw() { return tpw_off(L); }
  // Exchange tiles hold up to this many features (multiples of 32).
  static constexpr int fa() {
    int m = 0;
    for (int i = 0; i < L; ++i) m = 32 * wib(i) > m ? 32 * wib(i) : m;
    return m;
  }
  static constexpr int fz() {
    int m = 0;
    for (int i = 0; i < L; ++i) m = 32 * wob(i) > m ? 32 * wob(i) : m;
    return m;
  }
  static constexpr int ksmax() {
    int m = 0;
    for (int i = 0; i <= L; ++i) m = N::d[i] / 16 > m ? N::d[i] / 16 : m;
    return m;
  }
  static constexpr int kshid() {  // K-steps of the widest activation read from a stash
    int m = 1;
    for (int i = SEG ? 0 : 1; i < L; ++i) m = N::d[i] / 16 > m ? N::d[i] / 16 : m;
    return m;
  }
  // Recompute mode (N::rc): a_{L-1} = h_{L-1} is not read from the stash but
  // recomputed at the start of every round from h_{L-2} with W_{L-2}, whose
  // forward A fragments are read transposed out of its staged dgrad
  // fragments (no LDS of their own).
  static constexpr bool RC = N::rc;
  static constexpr int lds_bytes_with(int ntz) { return ndfrag() * 1024 + (fa() + ntz * fz()) * R * 2; }
  // dz through LDS: the dgrad reads its B operands (dz_l, the wave's own
  // rows) from the exchange tile and writes dz_{l-1} into a second one, so no
  // dz is held in registers across phases.  The 64 registers that frees
  // carry the per-layer prefetch below for 3-layer networks.
  static constexpr bool dzl() { return !N::gen && (!RC || FS) && L <= 3 && lds_bytes_with(2) <= 163840; }
  static constexpr int lds_bytes() { return lds_bytes_with(dzl() ? 2 : 1); }
  // The feature split with one dz tile (its dgrad fragments leave no room
  // for a second): dz_l goes into the tile at the start of the layer, the
  // dgrad reads it back (all of it, the partner's half too) after the
  // layer's barrier, and its output stays in registers until the next layer.
  static constexpr bool dzr() { return FS && !dzl() && !N::gen && !RC && L <= 3 && lds_bytes_with(1) <= 163840; }
  // Recompute under the feature split (RC with FS, dz through LDS): the
  // wave pair writes its halves of h_{L-2} as MFMA operands into the second
  // dz tile, which holds nothing at the start of a round, and each wave
  // recomputes its half of h_{L-1} with B operands read from there.
  // Per-layer prefetch: every stash layer (and x) gets its own register
  // buffer, reloaded for the next round right after its last use, so HBM
  // always has this wave's next rows in flight instead of one phase's rows
  // at a time between compute bursts.  Measured at M = 131072: the
  // two-layer kernel (lower half of the 5-layer backward) 37.5 -> 34.4 us.
  // Without dz through LDS the 3-layer 128-wide kernel spills with it, so
  // such kernels (the 4-wave ones and the single-tile feature split, 3-layer
  // with dx: 88.5 us with the prefetch, which spills, 77.9 us without, at
  // M = 131072) share one buffer loaded one phase ahead.
  static constexpr bool pf() { return !N::gen && (SEG ? dzl() : (L <= 2 || dzl())); }
  // Element offset of dW_l in the dW blocks laid out back to back.
  static constexpr int woff(int l) {
    int o = 0;
    for (int i = 0; i < l; ++i) o += N::d[i] * N::d[i + 1];
    return o;
  }
  static constexpr bool valid() {
    for (int i = 0; i <= L; ++i)
      if (N::d[i] > 128) return false;  // dgrad staging holds at most 4 x 8 fragments per layer
    for (int i = 1; i < L; ++i)
      if (N::d[i] % 32 != 0) return false;  // hidden widths in whole 32-feature blocks
    if (DX && N::d[0] % 32 != 0) return false;
    // recompute: 3-layer kernels and 2-layer segments of 128-wide networks
    if (RC && (N::gen || !(L == 3 || (L == 2 && SEG)))) return false;
    if (FS) {  // dz through LDS (the partner wave's half), whole 64-feature halves
      if (!dzl() && !dzr()) return false;
      for (int i = 0; i <= L; ++i)
        if (N::d[i] % 64 != 0) return false;
    }
    return N::valid() && R >= 128 && lds_bytes() <= 163840;
  }
};

// Fragment lane `item` (fragment-major, 64 lanes each) of layer l's dgrad A
// operands: 16 contiguous bytes of one W_l row.  For a runtime-width (Gen)
// network the true widths come from p.dims: W_l rows are p.dims[l + 1] wide
// (any width for the last layer), read element by element, and entries past
// the true widths stage as zeros.
template <class N, class Gm>
__device__ __forceinline__ f16x8 dgrad_fragment(const BwdParams& p, int l, int item) {
  const int Nout = N::gen ? p.dims[l + 1] : N::d[l + 1];
  const int KS = Gm::dks(l);
  const int f = item >> 6, lane = item & 63;
  const int mb = f / KS, s = f % KS;
  const int i = lane & 31, g = lane >> 5;
  const int row = outfeat(mb, i);
  const f16* __restrict__ w = p.w[l];
  if constexpr (N::gen) {
    f16x8 v;
    const int k0 = 16 * s + 8 * g;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      v[j] = (row < p.dims[l] && k0 + j < Nout) ? w[(int64_t)row * Nout + k0 + j] : (f16)0.0f;
    return v;
  } else {
    return *reinterpret_cast<const f16x8*>(w + (int64_t)row * Nout + 16 * s + 8 * g);
  }
}

// Stages the dgrad A fragments: fragment (mb, s) of layer l, lane (i, g) holds
// W_l[outfeat(mb, i)][16s + 8g + j], j = 0..7.  A thread issues the loads of
// all its fragment lanes, of every layer, before writing any of them to LDS:
// one memory round trip for the whole staging (3L-128 at NW = 4: 16 loads per
// thread; one at a time they took 12.6 K cycles, one layer at a time 6.2 K).
template <class N, class Gm>
struct DgradStage {
  static constexpr int kMaxItems = 4 * 8 * 64;  // 4 x 8 fragments of 64 lanes: a 128 x 128 layer
  template <int NT>
  static constexpr int per() { return (kMaxItems + NT - 1) / NT; }
};

template <class N, class Gm, int NT, int l = 0>
__device__ __forceinline__ void dgrad_load_all(const BwdParams& p, f16x8 (&v)[N::L][DgradStage<N, Gm>::template per<NT>()]) {
  if constexpr (l < N::L) {
    if constexpr (Gm::has_dgrad(l)) {
      constexpr int items = Gm::dmb(l) * Gm::dks(l) * 64;  // <= kMaxItems: widths are at most 128
#pragma unroll
      for (int k = 0; k < DgradStage<N, Gm>::template per<NT>(); ++k) {
        const int item = threadIdx.x + k * NT;
        if (item < items) v[l][k] = dgrad_fragment<N, Gm>(p, l, item);
      }
    }
    dgrad_load_all<N, Gm, NT, l + 1>(p, v);
  }
}

// Writes the fragment lanes dgrad_load_all loaded into LDS.
template <class N, class Gm, int NT>
__device__ __forceinline__ void dgrad_store_all(const f16x8 (&v)[N::L][DgradStage<N, Gm>::template per<NT>()],
                                                f16x8* lds) {
#pragma unroll
  for (int l = 0; l < N::L; ++l) {
    if (!Gm::has_dgrad(l)) continue;
    const int items = Gm::dmb(l) * Gm::dks(l) * 64;
#pragma unroll
    for (int k = 0; k < DgradStage<N, Gm>::template per<NT>(); ++k) {
      const int item = threadIdx.x + k * NT;
      if (item < items) lds[Gm::dfrag_off(l) * 64 + item] = v[l][k];
    }
  }
}

// Recompute mode for a network type: the backward recomputes h_{L-1} instead
// of reading it (the forward then stashes only h_1 .. h_{L-2}).
template <class Base>
struct Recompute : Base {
  static constexpr bool rc = true;
};

template <class N, int NW, bool DX, bool SEG>
struct BwdWave {
  using Gm = BwdGeom<N, NW, DX, SEG>;
  static constexpr int L = N::L;
  static constexpr int R = Gm::R;
  static constexpr int KSM = Gm::ksmax();
  static constexpr int KSH = Gm::kshid();
  static constexpr int KS0 = N::d[0] / 16;
  static constexpr int KSL = N::d[L] / 16;
  static constexpr int FA = Gm::fa(), FZ = Gm::fz();  // features per exchange-tile row
  static constexpr bool DZL = Gm::dzl();
  static constexpr int NFH = Gm::NFH;  // feature parts (FS: 2)
  static constexpr int KSHW = KSH / NFH, KS0W = KS0 / NFH, KSLW = KSL / NFH;  // K-steps this wave holds

  const BwdParams& p;
  const f16x8* wfr;  // staged dgrad fragments
  f16* ta;           // exchange tile: a_l, [row][feature] (FA features per row)
  f16* tz;           // exchange tile: dz_l, [row][feature] (FZ features per row); two of them with DZL
  int lane, n, g, wid;
  int64_t row0;    // first row of this wave's 32 in the current round
  int64_t rstep;   // rows between a workgroup's consecutive rounds
  int wsw;         // swizzle of this lane's row (the row it writes)
  int rrow[2];     // rows (within a K-step of 16) of this lane's two transposed reads
  int rcol;        // first of the 4 features the lane addresses in a read, less the block base
  f32x16 (&wacc)[Gm::ntpw()];
  int rb = 0, fh = 0;  // row block of the round and feature part (FS; else rb = wid)

  // Prefetched rows (issued one phase ahead of their use).
  static constexpr bool PF = Gm::pf();
  // With DZL, x and dL/dout take turns in one buffer: dL/dout is written to
  // its tile at the start of a round, then the round's x rows are loaded
  // into the buffer, and once they are in the a_0 tile the next round's
  // dL/dout is.
  static constexpr bool SHX = DZL && PF && !SEG && KS0 == KSL;
  static constexpr bool EARLY = DZL && PF;  // next-round rows requested before the layer's barrier
  // (Each holds this wave's feature part: K-steps fh * KS..W onwards.)
  f16x8 gbuf[KSLW];                 // dL/dout of the round = dz_{L-1}
  float hbuf[PF ? L : 1][KSHW][8];  // h_l, fp32: buffer l (PF) or one shared buffer
  f16x8 xown[SHX ? 1 : KS0W];       // x rows (SHX: in gbuf)
  __device__ __forceinline__ f16x8 (&xbuf())[KS0W] {
    if constexpr (SHX)
      return *reinterpret_cast<f16x8(*)[KS0W]>(gbuf);
    else
      return *reinterpret_cast<f16x8(*)[KS0W]>(xown);
  }

  // Tile layout: element (r, f) of a tile with F features per row sits at
  // r*F + (f ^ swz(r, F)).  The XOR moves whole 8-feature chunks, so every
  // 16-byte write and every 8-byte transposed read stays contiguous; eight
  // consecutive rows get eight distinct chunk slots (the writes of 8 lanes,
  // one row each, hit distinct banks) and rows r .. r+3 of one read land in
  // four distinct 16-feature windows.
  static __device__ __forceinline__ int swz(int r, int F) {
    return (16 * (r & 3) + 8 * ((r >> 2) & 1) + 64 * ((r >> 3) & 1)) & (F - 1);
  }

  __device__ __forceinline__ void init_slots() {
    rb = Gm::FS ? wid % Gm::RB : wid;
    fh = Gm::FS ? wid / Gm::RB : 0;
    wsw = rb * 32 + n;  // the row this lane writes (swizzle taken per tile width)
    // ds_read_b64_tr_b16, per 16-lane group: result lane i, element j is
    // element (i & 3) of the 8 bytes addressed by lane (i >> 2) + 4j.  Lane
    // 4j + c of group q addresses row 8*(q >> 1) + j (+4 for the second read)
    // and features 16*(q & 1) + 4c .. +3 of the fragment's 32, so result lane
    // i gets feature 16*(q & 1) + i of rows 8*(q >> 1) + 0..3 (then 4..7):
    // the 8 K-values of MFMA operand lane (m = lane & 31, g = lane >> 5).
    const int q = lane >> 4, i = lane & 15;
    rrow[0] = 8 * (q >> 1) + (i >> 2);
    rrow[1] = rrow[0] + 4;
    rcol = 16 * (q & 1) + 4 * (i & 3);
  }  // True width of activation / gradient level l (p.dims for Gen networks).
  __device__ __forceinline__ int dw_(int l) const { return N::gen ? p.dims[l] : N::d[l]; }
  __device__ __forceinline__ uint32_t nrows_at(int64_t r0) const {
    const int64_t left = p.M - r0;
    return (uint32_t)(left < 32 ? (left > 0 ? left : 0) : 32);
  }
  // Resource over this wave's 32 rows from r0 of a row-major [M, width] tensor;
  // loads past the valid rows read zeros and stores there are dropped.
  __device__ __forceinline__ rsrc_t rows_rsrc(const void* base, int width, int elem, int64_t r0) const {
    return make_rsrc(static_cast<const char*>(base) + r0 * width * elem, nrows_at(r0) * width * elem);
  }

  // dL/dout rows from r0 as B operands.  Row stride 0 broadcasts row 0; a
  // negative one (MLPMK_DOUT_SCALAR) element 0 to every row and feature below
  // the output width.
  __device__ __forceinline__ void load_dout(int64_t r0) {
    const int64_t st = p.dout_stride;
    const int OW = dw_(L);
    const uint32_t nr = nrows_at(r0);
    if (st < 0) {
      const rsrc_t r1 = make_rsrc(p.dout, nr ? 2u : 0u);
      const f16 v = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(r1, 0, 0, 0));
#pragma unroll
      for (int s = 0; s < KSLW; ++s) {
        const int c = 16 * (s + fh * KSLW) + 8 * g;
#pragma unroll
        for (int j = 0; j < 8; ++j) gbuf[s][j] = (!N::gen || c + j < OW) ? v : (f16)0.0f;
      }
      return;
    }
    const uint32_t bytes = nr ? (uint32_t)(((int64_t)(nr - 1) * st + OW) * 2) : 0u;
    const rsrc_t r = make_rsrc(p.dout + r0 * st, bytes);
    if constexpr (N::gen) {
      // Runtime output width OW: whole 8-feature pieces below OW in one
      // 16-byte load, the piece that straddles OW element by element (the
      // resource ends at the row's OW-th element, and a broadcast row may be
      // exactly OW long), pieces past OW zero.
#pragma unroll
      for (int s = 0; s < KSLW; ++s) {
        const int c = 16 * (s + fh * KSLW) + 8 * g;
        if (c + 8 <= OW) {
          gbuf[s] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(r, (int)((n * st + c) * 2), 0, 0));
        } else {
          gbuf[s] = f16x8{};
          if (c < OW) {
#pragma unroll
            for (int j = 0; j < 7; ++j)
              if (c + j < OW)
                gbuf[s][j] = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(r, (int)((n * st + c + j) * 2), 0, 0));
          }
        }
      }
      return;
    }
#pragma unroll
    for (int s = 0; s < KSLW; ++s)
      gbuf[s] = __builtin_bit_cast(
          f16x8, __builtin_amdgcn_raw_buffer_load_b128(r, (int)((n * st + 16 * (s + fh * KSLW) + 8 * g) * 2), 0, 0));
  }
  // a_l = h_l (stash[l-1], or p.h0 for layer 0 of a segment; fp32) rows from
  // r0: 8 consecutive features per K-step.
  template <int l>
  __device__ __forceinline__ void load_h(int64_t r0) {
    constexpr int B = PF ? l : 0;
    const int HW = dw_(l);  // a multiple of 16 for Gen networks: K-steps past it are zero
    const rsrc_t hr = rows_rsrc(l == 0 ? p.h0 : p.stash[l > 0 ? l - 1 : 0], HW, 4, r0);
    constexpr int KW = N::d[l] / 16 / NFH;  // K-steps of this wave's feature part
#pragma unroll
    for (int s = 0; s < KW; ++s) {
      const int sg = s + fh * KW;
      if (N::gen && 16 * sg >= HW) {
#pragma unroll
        for (int j = 0; j < 8; ++j) hbuf[B][s][j] = 0.0f;
        continue;
      }
      const int off = (n * HW + 16 * sg + 8 * g) * 4;
      const f32x4 lo = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(hr, off, 0, 0));
      const f32x4 hi = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(hr, off + 16, 0, 0));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        hbuf[B][s][j] = lo[j];
        hbuf[B][s][4 + j] = hi[j];
      }
    }
  }
  __device__ __forceinline__ void load_x(int64_t r0) {
    const int D = dw_(0);
    const rsrc_t xr = rows_rsrc(p.x, D, 2, r0);
#pragma unroll
    for (int s = 0; s < KS0W; ++s) {
      const int sg = s + fh * KS0W;
      xbuf()[s] = (N::gen && 16 * sg >= D)
                    ? f16x8{}
                    : __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(
                                                    xr, (int)((n * D + 16 * sg + 8 * g) * 2), 0, 0));
    }
  }

  // Writes the wave's 32 rows of KS K-steps of features from K-step s0 on
  // (row-per-lane B operands v[s]: row n, features 16(s0 + s) + 8g + [0..7])
  // into an exchange tile: one 16-byte write per K-step, straight from the
  // registers.
  template <int F, int KS>
  __device__ __forceinline__ void xwrite(f16* t, const f16x8 (&v)[KS], int s0 = 0) const {
    const int r = wsw, sw = swz(r, F);
#pragma unroll
    for (int s = 0; s < KS; ++s) *reinterpret_cast<f16x8*>(t + r * F + ((16 * (s0 + s) + 8 * g) ^ sw)) = v[s];
  }
  // MFMA operand for features fb .. fb+31 (fb % 32 == 0) over rows
  // 16kk .. 16kk+15 of the round: lane (m, g) gets rows 16kk + 8g + [0..7] of
  // feature fb + m, through two transposing LDS reads.
  template <int F>
  __device__ __forceinline__ f16x8 xread(const f16* t, int fb, int kk) const {
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    s16x4 h[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int r = rrow[k];  // swz(16kk + r) == swz(r)
      const f16* a = t + (16 * kk + r) * F + ((fb + rcol) ^ swz(r, F));
      h[k] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)const_cast<f16*>(a));
    }
    return __builtin_bit_cast(f16x8, __builtin_shufflevector(h[0], h[1], 0, 1, 2, 3, 4, 5, 6, 7));
  }

  // Wgrad of layer l over the R rows in the exchange tiles, for this wave's
  // tiles.  K-steps (16 rows) outermost keeps only one step's fragments live.
  template <int l>
  __device__ __forceinline__ void wgrad(const f16* tz) const {
    constexpr int OFF = Gm::tpw_off(l);
    if constexpr (!N::gen && Gm::quad(l) && Gm::quads(l) == NW) {
      // One 2x2 block of tiles per wave: the four operands of K-step kk + 1
      // are read while the four MFMAs of K-step kk run (two register sets),
      // one scheduling region per K-step.
      constexpr int QO = Gm::wob(l) / 2;
      constexpr int KK = R / 16;
      const int fi = 64 * (wid / QO), fo = 64 * (wid % QO);
      f16x8 op[2][4];
      op[0][0] = xread<FA>(ta, fi, 0);
      op[0][1] = xread<FA>(ta, fi + 32, 0);
      op[0][2] = xread<FZ>(tz, fo, 0);
      op[0][3] = xread<FZ>(tz, fo + 32, 0);
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        const int c = kk & 1;
        if (kk + 1 < KK) {
          op[c ^ 1][0] = xread<FA>(ta, fi, kk + 1);
          op[c ^ 1][1] = xread<FA>(ta, fi + 32, kk + 1);
          op[c ^ 1][2] = xread<FZ>(tz, fo, kk + 1);
          op[c ^ 1][3] = xread<FZ>(tz, fo + 32, kk + 1);
        }
        wacc[OFF + 0] = mfma32x32x16<N::bf>(op[c][0], op[c][2], wacc[OFF + 0]);
        wacc[OFF + 1] = mfma32x32x16<N::bf>(op[c][0], op[c][3], wacc[OFF + 1]);
        wacc[OFF + 2] = mfma32x32x16<N::bf>(op[c][1], op[c][2], wacc[OFF + 2]);
        wacc[OFF + 3] = mfma32x32x16<N::bf>(op[c][1], op[c][3], wacc[OFF + 3]);
        if (kk + 1 < KK) __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);  // DS reads first
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);                   // then the MFMAs
        __builtin_amdgcn_sched_barrier(0);
      }
      return;
    }
#pragma unroll
    for (int kk = 0; kk < R / 16; ++kk) {
      if constexpr (Gm::quad(l)) {
        constexpr int QO = Gm::wob(l) / 2;
#pragma unroll
        for (int k = 0; k < Gm::quads(l) / NW; ++k) {
          const int q = wid + k * NW;
          const int fi = 64 * (q / QO), fo = 64 * (q % QO);
          const f16x8 a0 = xread<FA>(ta, fi, kk), a1 = xread<FA>(ta, fi + 32, kk);
          const f16x8 b0 = xread<FZ>(tz, fo, kk), b1 = xread<FZ>(tz, fo + 32, kk);
          wacc[OFF + 4 * k + 0] = mfma32x32x16<N::bf>(a0, b0, wacc[OFF + 4 * k + 0]);
          wacc[OFF + 4 * k + 1] = mfma32x32x16<N::bf>(a0, b1, wacc[OFF + 4 * k + 1]);
          wacc[OFF + 4 * k + 2] = mfma32x32x16<N::bf>(a1, b0, wacc[OFF + 4 * k + 2]);
          wacc[OFF + 4 * k + 3] = mfma32x32x16<N::bf>(a1, b1, wacc[OFF + 4 * k + 3]);
        }
      } else {
        constexpr int WOB = Gm::wob(l);
#pragma unroll
        for (int k = 0; k < Gm::tpw(l); ++k) {
          const int t = wid + k * NW;
          if (Gm::tiles(l) % NW == 0 || t < Gm::tiles(l))
            wacc[OFF + k] =
                mfma32x32x16<N::bf>(xread<FA>(ta, 32 * (t / WOB), kk), xread<FZ>(tz, 32 * (t % WOB), kk), wacc[OFF + k]);
        }
      }
    }
  }

  // dgrad output block mb of layer l (features 32mb .. 32mb+31 of a_l, this
  // wave's 32 rows): registers 0..7 of the accumulator hold features 32mb +
  // 8g + [0..7] (K-step 2mb of a_l), 8..15 hold 32mb + 16 + 8g + [0..7]
  // (K-step 2mb + 1); h_l's K-steps 2mb, 2mb + 1 sit at 2hj, 2hj + 1 of this
  // wave's buffer.  Through a stash layer (HA) it is multiplied by
  // sigma(z) = 1 - exp(-h_l) into dz_{l-1} (or, for a segment's layer 0, the
  // dz handed to the launch below through p.dx); otherwise it is dx itself.
  template <int l, bool HA, int B>
  __device__ __forceinline__ void dgrad_epilogue(int mb, int hj, const f32x16& acc, f16x8 (&dzn)[KSM],
                                                 f16* tout) const {
    if constexpr (HA) {
      float v[16];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        v[j] = acc[j] * sig_from_h(hbuf[B][2 * hj][j]);
        v[8 + j] = acc[8 + j] * sig_from_h(hbuf[B][2 * hj + 1][j]);
      }
      const f16x8 lo = pack8<N::bf>(v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]);
      const f16x8 hi = pack8<N::bf>(v[8], v[9], v[10], v[11], v[12], v[13], v[14], v[15]);
      if constexpr (l >= 1 && DZL) {  // the wave's own rows of the dz_{l-1} tile
        const int r = wsw, sw = swz(r, FZ);
        *reinterpret_cast<f16x8*>(tout + r * FZ + ((32 * mb + 8 * g) ^ sw)) = lo;
        *reinterpret_cast<f16x8*>(tout + r * FZ + ((32 * mb + 16 + 8 * g) ^ sw)) = hi;
      } else if constexpr (l >= 1) {
        dzn[2 * hj] = lo;
        dzn[2 * hj + 1] = hi;
      } else {  // segment: dz of the layer below leaves through p.dx
        const int D = dw_(0);
        const rsrc_t dr = rows_rsrc(p.dx, D, 2, row0);
        const uint32_t e = (uint32_t)(n * D + 32 * mb + 8 * g);
        if (!N::gen || 32 * mb < D) buf_store16(lo, dr, e * 2);
        if (!N::gen || 32 * mb + 16 < D) buf_store16(hi, dr, e * 2 + 32);
      }
    } else {
      const int D = dw_(0);  // a multiple of 16 for Gen networks
      const rsrc_t dr = rows_rsrc(p.dx, D, 2, row0);
      const uint32_t e = (uint32_t)(n * D + 32 * mb + 8 * g);
      if (!N::gen || 32 * mb < D)
        buf_store16(pack8<N::bf>(acc[0], acc[1], acc[2], acc[3], acc[4], acc[5], acc[6], acc[7]), dr, e * 2);
      if (!N::gen || 32 * mb + 16 < D)
        buf_store16(pack8<N::bf>(acc[8], acc[9], acc[10], acc[11], acc[12], acc[13], acc[14], acc[15]), dr,
                    e * 2 + 32);
    }
  }

  // One layer of the backward for this wave's 32 rows.  On entry dz holds
  // dz_l and hbuf (l >= 1, or a segment) or xbuf (l = 0) holds a_l.
  // Publishes a_l and dz_l to the exchange tiles, runs dgrad into
  // dzn = dz_{l-1} (or dx), and after the barrier issues the next phase's
  // loads before the wgrad of dW_l so that their latency hides behind its
  // MFMAs.
  template <int l>
  __device__ __forceinline__ void phase(f16x8 (&dz)[KSM], f16x8 (&dzn)[KSM]) {
    constexpr int KSA = N::d[l] / 16;      // K-steps of a_l
    constexpr int KSZ = N::d[l + 1] / 16;  // K-steps of dz_l
    constexpr bool HA = l >= 1 || SEG;     // a_l came from a stash (fp32, in hbuf)
    constexpr int B = PF ? l : 0;          // its buffer
    // dz tiles: dz_l is read from tin; with DZL the dgrad writes dz_{l-1}
    // into the other tile (the layers alternate, starting from tile 0).
    f16* const tin = tz + (DZL ? ((L - 1 - l) & 1) * FZ * R : 0);
    f16* const tout = tz + (DZL ? ((L - l) & 1) * FZ * R : 0);
    if constexpr (!DZL) {  // (the wave's feature part of dz_l)
      constexpr int KW = KSZ / NFH;
      f16x8 zs[KW];
#pragma unroll
      for (int s = 0; s < KW; ++s) zs[s] = dz[s];
      xwrite<FZ>(tin, zs, fh * KW);
    }
    if constexpr (HA) {
      constexpr int KW = KSA / NFH;
      f16x8 as[KW];
#pragma unroll
      for (int s = 0; s < KW; ++s)
        as[s] = pack8<N::bf>(hbuf[B][s][0], hbuf[B][s][1], hbuf[B][s][2], hbuf[B][s][3], hbuf[B][s][4], hbuf[B][s][5],
                      hbuf[B][s][6], hbuf[B][s][7]);
      xwrite<FA>(ta, as, fh * KW);
    } else {
      xwrite<FA>(ta, xbuf(), fh * KS0W);
      if constexpr (SHX)
        load_dout(row0 + rstep);  // x is consumed: the next round's dL/dout takes its buffer
      else if constexpr (EARLY)
        load_x(row0 + rstep);  // x is consumed: the next round's rows
    }
    // The dgrad reads all of dz_l for the wave's rows.  With the feature
    // split the partner wave wrote half of them: of the round's dL/dout
    // tile (l = L-1) just now, so that dgrad waits for the barrier; the
    // dz_l of lower layers were written before the previous layer's.
    constexpr bool DG_LATE = Gm::FS && (l == L - 1 || !DZL);
    constexpr bool NEXT_H = EARLY && HA && !(Gm::RC && l == L - 1);  // (a recomputed h has no stash)
    if constexpr (Gm::has_dgrad(l) && !DG_LATE) dgrad<l, HA, B>(dz, dzn, tin, tout);
    if constexpr (NEXT_H && !DG_LATE) load_h<l>(row0 + rstep);  // h_l is consumed (sigma done): the next round's rows
    __syncthreads();  // every wave's rows are in the exchange tiles
    if constexpr (Gm::has_dgrad(l) && DG_LATE) dgrad<l, HA, B>(dz, dzn, tin, tout);
    if constexpr (NEXT_H && DG_LATE) load_h<l>(row0 + rstep);
    if constexpr (EARLY) {
    } else if constexpr (PF) {  // this layer's buffer is free: the next round's rows
      if constexpr (HA)
        load_h<l>(row0 + rstep);
      else
        load_x(row0 + rstep);
    } else if constexpr (l >= 2 || (l == 1 && SEG)) {
      load_h<l - 1>(row0);
    } else if constexpr (l == 1) {
      load_x(row0);
    } else {  // the next round of this workgroup (empty resources past the end)
      load_dout(row0 + rstep);
      if constexpr (Gm::RC)
        load_h<L - 2>(row0 + rstep);  // the round recomputes h_{L-1} from it
      else if constexpr (L >= 2)
        load_h<L - 1>(row0 + rstep);
    }
    wgrad<l>(tin);
    __syncthreads();  // the tiles are free for the next layer
  }

  // dgrad of layer l for this wave's 32 rows: dz_l (B operands: registers dz,
  // or with DZL the wave's own rows of tile tin) times the staged W_l
  // fragments, through the epilogue into dzn / tout / p.dx.
  //
  // Software pipeline over the 32-feature output blocks: block mb's MFMA
  // chain shares a scheduling region with block mb - 1's epilogue (VALU), and
  // the A fragments run through a ring of NQ reads in flight (fragment t + NQ
  // is requested right after the MFMA that consumes fragment t), so neither
  // the LDS latency nor the epilogue sits between two MFMAs of a chain.  One
  // opaque base keeps the reads on immediate offsets of a single address
  // register.  Runtime-width networks keep one block at a time: their
  // register budget has no room for the ring.
  template <int l, bool HA, int B>
  __device__ __forceinline__ void dgrad(const f16x8 (&dz)[KSM], f16x8 (&dzn)[KSM], const f16* tin, f16* tout) {
    constexpr int KSZ = N::d[l + 1] / 16;  // K-steps of dz_l
    constexpr int MB = N::d[l] / 32;
    constexpr int NF = MB * KSZ / NFH;  // fragments this wave reads
    constexpr int NQ = NF < 4 ? NF : 4;
    if constexpr (N::gen) {
      const int fbase = (Gm::dfrag_off(l) * 64 + lane) * 16;
      const char* wb = reinterpret_cast<const char*>(wfr);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const f16x8* frag = reinterpret_cast<const f16x8*>(wb + opaque(fbase + mb * KSZ * 1024));
        f32x16 a = {};
#pragma unroll
        for (int s = 0; s < KSZ; ++s) a = mfma32x32x16<N::bf>(frag[s * 64], dz[s], a);
        dgrad_epilogue<l, HA, B>(mb, mb, a, dzn, tout);
      }
      return;
    }
    f16x8 zb[KSZ];
    const int zr = wsw, zsw = swz(zr, FZ);
    auto zread = [&](int s) { return *reinterpret_cast<const f16x8*>(tin + zr * FZ + ((16 * s + 8 * g) ^ zsw)); };
    if constexpr (DZL || Gm::FS) {  // rows this wave (and with FS its partner, before a barrier) wrote
    } else {
#pragma unroll
      for (int s = 0; s < KSZ; ++s) zb[s] = dz[s];
    }
    // This wave's output blocks: MBW of them from block mb0 (FS: its half).
    constexpr int MBW = MB / NFH, NFW = MBW * KSZ;
    const int mb0 = fh * MBW;
    const char* wb =
        reinterpret_cast<const char*>(wfr) + opaque((Gm::dfrag_off(l) * 64 + lane) * 16 + mb0 * KSZ * 1024);
    f16x8 fq[NQ];
#pragma unroll
    for (int t = 0; t < NQ; ++t) fq[t] = *reinterpret_cast<const f16x8*>(wb + t * 1024);
    f32x16 acc[2];
#pragma unroll
    for (int j = 0; j <= MBW; ++j) {
      if (j < MBW) {
        f32x16 a = {};
#pragma unroll
        for (int s = 0; s < KSZ; ++s) {
          const int t = j * KSZ + s;
          a = mfma32x32x16<N::bf>(fq[t % NQ], (DZL || Gm::FS) ? zread(s) : zb[s], a);
          if (t + NQ < NFW) fq[t % NQ] = *reinterpret_cast<const f16x8*>(wb + (t + NQ) * 1024);
        }
        if constexpr (DZL || Gm::FS)
          dgrad_epilogue<l, HA, B>(mb0 + j, j, a, dzn, tout);
        else
          acc[j & 1] = a;
      }
      if (!(DZL || Gm::FS) && j > 0) dgrad_epilogue<l, HA, B>(mb0 + j - 1, j - 1, acc[(j - 1) & 1], dzn, tout);
      if (j < MBW) {
        // Per MFMA: the MFMA, the read it frees a ring slot for, a share of
        // the previous block's epilogue.
#pragma unroll
        for (int s = 0; s < KSZ; ++s) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          if (j * KSZ + s + NQ < NFW) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          if (!(DZL || Gm::FS) && j > 0) __builtin_amdgcn_sched_group_barrier(0x002, 160 / KSZ, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // First round with per-layer prefetch: every layer's rows.
  template <int l>
  __device__ __forceinline__ void prefetch_all(int64_t r0) {
    if constexpr (Gm::RC && l == L - 1) {
      // recomputed every round
    } else if constexpr (l >= 1 || SEG) {
      load_h<l>(r0);
    } else if constexpr (!SHX) {  // (SHX: each round loads its own x)
      load_x(r0);
    }
    if constexpr (l > 0) prefetch_all<l - 1>(r0);
  }

  template <int l>
  __device__ __forceinline__ void phases_from(f16x8 (&dz)[KSM], f16x8 (&dzn)[KSM]) {
    phase<l>(dz, dzn);
    if constexpr (l > 0) phases_from<l - 1>(dzn, dz);
  }

  // Recompute mode, start of a round: hbuf holds h_{L-2} (fp32, natural
  // units, as the stash keeps it); replace it by h_{L-1} = softplus(h_{L-2}
  // W_{L-2}).  The MFMA operands are those of the forward -- h_{L-2} in base-2
  // units packed to fp16 (the stash holds that value times ln 2) against the
  // unscaled fragments -- and the stored value is sp2 of the product times
  // ln 2 (u itself past 2^u's overflow, as in the forward's exact form).  The
  // fp32 round trip through ln 2 can move a packed operand by one fp16 ulp,
  // so h_{L-1} agrees with the stashed value to fp16 operand rounding, not
  // bit for bit.  Where some operand of the wave would overflow fp16 (h above
  // ~45400), the operands are halved and the products doubled, as the
  // forward's exact form does.
  // FIX: the exact form (sp2_fix per value); the fast form instead tracks the
  // largest u and returns whether some u reached 128 (2^u overflowed), in
  // which case the caller reloads h_{L-2} and runs the exact form.
  template <bool HALF, bool FIX>
  __device__ __forceinline__ bool recompute_t() {
    constexpr int l = L - 2;
    constexpr int KSI = N::d[l] / 16, MBO = N::d[l + 1] / 32;
    constexpr float sc = HALF ? 0.5f * kLog2e : kLog2e;
    f16x8 bop[KSI];
#pragma unroll
    for (int s = 0; s < KSI; ++s)
      bop[s] = pack8<N::bf>(hbuf[0][s][0] * sc, hbuf[0][s][1] * sc, hbuf[0][s][2] * sc, hbuf[0][s][3] * sc,
                     hbuf[0][s][4] * sc, hbuf[0][s][5] * sc, hbuf[0][s][6] * sc, hbuf[0][s][7] * sc);
    // Forward A fragment (output block mbo over W_l's columns, K-step so
    // over its rows): lane (i, g) needs W_l[16 so + 8g + j][outfeat(mbo, i)],
    // j = 0..7.  W_l is staged for dgrad with 16 contiguous bytes of a row per
    // lane (fragment (mb_d, s_d), lane (i_d, g_d): W_l[outfeat(mb_d, i_d)]
    // [16 s_d + 8 g_d + 0..7]), so 4 consecutive columns of one row are 8
    // contiguous bytes there, and two ds_read_b64_tr_b16 per fragment gather
    // the transpose.  Addressing lane u = a + 4e of a 16-lane group q serves
    // result lanes 4a .. 4a+3 with row 16 so + 8 (q >> 1) + 4k + e (read k)
    // and columns outfeat(mbo, 16 (q & 1) + 4a) + 0..3 = 32 mbo + 16 (q & 1) +
    // 8 (a & 1) + 4 (a >> 1) + 0..3.  That row sits in dgrad block mb_d =
    // so >> 1 at lane i_d = 16 (so & 1) + h(r) (h inverts outfeat within 16
    // rows), the columns in K-step s_d = 2 mbo + (q & 1), half g_d = a & 1,
    // bytes 8 (a >> 1) ..: a lane-dependent byte offset lk[k] plus a
    // compile-time one per (mbo, so).
    constexpr int KSD = Gm::dks(l);  // K-steps of W_l's dgrad fragments (its columns)
    int lk[2];
    {
      const int q = lane >> 4, u = lane & 15, a = u & 3, e = u >> 2;
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int r = 8 * (q >> 1) + 4 * k + e;
        const int h = 8 * ((r >> 2) & 1) + 4 * ((r >> 3) & 1) + (r & 3);
        lk[k] = Gm::dfrag_off(l) * 1024 + (q & 1) * 1024 + (32 * (a & 1) + h) * 16 + 8 * (a >> 1);
      }
    }
    const char* wb = reinterpret_cast<const char*>(wfr);
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    // Software pipeline over the 32-feature blocks: block mb's MFMA chain
    // shares a scheduling region with block mb - 1's activations, and the
    // fences keep the compiler from hoisting later blocks' fragment reads
    // (all 32 at once would not fit beside the weight-gradient accumulators).
    f32x16 acc[2];
    float umax = -INFINITY;
#pragma unroll
    for (int mb = 0; mb <= MBO; ++mb) {
      if (mb < MBO) {
        const char* b0 = wb + opaque(lk[0]);
        const char* b1 = wb + opaque(lk[1]);
        f32x16 a = {};
#pragma unroll
        for (int s = 0; s < KSI; ++s) {
          const int off = (s >> 1) * KSD * 1024 + 2 * mb * 1024 + 256 * (s & 1);  // a constant after unrolling
          const s16x4 t0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) s16x4*)const_cast<char*>(b0 + off));
          const s16x4 t1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) s16x4*)const_cast<char*>(b1 + off));
          a = mfma32x32x16<N::bf>(__builtin_bit_cast(f16x8, __builtin_shufflevector(t0, t1, 0, 1, 2, 3, 4, 5, 6, 7)),
                                  bop[s], a);
        }
        acc[mb & 1] = a;
      }
      if (mb > 0) {
        // Registers 0..7: features 32q + 8g + [0..7] (K-step 2q); 8..15: K-step 2q + 1.
        const int q = mb - 1;
        const f32x16& a = acc[q & 1];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float u0 = HALF ? 2.0f * a[j] : a[j], u1 = HALF ? 2.0f * a[8 + j] : a[8 + j];
          if constexpr (FIX) {
            hbuf[0][2 * q][j] = sp2_fix(u0, sp2(u0)) * kLn2;
            hbuf[0][2 * q + 1][j] = sp2_fix(u1, sp2(u1)) * kLn2;
          } else {
            hbuf[0][2 * q][j] = sp2(u0) * kLn2;
            hbuf[0][2 * q + 1][j] = sp2(u1) * kLn2;
            umax = fmaxf(umax, fmaxf(u0, u1));
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    return !FIX && __builtin_amdgcn_ballot_w64(umax >= 128.0f) != 0;
  }
  template <bool HALF>
  __device__ __forceinline__ void recompute_h() {
    if (__builtin_expect(recompute_t<HALF, false>(), 0)) {
      // Some 2^u overflowed: h_{L-2} again (an L2 hit), then the exact form.
      load_h<L - 2>(row0);
      recompute_t<HALF, true>();
    }
  }
  __device__ __forceinline__ void recompute() {
    constexpr int KSI = N::d[L - 2] / 16;
    float m = 0.0f;
#pragma unroll
    for (int s = 0; s < KSI; ++s)
#pragma unroll
      for (int j = 0; j < 8; j += 2) m = fmaxf(m, fmaxf(hbuf[0][s][j], hbuf[0][s][j + 1]));
    if (!N::bf && __builtin_amdgcn_ballot_w64(m * kLog2e > 65504.0f) != 0)  // bf16 has fp32's range
      recompute_h<true>();
    else
      recompute_h<false>();
    // Rows past M read h_{L-2} = 0 and would recompute softplus(0) = ln 2,
    // where a stash reads 0: with a broadcast dout (row stride 0) those rows
    // see a nonzero gradient, so their h_{L-1} must be 0 as well.
    if (nrows_at(row0) < 32 && row0 + n >= p.M) {
#pragma unroll
      for (int s = 0; s < N::d[L - 1] / 16; ++s)
#pragma unroll
        for (int j = 0; j < 8; ++j) hbuf[0][s][j] = 0.0f;
    }
  }

  // Recompute under the feature split (see BwdGeom::dzr): h_{L-1}'s half of
  // this wave from all of h_{L-2} (its half in buffer L-2, the partner's
  // through the second dz tile, halved operands), into buffer L-1: the
  // exact form, products doubled.
  __device__ __forceinline__ void recompute_fs_t(const f16* th) {
    constexpr int l = L - 2;
    constexpr int KSI = N::d[l] / 16, MBO = N::d[l + 1] / 32 / NFH;
    constexpr int KSD = Gm::dks(l);
    const int zr = wsw, zsw = swz(zr, FZ);
    int lk[2];
    {
      const int q = lane >> 4, u = lane & 15, a = u & 3, e = u >> 2;
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int r = 8 * (q >> 1) + 4 * k + e;
        const int h = 8 * ((r >> 2) & 1) + 4 * ((r >> 3) & 1) + (r & 3);
        lk[k] = Gm::dfrag_off(l) * 1024 + (q & 1) * 1024 + (32 * (a & 1) + h) * 16 + 8 * (a >> 1) +
                2 * fh * MBO * 1024;  // (this wave's first output block)
      }
    }
    const char* wb = reinterpret_cast<const char*>(wfr);
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    f32x16 acc[2];
#pragma unroll
    for (int mb = 0; mb <= MBO; ++mb) {
      if (mb < MBO) {
        const char* b0 = wb + opaque(lk[0]);
        const char* b1 = wb + opaque(lk[1]);
        f32x16 a = {};
#pragma unroll
        for (int s = 0; s < KSI; ++s) {
          const int off = (s >> 1) * KSD * 1024 + 2 * mb * 1024 + 256 * (s & 1);  // a constant after unrolling
          const s16x4 t0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) s16x4*)const_cast<char*>(b0 + off));
          const s16x4 t1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) s16x4*)const_cast<char*>(b1 + off));
          const f16x8 bo = *reinterpret_cast<const f16x8*>(th + zr * FZ + ((16 * s + 8 * g) ^ zsw));
          a = mfma32x32x16<N::bf>(__builtin_bit_cast(f16x8, __builtin_shufflevector(t0, t1, 0, 1, 2, 3, 4, 5, 6, 7)),
                                  bo, a);
        }
        acc[mb & 1] = a;
      }
      if (mb > 0) {
        const int q = mb - 1;
        const f32x16& a = acc[q & 1];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float u0 = 2.0f * a[j], u1 = 2.0f * a[8 + j];
          hbuf[L - 1][2 * q][j] = sp2_fix(u0, sp2(u0)) * kLn2;
          hbuf[L - 1][2 * q + 1][j] = sp2_fix(u1, sp2(u1)) * kLn2;
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  __device__ __forceinline__ void recompute_fs() {
    constexpr int l = L - 2;
    constexpr int KW = N::d[l] / 16 / NFH;
    static_assert(PF && DZL, "buffers L-2 and L-1, the second dz tile");
    // The operands are always halved (and the products doubled), so every
    // h_{L-2} the forward can produce (up to ~90,800) fits fp16 without a
    // workgroup-wide decision; only values below ~8.5e-5, whose products
    // are negligible, lose bits as fp16 subnormals.  The tile was last read
    // before the previous round's last barriers.
    f16* const th = tz + FZ * R;  // the second dz tile
    {
      constexpr float sc = 0.5f * kLog2e;
      f16x8 v[KW];
#pragma unroll
      for (int s = 0; s < KW; ++s)
        v[s] = pack8<N::bf>(hbuf[l][s][0] * sc, hbuf[l][s][1] * sc, hbuf[l][s][2] * sc, hbuf[l][s][3] * sc,
                            hbuf[l][s][4] * sc, hbuf[l][s][5] * sc, hbuf[l][s][6] * sc, hbuf[l][s][7] * sc);
      xwrite<FZ>(th, v, fh * KW);
    }
    __syncthreads();  // both halves of every row's operands are in the tile
    // The exact form at once (two more VALU per value than the fast form
    // and its overflow check; a second instance of the loop for the rare
    // rerun did not fit beside the rest).
    recompute_fs_t(th);
    // Rows past M: h_{L-1} = 0 as a stash would hold (see recompute()).
    if (nrows_at(row0) < 32 && row0 + n >= p.M) {
#pragma unroll
      for (int s = 0; s < N::d[L - 1] / 16 / NFH; ++s)
#pragma unroll
        for (int j = 0; j < 8; ++j) hbuf[L - 1][s][j] = 0.0f;
    }
  }

  __device__ __forceinline__ void round() {
    if constexpr (Gm::RC && Gm::FS)
      recompute_fs();
    else if constexpr (Gm::RC)
      recompute();
    f16x8 dz[KSM], dzn[KSM];
    if constexpr (DZL) {
      xwrite<FZ>(tz, gbuf, fh * KSLW);  // dz_{L-1} = dL/dout into tile 0
    } else {
#pragma unroll
      for (int s = 0; s < KSLW; ++s) dz[s] = gbuf[s];
    }
    if constexpr (SHX)
      load_x(row0);  // this round's x into the buffer dL/dout left
    else if constexpr (PF)
      load_dout(row0 + rstep);
    phases_from<L - 1>(dz, dzn);
  }

  // Adds one accumulated 32x32 tile (ti, to) of dW_l to global memory, or
  // stores it into this workgroup's partial-sum block (p.part non-null).
  template <int l>
  __device__ __forceinline__ void flush_tile(const f32x16& acc, int ti, int to) const {
    const int K = dw_(l), NO = dw_(l + 1);
    int64_t welems = N::weight_elems(), woff = Gm::woff(l);
    if constexpr (N::gen) {  // partial-sum blocks laid out with the true widths
      welems = 0;
      woff = 0;
#pragma unroll
      for (int i = 0; i < N::L; ++i) {
        if (i < l) woff += (int64_t)p.dims[i] * p.dims[i + 1];
        welems += (int64_t)p.dims[i] * p.dims[i + 1];
      }
    }
    const int fo = 32 * to + (lane & 31);
    // C layout: lane (o, g) holds rows 8a + 4g + b of its column, register 4a + b.
    if (p.part) {
      // Buffer stores over this workgroup's block of dW_l: a per-lane offset
      // (column, g) and a wave-uniform one per register, so the stores need
      // no 64-bit addresses.  Each element goes through an opaque copy:
      // stores of single accumulator elements have been compiled as stores
      // of element 0.
      const rsrc_t r = make_rsrc(p.part + (int64_t)blockIdx.x * welems + woff, (uint32_t)(K * NO * 4));
      const int vo = (4 * g * NO + fo) * 4;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int fr = 32 * ti + 8 * (e >> 2) + (e & 3);
        float t = acc[e];
        asm volatile("" : "+v"(t));
        if (fr + 4 * g < K && fo < NO)
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, t), r, vo, fr * NO * 4, 0);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int fi = 32 * ti + 8 * (e >> 2) + 4 * g + (e & 3);
        if (fi < K && fo < NO) unsafeAtomicAdd(p.dw[l] + (int64_t)fi * NO + fo, acc[e]);
      }
    }
  }

  template <int l>
  __device__ __forceinline__ void flush_all() const {
    flush<l>();
    if constexpr (l + 1 < L) flush_all<l + 1>();
  }
  // Adds this wave's tiles of dW_l to global memory (fp32 atomics) or
  // stores them into the workgroup's partial-sum block.
  template <int l>
  __device__ __forceinline__ void flush() const {
    constexpr int OFF = Gm::tpw_off(l);
    if constexpr (Gm::quad(l)) {
      constexpr int QO = Gm::wob(l) / 2;
#pragma unroll
      for (int k = 0; k < Gm::quads(l) / NW; ++k) {
        const int q = wid + k * NW;
        const int ti = 2 * (q / QO), to = 2 * (q % QO);
        flush_tile<l>(wacc[OFF + 4 * k + 0], ti, to);
        flush_tile<l>(wacc[OFF + 4 * k + 1], ti, to + 1);
        flush_tile<l>(wacc[OFF + 4 * k + 2], ti + 1, to);
        flush_tile<l>(wacc[OFF + 4 * k + 3], ti + 1, to + 1);
      }
    } else {
      constexpr int WOB = Gm::wob(l);
#pragma unroll
      for (int k = 0; k < Gm::tpw(l); ++k) {
        const int t = wid + k * NW;
        if (t < Gm::tiles(l)) flush_tile<l>(wacc[OFF + k], t / WOB, t % WOB);
      }
    }
  }
};


template <class N, int NW, bool DX, bool SEG>
__global__ __launch_bounds__(NW * 64) void bwd_kernel(BwdParams p) {
  using Gm = BwdGeom<N, NW, DX, SEG>;
  static_assert(Gm::valid(), "unsupported backward shape");
  constexpr int R = Gm::R;
  __shared__ f16x8 wfr[Gm::ndfrag() * 64];
  __shared__ f16 ta[Gm::fa() * R];
  __shared__ f16 tz[Gm::fz() * R * (Gm::dzl() ? 2 : 1)];
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  f32x16 wacc[Gm::ntpw()];
#pragma unroll
  for (int k = 0; k < Gm::ntpw(); ++k) wacc[k] = (f32x16){};
  BwdWave<N, NW, DX, SEG> wv{p, wfr, ta, tz, lane, lane & 31, lane >> 5, wid, 0, (int64_t)gridDim.x * R, 0, {}, 0, wacc};
  wv.init_slots();

  // Every wave of a workgroup runs the same rounds (the barriers need all of them).
  // The weight staging's loads (L2 hits once any workgroup has read W) are
  // issued first and the first round's rows right after them, so the rows
  // stream in while the staging completes: the LDS writes of the staging
  // wait for the weights alone (memory operations are counted in issue
  // order).
  const int64_t nrounds = (p.M + R - 1) / R;
  {
    f16x8 sv[N::L][DgradStage<N, Gm>::template per<NW * 64>()];
    dgrad_load_all<N, Gm, NW * 64>(p, sv);
    wv.row0 = (int64_t)blockIdx.x * R + wv.rb * 32;
    wv.load_dout(wv.row0);
    if constexpr (BwdWave<N, NW, DX, SEG>::PF) {
      wv.template prefetch_all<N::L - 1>(wv.row0);
    } else if constexpr (Gm::RC) {
      wv.template load_h<N::L - 2>(wv.row0);
    } else if constexpr (N::L >= 2) {
      wv.template load_h<N::L - 1>(wv.row0);
    }
    dgrad_store_all<N, Gm, NW * 64>(sv, wfr);
  }
  __syncthreads();
  for (int64_t rnd = blockIdx.x; rnd < nrounds; rnd += gridDim.x) {
    wv.round();
    wv.row0 += wv.rstep;
  }
  wv.template flush_all<0>();
}

// Sums the per-workgroup weight-gradient partials into dw.  A workgroup owns
// kCombineCols consecutive dW elements; its kCombineGroups thread groups each
// sum every kCombineGroups-th partial (consecutive threads, consecutive
// elements: a wave's load reads 256 contiguous bytes), the group sums meet in
// LDS, and one thread per element adds the total to dw with a plain
// read-modify-write -- each element has exactly one owner, so no atomics.
constexpr int kCombineCols = 64, kCombineGroups = 8;
struct CombineLayout {
  int L;
  int64_t nelem;                    // sum_l d[l] * d[l+1]
  int64_t off[kMaxLayersHost + 1];  // element offset of dW_l; off[L] = nelem
  float* dw[kMaxLayersHost];
};

__global__ __launch_bounds__(kCombineCols* kCombineGroups) void bwd_combine_kernel(const float* __restrict__ part,
                                                                                   int G, CombineLayout lay,
                                                                                   int write) {
  __shared__ float red[kCombineGroups][kCombineCols];
  const int c = threadIdx.x % kCombineCols, q = threadIdx.x / kCombineCols;
  const int64_t e = (int64_t)blockIdx.x * kCombineCols + c;
  const bool live = e < lay.nelem;
  float s[4] = {};
  if (live) {
    int g = q;
    for (; g + 3 * kCombineGroups < G; g += 4 * kCombineGroups) {
#pragma unroll
      for (int i = 0; i < 4; ++i) s[i] += part[(int64_t)(g + i * kCombineGroups) * lay.nelem + e];
    }
    for (; g < G; g += kCombineGroups) s[0] += part[(int64_t)g * lay.nelem + e];
  }
  red[q][c] = (s[0] + s[1]) + (s[2] + s[3]);
  __syncthreads();
  if (q != 0 || !live) return;
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < kCombineGroups; ++i) sum += red[i][c];
  int l = 0;
#pragma unroll
  for (int i = 1; i < kMaxLayersHost; ++i)
    if (i < lay.L && e >= lay.off[i]) l = i;
  float* d = lay.dw[l] + (e - lay.off[l]);
  *d = write ? sum : *d + sum;  // MLPMK_BWD_WRITE_DW: written, else accumulated
}

// Clears the dW blocks of a launch whose workgroups add their partial sums
// with atomics straight into dw, when dw is to be written (=).
__global__ __launch_bounds__(256) void bwd_zero_dw_kernel(CombineLayout lay) {
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < lay.nelem;
       e += (int64_t)gridDim.x * blockDim.x) {
    int l = 0;
#pragma unroll
    for (int i = 1; i < kMaxLayersHost; ++i)
      if (i < lay.L && e >= lay.off[i]) l = i;
    lay.dw[l][e - lay.off[l]] = 0.0f;
  }
}

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------


typedef Net<128, 128, 128, 128> BNet3L128;
typedef Net<128, 128, 128, 128, 128, 128> BNet5L128;
typedef Net<128, 128, 128> BNet2L128;  // layers 4..3 of the 5-layer network
typedef Net<32, 64, 64, 16> BNetNarrow;

template <class N>
static bool bdims_match(int L, const int* dims) {
  if (L != N::L) return false;
  for (int i = 0; i <= L; ++i)
    if (dims[i] != N::d[i]) return false;
  return true;
}

// An empty batch with MLPMK_BWD_WRITE_DW: the gradient of no rows, dW = 0.
int bwd_clear_dw(int L, const int* dims, float* const* dw, hipStream_t st) {
  CombineLayout lay = {};
  lay.L = L;
  int64_t o = 0;
  for (int l = 0; l < L; ++l) {
    lay.off[l] = o;
    o += (int64_t)dims[l] * dims[l + 1];
    lay.dw[l] = dw[l];
  }
  lay.off[L] = lay.nelem = o;
  (void)hipGetLastError();
  hipLaunchKernelGGL(bwd_zero_dw_kernel, dim3((unsigned)((lay.nelem + 255) / 256)), dim3(256), 0, st, lay);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MLPMK_OK : hip_fail(e, "dW clear kernel launch");
}

// Grid of the persistent backward: one workgroup per round of R rows, at
// most CUs x occupancy.
template <class N, int NW, bool DX, bool SEG>
static int bwd_grid(int64_t M, int* grid) {
  constexpr int kMaxDev = 64;
  static int occ_cache[kMaxDev];  // 0 = unknown; benign race (idempotent value)
  int cus = 0;
  int rc = current_device_cus(&cus);
  if (rc != MLPMK_OK) return rc;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  const void* kern = reinterpret_cast<const void*>(&bwd_kernel<N, NW, DX, SEG>);
  int occ = (dev >= 0 && dev < kMaxDev) ? occ_cache[dev] : 0;
  if (occ <= 0) {
    rc = kernel_occupancy(kern, NW * 64, &occ);
    if (rc != MLPMK_OK) return rc;
    if (dev >= 0 && dev < kMaxDev) occ_cache[dev] = occ;
  }
  constexpr int R = BwdGeom<N, NW, DX, SEG>::R;
  const int64_t nrounds = (M + R - 1) / R;
  const int64_t cap = (int64_t)cus * occ;
  *grid = (int)(nrounds < cap ? nrounds : cap);
  return MLPMK_OK;
}

// Below this many workgroups the fp32 atomics of the per-workgroup flush
// cost less than the second launch (M = 4096, 32 workgroups: 25.5 us with
// atomics, 29.8 us with the workspace), so the workspace goes unused.
constexpr int kPartialMinGrid = 64;

template <class N, int NW, bool DX, bool SEG = false>
static int launch_bwd(const BwdParams& p_in, hipStream_t st) {
  int grid = 0;
  int rc = bwd_grid<N, NW, DX, SEG>(p_in.M, &grid);
  if (rc != MLPMK_OK) return rc;
  BwdParams p = p_in;
  if (grid < kPartialMinGrid) p.part = nullptr;
  // The dW blocks back to back with the layers' true widths (the same
  // offsets flush_tile writes the partials at).
  CombineLayout lay = {};
  lay.L = N::L;
  {
    int64_t o = 0;
    for (int l = 0; l < N::L; ++l) {
      lay.off[l] = o;
      o += N::gen ? (int64_t)p.dims[l] * p.dims[l + 1] : (int64_t)N::d[l] * N::d[l + 1];
      lay.dw[l] = p.dw[l];
    }
    lay.off[N::L] = lay.nelem = o;
  }
  (void)hipGetLastError();
  hipError_t e = hipSuccess;
  if (p.write_dw && !p.part) {  // atomics straight into dw: clear it first
    hipLaunchKernelGGL(bwd_zero_dw_kernel, dim3((unsigned)((lay.nelem + 255) / 256)), dim3(256), 0, st, lay);
    e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "dW clear kernel launch");
  }
  hipLaunchKernelGGL((bwd_kernel<N, NW, DX, SEG>), dim3(grid), dim3(NW * 64), 0, st, p);
  e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "bwd kernel launch");
  if (p.part) {
    hipLaunchKernelGGL(bwd_combine_kernel, dim3((unsigned)((lay.nelem + kCombineCols - 1) / kCombineCols)),
                       dim3(kCombineCols * kCombineGroups), 0, st, p.part, grid, lay, p.write_dw);
    e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "bwd combine kernel launch");
  }
  return MLPMK_OK;
}

// Waves per workgroup of the backward for N: the 8-wave feature split where
// its geometry is valid (dz through LDS, whole 64-feature halves), else 4.
template <class N, bool DX, bool SEG = false>
constexpr int bwd_waves() {
  return BwdGeom<N, 8, DX, SEG>::valid() ? 8 : 4;
}

template <class N>
static int launch_bwd_any(const BwdParams& p, hipStream_t st) {
  return p.dx ? launch_bwd<N, bwd_waves<N, true>(), true>(p, st) : launch_bwd<N, bwd_waves<N, false>(), false>(p, st);
}

static int64_t weight_elems_of(int L, const int* dims) {
  int64_t e = 0;
  for (int l = 0; l < L; ++l) e += (int64_t)dims[l] * dims[l + 1];
  return e;
}

// Partial-sum bytes: one block of `welems` floats (the dW blocks at their
// true widths) per workgroup of the grid.
template <class N, int NW, bool DX, bool SEG = false>
static int partial_bytes(int64_t M, int64_t welems, int64_t* bytes) {
  int grid = 0;
  const int rc = bwd_grid<N, NW, DX, SEG>(M, &grid);
  if (rc == MLPMK_OK) *bytes = (int64_t)grid * welems * (int64_t)sizeof(float);
  return rc;
}

template <class N>
static int bwd_workspace_any(int64_t M, bool dx, int64_t welems, int64_t* bytes) {
  return dx ? partial_bytes<N, bwd_waves<N, true>(), true>(M, welems, bytes)
            : partial_bytes<N, bwd_waves<N, false>(), false>(M, welems, bytes);
}

// Deeper networks in two launches: layers L-1..S as a segment (kernel A, the
// top L - S layers), whose fp16 dz_{S-1} goes through the workspace to
// layers S-1..0 (kernel B, the S-layer network with dz_{S-1} as its output
// gradient); S = BOT::L.  The 5-layer 128-wide network splits at S = 3: a
// 2-layer segment and the 3-layer network, both on the 8-wave kernel (four
// dgrad weight blocks and the exchange tiles would not fit the 160 KiB of
// one workgroup together).  Runtime-width networks split at S = 2.
// Workspace: dz_{S-1} [M, d[S] <= 128] fp16, then the weight-gradient
// partials of whichever launch needs more (the launches run in stream
// order, so they share the block).
static int64_t dz_bytes(int64_t M) { return (M * 128 * 2 + 255) / 256 * 256; }

template <class TOP, class BOT>
static int bwd_split_workspace(int L, const int* dims, int64_t M, bool dx, int64_t* bytes) {
  constexpr int S = BOT::L;
  int64_t a = 0, b = 0;
  int rc = partial_bytes<TOP, bwd_waves<TOP, true, true>(), true, true>(M, weight_elems_of(L - S, dims + S), &a);
  if (rc != MLPMK_OK) return rc;
  const int64_t wb = weight_elems_of(S, dims);
  rc = bwd_workspace_any<BOT>(M, dx, wb, &b);
  if (rc != MLPMK_OK) return rc;
  *bytes = dz_bytes(M) + (a > b ? a : b);
  return MLPMK_OK;
}

template <class TOP, class BOT>
static int launch_bwd_split(const BwdParams& p, int L, hipStream_t st) {
  constexpr int S = BOT::L;
  static_assert(TOP::L >= 2 && S >= 2, "segment shapes");
  if (L != TOP::L + S) return fail(MLPMK_ERR_UNSUPPORTED_SHAPE, "split backward: %d layers", L);
  if (!p.part)
    return fail(MLPMK_ERR_INVALID_ARG,
                "a backward of more than 3 layers passes dz between two launches through the workspace: "
                "use mlpmk_bwd_ws");
  char* const ws = reinterpret_cast<char*>(p.part);
  _Float16* const dzs = reinterpret_cast<_Float16*>(ws);
  float* const part = reinterpret_cast<float*>(ws + dz_bytes(p.M));
  BwdParams a = {};
  for (int l = 0; l < L - S; ++l) {
    a.w[l] = p.w[S + l];
    a.dw[l] = p.dw[S + l];
  }
  for (int l = 0; l + 1 < L - S; ++l) a.stash[l] = p.stash[S + l];  // h_{S+1} .. h_{L-1}
  for (int l = 0; l <= L - S; ++l) a.dims[l] = p.dims[S + l];
  a.h0 = p.stash[S - 1];  // h_S
  a.dout = p.dout;
  a.dout_stride = p.dout_stride;
  a.dx = dzs;
  a.M = p.M;
  a.part = part;
  a.write_dw = p.write_dw;
  int rc = launch_bwd<TOP, bwd_waves<TOP, true, true>(), true, true>(a, st);
  if (rc != MLPMK_OK) return rc;
  BwdParams b = {};
  b.x = p.x;
  for (int l = 0; l < S; ++l) {
    b.w[l] = p.w[l];
    b.dw[l] = p.dw[l];
  }
  for (int l = 0; l <= S; ++l) b.dims[l] = p.dims[l];
  for (int l = 0; l + 1 < S; ++l) b.stash[l] = p.stash[l];  // h_1 .. h_{S-1}
  b.dout = dzs;
  b.dout_stride = p.dims[S];
  b.dx = p.dx;
  b.M = p.M;
  b.part = part;
  b.write_dw = p.write_dw;
  return launch_bwd_any<BOT>(b, st);
}

// Runtime-width networks (compiled at width 128, true widths in BwdParams::dims):
// 2..5 layers, input and hidden widths multiples of 16 in [16, 128], any
// output width in [1, 128] -- the forward's generic shapes.  2 and 3 layers run
// in one launch, 4 and 5 in two (layers L-1..2, then 1..0).
typedef Gen<BNet2L128> GBNet2;
typedef Gen<BNet3L128> GBNet3;

bool bwd_generic_dims(int L, const int* dims) {
  if (L < 2 || L > 5) return false;
  for (int i = 0; i < L; ++i)
    if (dims[i] < 16 || dims[i] > 128 || dims[i] % 16 != 0) return false;
  return dims[L] >= 1 && dims[L] <= 128;
}

static bool bwd_exact_shape(int L, const int* dims) {
  return bdims_match<BNet3L128>(L, dims) || bdims_match<BNet5L128>(L, dims) || bdims_match<BNetNarrow>(L, dims);
}

// B: bf16 tensors (every shape is instantiated for both element formats; the
// grids, and so the workspace sizes, are taken from the kernels that run).
template <bool B>
static int bwd_workspace_t(int L, const int* dims, int64_t M, bool dx, int64_t* bytes) {
  typedef typename ElemNet<B, BNet3L128>::type N3;
  typedef typename ElemNet<B, BNet2L128>::type N2;
  typedef typename ElemNet<B, BNetNarrow>::type NN;
  typedef typename ElemNet<B, GBNet2>::type G2;
  typedef typename ElemNet<B, GBNet3>::type G3;
  const int64_t we = weight_elems_of(L, dims);
  // The 128-wide 3- and 5-layer backward may also run in recompute mode
  // (the last stash entry NULL, decided per call), whose kernel has its own
  // grid: size for the larger of the two.
  if (bdims_match<BNet3L128>(L, dims)) {
    int rc = bwd_workspace_any<N3>(M, dx, we, bytes);
    if (rc != MLPMK_OK) return rc;
    int64_t rcb = 0;
    rc = bwd_workspace_any<Recompute<N3>>(M, dx, we, &rcb);
    if (rc == MLPMK_OK && rcb > *bytes) *bytes = rcb;
    return rc;
  }
  if (bdims_match<BNet5L128>(L, dims)) {
    int rc = bwd_split_workspace<N2, N3>(L, dims, M, dx, bytes);
    if (rc != MLPMK_OK) return rc;
    int64_t rcb = 0;
    rc = bwd_split_workspace<Recompute<N2>, N3>(L, dims, M, dx, &rcb);
    if (rc == MLPMK_OK && rcb > *bytes) *bytes = rcb;
    return rc;
  }
  if (bdims_match<BNetNarrow>(L, dims)) return bwd_workspace_any<NN>(M, dx, we, bytes);
  if (bwd_generic_dims(L, dims)) {
    switch (L) {
      case 2: return bwd_workspace_any<G2>(M, dx, we, bytes);
      case 3: return bwd_workspace_any<G3>(M, dx, we, bytes);
      case 4: return bwd_split_workspace<G2, G2>(L, dims, M, dx, bytes);
      default: return bwd_split_workspace<G3, G2>(L, dims, M, dx, bytes);
    }
  }
  return fail(MLPMK_ERR_UNSUPPORTED_SHAPE, "no backward kernel for these widths");
}

bool tp_supported(int L, const int* dims, int dtype);
int tp_workspace_bytes(int L, const int* dims, int dtype, int64_t M, int64_t* bytes);
int tp_dispatch(int L, const int* dims, int dtype, const BwdParams& bp, void* ws, hipStream_t st);

static bool fused_supported(int L, const int* dims) {
  return bwd_exact_shape(L, dims) || bwd_generic_dims(L, dims);
}

// Batches up to this many rows take the two-pass backward (bwd_tp.hip) where
// both it and the one-pass megakernel exist: at a few thousand rows the
// megakernel runs one 128-row round per workgroup on M / 128 CUs.
#ifndef MLPMK_TP_MAX_ROWS
#define MLPMK_TP_MAX_ROWS 16384
#endif

// Which backward runs: 0 the one-pass megakernel, 1 the two-pass backward,
// -1 neither (an error).  fp32 tensors and widths above 128 have only the
// two-pass kernels; the recomputing backward (last stash entry NULL) only
// the one-pass ones.
static int bwd_path(int L, const int* dims, int dtype, int64_t M, bool recompute) {
  const bool tp = tp_supported(L, dims, dtype);
  const bool fused = dtype != MLPMK_DTYPE_F32 && fused_supported(L, dims);
  if (recompute) return fused ? 0 : -1;
  if (tp && (!fused || M <= MLPMK_TP_MAX_ROWS)) return 1;
  return fused ? 0 : -1;
}

int bwd_workspace_bytes(int L, const int* dims, int64_t M, bool dx, int dtype, int64_t* bytes) {
  const bool bf = dtype == MLPMK_DTYPE_BF16;
  int64_t fused = 0, two = 0;
  if (bwd_path(L, dims, dtype, M, false) == 1) {
    int rc = tp_workspace_bytes(L, dims, dtype, M, &two);
    if (rc != MLPMK_OK) return rc;
  }
  // The one-pass kernels (also for a recomputing call at a two-pass batch
  // size: whether the last stash entry is NULL is decided per call).
  if (dtype != MLPMK_DTYPE_F32 && fused_supported(L, dims)) {
    int rc = bf ? bwd_workspace_t<true>(L, dims, M, dx, &fused) : bwd_workspace_t<false>(L, dims, M, dx, &fused);
    if (rc != MLPMK_OK) return rc;
  }
  *bytes = fused > two ? fused : two;
  return MLPMK_OK;
}

// Library-owned workspace of mlpmk_bwd_noalloc, for callers that cannot
// allocate device memory (code under graph capture, serving loops, harnesses
// that forbid hipMalloc): the same kernels as mlpmk_bwd_ws, with this array
// in place of the caller's workspace.  Each device holds its own copy, at its
// own address, until the process ends.  Every call on a device shares it and
// leaves its contents behind; nothing in it needs to start at zero (every
// partial-sum block and the dz hand-over are written in full before they
// are read), and calls that overlap on one device (two streams) race.
static __device__ __align__(256) char scratch[MLPMK_NOALLOC_SCRATCH_BYTES];

// Device address of `scratch` on the current device.  In host code the
// array's name is only a stand-in for the symbol: the address comes from
// hipGetSymbolAddress, looked up once per device (on the device's first
// mlpmk_bwd_noalloc call, with that device current) and kept.
int scratch_workspace(void** ptr, int64_t* bytes) {
  constexpr int kMaxDev = 64;
  static std::atomic<void*> addr[kMaxDev];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDev) return fail(MLPMK_ERR_NO_DEVICE, "device %d: at most %d devices", dev, kMaxDev);
  void* a = addr[dev].load(std::memory_order_acquire);
  if (!a) {
    int cus = 0;
    int rc = current_device_cus(&cus);  // a gfx950 device, or no code object to look in
    if (rc != MLPMK_OK) return rc;
    e = hipGetSymbolAddress(&a, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!a) return fail(MLPMK_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL");
    addr[dev].store(a, std::memory_order_release);  // same value from every racing thread
  }
  *ptr = a;
  *bytes = MLPMK_NOALLOC_SCRATCH_BYTES;
  return MLPMK_OK;
}

bool bwd_supported_dims(int L, const int* dims) {
  return fused_supported(L, dims) || tp_supported(L, dims, MLPMK_DTYPE_F16);
}

// fp32 tensors: the two-pass backward's shapes (widths up to 128).
bool bwd_supported_dtype(int L, const int* dims, int dtype) {
  if (dtype == MLPMK_DTYPE_F32) return tp_supported(L, dims, dtype);
  return bwd_supported_dims(L, dims);
}

// The 3- and 5-layer 128-wide networks also run in recompute mode: with a
// NULL stash entry for h_{L-1} (the forward then does not write it) the
// backward recomputes it from h_{L-2} at the start of every round (for 5
// layers in the launch of layers 4..3), with or without dx.  The workspace
// size covers both kernels' grids (bwd_workspace_t).
bool bwd_recompute_supported(int L, const int* dims) {
  return bdims_match<BNet3L128>(L, dims) || bdims_match<BNet5L128>(L, dims);
}

template <bool B>
static int bwd_dispatch_t(int L, const int* dims, const BwdParams& p, hipStream_t st) {
  typedef typename ElemNet<B, BNet3L128>::type N3;
  typedef typename ElemNet<B, BNet2L128>::type N2;
  typedef typename ElemNet<B, BNetNarrow>::type NN;
  typedef typename ElemNet<B, GBNet2>::type G2;
  typedef typename ElemNet<B, GBNet3>::type G3;
  if (bdims_match<BNet3L128>(L, dims) && !p.stash[1]) return launch_bwd_any<Recompute<N3>>(p, st);
  // Without dx the 8-wave feature split (two waves per SIMD); with dx the
  // third layer's dgrad fragments leave no LDS for the second dz tile.
  if (bdims_match<BNet3L128>(L, dims)) return launch_bwd_any<N3>(p, st);
  if (bdims_match<BNet5L128>(L, dims) && !p.stash[3]) return launch_bwd_split<Recompute<N2>, N3>(p, L, st);
  if (bdims_match<BNet5L128>(L, dims)) return launch_bwd_split<N2, N3>(p, L, st);
  if (bdims_match<BNetNarrow>(L, dims)) return launch_bwd_any<NN>(p, st);
  if (bwd_generic_dims(L, dims)) {
    switch (L) {
      case 2: return launch_bwd_any<G2>(p, st);
      case 3: return launch_bwd_any<G3>(p, st);
      case 4: return launch_bwd_split<G2, G2>(p, L, st);
      default: return launch_bwd_split<G3, G2>(p, L, st);
    }
  }
  return fail(MLPMK_ERR_UNSUPPORTED_SHAPE, "no backward kernel for these widths");
}

int bwd_dispatch(int L, const int* dims, const BwdParams& p, int dtype, hipStream_t st) {
  const bool recompute = L > 2 && !p.stash[L - 2];
  int path = bwd_path(L, dims, dtype, p.M, recompute);
  // The two-pass backward hands dz between its passes through the
  // workspace: without one (mlpmk_bwd) the one-pass kernels run if they can.
  if (path == 1 && !p.part) path = (dtype != MLPMK_DTYPE_F32 && fused_supported(L, dims)) ? 0 : -2;
  if (path == 1) return tp_dispatch(L, dims, dtype, p, p.part, st);
  if (path == -2)
    return fail(MLPMK_ERR_INVALID_ARG,
                "this backward (fp32 tensors or widths above 128) hands dz between two passes through the "
                "workspace: use mlpmk_bwd_ws");
  if (path < 0) return fail(MLPMK_ERR_UNSUPPORTED_SHAPE, "no backward kernel for these widths and dtype");
  return dtype == MLPMK_DTYPE_BF16 ? bwd_dispatch_t<true>(L, dims, p, st) : bwd_dispatch_t<false>(L, dims, p, st);
}

}  // namespace mlpmk
