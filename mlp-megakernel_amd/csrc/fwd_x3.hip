// Forward megakernel for fp32 tensors on gfx950 (MI355X): the reference's
// INPUT_DTYPE = fp32 kernels (/root/reference/mlp_fused.md:159-166), whose
// launcher passes fp32 x on (/root/reference/kernel.py:130-138) and whose
// tl.dot rounds fp32 operands to TF32 (10-bit significand, fp32 exponent
// range).
//
// Every MFMA operand -- x, the weights and the hidden activations -- is
// split into bf16 hi + lo (hi = bf16(v), lo = bf16(v - hi)) and each product
// is hi*hi + hi*lo + lo*hi on v_mfma_f32_32x32x16_bf16: fp32's exponent
// range (|x| or h past fp16's 65,504 are ordinary values here) and a ~16-bit
// significand, with fp32 accumulation, softplus and output rows.  The fp32
// backward (bwd_tp.hip) uses the same operands, so a training step keeps
// fp32's range end to end.
//
// Mapping: the feature split of fwd_split.hip.  A workgroup of NWV waves
// (one per 32-feature output block of the widest layer, one per SIMD) runs
// 32-row blocks, persistent over the batch; wave w computes output features
// [32w, 32w + 32) of every layer in the transposed orientation (MFMA M =
// features, N = rows, K = input features), its A fragments (hi and lo) held
// in registers for the whole kernel where they fit (up to 3 layers) and
// read from L2 per block otherwise.  Layers hand their activations to the
// next as B operands through two LDS tiles [32 rows][features] (hi, lo).
//
// Softplus in base 2: u = z log2(e), softplus(z) = ln2 * sp2(u) with sp2(u)
// = log2(1 + 2^u), and u itself where 2^u overflows (u >= 128, z > 88.7; the
// reference's threshold branch, kernel.py:108, gives z there too).  The
// fp32 stash (training) holds softplus(z) as the backward reads it.
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
  static constexpr int NWV = nwv(), KSM = ksm(), TW = tw(), CH = TW / 8;
  static constexpr bool RES = L <= 3;  // fragments resident in registers
  static constexpr bool valid() {
    for (int i = 0; i < L; ++i)
      if (N::d[i] > 128 || N::d[i] % 16 != 0) return false;
    return L >= 2 && N::d[L] <= 128;
  }
};

template <class N>
struct FxWave {
  using G = FxGeo<N>;
  static constexpr int L = N::L, CH = G::CH, EM = EM_F32;
  const FwdParams& p;
  f16x8 (*tile)[2][32 * CH];  // [2][hi, lo][32 * CH]
  int lane, n, g, w;
  int par = 0;
  Opnd fr[G::RES ? L : 1][G::KSM];  // this wave's A fragments (output block w)
  Opnd B[G::KSM];                   // B operands of the current layer: row n

  __device__ __forceinline__ bool owns(int l) const { return 32 * w < dimw<N>(p, l + 1); }

  // Fragment (block w, K-step s) of layer l: lane (i, g) holds
  // W_l[16s + 8g + j][outfeat(w, i)], j = 0..7 -- for fixed (s, g, j) the 32
  // lanes of a half-wave read 32 consecutive columns of one row (128 bytes).
  // Rows past the true input width read zeros through the resource; columns
  // past the true output width are masked.
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
        v[j] = ok ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (row * Nout + col) * 4, 0, 0))
                  : 0.0f;
      }
      f[s] = make_op<EM>(v);
    }
  }
  template <int l = 0>
  __device__ __forceinline__ void load_all_frags() {
    if constexpr (l < L) {
      if (owns(l)) load_frags<l>(fr[l]);
      load_all_frags<l + 1>();
    }
  }

  // x rows from row0 as B operands: lane (n, g), K-step s: x[row n][16s + 8g + 0..7].
  __device__ __forceinline__ void load_x(int64_t row0) {
    const int D = dimw<N>(p, 0);
    const rsrc_t r = make_rsrc(reinterpret_cast<const float*>(p.x) + row0 * D, rows_at(p.M, row0, 32) * D * 4u);
#pragma unroll
    for (int s = 0; s < G::ks(0); ++s) {
      B[s] = load_op<EM>(r, (uint32_t)(n * D + 16 * s + 8 * g));
      if (N::gen && 16 * s + 8 * g >= D) B[s] = Opnd{f16x8{}, f16x8{}};
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

  // Layer l of one 32-row block: B holds the layer's input rows.  Owning
  // waves compute their 32 output features; hidden layers hand the whole
  // activation on through the tile.
  template <int l>
  __device__ __forceinline__ void layer(int64_t row0) {
    if (owns(l)) {
      f32x16 acc = {}, acc2 = {};  // two chains: even and odd K-steps
      if constexpr (G::RES) {
#pragma unroll
        for (int s = 0; s < G::ks(l); ++s) {
          if (s & 1)
            acc2 = mma<EM>(fr[l][s], B[s], acc2);
          else
            acc = mma<EM>(fr[l][s], B[s], acc);
        }
      } else {
        Opnd f[G::KSM];
        load_frags<l>(f);
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
      if constexpr (l + 1 < L) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const float u = acc[j] * kLog2e;
          v[j] = sp2_fix(u, sp2(u)) * kLn2;
        }
        if (p.stash[l]) store_row16(p.stash[l], dimw<N>(p, l + 1), row0, v);
        const Opnd lo = make_op<EM>(*reinterpret_cast<const float(*)[8]>(v));
        const Opnd hi = make_op<EM>(*reinterpret_cast<const float(*)[8]>(v + 8));
        tile[par][0][slot<CH>(n, 4 * w + g)] = lo.h;
        tile[par][0][slot<CH>(n, 4 * w + 2 + g)] = hi.h;
        tile[par][1][slot<CH>(n, 4 * w + g)] = lo.l;
        tile[par][1][slot<CH>(n, 4 * w + 2 + g)] = hi.l;
      } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = acc[j];
        store_row16(reinterpret_cast<float*>(p.out), dimw<N>(p, L), row0, v);
      }
    }
    if constexpr (l + 1 < L) {
      __syncthreads();  // the whole hidden activation of these rows is in the tile
      const int Wd = dimw<N>(p, l + 1);
#pragma unroll
      for (int s = 0; s < G::ks(l + 1); ++s) {
        B[s].h = tile[par][0][slot<CH>(n, 2 * s + g)];
        B[s].l = tile[par][1][slot<CH>(n, 2 * s + g)];
        // (past the true width the tile holds stale values: zero operands)
        if (N::gen && 16 * s + 8 * g >= Wd) B[s] = Opnd{f16x8{}, f16x8{}};
      }
      // The next hand-over writes the other tile: this one is read until
      // every wave has passed the next barrier.
      par ^= 1;
      layer<l + 1>(row0);
    }
  }
};

template <class N>
__global__ __launch_bounds__((FxGeo<N>::NWV * 64)) void fwd_x3_kernel(FwdParams p) {
  using G = FxGeo<N>;
  static_assert(G::valid(), "fp32-tensor forward shape");
  __shared__ f16x8 tile[2][2][32 * G::CH];
  const int lane = threadIdx.x & 63;
  FxWave<N> wv{p, tile, lane, lane & 31, lane >> 5, __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6))};
  const int64_t nblk = (p.M + 31) / 32;
  for (int64_t b = blockIdx.x; b < nblk; b += gridDim.x) {
    const int64_t row0 = b * 32;
    wv.load_x(row0);
    if constexpr (G::RES) {
      if (b == blockIdx.x) wv.template load_all_frags<>();
    }
    wv.template layer<0>(row0);
  }
}

}  // namespace tp

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------

namespace {

template <class N>
int launch_x3(const FwdParams& p, hipStream_t st, LaunchInfo* info) {
  using G = tp::FxGeo<N>;
  constexpr int kMaxDev = 64;
  static int occ_cache[kMaxDev];  // benign race: the value is idempotent
  int cus = 0;
  int rc = current_device_cus(&cus);
  if (rc != MLPMK_OK) return rc;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  int occ = (dev >= 0 && dev < kMaxDev) ? occ_cache[dev] : 0;
  if (occ <= 0) {
    rc = kernel_occupancy(reinterpret_cast<const void*>(&tp::fwd_x3_kernel<N>), G::NWV * 64, &occ);
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
  hipLaunchKernelGGL((tp::fwd_x3_kernel<N>), dim3(grid), dim3(G::NWV * 64), 0, st, p);
  e = hipGetLastError();
  return e == hipSuccess ? MLPMK_OK : hip_fail(e, "fp32 forward kernel launch");
}

}  // namespace

bool fwd_generic_dims(int L, const int* dims);

// fp32 tensors: every shape of the 128-wide kernels (the three compiled
// ones and the runtime-width networks of 2..5 layers).  The stash flag needs
// no separate kernel: NULL stash entries are simply not written.
int fwd_dispatch_f32(int L, const int* dims, const FwdParams& p, bool stash, hipStream_t st, LaunchInfo* info) {
  (void)stash;
  if (L == 3 && dims[0] == 128 && dims[1] == 128 && dims[2] == 128 && dims[3] == 128)
    return launch_x3<Net<128, 128, 128, 128>>(p, st, info);
  if (fwd_generic_dims(L, dims)) {  // (includes 5 x 128 and 32-64-64-16)
    switch (L) {
      case 2: return launch_x3<Gen<Net<128, 128, 128>>>(p, st, info);
      case 3: return launch_x3<Gen<Net<128, 128, 128, 128>>>(p, st, info);
      case 4: return launch_x3<Gen<Net<128, 128, 128, 128, 128>>>(p, st, info);
      default: return launch_x3<Gen<Net<128, 128, 128, 128, 128, 128>>>(p, st, info);
    }
  }
  return fail(MLPMK_ERR_UNSUPPORTED_SHAPE, "no fp32-tensor forward kernel for these widths (all at most 128)");
}

}  // namespace mlpmk
