// Forward megakernel host dispatch for fp16 and bf16 tensors (the kernels are
// templates in fwd_kernel.h; fp32 tensors dispatch through fwd_x3.hip).
#include "fwd_kernel.h"


// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------
#include "host_common.h"

namespace mlpmk {

// Runtime-width networks of 2..5 layers, compiled at width 128: any input
// and hidden widths that are multiples of 16 in [16, 128] (whole MFMA
// K-steps, so every width test is wave-uniform) and any output width in
// [1, 128] (the reference masks its output columns, kernel.py:86-87,121-123;
// its input and hidden widths are whole tiles, AGENTS.md:84-85).  GNet2 ..
// GNet5 (fwd_kernel.h) are those kernels.
bool fwd_generic_dims(int L, const int* dims) {
  if (L < 2 || L > 5) return false;
  for (int i = 0; i < L; ++i)
    if (dims[i] < 16 || dims[i] > 128 || dims[i] % 16 != 0) return false;
  return dims[L] >= 1 && dims[L] <= 128;
}

bool fwd_wide_dims(int L, const int* dims);
int fwd_wide_dispatch(int L, const int* dims, const FwdParams& p, bool stash, bool bf, hipStream_t st,
                      LaunchInfo* info);

bool fwd_supported_dims(int L, const int* dims) {
  return dims_match<Net3L128>(L, dims) || dims_match<Net5L128>(L, dims) ||
         dims_match<NetNarrow>(L, dims) || fwd_generic_dims(L, dims) || fwd_wide_dims(L, dims);
}

// The same for tensors of one element type: fp32 tensors run the split-operand
// kernels of fwd_x3.hip, whose widths are at most 128 (fwd_dispatch_f32).
bool fwd_supported_dtype(int L, const int* dims, int dtype) {
  if (dtype == MLPMK_DTYPE_F32) return dims_match<Net3L128>(L, dims) || fwd_generic_dims(L, dims);
  return fwd_supported_dims(L, dims);
}

int fwd_split_dispatch(int L, const int* dims, const FwdParams& p, bool stash, bool bf, hipStream_t st, int cus,
                       LaunchInfo* info);

// B: bf16 tensors (every shape is instantiated for both element formats).
template <bool B>
static int fwd_dispatch_t(int L, const int* dims, const FwdParams& p, bool stash, hipStream_t st, LaunchInfo* info) {
  if (dims_match<Net3L128>(L, dims))
    return launch_fwd_any<typename ElemNet<B, Net3L128>::type, 1, 12, 1, 8, 1>(p, stash, st, info);
  if (dims_match<Net5L128>(L, dims))
    return launch_fwd_any<typename ElemNet<B, Net5L128>::type, 1, 12, 1, 8, 1>(p, stash, st, info);
  if (dims_match<NetNarrow>(L, dims))
    return launch_fwd_any<typename ElemNet<B, NetNarrow>::type, 2, 16, 1, 16, 1>(p, stash, st, info);
  if (fwd_generic_dims(L, dims)) {
    switch (L) {
      // At most 8 waves (4 for the 5-layer stash kernel): the runtime
      // strides cannot fold into immediate offsets, and the 12-wave kernels
      // (168 VGPRs) spill.
      case 2: return launch_fwd_any<typename ElemNet<B, GNet2>::type, 1, 8, 1, 8, 1>(p, stash, st, info);
      case 3: return launch_fwd_any<typename ElemNet<B, GNet3>::type, 1, 8, 1, 8, 1>(p, stash, st, info);
      case 4: return launch_fwd_any<typename ElemNet<B, GNet4>::type, 1, 8, 1, 8, 1>(p, stash, st, info);
      default: return launch_fwd_any<typename ElemNet<B, GNet5>::type, 1, 8, 1, 4, 1>(p, stash, st, info);
    }
  }
  return fail(MLPMK_ERR_UNSUPPORTED_SHAPE, "no forward kernel for these widths");
}

int fwd_dispatch_f32(int L, const int* dims, const FwdParams& p, bool stash, hipStream_t st, LaunchInfo* info);

// dtype: element type of x, W and out (MLPMK_DTYPE_*).
int fwd_dispatch(int L, const int* dims, const FwdParams& p, bool stash, int dtype, hipStream_t st,
                 LaunchInfo* info) {
  if (dtype == MLPMK_DTYPE_F32) return fwd_dispatch_f32(L, dims, p, stash, st, info);
  const bool bf = dtype == MLPMK_DTYPE_BF16;
  // Widths above 128 (up to 256): the streamed-weight kernel (fwd_wide.hip).
  if (fwd_wide_dims(L, dims)) return fwd_wide_dispatch(L, dims, p, stash, bf, st, info);
  int cus = 0;
  const int rc = current_device_cus(&cus);
  if (rc != MLPMK_OK) return rc;
  // Small batches run the feature-split kernel (fwd_split.hip) when it has one
  // for these widths and batch size.
  const int rs = fwd_split_dispatch(L, dims, p, stash, bf, st, cus, info);
  if (rs != MLPMK_ERR_UNSUPPORTED_SHAPE) return rs;
  return bf ? fwd_dispatch_t<true>(L, dims, p, stash, st, info) : fwd_dispatch_t<false>(L, dims, p, stash, st, info);
}

}  // namespace mlpmk
