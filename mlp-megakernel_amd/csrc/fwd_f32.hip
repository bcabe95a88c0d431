// Forward megakernel host dispatch for fp32 tensors (F32IO networks: fp32 x,
// W and out; fp16 MFMA operands, fp32 accumulation and softplus; the
// kernels are the templates of fwd_kernel.h).  The reference's kernels take
// fp32 tensors through INPUT_DTYPE (/root/reference/mlp_fused.md:159-166) and
// its launcher passes fp32 x on (/root/reference/kernel.py:130-138); there,
// tl.dot rounds fp32 operands to TF32, whose 10-bit mantissa the fp16
// operands here keep (with fp16's exponent range: |x|, scaled |W| and the
// hidden activations below 65,504, as on the fp16 path).
//
// Every batch size runs the persistent kernel (no feature-split kernel for
// fp32 tensors), at most 8 waves per workgroup: the fp32 x rows in flight
// take twice the registers of fp16 ones (and 4 where 8 would spill).
#include "fwd_kernel.h"

namespace mlpmk {

bool fwd_generic_dims(int L, const int* dims);

int fwd_dispatch_f32(int L, const int* dims, const FwdParams& p, bool stash, hipStream_t st, LaunchInfo* info) {
  // Waves per workgroup (inference / stash): 8 where the kernel fits 256
  // VGPRs without spilling, else 4.
  if (dims_match<Net3L128>(L, dims)) return launch_fwd_any<F32IO<Net3L128>, 1, 8, 1, 4, 1>(p, stash, st, info);
  if (dims_match<Net5L128>(L, dims)) return launch_fwd_any<F32IO<Net5L128>, 1, 8, 1, 4, 1>(p, stash, st, info);
  if (dims_match<NetNarrow>(L, dims)) return launch_fwd_any<F32IO<NetNarrow>, 1, 8, 1, 8, 1>(p, stash, st, info);
  if (fwd_generic_dims(L, dims)) {
    switch (L) {
      case 2: return launch_fwd_any<F32IO<GNet2>, 1, 8, 1, 4, 1>(p, stash, st, info);
      case 3: return launch_fwd_any<F32IO<GNet3>, 1, 4, 1, 4, 1>(p, stash, st, info);
      case 4: return launch_fwd_any<F32IO<GNet4>, 1, 8, 1, 4, 1>(p, stash, st, info);
      default: return launch_fwd_any<F32IO<GNet5>, 1, 4, 1, 4, 1>(p, stash, st, info);
    }
  }
  return fail(MLPMK_ERR_UNSUPPORTED_SHAPE, "no forward kernel for these widths");
}

}  // namespace mlpmk
