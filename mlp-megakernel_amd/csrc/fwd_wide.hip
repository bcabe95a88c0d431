// Host dispatch of the streamed-weight forward for widths above 128 (the
// kernels are in fwd_wide.h).  Workgroups of 8 waves (rounds of 256 rows, two
// waves per SIMD) from 256 rounds of them, i.e. batches that give every CU a
// round; below, workgroups of 4 waves (rounds of 128 rows, one wave per
// SIMD on twice as many CUs), compiled in fwd_wide_nw4.hip so that the two
// sets of kernels build in parallel.
#include "fwd_wide.h"

namespace mlpmk {

// Networks of 2..5 layers whose input and hidden widths are multiples of 16
// in [16, 256] and whose output width is in [1, 256], with some width above
// 128 (narrower ones have the resident-weight kernels of fwd.hip).
bool fwd_wide_dims(int L, const int* dims) {
  if (L < 2 || L > 5) return false;
  bool wide = false;
  for (int i = 0; i < L; ++i) {
    if (dims[i] < 16 || dims[i] > kWideMax || dims[i] % 16 != 0) return false;
    wide = wide || dims[i] > 128;
  }
  if (dims[L] < 1 || dims[L] > kWideMax) return false;
  return wide || dims[L] > 128;
}

int fwd_wide_dispatch_nw4(int L, const int* dims, const FwdParams& p, bool stash, bool bf, int cus, hipStream_t st,
                          LaunchInfo* info);

int fwd_wide_dispatch(int L, const int* dims, const FwdParams& p, bool stash, bool bf, hipStream_t st,
                      LaunchInfo* info) {
  if (!fwd_wide_dims(L, dims)) return fail(MLPMK_ERR_UNSUPPORTED_SHAPE, "no forward kernel for these widths");
  int cus = 0;
  const int rc = current_device_cus(&cus);
  if (rc != MLPMK_OK) return rc;
  if (p.M < (int64_t)256 * cus) return fwd_wide_dispatch_nw4(L, dims, p, stash, bf, cus, st, info);
  return wide_dispatch_nw<8>(L, dims, p, stash, bf, cus, st, info);
}

}  // namespace mlpmk
