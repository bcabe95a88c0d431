// The streamed-weight forward's 4-wave kernels (rounds of 128 rows), for
// batches below 256 rounds of 256 rows; dispatched by fwd_wide.hip.
#include "fwd_wide.h"

namespace mlpmk {

int fwd_wide_dispatch_nw4(int L, const int* dims, const FwdParams& p, bool stash, bool bf, int cus, hipStream_t st,
                          LaunchInfo* info) {
  return wide_dispatch_nw<4>(L, dims, p, stash, bf, cus, st, info);
}

}  // namespace mlpmk
