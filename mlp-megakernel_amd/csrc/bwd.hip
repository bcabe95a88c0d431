// Backward megakernel (placeholder until the kernel lands): reports every
// shape as unsupported so callers fail loudly instead of computing anything.
#include "device_common.h"
#include "host_common.h"
#include "params.h"

namespace mlpmk {

bool bwd_supported_dims(int, const int*) { return false; }

int bwd_dispatch(int, const int*, const BwdParams&, hipStream_t) {
  return fail(MLPMK_ERR_UNSUPPORTED_SHAPE, "no backward kernel for these widths");
}

}  // namespace mlpmk
