// Kernel parameter blocks shared by the host dispatch and the kernels.
#pragma once
#include <stdint.h>

namespace mlpmk {

constexpr int kMaxLayersHost = 8;

struct FwdParams {
  const _Float16* x;
  _Float16* out;
  const _Float16* w[kMaxLayersHost];
  float* stash[kMaxLayersHost];  // stash[l] = h_{l+1}, fp32 [M, d[l+1]]; unused if no stash
  int64_t M;
  // The network's widths d[0] .. d[L].  Read only by the runtime-width
  // kernels (Gen networks), whose compile-time widths are padded to 128.
  int dims[kMaxLayersHost + 1];
};

}  // namespace mlpmk

namespace mlpmk {

struct BwdParams {
  const _Float16* x;
  const _Float16* w[kMaxLayersHost];
  const float* stash[kMaxLayersHost];  // stash[l] = h_{l+1}, fp32 [M, d[l+1]]
  const _Float16* dout;                // dL/dout; row r at dout + r * dout_stride
  int64_t dout_stride;                 // elements; 0 broadcasts row 0, -1 element 0
  _Float16* dx;                        // nullable
  float* dw[kMaxLayersHost];           // fp32 [d[l], d[l+1]], accumulated with atomics
  int64_t M;
  // Nonzero: dw is written (=), not accumulated into (MLPMK_BWD_WRITE_DW).
  int write_dw;
  // Null: every workgroup adds its weight-gradient partial sums to dw with
  // fp32 atomics.  Otherwise workgroup b stores them, laid out like the dW
  // blocks back to back, at part + b * (sum_l d[l] * d[l+1]), and a second
  // kernel sums the partials into dw.
  float* part;
  // Segment mode only (the upper layers of a deeper network): the fp32
  // activation feeding layer 0, h_{l0} of the full network, in place of x.
  const float* h0;
  // The widths d[0] .. d[L] of the layers this launch runs (as for FwdParams,
  // read only by the runtime-width kernels).
  int dims[kMaxLayersHost + 1];
};

}  // namespace mlpmk

namespace mlpmk {

// Launch parameters of the two-pass backward (bwd_tp.hip).  Tensors are
// 16-bit (fp16 / bf16 payloads) or fp32 as the launch's element mode says;
// pointers are untyped here.
struct TpParams {
  const void* x;
  const void* w[kMaxLayersHost];
  const float* stash[kMaxLayersHost];  // stash[l] = h_{l+1}, fp32 [M, d[l+1]]
  const void* dout;                    // dL/dout; row r at dout + r * dout_stride
  int64_t dout_stride;                 // elements; 0 broadcasts row 0, -1 element 0
  void* dx;                            // nullable
  float* dw[kMaxLayersHost];           // fp32 [d[l], d[l+1]], accumulated into (fp32 atomics)
  void* dz[kMaxLayersHost];            // dz_l, l = 0 .. L-2: [M, d[l+1]] in the workspace
  int64_t M;
  int64_t chunk_rows;                  // rows per weight-gradient chunk
  // Nonzero: the data-gradient pass clears dw before the weight-gradient
  // pass adds to it (MLPMK_BWD_WRITE_DW).
  int zero_dw;
  int dims[kMaxLayersHost + 1];
};

}  // namespace mlpmk

