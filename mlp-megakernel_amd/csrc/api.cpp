// C ABI of libmlpmk.so: argument validation, error reporting and device
// queries.  Every check here runs on the host before any launch; nothing in
// this file touches device memory.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>

#include "host_common.h"
#include "params.h"

namespace mlpmk {

bool fwd_supported_dims(int L, const int* dims);
bool fwd_supported_dtype(int L, const int* dims, int dtype);
int fwd_dispatch(int L, const int* dims, const FwdParams& p, bool stash, int dtype, hipStream_t st, LaunchInfo* info);
bool bwd_supported_dims(int L, const int* dims);
bool bwd_supported_dtype(int L, const int* dims, int dtype);
bool bwd_recompute_supported(int L, const int* dims);
int bwd_dispatch(int L, const int* dims, const BwdParams& p, int dtype, hipStream_t st);
int bwd_clear_dw(int L, const int* dims, float* const* dw, hipStream_t st);
int bwd_workspace_bytes(int L, const int* dims, int64_t M, bool dx, int dtype, int64_t* bytes);
int scratch_workspace(void** ptr, int64_t* bytes);
int wn_fwd_dispatch(int L, const int* dims, int dtype, int w_dtype, const void* v, const void* g, void* w_out,
                    float* inv_norm, hipStream_t st);
int wn_bwd_dispatch(int L, const int* dims, int dtype, const float* dw, const void* v, const void* g,
                    const float* inv_norm, void* dv, void* dg, hipStream_t st);
int copy_dispatch(const void* src, void* dst, int64_t bytes, hipStream_t st);
int softplus_f32_dispatch(const float* z, float* h, int64_t n, hipStream_t st);
int sigmoid_h_mul_dispatch(const float* h, const void* dh, int dh_dtype, float* dz32, void* dz16, int dz16_dtype,
                           int64_t n, hipStream_t st);

static thread_local char g_last_error[512];

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

int hip_fail(hipError_t e, const char* what) {
  const int st = (e == hipErrorNoDevice || e == hipErrorInvalidDevice) ? MLPMK_ERR_NO_DEVICE : MLPMK_ERR_HIP;
  return fail(st, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

namespace {
constexpr int kMaxDev = 64;
std::atomic<int> g_cus[kMaxDev];  // 0 = unknown, -1 = not gfx950, else CU count
}  // namespace

int current_device_cus(int* cus) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  int cached = (dev >= 0 && dev < kMaxDev) ? g_cus[dev].load(std::memory_order_relaxed) : 0;
  if (cached == 0) {
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
    cached = (strncmp(prop.gcnArchName, "gfx950", 6) == 0) ? prop.multiProcessorCount : -1;
    if (cached == 0) cached = -1;
    if (dev >= 0 && dev < kMaxDev) g_cus[dev].store(cached, std::memory_order_relaxed);
    if (cached < 0)
      return fail(MLPMK_ERR_NO_DEVICE, "device %d is %s; libmlpmk is built for gfx950 only", dev,
                  prop.gcnArchName);
  }
  if (cached < 0) return fail(MLPMK_ERR_NO_DEVICE, "device %d is not a gfx950 part", dev);
  *cus = cached;
  return MLPMK_OK;
}

int kernel_occupancy(const void* kernel, int threads, int* wgs_per_cu) {
  int occ = 0;
  hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, threads, 0);
  if (e != hipSuccess) return hip_fail(e, "hipOccupancyMaxActiveBlocksPerMultiprocessor");
  *wgs_per_cu = occ > 0 ? occ : 1;
  return MLPMK_OK;
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Element format of the backward's x, w, dout and dx.
static int check_bwd_dtype(int dtype) {
  if (dtype == MLPMK_DTYPE_F16 || dtype == MLPMK_DTYPE_BF16 || dtype == MLPMK_DTYPE_F32) return MLPMK_OK;
  return fail(MLPMK_ERR_INVALID_ARG, "dtype=%d (0 = fp32, 1 = fp16, 2 = bf16)", dtype);
}

// Element format of the forward's x, W and out: fp32 tensors are taken too
// (bf16 hi/lo split MFMA operands, fp32 rows).
static int check_fwd_dtype(int dtype) {
  if (dtype == MLPMK_DTYPE_F16 || dtype == MLPMK_DTYPE_BF16 || dtype == MLPMK_DTYPE_F32) return MLPMK_OK;
  return fail(MLPMK_ERR_INVALID_ARG, "dtype=%d (0 = fp32, 1 = fp16, 2 = bf16)", dtype);
}

static int check_dims(int L, const int* dims) {
  if (!dims) return fail(MLPMK_ERR_INVALID_ARG, "dims is NULL");
  if (L < 2 || L > kMaxLayersHost)
    return fail(MLPMK_ERR_UNSUPPORTED_SHAPE, "num_layers=%d (supported: 2..%d)", L, kMaxLayersHost);
  for (int i = 0; i <= L; ++i)
    if (dims[i] <= 0) return fail(MLPMK_ERR_INVALID_ARG, "dims[%d]=%d must be positive", i, dims[i]);
  return MLPMK_OK;
}

static int check_ptr(const void* p, const char* name) {
  if (!p) return fail(MLPMK_ERR_INVALID_ARG, "%s is NULL", name);
  if (!aligned16(p)) return fail(MLPMK_ERR_MISALIGNED, "%s=%p is not 16-byte aligned", name, p);
  return MLPMK_OK;
}

}  // namespace mlpmk

using namespace mlpmk;

extern "C" {

int mlpmk_version(void) { return 204; }  // 2.04: mlpmk_softplus_f32, mlpmk_fwd_supported_dtype (2.03: MLPMK_BWD_WRITE_DW)

const char* mlpmk_status_string(int status) {
  switch (status) {
    case MLPMK_OK: return "ok";
    case MLPMK_ERR_INVALID_ARG: return "invalid argument";
    case MLPMK_ERR_UNSUPPORTED_SHAPE: return "unsupported shape";
    case MLPMK_ERR_MISALIGNED: return "pointer not 16-byte aligned";
    case MLPMK_ERR_HIP: return "HIP runtime error";
    case MLPMK_ERR_NO_DEVICE: return "no usable gfx950 device";
    default: return "unknown status";
  }
}

const char* mlpmk_last_error(void) { return g_last_error; }

int mlpmk_fwd_supported(int num_layers, const int* dims) {
  if (!dims || num_layers < 2 || num_layers > kMaxLayersHost) return 0;
  return fwd_supported_dims(num_layers, dims) ? 1 : 0;
}

int mlpmk_fwd_supported_dtype(int num_layers, const int* dims, int dtype) {
  if (!dims || num_layers < 2 || num_layers > kMaxLayersHost) return 0;
  if (dtype != MLPMK_DTYPE_F16 && dtype != MLPMK_DTYPE_BF16 && dtype != MLPMK_DTYPE_F32) return 0;
  return fwd_supported_dtype(num_layers, dims, dtype) ? 1 : 0;
}

int mlpmk_bwd_supported(int num_layers, const int* dims) {
  if (!dims || num_layers < 2 || num_layers > kMaxLayersHost) return 0;
  return bwd_supported_dims(num_layers, dims) ? 1 : 0;
}

int mlpmk_bwd_supported_dtype(int num_layers, const int* dims, int dtype) {
  if (!dims || num_layers < 2 || num_layers > kMaxLayersHost) return 0;
  if (dtype != MLPMK_DTYPE_F16 && dtype != MLPMK_DTYPE_BF16 && dtype != MLPMK_DTYPE_F32) return 0;
  return bwd_supported_dtype(num_layers, dims, dtype) ? 1 : 0;
}

int mlpmk_bwd_recompute_supported(int num_layers, const int* dims) {
  if (!dims || num_layers < 2 || num_layers > kMaxLayersHost) return 0;
  return bwd_recompute_supported(num_layers, dims) ? 1 : 0;
}

int mlpmk_fwd(int num_layers, const int* dims, int dtype, const void* x, const void* const* w, void* out,
              float* const* stash, int64_t M, void* stream) {
  g_last_error[0] = 0;
  int rc = check_dims(num_layers, dims);
  if (rc) return rc;
  if ((rc = check_fwd_dtype(dtype))) return rc;
  if (M < 0) return fail(MLPMK_ERR_INVALID_ARG, "M=%lld is negative", (long long)M);
  if (!w) return fail(MLPMK_ERR_INVALID_ARG, "w is NULL");
  if (!fwd_supported_dims(num_layers, dims))
    return fail(MLPMK_ERR_UNSUPPORTED_SHAPE, "no forward kernel for these widths");
  FwdParams p = {};
  for (int l = 0; l < num_layers; ++l) {
    char name[16];
    snprintf(name, sizeof(name), "w[%d]", l);
    if ((rc = check_ptr(w[l], name))) return rc;
    p.w[l] = static_cast<const _Float16*>(w[l]);
  }
  if (M == 0) return MLPMK_OK;
  if ((rc = check_ptr(x, "x"))) return rc;
  if ((rc = check_ptr(out, "out"))) return rc;
  if (stash) {
    for (int l = 0; l < num_layers - 1; ++l) {
      if (!stash[l]) continue;  // not written
      char name[16];
      snprintf(name, sizeof(name), "stash[%d]", l);
      if ((rc = check_ptr(stash[l], name))) return rc;
      p.stash[l] = stash[l];
    }
  }
  p.x = static_cast<const _Float16*>(x);
  p.out = static_cast<_Float16*>(out);
  p.M = M;
  for (int l = 0; l <= num_layers; ++l) p.dims[l] = dims[l];
  return fwd_dispatch(num_layers, dims, p, stash != nullptr, dtype, static_cast<hipStream_t>(stream), nullptr);
}

int mlpmk_fwd_launch_info(int num_layers, const int* dims, int dtype, int64_t M, int stash, int* info) {
  g_last_error[0] = 0;
  int rc = check_dims(num_layers, dims);
  if (rc) return rc;
  if ((rc = check_fwd_dtype(dtype))) return rc;
  if (M < 0) return fail(MLPMK_ERR_INVALID_ARG, "M=%lld is negative", (long long)M);
  if (!info) return fail(MLPMK_ERR_INVALID_ARG, "info is NULL");
  if (!fwd_supported_dims(num_layers, dims))
    return fail(MLPMK_ERR_UNSUPPORTED_SHAPE, "no forward kernel for these widths");
  if (M == 0) {  // mlpmk_fwd launches nothing
    const int none[5] = {MLPMK_KERNEL_NONE, 0, 0, 0, 0};
    memcpy(info, none, sizeof(none));
    return MLPMK_OK;
  }
  FwdParams p = {};
  p.M = M;
  for (int l = 0; l <= num_layers; ++l) p.dims[l] = dims[l];
  LaunchInfo li = {};
  rc = fwd_dispatch(num_layers, dims, p, stash != 0, dtype, nullptr, &li);
  if (rc) return rc;
  const int out[5] = {li.kernel, li.rows_per_block, li.waves, li.grid, li.wgs_per_cu};
  memcpy(info, out, sizeof(out));
  return MLPMK_OK;
}

// use_scratch: the workspace is the library's own scratch array
// (mlpmk_bwd_noalloc), looked up after the arguments are validated.
static int bwd_common(int num_layers, const int* dims, int dtype, const void* x, const void* const* w,
                      const float* const* stash, const void* dout, int64_t dout_row_stride, void* dx,
                      float* const* dw, void* workspace, int64_t workspace_bytes, int64_t M, void* stream,
                      bool use_scratch = false) {
  int rc = check_dims(num_layers, dims);
  if (rc) return rc;
  const bool write_dw = (dtype & MLPMK_BWD_WRITE_DW) != 0;
  dtype &= ~MLPMK_BWD_WRITE_DW;
  if ((rc = check_bwd_dtype(dtype))) return rc;
  if (M < 0) return fail(MLPMK_ERR_INVALID_ARG, "M=%lld is negative", (long long)M);
  const bool dout_scalar = dout_row_stride == MLPMK_DOUT_SCALAR;
  if (dout_row_stride < 0 && !dout_scalar)
    return fail(MLPMK_ERR_INVALID_ARG, "dout_row_stride=%lld is negative (MLPMK_DOUT_SCALAR is %d)",
                (long long)dout_row_stride, (int)MLPMK_DOUT_SCALAR);
  if (!w || !dw) return fail(MLPMK_ERR_INVALID_ARG, "w or dw is NULL");
  if (num_layers > 1 && !stash) return fail(MLPMK_ERR_INVALID_ARG, "stash is NULL");
  if (!bwd_supported_dtype(num_layers, dims, dtype))
    return fail(MLPMK_ERR_UNSUPPORTED_SHAPE, "no backward kernel for these widths%s",
                dtype == MLPMK_DTYPE_F32 ? " with fp32 tensors (widths up to 128, output width a multiple of 8)" : "");
  const int out_w = dims[num_layers];
  if (dout_row_stride > 0 && dout_row_stride < out_w)
    return fail(MLPMK_ERR_INVALID_ARG, "dout_row_stride=%lld is below the output width %d",
                (long long)dout_row_stride, out_w);
  if (!dout_scalar && dout_row_stride % 8 != 0)
    return fail(MLPMK_ERR_MISALIGNED, "dout_row_stride=%lld is not a multiple of 8 elements",
                (long long)dout_row_stride);
  BwdParams p = {};
  p.write_dw = write_dw;
  for (int l = 0; l < num_layers; ++l) {
    char name[16];
    snprintf(name, sizeof(name), "w[%d]", l);
    if ((rc = check_ptr(w[l], name))) return rc;
    snprintf(name, sizeof(name), "dw[%d]", l);
    if ((rc = check_ptr(dw[l], name))) return rc;
    p.w[l] = static_cast<const _Float16*>(w[l]);
    p.dw[l] = dw[l];
  }
  // No rows: nothing to accumulate, or (written) the gradient is zero.
  if (M == 0) return write_dw ? bwd_clear_dw(num_layers, dims, dw, static_cast<hipStream_t>(stream)) : MLPMK_OK;
  if ((rc = check_ptr(x, "x"))) return rc;
  if (dout_scalar) {
    if (!dout) return fail(MLPMK_ERR_INVALID_ARG, "dout is NULL");
    const uintptr_t al = dtype == MLPMK_DTYPE_F32 ? 3u : 1u;
    if (reinterpret_cast<uintptr_t>(dout) & al)
      return fail(MLPMK_ERR_MISALIGNED, "dout=%p is not %d-byte aligned", dout, (int)al + 1);
  } else if ((rc = check_ptr(dout, "dout"))) {
    return rc;
  }
  for (int l = 0; l < num_layers - 1; ++l) {
    char name[16];
    snprintf(name, sizeof(name), "stash[%d]", l);
    if (!stash[l] && l == num_layers - 2 && num_layers > 2 && bwd_recompute_supported(num_layers, dims))
      continue;  // the kernel recomputes h_{L-1}
    if ((rc = check_ptr(stash[l], name))) return rc;
    p.stash[l] = stash[l];
  }
  if (dx && (rc = check_ptr(dx, "dx"))) return rc;
  p.x = static_cast<const _Float16*>(x);
  p.dout = static_cast<const _Float16*>(dout);
  p.dout_stride = dout_row_stride;
  p.dx = static_cast<_Float16*>(dx);
  p.M = M;
  for (int l = 0; l <= num_layers; ++l) p.dims[l] = dims[l];
  if (use_scratch && (rc = scratch_workspace(&workspace, &workspace_bytes))) return rc;
  if (workspace) {
    if ((rc = check_ptr(workspace, "workspace"))) return rc;
    int64_t need = 0;
    if ((rc = bwd_workspace_bytes(num_layers, dims, M, dx != nullptr, dtype, &need))) return rc;
    if (use_scratch && need > workspace_bytes)
      return fail(MLPMK_ERR_UNSUPPORTED_SHAPE,
                  "M=%lld needs %lld bytes of workspace; mlpmk_bwd_noalloc's scratch holds %lld "
                  "(MLPMK_NOALLOC_SCRATCH_BYTES): use mlpmk_bwd_ws with a larger workspace",
                  (long long)M, (long long)need, (long long)workspace_bytes);
    if (workspace_bytes < need)
      return fail(MLPMK_ERR_INVALID_ARG, "workspace_bytes=%lld is below the %lld bytes needed",
                  (long long)workspace_bytes, (long long)need);
    p.part = static_cast<float*>(workspace);
  }
  return bwd_dispatch(num_layers, dims, p, dtype, static_cast<hipStream_t>(stream));
}

int mlpmk_bwd(int num_layers, const int* dims, int dtype, const void* x, const void* const* w,
              const float* const* stash, const void* dout, int64_t dout_row_stride, void* dx,
              float* const* dw, int64_t M, void* stream) {
  g_last_error[0] = 0;
  return bwd_common(num_layers, dims, dtype, x, w, stash, dout, dout_row_stride, dx, dw, nullptr, 0, M, stream);
}

int mlpmk_bwd_ws(int num_layers, const int* dims, int dtype, const void* x, const void* const* w,
                 const float* const* stash, const void* dout, int64_t dout_row_stride, void* dx,
                 float* const* dw, void* workspace, int64_t workspace_bytes, int64_t M, void* stream) {
  g_last_error[0] = 0;
  if (!workspace) return fail(MLPMK_ERR_INVALID_ARG, "workspace is NULL");
  return bwd_common(num_layers, dims, dtype, x, w, stash, dout, dout_row_stride, dx, dw, workspace,
                    workspace_bytes, M, stream);
}

int mlpmk_bwd_noalloc(int num_layers, const int* dims, int dtype, const void* x, const void* const* w,
                      const float* const* stash, const void* dout, int64_t dout_row_stride, void* dx,
                      float* const* dw, int64_t M, void* stream) {
  g_last_error[0] = 0;
  return bwd_common(num_layers, dims, dtype, x, w, stash, dout, dout_row_stride, dx, dw, nullptr, 0, M, stream,
                    true);
}

int mlpmk_bwd_workspace_size(int num_layers, const int* dims, int dtype, int64_t M, int with_dx, int64_t* bytes) {
  g_last_error[0] = 0;
  if (!bytes) return fail(MLPMK_ERR_INVALID_ARG, "bytes is NULL");
  *bytes = 0;
  int rc = check_dims(num_layers, dims);
  if (rc) return rc;
  dtype &= ~MLPMK_BWD_WRITE_DW;  // (the same workspace either way)
  if ((rc = check_bwd_dtype(dtype))) return rc;
  if (M < 0) return fail(MLPMK_ERR_INVALID_ARG, "M=%lld is negative", (long long)M);
  if (!bwd_supported_dtype(num_layers, dims, dtype))
    return fail(MLPMK_ERR_UNSUPPORTED_SHAPE, "no backward kernel for these widths and dtype");
  if (M == 0) return MLPMK_OK;
  return bwd_workspace_bytes(num_layers, dims, M, with_dx != 0, dtype, bytes);
}

static int check_wn(int num_layers, const int* dims, int dtype) {
  int rc = check_dims(num_layers, dims);
  if (rc) return rc;
  if (dtype != MLPMK_DTYPE_F32 && dtype != MLPMK_DTYPE_F16 && dtype != MLPMK_DTYPE_BF16)
    return fail(MLPMK_ERR_INVALID_ARG, "param_dtype=%d (0 = fp32, 1 = fp16, 2 = bf16)", dtype);
  return MLPMK_OK;  // element-wise kernels: any positive widths
}

int mlpmk_wn_fwd(int num_layers, const int* dims, int param_dtype, int w_dtype, const void* v, const void* g,
                 void* w_out, float* inv_norm, void* stream) {
  g_last_error[0] = 0;
  int rc = check_wn(num_layers, dims, param_dtype);
  if (rc) return rc;
  if (w_dtype != MLPMK_DTYPE_F16 && w_dtype != MLPMK_DTYPE_BF16 && w_dtype != MLPMK_DTYPE_F32)
    return fail(MLPMK_ERR_INVALID_ARG, "w_dtype=%d (0 = fp32, 1 = fp16, 2 = bf16)", w_dtype);
  if ((rc = check_ptr(v, "v")) || (rc = check_ptr(g, "g")) || (rc = check_ptr(w_out, "w_out")) ||
      (rc = check_ptr(inv_norm, "inv_norm")))
    return rc;
  return wn_fwd_dispatch(num_layers, dims, param_dtype, w_dtype, v, g, w_out, inv_norm,
                         static_cast<hipStream_t>(stream));
}

int mlpmk_wn_bwd(int num_layers, const int* dims, int param_dtype, const float* dw, const void* v,
                 const void* g, const float* inv_norm, void* dv, void* dg, void* stream) {
  g_last_error[0] = 0;
  int rc = check_wn(num_layers, dims, param_dtype);
  if (rc) return rc;
  if ((rc = check_ptr(dw, "dw")) || (rc = check_ptr(v, "v")) || (rc = check_ptr(g, "g")) ||
      (rc = check_ptr(inv_norm, "inv_norm")) || (rc = check_ptr(dv, "dv")) || (rc = check_ptr(dg, "dg")))
    return rc;
  return wn_bwd_dispatch(num_layers, dims, param_dtype, dw, v, g, inv_norm, dv, dg,
                         static_cast<hipStream_t>(stream));
}

int mlpmk_sigmoid_h_mul(const float* h, const void* dh, int dh_dtype, float* dz32, void* dz16, int dz16_dtype,
                        int64_t n, void* stream) {
  g_last_error[0] = 0;
  if (n < 0) return fail(MLPMK_ERR_INVALID_ARG, "n=%lld is negative", (long long)n);
  if (dh_dtype != MLPMK_DTYPE_F32 && dh_dtype != MLPMK_DTYPE_F16 && dh_dtype != MLPMK_DTYPE_BF16)
    return fail(MLPMK_ERR_INVALID_ARG, "dh_dtype=%d (0 = fp32, 1 = fp16, 2 = bf16)", dh_dtype);
  if (dz16 && dz16_dtype != MLPMK_DTYPE_F16 && dz16_dtype != MLPMK_DTYPE_BF16)
    return fail(MLPMK_ERR_INVALID_ARG, "dz16_dtype=%d (1 = fp16, 2 = bf16)", dz16_dtype);
  if (n == 0) return MLPMK_OK;
  int rc;
  if ((rc = check_ptr(h, "h")) || (rc = check_ptr(dh, "dh")) || (rc = check_ptr(dz32, "dz32"))) return rc;
  if (dz16 && (rc = check_ptr(dz16, "dz16"))) return rc;
  return sigmoid_h_mul_dispatch(h, dh, dh_dtype, dz32, dz16, dz16_dtype, n, static_cast<hipStream_t>(stream));
}

int mlpmk_softplus_f32(const float* z, float* h, int64_t n, void* stream) {
  g_last_error[0] = 0;
  if (n < 0) return fail(MLPMK_ERR_INVALID_ARG, "n=%lld is negative", (long long)n);
  if (n == 0) return MLPMK_OK;
  int rc;
  if ((rc = check_ptr(z, "z")) || (rc = check_ptr(h, "h"))) return rc;
  return softplus_f32_dispatch(z, h, n, static_cast<hipStream_t>(stream));
}

int mlpmk_copy(const void* src, void* dst, int64_t bytes, void* stream) {
  g_last_error[0] = 0;
  if (bytes < 0 || bytes % 16 != 0)
    return fail(MLPMK_ERR_INVALID_ARG, "bytes=%lld must be a non-negative multiple of 16", (long long)bytes);
  if (bytes == 0) return MLPMK_OK;
  int rc;
  if ((rc = check_ptr(src, "src")) || (rc = check_ptr(dst, "dst"))) return rc;
  return copy_dispatch(src, dst, bytes, static_cast<hipStream_t>(stream));
}

}  // extern "C"
