// Weight-norm kernels (one launch per direction for ALL layers) and the
// byte-counter calibration copy.
//
// Replaces `_wn_fwd_kernel` and `_wn_bwd_from_dw_T_kernel` of the reference's
// training path (/root/reference/mlp_fused.md:466-486; the code itself is not
// in the snapshot).  Parameters are contiguous blocks v_all / g_all, layer
// after layer (mlp_fused.md:478-480).  Norms are per output column of the
// [in, out] matrices; adjacent threads take adjacent columns, so every row
// access of a wave is one contiguous segment of the row-major matrix (the
// column-wise read of fp32 dW needs no transposed copy).
#include "device_common.h"
#include "host_common.h"

namespace mlpmk {

struct WnLayout {
  int L;
  int in[kMaxLayers], out[kMaxLayers];
  int64_t v_off[kMaxLayers];    // element offset of layer l in v / w / dw
  int g_off[kMaxLayers];        // element offset of layer l in g / inv_norm
  int blk_off[kMaxLayers + 1];  // first workgroup of layer l
};

// A workgroup owns 32 consecutive output columns of one layer; its 8 row
// groups of 32 threads walk rows rg, rg + 8, ...  Each wave therefore reads
// two rows x 32 columns per instruction (contiguous 64/128-byte segments), and
// the per-column sums are reduced across the row groups in LDS.
constexpr int kWnCols = 32, kWnRowGroups = 8, kWnThreads = kWnCols * kWnRowGroups;

template <class P>
__device__ __forceinline__ float ldp(const P* p, int64_t i) {
  return (float)p[i];
}

__device__ __forceinline__ int wn_layer_of(const WnLayout& lay, int blk) {
  int l = 0;
#pragma unroll
  for (int i = 1; i < kMaxLayers; ++i)
    if (i < lay.L && blk >= lay.blk_off[i]) l = i;
  return l;
}

// Sum over the row groups of a per-thread column partial; every thread of the
// column gets the total.
__device__ __forceinline__ float wn_colsum(float part, float (&red)[kWnRowGroups][kWnCols], int c, int rg) {
  red[rg][c] = part;
  __syncthreads();
  float t = 0.0f;
#pragma unroll
  for (int i = 0; i < kWnRowGroups; ++i) t += red[i][c];
  return t;
}

// Rows per thread held in registers: every load of a column chunk is issued
// before the first use, so a launch costs about two memory round trips (read
// v, write w) instead of one per row; widths above kWnRowGroups * kWnRegRows
// loop over chunks.
constexpr int kWnRegRows = 16;

// P: parameter type (float, fp16 or bf16); O: element type of W (fp16, bf16 or fp32).
template <class P, class O>
__global__ __launch_bounds__(kWnThreads) void wn_fwd_kernel(WnLayout lay, const P* __restrict__ v,
                                                            const P* __restrict__ g, O* __restrict__ w,
                                                            float* __restrict__ inv_norm) {
  __shared__ float red[kWnRowGroups][kWnCols];
  const int l = wn_layer_of(lay, blockIdx.x);
  const int c = threadIdx.x % kWnCols, rg = threadIdx.x / kWnCols;
  const int j = (blockIdx.x - lay.blk_off[l]) * kWnCols + c;
  const int K = lay.in[l], N = lay.out[l];
  const bool col = j < N;  // out widths are multiples of 16: a block may be half used
  const int64_t base = lay.v_off[l] + j;
  float ss = 0.0f;
  float t[kWnRegRows];
  if (col) {
    for (int k0 = 0; k0 < K; k0 += kWnRowGroups * kWnRegRows) {
#pragma unroll
      for (int i = 0; i < kWnRegRows; ++i) {
        const int k = k0 + rg + i * kWnRowGroups;
        t[i] = k < K ? ldp(v, base + (int64_t)k * N) : 0.0f;
      }
#pragma unroll
      for (int i = 0; i < kWnRegRows; ++i) ss = fmaf(t[i], t[i], ss);
    }
  }
  const float inv = 1.0f / sqrtf(wn_colsum(ss, red, c, rg));
  if (!col) return;  // after the only barrier
  const float scale = ldp(g + lay.g_off[l], j) * inv;
  if (K <= kWnRowGroups * kWnRegRows) {  // the column chunk is still in registers
#pragma unroll
    for (int i = 0; i < kWnRegRows; ++i) {
      const int k = rg + i * kWnRowGroups;
      if (k < K) w[base + (int64_t)k * N] = (O)(t[i] * scale);
    }
  } else {
    for (int k = rg; k < K; k += kWnRowGroups) {
      const int64_t e = base + (int64_t)k * N;
      w[e] = (O)(ldp(v, e) * scale);
    }
  }
  if (rg == 0) inv_norm[lay.g_off[l] + j] = inv;
}

template <class P>
__global__ __launch_bounds__(kWnThreads) void wn_bwd_kernel(WnLayout lay, const float* __restrict__ dw,
                                                            const P* __restrict__ v, const P* __restrict__ g,
                                                            const float* __restrict__ inv_norm,
                                                            P* __restrict__ dv, P* __restrict__ dg) {
  __shared__ float red[kWnRowGroups][kWnCols];
  const int l = wn_layer_of(lay, blockIdx.x);
  const int c = threadIdx.x % kWnCols, rg = threadIdx.x / kWnCols;
  const int j = (blockIdx.x - lay.blk_off[l]) * kWnCols + c;
  const int K = lay.in[l], N = lay.out[l];
  const bool col = j < N;
  const int64_t base = lay.v_off[l] + j;
  float dot = 0.0f;  // <dW_j, v_j>
  float tw[kWnRegRows], tv[kWnRegRows];
  if (col) {
    for (int k0 = 0; k0 < K; k0 += kWnRowGroups * kWnRegRows) {
#pragma unroll
      for (int i = 0; i < kWnRegRows; ++i) {
        const int k = k0 + rg + i * kWnRowGroups;
        const int64_t e = base + (int64_t)k * N;
        tw[i] = k < K ? dw[e] : 0.0f;
        tv[i] = k < K ? ldp(v, e) : 0.0f;
      }
#pragma unroll
      for (int i = 0; i < kWnRegRows; ++i) dot = fmaf(tw[i], tv[i], dot);
    }
  }
  dot = wn_colsum(dot, red, c, rg);
  if (!col) return;  // after the only barrier
  const float inv = inv_norm[lay.g_off[l] + j];
  const float dgj = dot * inv;  // <dW_j, u_j>, u = v * inv
  const float gs = ldp(g + lay.g_off[l], j) * inv;
  const float vs = dgj * inv;
  if (K <= kWnRowGroups * kWnRegRows) {  // the column chunk is still in registers
#pragma unroll
    for (int i = 0; i < kWnRegRows; ++i) {
      const int k = rg + i * kWnRowGroups;
      if (k < K) dv[base + (int64_t)k * N] = (P)(gs * (tw[i] - vs * tv[i]));
    }
  } else {
    for (int k = rg; k < K; k += kWnRowGroups) {
      const int64_t e = base + (int64_t)k * N;
      dv[e] = (P)(gs * (dw[e] - vs * ldp(v, e)));
    }
  }
  if (rg == 0) dg[lay.g_off[l] + j] = (P)dgj;
}

static int wn_layout(int L, const int* dims, WnLayout* lay) {
  if (L > kMaxLayers) return fail(MLPMK_ERR_UNSUPPORTED_SHAPE, "num_layers=%d too large", L);
  lay->L = L;
  int64_t vo = 0;
  int go = 0, bo = 0;
  for (int l = 0; l < L; ++l) {
    lay->in[l] = dims[l];
    lay->out[l] = dims[l + 1];
    lay->v_off[l] = vo;
    lay->g_off[l] = go;
    lay->blk_off[l] = bo;
    vo += (int64_t)dims[l] * dims[l + 1];
    go += dims[l + 1];
    bo += (dims[l + 1] + kWnCols - 1) / kWnCols;
  }
  lay->blk_off[L] = bo;
  return MLPMK_OK;
}

template <class P, class O>
static void launch_wn_fwd(const WnLayout& lay, const void* v, const void* g, void* w_out, float* inv_norm,
                          hipStream_t st) {
  hipLaunchKernelGGL((wn_fwd_kernel<P, O>), dim3(lay.blk_off[lay.L]), dim3(kWnThreads), 0, st, lay,
                     (const P*)v, (const P*)g, (O*)w_out, inv_norm);
}

template <class P>
static void launch_wn_fwd_p(const WnLayout& lay, int w_dtype, const void* v, const void* g, void* w_out,
                            float* inv_norm, hipStream_t st) {
  if (w_dtype == MLPMK_DTYPE_BF16)
    launch_wn_fwd<P, __bf16>(lay, v, g, w_out, inv_norm, st);
  else if (w_dtype == MLPMK_DTYPE_F32)
    launch_wn_fwd<P, float>(lay, v, g, w_out, inv_norm, st);
  else
    launch_wn_fwd<P, f16>(lay, v, g, w_out, inv_norm, st);
}

int wn_fwd_dispatch(int L, const int* dims, int dtype, int w_dtype, const void* v, const void* g, void* w_out,
                    float* inv_norm, hipStream_t st) {
  WnLayout lay;
  int rc = wn_layout(L, dims, &lay);
  if (rc) return rc;
  int cus = 0;
  if ((rc = current_device_cus(&cus))) return rc;
  (void)hipGetLastError();
  if (dtype == MLPMK_DTYPE_F32)
    launch_wn_fwd_p<float>(lay, w_dtype, v, g, w_out, inv_norm, st);
  else if (dtype == MLPMK_DTYPE_BF16)
    launch_wn_fwd_p<__bf16>(lay, w_dtype, v, g, w_out, inv_norm, st);
  else
    launch_wn_fwd_p<f16>(lay, w_dtype, v, g, w_out, inv_norm, st);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? MLPMK_OK : hip_fail(e, "wn_fwd kernel launch");
}

int wn_bwd_dispatch(int L, const int* dims, int dtype, const float* dw, const void* v, const void* g,
                    const float* inv_norm, void* dv, void* dg, hipStream_t st) {
  WnLayout lay;
  int rc = wn_layout(L, dims, &lay);
  if (rc) return rc;
  int cus = 0;
  if ((rc = current_device_cus(&cus))) return rc;
  (void)hipGetLastError();
  if (dtype == MLPMK_DTYPE_F32)
    hipLaunchKernelGGL(wn_bwd_kernel<float>, dim3(lay.blk_off[L]), dim3(kWnThreads), 0, st, lay, dw,
                       (const float*)v, (const float*)g, inv_norm, (float*)dv, (float*)dg);
  else if (dtype == MLPMK_DTYPE_BF16)
    hipLaunchKernelGGL(wn_bwd_kernel<__bf16>, dim3(lay.blk_off[L]), dim3(kWnThreads), 0, st, lay, dw,
                       (const __bf16*)v, (const __bf16*)g, inv_norm, (__bf16*)dv, (__bf16*)dg);
  else
    hipLaunchKernelGGL(wn_bwd_kernel<f16>, dim3(lay.blk_off[L]), dim3(kWnThreads), 0, st, lay, dw,
                       (const f16*)v, (const f16*)g, inv_norm, (f16*)dv, (f16*)dg);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? MLPMK_OK : hip_fail(e, "wn_bwd kernel launch");
}

// ---------------------------------------------------------------------------
// Calibration copy: 16-byte loads/stores, grid-stride, the access width and
// cache policy of the forward megakernel's x and out traffic (default loads,
// non-temporal stores).  Used to scale FETCH_SIZE / WRITE_SIZE counters and as
// the achievable-HBM reference of the benchmark.  Grid: 3 workgroups of 256
// threads per CU, the fastest of the grid-stride and per-workgroup-chunk
// copies measured on MI355X at 512 MiB each way (6.13 TB/s; 8 per CU: 5.15,
// 1 per CU with 1024 threads: 6.02, 8 KiB chunks per workgroup: 6.08).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void copy_kernel(const f32x4* __restrict__ src, f32x4* __restrict__ dst,
                                                   int64_t n16) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (int64_t)gridDim.x * 256)
    __builtin_nontemporal_store(src[i], &dst[i]);
}

int copy_dispatch(const void* src, void* dst, int64_t bytes, hipStream_t st) {
  int cus = 0;
  int rc = current_device_cus(&cus);
  if (rc) return rc;
  const int64_t n16 = bytes / 16;
  int64_t grid = (n16 + 255) / 256;
  if (grid > (int64_t)cus * 3) grid = (int64_t)cus * 3;
  (void)hipGetLastError();
  hipLaunchKernelGGL(copy_kernel, dim3((unsigned)grid), dim3(256), 0, st, (const f32x4*)src, (f32x4*)dst, n16);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? MLPMK_OK : hip_fail(e, "copy kernel launch");
}

}  // namespace mlpmk
