// Elementwise kernel of the reference's large-M backward fallback
// (/root/reference/mlp_fused.md:114-146): its fused `sigmoid_h_mul` Triton
// kernel computes dz = (1 - exp(-h)) * dh in one launch between the
// library GEMMs of the data and weight gradients.  Here it is one grid-stride
// HIP kernel over 8 elements per thread and step: h is the fp32 activation
// stash, dh the data-gradient GEMM's output (fp16, bf16 or fp32), and dz is
// written in fp32 (for the fp32 weight-gradient GEMM) and optionally also in
// the 16-bit type of the next data-gradient GEMM -- one read of h and dh for
// both.  sigma = 1 - exp(-h) is evaluated as -expm1(-h) (sig_from_h).
#include "device_common.h"
#include "host_common.h"

namespace mlpmk {

template <int DT>
struct Elem;
template <>
struct Elem<MLPMK_DTYPE_F32> {
  typedef float T;
};
template <>
struct Elem<MLPMK_DTYPE_F16> {
  typedef _Float16 T;
};
template <>
struct Elem<MLPMK_DTYPE_BF16> {
  typedef __bf16 T;
};

template <int DH, int DZ>
__global__ __launch_bounds__(256) void sigmoid_h_mul_kernel(const float* __restrict__ h,
                                                            const typename Elem<DH>::T* __restrict__ dh,
                                                            float* __restrict__ dz32,
                                                            typename Elem<DZ>::T* __restrict__ dz16, int64_t n) {
  typedef typename Elem<DH>::T TH;
  typedef typename Elem<DZ>::T TZ;
  const int64_t n8 = n / 8;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += stride) {
    typedef float f32x8 __attribute__((ext_vector_type(8)));
    typedef TH th8 __attribute__((ext_vector_type(8)));
    typedef TZ tz8 __attribute__((ext_vector_type(8)));
    const f32x8 hv = reinterpret_cast<const f32x8*>(h)[i];
    const th8 dv = reinterpret_cast<const th8*>(dh)[i];
    f32x8 z;
#pragma unroll
    for (int j = 0; j < 8; ++j) z[j] = (float)dv[j] * sig_from_h(hv[j]);
    reinterpret_cast<f32x8*>(dz32)[i] = z;
    if (dz16) reinterpret_cast<tz8*>(dz16)[i] = __builtin_convertvector(z, tz8);
  }
  // tail (n % 8 elements), one thread each
  const int64_t t = n8 * 8 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t < n && t < n8 * 8 + 8) {
    const float z = (float)dh[t] * sig_from_h(h[t]);
    dz32[t] = z;
    if (dz16) dz16[t] = (TZ)z;
  }
}

template <int DH, int DZ>
static int launch_shm(const float* h, const void* dh, float* dz32, void* dz16, int64_t n, hipStream_t st) {
  int cus = 0;
  int rc = current_device_cus(&cus);
  if (rc != MLPMK_OK) return rc;
  const int64_t want = (n / 8 + 255) / 256;
  const int64_t cap = (int64_t)cus * 8;
  const unsigned grid = (unsigned)(want < 1 ? 1 : (want < cap ? want : cap));
  (void)hipGetLastError();
  hipLaunchKernelGGL((sigmoid_h_mul_kernel<DH, DZ>), dim3(grid), dim3(256), 0, st, h,
                     static_cast<const typename Elem<DH>::T*>(dh), dz32, static_cast<typename Elem<DZ>::T*>(dz16), n);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? MLPMK_OK : hip_fail(e, "sigmoid_h_mul kernel launch");
}

template <int DH>
static int shm_dz(const float* h, const void* dh, float* dz32, void* dz16, int dz16_dtype, int64_t n,
                  hipStream_t st) {
  if (dz16_dtype == MLPMK_DTYPE_BF16) return launch_shm<DH, MLPMK_DTYPE_BF16>(h, dh, dz32, dz16, n, st);
  return launch_shm<DH, MLPMK_DTYPE_F16>(h, dh, dz32, dz16, n, st);
}

int sigmoid_h_mul_dispatch(const float* h, const void* dh, int dh_dtype, float* dz32, void* dz16, int dz16_dtype,
                           int64_t n, hipStream_t st) {
  switch (dh_dtype) {
    case MLPMK_DTYPE_F32: return shm_dz<MLPMK_DTYPE_F32>(h, dh, dz32, dz16, dz16_dtype, n, st);
    case MLPMK_DTYPE_F16: return shm_dz<MLPMK_DTYPE_F16>(h, dh, dz32, dz16, dz16_dtype, n, st);
    default: return shm_dz<MLPMK_DTYPE_BF16>(h, dh, dz32, dz16, dz16_dtype, n, st);
  }
}

// softplus(z) = log(1 + e^z) with the reference's threshold (torch's
// softplus, beta 1, threshold 20: z itself above 20), in fp32 to a few ulp:
// below the threshold softplus(z) = max(z, 0) + log1p(e), e = exp(-|z|).
//  * e = 2^(-|z| log2 e) with the product carried in two parts (p + q, q the
//    rounding error of p plus |z| times log2 e's own fp32 rounding error), so
//    e keeps fp32 accuracy for large |z| as well: e = 2^p (1 + q ln 2).
//  * log1p(e) = log(1 + e) * e / ((1 + e) - 1): the quotient undoes the
//    rounding of 1 + e (the subtraction is exact); e itself where 1 + e
//    rounds to 1.
// -inf gives 0 (|z| clamped to 200, where e^-|z| is 0 in fp32), +inf gives
// +inf, NaN stays NaN.
constexpr float kLog2eLo = 1.925963033500011e-08f;  // log2(e) - kLog2e

__device__ __forceinline__ float softplus_exact(float z) {
  if (z > 20.0f) return z;
  float a = -__builtin_fabsf(z);
  a = a < -200.0f ? -200.0f : a;
  const float p = a * kLog2e;
  const float q = __builtin_fmaf(a, kLog2e, -p) + a * kLog2eLo;
  const float e = __builtin_amdgcn_exp2f(p) * __builtin_fmaf(q, kLn2, 1.0f);
  const float u = 1.0f + e, d = u - 1.0f;
  const float l = d == 0.0f ? e : kLn2 * __builtin_amdgcn_logf(u) * (e / d);
  return __builtin_fmaxf(z, 0.0f) + l;
}

// h[i] = softplus(z[i]), i < n, four elements per thread and step (h may be z).
__global__ __launch_bounds__(256) void softplus_f32_kernel(const float* z, float* h, int64_t n) {
  const int64_t n4 = n / 4;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
    f32x4 v = reinterpret_cast<const f32x4*>(z)[i];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = softplus_exact(v[j]);
    reinterpret_cast<f32x4*>(h)[i] = v;
  }
  const int64_t t = n4 * 4 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // tail, one thread each
  if (t < n && t < n4 * 4 + 4) h[t] = softplus_exact(z[t]);
}

int softplus_f32_dispatch(const float* z, float* h, int64_t n, hipStream_t st) {
  int cus = 0;
  const int rc = current_device_cus(&cus);
  if (rc != MLPMK_OK) return rc;
  const int64_t want = (n / 4 + 255) / 256;
  const int64_t cap = (int64_t)cus * 8;
  const unsigned grid = (unsigned)(want < 1 ? 1 : (want < cap ? want : cap));
  (void)hipGetLastError();
  hipLaunchKernelGGL(softplus_f32_kernel, dim3(grid), dim3(256), 0, st, z, h, n);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MLPMK_OK : hip_fail(e, "softplus kernel launch");
}

}  // namespace mlpmk
