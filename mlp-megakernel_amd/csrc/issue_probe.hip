// Issue-rate probe for gfx950: what one SIMD pays per wave-instruction for
// the instruction kinds the forward megakernel's epilogue is made of, and
// whether two kinds issued by different waves of one SIMD overlap (co-issue).
// The numbers bound what any softplus evaluation can cost per value.
//
// One 16-wave workgroup per CU (96 KiB of LDS keeps a second one out), so each
// SIMD holds four waves.  Each wave reads its SIMD from HW_ID and takes a rank
// among that SIMD's waves; ranks below nA run kind A, the others kind B (or
// idle when B's iteration count is 0).  Every wave runs 16 independent
// dependency chains per loop iteration, so issue, not latency, bounds it.
// Cycles are the shader clock (s_memtime); s_memrealtime (100 MHz) gives the
// clock frequency over the same interval.
//
//   issue_probe [iters]        prints one JSON object
//
// solo: SIMD cycles per wave-instruction with 4 (and 2) waves of one kind.
// pair: two waves of A and two of B per SIMD, iteration counts balanced so
// that each half alone would take about as long; overlap = (serial - t) /
// (serial - parallel), where serial is the sum and parallel the larger of the
// two halves' solo (2-wave) times: 0 = no co-issue, 1 = full overlap.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <utility>
#include <vector>

#define CHECK(x)                                                                               \
  do {                                                                                         \
    hipError_t e_ = (x);                                                                       \
    if (e_ != hipSuccess) {                                                                    \
      std::fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);     \
      std::exit(1);                                                                            \
    }                                                                                          \
  } while (0)

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

enum Kind {
  K_EXP_F32,
  K_LOG_F32,
  K_EXP_F16,
  K_FMA_F32,
  K_ADD_F32,
  K_MAX_F32,
  K_MAXIMUM3_F32,
  K_CVT_PK_F16,
  K_PK_FMA_F16,
  K_PK_MAXIMUM3_F16,
  K_FRACT_F32,
  K_LDEXP_F32,
  K_CVT_I32_F32,
  K_MFMA_32X32X16_F16,
  K_MFMA_16X16X32_F16,
  K_MFMA_32X32X16_F16_AGPR,
  K_COUNT
};
static const char* kKindName[K_COUNT] = {
    "v_exp_f32",        "v_log_f32",       "v_exp_f16",        "v_fma_f32",         "v_add_f32",
    "v_max_f32",        "v_maximum3_f32",  "v_cvt_pk_f16_f32", "v_pk_fma_f16",      "v_pk_maximum3_f16",
    "v_fract_f32",      "v_ldexp_f32",     "v_cvt_i32_f32",    "v_mfma_f32_32x32x16_f16", "v_mfma_f32_16x16x32_f16",
    "v_mfma_f32_32x32x16_f16 (acc in AGPRs)"};

struct Rec {
  unsigned long long cyc, rt;
  int simd, rank, role, pad;
};

// 16 instructions of kind K on 16 independent registers.
template <int K>
__device__ __forceinline__ void valu16(float (&v)[16], const float (&w)[16]) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    float x = v[i];
    if constexpr (K == K_EXP_F32) asm volatile("v_exp_f32 %0, %0" : "+v"(x));
    if constexpr (K == K_LOG_F32) asm volatile("v_log_f32 %0, %0" : "+v"(x));
    if constexpr (K == K_EXP_F16) asm volatile("v_exp_f16 %0, %0" : "+v"(x));
    if constexpr (K == K_FMA_F32) asm volatile("v_fma_f32 %0, %0, %1, 1.0" : "+v"(x) : "v"(w[i]));
    if constexpr (K == K_ADD_F32) asm volatile("v_add_f32 %0, 1.0, %0" : "+v"(x));
    if constexpr (K == K_MAX_F32) asm volatile("v_max_f32 %0, %1, %0" : "+v"(x) : "v"(w[i]));
    if constexpr (K == K_MAXIMUM3_F32) asm volatile("v_maximum3_f32 %0, %0, %1, %1" : "+v"(x) : "v"(w[i]));
    if constexpr (K == K_CVT_PK_F16) asm volatile("v_cvt_pk_f16_f32 %0, %0, %1" : "+v"(x) : "v"(w[i]));
    if constexpr (K == K_PK_FMA_F16) asm volatile("v_pk_fma_f16 %0, %0, %1, %1" : "+v"(x) : "v"(w[i]));
    if constexpr (K == K_PK_MAXIMUM3_F16) asm volatile("v_pk_maximum3_f16 %0, %0, %1, %1" : "+v"(x) : "v"(w[i]));
    if constexpr (K == K_FRACT_F32) asm volatile("v_fract_f32 %0, %0" : "+v"(x));
    if constexpr (K == K_LDEXP_F32) asm volatile("v_ldexp_f32 %0, %0, 3" : "+v"(x));
    if constexpr (K == K_CVT_I32_F32) asm volatile("v_cvt_i32_f32 %0, %0" : "+v"(x));
    v[i] = x;
  }
}

template <int K>
__device__ __forceinline__ float run_kind(int iters, float seed) {
  if constexpr (K == K_MFMA_32X32X16_F16_AGPR) {
    // Accumulators pinned to AGPRs (inline asm "a" operands): the MFMA then
    // writes no VGPR.  Four independent accumulators, no reads in between, so
    // no dependency hazard inside the asm sequence.
    f16x8 a, b;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      a[j] = (_Float16)(seed * (j + 1));
      b[j] = (_Float16)(seed * (j + 2));
    }
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        asm volatile(
            "v_mfma_f32_32x32x16_f16 %0, %4, %5, %0\n\t"
            "v_mfma_f32_32x32x16_f16 %1, %4, %5, %1\n\t"
            "v_mfma_f32_32x32x16_f16 %2, %4, %5, %2\n\t"
            "v_mfma_f32_32x32x16_f16 %3, %4, %5, %3"
            : "+a"(c0), "+a"(c1), "+a"(c2), "+a"(c3)
            : "v"(a), "v"(b));
    }
    asm volatile("s_nop 15\n\ts_nop 15\n\ts_nop 15" ::: "memory");  // results settle before the reads below
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) s += c0[j] + c1[j] + c2[j] + c3[j];
    return s;
  } else if constexpr (K == K_MFMA_32X32X16_F16 || K == K_MFMA_16X16X32_F16) {
    f16x8 a, b;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      a[j] = (_Float16)(seed * (j + 1));
      b[j] = (_Float16)(seed * (j + 2));
    }
    if constexpr (K == K_MFMA_32X32X16_F16) {
      f32x16 c[4] = {};
      for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int q = 0; q < 4; ++q) c[q] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c[q], 0, 0, 0);
      }
      float s = 0.0f;
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int j = 0; j < 16; ++j) s += c[q][j];
      return s;
    } else {
      f32x4 c[8] = {};
      for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
          for (int q = 0; q < 8; ++q) c[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c[q], 0, 0, 0);
      }
      float s = 0.0f;
#pragma unroll
      for (int q = 0; q < 8; ++q)
#pragma unroll
        for (int j = 0; j < 4; ++j) s += c[q][j];
      return s;
    }
  } else {
    float v[16], w[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      v[i] = seed * (float)(threadIdx.x + i) * 1e-3f + 0.5f;
      w[i] = seed * (float)i;
    }
    for (int it = 0; it < iters; ++it) valu16<K>(v, w);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) s += v[i];
    return s;
  }
}

template <int K>
__device__ __forceinline__ void run_if(int k, int iters, float seed, float& sink) {
  if (k == K) sink += run_kind<K>(iters, seed);
}
template <int... Ks>
__device__ __forceinline__ void dispatch(std::integer_sequence<int, Ks...>, int k, int iters, float seed,
                                         float& sink) {
  (run_if<Ks>(k, iters, seed, sink), ...);
}

constexpr int kWaves = 16;

__global__ __launch_bounds__(kWaves * 64) void probe_kernel(int ka, int ita, int kb, int itb, int na, float seed,
                                                            float* out, Rec* rec) {
  extern __shared__ int lds[];  // 96 KiB requested: one workgroup per CU
  if (threadIdx.x < 4) lds[threadIdx.x] = 0;
  __syncthreads();
  const unsigned hw = __builtin_amdgcn_s_getreg((31 << 11) | (0 << 6) | 4);  // HW_ID, all 32 bits
  const int simd = (int)((hw >> 4) & 3);
  int rank = 0;
  if ((threadIdx.x & 63) == 0) rank = __hip_atomic_fetch_add(&lds[simd], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  rank = __builtin_amdgcn_readfirstlane(rank);
  __syncthreads();
  const int role = rank < na ? 0 : 1;
  const int k = role == 0 ? ka : kb, iters = role == 0 ? ita : itb;
  float sink = 0.0f;
  const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  if (iters > 0) dispatch(std::make_integer_sequence<int, K_COUNT>{}, k, iters, seed, sink);
  const unsigned long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  out[blockIdx.x * blockDim.x + threadIdx.x] = sink;
  if ((threadIdx.x & 63) == 0)
    rec[blockIdx.x * kWaves + (threadIdx.x >> 6)] = Rec{t1 - t0, r1 - r0, simd, rank, role, iters > 0 ? 1 : 0};
}

struct Result {
  double simd_cycles;  // mean over SIMDs of the slowest wave's cycles
  double mhz;          // mean shader clock over the busy waves
};
static bool g_layout_ok = true;  // every SIMD of every CU held 4 waves

static int g_cus = 0;
static float* g_out = nullptr;
static Rec* g_rec = nullptr;

static Result run(int ka, int ita, int kb, int itb, int na) {
  const size_t lds = 96 * 1024;
  hipLaunchKernelGGL(probe_kernel, dim3(g_cus), dim3(kWaves * 64), lds, 0, ka, ita, kb, itb, na, 1.0f, g_out, g_rec);
  CHECK(hipGetLastError());
  CHECK(hipDeviceSynchronize());
  std::vector<Rec> h((size_t)g_cus * kWaves);
  CHECK(hipMemcpy(h.data(), g_rec, h.size() * sizeof(Rec), hipMemcpyDeviceToHost));
  double sum = 0.0, mhz = 0.0;
  int nsimd = 0, nbusy = 0;
  for (int b = 0; b < g_cus; ++b) {
    unsigned long long mx[4] = {0, 0, 0, 0};
    int cnt[4] = {0, 0, 0, 0};
    for (int w = 0; w < kWaves; ++w) {
      const Rec& r = h[(size_t)b * kWaves + w];
      ++cnt[r.simd];
      if (r.cyc > mx[r.simd]) mx[r.simd] = r.cyc;
      if (r.pad && r.rt > 0) {
        mhz += 100.0 * (double)r.cyc / (double)r.rt;
        ++nbusy;
      }
    }
    for (int s = 0; s < 4; ++s) {
      if (cnt[s] != kWaves / 4) g_layout_ok = false;
      sum += (double)mx[s];
      ++nsimd;
    }
  }
  return Result{sum / nsimd, nbusy ? mhz / nbusy : 0.0};
}

int main(int argc, char** argv) {
  const int iters = argc > 1 ? std::atoi(argv[1]) : 20000;
  hipDeviceProp_t prop;
  CHECK(hipGetDeviceProperties(&prop, 0));
  g_cus = prop.multiProcessorCount;
  CHECK(hipFuncSetAttribute((const void*)probe_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024));
  CHECK(hipMalloc(&g_out, (size_t)g_cus * kWaves * 64 * sizeof(float)));
  CHECK(hipMalloc(&g_rec, (size_t)g_cus * kWaves * sizeof(Rec)));
  run(K_FMA_F32, iters, K_FMA_F32, iters, 2);  // clock ramp
  std::printf("{\"device\": \"%s\", \"cus\": %d, \"iters\": %d,\n \"solo\": {", prop.gcnArchName, g_cus, iters);
  double c2[K_COUNT], c4[K_COUNT];
  for (int k = 0; k < K_COUNT; ++k) {
    // instructions per wave: 16 per iteration
    const int it = k >= K_MFMA_32X32X16_F16 ? iters / 4 : iters;
    const Result r4 = run(k, it, k, it, 4);
    const Result r2 = run(k, it, k, 0, 2);
    c4[k] = r4.simd_cycles / (4.0 * 16.0 * it);
    c2[k] = r2.simd_cycles / (2.0 * 16.0 * it);
    std::printf("%s\n  \"%s\": {\"cycles_4_waves\": %.2f, \"cycles_2_waves\": %.2f, \"mhz\": %.0f}", k ? "," : "",
                kKindName[k], c4[k], c2[k], r4.mhz);
  }
  std::printf("},\n \"pair\": {");
  const int pairs[][2] = {{K_EXP_F32, K_FMA_F32},          {K_EXP_F32, K_ADD_F32},
                          {K_LOG_F32, K_FMA_F32},          {K_EXP_F32, K_CVT_PK_F16},
                          {K_EXP_F32, K_LOG_F32},          {K_EXP_F32, K_MFMA_32X32X16_F16},
                          {K_FMA_F32, K_MFMA_32X32X16_F16}, {K_CVT_PK_F16, K_MFMA_32X32X16_F16},
                          {K_ADD_F32, K_MFMA_32X32X16_F16}, {K_LOG_F32, K_MFMA_32X32X16_F16},
                          {K_EXP_F32, K_MFMA_16X16X32_F16}, {K_CVT_PK_F16, K_MFMA_16X16X32_F16},
                          {K_EXP_F32, K_MFMA_32X32X16_F16_AGPR}, {K_FMA_F32, K_MFMA_32X32X16_F16_AGPR},
                          {K_CVT_PK_F16, K_MFMA_32X32X16_F16_AGPR}};
  const int np = sizeof(pairs) / sizeof(pairs[0]);
  for (int i = 0; i < np; ++i) {
    const int a = pairs[i][0], b = pairs[i][1];
    const bool ma = a >= K_MFMA_32X32X16_F16;
    const int ita = ma ? iters / 4 : iters;
    // balance: B's two waves alone take as long as A's two waves alone
    int itb = (int)(ita * c2[a] / c2[b] + 0.5);
    if (itb < 1) itb = 1;
    const Result r = run(a, ita, b, itb, 2);
    const double ta = 2.0 * 16.0 * ita * c2[a], tb = 2.0 * 16.0 * itb * c2[b];
    const double serial = ta + tb, par = ta > tb ? ta : tb;
    const double overlap = (serial - r.simd_cycles) / (serial - par);
    std::printf("%s\n  \"%s + %s\": {\"simd_cycles\": %.0f, \"serial\": %.0f, \"parallel\": %.0f, \"overlap\": %.2f}",
                i ? "," : "", kKindName[a], kKindName[b], r.simd_cycles, serial, par, overlap);
  }
  std::printf("},\n \"four_waves_per_simd\": %s}\n", g_layout_ok ? "true" : "false");
  CHECK(hipFree(g_out));
  CHECK(hipFree(g_rec));
  return 0;
}
