// mfma-valu-probe: does a SIMD run one wave's VALU instructions while the matrix core runs
// another wave's (or the same wave's) MFMAs?  Register-only loops, no memory traffic:
//
//   mfma-valu-probe
//
// Each wave runs `iters` iterations of NM v_mfma_f32_32x32x16_bf16 (four independent
// accumulators) and NV v_fma_f32 (eight independent chains), written as inline assembly so the
// instruction order is exactly the one below:
//   mfma    NM MFMAs only
//   valu    NV FMAs only
//   inter   NV / NM FMAs after each MFMA (a wave overlaps its own MFMAs)
//   phases  NM MFMAs, then NV FMAs (only another wave can fill the MFMA's cycles)
// with the accumulators in VGPRs (as the attention kernel keeps them, so that the softmax works on
// the scores in place) or in AGPRs, at 1, 2 and 3 waves per SIMD (workgroups of 4 waves, 1-3 per
// CU, one round over all CUs).  Prints the device time per iteration (event-timed launches) of
// each, against the sum (no overlap) and the max (full overlap) of the MFMA-only and VALU-only
// times at the same occupancy.  Not part of the library; built by python -m layamd_amd.build --probes.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <vector>

typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

constexpr int NM = 16, NV = 128, ITERS = 2000;

#define CHECK(x)                                                                          \
  do {                                                                                    \
    hipError_t e_ = (x);                                                                  \
    if (e_ != hipSuccess) {                                                               \
      fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
      exit(1);                                                                            \
    }                                                                                     \
  } while (0)

template <bool AGPR>
__device__ __forceinline__ void mfma(f32x16_t& acc, const bf16x8_t& a, const bf16x8_t& b) {
  if constexpr (AGPR) asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
  else asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b));
}
__device__ __forceinline__ void fma_(float& x, float m, float c) {
  asm volatile("v_fma_f32 %0, %0, %1, %2" : "+v"(x) : "v"(m), "v"(c));
}

// MODE: 0 mfma, 1 valu, 2 inter, 3 phases
template <int MODE, bool AGPR>
__global__ __launch_bounds__(256) void k_probe(float* out, int iters) {
  const int lane = threadIdx.x & 63;
  bf16x8_t a, b;
  for (int i = 0; i < 8; i++) {
    a[i] = (__bf16)(0.001f * (lane + i));
    b[i] = (__bf16)(0.002f * (lane - i));
  }
  f32x16_t acc[4];
  for (int k = 0; k < 4; k++)
    for (int e = 0; e < 16; e++) acc[k][e] = 0.f;
  float x[8];
  for (int i = 0; i < 8; i++) x[i] = 0.01f * (lane + i);
  const float m = 0.999f, c = 0.001f;
  __syncthreads();
  for (int it = 0; it < iters; it++) {
    if constexpr (MODE == 0) {
#pragma unroll
      for (int j = 0; j < NM; j++) mfma<AGPR>(acc[j & 3], a, b);
    } else if constexpr (MODE == 1) {
#pragma unroll
      for (int j = 0; j < NV; j++) fma_(x[j & 7], m, c);
    } else if constexpr (MODE == 2) {
#pragma unroll
      for (int j = 0; j < NM; j++) {
        mfma<AGPR>(acc[j & 3], a, b);
#pragma unroll
        for (int v = 0; v < NV / NM; v++) fma_(x[v & 7], m, c);
      }
    } else {
#pragma unroll
      for (int j = 0; j < NM; j++) mfma<AGPR>(acc[j & 3], a, b);
#pragma unroll
      for (int j = 0; j < NV; j++) fma_(x[j & 7], m, c);
    }
  }
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  float s = 0.f;
  for (int k = 0; k < 4; k++)
    for (int e = 0; e < 16; e++) s += acc[k][e];
  for (int i = 0; i < 8; i++) s += x[i];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// nanoseconds per iteration: the launch's device time (one round of workgroups, all resident at
// once) over the iterations, the median of 5 launches after a warm-up launch
template <int MODE, bool AGPR>
static double run(int per_cu, int cus, float* out) {
  const int grid = per_cu * cus;
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  hipLaunchKernelGGL((k_probe<MODE, AGPR>), dim3(grid), dim3(256), 0, 0, out, ITERS);  // warm-up
  std::vector<double> t;
  for (int r = 0; r < 5; r++) {
    CHECK(hipEventRecord(e0, 0));
    hipLaunchKernelGGL((k_probe<MODE, AGPR>), dim3(grid), dim3(256), 0, 0, out, ITERS);
    CHECK(hipEventRecord(e1, 0));
    CHECK(hipEventSynchronize(e1));
    float ms = 0.f;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    t.push_back(ms * 1e6 / ITERS);
  }
  CHECK(hipGetLastError());
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
  std::sort(t.begin(), t.end());
  return t[2];
}

int main() {
  int cus = 0;
  CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
  float* out;
  CHECK(hipMalloc(&out, (size_t)3 * cus * 256 * sizeof(float)));
  printf("ns per iteration (each wave: %d MFMA 32x32x16 bf16, %d v_fma_f32 per iteration; the MFMAs of all\n"
         "the waves of a SIMD take %d matrix-core cycles per wave at 32 cycles each)\n", NM, NV, NM * 32);
  for (int agpr = 0; agpr < 2; agpr++) {
    for (int w = 1; w <= 3; w++) {
      double tm, tv, ti, tp;
      if (agpr) {
        tm = run<0, true>(w, cus, out); tv = run<1, true>(w, cus, out);
        ti = run<2, true>(w, cus, out); tp = run<3, true>(w, cus, out);
      } else {
        tm = run<0, false>(w, cus, out); tv = run<1, false>(w, cus, out);
        ti = run<2, false>(w, cus, out); tp = run<3, false>(w, cus, out);
      }
      printf("acc in %s, %d wave(s)/SIMD: mfma %7.1f  valu %7.1f  inter %7.1f  phases %7.1f | "
             "no overlap (mfma + valu) %7.1f, full overlap (max) %7.1f\n",
             agpr ? "AGPRs" : "VGPRs", w, tm, tv, ti, tp, tm + tv, std::max(tm, tv));
    }
  }
  CHECK(hipFree(out));
  return 0;
}
