// Shared device/host helpers for the gfx950 Laya engine: error checks, the two element types
// (bf16 storage with fp32 math, or fp32), and wave64 reductions.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <cstdint>
#include <cstdio>
#include <cstdlib>

#define LAYA_HIP(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { \
  fprintf(stderr, "[laya] HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); exit(1); } } while (0)

namespace laya {

// Kernel timing for the stage profiler.  While a LaunchTimer is installed on the calling thread,
// every kernel launch of this library takes an event pair from it and goes through
// hipExtLaunchKernelGGL, which stores that kernel's own start and end times in the two events: no
// marker between launches and no host synchronization, so a stage's time is its kernels' device
// time, as a kernel trace reports it.
struct LaunchTimer {
  virtual void events(hipEvent_t* start, hipEvent_t* stop) = 0;
};
extern thread_local LaunchTimer* g_launch_timer;

#define LAYA_LAUNCH(kernel, grid, block, shmem, stream, ...)                                    \
  do {                                                                                          \
    if (laya::g_launch_timer) {                                                                 \
      hipEvent_t ev_a_, ev_b_;                                                                  \
      laya::g_launch_timer->events(&ev_a_, &ev_b_);                                             \
      hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, ev_a_, ev_b_, 0u, __VA_ARGS__); \
    } else {                                                                                    \
      hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__);                      \
    }                                                                                           \
  } while (0)

typedef uint16_t bf16_t;                       // bf16 bit pattern in memory

__host__ __device__ inline float bf2f(bf16_t b) {
  union { uint32_t u; float f; } c; c.u = (uint32_t)b << 16; return c.f;
}
__host__ __device__ inline bf16_t f2bf(float f) {     // round to nearest even (finite inputs)
  union { uint32_t u; float f; } c; c.f = f;
  uint32_t r = ((c.u >> 16) & 1u) + 0x7FFFu;
  return (bf16_t)((c.u + r) >> 16);
}

// Element-type traits: loads/stores of one element with fp32 math.
template <typename T> struct Elt;
template <> struct Elt<float> {
  static __device__ __forceinline__ float ld(const float* p) { return *p; }
  static __device__ __forceinline__ void st(float* p, float v) { *p = v; }
};
template <> struct Elt<bf16_t> {
  static __device__ __forceinline__ float ld(const bf16_t* p) { return bf2f(*p); }
  static __device__ __forceinline__ void st(bf16_t* p, float v) { *p = f2bf(v); }
};

// Wave64 reductions (all 64 lanes active): within each 16-lane row by DPP (quad_perm xor 1,
// quad_perm xor 2, row_half_mirror, row_mirror: each step pairs lanes whose values are equal
// within their groups, so every lane of a row ends with the same row total), then the four row
// totals read as scalars and combined as (r0 + r1) + (r2 + r3).  No LDS round trip.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_f32(float v, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); }
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f32<0xB1>(v);                                  // quad_perm [1, 0, 3, 2]
  v += dpp_f32<0x4E>(v);                                  // quad_perm [2, 3, 0, 1]
  v += dpp_f32<0x141>(v);                                 // row_half_mirror
  v += dpp_f32<0x140>(v);                                 // row_mirror
  return (lane_f32(v, 0) + lane_f32(v, 16)) + (lane_f32(v, 32) + lane_f32(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x141>(v));
  v = fmaxf(v, dpp_f32<0x140>(v));
  return fmaxf(fmaxf(lane_f32(v, 0), lane_f32(v, 16)), fmaxf(lane_f32(v, 32), lane_f32(v, 48)));
}

// exact (erf) GELU, as torch.nn.functional.gelu with approximate="none"
__device__ __forceinline__ float gelu_erf(float x) { return 0.5f * x * (1.f + erff(x * 0.70710678118654752440f)); }

// The same erf GELU with erf from Abramowitz & Stegun, Handbook of Mathematical Functions, formula
// 7.1.26: erf(z) = 1 - (a1 t + a2 t^2 + a3 t^3 + a4 t^4 + a5 t^5) exp(-z^2), t = 1 / (1 + p z),
// z >= 0, |error| <= 1.5e-7.  Used where the result is rounded to bf16 (2^-9 relative), about a
// quarter of the instructions of the library erff.  z = |x| / sqrt(2) is folded into the
// constants: p z = (p / sqrt 2) |x| and exp(-z^2) = 2^(-x^2 log2(e) / 2); the result is
// x (1/2 + erf / 2) with the sign of x on the erf term.
__device__ __forceinline__ float gelu_erf_as(float x) {
  const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f * 0.70710678118654752440f, fabsf(x), 1.0f));
  const float poly = t * fmaf(t, fmaf(t, fmaf(t, fmaf(t, 1.061405429f, -1.453152027f), 1.421413741f), -0.284496736f),
                              0.254829592f);
  const float e = fmaf(-poly, __builtin_amdgcn_exp2f(x * x * -0.72134752044448170368f), 1.0f);
  return x * fmaf(0.5f, copysignf(e, x), 0.5f);
}

}  // namespace laya
