// gemm-wave-probe: the engine's bf16 GEMM K loop (64-deep LDS DMA stages in two buffers, swizzled
// 128-byte rows, four 16-deep sub-steps per stage, fills in two bursts) in a standalone kernel
// with a plain store epilogue, built for several tile shapes and wave counts, to compare them on
// one shape with each workgroup's timeline:
//
//   gemm-wave-probe M N K        (N a multiple of 256, K of 64, M of 64)
//
// Variants: 256x256 tiles with 4 waves (2x2, 128x128 each, one wave per SIMD) and with 8 waves
// (2x4, 128x64 each, two per SIMD); 192x256 with 4 (96x128) and 8 (96x64) waves; 160x256 with 4
// waves (1x4, 160x64: the engine's tile for the N = 1024 GEMMs).  For each: device time per launch
// (20 launches), the shader clock the workgroups ran at (s_memtime cycles over s_memrealtime time),
// mean prologue, K loop, wave 0's stage waits (wait + barrier) and epilogue per workgroup, and the
// K loop's MFMA rate against the CU's rate at that clock (4 SIMDs x 1024 flop per cycle).  Results
// are checked against an fp32 product on 64 sampled rows (max relative error).  Not part of the
// library; built by python -m layamd_amd.build --probes.
#include <hip/hip_runtime.h>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef unsigned short bf16_t;

__device__ __forceinline__ u32x4_t make_rsrc(const void* p, uint32_t bytes) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  u32x4_t r;
  r[0] = (uint32_t)v;
  r[1] = (uint32_t)(v >> 32) & 0xFFFFu;
  r[2] = bytes;
  r[3] = 0x00020000u;
  return r;
}
__device__ __forceinline__ void dma16(u32x4_t rsrc, uint32_t lds, uint32_t voff, uint32_t soff) {
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" : : "{m0}"(lds), "v"(voff), "s"(rsrc), "s"(soff) : "memory");
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
#define WAIT_VM(n) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(n) : "memory")

__device__ __forceinline__ int xcd_remap(int pid, int n) {
  const int q = n >> 3, r = n & 7, x = pid & 7, j = pid >> 3;
  return x * q + min(x, r) + j;
}
__device__ __forceinline__ uint32_t dma64_voff(int row0, int r8, int ld_bytes, int lane, int odd) {
  const int rl = lane >> 3;
  return (uint32_t)(row0 + r8 + rl) * (uint32_t)ld_bytes + ((uint32_t)((lane & 7) ^ rl ^ odd) << 4);
}
__device__ __forceinline__ unsigned short f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (unsigned short)(u >> 16);
}


__device__ unsigned long long g_rec[8 * 8192];

template <int BM, int NWV, int WM, int WN>
__global__ __launch_bounds__(64 * NWV, 1) void k_probe(const bf16_t* __restrict__ A, const bf16_t* __restrict__ W,
                                                        bf16_t* __restrict__ C, int M, int N, int K) {
  const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  constexpr int BN = 256, WTM = BM / WM, WTN = BN / WN, FM = WTM / 32, FN = WTN / 32;
  constexpr int PA = BM / 8 / NWV, PB = BN / 8 / NWV;     // DMA instructions per wave and part
  static_assert(PA * 8 * NWV == BM && PB * 8 * NWV == BN, "dma plan");
  constexpr int SA = BM * 8, SW = BN * 8;                 // 16-byte chunks per part
  static_assert(WM * WN == NWV, "waves");
  __shared__ u32x4_t L[2 * (SA + SW)];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN, l32 = lane & 31, hi = lane >> 5;
  const int tilesN = (N + BN - 1) / BN, tilesM = (M + BM - 1) / BM;
  const int p = xcd_remap(blockIdx.x, tilesM * tilesN);
  constexpr int G = 8;
  const int per = G * tilesN, first = (p / per) * G, gs = min(tilesM - first, G), rr = p % per;
  const int tm = first + rr % gs, tn = rr / gs;
  const int m0 = tm * BM, n0 = tn * BN;

  const u32x4_t rA = make_rsrc(A, (uint32_t)((size_t)M * K * 2)), rB = make_rsrc(W, (uint32_t)((size_t)N * K * 2));
  const u32x4_t rNone = make_rsrc(A, 0u);
  const int ldb = K * 2;
  uint32_t va[2], vb[2];
  va[0] = dma64_voff(m0, wave * PA * 8, ldb, lane, (wave * PA) & 1);
  va[1] = dma64_voff(m0, wave * PA * 8, ldb, lane, ((wave * PA) & 1) ^ 1);
  vb[0] = dma64_voff(n0, wave * PB * 8, ldb, lane, (wave * PB) & 1);
  vb[1] = dma64_voff(n0, wave * PB * 8, ldb, lane, ((wave * PB) & 1) ^ 1);
  const uint32_t wsa = (uint32_t)__builtin_amdgcn_readfirstlane(wave) * (uint32_t)(PA * 1024);
  const uint32_t wsb = (uint32_t)__builtin_amdgcn_readfirstlane(wave) * (uint32_t)(PB * 1024);
  const int ns = K / 32;
  u32x4_t* T0a = L;
  u32x4_t* T0b = L + SA;
  u32x4_t* T1a = L + SA + SW;
  u32x4_t* T1b = L + 2 * SA + SW;
  auto op_a = [&](int o, uint32_t la, int g) {
    dma16(2 * g < ns ? rA : rNone, la + wsa + o * 1024, va[o & 1], (uint32_t)g * 128u + (uint32_t)(o * 8 * ldb));
  };
  auto op_b = [&](int o, uint32_t lb, int g) {
    dma16(2 * g < ns ? rB : rNone, lb + wsb + o * 1024, vb[o & 1], (uint32_t)g * 128u + (uint32_t)(o * 8 * ldb));
  };
#pragma unroll
  for (int o = 0; o < PA; o++) op_a(o, lds_addr(T0a), 0);
#pragma unroll
  for (int o = 0; o < PB; o++) op_b(o, lds_addr(T0b), 0);
#pragma unroll
  for (int o = 0; o < PA; o++) op_a(o, lds_addr(T1a), 1);

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;
  const int arow = wm * WTM + l32, brow = wn * WTN + l32;
  const int sw = (lane & 7) ^ ((lane >> 3) & 1);
  struct Fr { u32x4_t a[FM], b[FN]; };
  Fr F0, F1;
  constexpr int NMM = FM * FN, E = FM + FN, EW = PB + E, EA = PA + E;
  auto ld = [&](Fr& f, int idx, const u32x4_t* As, const u32x4_t* Bs, int s) {
    if (idx < FM) f.a[idx] = As[(arow + idx * 32) * 8 + ((2 * s + hi) ^ sw)];
    else f.b[idx - FM] = Bs[(brow + (idx - FM) * 32) * 8 + ((2 * s + hi) ^ sw)];
  };
  auto mma = [&](const Fr& f, int t) {
    const int i = t / FN, j = t % FN;
    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, f.b[j]),
                                                        __builtin_bit_cast(bf16x8_t, f.a[i]), acc[i][j], 0, 0, 0);
  };
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  WAIT_VM(PA);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
#pragma unroll
  for (int o = 0; o < E; o++) ld(F0, o, T0a, T0b, 0);
  auto sub = [&](Fr& FX, Fr& FY, const u32x4_t* Ca, const u32x4_t* Cb, int s) {
#pragma unroll
    for (int t = 0; t < NMM; t++) {
      mma(FX, t);
#pragma unroll
      for (int o = t * E / NMM; o < (t + 1) * E / NMM; o++) ld(FY, o, Ca, Cb, s);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  unsigned long long wsum = 0;
  auto stage = [&](u32x4_t* Ca, u32x4_t* Cb, u32x4_t* Na, u32x4_t* Nb, int g) {
#pragma unroll
    for (int t = 0; t < NMM; t++) {
      mma(F0, t);
#pragma unroll
      for (int o = t * EW / NMM; o < (t + 1) * EW / NMM; o++) {
        if (o < PB) op_b(o, lds_addr(Nb), g + 1);
        else ld(F1, o - PB, Ca, Cb, 1);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    sub(F1, F0, Ca, Cb, 2);
    sub(F0, F1, Ca, Cb, 3);
    const unsigned long long w0 = __builtin_amdgcn_s_memtime();
    WAIT_VM(0);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    { const unsigned long long w1 = __builtin_amdgcn_s_memtime(); __builtin_amdgcn_s_waitcnt(0xC07F); wsum += w1 - w0; }
#pragma unroll
    for (int t = 0; t < NMM; t++) {
      mma(F1, t);
#pragma unroll
      for (int o = t * EA / NMM; o < (t + 1) * EA / NMM; o++) {
        if (o < PA) op_a(o, lds_addr(Ca), g + 2);
        else ld(F0, o - PA, Na, Nb, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  const int nst = ns / 2;
  int g = 0;
  for (; g + 2 < nst; g += 2) {
    stage(T0a, T0b, T1a, T1b, g);
    stage(T1a, T1b, T0a, T0b, g + 1);
  }
  const u32x4_t *La = T0a, *Lb = T0b;
  if (g + 2 == nst) {
    stage(T0a, T0b, T1a, T1b, g);
    La = T1a; Lb = T1b;
  }
  sub(F0, F1, La, Lb, 1);
  sub(F1, F0, La, Lb, 2);
  sub(F0, F1, La, Lb, 3);
#pragma unroll
  for (int t = 0; t < NMM; t++) mma(F1, t);
  WAIT_VM(0);
  const unsigned long long t2 = __builtin_amdgcn_s_memtime();

  // lane: row m0 + wm WTM + 32 i + l32, columns n0 + wn WTN + 32 j + 8 g + 4 hi + (0..3)
#pragma unroll
  for (int i = 0; i < FM; i++) {
    const int row = m0 + wm * WTM + 32 * i + l32;
    if (row >= M) continue;
#pragma unroll
    for (int j = 0; j < FN; j++)
#pragma unroll
      for (int gg = 0; gg < 4; gg++) {
        const int col = n0 + wn * WTN + 32 * j + 8 * gg + 4 * hi;
        if (col >= N) continue;
        uint2 u;
        u.x = (uint32_t)f2bf(acc[i][j][4 * gg + 0]) | ((uint32_t)f2bf(acc[i][j][4 * gg + 1]) << 16);
        u.y = (uint32_t)f2bf(acc[i][j][4 * gg + 2]) | ((uint32_t)f2bf(acc[i][j][4 * gg + 3]) << 16);
        *reinterpret_cast<uint2*>(C + (size_t)row * N + col) = u;
      }
  }
  if (tid == 0 && blockIdx.x < 8192) {
    const unsigned long long t3 = __builtin_amdgcn_s_memtime(), r3 = __builtin_amdgcn_s_memrealtime();
    unsigned long long* q = g_rec + 8 * blockIdx.x;
    q[0] = r0; q[1] = r3; q[2] = t1 - t0; q[3] = t2 - t1; q[4] = t3 - t2; q[5] = wsum; q[6] = 0; q[7] = t3 - t0;
  }
}

// reference: one thread per output, fp32
__global__ void k_ref(const bf16_t* A, const bf16_t* W, float* C, int M, int N, int K, int rows) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= rows * N) return;
  const int r = (idx / N) * (M / rows), n = idx % N;
  float s = 0.f;
  for (int k = 0; k < K; k++)
    s += __uint_as_float((uint32_t)A[(size_t)r * K + k] << 16) * __uint_as_float((uint32_t)W[(size_t)n * K + k] << 16);
  C[idx] = s;
}

static unsigned short host_bf(float f) {
  uint32_t u; memcpy(&u, &f, 4);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (unsigned short)(u >> 16);
}

int main(int argc, char** argv) {
  const int M = atoi(argv[1]), N = atoi(argv[2]), K = atoi(argv[3]);
  if (N % 256 || K % 64 || M % 64) { printf("N multiple of 256, K of 64, M of 64\n"); return 1; }
  std::vector<unsigned short> hA((size_t)M * K), hW((size_t)N * K);
  uint32_t s = 12345;
  auto rnd = [&]() { s = s * 1664525u + 1013904223u; return ((s >> 8) & 0xFFFF) / 65536.0f - 0.5f; };
  for (auto& x : hA) x = host_bf(rnd());
  for (auto& x : hW) x = host_bf(0.05f * rnd());
  bf16_t *dA, *dW, *dC;
  float* dR;
  const int rows = 64;
  hipMalloc(&dA, hA.size() * 2); hipMalloc(&dW, hW.size() * 2); hipMalloc(&dC, (size_t)M * N * 2);
  hipMalloc(&dR, (size_t)rows * N * 4);
  hipMemcpy(dA, hA.data(), hA.size() * 2, hipMemcpyHostToDevice);
  hipMemcpy(dW, hW.data(), hW.size() * 2, hipMemcpyHostToDevice);
  hipLaunchKernelGGL(k_ref, dim3((rows * N + 255) / 256), dim3(256), 0, 0, dA, dW, dR, M, N, K, rows);
  std::vector<float> hR((size_t)rows * N);
  hipMemcpy(hR.data(), dR, hR.size() * 4, hipMemcpyDeviceToHost);
  hipEvent_t e0, e1; hipEventCreate(&e0); hipEventCreate(&e1);
  void* recp = nullptr;
  hipGetSymbolAddress(&recp, HIP_SYMBOL(g_rec));
  auto run = [&](auto kern, int bm, int threads, const char* name) {
    const int tiles = ((M + bm - 1) / bm) * (N / 256);
    if (tiles > 8192) { printf("too many tiles\n"); return; }
    hipMemset(dC, 0, (size_t)M * N * 2);
    hipLaunchKernelGGL(kern, dim3(tiles), dim3(threads), 0, 0, dA, dW, dC, M, N, K);
    hipDeviceSynchronize();
    std::vector<unsigned short> hC((size_t)M * N);
    hipMemcpy(hC.data(), dC, hC.size() * 2, hipMemcpyDeviceToHost);
    double maxerr = 0;
    for (int i = 0; i < rows; i++)
      for (int n = 0; n < N; n++) {
        const int r = i * (M / rows);
        uint32_t u = (uint32_t)hC[(size_t)r * N + n] << 16; float c; memcpy(&c, &u, 4);
        const double ref = hR[(size_t)i * N + n];
        maxerr = fmax(maxerr, fabs(c - ref) / (fabs(ref) + 0.05));
      }
    const int it = 20;
    hipEventRecord(e0);
    for (int k = 0; k < it; k++) hipLaunchKernelGGL(kern, dim3(tiles), dim3(threads), 0, 0, dA, dW, dC, M, N, K);
    hipEventRecord(e1); hipEventSynchronize(e1);
    float ms; hipEventElapsedTime(&ms, e0, e1);
    std::vector<unsigned long long> rec((size_t)tiles * 8);
    hipMemcpy(rec.data(), recp, rec.size() * 8, hipMemcpyDeviceToHost);
    double cyc = 0, rt = 0, pro = 0, kl = 0, ep = 0, w = 0; unsigned long long rmin = ~0ull, rmax = 0;
    for (int t = 0; t < tiles; t++) {
      const unsigned long long* q = &rec[(size_t)t * 8];
      cyc += q[7]; rt += (double)(q[1] - q[0]) / 100.0; pro += q[2]; kl += q[3]; ep += q[4]; w += q[5];
      rmin = q[0] < rmin ? q[0] : rmin; rmax = q[1] > rmax ? q[1] : rmax;
    }
    const double ghz = cyc / rt / 1e3;
    const double klus = kl / tiles / ghz / 1e3;
    const double rate = 2.0 * bm * 256 * K / (klus * 1e-6), peak = 4096.0 * ghz * 1e9;
    const double us = ms * 1e3 / it;
    printf("%-14s %5dx%5dx%5d tiles %4d: %6.1f us %5.0f TF | clk %.2f GHz pro %.2f kloop %.2f (waits %.2f) epi %.2f us, kloop %.0f%% of MFMA at clk | err %.4f\n",
           name, M, N, K, tiles, us, 2.0 * M * N * K / us / 1e6, ghz, pro / tiles / ghz / 1e3, klus, w / tiles / ghz / 1e3,
           ep / tiles / ghz / 1e3, 100 * rate / peak, maxerr);
  };
  run(k_probe<256, 4, 2, 2>, 256, 256, "256x256 w4");
  run(k_probe<256, 8, 2, 4>, 256, 512, "256x256 w8 2x4");
  run(k_probe<192, 4, 2, 2>, 192, 256, "192x256 w4");
  run(k_probe<192, 8, 2, 4>, 192, 512, "192x256 w8 2x4");
  run(k_probe<160, 4, 1, 4>, 160, 256, "160x256 w4 1x4");
  return 0;
}
