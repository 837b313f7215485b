// MFMA GEMM for gfx950: C[M,N] = A[M,K] . W[N,K]^T with fused epilogues.
//
// Both operands are K-contiguous (activations [rows, K], weights in their checkpoint [out, in]
// layout), which is the layout the MFMA operand registers want: a lane of
// v_mfma_f32_16x16x32_bf16 holds 8 consecutive K values of one row of A and one column of B, so
// every fragment is one 16-byte LDS read and no weight is ever transposed.  The fp32 path uses
// v_mfma_f32_16x16x4_f32 on the same tiles (a 16-byte chunk = 4 K values = 4 MFMAs).
//
// Tiling: a 256-thread workgroup (4 wave64s in a WM x WN grid) computes a BM x BN tile; K
// advances in 128-byte slices (64 bf16 / 32 fp32) through double-buffered LDS with an XOR
// swizzle of the 16-byte chunks (chunk ^ (row & 7)) so a fragment read by 16 lanes covers all
// banks.  The next slice is fetched into registers while the current one feeds the MFMAs.
// Workgroup ids are remapped so each of the 8 XCDs (own L2) walks a contiguous run of tiles.
//
// Epilogues (accumulator element i of lane l in a 16x16 block is row 4*(l/16)+i, col l%16):
//   EPI_STORE  C = act(acc + bias)                        (storage type)
//   EPI_RESID  X += acc + bias                            (fp32 residual stream)
//   EPI_QKV    q,k (RoPE when tables are given) -> Q, K [rows][H*HD]; v -> V^T [H*HD][ldv] at
//              column vcol[row].  With RoPE the q/k weight rows of each head are stored in the
//              order d = [0..15, 32..47, 16..31, 48..63], so rotate_half partners (d, d+32) sit in
//              adjacent 16-column blocks of the same lane.
//   EPI_GEGLU  W rows stored as alternating 16-row blocks of input and gate rows; writes
//              gelu_erf(input) * gate into C [rows][N/2].
#include "kernels.h"

namespace laya {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));   // one 16-byte chunk

template <typename T> struct Mma;
template <> struct Mma<bf16_t> {
  static __device__ __forceinline__ void run(f32x4_t& c, const u32x4_t& a, const u32x4_t& b) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c, 0,
                                                0, 0);
  }
};
template <> struct Mma<float> {
  static __device__ __forceinline__ void run(f32x4_t& c, const u32x4_t& a, const u32x4_t& b) {
    const f32x4_t fa = __builtin_bit_cast(f32x4_t, a), fb = __builtin_bit_cast(f32x4_t, b);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[0], fb[0], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[1], fb[1], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[2], fb[2], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[3], fb[3], c, 0, 0, 0);
  }
};

// Workgroups are dispatched round-robin over the 8 XCDs; give XCD x the contiguous tile range
// [x*q + min(x, r), ...) so neighbouring tiles (sharing A rows) share an L2.  Bijective on [0, n).
__device__ __forceinline__ int xcd_remap(int pid, int n) {
  const int q = n >> 3, r = n & 7, x = pid & 7, j = pid >> 3;
  return x * q + min(x, r) + j;
}

template <typename T>
__device__ __forceinline__ void store_elt(void* base, size_t idx, float v) {
  Elt<T>::st(reinterpret_cast<T*>(base) + idx, v);
}

template <typename T, int BM, int BN, int WM, int WN, int EPI>
__global__ __launch_bounds__(256) void k_gemm(const GemmArgs a) {
  constexpr int BK = 128 / (int)sizeof(T);
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 16, FN = WTN / 16;
  constexpr int ACH = BM / 32, BCH = BN / 32;
  static_assert(WM * WN == 4, "4 waves");
  static_assert(WTM % 16 == 0 && WTN % 16 == 0, "wave tile");
  __shared__ u32x4_t As[2][BM * 8];
  __shared__ u32x4_t Bs[2][BN * 8];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN, l16 = lane & 15, g = lane >> 4;
  const int tilesN = (a.N + BN - 1) / BN, tilesM = (a.M + BM - 1) / BM;
  const int pid = xcd_remap(blockIdx.x, tilesM * tilesN);
  const int m0 = (pid / tilesN) * BM, n0 = (pid % tilesN) * BN;

  const int crow = tid >> 3, cch = tid & 7;
  const char* aptr[ACH];
  const char* bptr[BCH];
#pragma unroll
  for (int j = 0; j < ACH; j++) {
    const int r = min(m0 + crow + 32 * j, a.M - 1);
    aptr[j] = reinterpret_cast<const char*>(a.A) + (size_t)r * a.lda * sizeof(T) + cch * 16;
  }
#pragma unroll
  for (int j = 0; j < BCH; j++) {
    const int r = min(n0 + crow + 32 * j, a.N - 1);
    bptr[j] = reinterpret_cast<const char*>(a.W) + (size_t)r * a.ldw * sizeof(T) + cch * 16;
  }
  u32x4_t ra[ACH], rb[BCH];
  f32x4_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++) acc[i][j] = (f32x4_t){0.f, 0.f, 0.f, 0.f};

  const int nk = a.K / BK;
#pragma unroll
  for (int j = 0; j < ACH; j++) ra[j] = *reinterpret_cast<const u32x4_t*>(aptr[j]);
#pragma unroll
  for (int j = 0; j < BCH; j++) rb[j] = *reinterpret_cast<const u32x4_t*>(bptr[j]);
#pragma unroll
  for (int j = 0; j < ACH; j++) { const int r = crow + 32 * j; As[0][r * 8 + (cch ^ (r & 7))] = ra[j]; }
#pragma unroll
  for (int j = 0; j < BCH; j++) { const int r = crow + 32 * j; Bs[0][r * 8 + (cch ^ (r & 7))] = rb[j]; }
  __syncthreads();

  for (int kt = 0; kt < nk; kt++) {
    const int stg = kt & 1;
    if (kt + 1 < nk) {
      const size_t off = (size_t)(kt + 1) * 128;
#pragma unroll
      for (int j = 0; j < ACH; j++) ra[j] = *reinterpret_cast<const u32x4_t*>(aptr[j] + off);
#pragma unroll
      for (int j = 0; j < BCH; j++) rb[j] = *reinterpret_cast<const u32x4_t*>(bptr[j] + off);
    }
#pragma unroll
    for (int s = 0; s < 2; s++) {
      const int ch = (4 * s + g) ^ (l16 & 7);
      u32x4_t af[FM], bfr[FN];
#pragma unroll
      for (int i = 0; i < FM; i++) af[i] = As[stg][(wm * WTM + i * 16 + l16) * 8 + ch];
#pragma unroll
      for (int j = 0; j < FN; j++) bfr[j] = Bs[stg][(wn * WTN + j * 16 + l16) * 8 + ch];
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) Mma<T>::run(acc[i][j], af[i], bfr[j]);
    }
    if (kt + 1 < nk) {
#pragma unroll
      for (int j = 0; j < ACH; j++) { const int r = crow + 32 * j; As[stg ^ 1][r * 8 + (cch ^ (r & 7))] = ra[j]; }
#pragma unroll
      for (int j = 0; j < BCH; j++) { const int r = crow + 32 * j; Bs[stg ^ 1][r * 8 + (cch ^ (r & 7))] = rb[j]; }
    }
    __syncthreads();
  }

  // ---------------- epilogue ----------------
  const int rbase = m0 + wm * WTM + 4 * g, cbase = n0 + wn * WTN;
  if constexpr (EPI == EPI_STORE || EPI == EPI_RESID) {
#pragma unroll
    for (int j = 0; j < FN; j++) {
      const int col = cbase + j * 16 + l16;
      if (col >= a.N) continue;
      const float bb = a.bias ? a.bias[col] : 0.f;
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int row = rbase + i * 16 + e;
          if (row >= a.M) continue;
          float v = acc[i][j][e] + bb;
          if constexpr (EPI == EPI_STORE) {
            if (a.act == ACT_RELU) v = fmaxf(v, 0.f);
            else if (a.act == ACT_GELU) v = gelu_erf(v);
            store_elt<T>(a.C, (size_t)row * a.ldc + col, v);
          } else {
            float* xp = a.X + (size_t)row * a.ldx + col;
            *xp += v;
          }
        }
    }
  } else if constexpr (EPI == EPI_GEGLU) {
    static_assert(WTN % 32 == 0, "GeGLU pairs");
#pragma unroll
    for (int j = 0; j < FN; j += 2) {
      const int cin = cbase + j * 16;          // first column of the input block
      if (cin + l16 >= a.N) continue;
      const int oc = cin / 2 + l16;
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int row = rbase + i * 16 + e;
          if (row >= a.M) continue;
          const float x = acc[i][j][e] + (a.bias ? a.bias[cin + l16] : 0.f);
          const float y = acc[i][j + 1][e] + (a.bias ? a.bias[cin + 16 + l16] : 0.f);
          store_elt<T>(a.C, (size_t)row * a.ldc + oc, gelu_erf(x) * y);
        }
    }
  } else {  // EPI_QKV
    const int D = a.H * a.HD;
    const bool rope = a.rope_cos != nullptr;
#pragma unroll
    for (int j = 0; j < FN; j++) {
      const int c0 = cbase + j * 16;           // block start column
      if (c0 >= a.N) continue;
      const int sec = c0 / D, e0 = c0 % D, h = e0 / a.HD, t = e0 % a.HD;
      const float* bb = a.bias ? a.bias + c0 : nullptr;
      if (sec == 2) {
        T* vt = reinterpret_cast<T*>(a.Vt) + (size_t)(h * a.HD + t + l16) * a.ldv;
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const int row = rbase + i * 16 + e;
            if (row >= a.M) continue;
            Elt<T>::st(vt + a.vcol[row], acc[i][j][e] + (bb ? bb[l16] : 0.f));
          }
        continue;
      }
      T* dst = reinterpret_cast<T*>(sec == 0 ? a.Q : a.Kt);
      if (!rope) {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const int row = rbase + i * 16 + e;
            if (row >= a.M) continue;
            Elt<T>::st(dst + (size_t)row * a.ldqk + h * a.HD + t + l16, acc[i][j][e] + (bb ? bb[l16] : 0.f));
          }
        continue;
      }
      // rope: blocks of a head are (t=0: d 0..15), (16: d 32..47), (32: d 16..31), (48: d 48..63);
      // the pair (a, b) = (d, d + 32) lives in blocks j and j + 1 when t is 0 or 32.
      if (t != 0 && t != 32) continue;         // handled together with its partner block
      if (j + 1 >= FN) continue;               // cannot happen: WTN is a multiple of 64
      const int dlo = t == 0 ? 0 : 16;         // frequency index base and first-half dim base
      const float* bb2 = a.bias ? a.bias + c0 + 16 : nullptr;
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int row = rbase + i * 16 + e;
          if (row >= a.M) continue;
          const int p = a.pos[row];
          const float c = a.rope_cos[p * (a.HD / 2) + dlo + l16], s = a.rope_sin[p * (a.HD / 2) + dlo + l16];
          const float x1 = acc[i][j][e] + (bb ? bb[l16] : 0.f);
          const float x2 = acc[i][j + 1][e] + (bb2 ? bb2[l16] : 0.f);
          T* o = dst + (size_t)row * a.ldqk + h * a.HD + dlo + l16;
          Elt<T>::st(o, x1 * c - x2 * s);
          Elt<T>::st(o + a.HD / 2, x2 * c + x1 * s);
        }
    }
  }
}

template <typename T, int BM, int BN, int WM, int WN>
static void launch_cfg(int epi, const GemmArgs& a, hipStream_t st) {
  const int tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  switch (epi) {
    case EPI_STORE: hipLaunchKernelGGL((k_gemm<T, BM, BN, WM, WN, EPI_STORE>), dim3(tiles), dim3(256), 0, st, a); break;
    case EPI_RESID: hipLaunchKernelGGL((k_gemm<T, BM, BN, WM, WN, EPI_RESID>), dim3(tiles), dim3(256), 0, st, a); break;
    case EPI_QKV: hipLaunchKernelGGL((k_gemm<T, BM, BN, WM, WN, EPI_QKV>), dim3(tiles), dim3(256), 0, st, a); break;
    case EPI_GEGLU: hipLaunchKernelGGL((k_gemm<T, BM, BN, WM, WN, EPI_GEGLU>), dim3(tiles), dim3(256), 0, st, a); break;
    default: fprintf(stderr, "[laya] gemm: bad epilogue %d\n", epi); exit(1);
  }
}

bool gemm_shape_ok(int epi, const GemmArgs& a, int elt_bytes, const char** why) {
  const int bk = 128 / elt_bytes, align = 16 / elt_bytes;
  if (a.M <= 0 || a.N <= 0) { *why = "empty"; return false; }
  if (a.K <= 0 || a.K % bk) { *why = "K must be a positive multiple of the 128-byte K slice"; return false; }
  if (a.lda % align || a.ldw % align || a.lda < a.K || a.ldw < a.K) { *why = "row strides must be 16-byte multiples >= K"; return false; }
  if ((reinterpret_cast<uintptr_t>(a.A) | reinterpret_cast<uintptr_t>(a.W)) & 15) { *why = "operands must be 16-byte aligned"; return false; }
  if (epi == EPI_GEGLU && a.N % 32) { *why = "GeGLU needs N % 32 == 0"; return false; }
  if (epi == EPI_QKV) {
    if (a.N != 3 * a.H * a.HD || a.HD % 16) { *why = "QKV needs N == 3*H*HD, HD % 16 == 0"; return false; }
    if (a.rope_cos && a.HD != 64) { *why = "fused RoPE needs HD == 64"; return false; }
  }
  return true;
}

template <typename T>
void launch_gemm(int epi, const GemmArgs& a, hipStream_t st) {
  const char* why = "";
  if (!gemm_shape_ok(epi, a, (int)sizeof(T), &why)) {
    fprintf(stderr, "[laya] gemm %dx%dx%d epi %d rejected: %s\n", a.M, a.N, a.K, epi, why);
    exit(1);
  }
  launch_cfg<T, 128, 128, 2, 2>(epi, a, st);
}

template void launch_gemm<float>(int, const GemmArgs&, hipStream_t);
template void launch_gemm<bf16_t>(int, const GemmArgs&, hipStream_t);

}  // namespace laya
