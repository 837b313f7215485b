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
//              column = row.  A wave's column range covers whole 64-wide heads, so the
//              rotate_half partners (d, d+32) of a row sit in the same lane.
//   EPI_GEGLU  W rows stored as alternating 32-row blocks of input and gate rows; writes
//              gelu_erf(input) * gate into C [rows][N/2].
#include <cmath>

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
    // 32-column groups [input 32 | gate 32]: block j pairs with block j + 2
    static_assert(WTN % 64 == 0, "GeGLU pairs");
#pragma unroll
    for (int j = 0; j < FN; j++) {
      if ((j & 3) >= 2) continue;
      const int cin = cbase + j * 16;          // first column of the input block
      if (cin + l16 >= a.N) continue;
      const int oc = (cin / 64) * 32 + (cin % 64) + l16;
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int row = rbase + i * 16 + e;
          if (row >= a.M) continue;
          const float x = acc[i][j][e] + (a.bias ? a.bias[cin + l16] : 0.f);
          const float y = acc[i][j + 2][e] + (a.bias ? a.bias[cin + 32 + l16] : 0.f);
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
            Elt<T>::st(vt + row, acc[i][j][e] + (bb ? bb[l16] : 0.f));
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
      // rope: rotate_half partners (d, d + 32) are blocks j and j + 2 of the head (t = 0 or 16)
      if (t >= 32) continue;                   // handled together with its partner block
      const float* bb2 = a.bias ? a.bias + c0 + 32 : nullptr;
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int row = rbase + i * 16 + e;
          if (row >= a.M) continue;
          const int p = a.pos[row];
          const float c = a.rope_cos[p * (a.HD / 2) + t + l16], s = a.rope_sin[p * (a.HD / 2) + t + l16];
          const float x1 = acc[i][j][e] + (bb ? bb[l16] : 0.f);
          const float x2 = acc[i][j + 2][e] + (bb2 ? bb2[l16] : 0.f);
          T* o = dst + (size_t)row * a.ldqk + h * a.HD + t + l16;
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



typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// two floats -> packed bf16 pair (v_cvt_pk_bf16_f32, round to nearest even)
__device__ __forceinline__ uint32_t pk_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}

// Adjacent lanes hold adjacent columns; each lane holds rows r and r+1 of its column (ve, ve1).
// One DPP swap (quad_perm 1,0,3,2 = lane ^ 1) gives the even lane row r of columns (c, c+1) and
// the odd lane row r+1 of columns (c-1, c), packed as bf16 pairs.
__device__ __forceinline__ uint32_t pair_rows_to_cols(float ve, float ve1, bool odd) {
  const float send = odd ? ve : ve1;
  const float recv = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, send), 0xB1, 0xF, 0xF, false));
  return odd ? pk_bf16(recv, ve1) : pk_bf16(ve, recv);
}

// ======================================================================================
// Large-tile bf16 GEMM (v_mfma_f32_32x32x16_bf16).  A workgroup of 4 wave64s computes a
// BM x BN tile (256x256 by default, one workgroup per CU, 128 KiB of LDS for two K stages);
// each wave owns a (BM/WM) x (BN/WN) sub-tile held in 32x32 accumulator blocks, so one
// 16-byte LDS fragment feeds 4 MFMAs and LDS traffic stays well under the MFMA rate.
// Global loads go through buffer resources: rows beyond M (or N) fall outside the resource and
// read as zero, so partial tiles need no clamping.  Tiles are ordered in groups of 8 tile rows
// inside each XCD's contiguous range so the tiles running at once on an XCD share A rows and
// W columns in its L2.
//
// 32x32 accumulator layout: element e of lane l is row 8*(e/4) + 4*(l/32) + e%4, col l%32.
// A/B operand: lane l holds 8 consecutive K values of row (col) l%32, K offset 8*(l/32).
// ======================================================================================
typedef float f32x16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ void tile_coords(int bid, int tilesM, int tilesN, int& tm, int& tn) {
  const int p = xcd_remap(bid, tilesM * tilesN);
  constexpr int G = 8;
  const int per = G * tilesN, first = (p / per) * G, gs = min(tilesM - first, G), r = p % per;
  tm = first + r % gs;
  tn = r / gs;
}

// Buffer resource (V#) of a raw byte range: base, stride 0, num_records = bytes (offsets at or past
// it read as zero without touching memory), dword 3 = the gfx9 raw-buffer format word.
__device__ __forceinline__ u32x4_t make_rsrc(const void* p, uint32_t bytes) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  u32x4_t r;
  r[0] = (uint32_t)v;
  r[1] = (uint32_t)(v >> 32) & 0xFFFFu;
  r[2] = bytes;
  r[3] = 0x00020000u;
  return r;
}

// One LDS DMA instruction: lane l copies 16 bytes at rsrc + voff + soff to LDS address lds + 16 l.
// Issued as inline assembly (M0 holds the LDS base; one wait state between the M0 write and the
// DMA; no compiler-generated code in these kernels reads M0, which gfx9 LDS instructions ignore),
// so the compiler sees no LDS write and inserts no waits of its own between these fills and the
// fragment reads: the main loop orders them with explicit vmcnt waits and barriers.  The memory
// clobber keeps the compiler from moving LDS reads across the fill.
__device__ __forceinline__ void dma16(u32x4_t rsrc, uint32_t lds, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(lds), "v"(voff), "s"(rsrc), "s"(soff)
               : "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// LDS fill by DMA: each wave instruction fills 64 consecutive 16-byte chunks = 16 tile rows of
// one 32-deep K slice (64 bytes per row).  The swizzle is applied on the global side: the lane
// landing at row r, chunk position c loads global chunk c ^ f(r), f(r) = ((r >> 1) & 3) ^
// ((r >> 3) & 1).  A fragment read has lane l on row l % 32 at one logical chunk; with 64 banks of
// 4 bytes each group of 16 lanes then covers 16 distinct 16-byte bank positions ((r & 3) * 4 +
// (k ^ f(r)) over r = 0..15), and each group of 8 covers 8 of 8 with 32 banks, so the reads are
// conflict-free.  The per-lane offset (row * ld + swizzled chunk) is fixed over K; the slice's K
// byte offset goes in the scalar offset.  Rows past M (or N) are out of range by the per-lane
// offset alone and arrive as zeros; a slice past the last one is fetched through a resource of
// zero length, so it reads nothing.
__device__ __forceinline__ uint32_t dma_voff(int row0, int r, int ld_bytes, int lane) {
  const int cpos = lane & 3;
  return (uint32_t)(row0 + r) * (uint32_t)ld_bytes + ((uint32_t)(cpos ^ ((r >> 1) & 3) ^ ((r >> 3) & 1)) << 4);
}

// Fragments of one 16-deep K step: lane l holds 8 consecutive K values (16 bytes) of tile row
// (row base + 32 i + l % 32), K offset 8 * (l / 32); ks selects the step within the 32-deep slice.
template <int FM, int FN>
struct Frags {
  u32x4_t a[FM], b[FN];
};

template <int FM, int FN>
__device__ __forceinline__ void load_frags(Frags<FM, FN>& f, const u32x4_t* As, const u32x4_t* Bs, int arow, int brow,
                                           int ks, int hi, int sw) {
#pragma unroll
  for (int i = 0; i < FM; i++) f.a[i] = As[(arow + i * 32) * 4 + ((2 * ks + hi) ^ sw)];
#pragma unroll
  for (int j = 0; j < FN; j++) f.b[j] = Bs[(brow + j * 32) * 4 + ((2 * ks + hi) ^ sw)];
}

template <int FM, int FN>
__device__ __forceinline__ void mma_frags(f32x16_t (&acc)[FM][FN], const Frags<FM, FN>& f) {
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++)
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, f.a[i]),
                                                          __builtin_bit_cast(bf16x8_t, f.b[j]), acc[i][j], 0, 0, 0);
}

// single-fragment and single-MFMA forms of the above, for interleaved issue
template <int FM, int FN>
__device__ __forceinline__ void load_frag(Frags<FM, FN>& f, int idx, const u32x4_t* As, const u32x4_t* Bs, int arow,
                                          int brow, int ks, int hi, int sw) {
  if (idx < FM) f.a[idx] = As[(arow + idx * 32) * 4 + ((2 * ks + hi) ^ sw)];
  else f.b[idx - FM] = Bs[(brow + (idx - FM) * 32) * 4 + ((2 * ks + hi) ^ sw)];
}

template <int FM, int FN>
__device__ __forceinline__ void mma_one(f32x16_t (&acc)[FM][FN], const Frags<FM, FN>& f, int t) {
  const int i = t / FN, j = t % FN;
  acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, f.a[i]), __builtin_bit_cast(bf16x8_t, f.b[j]),
                                                      acc[i][j], 0, 0, 0);
}

// s_waitcnt vmcnt(n) lgkmcnt(0): all but this wave's n most recent vector-memory instructions
// (here: DMA fills) have completed, and so have all of its LDS reads.  Placed before each barrier:
// after it, no wave has an LDS read of an older stage in flight.
#define LAYA_WAIT_VMCNT(n) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(n) : "memory")

template <int BM, int BN, int WM, int WN, int EPI, int ACT>
__global__ __launch_bounds__(256, 1) void k_gemm_xl(const GemmArgs a) {
  using T = bf16_t;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 32, FN = WTN / 32;
  constexpr int PER_SLICE = BM / 64 + BN / 64;         // DMA instructions per thread per K slice
  static_assert(WM * WN == 4 && WTM % 32 == 0 && WTN % 32 == 0, "tile");
  // the epilogue stages each wave's output in one whole stage ((BM + BN) * 64 bytes)
  static_assert(WTM * (EPI == EPI_GEGLU ? WTN / 2 : WTN) * 2 <= (BM + BN) * 64 && 32 * 64 * 4 <= (BM + BN) * 64,
                "epilogue staging");
  // five 32-deep K stages ((BM + BN) * 64 bytes each), separate objects so the compiler sees that
  // the DMA into one stage and the fragment reads of another never alias
  struct Stage { u32x4_t a[BM * 4]; u32x4_t b[BN * 4]; };
  __shared__ Stage S0, S1, S2, S3, S4;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN, l32 = lane & 31, hi = lane >> 5;
  const int tilesN = (a.N + BN - 1) / BN, tilesM = (a.M + BM - 1) / BM;
  int tm, tn;
  tile_coords(blockIdx.x, tilesM, tilesN, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;

  const u32x4_t rA = make_rsrc(a.A, (uint32_t)((size_t)a.M * a.lda * sizeof(T)));
  const u32x4_t rB = make_rsrc(a.W, (uint32_t)((size_t)a.N * a.ldw * sizeof(T)));
  const int lda_b = a.lda * (int)sizeof(T), ldw_b = a.ldw * (int)sizeof(T);

  const int arow = wm * WTM + l32, brow = wn * WTN + l32;
  const int nk = a.K / 32;
  const int sw = ((lane >> 1) & 3) ^ ((lane >> 3) & 1);   // f(row) of fragment rows 32 n + lane % 32
  constexpr int PA = BM / 64, PB = BN / 64;             // DMA instructions per wave and slice
  // per-lane offsets of this wave's DMA instructions (fixed over K) and their LDS destinations
  uint32_t voff[PA + PB];
#pragma unroll
  for (int o = 0; o < PA + PB; o++)
    voff[o] = o < PA ? dma_voff(m0, (wave * PA + o) * 16 + (lane >> 2), lda_b, lane)
                     : dma_voff(n0, (wave * PB + o - PA) * 16 + (lane >> 2), ldw_b, lane);
  const uint32_t wsa = (uint32_t)__builtin_amdgcn_readfirstlane(wave) * (uint32_t)(PA * 1024);
  const uint32_t wsb = (uint32_t)__builtin_amdgcn_readfirstlane(wave) * (uint32_t)(PB * 1024);
  const u32x4_t rNone = make_rsrc(a.A, 0u);               // zero length: every offset out of range
  // instruction o (A rows first, then W rows) of slice kt into stage S
  auto dma_op = [&](int o, Stage& S, int kt) {
    const bool live = kt < nk;
    if (o < PA) dma16(live ? rA : rNone, lds_addr(S.a) + wsa + o * 1024, voff[o], (uint32_t)kt * 64u);
    else dma16(live ? rB : rNone, lds_addr(S.b) + wsb + (o - PA) * 1024, voff[o], (uint32_t)kt * 64u);
  };
  auto dma = [&](int kt, Stage& S) {
#pragma unroll
    for (int o = 0; o < PA + PB; o++) dma_op(o, S, kt);
  };
  // Pipeline: slice s is fetched into stage s % 5 four steps ahead.  Step kt multiplies the two
  // 16-deep halves of slice kt from registers (F0, F1) while loading the next half: F1 (slice kt,
  // second half) during the first, F0 (slice kt + 1, first half) during the second.  Between the
  // halves each wave waits for its own part of slice kt + 1 (two later slices may stay in flight),
  // then the barrier makes slice kt + 1 visible to all waves and frees stage (kt - 1) % 5, whose
  // last reads (F1 of slice kt - 1) were consumed before every wave reached this point; the refill
  // of that stage with slice kt + 4 is issued right after it.  Every step issues the same number of
  // DMA instructions (past the last slice they are out of range), so the wait count is constant.
  // The loop body starts after a step's barrier: (refill, F0 <- next slice, F1 MFMAs) | (F1 <- next
  // slice, F0 MFMAs, wait, barrier).
  dma(0, S0);
  dma(1, S1);
  dma(2, S2);
  dma(3, S3);

  f32x16_t acc[FM][FN];
  if constexpr (EPI == EPI_RESID) {
    // the residual update X += A W^T + b starts the accumulators at X (rows/cols outside X read 0),
    // so the epilogue issues no global load after its first store.  These loads come after the
    // DMA fills, so the wait for them (before the first MFMA) also covers the prologue slices.
    const __amdgpu_buffer_rsrc_t rX = __builtin_amdgcn_make_buffer_rsrc(
        a.X, (short)0, (int)((size_t)a.M * a.ldx * sizeof(float)), 0x00020000);
    const int r0 = m0 + wm * WTM + 4 * hi, c0 = n0 + wn * WTN + l32;
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int j = 0; j < FN; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const int row = r0 + i * 32 + 8 * (e >> 2) + (e & 3), col = c0 + j * 32;
          const int off = col < a.N ? (row * a.ldx + col) * 4 : 0x7FFFFFF0;
          acc[i][j][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rX, off, 0, 0));
        }
  } else {
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int j = 0; j < FN; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;
  }

  Frags<FM, FN> F0, F1;
  LAYA_WAIT_VMCNT(3 * PER_SLICE);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  load_frags(F0, S0.a, S0.b, arow, brow, 0, hi, sw);
  load_frags(F1, S0.a, S0.b, arow, brow, 1, hi, sw);
  mma_frags(acc, F0);
  LAYA_WAIT_VMCNT(2 * PER_SLICE);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  // one step from the barrier of step kt - 1 to that of step kt: refill stage SR with slice
  // kt + 3, F0 <- slice kt (SN) first half, MFMAs of F1 (slice kt - 1, second half), F1 <- slice kt
  // second half, MFMAs of F0, wait for slice kt + 1, barrier.
// With one or two waves per SIMD the MFMA pipe idles whenever a wave issues anything else, so the
// DMA instructions and the fragment loads of the next half are spread between the MFMAs of the
// current one (first half: DMA then F0 loads; second half: F1 loads), each MFMA followed by its
// share, fixed by scheduling fences.
  constexpr int NMM = FM * FN, E1 = PA + PB + FM + FN, E2 = FM + FN;
#define LAYA_GEMM_STEP(SN, SR)                                                            \
  {                                                                                       \
    _Pragma("unroll") for (int t = 0; t < NMM; t++) {                                     \
      mma_one(acc, F1, t);                                                                \
      _Pragma("unroll") for (int o = t * E1 / NMM; o < (t + 1) * E1 / NMM; o++) {        \
        if (o < PA + PB) dma_op(o, SR, kt + 4);                                           \
        else load_frag(F0, o - PA - PB, SN.a, SN.b, arow, brow, 0, hi, sw);               \
      }                                                                                   \
      __builtin_amdgcn_sched_barrier(0);                                                  \
    }                                                                                     \
    ++kt;                                                                                 \
    _Pragma("unroll") for (int t = 0; t < NMM; t++) {                                     \
      mma_one(acc, F0, t);                                                                \
      _Pragma("unroll") for (int o = t * E2 / NMM; o < (t + 1) * E2 / NMM; o++)          \
        load_frag(F1, o, SN.a, SN.b, arow, brow, 1, hi, sw);                              \
      __builtin_amdgcn_sched_barrier(0);                                                  \
    }                                                                                     \
    LAYA_WAIT_VMCNT(2 * PER_SLICE);                                                       \
    __builtin_amdgcn_s_barrier();                                                         \
    asm volatile("" ::: "memory");                                                        \
  }
  int kt = 0;                              // slice whose first half has been multiplied
  for (; kt + 6 <= nk;) {                  // five whole steps, the last one loading slice kt + 5
    LAYA_GEMM_STEP(S1, S4)
    LAYA_GEMM_STEP(S2, S0)
    LAYA_GEMM_STEP(S3, S1)
    LAYA_GEMM_STEP(S4, S2)
    LAYA_GEMM_STEP(S0, S3)
  }
  if (kt + 1 < nk) {                       // at most four whole steps remain
    LAYA_GEMM_STEP(S1, S4)
    if (kt + 1 < nk) {
      LAYA_GEMM_STEP(S2, S0)
      if (kt + 1 < nk) {
        LAYA_GEMM_STEP(S3, S1)
        if (kt + 1 < nk) LAYA_GEMM_STEP(S4, S2)
      }
    }
  }
  mma_frags(acc, F1);                      // second half of the last slice
#undef LAYA_GEMM_STEP
  LAYA_WAIT_VMCNT(0);                      // the out-of-range refills of the last steps

  // ---------------- epilogue ----------------
  // On gfx9 vmcnt counts stores as well as loads, so a global load issued after a store waits for
  // that store.  The epilogue therefore loads everything it needs (bias, positions, RoPE tables)
  // before its first store: residual updates started their accumulators at X above and only add
  // a preloaded bias; the other epilogues finish every value of the wave's tile into LDS first
  // (bf16, the K stages are idle) and then stream it out as 16-byte row segments.
  __syncthreads();
  const int rbase = m0 + wm * WTM, cbase = n0 + wn * WTN;
  auto pack8 = [](float4 x, float4 y) {
    u32x4_t u;
    u[0] = (uint32_t)f2bf(x.x) | ((uint32_t)f2bf(x.y) << 16);
    u[1] = (uint32_t)f2bf(x.z) | ((uint32_t)f2bf(x.w) << 16);
    u[2] = (uint32_t)f2bf(y.x) | ((uint32_t)f2bf(y.y) << 16);
    u[3] = (uint32_t)f2bf(y.z) | ((uint32_t)f2bf(y.w) << 16);
    return u;
  };
  if constexpr (EPI == EPI_RESID) {
    // per 32 x 64 block through an fp32 scratch of 8 KiB per wave; no loads in the loop
    float* scr = reinterpret_cast<float*>(wave == 0 ? &S0 : wave == 1 ? &S1 : wave == 2 ? &S2 : &S3);
    auto sidx = [](int r, int c) { return r * 64 + ((((c >> 2) ^ (r & 15))) << 2) + (c & 3); };
    float bias[FN];
#pragma unroll
    for (int j = 0; j < FN; j++) {
      const int col = cbase + j * 32 + l32;
      bias[j] = (a.bias && col < a.N) ? a.bias[col] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < FM; i++) {
#pragma unroll
      for (int jp = 0; jp < FN; jp += 2) {
        const int row0 = rbase + i * 32, c0 = cbase + jp * 32;
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
          for (int e = 0; e < 16; e++) scr[sidx(8 * (e >> 2) + 4 * hi + (e & 3), 32 * b + l32)] = acc[i][jp + b][e] + bias[jp + b];
        __builtin_amdgcn_s_waitcnt(0xC07F);                 // lgkmcnt(0): this wave's LDS writes are done
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int it = 0; it < 8; it++) {
          const int item = lane + 64 * it, r = item >> 4, q = item & 15;
          const int row = row0 + r, col = c0 + 4 * q;
          if (row < a.M && col < a.N)
            *reinterpret_cast<float4*>(a.X + (size_t)row * a.ldx + col) =
                *reinterpret_cast<const float4*>(scr + r * 64 + ((q ^ (r & 15)) << 2));
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
      }
    }
  } else {
    // phase 1: the wave's finished tile -> LDS as bf16, [WTM][OW] with 16-byte chunks swizzled by row
    constexpr int OW = EPI == EPI_GEGLU ? WTN / 2 : WTN;     // output columns of the wave tile
    constexpr int CPRW = OW / 8;                             // 16-byte chunks per row
    bf16_t* wt = reinterpret_cast<bf16_t*>(wave == 0 ? &S0 : wave == 1 ? &S1 : wave == 2 ? &S2 : &S3);
    auto oidx = [](int r, int c) { return r * OW + ((((c >> 3) ^ (r & 7)) & (CPRW - 1)) << 3) + (c & 7); };
    const bool odd = lane & 1;
    // element e of a 32x32 block is row 8*(e/4) + 4*hi + e%4: elements (e, e+1), e even, are rows
    // (r, r+1) of column l32; after the pair swap this lane writes 4 bytes at (r + odd, l32 & ~1)
    auto put = [&](int i, int e, int cblk, float ve, float ve1) {
      const int r = i * 32 + 8 * (e >> 2) + 4 * hi + (e & 3) + (odd ? 1 : 0);
      *reinterpret_cast<uint32_t*>(wt + oidx(r, cblk + (l32 & ~1))) = pair_rows_to_cols(ve, ve1, odd);
    };
    const int D = a.H * a.HD;
#pragma unroll
    for (int i = 0; i < FM; i++) {
#pragma unroll
      for (int jp = 0; jp < FN; jp += 2) {
        const int c0 = cbase + jp * 32;
        if constexpr (EPI == EPI_GEGLU) {
          const bool ok = c0 < a.N;
          const float bx = (a.bias && ok) ? a.bias[c0 + l32] : 0.f, by = (a.bias && ok) ? a.bias[c0 + 32 + l32] : 0.f;
#pragma unroll
          for (int e = 0; e < 16; e += 2)
            put(i, e, jp * 16, gelu_erf_as(acc[i][jp][e] + bx) * (acc[i][jp + 1][e] + by),
                gelu_erf_as(acc[i][jp][e + 1] + bx) * (acc[i][jp + 1][e + 1] + by));
        } else if constexpr (EPI == EPI_QKV) {
          const bool ok = c0 < a.N;
          const float b0 = (a.bias && ok) ? a.bias[c0 + l32] : 0.f, b1 = (a.bias && ok) ? a.bias[c0 + 32 + l32] : 0.f;
          if (a.rope_cos && c0 < 2 * D) {
#pragma unroll
            for (int e = 0; e < 16; e += 2) {
              float o1[2], o2[2];
#pragma unroll
              for (int u = 0; u < 2; u++) {
                const int r = i * 32 + 8 * ((e + u) >> 2) + 4 * hi + ((e + u) & 3);
                const int p = a.pos[min(rbase + r, a.M - 1)];
                const float c = a.rope_cos[p * 32 + l32], sn = a.rope_sin[p * 32 + l32];
                const float x1 = acc[i][jp][e + u] + b0, x2 = acc[i][jp + 1][e + u] + b1;
                o1[u] = x1 * c - x2 * sn;
                o2[u] = x2 * c + x1 * sn;
              }
              put(i, e, jp * 32, o1[0], o1[1]);
              put(i, e, jp * 32 + 32, o2[0], o2[1]);
            }
          } else {
#pragma unroll
            for (int e = 0; e < 16; e += 2) {
              put(i, e, jp * 32, acc[i][jp][e] + b0, acc[i][jp][e + 1] + b0);
              put(i, e, jp * 32 + 32, acc[i][jp + 1][e] + b1, acc[i][jp + 1][e + 1] + b1);
            }
          }
        } else {  // EPI_STORE
#pragma unroll
          for (int b = 0; b < 2; b++) {
            const int col = c0 + 32 * b + l32;
            const float bb = (a.bias && col < a.N) ? a.bias[col] : 0.f;
            auto f = [&](float v) {
              v += bb;
              if constexpr (ACT == ACT_RELU) v = fmaxf(v, 0.f);
              if constexpr (ACT == ACT_GELU) v = gelu_erf_as(v);
              return v;
            };
#pragma unroll
            for (int e = 0; e < 16; e += 2) put(i, e, (jp + b) * 32, f(acc[i][jp + b][e]), f(acc[i][jp + b][e + 1]));
          }
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_wave_barrier();
    // phase 2: stores only
    if constexpr (EPI == EPI_QKV) {
#pragma unroll
      for (int hb = 0; hb < WTN / 64; hb++) {                // one 64-column head block at a time
        const int c0 = cbase + hb * 64;
        if (c0 >= a.N) break;
        const int sec = c0 / D, h = (c0 % D) / a.HD;
        if (sec == 2) {                                      // V^T: 8 consecutive rows of one column
          T* vt = reinterpret_cast<T*>(a.Vt) + (size_t)h * a.HD * a.ldv;
#pragma unroll
          for (int it = 0; it < WTM / 8; it++) {
            const int item = lane + 64 * it, c = item >> (WTM == 128 ? 4 : 3), rg = item & (WTM / 8 - 1);
            const int row = rbase + 8 * rg;
            if (row >= a.M) continue;
            uint32_t u[4];
#pragma unroll
            for (int t = 0; t < 4; t++)
              u[t] = (uint32_t)wt[oidx(8 * rg + 2 * t, hb * 64 + c)] | ((uint32_t)wt[oidx(8 * rg + 2 * t + 1, hb * 64 + c)] << 16);
            T* dst = vt + (size_t)c * a.ldv + row;
            if (row + 7 < a.M) {
              *reinterpret_cast<u32x4_t*>(dst) = (u32x4_t){u[0], u[1], u[2], u[3]};
            } else {
              for (int t = 0; t < 8 && row + t < a.M; t++) dst[t] = (bf16_t)(u[t >> 1] >> (16 * (t & 1)));
            }
          }
        } else {
          T* base = reinterpret_cast<T*>(sec == 0 ? a.Q : a.Kt) + h * a.HD;
#pragma unroll
          for (int it = 0; it < WTM / 8; it++) {
            const int item = lane + 64 * it, r = item >> 3, q = item & 7;
            const int row = rbase + r;
            if (row < a.M)
              *reinterpret_cast<u32x4_t*>(base + (size_t)row * a.ldqk + 8 * q) =
                  *reinterpret_cast<const u32x4_t*>(wt + oidx(r, hb * 64 + 8 * q));
          }
        }
      }
    } else {
      const int ocol0 = EPI == EPI_GEGLU ? cbase / 2 : cbase;
      const int ncols = EPI == EPI_GEGLU ? a.N / 2 : a.N;
#pragma unroll
      for (int it = 0; it < WTM * CPRW / 64; it++) {
        const int item = lane + 64 * it, r = item / CPRW, q = item % CPRW;
        const int row = rbase + r, col = ocol0 + 8 * q;
        if (row < a.M && col < ncols)
          *reinterpret_cast<u32x4_t*>(reinterpret_cast<T*>(a.C) + (size_t)row * a.ldc + col) =
              *reinterpret_cast<const u32x4_t*>(wt + oidx(r, 8 * q));
      }
    }
  }
}

template <int BM, int BN, int WM, int WN>
static void launch_xl(int epi, const GemmArgs& a, hipStream_t st) {
  const int tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  if (epi == EPI_STORE) {
    if (a.act == ACT_RELU) hipLaunchKernelGGL((k_gemm_xl<BM, BN, WM, WN, EPI_STORE, ACT_RELU>), dim3(tiles), dim3(256), 0, st, a);
    else if (a.act == ACT_GELU) hipLaunchKernelGGL((k_gemm_xl<BM, BN, WM, WN, EPI_STORE, ACT_GELU>), dim3(tiles), dim3(256), 0, st, a);
    else hipLaunchKernelGGL((k_gemm_xl<BM, BN, WM, WN, EPI_STORE, ACT_NONE>), dim3(tiles), dim3(256), 0, st, a);
    return;
  }
  switch (epi) {
    case EPI_RESID: hipLaunchKernelGGL((k_gemm_xl<BM, BN, WM, WN, EPI_RESID, ACT_NONE>), dim3(tiles), dim3(256), 0, st, a); break;
    case EPI_QKV: hipLaunchKernelGGL((k_gemm_xl<BM, BN, WM, WN, EPI_QKV, ACT_NONE>), dim3(tiles), dim3(256), 0, st, a); break;
    case EPI_GEGLU: hipLaunchKernelGGL((k_gemm_xl<BM, BN, WM, WN, EPI_GEGLU, ACT_NONE>), dim3(tiles), dim3(256), 0, st, a); break;
    default: fprintf(stderr, "[laya] gemm: bad epilogue %d\n", epi); exit(1);
  }
}

// Tile configurations for the bf16 path and the planner that picks one per GEMM: estimated time
// = rounds of concurrently resident tiles x per-tile cost, with the per-CU throughput of each
// shape relative to 256x256.  Measured on MI355X at the ModernBERT-large shapes: two resident
// 128x128 workgroups per CU (64 KiB of LDS each) beat one 256x256 workgroup by ~1.4x, because
// one workgroup's epilogue (LDS staging, GELU/RoPE math, output stores) overlaps the other's
// MFMA main loop, while a lone 256x256 workgroup leaves the MFMA pipe idle during its epilogue.
struct XlCfg { int bm, bn, per_cu; float rel; };
static const XlCfg kXl[] = {{256, 256, 1, 1.00f}, {256, 128, 1, 0.90f}, {128, 256, 1, 0.90f}, {128, 128, 2, 1.40f}};

int gemm_pick(int M, int N, int /*epi*/) {
  int best = -1;
  double bt = 1e300;
  for (int i = 0; i < (int)(sizeof(kXl) / sizeof(kXl[0])); i++) {
    const XlCfg& c = kXl[i];
    const double tiles = (double)((M + c.bm - 1) / c.bm) * ((N + c.bn - 1) / c.bn);
    const double slots = 256.0 * c.per_cu;
    const double t = std::ceil(tiles / slots) * (double)c.bm * c.bn * c.per_cu / c.rel;
    if (t < bt * 0.999) { bt = t; best = i; }
  }
  return best;
}

bool gemm_shape_ok(int epi, const GemmArgs& a, int elt_bytes, const char** why) {
  const int bk = 128 / elt_bytes, align = 16 / elt_bytes;
  if (a.M <= 0 || a.N <= 0) { *why = "empty"; return false; }
  if (a.K <= 0 || a.K % bk) { *why = "K must be a positive multiple of the 128-byte K slice"; return false; }
  if (a.lda % align || a.ldw % align || a.lda < a.K || a.ldw < a.K) { *why = "row strides must be 16-byte multiples >= K"; return false; }
  if ((reinterpret_cast<uintptr_t>(a.A) | reinterpret_cast<uintptr_t>(a.W)) & 15) { *why = "operands must be 16-byte aligned"; return false; }
  if (epi == EPI_GEGLU && a.N % 64) { *why = "GeGLU needs N % 64 == 0"; return false; }
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
  if constexpr (sizeof(T) == 2) {
    const size_t abytes = (size_t)a.M * a.lda * sizeof(T), wbytes = (size_t)a.N * a.ldw * sizeof(T);
    // 16-byte epilogue stores need N, the row strides and the output bases in multiples of 8 elements
    const bool aligned = a.N % 8 == 0 && ((epi == EPI_STORE || epi == EPI_GEGLU) ? a.ldc % 8 == 0 : true) &&
                         (epi == EPI_RESID ? a.ldx % 4 == 0 : true) && (epi == EPI_QKV ? a.ldqk % 8 == 0 && a.ldv % 8 == 0 : true);
    const bool xl_ok = aligned && abytes < (1u << 31) - 65536 && wbytes < (1u << 31) - 65536;
    if (xl_ok) {
      // LAYA_GEMM_CFG=0..3 pins one tile configuration (256x256, 256x128, 128x256, 128x128)
      static const int forced = getenv("LAYA_GEMM_CFG") ? atoi(getenv("LAYA_GEMM_CFG")) : -1;
      switch (forced >= 0 && forced < 4 ? forced : gemm_pick(a.M, a.N, epi)) {
        case 0: launch_xl<256, 256, 2, 2>(epi, a, st); return;
        case 1: launch_xl<256, 128, 2, 2>(epi, a, st); return;
        case 2: launch_xl<128, 256, 2, 2>(epi, a, st); return;
        default: launch_xl<128, 128, 2, 2>(epi, a, st); return;
      }
    }
  }
  launch_cfg<T, 128, 128, 2, 2>(epi, a, st);
}

template void launch_gemm<float>(int, const GemmArgs&, hipStream_t);
template void launch_gemm<bf16_t>(int, const GemmArgs&, hipStream_t);

}  // namespace laya
