// MFMA GEMMs for gfx950: C[M,N] = A[M,K] . W[N,K]^T with fused epilogues.
//
// Both operands are K-contiguous (activations [rows, K], weights in their checkpoint [out, in]
// layout), which is the layout the MFMA operand registers want: a lane holds 8 consecutive K values
// of one row of each operand, so every fragment is one 16-byte LDS read and no weight is ever
// transposed.  Two kernels:
//
//   k_gemm_xl  bf16, the engine's path.  256-thread workgroups, tiles from 128x128 to 256x256 on
//              v_mfma_f32_32x32x16_bf16; K advances in 64-deep stages (whole 128-byte lines of
//              every tile row), filled ahead by LDS DMA (buffer_load ... lds): two stage buffers,
//              or for 128x128 tiles three A buffers (two workgroups per CU) or four stage buffers
//              (grids of at most one tile per CU).  The product is computed
//              transposed so each lane holds four consecutive output columns; the epilogue is
//              staged through LDS and leaves as full-line 16-byte stores.  The engine picks the
//              tile shape (and an optional row split over two launches) per GEMM by timing.
//   k_gemm     fp32 operands, and bf16 shapes the tiled kernel cannot take (unaligned N or
//              strides).  128x128, 64x64 or 32x64 tiles by how many fill the chip, K in 128-byte
//              slices through double-buffered LDS with register prefetch,
//              v_mfma_f32_16x16x4_f32 / v_mfma_f32_16x16x32_bf16.
//
// Both remap workgroup ids so each of the 8 XCDs (own L2) walks a contiguous run of tiles.
//
// Epilogues:
//   EPI_STORE  C = act(acc + bias)                        (storage type)
//   EPI_RESID  X += acc + bias (fp32 residual stream), rounded as X + (acc + bias) in k_gemm and as
//              (acc + X) + bias in k_gemm_xl
//   EPI_QKV    q,k (RoPE when tables are given) -> Q, K [rows][H*HD]; v -> V^T [H*HD][ldv] at
//              column = row.  A wave's column range covers whole 64-wide heads, so the
//              rotate_half partners (d, d+32) of a row sit in the same lane.
//   EPI_GEGLU  W rows stored as alternating 32-row blocks of input and gate rows; writes
//              gelu_erf(input) * gate into C [rows][N/2].
#include <cmath>

#include "kernels.h"

#include <atomic>
#include <type_traits>

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
  // accumulator element i of lane l in a 16x16 block is row 4 (l / 16) + i, column l % 16
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
    case EPI_STORE: LAYA_LAUNCH((k_gemm<T, BM, BN, WM, WN, EPI_STORE>), dim3(tiles), dim3(256), 0, st, a); break;
    case EPI_RESID: LAYA_LAUNCH((k_gemm<T, BM, BN, WM, WN, EPI_RESID>), dim3(tiles), dim3(256), 0, st, a); break;
    case EPI_QKV: LAYA_LAUNCH((k_gemm<T, BM, BN, WM, WN, EPI_QKV>), dim3(tiles), dim3(256), 0, st, a); break;
    case EPI_GEGLU: LAYA_LAUNCH((k_gemm<T, BM, BN, WM, WN, EPI_GEGLU>), dim3(tiles), dim3(256), 0, st, a); break;
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
// BM x BN tile (256x256 by default, one workgroup per CU, 128 KiB of LDS for two K stages and
// 32 KiB for the epilogue's staging);
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

// widest power-of-two column count <= cap that divides w
constexpr int xl_fitw(int w, int cap) { int c = w & -w; while (c > cap) c /= 2; return c; }

// ---- optional per-tile timeline (built only with -DLAYA_TILE_TRACE: liblaya_trace.so) ----
// Thread 0 of every workgroup of k_gemm_xl records, at its exit: its start and end on the 100 MHz
// real-time clock, its prologue, K loop and epilogue in shader-clock cycles, the cycles wave 0 spent
// in the K loop's stage waits and barriers (two-buffer loop only), and its hardware id.  One record
// of 8 words per workgroup, at index blockIdx.x, in a device array read back by
// laya_tile_trace_read (tile_trace.h).
#ifdef LAYA_TILE_TRACE
constexpr int kTileTraceMax = 65536;
__device__ unsigned long long g_tile_trace[8 * kTileTraceMax];
struct TileTrace {
  unsigned long long t0, t1, t2, r0, w;
  __device__ void start() {
    t0 = __builtin_amdgcn_s_memtime();
    r0 = __builtin_amdgcn_s_memrealtime();
    t1 = t2 = t0;
    w = 0;
  }
  __device__ ~TileTrace() {
    if (threadIdx.x != 0 || blockIdx.x >= (unsigned)kTileTraceMax) return;
    const unsigned long long t3 = __builtin_amdgcn_s_memtime(), r3 = __builtin_amdgcn_s_memrealtime();
    unsigned hw, xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    unsigned long long* p = g_tile_trace + 8 * (size_t)blockIdx.x;
    p[0] = r0; p[1] = r3; p[2] = t1 - t0; p[3] = t2 - t1; p[4] = t3 - t2; p[5] = w;
    p[6] = ((unsigned long long)xcc << 32) | hw; p[7] = t3 - t0;
  }
};
#define LAYA_TT_MARK(field) do { if (threadIdx.x == 0) tt.field = __builtin_amdgcn_s_memtime(); } while (0)
#define LAYA_TT_WAIT_BEGIN const unsigned long long tt_w0_ = __builtin_amdgcn_s_memtime();
#define LAYA_TT_WAIT_END                                                                          \
  { const unsigned long long tt_w1_ = __builtin_amdgcn_s_memtime(); __builtin_amdgcn_s_waitcnt(0xC07F); tw += tt_w1_ - tt_w0_; }
#else
#define LAYA_TT_MARK(field) do { } while (0)
#define LAYA_TT_WAIT_BEGIN
#define LAYA_TT_WAIT_END
#endif

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
// Issued as inline assembly, so the compiler sees no LDS write and inserts no waits of its own
// between these fills and the fragment reads: the main loop orders them with explicit vmcnt waits
// and barriers.  The LDS base is an operand bound to M0 ("{m0}"), so the compiler writes M0 itself
// and knows the instruction reads it; the asm adds one wait state between that write and the DMA.
// The memory clobber keeps the compiler from moving LDS reads across the fill.
__device__ __forceinline__ void dma16(u32x4_t rsrc, uint32_t lds, uint32_t voff, uint32_t soff) {
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "{m0}"(lds), "v"(voff), "s"(rsrc), "s"(soff)
               : "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Fragments of one 16-deep K sub-step: lane l holds 8 consecutive K values (16 bytes) of tile row
// (row base + 32 i + l % 32), K offset 8 * (l / 32).
template <int FM, int FN>
struct Frags {
  u32x4_t a[FM], b[FN];
};

// s_waitcnt vmcnt(n) lgkmcnt(0): all but this wave's n most recent vector-memory instructions
// (here: DMA fills) have completed, and so have all of its LDS reads.  Placed before each barrier:
// after it, no wave has an LDS read of an older stage in flight.
#define LAYA_WAIT_VMCNT(n) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(n) : "memory")

// acc[i][j] += A block i . W block j^T (SWAP: the transposed product W block j . A block i^T,
// whose accumulator layout gives each lane 4 consecutive output columns of one row)
template <bool SWAP, int FM, int FN>
__device__ __forceinline__ void mma_one_x(f32x16_t (&acc)[FM][FN], const Frags<FM, FN>& f, int t) {
  const int i = t / FN, j = t % FN;
  if constexpr (SWAP)
    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, f.b[j]),
                                                        __builtin_bit_cast(bf16x8_t, f.a[i]), acc[i][j], 0, 0, 0);
  else
    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, f.a[i]),
                                                        __builtin_bit_cast(bf16x8_t, f.b[j]), acc[i][j], 0, 0, 0);
}

// ---- 64-deep stages: one whole 128-byte line of every tile row per stage ----
// A 32-deep K slice would use 64 bytes of each 128-byte line, and the other half of the line (the
// next slice) is no longer in the CU's 32 KB L1 when it is asked for, so each half line would cost
// a whole-line L2 request.  A stage of 64 K values per row fetches each line once.
//
// Stage rows are 128 bytes (8 chunks of 16 bytes); the chunk at slot c of row r holds logical chunk
// c ^ g(r), g(r) = (r & 7) ^ ((r >> 3) & 1).  A fragment read has lane l on row l % 32 at one
// logical chunk: a group of 16 lanes (rows r0..r0+15) covers 16 distinct 16-byte positions of the
// 256 bytes that 64 banks span (even and odd rows each see 8 distinct g), and a group of 8 covers
// the 8 positions of 32 banks, so the reads are conflict-free.  One DMA instruction fills 8 rows:
// lane l writes row 8 q + l / 8 (q = instruction index within the stage part), slot l % 8.
__device__ __forceinline__ uint32_t dma64_voff(int row0, int r8, int ld_bytes, int lane, int odd) {
  const int rl = lane >> 3;
  return (uint32_t)(row0 + r8 + rl) * (uint32_t)ld_bytes + ((uint32_t)((lane & 7) ^ rl ^ odd) << 4);
}

// RoPE table rows in LDS (128 bytes: 32 floats, of cos or of sin): 16-byte chunk c of row r sits in
// slot c ^ rope_sw(r).  The epilogue's reads (lanes on 16 consecutive rows, one chunk each) then
// cover 16 distinct 16-byte bank positions; unswizzled, the 128-byte row stride put eight of them
// on the same banks.
__device__ __forceinline__ int rope_sw(int r) { return (r >> 1) & 7; }

// DMA plan of one workgroup for 64-deep stages: PA + PB instructions per wave and stage.  The
// per-lane offset depends only on the parity of the instruction index (the swizzle's row term);
// the instruction's row step and the stage's K offset go in the scalar offset.
template <int PA, int PB>
struct XlDma64 {
  u32x4_t rA, rB, rNone;
  uint32_t va[2], vb[2];
  uint32_t wsa, wsb;
  int lda8, ldw8;   // bytes of 8 rows
  int ns;           // 32-deep slices (even: whole 64-deep stages)
  // instruction o of the A (W) part of stage g, into the buffer at LDS byte address la (lb)
  __device__ __forceinline__ void op_a(int o, uint32_t la, int g) const {
    dma16(2 * g < ns ? rA : rNone, la + wsa + o * 1024, va[o & 1], (uint32_t)g * 128u + (uint32_t)(o * lda8));
  }
  __device__ __forceinline__ void op_b(int o, uint32_t lb, int g) const {
    dma16(2 * g < ns ? rB : rNone, lb + wsb + o * 1024, vb[o & 1], (uint32_t)g * 128u + (uint32_t)(o * ldw8));
  }
};

// f(integral_constant<int, I>) for I = B .. E - 1, in order
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// fragment idx (A blocks, then W blocks) of 16-deep sub-step s of a 64-deep stage
template <int FM, int FN>
__device__ __forceinline__ void load_frag64(Frags<FM, FN>& f, int idx, const u32x4_t* As, const u32x4_t* Bs, int arow,
                                            int brow, int s, int hi, int sw) {
  if (idx < FM) f.a[idx] = As[(arow + idx * 32) * 8 + ((2 * s + hi) ^ sw)];
  else f.b[idx - FM] = Bs[(brow + (idx - FM) * 32) * 8 + ((2 * s + hi) ^ sw)];
}

// The K loop over 64-deep stages in two LDS buffers (one workgroup per CU: a stage's MFMAs cover
// the fill of the next one).  Stage 0 and the A part of stage 1 were issued by the caller.
// Stage g runs four 16-deep sub-steps, each multiplying one register set while the other is
// loaded with the next sub-step's fragments.  After the third sub-step's
// fragment loads every wave has all of stage g in registers; one wait and one barrier then publish
// stage g + 1 and free stage g's buffer.  The A part of stage g + 2 goes into that buffer between
// the fourth sub-step's MFMAs, together with the loads of stage g + 1's first fragments; its W part
// follows between the MFMAs of stage g + 1's first sub-step.  Issuing a stage's fills in two
// bursts instead of one keeps the texture address unit's command queue from filling (a wave that
// cannot issue its fill cannot issue its next MFMA either): 5-8% faster K loops.  A burst spread
// over three sub-steps leaves the last part too little time to land before the wait.  Every stage
// but the last issues the same DMA instructions (past the last stage they read nothing), so the
// wait is a constant vmcnt(0).  K is a multiple of 64 (every stage is whole).
// XP > 0: the first XP stages each also issue piece p of the caller's loads (xl(p), XS vector-memory
// instructions, e.g. the residual GEMM's x), after the W part of their next stage.  Their wait then
// leaves those XS loads in flight, vmcnt(XS), and the next stage's wait covers them, so each piece
// has about a stage and a half to land while the MFMAs run.  Pieces of stages that K does not
// reach are issued after the loop.
// NT > 0: tail() issues NT vector-memory loads of the caller's (the residual epilogue's first X
// block) before the last stage's final three sub-steps; the loop's closing wait leaves them in flight.
template <bool SWAP, int NX, int XP, int XS, int NT, int FM, int FN, int PA, int PB, class ST, class XL, class TL>
__device__ __forceinline__ void xl_k_loop64(f32x16_t (&acc)[FM][FN], ST& T0, ST& T1, const XlDma64<PA, PB>& d, int arow,
                                            int brow, int hi, int sw, XL&& xl, TL&& tail, unsigned long long& tw) {
  (void)tw;                                // cycles in stage waits (tile trace builds only)
  constexpr int NMM = FM * FN, E = FM + FN, EW = PB + FM + FN, EA = PA + FM + FN;
  Frags<FM, FN> F0, F1;
  // stage 0; the A part of stage 1 and NX later fills the caller issued may still be in flight
  LAYA_WAIT_VMCNT(PA + NX);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
#pragma unroll
  for (int o = 0; o < E; o++) load_frag64(F0, o, T0.a, T0.b, arow, brow, 0, hi, sw);
  // MFMAs of register set FX, with the loads of sub-step s of stage SL into FY spread between them
#define LAYA_SUB64(FX, FY, SL, s)                                                         \
  _Pragma("unroll") for (int t = 0; t < NMM; t++) {                                       \
    mma_one_x<SWAP>(acc, FX, t);                                                          \
    _Pragma("unroll") for (int o = t * E / NMM; o < (t + 1) * E / NMM; o++)              \
      load_frag64(FY, o, SL.a, SL.b, arow, brow, s, hi, sw);                              \
    __builtin_amdgcn_sched_barrier(0);                                                    \
  }
  // stage g in buffer C, followed by stage g + 1 in buffer N.  The first sub-step also issues the W
  // part of stage g + 1 (into N, free since the previous stage's barrier) and the fourth the A
  // part of stage g + 2, so a stage's fills leave in two bursts half the size of one.  P >= 0:
  // piece P of the caller's loads follows the W part.
#define LAYA_STAGE64(C, N, P)                                                             \
  {                                                                                       \
    _Pragma("unroll") for (int t = 0; t < NMM; t++) {                                     \
      mma_one_x<SWAP>(acc, F0, t);                                                        \
      _Pragma("unroll") for (int o = t * EW / NMM; o < (t + 1) * EW / NMM; o++) {        \
        if (o < PB) d.op_b(o, lds_addr(N.b), g + 1);                                      \
        else load_frag64(F1, o - PB, C.a, C.b, arow, brow, 1, hi, sw);                    \
      }                                                                                   \
      __builtin_amdgcn_sched_barrier(0);                                                  \
    }                                                                                     \
    if constexpr (P >= 0) {                                                               \
      xl(std::integral_constant<int, P>{});                                               \
      __builtin_amdgcn_sched_barrier(0);                                                  \
    }                                                                                     \
    LAYA_SUB64(F1, F0, C, 2)                                                              \
    LAYA_SUB64(F0, F1, C, 3)                                                              \
    LAYA_TT_WAIT_BEGIN                                                                    \
    if constexpr (P >= 0) LAYA_WAIT_VMCNT(XS);                                            \
    else LAYA_WAIT_VMCNT(0);                                                              \
    __builtin_amdgcn_s_barrier();                                                         \
    asm volatile("" ::: "memory");                                                        \
    LAYA_TT_WAIT_END                                                                      \
    _Pragma("unroll") for (int t = 0; t < NMM; t++) {                                     \
      mma_one_x<SWAP>(acc, F1, t);                                                        \
      _Pragma("unroll") for (int o = t * EA / NMM; o < (t + 1) * EA / NMM; o++) {        \
        if (o < PA) d.op_a(o, lds_addr(C.a), g + 2);                                      \
        else load_frag64(F0, o - PA, N.a, N.b, arow, brow, 0, hi, sw);                    \
      }                                                                                   \
      __builtin_amdgcn_sched_barrier(0);                                                  \
    }                                                                                     \
    ++g;                                                                                  \
  }
  const int nst = d.ns / 2;                // stages
  int g = 0;
  int xdone = 0;                           // pieces issued
  if constexpr (XP > 0) {
    static_for<0, (XP + 1) / 2>([&](auto q) {  // the stages that carry pieces, two at a time
      constexpr int P0 = 2 * decltype(q)::value, P1 = P0 + 1 < XP ? P0 + 1 : -1;
      if (g + 2 < nst) {
        LAYA_STAGE64(T0, T1, P0)
        LAYA_STAGE64(T1, T0, P1)
        xdone = P1 < 0 ? XP : P1 + 1;
      }
    });
  }
  for (; g + 2 < nst;) {                   // two stages, each followed by another
    LAYA_STAGE64(T0, T1, -1)
    LAYA_STAGE64(T1, T0, -1)
  }
  if (g + 2 == nst) LAYA_STAGE64(T0, T1, -1)  // g is even: stage g in T0; the last one is in T1
  ST& L = (g & 1) ? T1 : T0;               // the last stage (g == nst - 1)
  if constexpr (NT > 0) {
    tail();
    __builtin_amdgcn_sched_barrier(0);
  }
  LAYA_SUB64(F0, F1, L, 1)
  LAYA_SUB64(F1, F0, L, 2)
  LAYA_SUB64(F0, F1, L, 3)
#pragma unroll
  for (int t = 0; t < NMM; t++) mma_one_x<SWAP>(acc, F1, t);
#undef LAYA_STAGE64
#undef LAYA_SUB64
  LAYA_WAIT_VMCNT(NT);                     // the refills past the last stage (not the tail's loads)
  if constexpr (XP > 0) {
    static_for<0, XP>([&](auto p) {        // pieces of stages K did not reach
      if (decltype(p)::value >= xdone) xl(p);
    });
  }
}


// The K loop over 64-deep stages for two workgroups per CU, whose interleaved stages take twice
// as long in wall time, so one stage in flight no longer covers a fill.  The A parts of stages
// rotate through three LDS buffers and the W parts through two (A rows miss L2 more often than W
// columns, which every row tile shares), in one array L: A buffer i at L + i * SA, W buffer j at L + 3 SA + j * SW.  The caller issued W 0,
// A 0, W 1, A 1 and A 2, in that order.  Stage g runs four 16-deep sub-steps, each multiplying one
// register set while the other is loaded with the next sub-step's fragments.  After the third
// sub-step's fragment loads every wave has all of stage g in registers; one wait and one barrier
// then publish stage g + 1 and free stage g's buffers, which are refilled between the fourth
// sub-step's MFMAs with W of stage g + 2 and then A of stage g + 3, together with the loads of
// stage g + 1's first fragments.  Loads complete in issue order, so the wait for stage g + 1 lets
// exactly the A part of stage g + 2 stay in flight: vmcnt(PA).  Every stage but the last issues the
// same DMA instructions (past the last stage they read nothing).  K is a multiple of 64.
template <bool SWAP, int FM, int FN, int PA, int PB, int SA, int SW>
__device__ __forceinline__ void xl_k_loop64r(f32x16_t (&acc)[FM][FN], const u32x4_t* L, const XlDma64<PA, PB>& d,
                                             int arow, int brow, int hi, int sw) {
  constexpr int PS = PA + PB, NMM = FM * FN, E = FM + FN, E1 = PS + FM + FN, OB = 3 * SA;
  const uint32_t l0 = lds_addr(L);
  Frags<FM, FN> F0, F1;
  LAYA_WAIT_VMCNT(PB + 2 * PA);            // stage 0 (W 1, A 1 and A 2 may still be in flight)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
#pragma unroll
  for (int o = 0; o < E; o++) load_frag64(F0, o, L, L + OB, arow, brow, 0, hi, sw);
  // MFMAs of register set FX, with the loads of sub-step s of the stage in (CA, CB) into FY spread
  // between them
#define LAYA_SUB64(FX, FY, CA, CB, s)                                                     \
  _Pragma("unroll") for (int t = 0; t < NMM; t++) {                                       \
    mma_one_x<SWAP>(acc, FX, t);                                                          \
    _Pragma("unroll") for (int o = t * E / NMM; o < (t + 1) * E / NMM; o++)              \
      load_frag64(FY, o, CA, CB, arow, brow, s, hi, sw);                                  \
    __builtin_amdgcn_sched_barrier(0);                                                    \
  }
  const int nst = d.ns / 2;                // stages
  int ia = 0, ib = 0;                      // buffers of stage g
  for (int g = 0; g + 1 < nst; g++) {
    const int ia1 = ia == 2 ? 0 : ia + 1, ib1 = ib ^ 1;
    const u32x4_t* CA = L + ia * SA;
    const u32x4_t* CB = L + OB + ib * SW;
    const u32x4_t* NA = L + ia1 * SA;
    const u32x4_t* NB = L + OB + ib1 * SW;
    LAYA_SUB64(F0, F1, CA, CB, 1)
    LAYA_SUB64(F1, F0, CA, CB, 2)
    LAYA_SUB64(F0, F1, CA, CB, 3)
    LAYA_WAIT_VMCNT(PA);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const uint32_t la = l0 + (uint32_t)(ia * SA * 16), lb = l0 + (uint32_t)((OB + ib * SW) * 16);
#pragma unroll
    for (int t = 0; t < NMM; t++) {
      mma_one_x<SWAP>(acc, F1, t);
#pragma unroll
      for (int o = t * E1 / NMM; o < (t + 1) * E1 / NMM; o++) {
        if (o < PB) d.op_b(o, lb, g + 2);
        else if (o < PS) d.op_a(o - PB, la, g + 3);
        else load_frag64(F0, o - PS, NA, NB, arow, brow, 0, hi, sw);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    ia = ia1;
    ib = ib1;
  }
  {                                        // the last stage
    const u32x4_t* CA = L + ia * SA;
    const u32x4_t* CB = L + OB + ib * SW;
    LAYA_SUB64(F0, F1, CA, CB, 1)
    LAYA_SUB64(F1, F0, CA, CB, 2)
    LAYA_SUB64(F0, F1, CA, CB, 3)
  }
#pragma unroll
  for (int t = 0; t < NMM; t++) mma_one_x<SWAP>(acc, F1, t);
#undef LAYA_SUB64
  LAYA_WAIT_VMCNT(0);                      // the refills past the last stage
}

// The K loop for grids of 128x128 tiles that leave CUs without a second workgroup (a few hundred
// rows): NB whole stage buffers, NB - 1 stages issued ahead, so a fill has NB - 2 stages of
// multiplication to land in, not one.  With so few tiles a stage's MFMAs (a quarter of a
// microsecond) are far shorter than a fill's trip to L2 or HBM, and the two-buffer loop waited
// that trip out at every stage.  Stage g lives in buffer g % NB.  Each iteration waits until stage g
// has landed (the NB - 2 later stages may still be in flight: every stage issues the same PA + PB
// DMA instructions, past the last one from a resource without records), passes one barrier (after
// which no wave still reads stage g - 1's buffer) and refills that buffer with stage g + NB - 1:
// the A part between the first sub-step's MFMAs, the W part between the second's.  The K order of
// every accumulator is the one of the other loops, so the bits are too.
template <bool SWAP, int FM, int FN, int PA, int PB, int SA, int SW, int NB>
__device__ __forceinline__ void xl_k_loop64d(f32x16_t (&acc)[FM][FN], const u32x4_t* L, const XlDma64<PA, PB>& d,
                                             int arow, int brow, int hi, int sw) {
  constexpr int PS = PA + PB, NMM = FM * FN, E = FM + FN, EA = PA + FM + FN, EW = PB + FM + FN, SS = SA + SW;
  const uint32_t l0 = lds_addr(L);
  Frags<FM, FN> F0, F1;
  const int nst = d.ns / 2;
  int b = 0;                               // buffer of stage g
  for (int g = 0; g < nst; g++) {
    LAYA_WAIT_VMCNT((NB - 2) * PS);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const int bp = b == 0 ? NB - 1 : b - 1;
    const uint32_t la = l0 + (uint32_t)(bp * SS * 16), lb = la + (uint32_t)(SA * 16);
    const u32x4_t* CA = L + b * SS;
    const u32x4_t* CB = CA + SA;
#pragma unroll
    for (int o = 0; o < E; o++) load_frag64(F0, o, CA, CB, arow, brow, 0, hi, sw);
#pragma unroll
    for (int t = 0; t < NMM; t++) {
      mma_one_x<SWAP>(acc, F0, t);
#pragma unroll
      for (int o = t * EA / NMM; o < (t + 1) * EA / NMM; o++) {
        if (o < PA) d.op_a(o, la, g + NB - 1);
        else load_frag64(F1, o - PA, CA, CB, arow, brow, 1, hi, sw);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int t = 0; t < NMM; t++) {
      mma_one_x<SWAP>(acc, F1, t);
#pragma unroll
      for (int o = t * EW / NMM; o < (t + 1) * EW / NMM; o++) {
        if (o < PB) d.op_b(o, lb, g + NB - 1);
        else load_frag64(F0, o - PB, CA, CB, arow, brow, 2, hi, sw);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int t = 0; t < NMM; t++) {
      mma_one_x<SWAP>(acc, F0, t);
#pragma unroll
      for (int o = t * E / NMM; o < (t + 1) * E / NMM; o++) load_frag64(F1, o, CA, CB, arow, brow, 3, hi, sw);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int t = 0; t < NMM; t++) mma_one_x<SWAP>(acc, F1, t);
    b = b + 1 == NB ? 0 : b + 1;
  }
  LAYA_WAIT_VMCNT(0);                      // the refills past the last stage
}

// LDS of one tile (16-byte chunks): the K stages (two whole stages; LOOP 1: three A buffers and two
// W buffers; LOOP 2: four whole stages) and, for the QKV projection with two stages where it fits,
// the RoPE tables of the tile's rows
template <int BM, int BN, int EPI, int LOOP>
struct XlLds {
  static constexpr int BMQ = (BM + 31) / 32 * 32;
  static constexpr int SA = BMQ * 8, SW = BN * 8;
  static constexpr int NST = LOOP == 1 ? 3 * SA + 2 * SW : LOOP == 2 ? 4 * (SA + SW) : 2 * (SA + SW);
  static constexpr bool PRE = EPI == EPI_QKV && LOOP == 0 && (NST + BM * 16) * 16 < 160 * 1024;
  static constexpr int chunks = NST + (PRE ? BM * 16 : 0);
};

// One BM x BN output tile (tile bid0 of the GEMM; with EPI_PARTIAL, bid0 also selects the K chunk),
// computed by the 256 threads of the calling workgroup in the LDS array L (XlLds chunks).
// LOOP: the K loop.  0: two stage buffers (one workgroup per CU); 1 (128x128 tiles when the grid
// puts two workgroups on a CU): three A buffers and two W buffers; 2 (128x128 tiles, grid of at most
// one workgroup per CU): four stage buffers, two stages of lead.
// LNX: the LayerNorm fold of GemmArgs.  With EPI_RESID the kernel writes Xh and the per-group
// statistics; with EPI_STORE, EPI_QKV and EPI_GEGLU it applies the fold to its product.
template <int BM, int BN, int WM, int WN, int EPI, int ACT, bool HB, int LOOP, bool LNX>
__device__ __forceinline__ void xl_tile(const GemmArgs a, int bid0, u32x4_t* L) {
#include "gemm_xl_tile.inc"
}

template <int BM, int BN, int WM, int WN, int EPI, int ACT, bool HB, int LOOP, bool LNX>
__global__ __launch_bounds__(256, 1) void k_gemm_xl(const GemmArgs a) {
  __shared__ u32x4_t L[XlLds<BM, BN, EPI, LOOP>::chunks];
  const int bid0 = blockIdx.x;
#include "gemm_xl_tile.inc"
}

// A row split in one launch: the tiles of rows [0, split) in the first tile shape (a: those rows,
// nmain tiles, workgroups 0 .. nmain - 1), then the tiles of the remaining rows in the second
// (b: the same GEMM from row split on).  Workgroups are dispatched in order of their index, so the
// smaller tiles of the second shape start last and fill the CUs that the first shape's partial last
// round leaves idle, where a second launch would wait for the first to finish.  Every output keeps
// its K order, so the results are those of either shape alone.  Two workgroups per CU (both shapes
// fit 80 KB of LDS and 256 registers).
template <int BM, int BN, int WM, int WN, int LOOP, int BM2, int BN2, int WM2, int WN2, int LOOP2, int EPI>
__global__ __launch_bounds__(256, 1) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm_xl_pair(
    const GemmArgs a, const GemmArgs b, int nmain) {
  constexpr int C1 = XlLds<BM, BN, EPI, LOOP>::chunks, C2 = XlLds<BM2, BN2, EPI, LOOP2>::chunks;
  static_assert((C1 > C2 ? C1 : C2) * 16 <= 80 * 1024, "two workgroups per CU");
  __shared__ u32x4_t L[C1 > C2 ? C1 : C2];
  if ((int)blockIdx.x < nmain) xl_tile<BM, BN, WM, WN, EPI, ACT_NONE, false, LOOP, false>(a, blockIdx.x, L);
  else xl_tile<BM2, BN2, WM2, WN2, EPI, ACT_NONE, false, LOOP2, false>(b, (int)blockIdx.x - nmain, L);
}

// The achievable bf16 MFMA rate of the chip at the clock it holds under MFMA load: every wave
// issues v_mfma_f32_32x32x16_bf16 back to back on eight independent register accumulators, with
// no memory traffic, and stores one value per lane at the end (so the work is kept).  32768 flop
// per MFMA; blocks of 4 waves.
__global__ __launch_bounds__(256) void k_mfma_loop(float* __restrict__ out, int iters) {
  f32x16_t acc[8];
#pragma unroll
  for (int j = 0; j < 8; j++)
#pragma unroll
    for (int e = 0; e < 16; e++) acc[j][e] = 0.f;
  bf16x8_t a, b;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    a[i] = (__bf16)(1e-3f * (float)((threadIdx.x + i) & 7));
    b[i] = (__bf16)(1e-3f * (float)((threadIdx.x * 3 + i) & 7));
  }
  for (int it = 0; it < iters; it++)
#pragma unroll
    for (int j = 0; j < 8; j++) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[j], 0, 0, 0);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 8; j++)
#pragma unroll
    for (int e = 0; e < 16; e++) s += acc[j][e];
  out[(size_t)blockIdx.x * 256 + threadIdx.x] = s;
}

void launch_mfma_loop(float* out, int blocks, int iters, hipStream_t st) {
  LAYA_LAUNCH(k_mfma_loop, dim3(blocks), dim3(256), 0, st, out, iters);
}

// compute units of the current device, cached per device.  If the query fails (a process whose
// HIP runtime instance has no current device, e.g. a host that drives the library through streams
// of another runtime), the count is 256 and the query's error is cleared so that the caller's
// error check does not see it: the count only picks between two K loops that give the same bits.
static int num_cus() {
  static std::atomic<int> cached[16];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) {
    (void)hipGetLastError();
    return 256;
  }
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
      (void)hipGetLastError();
      n = 256;
    }
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// whether a launch uses the LayerNorm fold (GemmArgs), and whether this kernel set has it: the
// residual update (with or without bias), the QKV projection, GeGLU without bias and a ReLU store
// with bias, the epilogues the engine folds a LayerNorm into
static bool ln_fold(const GemmArgs& a) { return a.ln_mr != nullptr || a.stats != nullptr || a.Xh != nullptr; }

template <int EPI, int ACT>
static constexpr bool ln_fold_built(bool bias) {
  return EPI == EPI_RESID || EPI == EPI_QKV || (EPI == EPI_GEGLU && ACT == ACT_NONE) || (EPI == EPI_STORE && ACT == ACT_RELU);
}

// GEMMs without a bias run kernels without the bias code, except the QKV projection: its bias-free
// build allocates registers worse (it spills at 256x256), so it keeps the bias code (adding 0)
template <int BM, int BN, int WM, int WN, int EPI, int ACT, int LOOP>
static void launch_xl_ring(const GemmArgs& a, int tiles, hipStream_t st) {
  if (ln_fold(a)) {
    // (256x256 fold consumers are not built: they would spill; xl_cfg_fits never offers them)
    if constexpr (ln_fold_built<EPI, ACT>(true) && (EPI == EPI_RESID || BM * BN < 256 * 256)) {
      const bool hb = EPI == EPI_QKV || a.bias != nullptr;
      if constexpr (EPI == EPI_RESID) {
        if (hb) LAYA_LAUNCH((k_gemm_xl<BM, BN, WM, WN, EPI, ACT, true, LOOP, true>), dim3(tiles), dim3(256), 0, st, a);
        else LAYA_LAUNCH((k_gemm_xl<BM, BN, WM, WN, EPI, ACT, false, LOOP, true>), dim3(tiles), dim3(256), 0, st, a);
        return;
      } else if constexpr (EPI == EPI_QKV) {
        // the encoder's projection has no bias; its fold kernel leaves the bias code out
        if (a.bias) LAYA_LAUNCH((k_gemm_xl<BM, BN, WM, WN, EPI, ACT, true, LOOP, true>), dim3(tiles), dim3(256), 0, st, a);
        else LAYA_LAUNCH((k_gemm_xl<BM, BN, WM, WN, EPI, ACT, false, LOOP, true>), dim3(tiles), dim3(256), 0, st, a);
        return;
      } else if constexpr (EPI == EPI_STORE) {
        if (hb) { LAYA_LAUNCH((k_gemm_xl<BM, BN, WM, WN, EPI, ACT, true, LOOP, true>), dim3(tiles), dim3(256), 0, st, a); return; }
      } else {
        if (!hb) { LAYA_LAUNCH((k_gemm_xl<BM, BN, WM, WN, EPI, ACT, false, LOOP, true>), dim3(tiles), dim3(256), 0, st, a); return; }
      }
    }
    fprintf(stderr, "[laya] gemm: no LayerNorm-fold kernel for epilogue %d, activation %d, bias %d\n", EPI, ACT,
            (int)(a.bias != nullptr));
    exit(1);
  }
  if (EPI == EPI_QKV || a.bias) LAYA_LAUNCH((k_gemm_xl<BM, BN, WM, WN, EPI, ACT, true, LOOP, false>), dim3(tiles), dim3(256), 0, st, a);
  else if constexpr (EPI != EPI_QKV) LAYA_LAUNCH((k_gemm_xl<BM, BN, WM, WN, EPI, ACT, false, LOOP, false>), dim3(tiles), dim3(256), 0, st, a);
}

// 128x128 tiles take the three-A-buffer loop when the grid has more tiles than the chip has CUs,
// i.e. when CUs run two workgroups whose stages interleave, and the four-buffer loop otherwise
// (one workgroup per CU, few tiles: the fill latency is what a stage waits for).  Other tiles take
// the two-buffer loop.  All give the same bits.
template <int BM, int BN, int WM, int WN, int EPI, int ACT>
static void launch_xl_hb(const GemmArgs& a, hipStream_t st) {
  const int tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN) * (EPI == EPI_PARTIAL ? a.ksplit : 1);
  if constexpr (BM * BN <= 128 * 128) {
    if (tiles > num_cus()) launch_xl_ring<BM, BN, WM, WN, EPI, ACT, 1>(a, tiles, st);
    else launch_xl_ring<BM, BN, WM, WN, EPI, ACT, 2>(a, tiles, st);
    return;
  }
  launch_xl_ring<BM, BN, WM, WN, EPI, ACT, 0>(a, tiles, st);
}

template <int BM, int BN, int WM, int WN>
static void launch_xl(int epi, const GemmArgs& a, hipStream_t st) {
  if (epi == EPI_STORE) {
    if (a.act == ACT_RELU) launch_xl_hb<BM, BN, WM, WN, EPI_STORE, ACT_RELU>(a, st);
    else if (a.act == ACT_GELU) launch_xl_hb<BM, BN, WM, WN, EPI_STORE, ACT_GELU>(a, st);
    else launch_xl_hb<BM, BN, WM, WN, EPI_STORE, ACT_NONE>(a, st);
    return;
  }
  switch (epi) {
    case EPI_RESID: launch_xl_hb<BM, BN, WM, WN, EPI_RESID, ACT_NONE>(a, st); break;
    case EPI_QKV:
      if constexpr (BM <= BN) launch_xl_hb<BM, BN, WM, WN, EPI_QKV, ACT_NONE>(a, st);
      else { fprintf(stderr, "[laya] gemm: QKV tiles need BM <= BN\n"); exit(1); }
      break;
    case EPI_GEGLU: launch_xl_hb<BM, BN, WM, WN, EPI_GEGLU, ACT_NONE>(a, st); break;
    case EPI_PARTIAL: launch_xl_hb<BM, BN, WM, WN, EPI_PARTIAL, ACT_NONE>(a, st); break;
    default: fprintf(stderr, "[laya] gemm: bad epilogue %d\n", epi); exit(1);
  }
}

// Tile configurations for the bf16 path and the analytic planner that picks one per GEMM when no
// measured choice is given: estimated time = rounds of concurrently resident tiles x per-tile
// cost, with each shape's throughput per tile area relative to 256x256 (measured on MI355X at the
// ModernBERT-large shapes; it varies with K and the epilogue, which is why the engine times the
// candidates instead where it can).  One-workgroup-per-CU shapes run in lockstep rounds (a partial
// last round costs a whole one); two 128x128 workgroups per CU interleave, so their partial rounds
// cost their fraction.  QKV tiles must lie inside one of the q/k/v sections (D % BN == 0) and need
// BM <= BN.
struct XlCfg { int bm, bn, per_cu; float rel; };
static const XlCfg kXl[kGemmConfigs] = {{256, 256, 1, 1.00f}, {256, 128, 1, 0.80f}, {128, 256, 1, 0.83f},
                                        {128, 128, 2, 0.72f}, {192, 256, 1, 0.95f}, {160, 256, 1, 0.93f},
                                        {128, 192, 2, 0.80f}, {192, 128, 2, 0.80f}, {128, 64, 2, 0.50f}};

// tile configuration pinned for every bf16 launch, process-wide (-1: none), by gemm_config()
// (laya_ext_gemm_config); an engine's LAYA_GEMM_CFG is that engine's own and reaches the launches
// as the caller's configuration
static std::atomic<int> g_gemm_cfg{-1};

// row split applied with the pinned configuration (0: none)
static std::atomic<int> g_split_rows{0}, g_cfg_tail{-1};

int gemm_pinned() { return g_gemm_cfg.load(std::memory_order_relaxed); }

int gemm_config(int cfg) {
  const int prev = gemm_pinned();
  g_gemm_cfg.store(cfg, std::memory_order_relaxed);
  return prev;
}

static std::atomic<int> g_ksplit{0};

int gemm_pin_ksplit(int ks) { return g_ksplit.exchange(ks, std::memory_order_relaxed); }

void gemm_pin_split(int split_rows, int cfg_tail) {
  g_split_rows.store(split_rows, std::memory_order_relaxed);
  g_cfg_tail.store(cfg_tail, std::memory_order_relaxed);
}

// Largest operand, in bytes, that any GEMM launch accepts.  The tiled kernel reads A and W through
// buffer resources whose record count and offsets are 32-bit (it takes operands below 2 GiB,
// xl_usable, and hands larger ones to the generic kernel); a 4 GiB limit on every operand keeps
// all byte counts the launchers compute from int shapes exact, whichever kernel runs.
static constexpr size_t kMaxOperandBytes = (size_t)1 << 32;

bool gemm_shape_ok(int epi, const GemmArgs& a, int elt_bytes, const char** why) {
  const int bk = 128 / elt_bytes, align = 16 / elt_bytes;
  if (a.M <= 0 || a.N <= 0) { *why = "empty"; return false; }
  {
    const size_t M = (size_t)a.M, N = (size_t)a.N, e = (size_t)elt_bytes;
    size_t big = std::max(M * (size_t)std::max(a.lda, 0) * e, N * (size_t)std::max(a.ldw, 0) * e);
    if (epi == EPI_STORE || epi == EPI_GEGLU) big = std::max(big, M * (size_t)std::max(a.ldc, 0) * e);
    if (epi == EPI_RESID) big = std::max(big, M * (size_t)std::max(a.ldx, 0) * 4);
    if (epi == EPI_QKV)
      big = std::max(big, std::max(M * (size_t)std::max(a.ldqk, 0) * e, N / 3 * (size_t)std::max(a.ldv, 0) * e));
    if (a.Xh) big = std::max(big, M * (size_t)std::max(a.ldxh, 0) * 2);
    if (big >= kMaxOperandBytes) { *why = "every operand must be smaller than 4 GiB"; return false; }
  }
  if (a.K <= 0 || a.K % bk) { *why = "K must be a positive multiple of the 128-byte K slice"; return false; }
  if (a.lda % align || a.ldw % align || a.lda < a.K || a.ldw < a.K) { *why = "row strides must be 16-byte multiples >= K"; return false; }
  if ((reinterpret_cast<uintptr_t>(a.A) | reinterpret_cast<uintptr_t>(a.W)) & 15) { *why = "operands must be 16-byte aligned"; return false; }
  if (epi == EPI_GEGLU && a.N % 64) { *why = "GeGLU needs N % 64 == 0"; return false; }
  if (epi == EPI_QKV) {
    if (a.N != 3 * a.H * a.HD || a.HD % 16) { *why = "QKV needs N == 3*H*HD, HD % 16 == 0"; return false; }
    if (a.rope_cos && a.HD != 64) { *why = "fused RoPE needs HD == 64"; return false; }
  }
  if (ln_fold(a)) {
    if (elt_bytes != 2 || a.ksplit > 1) { *why = "the LayerNorm fold needs bf16 operands and no split-K"; return false; }
    if (a.ln_mr && (epi == EPI_RESID || epi == EPI_PARTIAL || !a.ln_c)) {
      *why = "LayerNorm-fold consumers: store, QKV or GeGLU epilogue with column sums";
      return false;
    }
    const bool prod = a.stats || a.Xh;
    if (prod && (epi != EPI_RESID || !a.stats || !a.Xh || a.N % 64 || a.ldxh % 8 || a.ldxh < a.N || a.ldst < a.M)) {
      *why = "LayerNorm-fold producers: residual epilogue with Xh and statistics, N a multiple of 64, ldst >= M";
      return false;
    }
  }
  return true;
}

// the tiled bf16 kernel needs 16-byte epilogue stores (N, the row strides and the output bases in
// multiples of 8 elements) and operands that 32-bit buffer offsets reach
static bool xl_usable(int epi, const GemmArgs& a) {
  const size_t abytes = (size_t)a.M * a.lda * 2, wbytes = (size_t)a.N * a.ldw * 2;
  const bool aligned = a.N % 8 == 0 && ((epi == EPI_STORE || epi == EPI_GEGLU) ? a.ldc % 8 == 0 : true) &&
                       (epi == EPI_RESID ? a.ldx % 4 == 0 : true) && (epi == EPI_QKV ? a.ldqk % 8 == 0 && a.ldv % 8 == 0 : true);
  return aligned && abytes < (1u << 31) - 65536 && wbytes < (1u << 31) - 65536;
}

static bool xl_cfg_fits(int epi, const GemmArgs& a, int cfg) {
  if (cfg < 0 || cfg >= kGemmConfigs) return false;
  // the LayerNorm-fold consumers do not fit 256x256 tiles' registers (they would spill)
  if (a.ln_mr && cfg == 0) return false;
  return epi != EPI_QKV || (kXl[cfg].bm <= kXl[cfg].bn && (a.H * a.HD) % kXl[cfg].bn == 0);
}

static int gemm_pick(int epi, const GemmArgs& a) {
  int best = -1;
  double bt = 1e300;
  for (int i = 0; i < kGemmConfigs; i++) {
    if (!xl_cfg_fits(epi, a, i)) continue;
    const XlCfg& c = kXl[i];
    const double tiles = (double)((a.M + c.bm - 1) / c.bm) * ((a.N + c.bn - 1) / c.bn);
    const double slots = 256.0 * c.per_cu;
    const double rounds = c.per_cu > 1 ? std::max(1.0, tiles / slots) : std::ceil(tiles / slots);
    const double t = rounds * (double)c.bm * c.bn * c.per_cu / c.rel;
    if (t < bt * 0.999) { bt = t; best = i; }
  }
  return best;
}

bool gemm_config_valid(int epi, const GemmArgs& a, int cfg) {
  const char* why = "";
  return gemm_shape_ok(epi, a, 2, &why) && xl_usable(epi, a) && xl_cfg_fits(epi, a, cfg);
}

int gemm_config_bm(int cfg) { return cfg >= 0 && cfg < kGemmConfigs ? kXl[cfg].bm : 0; }
int gemm_config_bn(int cfg) { return cfg >= 0 && cfg < kGemmConfigs ? kXl[cfg].bn : 0; }

// the same GEMM restricted to rows [r0, M): every row-indexed operand moves by r0 rows (V^T by r0
// columns); the K order of every output element is unchanged
static GemmArgs rows_from(const GemmArgs& a, int r0) {
  GemmArgs b = a;
  b.M = a.M - r0;
  b.A = reinterpret_cast<const bf16_t*>(a.A) + (size_t)r0 * a.lda;
  if (a.C) b.C = reinterpret_cast<bf16_t*>(a.C) + (size_t)r0 * a.ldc;
  if (a.X) b.X = a.X + (size_t)r0 * a.ldx;
  if (a.Xh) b.Xh = a.Xh + (size_t)r0 * a.ldxh;
  if (a.stats) b.stats = a.stats + (size_t)r0 * 2;
  if (a.ln_mr) b.ln_mr = a.ln_mr + (size_t)r0 * 2;
  if (a.Q) b.Q = reinterpret_cast<bf16_t*>(a.Q) + (size_t)r0 * a.ldqk;
  if (a.Kt) b.Kt = reinterpret_cast<bf16_t*>(a.Kt) + (size_t)r0 * a.ldqk;
  if (a.Vt) b.Vt = reinterpret_cast<bf16_t*>(a.Vt) + r0;
  if (a.pos) b.pos = a.pos + r0;
  b.split_rows = 0;
  return b;
}

bool gemm_split_valid(int epi, const GemmArgs& a, int cfg, int split_rows, int cfg_tail) {
  // 8-row multiples keep the moved V^T columns 16-byte aligned
  if (split_rows <= 0 || split_rows >= a.M || split_rows % 8) return false;
  GemmArgs head = a;
  head.M = split_rows;
  return gemm_config_valid(epi, head, cfg) && gemm_config_valid(epi, rows_from(a, split_rows), cfg_tail);
}

int gemm_planned(int epi, const GemmArgs& a) {
  const char* why = "";
  return gemm_shape_ok(epi, a, 2, &why) && xl_usable(epi, a) ? gemm_pick(epi, a) : -1;
}

static void launch_xl_cfg(int epi, const GemmArgs& a, int cfg, hipStream_t st) {
  switch (cfg) {
    case 0: launch_xl<256, 256, 2, 2>(epi, a, st); return;
    case 1: launch_xl<256, 128, 2, 2>(epi, a, st); return;
    case 2: launch_xl<128, 256, 2, 2>(epi, a, st); return;
    case 3: launch_xl<128, 128, 2, 2>(epi, a, st); return;
    case 4: launch_xl<192, 256, 2, 2>(epi, a, st); return;
    case 5: launch_xl<160, 256, 1, 4>(epi, a, st); return;
    case 6: launch_xl<128, 192, 4, 1>(epi, a, st); return;
    case 7: launch_xl<192, 128, 2, 2>(epi, a, st); return;
    case 8: launch_xl<128, 64, 4, 1>(epi, a, st); return;
    default: fprintf(stderr, "[laya] gemm: bad tile configuration %d\n", cfg); exit(1);
  }
}

// Row splits that run as one launch (k_gemm_xl_pair): 192x128 tiles (two per CU) over the first
// rows, then 128x64 or 128x128 tiles over the rest, for the plain store and the GeGLU epilogue
// without bias, activation or LayerNorm fold.  The second shape's tiles take the three-A-buffer
// loop, as they would in a launch of their own with two workgroups per CU.  Returns false for any
// other split (which then runs as two launches).
static bool launch_xl_pair(int epi, const GemmArgs& h, const GemmArgs& t, int cfg, int tail, hipStream_t st) {
  if (cfg != 7 || (tail != 8 && tail != 3) || (epi != EPI_STORE && epi != EPI_GEGLU) || h.bias || h.act != ACT_NONE ||
      ln_fold(h))
    return false;
  const int nmain = ((h.M + 191) / 192) * ((h.N + 127) / 128);
  const int bn2 = tail == 8 ? 64 : 128;
  const dim3 grid((unsigned)(nmain + ((t.M + 127) / 128) * ((t.N + bn2 - 1) / bn2)));
  if (tail == 8) {
    if (epi == EPI_STORE)
      LAYA_LAUNCH((k_gemm_xl_pair<192, 128, 2, 2, 0, 128, 64, 4, 1, 1, EPI_STORE>), grid, dim3(256), 0, st, h, t, nmain);
    else
      LAYA_LAUNCH((k_gemm_xl_pair<192, 128, 2, 2, 0, 128, 64, 4, 1, 1, EPI_GEGLU>), grid, dim3(256), 0, st, h, t, nmain);
  } else {
    if (epi == EPI_STORE)
      LAYA_LAUNCH((k_gemm_xl_pair<192, 128, 2, 2, 0, 128, 128, 2, 2, 1, EPI_STORE>), grid, dim3(256), 0, st, h, t, nmain);
    else
      LAYA_LAUNCH((k_gemm_xl_pair<192, 128, 2, 2, 0, 128, 128, 2, 2, 1, EPI_GEGLU>), grid, dim3(256), 0, st, h, t, nmain);
  }
  return true;
}

// Split-K reduction: out = epilogue(sum over the ks partial slices in slice order + bias), four
// columns per thread.  EPI_RESID adds into the fp32 residual X; EPI_STORE applies the activation
// and stores bf16.
template <int EPI, int ACT, bool HB>
__global__ __launch_bounds__(256) void k_splitk_reduce(const float* __restrict__ ws, int ks, int M, int N,
                                                       const float* __restrict__ bias, void* out, int ldo) {
  const size_t n4 = (size_t)M * N / 4, slice = (size_t)M * N;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
    const size_t e = i * 4;
    const int m = (int)(e / N), n = (int)(e % N);
    float4 v = *reinterpret_cast<const float4*>(ws + e);
    for (int k = 1; k < ks; k++) {
      const float4 t = *reinterpret_cast<const float4*>(ws + k * slice + e);
      v.x += t.x; v.y += t.y; v.z += t.z; v.w += t.w;
    }
    if constexpr (HB) {
      const float4 b = *reinterpret_cast<const float4*>(bias + n);
      v.x += b.x; v.y += b.y; v.z += b.z; v.w += b.w;
    }
    if constexpr (EPI == EPI_RESID) {
      float4* xp = reinterpret_cast<float4*>(reinterpret_cast<float*>(out) + (size_t)m * ldo + n);
      float4 x = *xp;
      x.x += v.x; x.y += v.y; x.z += v.z; x.w += v.w;
      *xp = x;
    } else {
      auto f = [](float t) {
        if constexpr (ACT == ACT_RELU) t = fmaxf(t, 0.f);
        if constexpr (ACT == ACT_GELU) t = gelu_erf_as(t);
        return t;
      };
      uint2 u;
      u.x = pk_bf16(f(v.x), f(v.y));
      u.y = pk_bf16(f(v.z), f(v.w));
      *reinterpret_cast<uint2*>(reinterpret_cast<bf16_t*>(out) + (size_t)m * ldo + n) = u;
    }
  }
}

template <int EPI, int ACT>
static void launch_reduce(const GemmArgs& a, const float* ws, int ks, int M, void* out, int ldo, hipStream_t st) {
  const size_t n4 = (size_t)M * a.N / 4;
  const unsigned blocks = (unsigned)std::min<size_t>((n4 + 255) / 256, 4096);
  if (a.bias) LAYA_LAUNCH((k_splitk_reduce<EPI, ACT, true>), dim3(blocks), dim3(256), 0, st, ws, ks, M, a.N, a.bias, out, ldo);
  else LAYA_LAUNCH((k_splitk_reduce<EPI, ACT, false>), dim3(blocks), dim3(256), 0, st, ws, ks, M, a.N, a.bias, out, ldo);
}

// Split-K over rows chunks that fit the workspace: per chunk one launch of ks x tiles workgroups
// writing fp32 partials (EPI_PARTIAL), then one reduction.
static void launch_splitk(int epi, const GemmArgs& a, int ks, hipStream_t st) {
  // chunks of `per` whole stages; ks drops to the number of non-empty chunks
  const int stages = a.K / 64, per = (stages + ks - 1) / ks;
  ks = (stages + per - 1) / per;
  const size_t row_bytes = (size_t)ks * a.N * sizeof(float);
  const int rc = (int)std::min<size_t>((size_t)a.M, a.ws_bytes / row_bytes);
  if (rc < 1) { fprintf(stderr, "[laya] gemm: split-K workspace too small\n"); exit(1); }
  for (int r0 = 0; r0 < a.M; r0 += rc) {
    const int mr = std::min(rc, a.M - r0);
    GemmArgs p = rows_from(a, r0);
    p.M = mr;
    p.K = per * 64;
    p.kfull = a.K;
    p.bias = nullptr;
    p.act = ACT_NONE;
    p.X = a.ws;
    p.ldx = a.N;
    p.ksplit = ks;
    launch_xl_cfg(EPI_PARTIAL, p, 3, st);                 // 128x128 tiles: the most workgroups
    if (epi == EPI_RESID && a.partials_only && rc >= a.M) return;    // the next LayerNorm reduces
    if (epi == EPI_RESID) {
      launch_reduce<EPI_RESID, ACT_NONE>(a, a.ws, ks, mr, a.X + (size_t)r0 * a.ldx, a.ldx, st);
    } else {
      void* out = reinterpret_cast<bf16_t*>(a.C) + (size_t)r0 * a.ldc;
      if (a.act == ACT_RELU) launch_reduce<EPI_STORE, ACT_RELU>(a, a.ws, ks, mr, out, a.ldc, st);
      else if (a.act == ACT_GELU) launch_reduce<EPI_STORE, ACT_GELU>(a, a.ws, ks, mr, out, a.ldc, st);
      else launch_reduce<EPI_STORE, ACT_NONE>(a, a.ws, ks, mr, out, a.ldc, st);
    }
  }
}

template <typename T>
void launch_gemm(int epi, const GemmArgs& a, hipStream_t st) {
  const char* why = "";
  if (!gemm_shape_ok(epi, a, (int)sizeof(T), &why)) {
    fprintf(stderr, "[laya] gemm %dx%dx%d epi %d rejected: %s\n", a.M, a.N, a.K, epi, why);
    exit(1);
  }
  if (ln_fold(a) && (sizeof(T) != 2 || !xl_usable(epi, a) || gemm_planned(epi, a) < 0)) {
    fprintf(stderr, "[laya] gemm %dx%dx%d epi %d: the LayerNorm fold needs the tiled bf16 kernel\n", a.M, a.N, a.K, epi);
    exit(1);
  }
  if constexpr (sizeof(T) == 2) {
    if (xl_usable(epi, a)) {
      const int pinned_ks = ln_fold(a) ? 0 : g_ksplit.load(std::memory_order_relaxed);
      const int ks = a.ksplit > 1 ? a.ksplit : pinned_ks;
      if (ks > 1 && (epi == EPI_STORE || epi == EPI_RESID) && a.K % 64 == 0 && a.K >= 128 && a.ws != nullptr) {
        launch_splitk(epi, a, ks, st);
        return;
      }
      // a pinned configuration (gemm_config, with its pinned row split) wins over the caller's,
      // which wins over the planner's; one this shape cannot use falls through
      int cfg = a.cfg, split = a.split_rows, tail = a.cfg_tail;
      const int pinned = gemm_pinned();
      if (xl_cfg_fits(epi, a, pinned)) {
        cfg = pinned;
        split = g_split_rows.load(std::memory_order_relaxed);
        tail = g_cfg_tail.load(std::memory_order_relaxed);
      }
      if (split > 0 && gemm_split_valid(epi, a, cfg, split, tail)) {
        GemmArgs head = a;
        head.M = split;
        const GemmArgs rest = rows_from(a, split);
        if (launch_xl_pair(epi, head, rest, cfg, tail, st)) return;
        launch_xl_cfg(epi, head, cfg, st);
        launch_xl_cfg(epi, rest, tail, st);
        return;
      }
      if (!xl_cfg_fits(epi, a, cfg)) cfg = gemm_pick(epi, a);
      if (cfg >= 0) { launch_xl_cfg(epi, a, cfg, st); return; }
    }
  }
  // fp32 (and bf16 shapes the MFMA path above cannot take): 128x128 tiles when they fill the chip,
  // else 64x64 tiles (waves 4x1, so each wave still holds whole 64-column groups for the GeGLU and
  // RoPE pairings) for four times the workgroups.  Every output's K order is the same in all of
  // them, so the choice changes no bits and a row's result does not depend on the batch.
  // Stores and residual updates whose 64x64 tiles still leave CUs idle take 32x64 tiles.
  const int tiles128 = ((a.M + 127) / 128) * ((a.N + 127) / 128);
  const int tiles64 = ((a.M + 63) / 64) * ((a.N + 63) / 64);
  if (tiles128 >= num_cus()) {
    launch_cfg<T, 128, 128, 2, 2>(epi, a, st);
  } else if (tiles64 < num_cus() && (epi == EPI_STORE || epi == EPI_RESID)) {
    const int tiles = ((a.M + 31) / 32) * ((a.N + 63) / 64);
    if (epi == EPI_STORE) LAYA_LAUNCH((k_gemm<T, 32, 64, 2, 2, EPI_STORE>), dim3(tiles), dim3(256), 0, st, a);
    else LAYA_LAUNCH((k_gemm<T, 32, 64, 2, 2, EPI_RESID>), dim3(tiles), dim3(256), 0, st, a);
  } else {
    launch_cfg<T, 64, 64, 4, 1>(epi, a, st);
  }
}

template void launch_gemm<float>(int, const GemmArgs&, hipStream_t);
template void launch_gemm<bf16_t>(int, const GemmArgs&, hipStream_t);

}  // namespace laya

#ifdef LAYA_TILE_TRACE
// the per-tile records of the GEMM launches since the last clear (see TileTrace)
extern "C" int laya_tile_trace_read(void* host, size_t records) {
  void* p = nullptr;
  if (records > (size_t)laya::kTileTraceMax || hipGetSymbolAddress(&p, HIP_SYMBOL(laya::g_tile_trace)) != hipSuccess) return -1;
  return hipMemcpy(host, p, records * 64, hipMemcpyDeviceToHost) == hipSuccess ? 0 : -1;
}
extern "C" int laya_tile_trace_clear() {
  void* p = nullptr;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(laya::g_tile_trace)) != hipSuccess) return -1;
  return hipMemset(p, 0, sizeof(laya::g_tile_trace)) == hipSuccess ? 0 : -1;
}
#endif
