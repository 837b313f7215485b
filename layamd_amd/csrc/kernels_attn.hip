// Attention over packed variable-length sequences for gfx950 (wave64 MFMA, fp32 online softmax).
// Two kernels: k_attention_bf16 (the bf16 engine's, described above it) and k_attention<T>, the
// fp32 engine's, described here.
//
// One 256-thread workgroup owns one query tile (<= 64 queries of one sequence) of one head;
// each wave64 owns 16 queries.  Keys advance in blocks of 64: the workgroup stages the block's
// K rows ([key][d], 16-byte chunks XOR-swizzled by key) and V^T rows ([d][key], swizzled by d)
// in LDS, then every wave computes
//
//     S^T = K Q^T    (MFMA A = K rows, B = Q rows, both d-contiguous)
//     O^T += V^T P^T (MFMA A = V^T rows from LDS, B = P^T straight from the S^T registers)
//
// Working in the transposed frame keeps one query per lane column (lane l holds query l % 16):
// the 16x16 accumulator layout puts S^T[key 4*(l/16)+i][query l%16] in lane l, which is exactly
// the B-operand layout P^T needs for the next MFMA, with keys relabelled consistently in the
// V^T operand, so P never goes through LDS.  Row max / row sum need only two cross-lane steps
// (lanes l, l^16, l^32, l^48 share a query).  Scores and the running max/sum are fp32; the
// score matrix never touches memory.
//
// Masks: key j of the sequence is visible to query position p when j < len and, for sliding
// layers, |p - j| <= window_half (inclusive, HF masking_utils.py:141-151).  Keys beyond the
// sequence are read (V^T columns up to the next 64-key boundary exist and hold finite values:
// padding rows, the next question, or the zero-initialised slack) but get probability exactly 0.
#include <type_traits>

#include "kernels.h"

namespace laya {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));   // one 16-byte chunk
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));   // 8 bytes

template <typename T>
__global__ __launch_bounds__(256) void k_attention(const T* __restrict__ Q, const T* __restrict__ K, int ldqk,
                                                   const T* __restrict__ Vt, int ldv, T* __restrict__ O, int ldo,
                                                   const AttnTile* __restrict__ tiles, const int* __restrict__ soff,
                                                   const int* __restrict__ vlen, const int* __restrict__ gq,
                                                   const int* __restrict__ grow,
                                                   int window_half, float scale) {
  constexpr int HD = 64;
  constexpr int CPR = HD * (int)sizeof(T) / 16;        // 16-byte chunks per 64-element row
  constexpr int EPC = 16 / (int)sizeof(T);             // elements per chunk
  __shared__ u32x4_t Ks[64 * CPR];                       // [key][chunk ^ (key % CPR)]
  __shared__ u32x4_t Vs[64 * CPR];                       // [d][...] swizzled by d

  const AttnTile tile = tiles[blockIdx.x];
  if (tile.nq <= 0) return;                              // an empty tile of the pass's tile capacity
  const int h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l16 = lane & 15, g = lane >> 4;
  const int b = tile.seq, len = vlen[b], base = soff[b], vb = base;   // V^T column = row

  // this lane's query (16 per wave)
  const int r = wave * 16 + l16;
  const bool qvalid = r < tile.nq;
  const int rr = qvalid ? r : 0;
  int p, orow;
  if (gq) { const int gi = gq[tile.q0 + rr]; p = grow[gi] - base; orow = gi; }
  else { p = tile.q0 + rr; orow = base + p; }

  // key range of the tile
  int lo = 0, hi = len;
  if (window_half > 0 && !gq) {
    lo = max(0, tile.q0 - window_half) & ~15;
    hi = min(len, tile.q0 + tile.nq - 1 + window_half + 1);
  }

  // Q fragments (B operand of S^T = K Q^T): lane holds Q[p][...] chunks
  const T* qrow = Q + (size_t)(base + p) * ldqk + h * HD;
  u32x4_t qf[4];
  if constexpr (sizeof(T) == 2) {
    qf[0] = reinterpret_cast<const u32x4_t*>(qrow)[g];          // d = 8g .. 8g+7
    qf[1] = reinterpret_cast<const u32x4_t*>(qrow)[4 + g];      // d = 32 + 8g ..
  } else {
#pragma unroll
    for (int c = 0; c < 4; c++) qf[c] = reinterpret_cast<const u32x4_t*>(qrow)[4 * g + c];   // d = 16g + 4c ..
  }

  f32x4_t o[4];
#pragma unroll
  for (int db = 0; db < 4; db++) o[db] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  for (int k0 = lo; k0 < hi; k0 += 64) {
    // ---- stage K rows and V^T rows of keys [k0, k0 + 64) ----
#pragma unroll
    for (int it = 0; it < (64 * CPR) / 256; it++) {
      const int idx = tid + it * 256;
      const int kr = idx / CPR, ch = idx % CPR;
      const int key = min(k0 + kr, len - 1);
      Ks[kr * CPR + (ch ^ (kr % CPR))] =
          reinterpret_cast<const u32x4_t*>(K + (size_t)(base + key) * ldqk + h * HD)[ch];
      const int d = kr;                                  // V^T row d, chunk ch covers keys ch*EPC ..
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(Vt + (size_t)(h * HD + d) * ldv + vb + k0 + ch * EPC);
      if constexpr (sizeof(T) == 2) {
        // 8-byte units (4 keys) swizzled by d so 16 lanes reading 16 rows hit distinct banks
        u32x2_t* vrow = reinterpret_cast<u32x2_t*>(&Vs[d * CPR]);
        vrow[(2 * ch) ^ (d & 15)] = (u32x2_t){v.x, v.y};
        vrow[(2 * ch + 1) ^ (d & 15)] = (u32x2_t){v.z, v.w};
      } else {
        Vs[d * CPR + (ch ^ (d & 15))] = v;
      }
    }
    __syncthreads();

    // ---- S^T = K Q^T for 4 sub-blocks of 16 keys ----
    f32x4_t st[4];
#pragma unroll
    for (int kb = 0; kb < 4; kb++) {
      st[kb] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
      const int kr = kb * 16 + l16;
      if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int s = 0; s < 2; s++) {
          const u32x4_t kf = Ks[kr * CPR + ((4 * s + g) ^ (kr % CPR))];
          st[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kf),
                                                           __builtin_bit_cast(bf16x8_t, qf[s]), st[kb], 0, 0, 0);
        }
      } else {
#pragma unroll
        for (int c = 0; c < 4; c++) {
          const f32x4_t kf = __builtin_bit_cast(f32x4_t, Ks[kr * CPR + ((4 * g + c) ^ (kr % CPR))]);
          const f32x4_t qv = __builtin_bit_cast(f32x4_t, qf[c]);
#pragma unroll
          for (int u = 0; u < 4; u++) st[kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[u], qv[u], st[kb], 0, 0, 0);
        }
      }
    }

    // ---- mask, online softmax (lane-local query; 4 lane groups share it) ----
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 4; kb++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int j = k0 + kb * 16 + 4 * g + i;
        const bool ok = j < len && (window_half == 0 || abs(p - j) <= window_half);
        const float v = ok ? st[kb][i] * scale : -INFINITY;
        st[kb][i] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    float alpha = 1.f, rs = 0.f;
    if (m_new != -INFINITY) {
      alpha = __expf(m_run - m_new);
#pragma unroll
      for (int kb = 0; kb < 4; kb++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const float e = st[kb][i] == -INFINITY ? 0.f : __expf(st[kb][i] - m_new);
          st[kb][i] = e;
          rs += e;
        }
    } else {
#pragma unroll
      for (int kb = 0; kb < 4; kb++) st[kb] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
    }
    rs += __shfl_xor(rs, 16, 64);
    rs += __shfl_xor(rs, 32, 64);
    l_run = l_run * alpha + rs;
    m_run = m_new;
#pragma unroll
    for (int db = 0; db < 4; db++) o[db] *= alpha;

    // ---- O^T += V^T P^T ----
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int t = 0; t < 2; t++) {
        // B operand: keys 32t + 4g + (0..3) and 32t + 16 + 4g + (0..3) of this lane's query
        bf16x8_t pb;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          pb[i] = (__bf16)st[2 * t][i];
          pb[4 + i] = (__bf16)st[2 * t + 1][i];
        }
#pragma unroll
        for (int db = 0; db < 4; db++) {
          const int d = db * 16 + l16;
          const u32x2_t* vrow = reinterpret_cast<const u32x2_t*>(&Vs[d * CPR]);
          const u32x2_t u0 = vrow[(8 * t + g) ^ (d & 15)];
          const u32x2_t u1 = vrow[(8 * t + 4 + g) ^ (d & 15)];
          const u32x4_t va = (u32x4_t){u0.x, u0.y, u1.x, u1.y};
          o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, va), pb, o[db], 0, 0, 0);
        }
      }
    } else {
#pragma unroll
      for (int kb = 0; kb < 4; kb++)
#pragma unroll
        for (int db = 0; db < 4; db++) {
          const int d = db * 16 + l16;
          const f32x4_t va = __builtin_bit_cast(f32x4_t, Vs[d * CPR + ((4 * kb + g) ^ (d & 15))]);  // keys 16kb+4g+0..3
#pragma unroll
          for (int u = 0; u < 4; u++) o[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(va[u], st[kb][u], o[db], 0, 0, 0);
        }
    }
    __syncthreads();
  }

  if (!qvalid) return;
  // o[db][i] = O^T[d = 16db + 4g + i][query]; write 4 consecutive d per block
  const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
  T* orow_p = O + (size_t)orow * ldo + h * HD;
#pragma unroll
  for (int db = 0; db < 4; db++) {
    const int d = db * 16 + 4 * g;
    if constexpr (sizeof(T) == 2) {
      u32x2_t u;
      u[0] = (uint32_t)f2bf(o[db][0] * inv) | ((uint32_t)f2bf(o[db][1] * inv) << 16);
      u[1] = (uint32_t)f2bf(o[db][2] * inv) | ((uint32_t)f2bf(o[db][3] * inv) << 16);
      *reinterpret_cast<u32x2_t*>(orow_p + d) = u;
    } else {
      *reinterpret_cast<float4*>(orow_p + d) = make_float4(o[db][0] * inv, o[db][1] * inv, o[db][2] * inv, o[db][3] * inv);
    }
  }
}

__device__ __forceinline__ uint32_t lds_addr_a(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// ======================================================================================
// bf16 attention (v_mfma_f32_32x32x16_bf16).  One workgroup of NW waves owns one query tile (<= 32 NW
// queries of one sequence) of one head; each wave owns 32 queries, so every K and V^T fragment read
// from LDS feeds a 32-query MFMA.  The engine runs NW = 2 (64-query tiles) in sliding-window layers
// and NW = 4 (128-query tiles, four waves per SIMD) in global ones: a 128-query tile fetches each
// key block once per 128 queries (global layers 5% faster), but walks 256 keys for 128 queries in a
// sliding-window layer instead of 192 for 64 (3% slower there: a tile's blocks run one after
// another, and half as many workgroups hide less of each block's fetch latency).  A query's blocks are the same in both
// tilings but for blocks masked for every query of its wave, which add exact zeros and move no
// maximum, so both give the same bits.  Keys advance in blocks of 64, fetched by LDS DMA
// (inline assembly, as in the GEMM): the next block's K while the current block is scored, the next
// block's V^T (one buffer) after the current PV step, each published by one wait and one barrier.
//
//   S^T[key][query] = K Q^T   A = K rows (32 keys x 16 d per MFMA), B = Q rows (registers)
//   O^T[d][query] += V^T P^T  A = V^T rows (32 d x 16 keys),       B = P^T from the S^T registers
//
// The 32x32 accumulator gives lane l query l % 32 and rows 8 (e / 4) + 4 (l / 32) + e % 4 of a
// 32-key sub-block; the K operand's rows are permuted so that these rows are keys
// 16 (e / 8) + 8 (l / 32) + e % 8.  Lanes l and l ^ 32 together hold a query's 64 scores: the row
// max takes one cross-lane step, and each lane sums its half of the probabilities, added to the
// other half's at the end.  Eight accumulator elements (e = 8 h' .. 8 h' + 7) are the B operand of one 16-key PV
// step with k-index i <-> key 16 h' + i, so the V^T operand of that step is one 16-byte LDS read per
// lane.  Scores are scaled into the log2 domain once (exp2).  Global layers' blocks but the last
// partial one skip the mask; sliding-window blocks all take it.
// ======================================================================================
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// LDS DMA of one 16-byte chunk per lane (see the GEMM's dma16: the LDS base is an operand bound
// to M0, the whole offset is range-checked, the memory clobber orders it against LDS reads)
__device__ __forceinline__ void attn_dma16(u32x4_t rsrc, uint32_t lds, uint32_t voff) {
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "{m0}"(lds), "v"(voff), "s"(rsrc)
               : "memory");
}

__device__ __forceinline__ u32x4_t attn_rsrc(const void* p, uint32_t bytes) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  u32x4_t r;
  r[0] = (uint32_t)v;
  r[1] = (uint32_t)(v >> 32) & 0xFFFFu;
  r[2] = bytes;
  r[3] = 0x00020000u;
  return r;
}

// Optional per-workgroup timeline (-DLAYA_TILE_TRACE, liblaya_trace.so only): thread 0 records at
// exit, at index blockIdx.y * gridDim.x + blockIdx.x: start and end on the 100 MHz real-time clock,
// shader cycles from entry to exit, key blocks processed, tile index and head, the cycles wave 0
// spent in the two waits of the key loop, its hardware id and the cycles before the first block.
#ifdef LAYA_TILE_TRACE
constexpr int kAttnTraceMax = 65536;
__device__ unsigned long long g_attn_trace[8 * kAttnTraceMax];
struct AttnTrace {
  unsigned long long t0, r0, ta = 0, t1 = 0, wv = 0, wk = 0, tw = 0;
  int blocks = 0;
  __device__ void wait_begin() { if (threadIdx.x == 0) tw = __builtin_amdgcn_s_memtime(); }
  __device__ void wait_end(unsigned long long& acc) {
    if (threadIdx.x == 0) acc += __builtin_amdgcn_s_memtime() - tw;
  }
  __device__ AttnTrace() : t0(__builtin_amdgcn_s_memtime()), r0(__builtin_amdgcn_s_memrealtime()) {}
  __device__ ~AttnTrace() {
    const unsigned idx = blockIdx.y * gridDim.x + blockIdx.x;
    if (threadIdx.x != 0 || idx >= (unsigned)kAttnTraceMax) return;
    const unsigned long long t3 = __builtin_amdgcn_s_memtime(), r3 = __builtin_amdgcn_s_memrealtime();
    unsigned hw, xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    unsigned long long* p = g_attn_trace + 8 * (size_t)idx;
    p[0] = r0; p[1] = r3; p[2] = t3 - t0; p[3] = (unsigned)blocks;
    p[4] = ((unsigned long long)blockIdx.y << 32) | blockIdx.x; p[5] = (wv << 32) | (wk & 0xFFFFFFFFull);
    p[6] = ((unsigned long long)xcc << 32) | hw; p[7] = ((ta ? ta - t0 : 0) << 32) | (t1 ? t1 - t0 : 0);
  }
};
#endif

template <int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(NW == 4 ? 4 : 3, 8))) void k_attention_bf16(const bf16_t* __restrict__ Q, const bf16_t* __restrict__ K,
                                                        int ldqk, int kv_rows, const bf16_t* __restrict__ Vt, int ldv,
                                                        int vt_rows, bf16_t* __restrict__ O, int ldo,
                                                        const AttnTile* __restrict__ tiles, const int* __restrict__ soff,
                                                        const int* __restrict__ vlen, const int* __restrict__ gq,
                                                        const int* __restrict__ grow, int window_half, float scale) {
  constexpr int HD = 64;
  constexpr int J = 8 / NW;                                // DMA instructions per wave per block
  static_assert(NW == 2 || NW == 4, "two or four waves");
  // [buffer][row][8 chunks of 16 bytes]: K rows are keys, V^T rows are d; chunk c of row r sits at
  // position c ^ ((r >> 1) & 7), so 16 lanes reading one chunk of 16 consecutive rows hit 16
  // distinct 16-byte bank positions
  // K is double-buffered (the next block's K is fetched while the current one is used); V^T has
  // one buffer, refilled right after the PV step and landing while the next block's scores and
  // softmax run.  24 KB per workgroup: six two-wave workgroups fit a CU (LDS, and three waves per
  // SIMD within the 168-VGPR limit), four four-wave ones (four waves per SIMD in 128 VGPRs).
  __shared__ u32x4_t Ks0[64 * 8], Ks1[64 * 8], Vs[64 * 8];

#ifdef LAYA_TILE_TRACE
  AttnTrace at;
#endif
  // heads are the fastest grid dimension, so the (longest-first) tiles start in order
  const AttnTile tile = tiles[blockIdx.y];
  if (tile.nq <= 0) return;                               // an empty tile of the pass's tile capacity
  const int h = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, hi = lane >> 5;
  const int b = tile.seq, len = vlen[b], base = soff[b];
#ifdef LAYA_TILE_TRACE
  asm volatile("s_waitcnt lgkmcnt(0)" ::"s"(len), "s"(base) : "memory");
  if (threadIdx.x == 0) at.ta = __builtin_amdgcn_s_memtime();
#endif

  // this lane's query (32 per wave)
  const int r = wave * 32 + l32;
  const bool qvalid = r < tile.nq;
  const int rr = qvalid ? r : 0;
  int p, orow;
  if (gq) { const int gi = gq[tile.q0 + rr]; p = grow[gi] - base; orow = gi; }
  else { p = tile.q0 + rr; orow = base + p; }

  // key range of the tile
  int lo = 0, hi_k = len;
  if (window_half > 0 && !gq) {
    const int pmin = tile.q0, pmax = tile.q0 + tile.nq - 1;
    lo = max(0, pmin - window_half) & ~15;
    hi_k = min(len, pmax + window_half + 1);
  }

  // keys visible to this lane's query: [jlo, jhi).  Both bounds grow with the query, so every
  // query of the tile sees [jlo_all, jhi_all): its last query's lower bound, its first one's upper.
  const bool win = window_half > 0 && !gq;
  const int jlo = win ? max(0, p - window_half) : 0;
  const int jhi = win ? min(len, p + window_half + 1) : len;
  const int jlo_all = win ? max(0, tile.q0 + tile.nq - 1 - window_half) : 0;
  const int jhi_all = win ? min(len, tile.q0 + window_half + 1) : len;

  // Q fragments (B operand): query row, d = 16 s + 8 hi .. + 7.  Loaded by inline assembly, so
  // that the compiler's wait analysis does not count them: the wait before the key loop below
  // (which is also what defines qf for the compiler) lets the first V^T block stay in flight.
  const char* qa = reinterpret_cast<const char*>(Q + (size_t)(base + p) * ldqk + h * HD) + 16 * hi;
  u32x4_t qf[4];
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(qf[0]) : "v"(qa) : "memory");
  asm volatile("global_load_dwordx4 %0, %1, off offset:32" : "=v"(qf[1]) : "v"(qa) : "memory");
  asm volatile("global_load_dwordx4 %0, %1, off offset:64" : "=v"(qf[2]) : "v"(qa) : "memory");
  asm volatile("global_load_dwordx4 %0, %1, off offset:96" : "=v"(qf[3]) : "v"(qa) : "memory");

  // DMA plan: instruction j (0..J-1 per wave) fills the 8 rows 8 g .. + 7 of the K block and of
  // the V^T block, g = (wave & 1) + 2 (j + J (wave >> 1)); lane -> row 8 g + lane / 8, position
  // lane % 8 (global chunk position ^ swizzle).  A wave's groups g all have the parity of its
  // wave, so its lanes' swizzle is the same in all of them and instruction j's offset is the
  // first one's plus 16 j rows: one offset register per operand.
  const u32x4_t rK = attn_rsrc(K, (uint32_t)((size_t)kv_rows * ldqk * 2));
  const u32x4_t rV = attn_rsrc(Vt, (uint32_t)((size_t)vt_rows * ldv * 2));
  const int g0 = (wave & 1) + 2 * J * (wave >> 1);
  const int row0 = 8 * g0 + (lane >> 3), c0 = (lane & 7) ^ ((row0 >> 1) & 7);
  const uint32_t kvo = ((uint32_t)(base + row0) * (uint32_t)ldqk + (uint32_t)(h * HD)) * 2u + (uint32_t)c0 * 16u;
  const uint32_t vvo = ((uint32_t)(h * HD + row0) * (uint32_t)ldv + (uint32_t)base) * 2u + (uint32_t)c0 * 16u;
  const uint32_t wsl = (uint32_t)__builtin_amdgcn_readfirstlane(g0) * 1024u;
  auto fetch_k = [&](int k0, u32x4_t* ks) {
#pragma unroll
    for (int j = 0; j < J; j++)
      attn_dma16(rK, lds_addr_a(ks) + wsl + j * 2048, kvo + (uint32_t)(k0 + 16 * j) * (uint32_t)ldqk * 2u);
  };
  auto fetch_v = [&](int k0) {
#pragma unroll
    for (int j = 0; j < J; j++)
      attn_dma16(rV, lds_addr_a(Vs) + wsl + j * 2048, vvo + (uint32_t)(16 * j) * (uint32_t)ldv * 2u + (uint32_t)k0 * 2u);
  };

  f32x16_t o[2];
#pragma unroll
  for (int e = 0; e < 16; e++) {
    o[0][e] = 0.f;
    o[1][e] = 0.f;
  }
  // m_run: a trailing running max of the raw scores (scale > 0 keeps the order); probabilities are
  // exp2(s * c - m * c) with c = scale * log2(e), one FMA per score.  The running sum of the
  // probabilities is summed over exactly the bf16 values that the PV product uses, two at a time
  // (v_dot2c_f32_bf16 with (1, 1): a bf16 pair's sum added in fp32), into two partial sums per lane
  // (even and odd pairs): lane l holds the keys 8 (l / 32) .. + 7 of each 16-key step, so a
  // query's sum is lane l's plus lane l ^ 32's, taken once at the end.
  float lsum[2] = {0.f, 0.f};
  float m_run = -INFINITY;
  constexpr float kLazyLog2 = 8.f;
  const bf16x2_t one2 = {(__bf16)1.f, (__bf16)1.f};
  const float c2 = scale * 1.44269504088896340736f;

  fetch_k(lo, Ks0);
  fetch_v(lo);
  // Q and the first K block have landed (this wave's part); the first V^T block (the last J loads)
  // may still be in flight: the first block waits for it before its PV step, so it lands while
  // that block's scores and softmax run.  Loads complete in issue order.  The wait redefines qf,
  // so no use of the Q registers can move above it.
  if constexpr (J == 4)
    asm volatile("s_waitcnt vmcnt(4)" : "+v"(qf[0]), "+v"(qf[1]), "+v"(qf[2]), "+v"(qf[3]) : : "memory");
  else
    asm volatile("s_waitcnt vmcnt(2)" : "+v"(qf[0]), "+v"(qf[1]), "+v"(qf[2]), "+v"(qf[3]) : : "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  // Key order of the score MFMA: its A row m (lane m of the K operand) is key pk(m) of the 32-key
  // sub-block, pk(8 a + 4 h + c) = 16 (a / 2) + 8 h + 4 (a % 2) + c.  Score element e of lane l
  // then holds key 16 (e / 8) + 8 (l / 32) + e % 8, so the eight elements that form the B operand
  // of a 16-key PV step are the eight consecutive keys at k-indices 8 (l / 32) .. + 7, and the V^T
  // operand of that step is one 16-byte chunk of each d row.
  const int krow = 16 * ((l32 >> 3) >> 1) + 8 * ((l32 >> 2) & 1) + 4 * ((l32 >> 3) & 1) + (l32 & 3);
  const int ksw = (krow >> 1) & 7;                         // swizzle of K rows 32 n + krow
  // One 64-key block: S^T = K Q^T, online softmax with the per-query key range, O^T += V^T P^T.
  // MASK says which bounds of the range may cut into the block: 0 none, 2 the upper only, 3 both.
  // The upper bound alone costs a compare and a select per score; both bounds, a subtract more.
  // Each MASK is a separate copy of the whole block, so that the scores go from the MFMA to the
  // softmax in the registers the MFMA wrote them to.
  auto block = [&](auto mask, int k0, bool first, bool more, const u32x4_t* ks) {
    constexpr int MASK = decltype(mask)::value;
    // this lane's visible keys relative to key k0 + 8 hi, the first of its score elements
    const int A = jlo - k0 - 8 * hi, B = jhi - k0 - 8 * hi;
    f32x16_t st[2];
#pragma unroll
    for (int kb = 0; kb < 2; kb++) {
#pragma unroll
      for (int e = 0; e < 16; e++) st[kb][e] = 0.f;
#pragma unroll
      for (int s = 0; s < 4; s++) {
        const u32x4_t kf = ks[(32 * kb + krow) * 8 + ((2 * s + hi) ^ ksw)];
        st[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, kf),
                                                         __builtin_bit_cast(bf16x8_t, qf[s]), st[kb], 0, 0, 0);
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        if constexpr (MASK != 0) {
          // element e holds key k0 + 8 hi + c
          const int c = 32 * kb + 16 * (e >> 3) + (e & 7);
          bool vis;
          if constexpr (MASK == 3) vis = (unsigned)(c - A) < (unsigned)(B - A);
          else vis = c < B;
          st[kb][e] = vis ? st[kb][e] : -INFINITY;
        }
        mx = fmaxf(mx, st[kb][e]);
      }
    {
      // lanes l and l ^ 32 hold one query's scores: v_permlane32_swap gives every lane the value
      // of lane l % 32 and of lane 32 + l % 32 (a VALU exchange; a shuffle would go through LDS)
      const auto hl = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
      mx = fmaxf(__uint_as_float(hl[0]), __uint_as_float(hl[1]));
    }
    // m_run, the exponent's reference, trails the running max: it moves (to every lane's max, with
    // the running output and sum rescaled) only when some valid query's max exceeds it by more
    // than 2^kLazyLog2 in probability, so probabilities stay at most 2^kLazyLog2 and most blocks
    // skip the 48 multiplies of the rescale.  The first block has nothing to rescale.  Lanes past
    // the tile's last query stand in for its first query and do not vote, so the points where a
    // wave moves m_run depend on its own queries only, whatever the tile size; the stand-ins track
    // their own max (their output is dropped).
    if (first) {
      m_run = mx;
    } else if (__any(qvalid && (mx - m_run) * c2 > kLazyLog2)) {
      // (m_run = -inf with a visible key: +inf > kLazyLog2; with none: NaN, no vote)
      const float m_new = fmaxf(m_run, mx);
      const float alpha = __builtin_amdgcn_exp2f(fmaf(m_run, c2, m_new == -INFINITY ? 0.f : -m_new * c2));
      lsum[0] *= alpha;
      lsum[1] *= alpha;
#pragma unroll
      for (int db = 0; db < 2; db++) o[db] *= alpha;
      m_run = m_new;
    }
    if (!qvalid) m_run = fmaxf(m_run, mx);
    // with no visible key yet (m_run = -inf) every exp2 below is exp2(-inf) = 0
    const float mc = m_run == -INFINITY ? 0.f : m_run * c2;
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int e = 0; e < 16; e++) st[kb][e] = __builtin_amdgcn_exp2f(fmaf(st[kb][e], c2, -mc));

    // this block's V^T (fetched after the previous PV step, before the K fetch) has landed in
    // every wave's part
#ifdef LAYA_TILE_TRACE
    at.wait_begin();
#endif
    if (more) {
      if constexpr (J == 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
      else asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
#ifdef LAYA_TILE_TRACE
    at.wait_end(at.wv);
#endif

    // ---- O^T += V^T P^T: four 16-key steps; step kk covers keys 16 kk + 8 hi + (0..7) in lane l ----
#pragma unroll
    for (int kk = 0; kk < 4; kk++) {
      const f32x16_t& sp = st[kk >> 1];
      const int e0 = 8 * (kk & 1);
      bf16x8_t pb;
#pragma unroll
      for (int i = 0; i < 8; i++) pb[i] = (__bf16)sp[e0 + i];
#pragma unroll
      for (int db = 0; db < 2; db++) {
        const int d = 32 * db + l32;
        const u32x4_t va = Vs[d * 8 + ((2 * kk + hi) ^ ((d >> 1) & 7))];
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, va), pb, o[db], 0, 0, 0);
      }
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const bf16x2_t pr = {pb[2 * q], pb[2 * q + 1]};
        lsum[q & 1] = __builtin_amdgcn_fdot2_f32_bf16(pr, one2, lsum[q & 1], false);
      }
    }
  };

  // One pass of the loop below: the block at k0 (K in buffer `it` % 2), then the fetches of the
  // next one.  Each call site of `block` holds its own copy of the whole block (no score register
  // is shared between copies).
  int it = 0, k0 = lo;
#ifdef LAYA_TILE_TRACE
  if (threadIdx.x == 0) at.t1 = __builtin_amdgcn_s_memtime();
#endif
  auto step = [&](auto mask) {
    const bool odd = it & 1;
    const u32x4_t* ks = odd ? Ks1 : Ks0;
    const bool more = k0 + 64 < hi_k;
    // the other K buffer was last read by the previous block's scores, before its final barrier
    if (more) fetch_k(k0 + 64, odd ? Ks0 : Ks1);
    block(mask, k0, it == 0, more, ks);
    // the next block's K has landed (this wave's part) and no wave still reads V^T or this K
#ifdef LAYA_TILE_TRACE
    at.wait_begin();
#endif
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
#ifdef LAYA_TILE_TRACE
    at.wait_end(at.wk);
#endif
    if (more) fetch_v(k0 + 64);
    k0 += 64;
    ++it;
#ifdef LAYA_TILE_TRACE
    at.blocks = it;
#endif
  };
  // Three runs of blocks: those cut by the lower bound of some query's range (a sliding tile's
  // first; they may be cut by the upper bound too, in a short question), those visible to every
  // query (all of a global tile's but a last partial one; a sliding tile's middle one) and those
  // cut only by the upper bound (a sliding tile's last, a global tile's partial last).  Three
  // loops, not one loop choosing among the copies: with both copies in one loop body the
  // registers no longer fit three waves per SIMD.
  while (k0 < hi_k && k0 < jlo_all) step(std::integral_constant<int, 3>{});
  while (k0 + 64 <= jhi_all) step(std::integral_constant<int, 0>{});
  while (k0 < hi_k) step(std::integral_constant<int, 2>{});

  // the query's sum: this lane's and lane l ^ 32's (v_permlane32_swap, with every lane still
  // active: the values of lanes l % 32 and 32 + l % 32, added in that order in both lanes)
  const float lh = lsum[0] + lsum[1];
  const auto lp = __builtin_amdgcn_permlane32_swap(__float_as_uint(lh), __float_as_uint(lh), false, false);
  const float l_run = __uint_as_float(lp[0]) + __uint_as_float(lp[1]);
  if (!qvalid) return;
  // o[db][e] = O^T[d = 32 db + 8 (e / 4) + 4 hi + e % 4][query]: 4 consecutive d per e / 4
  const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
  bf16_t* orow_p = O + (size_t)orow * ldo + h * HD;
#pragma unroll
  for (int db = 0; db < 2; db++)
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const int d = 32 * db + 8 * g + 4 * hi;
      u32x2_t u;
      u[0] = (uint32_t)f2bf(o[db][4 * g + 0] * inv) | ((uint32_t)f2bf(o[db][4 * g + 1] * inv) << 16);
      u[1] = (uint32_t)f2bf(o[db][4 * g + 2] * inv) | ((uint32_t)f2bf(o[db][4 * g + 3] * inv) << 16);
      *reinterpret_cast<u32x2_t*>(orow_p + d) = u;
    }
}

template <typename T>
void launch_attention(const T* Q, const T* K, int ldqk, int kv_rows, const T* Vt, int ldv, T* O, int ldo,
                      const AttnTile* tiles, int ntiles, int qtile, int H, const int* soff, const int* vlen,
                      const int* gq, const int* grow, int window_half, float scale, hipStream_t st) {
  if (ntiles <= 0) return;
  // (128-query tiles give the 64-query tiles' bits only when a sliding window's half width is a
  // multiple of the 64-key block: then both tilings start their key blocks at the same keys)
  if (qtile != 64 && !(qtile == 128 && sizeof(T) == 2 && !gq && window_half % 64 == 0)) {
    fprintf(stderr, "[laya] attention: unsupported query tile %d (window half %d)\n", qtile, window_half);
    exit(1);
  }
  if constexpr (sizeof(T) == 2) {
    if (qtile == 128)
      LAYA_LAUNCH(k_attention_bf16<4>, dim3(H, ntiles), dim3(256), 0, st, Q, K, ldqk, kv_rows, Vt, ldv, H * 64, O,
                         ldo, tiles, soff, vlen, gq, grow, window_half, scale);
    else
      LAYA_LAUNCH(k_attention_bf16<2>, dim3(H, ntiles), dim3(128), 0, st, Q, K, ldqk, kv_rows, Vt, ldv, H * 64, O,
                         ldo, tiles, soff, vlen, gq, grow, window_half, scale);
  } else {
    LAYA_LAUNCH((k_attention<T>), dim3(ntiles, H), dim3(256), 0, st, Q, K, ldqk, Vt, ldv, O, ldo, tiles, soff,
                       vlen, gq, grow, window_half, scale);
  }
}

template void launch_attention<float>(const float*, const float*, int, int, const float*, int, float*, int,
                                      const AttnTile*, int, int, int, const int*, const int*, const int*, const int*,
                                      int, float, hipStream_t);
template void launch_attention<bf16_t>(const bf16_t*, const bf16_t*, int, int, const bf16_t*, int, bf16_t*, int,
                                       const AttnTile*, int, int, int, const int*, const int*, const int*, const int*,
                                       int, float, hipStream_t);

}  // namespace laya

#ifdef LAYA_TILE_TRACE
// the per-workgroup records of the bf16 attention launches since the last clear
extern "C" int laya_attn_trace_read(void* host, size_t records) {
  void* p = nullptr;
  if (records > (size_t)laya::kAttnTraceMax || hipGetSymbolAddress(&p, HIP_SYMBOL(laya::g_attn_trace)) != hipSuccess) return -1;
  return hipMemcpy(host, p, records * 64, hipMemcpyDeviceToHost) == hipSuccess ? 0 : -1;
}
extern "C" int laya_attn_trace_clear() {
  void* p = nullptr;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(laya::g_attn_trace)) != hipSuccess) return -1;
  return hipMemset(p, 0, sizeof(laya::g_attn_trace)) == hipSuccess ? 0 : -1;
}
#endif
