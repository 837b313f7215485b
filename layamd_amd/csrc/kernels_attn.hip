// Attention over packed variable-length sequences for gfx950 (wave64 MFMA, fp32 online softmax).
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

template <typename T>
void launch_attention(const T* Q, const T* K, int ldqk, const T* Vt, int ldv, T* O, int ldo, const AttnTile* tiles,
                      int ntiles, int H, const int* soff, const int* vlen, const int* gq, const int* grow,
                      int window_half, float scale, hipStream_t st) {
  if (ntiles <= 0) return;
  hipLaunchKernelGGL((k_attention<T>), dim3(ntiles, H), dim3(256), 0, st, Q, K, ldqk, Vt, ldv, O, ldo, tiles, soff,
                     vlen, gq, grow, window_half, scale);
}

template void launch_attention<float>(const float*, const float*, int, const float*, int, float*, int, const AttnTile*,
                                      int, int, const int*, const int*, const int*, const int*, int, float, hipStream_t);
template void launch_attention<bf16_t>(const bf16_t*, const bf16_t*, int, const bf16_t*, int, bf16_t*, int,
                                       const AttnTile*, int, int, const int*, const int*, const int*, const int*, int,
                                       float, hipStream_t);

}  // namespace laya
