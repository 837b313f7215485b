// LayerNorm family, gathers, and the decision head's small kernels for gfx950.
//
// LayerNorm is HBM-bound: one wave64 owns two rows (one above 1024 columns), keeps them in
// registers (D/256 float4 per lane and row), reduces mean and variance with wave shuffles (no
// LDS, no barriers), and writes the normalised rows in one pass.  Four waves per workgroup.
#include "kernels.h"
#include <type_traits>

namespace laya {

static constexpr int kLnMaxChunks = 8;     // D <= 8 * 64 * 4 = 2048

template <typename Tin> struct Ld4;
template <> struct Ld4<float> {
  static __device__ __forceinline__ float4 at(const float* p, int c) { return reinterpret_cast<const float4*>(p)[c]; }
};
template <> struct Ld4<bf16_t> {
  static __device__ __forceinline__ float4 at(const bf16_t* p, int c) {
    uint2 u = reinterpret_cast<const uint2*>(p)[c];
    return make_float4(bf2f(u.x & 0xFFFF), bf2f(u.x >> 16), bf2f(u.y & 0xFFFF), bf2f(u.y >> 16));
  }
};
template <typename T> struct St4;
template <> struct St4<float> {
  static __device__ __forceinline__ void at(float* p, int c, float4 v) { reinterpret_cast<float4*>(p)[c] = v; }
};
template <> struct St4<bf16_t> {
  static __device__ __forceinline__ void at(bf16_t* p, int c, float4 v) {
    uint2 u;
    u.x = (uint32_t)f2bf(v.x) | ((uint32_t)f2bf(v.y) << 16);
    u.y = (uint32_t)f2bf(v.z) | ((uint32_t)f2bf(v.w) << 16);
    reinterpret_cast<uint2*>(p)[c] = u;
  }
};

// Each wave normalises RPW rows; all of their loads are issued before the first reduction so
// every lane keeps 4*RPW 16-byte loads in flight.
template <typename Tin, typename T, int RPW, int NCH, bool MR>
__global__ __launch_bounds__(256) void k_layernorm(const Tin* x, const int* __restrict__ gather, int rows, int D,
                                                   float eps, const float* __restrict__ w, const float* __restrict__ b,
                                                   const float* __restrict__ addtab, const int* __restrict__ qt,
                                                   const int* __restrict__ seq, float* y32,  // may alias x
                                                   T* __restrict__ yT, float* __restrict__ ymr) {
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW;
  const int nc = D >> 2;
  const float invd = 1.0f / (float)D;
  float4 v[RPW][NCH];
  float s[RPW];
#pragma unroll
  for (int q = 0; q < RPW; q++) {
    s[q] = 0.f;
    const int row = row0 + q;
    if (row >= rows) continue;
    const size_t src = gather ? (size_t)gather[row] : (size_t)row;
    const Tin* xr = x + src * D;
#pragma unroll
    for (int j = 0; j < NCH; j++) {
      const int c = lane + 64 * j;
      if (c < nc) v[q][j] = Ld4<Tin>::at(xr, c);
    }
  }
  // the weight, loaded once per wave for its rows, right behind the rows themselves: loaded per row
  // after the reductions, each row waited for its own round trip to L2 (11.6 -> 10.45 us per launch
  // at 9664 x 1024)
  float4 wv[NCH];
#pragma unroll
  for (int j = 0; j < NCH; j++) {
    const int c = lane + 64 * j;
    if (c < nc) wv[j] = reinterpret_cast<const float4*>(w)[c];
  }
#pragma unroll
  for (int q = 0; q < RPW; q++)
#pragma unroll
    for (int j = 0; j < NCH; j++)
      if (lane + 64 * j < nc) s[q] += (v[q][j].x + v[q][j].y) + (v[q][j].z + v[q][j].w);
#pragma unroll
  for (int q = 0; q < RPW; q++) {
    const int row = row0 + q;
    if (row >= rows) break;
    const float mean = wave_sum(s[q]) * invd;
    float qq = 0.f;
#pragma unroll
    for (int j = 0; j < NCH; j++) {
      const int c = lane + 64 * j;
      if (c < nc) {
        const float a = v[q][j].x - mean, bb = v[q][j].y - mean, cc = v[q][j].z - mean, d = v[q][j].w - mean;
        qq += (a * a + bb * bb) + (cc * cc + d * d);
      }
    }
    const float inv = rsqrtf(fmaf(wave_sum(qq), invd, eps));
    const float* add = addtab ? addtab + (size_t)qt[seq[row]] * D : nullptr;
    float4 ov[MR ? NCH : 1];
#pragma unroll
    for (int j = 0; j < NCH; j++) {
      const int c = lane + 64 * j;
      if (c < nc) {
        const float4 ww = wv[j];
        float4 o = make_float4((v[q][j].x - mean) * inv * ww.x, (v[q][j].y - mean) * inv * ww.y,
                               (v[q][j].z - mean) * inv * ww.z, (v[q][j].w - mean) * inv * ww.w);
        if (b) { const float4 bb = reinterpret_cast<const float4*>(b)[c]; o.x += bb.x; o.y += bb.y; o.z += bb.z; o.w += bb.w; }
        if (add) { const float4 aa = reinterpret_cast<const float4*>(add)[c]; o.x += aa.x; o.y += aa.y; o.z += aa.z; o.w += aa.w; }
        if (y32) reinterpret_cast<float4*>(y32 + (size_t)row * D)[c] = o;
        if (yT) St4<T>::at(yT + (size_t)row * D, c, o);
        if constexpr (MR) ov[j] = o;
      }
    }
    if constexpr (MR) {
      // mean and rstd of the output row (two passes over the values kept in registers)
      float os = 0.f;
#pragma unroll
      for (int j = 0; j < NCH; j++)
        if (lane + 64 * j < nc) os += (ov[j].x + ov[j].y) + (ov[j].z + ov[j].w);
      const float om = wave_sum(os) * invd;
      float oq = 0.f;
#pragma unroll
      for (int j = 0; j < NCH; j++)
        if (lane + 64 * j < nc) {
          const float a = ov[j].x - om, bb = ov[j].y - om, cc = ov[j].z - om, d = ov[j].w - om;
          oq += (a * a + bb * bb) + (cc * cc + d * d);
        }
      const float orr = rsqrtf(fmaf(wave_sum(oq), invd, eps));
      if (lane == 0) reinterpret_cast<float2*>(ymr)[row] = make_float2(om, orr);
    }
  }
}

// The same LayerNorm for a row whose residual update a split-K GEMM left as partial products
// (PendingPartials): one workgroup per row, thread t owns 16-byte chunk t of the row (D <= 1024).
// Each thread issues its chunk's loads of x and of all ks partial slices at once (a small pass's
// rows are few, so the latency of those loads is what counts), sums the partials in chunk order,
// adds the bias and then x, exactly as the split-K reduction does, and writes the updated row.
// The mean and variance are summed in the order of k_layernorm (lane l adds its chunks
// l, l + 64, ... in turn, then the wave sum), so the normalised row has the bits it would have had
// after a separate reduction.
constexpr int kPsMaxSlices = 16;
template <typename T>
__global__ __launch_bounds__(256) void k_layernorm_ps(const float* __restrict__ x, int D, float eps,
                                                      const float* __restrict__ w, const float* __restrict__ b,
                                                      const float* __restrict__ addtab, const int* __restrict__ qt,
                                                      const int* __restrict__ seq, float* y32, T* __restrict__ yT,
                                                      PendingPartials pend) {
  __shared__ float part[4][64];
  __shared__ float stat;
  const int row = blockIdx.x, t = threadIdx.x, lane = t & 63, j = t >> 6;
  const int nc = D >> 2, nch = (nc + 63) >> 6;
  const float invd = 1.0f / (float)D;
  const bool own = t < nc;
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (own) {
    const float* pr = pend.p + (size_t)row * D;
    float4 pk[kPsMaxSlices];
#pragma unroll
    for (int k = 0; k < kPsMaxSlices; k++)
      if (k < pend.ks) pk[k] = reinterpret_cast<const float4*>(pr + k * pend.stride)[t];
    v = reinterpret_cast<const float4*>(x + (size_t)row * D)[t];
    float4 acc = pk[0];
#pragma unroll
    for (int k = 1; k < kPsMaxSlices; k++)
      if (k < pend.ks) { acc.x += pk[k].x; acc.y += pk[k].y; acc.z += pk[k].z; acc.w += pk[k].w; }
    if (pend.bias) {
      const float4 bb = reinterpret_cast<const float4*>(pend.bias)[t];
      acc.x += bb.x; acc.y += bb.y; acc.z += bb.z; acc.w += bb.w;
    }
    v.x += acc.x; v.y += acc.y; v.z += acc.z; v.w += acc.w;
    if (pend.xout) reinterpret_cast<float4*>(pend.xout + (size_t)row * D)[t] = v;
  }
  // row sum: chunk sums gathered per lane, added in chunk order, then the wave sum (wave 0)
  part[j][lane] = own ? (v.x + v.y) + (v.z + v.w) : 0.f;
  __syncthreads();
  if (j == 0) {
    float s = 0.f;
    for (int q = 0; q < nch; q++)
      if (lane + 64 * q < nc) s += part[q][lane];
    const float m = wave_sum(s) * invd;
    if (lane == 0) stat = m;
  }
  __syncthreads();
  const float mean = stat;
  float dq = 0.f;
  if (own) {
    const float a = v.x - mean, bb = v.y - mean, cc = v.z - mean, d = v.w - mean;
    dq = (a * a + bb * bb) + (cc * cc + d * d);
  }
  __syncthreads();
  part[j][lane] = dq;
  __syncthreads();
  if (j == 0) {
    float qq = 0.f;
    for (int q = 0; q < nch; q++)
      if (lane + 64 * q < nc) qq += part[q][lane];
    const float inv = rsqrtf(fmaf(wave_sum(qq), invd, eps));
    if (lane == 0) stat = inv;
  }
  __syncthreads();
  const float inv = stat;
  if (!own) return;
  const float* add = addtab ? addtab + (size_t)qt[seq[row]] * D : nullptr;
  const float4 ww = reinterpret_cast<const float4*>(w)[t];
  float4 o = make_float4((v.x - mean) * inv * ww.x, (v.y - mean) * inv * ww.y, (v.z - mean) * inv * ww.z,
                         (v.w - mean) * inv * ww.w);
  if (b) { const float4 bb = reinterpret_cast<const float4*>(b)[t]; o.x += bb.x; o.y += bb.y; o.z += bb.z; o.w += bb.w; }
  if (add) { const float4 aa = reinterpret_cast<const float4*>(add)[t]; o.x += aa.x; o.y += aa.y; o.z += aa.z; o.w += aa.w; }
  if (y32) reinterpret_cast<float4*>(y32 + (size_t)row * D)[t] = o;
  if (yT) St4<T>::at(yT + (size_t)row * D, t, o);
}

// Two rows per wave for rows up to 1024 wide (about 2400 waves for 9.6k rows, 60 VGPRs: eight
// waves per SIMD, so all of them are resident at once).  In the pass a LayerNorm starts cold after
// a GEMM; one row per wave (twice the wave launches) or weights held in registers across the
// reductions (125 VGPRs, half the occupancy) both measured slower there.
template <typename Tin, typename T>
void launch_layernorm(const Tin* x, const int* gather, int rows, int D, float eps, const float* w, const float* b,
                      const float* addtab, const int* qt, const int* seq, float* y32, T* yT, hipStream_t st,
                      float* ymr, const PendingPartials* pend) {
  if (D % 4 || D > kLnMaxChunks * 256) {
    fprintf(stderr, "[laya] layernorm: unsupported width %d\n", D);
    exit(1);
  }
  const bool ps = pend && pend->p && pend->ks > 0;
  if (ps && (!std::is_same<Tin, float>::value || gather || ymr || D > 1024 || pend->ks > kPsMaxSlices ||
             pend->stride < (size_t)rows * D)) {
    fprintf(stderr, "[laya] layernorm: pending split-K partials need fp32 rows up to 1024 wide, at most %d slices, "
                    "no gather, no statistics\n", kPsMaxSlices);
    exit(1);
  }
  if (rows <= 0) return;
  if (ps) {
    if constexpr (std::is_same<Tin, float>::value)
      LAYA_LAUNCH((k_layernorm_ps<T>), dim3(rows), dim3(64 * ((D / 4 + 63) / 64)), 0, st, x, D, eps, w, b, addtab, qt,
                  seq, y32, yT, *pend);
    return;
  }
  auto go = [&](auto mr) {
    constexpr bool MR = decltype(mr)::value;
    if (D <= 1024) {
      constexpr int RPW = 2;
      LAYA_LAUNCH((k_layernorm<Tin, T, RPW, 4, MR>), dim3((rows + 4 * RPW - 1) / (4 * RPW)), dim3(256), 0, st, x,
                         gather, rows, D, eps, w, b, addtab, qt, seq, y32, yT, ymr);
    } else {
      LAYA_LAUNCH((k_layernorm<Tin, T, 1, kLnMaxChunks, MR>), dim3((rows + 3) / 4), dim3(256), 0, st, x, gather, rows,
                         D, eps, w, b, addtab, qt, seq, y32, yT, ymr);
    }
  };
  if (ymr) go(std::true_type{});
  else go(std::false_type{});
}

template void launch_layernorm<float, float>(const float*, const int*, int, int, float, const float*, const float*,
                                             const float*, const int*, const int*, float*, float*, hipStream_t, float*,
                                             const PendingPartials*);
template void launch_layernorm<float, bf16_t>(const float*, const int*, int, int, float, const float*, const float*,
                                              const float*, const int*, const int*, float*, bf16_t*, hipStream_t, float*,
                                              const PendingPartials*);
template void launch_layernorm<bf16_t, bf16_t>(const bf16_t*, const int*, int, int, float, const float*, const float*,
                                               const float*, const int*, const int*, float*, bf16_t*, hipStream_t, float*,
                                               const PendingPartials*);

// One thread per row: the G group pairs (sum, M2) of the row are read group-major (a group's rows
// are contiguous, so a wave's reads of one group are coalesced), all at once for up to 16 groups,
// and combined in group order, M2 = sum over g of (M2_g + (S_g - 64 mean)^2 / 64) (Chan et al.'s
// update for equal group sizes).
template <int GB>
__global__ __launch_bounds__(64) void k_ln_rowstats(const float2* __restrict__ stats, int ldst, int G, int rows,
                                                    float eps, float2* __restrict__ mr) {
  const int row = blockIdx.x * 64 + threadIdx.x;
  if (row >= rows) return;
  float2 p[GB];
#pragma unroll
  for (int g = 0; g < GB; g++) p[g] = g < G ? stats[(size_t)g * ldst + row] : make_float2(0.f, 0.f);
  const float invn = 1.0f / (64.f * (float)G);
  float sum = 0.f;
#pragma unroll
  for (int g = 0; g < GB; g++)
    if (g < G) sum = __fadd_rn(sum, p[g].x);
  const float mean = __fmul_rn(sum, invn);
  float m2 = 0.f;
#pragma unroll
  for (int g = 0; g < GB; g++)
    if (g < G) {
      const float d = fmaf(-64.f, mean, p[g].x);          // group sum - 64 mean
      m2 = __fadd_rn(m2, fmaf(__fmul_rn(d, d), 0.015625f, p[g].y));
    }
  mr[row] = make_float2(mean, rsqrtf(fmaf(m2, invn, eps)));
}

void launch_ln_rowstats(const float* stats, int ldst, int G, int rows, float eps, float* mr, hipStream_t st) {
  if (G < 1 || G > 32 || ldst < rows) {
    fprintf(stderr, "[laya] ln_rowstats: %d groups, %d rows per group for %d rows\n", G, ldst, rows);
    exit(1);
  }
  if (rows <= 0) return;
  auto* sp = reinterpret_cast<const float2*>(stats);
  auto* mp = reinterpret_cast<float2*>(mr);
  // one wave per workgroup: the few hundred waves spread over as many CUs
  if (G <= 16) LAYA_LAUNCH(k_ln_rowstats<16>, dim3((rows + 63) / 64), dim3(64), 0, st, sp, ldst, G, rows, eps, mp);
  else LAYA_LAUNCH(k_ln_rowstats<32>, dim3((rows + 63) / 64), dim3(64), 0, st, sp, ldst, G, rows, eps, mp);
}

// Deterministic finite pattern, uniform in [-1, 1), written over n elements (operands for GEMM
// tuning runs, which must see realistic MFMA power and produce finite results).
template <typename T>
__global__ __launch_bounds__(256) void k_fill_pattern(T* __restrict__ p, size_t n, uint32_t seed) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
    uint32_t h = (uint32_t)i * 0x9E3779B1u ^ seed;
    h ^= h >> 16; h *= 0x7FEB352Du; h ^= h >> 15; h *= 0x846CA68Bu; h ^= h >> 16;
    Elt<T>::st(p + i, (float)(h >> 8) * (2.0f / 16777216.0f) - 1.0f);
  }
}

template <typename T>
void launch_fill_pattern(T* p, size_t n, uint32_t seed, hipStream_t st) {
  if (n == 0) return;
  const size_t blocks = std::min<size_t>((n + 255) / 256, 8192);
  LAYA_LAUNCH(k_fill_pattern<T>, dim3((unsigned)blocks), dim3(256), 0, st, p, n, seed);
}
template void launch_fill_pattern<float>(float*, size_t, uint32_t, hipStream_t);
template void launch_fill_pattern<bf16_t>(bf16_t*, size_t, uint32_t, hipStream_t);

// Lane-strided dot products (scorer tail, act head): a lane's columns c = lane + 64 k are loaded
// kDotBatch at a time, all of a batch's loads in flight together (one memory round trip per batch
// instead of one per column), and accumulated in ascending k, as a plain loop would: the same
// bits, in 12 instead of 17 us for the act head.
constexpr int kDotBatch = 8;

__global__ __launch_bounds__(256) void k_gather_rows(const float* __restrict__ x, const int* __restrict__ rows,
                                                     float* __restrict__ xg, int R, int D) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= R) return;
  const float4* s = reinterpret_cast<const float4*>(x + (size_t)rows[r] * D);
  float4* d = reinterpret_cast<float4*>(xg + (size_t)r * D);
  for (int c = lane; c < D / 4; c += 64) d[c] = s[c];
}

void launch_gather_rows(const float* x, const int* rows, float* xg, int R, int D, hipStream_t st) {
  if (R <= 0) return;
  LAYA_LAUNCH(k_gather_rows, dim3((R + 3) / 4), dim3(256), 0, st, x, rows, xg, R, D);
}

// ---- scorer tail: one wave per row, fp32 accumulation ----
template <typename T>
__global__ __launch_bounds__(256) void k_row_dot(const T* __restrict__ h, int ldh, const float* __restrict__ w,
                                                 const float* __restrict__ b, float* __restrict__ logits, int R, int D) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= R) return;
  const T* hr = h + (size_t)r * ldh;
  float s = 0.f;
  for (int c0 = lane; c0 < D; c0 += 64 * kDotBatch) {
    float hv[kDotBatch], wv[kDotBatch];
#pragma unroll
    for (int k = 0; k < kDotBatch; k++) {
      const int c = c0 + 64 * k;
      hv[k] = c < D ? Elt<T>::ld(hr + c) : 0.f;
      wv[k] = c < D ? w[c] : 0.f;
    }
#pragma unroll
    for (int k = 0; k < kDotBatch; k++)
      if (c0 + 64 * k < D) s += hv[k] * wv[k];
  }
  s = wave_sum(s);
  if (lane == 0) logits[r] = s + b[0];
}

template <typename T>
void launch_row_dot(const T* h, int ldh, const float* w, const float* b, float* logits, int R, int D, hipStream_t st) {
  if (R <= 0) return;
  LAYA_LAUNCH((k_row_dot<T>), dim3((R + 3) / 4), dim3(256), 0, st, h, ldh, w, b, logits, R, D);
}
template void launch_row_dot<float>(const float*, int, const float*, const float*, float*, int, int, hipStream_t);
template void launch_row_dot<bf16_t>(const bf16_t*, int, const float*, const float*, float*, int, int, hipStream_t);

// ---- act head (ref/rl_common.py:116-123) ----
// p = softmax(logits over the question's markers); k = max(nmark, 2); features [top1,
// top1 - top2, -sum p log(max(p, 1e-9)) / ln k, k / 255]; hidden = GELU(W0 [cls, features] + b0)
// with W0 [256][D + 4]; out = W2 hidden + b2.
// k_act_hidden: grid (B, 16); each wave produces 4 hidden units.  The W0 . cls partial sums are
// issued first (their loads do not depend on the features); then every wave computes the
// question's 4 features itself from its <= 255 logits (lanes over markers, wave reductions), so no
// barrier is needed.  top2 is the second largest probability counted with multiplicity (top1 again
// when the maximum occurs twice), 0 when there is none.
__global__ __launch_bounds__(256) void k_act_hidden(const float* __restrict__ cls, int D, const float* __restrict__ logits,
                                                    const int* __restrict__ moff, const int* __restrict__ nmark,
                                                    const float* __restrict__ W0, const float* __restrict__ B0,
                                                    float* __restrict__ hidden) {
  const int b = blockIdx.x, t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const float* c = cls + (size_t)b * D;
  const int j0 = blockIdx.y * 16 + wv * 4;
  // the feature columns' weights and the biases do not depend on anything: loaded first
  float wf[4], b0[4];
#pragma unroll
  for (int u = 0; u < 4; u++) {
    wf[u] = lane < 4 ? W0[(size_t)(j0 + u) * (D + 4) + D + lane] : 0.f;
    b0[u] = B0[j0 + u];
  }
  // W0 . cls: each lane's columns i = lane + 64 k in ascending k, loaded kDotBatch columns at a time
  // (all loads of a batch in flight together, instead of one round trip per column), accumulated in
  // the same order
  float a[4] = {0.f, 0.f, 0.f, 0.f};
  for (int i0 = lane; i0 < D; i0 += 64 * kDotBatch) {
    float cv[kDotBatch], wv_[4][kDotBatch];
#pragma unroll
    for (int k = 0; k < kDotBatch; k++) {
      const int i = i0 + 64 * k;
      cv[k] = i < D ? c[i] : 0.f;
#pragma unroll
      for (int u = 0; u < 4; u++) wv_[u][k] = i < D ? W0[(size_t)(j0 + u) * (D + 4) + i] : 0.f;
    }
#pragma unroll
    for (int k = 0; k < kDotBatch; k++)
      if (i0 + 64 * k < D) {
#pragma unroll
        for (int u = 0; u < 4; u++) a[u] += wv_[u][k] * cv[k];
      }
  }

  const float* z = logits + moff[b];
  const int K = nmark[b];
  float zl[4], mx = -INFINITY;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int i = lane + 64 * q;
    zl[q] = i < K ? z[i] : -INFINITY;
    mx = fmaxf(mx, zl[q]);
  }
  mx = wave_max(mx);
  float e[4], se = 0.f;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    e[q] = lane + 64 * q < K ? expf(zl[q] - mx) : 0.f;
    se += e[q];
  }
  se = wave_sum(se);
  float p[4], ent = 0.f, t1 = 0.f;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    p[q] = e[q] / se;
    if (lane + 64 * q < K) {
      ent -= p[q] * logf(fmaxf(p[q], 1e-9f));
      t1 = fmaxf(t1, p[q]);
    }
  }
  ent = wave_sum(ent);
  t1 = wave_max(t1);
  float n1 = 0.f, t2 = 0.f;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    if (lane + 64 * q < K) {
      if (p[q] == t1) n1 += 1.f;
      else t2 = fmaxf(t2, p[q]);
    }
  }
  n1 = wave_sum(n1);
  t2 = n1 >= 2.f ? t1 : wave_max(t2);
  const float kf = (float)(K < 2 ? 2 : K);
  const float feat = lane == 0 ? t1 : lane == 1 ? t1 - t2 : lane == 2 ? ent / logf(kf) : kf / 255.f;

#pragma unroll
  for (int u = 0; u < 4; u++) {
    const int j = j0 + u;
    float v = a[u];
    if (lane < 4) v += wf[u] * feat;
    v = wave_sum(v);
    if (lane == 0) hidden[(size_t)b * 256 + j] = gelu_erf(v + b0[u]);
  }
}

// k_act_out: one wave per question, out[b][t] = W2[t] . hidden[b] + b2[t]
__global__ __launch_bounds__(64) void k_act_out(const float* __restrict__ hidden, const float* __restrict__ W2,
                                                const float* __restrict__ B2, int n_act, float* __restrict__ out) {
  const int b = blockIdx.x, lane = threadIdx.x;
  for (int j = 0; j < n_act; j++) {
    float a = 0.f;
    for (int i = lane; i < 256; i += 64) a += W2[(size_t)j * 256 + i] * hidden[(size_t)b * 256 + i];
    a = wave_sum(a);
    if (lane == 0) out[(size_t)b * n_act + j] = a + B2[j];
  }
}

void launch_act_head(const float* cls, int D, const float* logits, const int* moff, const int* nmark, const float* W0,
                     const float* B0, const float* W2, const float* B2, int n_act, float* out, float* hidden, int B,
                     hipStream_t st) {
  if (B <= 0) return;
  LAYA_LAUNCH(k_act_hidden, dim3(B, 16), dim3(256), 0, st, cls, D, logits, moff, nmark, W0, B0, hidden);
  LAYA_LAUNCH(k_act_out, dim3(B), dim3(64), 0, st, hidden, W2, B2, n_act, out);
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));   // one 16-byte chunk

// The achievable HBM rate: a device copy of n16 16-byte chunks.  Each thread of a 256-thread block
// moves four chunks per round (all four loads, then all four stores; consecutive threads on
// consecutive chunks), rounds striding over the grid.  Non-temporal loads and stores: the copy
// has no reuse, and without them the same kernel measured 5.6 against 6.0 TB/s on 1 GiB.
__global__ __launch_bounds__(256) void k_hbm_copy(const u32x4_t* __restrict__ src, u32x4_t* __restrict__ dst,
                                                  size_t n16) {
  const size_t step = (size_t)gridDim.x * 1024;
  for (size_t base = (size_t)blockIdx.x * 1024 + threadIdx.x; base < n16; base += step) {
    u32x4_t v[4];
#pragma unroll
    for (int u = 0; u < 4; u++)
      if (base + 256 * u < n16) v[u] = __builtin_nontemporal_load(src + base + 256 * u);
#pragma unroll
    for (int u = 0; u < 4; u++)
      if (base + 256 * u < n16) __builtin_nontemporal_store(v[u], dst + base + 256 * u);
  }
}

void launch_hbm_copy(const void* src, void* dst, size_t n16, int blocks, hipStream_t st) {
  LAYA_LAUNCH(k_hbm_copy, dim3(blocks), dim3(256), 0, st, static_cast<const u32x4_t*>(src),
                     static_cast<u32x4_t*>(dst), n16);
}

}  // namespace laya
