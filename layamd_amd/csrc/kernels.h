// Launchers of the gfx950 kernels.  T is the GEMM/attention storage type: float (fp32 path) or
// bf16_t (bf16 path).  The residual stream is always fp32; 1-D parameters (LayerNorm weights and
// biases, linear biases, type embedding) and the act head are always fp32.
#pragma once
#include <hip/hip_runtime.h>

#include "common.h"
#include "pack.h"

namespace laya {

// ---- LayerNorm family (one wave64 per row) ----
// y = LN(src[row]) * w (+ b) (+ addtab[qt[seq[row]]]); src row = gather ? gather[row] : row.
// Writes y32 (fp32, may alias x) and/or yT (storage type), and with ymr the mean and rstd (eps) of
// each output row, ymr[row * 2 + {0, 1}] (what the GEMMs' LayerNorm fold reads, GemmArgs::ln_mr).
// D % 4 == 0, D <= 2048.
// A split-K residual GEMM's partial products left for the next LayerNorm to add (see
// GemmArgs::partials_only): before normalising row r the kernel forms
//   x' = x + ((p[0][r] + p[1][r] + ... + p[ks - 1][r]) + bias)      (the split-K reduction's order)
// from slices p[k] = p + k * stride (rows of D floats), writes x' to xout (may alias x) and
// normalises x'.
struct PendingPartials {
  const float* p = nullptr;
  int ks = 0;
  size_t stride = 0;
  const float* bias = nullptr;
  float* xout = nullptr;
};
template <typename Tin, typename T>
void launch_layernorm(const Tin* x, const int* gather, int rows, int D, float eps, const float* w, const float* b,
                      const float* addtab, const int* qt, const int* seq, float* y32, T* yT, hipStream_t st,
                      float* ymr = nullptr, const PendingPartials* pend = nullptr);

// The mean and rstd (eps) of each of `rows` rows of width 64 G (G <= 32) from their per-group statistics
// (GemmArgs::stats layout, ldst rows per group), combined in group order:
// mr[row * 2 + {0, 1}] (GemmArgs::ln_mr).
void launch_ln_rowstats(const float* stats, int ldst, int G, int rows, float eps, float* mr, hipStream_t st);
// xg[r] = x[rows[r]] (fp32 rows of width D)
void launch_gather_rows(const float* x, const int* rows, float* xg, int R, int D, hipStream_t st);
// finite pattern in [-1, 1) over n elements (GEMM tuning operands)
template <typename T>
void launch_fill_pattern(T* p, size_t n, uint32_t seed, hipStream_t st);

// ---- MFMA GEMM: C = A[M,K] . W[N,K]^T with a fused epilogue ----
// EPI_PARTIAL is internal to split-K: fp32 partial products of one K chunk, no bias
enum GemmEpi { EPI_STORE = 0, EPI_RESID = 1, EPI_QKV = 2, EPI_GEGLU = 3, EPI_PARTIAL = 4 };
enum GemmAct { ACT_NONE = 0, ACT_RELU = 1, ACT_GELU = 2 };

struct GemmArgs {
  const void* A = nullptr; int lda = 0;          // [M][lda] T
  const void* W = nullptr; int ldw = 0;          // [N][ldw] T ([out,in] weight)
  int M = 0, N = 0, K = 0;
  const float* bias = nullptr;                   // [N] in stored column order, or null
  int act = ACT_NONE;                            // EPI_STORE only
  void* C = nullptr; int ldc = 0;                // EPI_STORE: [M][ldc] T; EPI_GEGLU: [M][ldc] T, N/2 wide
  float* X = nullptr; int ldx = 0;               // EPI_RESID: X[M][ldx] += result
  // EPI_QKV: columns [q | k | v], each H*HD wide; q and k get RoPE when rope_cos != null
  void* Q = nullptr; void* Kt = nullptr; int ldqk = 0;
  void* Vt = nullptr; int ldv = 0;               // V^T [H*HD][ldv], column = row
  int H = 0, HD = 0;
  const int* pos = nullptr;                      // RoPE position of each row
  const float* rope_cos = nullptr; const float* rope_sin = nullptr;  // [positions][HD/2]
  int cfg = -1;                                  // bf16 tile configuration (-1: the planner's pick)
  // rows [split_rows, M) run as a second launch with configuration cfg_tail (0: one launch); the
  // first launch then covers whole rounds of large tiles and the second the few rows left over
  int split_rows = 0, cfg_tail = -1;
  // split-K (bf16 EPI_STORE / EPI_RESID): K in ksplit chunks of whole 64-deep stages (equal when
  // ksplit divides K / 64, else ceil(K / 64 / ksplit) stages each and a shorter last one) whose
  // fp32 partial products go to the workspace ws (ws_bytes; rows are processed in chunks that fit
  // it) and are summed in chunk order, then bias, activation or the residual add.  The result of a row depends on ksplit, not
  // on M, so a call site that always passes the same ksplit stays independent of the batch.
  int ksplit = 1;
  float* ws = nullptr;
  size_t ws_bytes = 0;
  // K chunks of whole 64-deep stages: ceil(stages / ksplit) each, the last one shorter when ksplit
  // does not divide the stage count (set by the split-K launcher: kfull = the full K, K = a chunk)
  int kfull = 0;
  // EPI_RESID split-K whose M rows fit the workspace in one piece: write the partial products
  // (gemm_splitk_chunks(K, ksplit) slices of M x N floats at ws, slice k at ws + k M N) and leave
  // their reduction and the residual add to the next LayerNorm (PendingPartials); otherwise ignored
  bool partials_only = false;
  // LayerNorm folded across two GEMMs (bf16 tiled kernel only; not with split-K).
  //   Producer, EPI_RESID (N % 64 == 0): besides X, writes Xh [M][ldxh] = bf16 of the updated X
  //   and, per row and 64-column group g, the group's sum and its sum of squared deviations from
  //   the group mean, stats[(g * ldst + row) * 2 + {0, 1}] (group-major: a group's rows are
  //   contiguous), each computed in one fixed order whatever the tile shape.  launch_ln_rowstats
  //   then combines a row's groups into its mean and rstd.
  //   Consumer (EPI_STORE, EPI_QKV, EPI_GEGLU): A is the producer's Xh (LayerNorm input rows) and
  //   W holds the weight rows pre-scaled by the LayerNorm weight; with mean m and rstd r of row i
  //   (ln_mr[i * 2 + {0, 1}]) the product becomes r * (acc - m * ln_c[n]) before bias and
  //   activation, ln_c[n] = the sum of W's row n.  That is LN(x) w . W^T exactly in real
  //   arithmetic; a LayerNorm bias b enters through the caller's bias (W . b).
  bf16_t* Xh = nullptr; int ldxh = 0;
  float* stats = nullptr;
  int ldst = 0;                                  // rows per group in stats (>= M)
  const float* ln_mr = nullptr;
  const float* ln_c = nullptr;
};

template <typename T>
void launch_gemm(int epi, const GemmArgs& a, hipStream_t st);
bool gemm_shape_ok(int epi, const GemmArgs& a, int elt_bytes, const char** why);
// pins the bf16 tile configuration for later launches, process-wide (-1: none, the caller's or the
// planner's choice; 0..8: 256x256, 256x128,
// 128x256, 128x128, 192x256, 160x256, 128x192, 192x128, 128x64); returns the previous setting
int gemm_config(int cfg);
int gemm_pinned();                               // the pinned configuration, or -1
// row split used together with the pinned configuration: rows [split_rows, M) run as a second
// launch with cfg_tail (split_rows 0: none)
void gemm_pin_split(int split_rows, int cfg_tail);
// split-K factor applied to later bf16 EPI_STORE / EPI_RESID launches that name none (<= 1: none);
// returns the previous one
int gemm_pin_ksplit(int ks);
constexpr int kGemmConfigs = 9;
// the number of K chunks a split-K launch with factor ks uses for this K (whole 64-deep stages,
// ceil(stages / ks) per chunk, empty chunks dropped)
inline int gemm_splitk_chunks(int K, int ks) {
  const int stages = K / 64, per = (stages + ks - 1) / ks;
  return (stages + per - 1) / per;
}
// the achievable-MFMA probe: blocks x 4 waves, each iters x 8 MFMAs of 32x32x16 bf16 (32768 flop);
// out holds blocks x 256 floats
void launch_mfma_loop(float* out, int blocks, int iters, hipStream_t st);
// device copy of n16 16-byte chunks (16-byte aligned), non-temporal, on blocks workgroups
void launch_hbm_copy(const void* src, void* dst, size_t n16, int blocks, hipStream_t st);
// whether a bf16 launch of this shape can run tile configuration cfg (false for every cfg when the
// shape needs the generic kernel); the analytic planner's pick for it (-1: generic kernel)
bool gemm_config_valid(int epi, const GemmArgs& a, int cfg);
bool gemm_split_valid(int epi, const GemmArgs& a, int cfg, int split_rows, int cfg_tail);
// tile rows and columns of configuration cfg (0 for an invalid cfg)
int gemm_config_bm(int cfg);
int gemm_config_bn(int cfg);
int gemm_planned(int epi, const GemmArgs& a);

// ---- attention over packed sequences ----
// Query tiles of <= qtile queries from `tiles` (qtile 64, or 128 for bf16 outside gathered mode;
// anything else aborts); gathered mode when gq != null (queries are gathered rows
// grow[gq[tile.q0 + r]], outputs go to row gq[...] of O).  window_half = 0: all keys of the
// sequence; otherwise keys with |i - j| <= window_half.  V^T column = packed row; sequences start
// on 8-row boundaries and V^T has 64 columns of slack after the last row.  Q and K hold kv_rows
// rows; V^T has H * 64 rows.  Tiles with nq = 0 are skipped (a pass pads its tile list to a
// capacity that depends only on its bucket).
template <typename T>
void launch_attention(const T* Q, const T* K, int ldqk, int kv_rows, const T* Vt, int ldv, T* O, int ldo,
                      const AttnTile* tiles, int ntiles, int qtile, int H, const int* soff, const int* vlen,
                      const int* gq, const int* grow, int window_half, float scale, hipStream_t st);

// ---- scorer tail and act head ----
// logits[r] = dot(h[r], w) + b[0]   (fp32 accumulate)
template <typename T>
void launch_row_dot(const T* h, int ldh, const float* w, const float* b, float* logits, int R, int D, hipStream_t st);

// act head per question (ref/rl_common.py:116-123): softmax over its logits -> features
// [top1, top1-top2, H(p)/ln(max(k,2)), max(k,2)/255] ++ cls row -> GELU(W0 . + b0) -> W2 . + b2
// hidden: scratch [B][256] fp32
void launch_act_head(const float* cls, int D, const float* logits, const int* moff, const int* nmark,
                     const float* W0, const float* B0, const float* W2, const float* B2, int n_act, float* out,
                     float* hidden, int B, hipStream_t st);

}  // namespace laya
