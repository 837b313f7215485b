/* Measurement hooks of the MI355X Laya engine.  None of these has a counterpart in the reference
 * ABI (src/laya_api.h); they exist for benchmarking and debugging and are not needed by the
 * reference's callers. */
#pragma once
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Turns per-stage kernel timing on (1) or off (0) at run time.  While on, HIP graphs are bypassed
 * and every kernel a stage launches records its own device start and end time in a pair of HIP
 * events (hipExtLaunchKernel), with no marker or synchronisation between launches; a stage's time
 * is the sum of its kernels' durations, read once the pass has finished.  Returns the previous
 * state. */
int laya_ext_prof_enable(void* h, int on);

/* Stage i of the profile table: copies its name (NUL-terminated, at most name_len bytes), total
 * device milliseconds and number of launches.  Returns 0, or -1 when i is out of range. */
int laya_ext_prof_stage(void* h, int i, char* name, int name_len, double* ms, long long* calls);

/* The stage of every kernel launch of the most recent profiled pass, in launch order: stage
 * indices as laya_ext_prof_stage numbers them, the first cap of them into stages.  Returns the
 * number of launches (0 when no pass ran with profiling on), or -1 for invalid arguments.  Lets a
 * kernel trace of the same pass (graph replays launch the same kernels in the same order) be read
 * per stage. */
int laya_ext_prof_sequence(void* h, int* stages, int cap);

/* Re-runs the most recent pass `iters` times exactly as laya_forward_batch runs it (graph replay
 * when graphs are on) and stores the device time of all iterations, measured with HIP events on
 * the engine's stream, in *ms.  Inputs stay resident; only the pass's small index arrays are
 * re-copied from pinned host memory.  Returns 0, or -1 when no pass has run yet. */
int laya_ext_replay(void* h, int iters, float* ms);

/* "bf16" or "fp32": the storage type of GEMM and attention operands (LAYA_PRECISION). */
const char* laya_ext_precision(void* h);

/* Engine counters, the first n (<= 4) into out: [0] HIP graphs cached (one per pass bucket: rows
 * and marker rows padded to 64, question count), [1] graphs captured so far, [2] tuned GEMM plans,
 * [3] pass buckets whose GEMMs have been tuned.  Returns 0, or -1 for invalid arguments. */
int laya_ext_stats(void* h, long long* out, int n);

/* The engine's attention kernel on caller-owned device buffers, in the engine's packed layout:
 * dtype 0 fp32 / 1 bf16 operands; Q and K [kv_rows][ldqk] (head h at columns 64 h .. 64 h + 63),
 * V^T [H * 64][ldv] with column = packed row, O [..][ldo].  Question b owns rows soff[b] ..
 * soff[b] + vlen[b] - 1 (soff a multiple of 8); V^T must hold 64 columns past the last row of
 * every question.  tiles: ntiles x {question, first query, query count, 0} (int32; count 0 = skip),
 * qtile 64 (or 128 for bf16 outside gathered mode).  Gathered mode when gq and grow are both
 * non-NULL: tile queries are gathered rows gq[first + r], each the packed row grow[gq[...]], and
 * their outputs go to row gq[...] of O.  window_half 0: every key of the question; otherwise keys
 * with |i - j| <= window_half.  Launches on stream (hipStream_t) without waiting.  Returns 0, or
 * -1 for arguments outside these rules. */
int laya_ext_attention(int dtype, const void* Q, const void* K, int ldqk, int kv_rows, const void* Vt, int ldv, void* O,
                       int ldo, const int* tiles, int ntiles, int qtile, int H, const int* soff, const int* vlen,
                       const int* gq, const int* grow, int window_half, float scale, void* stream);

/* The engine's MFMA GEMM on caller-owned device buffers: C[M,N] = A[M,K] . W[N,K]^T.
 * dtype 0: fp32 operands, 1: bf16 operands (fp32 accumulate in both).
 * epi 0: C (dtype) = act(result + bias), act 0 none / 1 ReLU / 2 GELU;
 * epi 1: C is fp32 and C += result + bias.  bias is fp32 [N] or NULL.
 * Runs `iters` (>= 1) launches on `stream` (a hipStream_t, NULL = default stream); when ms is
 * non-NULL stores their total device time from HIP events.  Returns 0, or -1 when the shape or
 * alignment is not supported (K a multiple of 64 bf16 / 32 fp32 elements, 16-byte aligned rows). */
int laya_ext_gemm(int dtype, int epi, const void* A, const void* W, void* C, const float* bias, int act, int M, int N,
                  int K, void* stream, int iters, float* ms);

/* The chip's achievable bf16 MFMA rate: launches (does not wait for) blocks of 4 waves on stream,
 * each issuing iters x 8 independent v_mfma_f32_32x32x16_bf16 on registers (no memory traffic);
 * out is the caller's device buffer of blocks x 256 floats, *flops gets the launch's work.  The
 * caller times it with its own events.  No counterpart in the reference: it gives bench.py the
 * achievable peak next to the published one.  Returns 0, or -1 for invalid arguments. */
int laya_ext_mfma_loop(float* out, int blocks, int iters, void* stream, double* flops);

/* The chip's achievable HBM rate: launches (does not wait for) a copy of bytes from src to dst on
 * stream, non-temporal 16-byte loads and stores from two workgroups per CU striding over the range.
 * The caller times it with its own events (bytes read + bytes written per second).  No counterpart
 * in the reference: it gives bench.py a hand-written copy as the achievable bandwidth next to the
 * published one.  Returns 0, or -1 when bytes is 0 or not a multiple of 16, a pointer is null or
 * not 16-byte aligned, or the ranges overlap. */
int laya_ext_hbm_copy(const void* src, void* dst, size_t bytes, void* stream);

/* Pins the bf16 GEMM tile configuration of every later launch, process-wide: -1 removes the pin
 * (each engine's plans, or its own LAYA_GEMM_CFG read at laya_create, apply); 0..8 select 256x256, 256x128, 128x256, 128x128,
 * 192x256, 160x256, 128x192, 192x128 or 128x64 tiles (the QKV projection falls back to a shape that keeps its tiles inside one of
 * the q/k/v sections).  Passes already captured in HIP graphs keep their kernels.  Returns the
 * previous setting, or -2 for an invalid value. */
int laya_ext_gemm_config(int cfg);

/* Row split used with the pinned configuration: rows [split_rows, M) of every later pinned launch
 * run with tile configuration cfg_tail (0..8), in a second launch, or in the same launch after the
 * first configuration's tiles when that is 192x128 (7) and cfg_tail 128x64 (8) or 128x128 (3) on a
 * store without bias or activation (or a GeGLU GEMM of the engine); split_rows 0 removes the split.
 * A split the shape cannot take (split_rows >= M, not a multiple of 8, a tail configuration the
 * shape cannot use) runs as one launch of the first configuration.  Results are the same bits in
 * every case.  Returns 0, or -2 for an invalid value. */
int laya_ext_gemm_split(int split_rows, int cfg_tail);

/* Split-K factor (0 or 1: none, up to 64) for later bf16 laya_ext_gemm calls, process-wide: K
 * (at least 128) is cut into chunks of whole 64-deep stages, ceil(K / 64 / ks) stages each (the
 * last chunk shorter when ks does not divide K / 64; at most ks chunks), whose fp32 partial
 * products go to the caller's device workspace ws (ws_bytes; rows are processed in chunks that
 * fit it) and are summed in chunk order.  The engine uses it for its GEMMs on the gathered head
 * rows and the scorer, and, with LAYA_LATENCY=1, for the residual GEMMs over all rows.  Returns the
 * previous factor, or -2 for an invalid value. */
int laya_ext_gemm_ksplit(int ks, void* ws, size_t ws_bytes);

/* laya_ext_gemm's split-K path (bf16 operands, epi 0 store or 1 fp32 residual update, as for
 * laya_ext_gemm with laya_ext_gemm_ksplit(ksplit, ...)), allocating nothing: the fp32 partial
 * products go to a static device array of 8 MiB that the library holds on each GPU it runs on, not
 * to a caller's workspace.  No counterpart in the reference; it is for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * It calls no hipMalloc, hipFree or other allocating routine; it only launches on stream (a
 * hipStream_t) and does not wait.  Rows run in chunks whose ksplit * N fp32 partials fit the array;
 * ksplit * N * 4 bytes above 8 MiB is rejected.  Results are bit-identical to laya_ext_gemm with the
 * same split.  All calls on one GPU share its array: calls that overlap in time on one GPU (other
 * streams, other threads) race and must be serialized by the caller.  Returns 0; -1 for an
 * unsupported shape or argument (ksplit outside 2..64, K not a multiple of 64 * ksplit, shapes
 * laya_ext_gemm rejects); -2 when ksplit * N * 4 exceeds the array (an error is printed); -3 when
 * the current device's array cannot be located. */
int laya_ext_gemm_splitk_static(int epi, const void* A, const void* W, void* C, const float* bias, int act, int M,
                                int N, int K, int ksplit, void* stream);

#ifdef __cplusplus
}
#endif
