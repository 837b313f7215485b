/* Laya engine C ABI for AMD Instinct MI355X (gfx950).
 *
 * The same ten entry points, signatures and conventions as the reference engine's
 * src/laya_api.h:5-19, so its ctypes server binding (server/laya_server.py:20-31), laya-parity
 * (src/test_parity.cpp) and laya-bench (src/bench_engine.cpp) link against this library
 * unchanged.  Each declaration cites the reference entry point it replaces.
 *
 * Conventions (reference src/engine.hip:489-559):
 *   - ids: every question's tokens concatenated (sum(lens) int32, no padding);
 *   - markers: every question's option-marker positions concatenated (sum(nmark) int32), each a
 *     position inside its own question;
 *   - qtypes: 0 choice, 1 score, 2 noul (indexes the type embedding);
 *   - logits: caller-owned, receives sum(nmark) raw scorer logits; act: caller-owned, receives
 *     B * laya_n_act() raw act-head logits;
 *   - calls are synchronous and not thread-safe (one caller thread per handle);
 *   - there is no destroy function: an engine lives for the whole process.
 */
#pragma once
#ifdef __cplusplus
extern "C" {
#endif

/* Loads <dir>/encoder/config.json, <dir>/rl_agent_config.json and <dir>/model.safetensors and
 * allocates every buffer.  Exits the process on a missing file or tensor.
 * Replaces src/engine.hip:545 (laya_create). */
void* laya_create(const char* dir);

/* B questions in one call.  Returns 0, or -1 when any len < 1, len > max_len, nmark < 1,
 * nmark > 255, marker outside [0, len), qtype outside {0,1,2} or token id outside the vocabulary.
 * Replaces src/engine.hip:546-548 (laya_forward_batch). */
int laya_forward_batch(void* h, int B, const int* lens, const int* ids, const int* nmark, const int* markers,
                       const int* qtypes, float* logits, float* act);

/* One question; S is ignored (valid_len tokens are read).  Replaces src/engine.hip:549-551. */
void laya_forward(void* h, const int* ids, int S, int valid_len, const int* markers, int K, int qtype, float* logits,
                  float* act);

/* len(act_costs) + 1.  Replaces src/engine.hip:552. */
int laya_n_act(void* h);

/* rl_agent_config.json max_len.  Replaces src/engine.hip:553. */
int laya_max_len(void* h);

/* 255.  Replaces src/engine.hip:554. */
int laya_max_markers(void* h);

/* rl_agent_config.json temperature[qtype] (1.0 outside {0,1,2}).  Replaces src/engine.hip:555. */
float laya_temperature(void* h, int qtype);

/* Prints the per-stage device-time table accumulated while LAYA_PROFILE (or
 * laya_ext_prof_enable) is on, divided by iters.  Replaces src/engine.hip:556. */
void laya_prof_report(void* h, int iters);

/* Clears the per-stage table.  Replaces src/engine.hip:557. */
void laya_prof_reset(void* h);

/* GEMM tuning ahead of traffic: times the engine's tile configurations for every GEMM of every
 * row bucket up to the pass capacity (otherwise each new pass shape is timed before its first
 * run).  Replaces src/engine.hip:558 (laya_tune_all, which times hipBLASLt plans per bucket). */
void laya_tune_all(void* h);

#ifdef __cplusplus
}
#endif
