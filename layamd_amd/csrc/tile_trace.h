// Per-tile timeline of the bf16 GEMM kernel (k_gemm_xl), exported only by the measurement build
// liblaya_trace.so (python -m layamd_amd.build --tile-trace, compiled with -DLAYA_TILE_TRACE); the
// product library liblaya.so has neither the recording code nor these entry points.
//
// Every workgroup of a k_gemm_xl launch writes one record of 8 little-endian uint64 at index
// blockIdx.x (records of earlier launches stay until overwritten or cleared):
//   [0] start, [1] end          100 MHz real-time clock (s_memrealtime), comparable across CUs
//   [2] prologue                shader cycles from entry to the K loop (DMA of the first stages issued)
//   [3] K loop                  shader cycles
//   [4] epilogue                shader cycles from the end of the K loop to exit
//   [5] stage waits             shader cycles wave 0 spent in the K loop's wait + barrier per stage
//                               (two-buffer loop; 0 for the other loops)
//   [6] hardware id             XCC id << 32 | HW_ID register
//   [7] total                   shader cycles from entry to exit
#pragma once
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif
/* copies the first `records` records (at most 65536) to host memory; 0 or -1 */
int laya_tile_trace_read(void* host, size_t records);
/* zeroes every record; 0 or -1 */
int laya_tile_trace_clear(void);

/* The bf16 attention kernel (k_attention_bf16) keeps its own records, one per workgroup at index
 * blockIdx.y * gridDim.x + blockIdx.x (tile-major, heads fastest), 8 uint64 each:
 *   [0] start, [1] end (100 MHz real-time clock), [2] shader cycles entry to exit,
 *   [3] 64-key blocks processed, [4] tile index << 32 | head,
 *   [5] shader cycles wave 0 spent in the V^T wait + barrier before each PV step (summed) << 32 |
 *       those in the wait + barrier at the end of each block (next K landed, buffers free),
 *   [6] XCC id << 32 | HW_ID,
 *   [7] shader cycles from entry to the tile's question offset and length loaded << 32 |
 *       those from entry to the first key block (Q and the first K, V^T block loaded). */
int laya_attn_trace_read(void* host, size_t records);
int laya_attn_trace_clear(void);
#ifdef __cplusplus
}
#endif
