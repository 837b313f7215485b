// Packing of a laya_forward_batch call into GPU passes (host only, no HIP dependency).
//
// Semantics follow the reference's Engine::forward_batch (src/engine.hip:489-539): the same
// input validation (-1 on len < 1, len > max_len, nmark < 1, nmark > 255, marker outside
// [0, len)), questions taken greedily in order into passes, each question its own sequence,
// outputs unpacked per question.  The layout inside a pass is this engine's own:
//
//   * rows are packed back to back with each question starting on a multiple of kRowAlign rows:
//     question i owns rows [soff[i], soff[i] + len[i]) and up to kRowAlign - 1 padding rows after
//     them (pad token, positions continuing past len); padding rows are computed and never read,
//     and every aligned group of kRowAlign rows belongs to one question, so the GEMM epilogue can
//     write V^T [H][head_dim][rows] (column = row) with 16-byte stores;
//   * attention work is a list of query tiles (seq, first query, query count) of <= q_tile
//     queries for the sliding-window layers (64; 128 on request for the bf16 engine) and one of
//     <= q_tile_global queries for the global layers (128 in the bf16 engine, 64 in fp32);
//     gathered tiles hold <= 64 queries;
//   * the last head layer works on R = KT + B gathered rows: the sum(nmark) marker rows in
//     question order, padded with copies of row 0 to KT rows (a multiple of kMarkerBucket), then
//     one CLS row per question; gathered query tiles index a list of gathered-row ids;
//   * a pass's rows are padded to a multiple of kRowBucket with pad-token rows (position 0,
//     assigned to the last question, computed and never read), and its tile lists are padded to
//     capacities that depend only on (rows, B, KT) with empty tiles (nq = 0, which the attention
//     kernels skip).  A pass's launches and array layout therefore depend only on the bucket
//     (rows, B, KT), so one captured HIP graph serves every batch of that bucket, as the
//     reference's graph cache keys its passes by (64-row T, B, 64-row KT) (src/engine.hip:468-486,
//     505).
#pragma once
#include <cstdint>
#include <vector>

namespace laya {

constexpr int kMaxMarkers = 255;     // options per question (the act head encodes k/255)
constexpr int kQTile = 64;           // queries per gathered attention tile (and default encoder tile)
constexpr int kRowAlign = 8;         // rows per aligned group (first row of every question)
constexpr int kRowBucket = 64;       // a pass's rows are a multiple of this
constexpr int kMarkerBucket = 64;    // a pass's marker rows (KT) are a multiple of this

// attention tile capacities of a pass bucket: sum over questions of ceil(len / q_tile) <= rows / 64
// + B for q_tile >= 64, and sum of ceil((nmark + 1) / 64) <= R / 64 + B
inline int tiles_cap(int rows, int B) { return rows / kRowBucket + B; }
inline int gtiles_cap(int R, int B) { return R / kQTile + B; }

struct PackLimits {
  int max_len = 512;
  int pass_tokens = 65536;           // rows per pass
  int max_seqs = 512;                // questions per pass
  int max_grows = 32768;             // gathered rows (sum of nmark + 1) per pass
  int vocab = 0;                     // > 0: ids must lie in [0, vocab)
  int pad_id = 0;                    // token id of padding rows
  int q_tile = kQTile;               // queries per sliding-window attention tile (64 or 128)
  int q_tile_global = kQTile;        // queries per global attention tile (encoder, head 0; 64 or 128)
};

struct AttnTile { int32_t seq, q0, nq, pad; };

struct PassPlan {
  int first = 0, B = 0;              // questions [first, first + B) of the call
  int T = 0, KT = 0, R = 0;          // rows, marker rows (both padded to their buckets), gathered rows
  int valid = 0;                     // sum of lens
  int markers = 0;                   // sum of nmark (KT before padding)
  std::vector<int32_t> ids, pos, seq;                       // [T]
  std::vector<int32_t> soff, vlen, qt, nm, moff;            // [B] (soff has B + 1)
  std::vector<AttnTile> tiles;                              // sliding-window query tiles (tiles_cap)
  std::vector<AttnTile> gltiles;                            // global query tiles (tiles_cap)
  std::vector<AttnTile> gtiles;                             // gathered query tiles (gtiles_cap)
  std::vector<int32_t> gq;                                  // gathered ids referenced by gtiles
  std::vector<int32_t> grow;                                // [R] packed row of each gathered row
};

// Validates the call; returns 0 and fills `passes`, or -1 on an invalid input.
// Passes hold at most pass_tokens rows before the padding to kRowBucket rows.
int plan_passes(int B, const int* lens, const int* ids, const int* nmark, const int* markers, const int* qtypes,
                const PackLimits& lim, std::vector<PassPlan>* passes);

// Largest sizes a pass can reach under `lim` (for buffer allocation).
struct PassCaps { int64_t rows, tiles, gtiles, grows; int seqs; };
PassCaps pass_caps(const PackLimits& lim);

}  // namespace laya
