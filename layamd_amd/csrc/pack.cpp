// Pass packing for laya_forward_batch (host only).  Validation and pass splitting follow the
// reference (src/engine.hip:491-504); the per-pass layout is described in pack.h.
#include "pack.h"

#include <algorithm>

namespace laya {

static inline int align_up(int x, int a) { return (x + a - 1) / a * a; }

int plan_passes(int B, const int* lens, const int* ids, const int* nmark, const int* markers, const int* qtypes,
                const PackLimits& lim, std::vector<PassPlan>* passes) {
  const int pad_id = lim.pad_id;
  passes->clear();
  if (B < 0) return -1;
  std::vector<int64_t> ioff(B + 1, 0), moff(B + 1, 0);
  for (int b = 0; b < B; b++) {
    if (lens[b] < 1 || lens[b] > lim.max_len || nmark[b] < 1 || nmark[b] > kMaxMarkers) return -1;
    if (qtypes[b] < 0 || qtypes[b] > 2) return -1;       // indexes type_emb [3, D]
    ioff[b + 1] = ioff[b] + lens[b];
    moff[b + 1] = moff[b] + nmark[b];
    for (int k = 0; k < nmark[b]; k++) {
      int m = markers[moff[b] + k];
      if (m < 0 || m >= lens[b]) return -1;
    }
    if (lim.vocab > 0)
      for (int j = 0; j < lens[b]; j++) {
        int t = ids[ioff[b] + j];
        if (t < 0 || t >= lim.vocab) return -1;
      }
  }
  const int pass_rows = std::max(lim.pass_tokens, align_up(lim.max_len, kRowAlign));
  const int grows_cap = std::max(lim.max_grows, align_up(kMaxMarkers, kMarkerBucket) + 1);
  int b0 = 0;
  while (b0 < B) {
    int n = 0, T = 0, kt = 0;
    // questions in order while the rows fit the pass and the gathered rows (markers padded to
    // their bucket, plus one CLS row per question) fit the gathered buffers
    while (b0 + n < B && n < lim.max_seqs && T + align_up(lens[b0 + n], kRowAlign) <= pass_rows &&
           align_up(kt + nmark[b0 + n], kMarkerBucket) + n + 1 <= grows_cap) {
      T += align_up(lens[b0 + n], kRowAlign); kt += nmark[b0 + n]; n++;
    }
    PassPlan p;
    p.first = b0; p.B = n; p.T = align_up(T, kRowBucket);
    p.markers = kt;
    p.KT = align_up(kt, kMarkerBucket);
    p.R = p.KT + n;
    p.ids.resize(p.T); p.pos.resize(p.T); p.seq.resize(p.T);
    p.soff.resize(n + 1); p.vlen.resize(n); p.qt.resize(n); p.nm.resize(n); p.moff.resize(n);
    int r = 0, mo = 0;
    for (int i = 0; i < n; i++) {
      const int b = b0 + i, len = lens[b], rows = align_up(len, kRowAlign);
      p.soff[i] = r; p.vlen[i] = len; p.qt[i] = qtypes[b]; p.nm[i] = nmark[b]; p.moff[i] = mo;
      for (int j = 0; j < rows; j++) {
        p.ids[r + j] = j < len ? ids[ioff[b] + j] : pad_id; p.pos[r + j] = j; p.seq[r + j] = i;
      }
      for (int q0 = 0; q0 < len; q0 += lim.q_tile) p.tiles.push_back({i, q0, std::min(lim.q_tile, len - q0), 0});
      for (int q0 = 0; q0 < len; q0 += lim.q_tile_global)
        p.gltiles.push_back({i, q0, std::min(lim.q_tile_global, len - q0), 0});
      r += rows; mo += nmark[b]; p.valid += len;
    }
    p.soff[n] = r;
    for (int j = r; j < p.T; j++) { p.ids[j] = pad_id; p.pos[j] = 0; p.seq[j] = n - 1; }   // the bucket's tail rows
    p.grow.assign(p.R, 0);                                 // marker padding: row 0, computed, never read
    for (int i = 0; i < n; i++) {
      const int b = b0 + i;
      for (int k = 0; k < nmark[b]; k++) p.grow[p.moff[i] + k] = p.soff[i] + markers[moff[b] + k];
      p.grow[p.KT + i] = p.soff[i];                        // CLS row
      // this question's gathered queries: its markers, then its CLS row
      std::vector<int32_t> q;
      for (int k = 0; k < nmark[b]; k++) q.push_back(p.moff[i] + k);
      q.push_back(p.KT + i);
      for (size_t s = 0; s < q.size(); s += kQTile) {
        int cnt = (int)std::min<size_t>(kQTile, q.size() - s);
        p.gtiles.push_back({i, (int)p.gq.size(), cnt, 0});
        p.gq.insert(p.gq.end(), q.begin() + s, q.begin() + s + cnt);
      }
    }
    // longest questions first: an attention launch then starts its longest tiles (which visit the
    // most key blocks) before the short ones instead of ending on them (tile order does not change
    // any result)
    auto by_len = [&](const AttnTile& x, const AttnTile& y) { return p.vlen[x.seq] > p.vlen[y.seq]; };
    std::stable_sort(p.tiles.begin(), p.tiles.end(), by_len);
    std::stable_sort(p.gltiles.begin(), p.gltiles.end(), by_len);
    std::stable_sort(p.gtiles.begin(), p.gtiles.end(), by_len);
    // empty tiles up to the bucket's capacities (the launch grids)
    p.tiles.resize(tiles_cap(p.T, n), AttnTile{0, 0, 0, 0});
    p.gltiles.resize(tiles_cap(p.T, n), AttnTile{0, 0, 0, 0});
    p.gtiles.resize(gtiles_cap(p.R, n), AttnTile{0, 0, 0, 0});
    passes->push_back(std::move(p));
    b0 += n;
  }
  return 0;
}

PassCaps pass_caps(const PackLimits& lim) {
  PassCaps c;
  c.rows = align_up(std::max(lim.pass_tokens, align_up(lim.max_len, kRowAlign)), kRowBucket);
  c.seqs = std::max(1, lim.max_seqs);
  c.grows = std::max(lim.max_grows, align_up(kMaxMarkers, kMarkerBucket) + 1);
  c.tiles = tiles_cap((int)c.rows, c.seqs);
  c.gtiles = gtiles_cap((int)c.grows, c.seqs);
  return c;
}

}  // namespace laya
