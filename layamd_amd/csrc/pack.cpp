// Pass packing for laya_forward_batch (host only).  Validation and pass splitting follow the
// reference (src/engine.hip:491-504); the per-pass layout is described in pack.h.
#include "pack.h"

#include <algorithm>

namespace laya {

static inline int align_up(int x, int a) { return (x + a - 1) / a * a; }

int plan_passes(int B, const int* lens, const int* ids, const int* nmark, const int* markers, const int* qtypes,
                const PackLimits& lim, std::vector<PassPlan>* passes) {
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
  const int pass_rows = std::max(lim.pass_tokens, lim.max_len);
  int b0 = 0;
  while (b0 < B) {
    int n = 0, T = 0, R = 0;
    while (b0 + n < B && n < lim.max_seqs && T + lens[b0 + n] <= pass_rows &&
           R + nmark[b0 + n] + 1 <= std::max(lim.max_grows, kMaxMarkers + 1)) {
      T += lens[b0 + n]; R += nmark[b0 + n] + 1; n++;
    }
    PassPlan p;
    p.first = b0; p.B = n; p.T = T;
    p.ids.resize(T); p.pos.resize(T); p.seq.resize(T); p.vcol.resize(T);
    p.soff.resize(n + 1); p.vlen.resize(n); p.vbase.resize(n); p.qt.resize(n); p.nm.resize(n); p.moff.resize(n);
    int r = 0, vc = 0, kt = 0;
    for (int i = 0; i < n; i++) {
      const int b = b0 + i, len = lens[b];
      p.soff[i] = r; p.vlen[i] = len; p.vbase[i] = vc; p.qt[i] = qtypes[b]; p.nm[i] = nmark[b]; p.moff[i] = kt;
      for (int j = 0; j < len; j++) {
        p.ids[r + j] = ids[ioff[b] + j]; p.pos[r + j] = j; p.seq[r + j] = i; p.vcol[r + j] = vc + j;
      }
      for (int q0 = 0; q0 < len; q0 += kQTile) p.tiles.push_back({i, q0, std::min(kQTile, len - q0), 0});
      r += len; vc += align_up(len, kVAlign); kt += nmark[b];
    }
    p.soff[n] = r;
    p.VT = vc; p.KT = kt; p.R = kt + n;
    p.grow.resize(p.R);
    for (int i = 0; i < n; i++) {
      const int b = b0 + i;
      for (int k = 0; k < nmark[b]; k++) p.grow[p.moff[i] + k] = p.soff[i] + markers[moff[b] + k];
      p.grow[kt + i] = p.soff[i];                          // CLS row
      // this question's gathered queries: its markers, then its CLS row
      std::vector<int32_t> q;
      for (int k = 0; k < nmark[b]; k++) q.push_back(p.moff[i] + k);
      q.push_back(kt + i);
      for (size_t s = 0; s < q.size(); s += kQTile) {
        int cnt = (int)std::min<size_t>(kQTile, q.size() - s);
        p.gtiles.push_back({i, (int)p.gq.size(), cnt, 0});
        p.gq.insert(p.gq.end(), q.begin() + s, q.begin() + s + cnt);
      }
    }
    passes->push_back(std::move(p));
    b0 += n;
  }
  return 0;
}

PassCaps pass_caps(const PackLimits& lim) {
  PassCaps c;
  const int64_t rows = std::max(lim.pass_tokens, lim.max_len);
  c.rows = rows;
  c.vt_cols = rows + (int64_t)lim.max_seqs * kVAlign + 64;  // alignment gaps + one key block of slack
  c.tiles = rows / kQTile + lim.max_seqs;
  c.grows = std::max(lim.max_grows, kMaxMarkers + 1);
  c.gtiles = c.grows / kQTile + lim.max_seqs;
  return c;
}

}  // namespace laya
