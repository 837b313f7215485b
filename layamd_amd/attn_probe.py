"""Per-workgroup timeline of the bf16 attention kernel at a benchmark batch's lengths:

    python -m layamd_amd.build --tile-trace && python -m layamd_amd.attn_probe [--config c3] [--qtile 64]

Loads the measurement library liblaya_trace.so (its attention kernel records, per workgroup, start
and end on the 100 MHz real-time clock, shader cycles and the 64-key blocks it processed:
csrc/tile_trace.h) and runs the encoder's sliding-window (+-64) and global attention once each on
random bf16 Q, K, V^T packed as the engine packs the batch's questions (16 heads of 64; tiles of
<= qtile queries, longest questions first, then the bucket's empty tiles).  Prints per launch: the
device time (mean of 10 launches), the span of the traced launch, the clock, how many workgroups
were resident at once at most, the mean workgroup time per count of key blocks (and how much of it
came before the first block: the tile's lookups (tile, then its question's offset and length),
Q and the first K and V^T block; and how much
wave 0 spent in the key loop's two waits: V^T landed before the PV step, and the next K landed at
the end of the block, each with its barrier), how busy the
resident slots were over the span (sum of workgroup times / (span x the most resident at once)),
and when the last workgroups started.
"""
import argparse
import ctypes

import numpy as np

from layamd_amd import engine as le
from layamd_amd import workloads as wl


def _up(x, a):
    return (int(x) + a - 1) // a * a


def packed(lens, H, seed=0):
    import torch
    soff = np.concatenate([[0], np.cumsum([_up(L, 8) for L in lens])]).astype(np.int32)
    rows = _up(soff[-1], 64)
    ldv = _up(rows + 64, 64)
    g = torch.Generator(device="cpu").manual_seed(seed)
    D = 64 * H
    q = torch.randn(rows, D, generator=g).to(torch.bfloat16).cuda()
    k = torch.randn(rows, D, generator=g).to(torch.bfloat16).cuda()
    vt = torch.randn(D, ldv, generator=g).to(torch.bfloat16).cuda()
    return q, k, vt, torch.as_tensor(soff).cuda(), torch.as_tensor(np.asarray(lens, np.int32)).cuda(), rows


def tiles_for(lens, qtile, rows):
    t = [(b, q0, min(qtile, L - q0), 0) for b, L in enumerate(lens) for q0 in range(0, L, qtile)]
    t.sort(key=lambda x: -lens[x[0]])
    cap = rows // 64 + len(lens)                     # the engine's tile capacity for the bucket
    return np.array(t + [(0, 0, 0, 0)] * (cap - len(t)), np.int32)


def main():
    import torch
    from layamd_amd import build
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="c3", choices=["c3", "c4", "c5"])
    ap.add_argument("--qtile", type=int, default=64)
    a = ap.parse_args()
    lib = le.load_library(build.TRACE_LIB)
    lib.laya_attn_trace_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    lib.laya_attn_trace_read.restype = ctypes.c_int
    lib.laya_attn_trace_clear.restype = ctypes.c_int
    batch = wl.CONFIGS[a.config](0)
    lens = [int(x) for x in batch.lens]
    H = batch.cfg.n_heads
    q, k, vt, soff, vlen, rows = packed(lens, H)
    O = torch.zeros(rows, 64 * H, dtype=torch.bfloat16, device="cuda")
    tiles = torch.as_tensor(tiles_for(lens, a.qtile, rows)).cuda()
    nt = tiles.shape[0]
    print("%s: %d questions, %d tokens, %d heads, %d tiles of <= %d queries (%d empty)"
          % (batch.name, len(lens), sum(lens), H, nt, a.qtile, nt - sum((L + a.qtile - 1) // a.qtile for L in lens)))
    for name, wh in (("sliding +-64", batch.cfg.local_attention // 2), ("global", 0)):
        run = lambda: le.attention(lib, 1, q, k, vt, O, tiles, soff, vlen, H, wh, 0.125, qtile=a.qtile)
        for _ in range(3):
            run()
        torch.cuda.synchronize()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        for _ in range(10):
            run()
        ev1.record()
        torch.cuda.synchronize()
        per = ev0.elapsed_time(ev1) / 10 * 1e3
        assert lib.laya_attn_trace_clear() == 0
        run()
        torch.cuda.synchronize()
        n = nt * H
        rec = np.zeros(8 * n, np.uint64)
        assert lib.laya_attn_trace_read(rec.ctypes.data, n) == 0
        r_keep = rec.reshape(n, 8)[:, 3] > 0                  # workgroups of non-empty tiles
        r = rec.reshape(n, 8)[r_keep].astype(np.float64)
        r0, r3 = r[:, 0], r[:, 1]
        dur = (r3 - r0) / 100.0
        ghz = r[:, 2].sum() / dur.sum() / 1e3
        t0 = r0.min()
        span = (r3.max() - t0) / 100.0
        # resident workgroups over time (events sorted)
        ev = np.concatenate([np.stack([r0, np.ones_like(r0)], 1), np.stack([r3, -np.ones_like(r3)], 1)])
        ev = ev[np.lexsort((ev[:, 1], ev[:, 0]))]
        peak = int(np.cumsum(ev[:, 1]).max())
        busy = dur.sum() / (span * peak)
        print("%-13s %6.1f us per launch | span %.1f us, clock %.2f GHz, %d workgroups, at most %d resident, "
              "slots busy %.0f%%, last start at %.1f us" % (name, per, span, ghz, len(r), peak, 100 * busy,
                                                            (r0.max() - t0) / 100.0))
        w7 = rec.reshape(n, 8)[r_keep, 7]
        pro = (w7 & np.uint64(0xFFFFFFFF)).astype(np.float64) / ghz / 1e3   # entry to the first key block
        pra = (w7 >> np.uint64(32)).astype(np.float64) / ghz / 1e3          # entry to the tile's lookups done
        w5 = rec.reshape(n, 8)[r_keep, 5]
        wv = (w5 >> np.uint64(32)).astype(np.float64) / ghz / 1e3
        wk = (w5 & np.uint64(0xFFFFFFFF)).astype(np.float64) / ghz / 1e3
        for nb in sorted(set(r[:, 3].astype(int))):
            m = r[:, 3] == nb
            print("    %d key blocks: %4d workgroups, %.2f us each (p10 %.2f, p90 %.2f): %.2f us before the first "
                  "block (%.2f to the tile's lookups), %.2f us in V^T waits, %.2f us in end-of-block waits"
                  % (nb, m.sum(), dur[m].mean(), np.percentile(dur[m], 10), np.percentile(dur[m], 90),
                     pro[m].mean(), pra[m].mean(), wv[m].mean(), wk[m].mean()))


if __name__ == "__main__":
    main()
