"""Runs the engine's bf16 MFMA GEMM on one shape through laya_ext_gemm, for timing and for counter
runs (rocprofv3 --pmc) of a single kernel:

    python -m layamd_amd.gemm_probe --M 16384 --N 4096 --K 4096 --cfg 0 --iters 4

A = N(0,1) and W = N(0,0.02) in bf16, C = A W^T stored in bf16 (plain epilogue, no bias).  --cfg
pins the tile configuration (0..8, see include/laya_ext.h; -1: the planner).  Prints the time per
launch and the TFLOP/s on 2 M N K flop.

    python -m layamd_amd.gemm_probe --c2

times the GEMM microbenchmark shapes instead: M in {512, 16384}, (N, K) in {(3072, 1024),
(1024, 1024), (5248, 1024), (1024, 2624)}, bf16 and fp32 operands, against torch.mm (hipBLASLt or
rocBLAS) on the same device.  bf16 tries the planner and every tile configuration (with split-K
factors 2, 4 and 8 at M = 512 where K allows them) and reports the best; each engine result is checked
against torch.mm.  Prints a markdown table.

    python -m layamd_amd.gemm_probe --c3

does the same, bf16 only, for the encoder GEMMs of the b32 x s512 ModernBERT-large pass: M = 9664
rows (the pass's 9514 tokens, packed and padded to 64), (N, K) as above.

    python -m layamd_amd.build --tile-trace && python -m layamd_amd.gemm_probe --tile-trace

loads the measurement library liblaya_trace.so instead and prints, for the pass's encoder GEMM
shapes (plain store for the QKV and Wi shapes, the fp32 residual update for the two N = 1024 ones)
on their tile configurations, the per-tile timeline its GEMM records (csrc/tile_trace.h): the
shader clock the tiles ran at, prologue, K loop, the K loop's stage waits and the epilogue per tile,
how the tiles' start times spread over the launch, and the K loop's MFMA rate against the rate the
CU has at that clock (4 SIMDs x 1024 flop per cycle: one v_mfma_f32_32x32x16_bf16 per 32 cycles).
With --M/--N/--K/--cfg given explicitly it traces that one shape (plain store); --split R --tail C
with --cfg 7 (C = 8 or 3) traces a row split that runs as one launch (k_gemm_xl_pair): per-tile
figures of the first shape's tiles, the span and start spread of all, and when the tail tiles
started and ended.  The b32 x s512 list includes the Wi shape's split at row 9408 (the tuner's
plan for the GeGLU GEMM there).
"""
import argparse
import time

from layamd_amd import engine as le


ENCODER_NK = ((3072, 1024), (1024, 1024), (5248, 1024), (1024, 2624))
C2_SHAPES = [(M, N, K) for M in (512, 16384) for (N, K) in ENCODER_NK]
C3_SHAPES = [(9664, N, K) for (N, K) in ENCODER_NK]


def _spin():
    """Queues a few milliseconds of GPU spinning, so that the host enqueues the timed calls while the
    GPU is busy and they then run back to back (small GEMMs would otherwise wait on the host)."""
    import torch
    torch.cuda._sleep(20_000_000)


def _time(fn, iters=20):
    """Device time per call of fn (us), over back-to-back calls bracketed by events."""
    import torch
    fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    _spin()
    a.record()
    for _ in range(iters):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / iters * 1e3                # us per call


def c2(lib, shapes=C2_SHAPES, dtypes=None):
    import torch
    dtypes = dtypes or (torch.bfloat16, torch.float32)
    g = torch.Generator(device="cpu").manual_seed(0)
    ws = torch.empty(64 << 20, dtype=torch.float32, device="cuda")   # split-K partials (256 MiB)
    print("| M | N | K | dtype | torch.mm us | TFLOP/s | engine us | TFLOP/s | engine plan | planner us | max rel err vs torch.mm |")
    print("|---:|---:|---:|---|---:|---:|---:|---:|---|---:|---:|")
    for (M, N, K) in shapes:
        fl = 2.0 * M * N * K
        A32 = torch.randn(M, K, generator=g).cuda()
        W32 = (torch.randn(N, K, generator=g) * 0.02).cuda()
        for dt in dtypes:
            A, W = A32.to(dt), W32.to(dt)
            Wt = W.t()
            ref = torch.empty(M, N, dtype=dt, device="cuda")
            t_mm = _time(lambda: torch.mm(A, Wt, out=ref))
            C = torch.empty(M, N, dtype=dt, device="cuda")
            plans = [(-1, 1)]
            if dt == torch.bfloat16:
                plans += [(c, 1) for c in range(9)]
                if M <= 4096:
                    plans += [(c, ks) for ks in (2, 4, 8) if K % (64 * ks) == 0 for c in range(9)]
            best, t_plan = None, None
            for cfg, ks in plans:
                le.gemm_config(lib, cfg)
                le.gemm_ksplit(lib, ks if ks > 1 else 0, ws if ks > 1 else None)
                le.gemm(lib, A, W, C)                      # warm-up
                _spin()
                t = le.gemm(lib, A, W, C, iters=20) / 20 * 1e3  # back-to-back launches, device events
                err = ((C.float() - ref.float()).abs().max() / ref.float().abs().max()).item()
                if cfg == -1:
                    t_plan = t
                if best is None or t < best[0]:
                    best = (t, cfg, ks, err)
            le.gemm_config(lib, -1)
            le.gemm_ksplit(lib, 0, None)
            t, cfg, ks, err = best
            plan = "planner" if cfg == -1 else "cfg %d%s" % (cfg, ", split-K %d" % ks if ks > 1 else "")
            print("| %d | %d | %d | %s | %.1f | %.0f | %.1f | %.0f | %s | %.1f | %.1e |"
                  % (M, N, K, "bf16" if dt == torch.bfloat16 else "fp32", t_mm, fl / t_mm / 1e6, t, fl / t / 1e6, plan,
                     t_plan, err), flush=True)


# (label, residual epilogue, N, K, tile configuration) at M = 9664: the encoder GEMMs of the
# b32 x s512 pass on the tiles the tuner picks for them there (and 256x256 for the QKV shape)
TRACE_C3 = [("QKV shape, store", False, 3072, 1024, 5), ("QKV shape, store", False, 3072, 1024, 0),
            ("out-proj, residual", True, 1024, 1024, 5), ("Wi shape, store", False, 5248, 1024, 7),
            ("Wi shape, store", False, 5248, 1024, 7, 9408, 8), ("MLP-out, residual", True, 1024, 2624, 5)]
# row splits that run as one launch (k_gemm_xl_pair): (first configuration, tail configuration)
PAIRS = {(7, 8), (7, 3)}
# (tile rows, tile columns, workgroups per CU) of the tile configurations
TILES = {0: (256, 256, 1), 1: (256, 128, 1), 2: (128, 256, 1), 3: (128, 128, 2), 4: (192, 256, 1),
         5: (160, 256, 1), 6: (128, 192, 2), 7: (192, 128, 2), 8: (128, 64, 2)}


def tile_trace(M, cases):
    import ctypes
    import numpy as np
    import torch
    from layamd_amd import build
    lib = le.load_library(build.TRACE_LIB)
    lib.laya_tile_trace_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    lib.laya_tile_trace_read.restype = ctypes.c_int
    lib.laya_tile_trace_clear.restype = ctypes.c_int
    g = torch.Generator(device="cpu").manual_seed(0)
    print("| GEMM (M = %d) | tile | tiles (rounds) | us per launch | span us | clock GHz | prologue us | K loop us "
          "| stage waits us | epilogue us | K loop MFMA rate at that clock | start spread us (p50, max) |" % M)
    print("|---|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---|")
    for case in cases:
        label, resid, N, K, cfg = case[:5]
        split, tail = case[5:7] if len(case) > 5 else (0, -1)
        # a split is traced only where it runs as one launch (one record per workgroup)
        assert split == 0 or ((cfg, tail) in PAIRS and not resid and 0 < split < M), case
        A = torch.randn(M, K, generator=g).to(torch.bfloat16).cuda()
        W = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).cuda()
        C = torch.zeros(M, N, dtype=torch.float32 if resid else torch.bfloat16, device="cuda")
        le.gemm_config(lib, cfg)
        le.gemm_split(lib, split, tail)
        for _ in range(3):
            le.gemm(lib, A, W, C, residual=resid)
        torch.cuda.synchronize()
        _spin()
        per_us = le.gemm(lib, A, W, C, residual=resid, iters=10) / 10 * 1e3
        torch.cuda.synchronize()
        assert lib.laya_tile_trace_clear() == 0
        le.gemm(lib, A, W, C, residual=resid)
        torch.cuda.synchronize()
        bm, bn, per_cu = TILES[cfg]
        nt = ((min(split or M, M) + bm - 1) // bm) * ((N + bn - 1) // bn)          # the first shape's tiles
        ntt = 0
        if split:
            bm2, bn2, _ = TILES[tail]
            ntt = ((M - split + bm2 - 1) // bm2) * ((N + bn2 - 1) // bn2)          # then the tail's
        rec = np.zeros(8 * (nt + ntt), np.uint64)
        assert lib.laya_tile_trace_read(rec.ctypes.data, nt + ntt) == 0
        rall = rec.reshape(nt + ntt, 8).astype(np.float64)
        assert (rall[:, 7] > 0).all(), "a tile left no record"
        r = rall[:nt]                                       # per-tile figures: the first shape's tiles
        r0, r3 = r[:, 0], r[:, 1]
        dur_us = (r3 - r0) / 100.0                          # 100 MHz real-time clock
        ghz = r[:, 7].sum() / dur_us.sum() / 1e3
        us = lambda col: r[:, col].mean() / ghz / 1e3
        kloop = us(3)
        rate = 2.0 * bm * bn * K / (kloop * 1e-6) * per_cu        # flop/s of one CU in the K loop
        peak = 4 * 1024 * ghz * 1e9
        t0 = rall[:, 0].min()
        start = (rall[:, 0] - t0) / 100.0
        shape = "%dx%d%s" % (bm, bn, ", 2 per CU" if per_cu == 2 else "")
        tiles = "%d (%.2f)" % (nt, nt / (256.0 * per_cu))
        spread = "%.1f, %.1f" % (np.percentile(start, 50), start.max())
        if split:
            tst = start[nt:]
            shape += " to row %d, then %dx%d" % (split, bm2, bn2)
            tiles = "%d + %d" % (nt, ntt)
            spread += "; tail tiles start %.1f-%.1f, end by %.1f" % (tst.min(), tst.max(), (rall[nt:, 1].max() - t0) / 100.0)
        print("| %s %dx%dx%d | %s | %s | %.1f | %.1f | %.2f | %.2f | %.2f | %.2f (%.0f%%) | %.2f | %.0f%% | %s |"
              % (label, M, N, K, shape, tiles, per_us, (rall[:, 1].max() - t0) / 100.0, ghz, us(2), kloop, us(5),
                 100 * us(5) / kloop, us(4), 100 * rate / peak, spread), flush=True)
    le.gemm_split(lib, 0)
    le.gemm_config(lib, -1)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--M", type=int, default=16384)
    ap.add_argument("--N", type=int, default=4096)
    ap.add_argument("--K", type=int, default=4096)
    ap.add_argument("--cfg", type=int, default=0)
    ap.add_argument("--iters", type=int, default=4)
    ap.add_argument("--c2", action="store_true", help="time the microbenchmark shapes against torch.mm")
    ap.add_argument("--c3", action="store_true", help="time the b32 x s512 pass's encoder GEMM shapes against torch.mm")
    ap.add_argument("--torch", action="store_true",
                    help="after the engine launches, run torch.mm on the same operands as many times")
    ap.add_argument("--tile-trace", action="store_true",
                    help="per-tile timeline from liblaya_trace.so (python -m layamd_amd.build --tile-trace)")
    ap.add_argument("--split", type=int, default=0,
                    help="with --tile-trace and --cfg 7: rows from --split on in --tail tiles, in the same launch")
    ap.add_argument("--tail", type=int, default=8)
    a, _ = ap.parse_known_args()
    if a.tile_trace:
        import sys
        explicit = any(x.split("=")[0] in ("--M", "--N", "--K", "--cfg") for x in sys.argv[1:])
        case = ("store", False, a.N, a.K, a.cfg) + ((a.split, a.tail) if a.split else ())
        tile_trace(a.M if explicit else 9664, [case] if explicit else TRACE_C3)
        return
    lib = le.load_library()
    import torch
    if a.c2:
        c2(lib)
        return
    if a.c3:
        c2(lib, C3_SHAPES, (torch.bfloat16,))
        return
    g = torch.Generator(device="cpu").manual_seed(0)
    A = torch.randn(a.M, a.K, generator=g).to(torch.bfloat16).cuda()
    W = (torch.randn(a.N, a.K, generator=g) * 0.02).to(torch.bfloat16).cuda()
    C = torch.zeros(a.M, a.N, dtype=torch.bfloat16, device="cuda")
    le.gemm_config(lib, a.cfg)
    le.gemm(lib, A, W, C)                                  # warm-up
    torch.cuda.synchronize()
    t = time.perf_counter()
    ms = le.gemm(lib, A, W, C, iters=a.iters)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t) * 1e3
    per = ms / a.iters
    print("gemm %dx%dx%d cfg %d: %.1f us per launch (%.1f ms wall for %d), %.0f TFLOP/s"
          % (a.M, a.N, a.K, a.cfg, per * 1e3, wall, a.iters, 2.0 * a.M * a.N * a.K / (per * 1e-3) / 1e12))
    if a.torch:
        Wt = W.t()
        torch.mm(A, Wt, out=C)                             # warm-up
        t = _time(lambda: torch.mm(A, Wt, out=C), a.iters)
        print("torch.mm %dx%dx%d: %.1f us per call, %.0f TFLOP/s" % (a.M, a.N, a.K, t, 2.0 * a.M * a.N * a.K / t / 1e6))


if __name__ == "__main__":
    main()
