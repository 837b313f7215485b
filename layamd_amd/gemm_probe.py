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
With --M/--N/--K/--cfg given explicitly it traces that one shape (plain store).
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
            ("MLP-out, residual", True, 1024, 2624, 5)]
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
    for label, resid, N, K, cfg in cases:
        A = torch.randn(M, K, generator=g).to(torch.bfloat16).cuda()
        W = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).cuda()
        C = torch.zeros(M, N, dtype=torch.float32 if resid else torch.bfloat16, device="cuda")
        le.gemm_config(lib, cfg)
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
        nt = ((M + bm - 1) // bm) * ((N + bn - 1) // bn)
        rec = np.zeros(8 * nt, np.uint64)
        assert lib.laya_tile_trace_read(rec.ctypes.data, nt) == 0
        r = rec.reshape(nt, 8).astype(np.float64)
        assert (r[:, 7] > 0).all(), "a tile left no record"
        r0, r3 = r[:, 0], r[:, 1]
        dur_us = (r3 - r0) / 100.0                          # 100 MHz real-time clock
        ghz = r[:, 7].sum() / dur_us.sum() / 1e3
        us = lambda col: r[:, col].mean() / ghz / 1e3
        kloop = us(3)
        rate = 2.0 * bm * bn * K / (kloop * 1e-6) * per_cu        # flop/s of one CU in the K loop
        peak = 4 * 1024 * ghz * 1e9
        start = (r0 - r0.min()) / 100.0
        print("| %s %dx%dx%d | %dx%d%s | %d (%.2f) | %.1f | %.1f | %.2f | %.2f | %.2f | %.2f (%.0f%%) | %.2f | %.0f%% | %.1f, %.1f |"
              % (label, M, N, K, bm, bn, ", 2 per CU" if per_cu == 2 else "", nt, nt / (256.0 * per_cu), per_us,
                 (r3.max() - r0.min()) / 100.0, ghz, us(2), kloop, us(5), 100 * us(5) / kloop, us(4), 100 * rate / peak,
                 np.percentile(start, 50), start.max()), flush=True)
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
    a, _ = ap.parse_known_args()
    if a.tile_trace:
        import sys
        explicit = any(x.split("=")[0] in ("--M", "--N", "--K", "--cfg") for x in sys.argv[1:])
        tile_trace(a.M if explicit else 9664, [("store", False, a.N, a.K, a.cfg)] if explicit else TRACE_C3)
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
