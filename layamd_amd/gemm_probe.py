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
    a = ap.parse_args()
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
