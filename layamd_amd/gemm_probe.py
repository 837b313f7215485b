"""Runs the engine's bf16 MFMA GEMM on one shape through laya_ext_gemm, for timing and for counter
runs (rocprofv3 --pmc) of a single kernel:

    python -m layamd_amd.gemm_probe --M 16384 --N 4096 --K 4096 --cfg 0 --iters 4

A = N(0,1) and W = N(0,0.02) in bf16, C = A W^T stored in bf16 (plain epilogue, no bias).  --cfg
pins the tile configuration (0..5, see include/laya_ext.h; -1: the planner).  Prints the time per
launch and the TFLOP/s on 2 M N K flop.
"""
import argparse
import time

from layamd_amd import engine as le


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--M", type=int, default=16384)
    ap.add_argument("--N", type=int, default=4096)
    ap.add_argument("--K", type=int, default=4096)
    ap.add_argument("--cfg", type=int, default=0)
    ap.add_argument("--iters", type=int, default=4)
    a = ap.parse_args()
    lib = le.load_library()
    import torch
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


if __name__ == "__main__":
    main()
