"""Builds the engine in-tree:

    layamd_amd/liblaya.so       the laya_api.h C ABI + gfx950 kernels (hipcc --offload-arch=gfx950)
    layamd_amd/liblaya_host.so  host-only packer/loader entry points for the CPU tests (g++)
    layamd_amd/laya-parity      golden-format parity tool, a plain C++ caller of laya_api.h (g++)
    layamd_amd/laya-bench       ABI latency tool (p50 per laya_forward_batch call), same (g++)

    python -m layamd_amd.build [--jobs N]
    python -m layamd_amd.build --tile-trace

--probes builds only layamd_amd/gemm-wave-probe, a standalone GEMM K-loop probe (4 against 8 waves
per tile).  --tile-trace builds only layamd_amd/liblaya_trace.so, a measurement copy of the library whose GEMM
kernel records a per-tile timeline (csrc/tile_trace.h; read by python -m layamd_amd.gemm_probe
--tile-trace).  The product library never contains that code.

Each translation unit is compiled separately (in parallel) into layamd_amd/_build/, then linked.
HIP code is built with packed-fp32 instruction generation disabled.
"""
import argparse
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(REPO, "include")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "liblaya.so")
HOST_LIB = os.path.join(PKG, "liblaya_host.so")
TOOLS = {"laya-parity": "laya_parity.cpp", "laya-bench": "laya_bench.cpp"}

HIP_SOURCES = ["engine.hip", "kernels_gemm.hip", "kernels_attn.hip", "kernels_norm.hip"]
CPP_SOURCES = ["model.cpp", "pack.cpp"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-I" + CSRC, "-I" + INCLUDE,
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wno-unused-result"]
CXX_FLAGS = ["-O2", "-fPIC", "-std=c++17", "-I" + CSRC, "-I" + INCLUDE, "-Wall"]
# attention keeps its small MFMA accumulators in VGPRs (the softmax works on them directly); the
# GEMM keeps its large ones in AGPRs
TU_FLAGS = {"kernels_attn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError("build step failed: %s\n%s" % (" ".join(cmd), out))
    return out


def _newer(target, deps):
    if not os.path.exists(target):
        return False
    t = os.path.getmtime(target)
    return all(os.path.getmtime(d) <= t for d in deps)


TRACE_LIB = os.path.join(PKG, "liblaya_trace.so")
TRACE_BUILD = os.path.join(PKG, "_build_trace")


def build_trace(jobs: int = 8, verbose: bool = True) -> str:
    """liblaya_trace.so: the HIP sources compiled with -DLAYA_TILE_TRACE (GEMM per-tile timeline)."""
    os.makedirs(TRACE_BUILD, exist_ok=True)
    steps = []
    for s in HIP_SOURCES:
        src, obj = os.path.join(CSRC, s), os.path.join(TRACE_BUILD, s + ".o")
        steps.append([HIPCC] + HIP_FLAGS + TU_FLAGS.get(s, []) + ["-DLAYA_TILE_TRACE", "-c", src, "-o", obj])
    for s in CPP_SOURCES:
        src, obj = os.path.join(CSRC, s), os.path.join(TRACE_BUILD, s + ".o")
        steps.append(["g++"] + CXX_FLAGS + ["-c", src, "-o", obj])
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        list(ex.map(_run, steps))
    objs = [st[-1] for st in steps]
    tmp = TRACE_LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs + ["-lpthread"])
    os.replace(tmp, TRACE_LIB)
    if verbose:
        print("[build] %s" % TRACE_LIB)
    return TRACE_LIB


PROBES = {"gemm-wave-probe": "gemm_wave_probe.hip", "mfma-valu-probe": "mfma_valu_probe.hip"}


def build_probes(verbose: bool = True) -> None:
    """Standalone measurement programs (layamd_amd/<name>), not part of the library."""
    for exe, src in PROBES.items():
        out = os.path.join(PKG, exe)
        _run([HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Wno-unused-result", "-Wno-unused-value",
              "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-o", out + ".tmp",
              os.path.join(CSRC, "tools", src)])
        os.replace(out + ".tmp", out)
        if verbose:
            print("[build] %s" % out)


def build(jobs: int = 8, force: bool = True, verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    headers = [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".h", ".inc"))] + \
              [os.path.join(INCLUDE, f) for f in os.listdir(INCLUDE) if f.endswith(".h")]
    steps = []
    for s in HIP_SOURCES:
        src, obj = os.path.join(CSRC, s), os.path.join(BUILD, s + ".o")
        steps.append((obj, [src] + headers, [HIPCC] + HIP_FLAGS + TU_FLAGS.get(s, []) + ["-c", src, "-o", obj]))
    for s in CPP_SOURCES:
        src, obj = os.path.join(CSRC, s), os.path.join(BUILD, s + ".o")
        steps.append((obj, [src] + headers, ["g++"] + CXX_FLAGS + ["-c", src, "-o", obj]))
    todo = [st for st in steps if force or not _newer(st[0], st[1])]
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        for out in ex.map(lambda st: _run(st[2]), todo):
            if out.strip() and verbose:
                print(out)
    objs = [st[0] for st in steps]
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs + ["-lpthread"])
    os.replace(tmp, LIB)
    tmp = HOST_LIB + ".tmp"
    _run(["g++"] + CXX_FLAGS + ["-shared", "-o", tmp, os.path.join(CSRC, "host_probe.cpp"),
                                os.path.join(CSRC, "model.cpp"), os.path.join(CSRC, "pack.cpp")])
    os.replace(tmp, HOST_LIB)
    # the C++ tools link the library like any C caller of laya_api.h would (found next to them)
    for exe, src in TOOLS.items():
        out = os.path.join(PKG, exe)
        _run(["g++"] + CXX_FLAGS + ["-o", out + ".tmp", os.path.join(CSRC, "tools", src), "-L" + PKG, "-llaya",
                                    "-Wl,-rpath,$ORIGIN"])
        os.replace(out + ".tmp", out)
    if verbose:
        print("[build] %s\n[build] %s\n[build] %s" % (LIB, HOST_LIB, ", ".join(os.path.join(PKG, e) for e in TOOLS)))
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=8)
    ap.add_argument("--incremental", action="store_true")
    ap.add_argument("--tile-trace", action="store_true", help="build only the measurement library liblaya_trace.so")
    ap.add_argument("--probes", action="store_true", help="build only the standalone measurement programs")
    a = ap.parse_args()
    try:
        if a.probes:
            build_probes()
        elif a.tile_trace:
            build_trace(a.jobs)
        else:
            build(a.jobs, force=not a.incremental)
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
