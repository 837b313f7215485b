"""Times the reference's own CPU PyTorch model and this repo's CPU restatement on the same C1
input (ModernBERT-large + head, fp32, batch 1 x 128), in the build container only.

    python tests/golden/time_reference_c1.py [--threads 8] [--runs 10]

The reference is ref/rl_common.py's DecisionModel built offline exactly as make_golden.py builds
it; the restatement is oracle/model.py.  Both run on the seed-0 checkpoint with
torch.set_num_threads(threads): three warm-up forwards, then the median of `runs` timed forwards.
Writes tests/golden/large/cpu_timing.json (data only): both medians, their ratio, the thread count
and the CPU model.  bench.py reports the ratio next to the restatement's timing on the GPU host,
where the reference's Python is not available.
"""
import argparse
import json
import os
import platform
import statistics
import sys
import time

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)
sys.path.insert(0, HERE)

from layamd_amd import checkpoint as ck  # noqa: E402
from layamd_amd import workloads as wl  # noqa: E402
from make_golden import load_reference_model  # noqa: E402
from oracle import model as om  # noqa: E402


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def median_ms(fn, runs):
    for _ in range(3):
        fn()
    t = []
    for _ in range(runs):
        a = time.perf_counter()
        fn()
        t.append(1e3 * (time.perf_counter() - a))
    return statistics.median(t), t


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--threads", type=int, default=8)
    ap.add_argument("--runs", type=int, default=10)
    a = ap.parse_args()
    torch.set_num_threads(a.threads)
    torch.set_grad_enabled(False)
    mdir = ck.cached_checkpoint("large")
    b = wl.c1(0)
    ids, att, mpos, mmask, qt = (torch.as_tensor(x) for x in b.padded())
    ref = load_reference_model(mdir)
    _, W = ck.load_checkpoint(mdir)
    Wt = om.Weights(W)
    cfg = ck.PRESETS["large"]
    ref_ms, ref_all = median_ms(lambda: ref(ids, att, mpos, mmask, qt), a.runs)
    ora_ms, ora_all = median_ms(lambda: om.forward(Wt, cfg, ids, att, mpos, mmask, qt), a.runs)
    lo_ref, _ = ref(ids, att, mpos, mmask, qt)
    lo_ora, _ = om.forward(Wt, cfg, ids, att, mpos, mmask, qt)
    out = {"workload": b.name, "threads": a.threads, "cpu_model": cpu_model(), "os_cpu_count": os.cpu_count(),
           "runs": a.runs, "warmups": 3, "reference_ms_median": round(ref_ms, 2),
           "restatement_ms_median": round(ora_ms, 2), "restatement_over_reference": round(ora_ms / ref_ms, 3),
           "max_abs_logit_difference": float(np.abs(lo_ref.numpy() - lo_ora.numpy()).max()),
           "reference_ms_all": [round(x, 2) for x in ref_all], "restatement_ms_all": [round(x, 2) for x in ora_all],
           "torch": torch.__version__}
    path = os.path.join(HERE, "large", "cpu_timing.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out, indent=1))


if __name__ == "__main__":
    main()
