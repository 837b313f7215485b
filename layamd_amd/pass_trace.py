"""Passes of one batch shape, for a kernel trace read per stage by layamd_amd.trace_table:

    rocprofv3 --kernel-trace --output-format csv -d OUT -o run -- \\
        python3 -m layamd_amd.pass_trace --questions 1 --tokens 128 [--latency] --sequence SEQ
    python -m layamd_amd.trace_table OUT/run_kernel_trace.csv SEQ

Builds a bf16 engine on the seeded ModernBERT-large checkpoint (LAYA_LATENCY=1 with --latency),
runs the batch (questions x tokens, 4 markers each) twice (eager, then graph capture), replays the
graph --replays times and prints the device time per replayed pass (event-timed), then runs three
profiled eager passes and writes the stage of each of the pass's kernel launches to SEQ, in launch
order, as bench.py --stage-sequence does for the benchmark batches.

Under the kernel trace, the host's submission of a graph's launches slows down (the profiler
handles every dispatch), so a pass whose kernels are short can end up waiting for its launches:
read the per-stage kernel times from such a trace, and the pass time from a run without it.
"""
import argparse


def main():
    from layamd_amd import checkpoint as ck
    from layamd_amd import engine as le
    from layamd_amd import workloads as wl
    ap = argparse.ArgumentParser()
    ap.add_argument("--questions", type=int, default=1)
    ap.add_argument("--tokens", type=int, default=128)
    ap.add_argument("--latency", action="store_true", help="LAYA_LATENCY=1 (split-K residual GEMMs)")
    ap.add_argument("--replays", type=int, default=20)
    ap.add_argument("--sequence", required=True, metavar="FILE")
    a = ap.parse_args()
    d = ck.cached_checkpoint("large")
    e = le.Engine(None, d, precision="bf16", env={"LAYA_LATENCY": "1" if a.latency else "0"})
    batch = wl.make_batch(ck.PRESETS["large"], [a.tokens] * a.questions, [4] * a.questions, seed=5)
    flat = batch.flat()
    e.forward_flat(*flat)
    e.forward_flat(*flat)
    print("%d x %d tokens%s: %.3f ms per replayed pass (device)"
          % (a.questions, a.tokens, ", LAYA_LATENCY=1" if a.latency else "", e.replay(a.replays) / a.replays),
          flush=True)
    e.prof_enable(True)
    for _ in range(3):
        e.forward_flat(*flat)
    with open(a.sequence, "w") as f:
        f.write("\n".join(e.prof_sequence()) + "\n")
    e.prof_enable(False)


if __name__ == "__main__":
    main()
