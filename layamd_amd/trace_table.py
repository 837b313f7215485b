"""Reads a rocprofv3 kernel trace of bench.py per stage of the pass:

    rocprofv3 --kernel-trace --output-format csv -d OUT -o run -- python3 bench.py --stage-sequence SEQ ...
    python -m layamd_amd.trace_table OUT/.../run_kernel_trace.csv SEQ [--bench BENCH_LOG]

SEQ (written by `bench.py --stage-sequence`) holds the stage of every kernel launch of one pass, in
launch order, as the engine's profiler recorded it.  Graph replays launch the same kernels in the
same order, so each pass of the trace can be read launch by launch.  The trace is cut into passes
after each act-head output kernel (the last kernel of a pass); the runtime's copy kernels are left
out.  Passes whose kernel count is not the sequence's (the first pass, which also holds the tile
tuner's launches) are skipped; the last three are bench.py's profiled passes (run eagerly, each
kernel with its own timing events, the passes the bench line's stage times come from), the rest
graph replays.  Per stage it prints the kernels and executions per pass and the kernel time per
execution in both sets, and, with the bench line (BENCH_LOG: bench.py's output, the JSON line
last), the bench's `kernels.<stage>.ms_per_launch` beside them.

In graph replays the kernels run back to back and each one's recorded start precedes the previous
one's end (the next dispatch is processed while the previous drains): their durations include that
wait, about 1 us, and sum to the pass's span.  The eager passes leave 8-9 us between kernels.
"""
import argparse
import csv
import json
import statistics


def passes_of(trace_csv):
    rows = list(csv.DictReader(open(trace_csv)))
    rows = [r for r in rows if "__amd_rocclr" not in r["Kernel_Name"]]
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    out, cur = [], []
    for r in rows:
        cur.append(r)
        if "k_act_out" in r["Kernel_Name"]:
            out.append(cur)
            cur = []
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("trace_csv")
    ap.add_argument("sequence")
    ap.add_argument("--bench", default=None)
    ap.add_argument("--eager", type=int, default=3, help="trailing full-length passes that ran eagerly (profiled)")
    a = ap.parse_args()
    seq = [l.strip() for l in open(a.sequence) if l.strip()]
    allp = passes_of(a.trace_csv)
    full = [p for p in allp if len(p) == len(seq)]
    sel = full[:len(full) - a.eager] if a.eager else full
    eag = full[len(full) - a.eager:] if a.eager else []
    if not sel:
        raise SystemExit("no pass of %d kernels in the trace (pass sizes: %s)" % (len(seq), [len(p) for p in allp]))
    names = [r["Kernel_Name"] for r in sel[0]]
    assert all([r["Kernel_Name"] for r in p] == names for p in sel), "passes launch different kernels"
    # executions of a stage: runs of consecutive launches of it
    execs = {}
    for i, s in enumerate(seq):
        if i == 0 or seq[i - 1] != s:
            execs[s] = execs.get(s, 0) + 1
    order, tot, tote, kern = [], {}, {}, {}
    dur = lambda r: (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    for i, s in enumerate(seq):
        if s not in tot:
            order.append(s)
            tot[s] = tote[s] = 0.0
            kern[s] = set()
        kern[s].add(names[i])
        tot[s] += sum(dur(p[i]) for p in sel)
        tote[s] += sum(dur(p[i]) for p in eag)
    bench = {}
    if a.bench:
        line = [l for l in open(a.bench) if l.startswith("{")][-1]
        bench = json.loads(line).get("kernels", {})
    span = statistics.mean((int(p[-1]["End_Timestamp"]) - int(p[0]["Start_Timestamp"])) / 1e3 for p in sel)
    ksum = sum(tot.values()) / len(sel)
    print("%d graph-replayed and %d eager passes of %d kernels (of %d passes in the trace); graph-replayed pass: "
          "span %.1f us, kernel time %.1f us" % (len(sel), len(eag), len(seq), len(allp), span, ksum))
    print()
    print("| stage | executions / pass | kernels / pass | us per execution, graph replays | us per execution, eager "
          "passes | bench ms_per_launch (us) | bench / eager | bench / graph |")
    print("|---|---:|---:|---:|---:|---:|---:|---:|")
    f = lambda x: "%.3f" % x if x else ""
    for s in sorted(order, key=lambda s: -tot[s]):
        per = tot[s] / len(sel) / execs[s]
        pe = tote[s] / len(eag) / execs[s] if eag else None
        b = bench.get(s, {}).get("ms_per_launch")
        b = b * 1e3 if b else None
        print("| %s | %d | %d | %.2f | %s | %s | %s | %s |" % (s, execs[s], seq.count(s), per, "%.2f" % pe if pe else "",
                                                          "%.2f" % b if b else "", f(b / pe if b and pe else None),
                                                          f(b / per if b else None)))
    print()
    print("Kernels per stage:")
    for s in order:
        print("- %s: %s" % (s, ", ".join("`%s`" % k[:110] for k in sorted(kern[s]))))


if __name__ == "__main__":
    main()
