"""The measurement tools behind the committed profile summaries, without a GPU:
layamd_amd/trace_table.py reading a synthetic kernel trace per stage of the pass, and the traffic
record that bench.py reports belonging to the GEMM sources in the tree."""
import csv
import json
import subprocess
import sys

import pytest

from layamd_amd import trace_table

FIELDS = ["Kernel_Name", "Start_Timestamp", "End_Timestamp"]
# one pass: a LayerNorm, one GEMM stage of two launches (a row split), the act head's last kernel
SEQ = ["enc:ln", "enc:gemm", "enc:gemm", "act_head"]
NAMES = ["void laya::k_layernorm<float>()", "void laya::k_gemm_xl<7>()", "void laya::k_gemm_xl<3>()",
         "laya::k_act_out(float const*)"]


def _trace(path):
    """A trace of 7 passes (times in ns): the first with two extra tuning launches, three graph
    replays (kernels back to back, each start 1 us before the previous end; durations 10, 20, 20,
    5 us), then three eager passes (8 us gaps; durations 9, 19, 19, 4 us), plus a runtime copy
    kernel that the tool leaves out."""
    rows, t = [], 1_000_000

    def add(name, dur_us, gap_us):
        nonlocal t
        t += int(gap_us * 1000)
        rows.append({"Kernel_Name": name, "Start_Timestamp": t, "End_Timestamp": t + int(dur_us * 1000)})
        t += int(dur_us * 1000)

    add("void laya::k_gemm_xl<0>()", 30, 5)                 # tuning launches of the first pass
    add("void laya::k_gemm_xl<5>()", 30, 5)
    for n, d in zip(NAMES, (10, 20, 20, 5)):
        add(n, d, 8)
    for _ in range(3):
        for n, d in zip(NAMES, (10, 20, 20, 5)):
            add(n, d, -1)
    add("__amd_rocclr_copyBuffer", 3, 2)
    for _ in range(3):
        for n, d in zip(NAMES, (9, 19, 19, 4)):
            add(n, d, 8)
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, FIELDS)
        w.writeheader()
        w.writerows(rows)


def test_trace_table_reads_passes_per_stage(tmp_path):
    tr, seq, bench = tmp_path / "trace.csv", tmp_path / "seq.txt", tmp_path / "bench.log"
    _trace(tr)
    seq.write_text("\n".join(SEQ) + "\n")
    bench.write_text("[bench] log line\n" + json.dumps({"kernels": {"enc:gemm": {"ms_per_launch": 0.038},
                                                                   "enc:ln": {"ms_per_launch": 0.0099}}}) + "\n")
    passes = trace_table.passes_of(str(tr))
    assert [len(p) for p in passes] == [6, 4, 4, 4, 4, 4, 4]       # cut after each act-head kernel, copies dropped
    out = subprocess.run([sys.executable, "-m", "layamd_amd.trace_table", str(tr), str(seq), "--bench", str(bench)],
                         capture_output=True, text=True, check=True).stdout
    assert out.startswith("3 graph-replayed and 3 eager passes of 4 kernels (of 7 passes in the trace)")
    rows = {l.split("|")[1].strip(): [c.strip() for c in l.split("|")[2:-1]] for l in out.splitlines()
            if l.startswith("| enc:") or l.startswith("| act_head")}
    # stage: executions per pass (runs of consecutive launches), kernels per pass, us per execution in
    # the graph replays and in the eager passes, the bench line's figure and its two ratios
    assert rows["enc:gemm"][:4] == ["1", "2", "40.00", "38.00"]
    assert rows["enc:gemm"][4:] == ["38.00", "1.000", "0.950"]
    assert rows["enc:ln"][:5] == ["1", "1", "10.00", "9.00", "9.90"]
    assert rows["act_head"][:4] == ["1", "1", "5.00", "4.00"]
    # the graph-replayed pass spans its kernels minus the three 1 us overlaps
    assert "span 52.0 us, kernel time 55.0 us" in out


def test_trace_table_rejects_a_trace_without_the_sequence(tmp_path):
    tr, seq = tmp_path / "trace.csv", tmp_path / "seq.txt"
    _trace(tr)
    seq.write_text("\n".join(SEQ + ["enc:extra"]) + "\n")
    r = subprocess.run([sys.executable, "-m", "layamd_amd.trace_table", str(tr), str(seq)], capture_output=True, text=True)
    assert r.returncode != 0 and "no pass of 5 kernels" in r.stderr


def test_recorded_traffic_belongs_to_these_gemm_sources():
    """bench.py reports the dominant GEMM's fabric traffic from the counter runs recorded in
    profiles/ only for the GEMM sources those runs measured (their hash is recorded beside the
    figure).  The committed record must belong to the committed sources: a change to the GEMM
    sources needs the two counter runs again."""
    import importlib.util
    import os
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    spec = importlib.util.spec_from_file_location("bench_module", os.path.join(root, "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    rec, note = bench.measured_traffic("enc:gemm_mlp_in_geglu")
    assert rec is not None, note
    assert rec > 81e6                     # at least the operands and output (81.2 MB per launch)


if __name__ == "__main__":
    sys.exit(pytest.main([__file__, "-q"]))
