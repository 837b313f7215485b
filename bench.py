"""Throughput of the Laya encoder + decision-head forward pass on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c3] [--no-cpu-baseline]

Workload (default, "c3"): ModernBERT-large encoder + 2-layer decision head, bf16, batch 32,
sequence lengths uniform in [32, 512] (seed 0, packed without padding), 4 option markers per
question, random-init N(0, 0.02) weights from the seeded generator.  A step is one full forward
pass of that batch (embeddings, 28 encoder layers, head, scorer, act head).

Timed region: K back-to-back replays of the pass (HIP graph, inputs resident in HBM; only the
pass's few-KB index arrays are re-copied from pinned memory), bracketed by
torch.cuda.synchronize().  `abi_seqs_per_s` times the same K steps through laya_forward_batch
(host packing, H2D/D2H and synchronisation included).

roofline: per-stage device times are kernel times: with laya_ext_prof_enable every kernel of a
profiled pass records its own start and end (hipExtLaunchKernel events on the engine's stream,
nothing waiting between launches), summed per stage; the dominant kernel's achieved rate is its
algorithmic work per launch (2*M*N*K flops for a GEMM over the valid tokens) divided by its
average launch time.  `traffic` is the dominant kernel's HBM traffic per launch from the
committed rocprofv3 --pmc summary, reported only when that summary was measured on the GEMM
sources being benched (their hash is recorded beside the figure).

cpu_baseline: the CPU PyTorch restatement of the reference path (oracle/model.py, fp32 torch on
this host's cores): the first questions of the same batch (about cpu-budget seconds), plus the
median of five b1 x s128 ModernBERT-large forwards.  The restatement's speed relative to the
reference's own CPU model was measured in the build container (tests/golden/large/cpu_timing.json)
and is reported with it.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

PEAK_BF16 = 2.5e15
PEAK_FP32 = 157.3e12
PEAK_HBM = 8.0e12
PMC_COPY_BYTES = 256 << 20
# calibrated HBM traffic per launch of the dominant kernel, from the committed rocprofv3 --pmc
# summary (FETCH_SIZE and WRITE_SIZE runs of `bench.py --pmc-probe`, scaled by the copy kernel)
TRAFFIC_FILE = os.path.join(REPO, "profiles", "c3_geglu_gemm_hbm_traffic.md")
TRAFFIC_SOURCE = ("rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs of bench.py --pmc-probe, copy-calibrated, "
                  "recorded in profiles/c3_geglu_gemm_hbm_traffic.md for GEMM sources with hash %s (the sources "
                  "benched here)")
# the sources that decide the GEMM kernel's memory traffic
GEMM_SOURCES = [os.path.join(REPO, "layamd_amd", "csrc", f)
                for f in ("kernels_gemm.hip", "gemm_xl_tile.inc", "kernels.h", "common.h")]


def gemm_source_hash():
    import hashlib
    h = hashlib.sha256()
    for f in GEMM_SOURCES:
        with open(f, "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


def measured_traffic(kernel_stage):
    """(bytes per launch, source note) recorded for kernel_stage in the traffic summary when it was
    measured on the GEMM sources of this tree, else (None, why)."""
    rec, src = None, None
    try:
        for line in open(TRAFFIC_FILE):
            if line.startswith("traffic_bytes_per_launch ") and line.split()[1] == kernel_stage:
                rec = int(line.split()[2])
            if line.startswith("gemm_sources_sha256_16 "):
                src = line.split()[1]
    except OSError:
        return None, "no traffic summary"
    if rec is None:
        return None, "no traffic recorded for %s" % kernel_stage
    here = gemm_source_hash()
    if src != here:
        return None, ("the recorded traffic (%d bytes) was measured on GEMM sources %s, not these (%s): dropped"
                      % (rec, src, here))
    return rec, TRAFFIC_SOURCE % here


def stage_work(name, cfg, T, R, KT, B, elt, attn_flops):
    """Algorithmic (flops, bytes) of one launch of a stage; R/KT/B only for the head-1 stages."""
    D, I, FF = cfg.d, cfg.intermediate, cfg.head_ffn
    g = lambda m, n, k: (2.0 * m * n * k, float(elt * (m * k + n * k + m * n)))
    table = {
        "enc:gemm_qkv_rope": g(T, 3 * D, D),
        "enc:gemm_attn_out_res": g(T, D, D),
        "enc:gemm_mlp_in_geglu": g(T, 2 * I, D),
        "enc:gemm_mlp_out_res": g(T, D, I),
        "head:gemm_qkv": g(T, 3 * D, D),
        "scorer:gemm_gelu": g(KT, D, D),
        "enc:embed_ln": (0.0, float(T * D * (4 + 4 + elt))),
        "enc:ln": (0.0, float(T * D * (4 + elt))),
        "enc:final_ln_type": (0.0, float(T * D * 8)),
        "enc:attn_sliding": (attn_flops["sliding"], float(T * D * 4 * elt)),
        "enc:attn_global": (attn_flops["global"], float(T * D * 4 * elt)),
    }
    return table.get(name)


def attention_flops(lens, D, half_window):
    """4*D flops per (query, visible key) pair: QK^T and PV, all heads."""
    s_glob = s_slide = 0
    for L in lens:
        p = np.arange(L)
        s_glob += L * L
        s_slide += int((np.minimum(L, p + half_window + 1) - np.maximum(0, p - half_window)).sum())
    return {"global": 4.0 * D * s_glob, "sliding": 4.0 * D * s_slide}


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_threads():
    """Threads for the CPU baseline: this process's CPU share.  A GPU host gives each GPU's jobs a
    share of its cores (OMP_NUM_THREADS says how many); os.cpu_count() counts the whole machine."""
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    return max(1, min(avail, share) if share > 0 else avail)


def cpu_baseline(cfg_name, batch, budget_s=20.0):
    import statistics
    import torch
    from layamd_amd import checkpoint as ck
    from layamd_amd import workloads as wl
    from oracle import model as om
    threads = cpu_threads()
    torch.set_num_threads(threads)
    cfg, W = ck.load_checkpoint(ck.cached_checkpoint(batch.cfg.name))
    Wt = om.Weights(W)
    idx, n_tok, t_used = [], 0, 0.0
    t0 = time.time()
    for i in range(batch.B):
        t = time.time()
        om.run_batch(Wt, batch.cfg, batch.subset([i]))
        t_used += time.time() - t
        idx.append(i)
        n_tok += int(batch.lens[i])
        if time.time() - t0 > budget_s:
            break
    # b1 x s128 ModernBERT-large, fp32: the configuration the reference's CPU path was timed on
    c1 = wl.c1(0)
    _, W1 = ck.load_checkpoint(ck.cached_checkpoint("large"))
    W1t = om.Weights(W1)
    ms = []
    for r in range(2 + 5):
        t = time.perf_counter()
        om.run_batch(W1t, c1.cfg, c1)
        if r >= 2:
            ms.append(1e3 * (time.perf_counter() - t))
    ratio = None
    try:
        with open(os.path.join(REPO, "tests", "golden", "large", "cpu_timing.json")) as f:
            ratio = json.load(f)
    except OSError:
        pass
    out = {"value": round(len(idx) / t_used, 4), "unit": "seqs/s", "cores": threads, "kind": "port",
           "tokens_per_s": round(n_tok / t_used, 1),
           "c1_b1s128_ms_median": round(statistics.median(ms), 2),
           "os_cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads(), "cpu_model": cpu_model(),
           "sample": "first %d of the %d questions (%d tokens) of %s, fp32 CPU PyTorch restatement of the reference "
                     "path (oracle/model.py), one question per forward like the engine's packing, on %d threads (this "
                     "process's CPU share; the host has %s logical CPUs); plus the median of 5 b1 x s128 forwards"
                     % (len(idx), batch.B, n_tok, batch.name, threads, os.cpu_count())}
    if ratio:
        out["restatement_over_reference"] = ratio["restatement_over_reference"]
        out["ratio_measured_on"] = "%s, %d threads, %s (reference DecisionModel %.1f ms, restatement %.1f ms at b1 x s128)" % (
            ratio["cpu_model"], ratio["threads"], ratio["torch"], ratio["reference_ms_median"], ratio["restatement_ms_median"])
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c3", choices=["c3", "c4", "c5", "c1"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--stage-sequence", default=None, metavar="FILE",
                    help="write the stage of every kernel launch of one pass, in launch order (to read a kernel "
                         "trace of the same run per stage: python -m layamd_amd.trace_table)")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="for rocprofv3 --pmc runs: one plain copy of 256 MiB (the counter calibration), then "
                         "three forward passes without graphs, then exit")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: the decision pass is data parallel with no cross-GPU exchange, "
              "so only --gpus 1 is supported", file=sys.stderr)
        sys.exit(2)

    import torch
    from layamd_amd import checkpoint as ck
    from layamd_amd import engine as le
    from layamd_amd import workloads as wl

    batch = wl.CONFIGS[a.config](0)
    cfg = batch.cfg
    precision = batch.dtype
    elt = 2 if precision == "bf16" else 4
    t0 = time.time()
    mdir = ck.cached_checkpoint(cfg.name)
    print("[bench] checkpoint %s ready in %.1fs" % (mdir, time.time() - t0), file=sys.stderr, flush=True)
    max_tokens = max(16384, int(batch.tokens) + 1024)
    env = {"LAYA_MAX_TOKENS": max_tokens, "LAYA_GRAPHS": 0 if a.pmc_probe else 1, "LAYA_DUMP_DIR": None,
           "LAYA_PROFILE": None}
    if a.pmc_probe:
        # counter runs serialize every dispatch, so tile timing is meaningless there: pin the plan the
        # tuner picks for the dominant stage at this workload: 192x128 tiles (two per CU) over the rows
        # that fill whole rounds of the 2 x 256 slots, 128x64 tiles over the rest, in one launch
        rows = -(-int(sum(-(-int(L) // 8) * 8 for L in batch.lens)) // 64) * 64
        tn = -(-2 * cfg.intermediate // 128)            # Wi: both GeGLU halves
        split = -(-rows // 192) * tn // 512 * 512 // tn * 192
        env.update({"LAYA_GEMM_CFG": 7, "LAYA_GEMM_SPLIT": "%d,8" % split} if 0 < split < rows else {"LAYA_GEMM_CFG": 7})
    eng = le.Engine(None, mdir, precision=precision, env=env)
    flat = batch.flat()
    if a.pmc_probe:
        src = torch.ones(PMC_COPY_BYTES, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)                                    # reads and writes exactly PMC_COPY_BYTES
        torch.cuda.synchronize()
        del src, dst
        for _ in range(3):
            eng.forward_flat(*flat)
        torch.cuda.synchronize()
        print("[bench] pmc probe done: copy of %d bytes, 3 passes of %s" % (PMC_COPY_BYTES, batch.name), file=sys.stderr)
        return
    for _ in range(max(1, a.warmup)):
        eng.forward_flat(*flat)
    torch.cuda.synchronize()

    # timed region: K device-resident replays of the pass
    torch.cuda.synchronize()
    t = time.perf_counter()
    dev_ms = eng.replay(a.steps)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t
    ms_per_step = 1000.0 * wall / a.steps
    seqs_s = batch.B * a.steps / wall
    tok_s = batch.tokens * a.steps / wall

    # same K steps through the C ABI (host packing + copies included)
    torch.cuda.synchronize()
    t = time.perf_counter()
    for _ in range(a.steps):
        eng.forward_flat(*flat)
    torch.cuda.synchronize()
    abi_wall = time.perf_counter() - t
    print("[bench] %s: %.3f ms/step (device %.3f ms), %.1f seqs/s, %.0f tok/s; ABI %.3f ms/step"
          % (a.config, ms_per_step, dev_ms / a.steps, seqs_s, tok_s, 1000 * abi_wall / a.steps),
          file=sys.stderr, flush=True)

    # per-stage kernel times (each kernel's own start and end events, graphs bypassed)
    eng.prof_enable(True)
    eng.prof_reset()
    n_prof = 3
    for _ in range(n_prof):
        eng.forward_flat(*flat)
    stages = eng.prof_stages()
    if a.stage_sequence:
        with open(a.stage_sequence, "w") as f:
            f.write("\n".join(eng.prof_sequence()) + "\n")
    eng.prof_enable(False)
    eng.prof_report(n_prof)
    sys.stdout.flush()

    # achievable peaks on this box, outside the timed region: a register-only MFMA loop on every
    # CU (the clock the chip holds under MFMA load) and the faster of two device copies of 1 GiB,
    # the library's non-temporal stream copy and torch's device-to-device copy
    mfma_ach = le.mfma_peak(eng.lib)
    # the same loop held for ~20 ms, about twice a pass: the clock the chip sustains under MFMA load
    mfma_sus = le.mfma_peak(eng.lib, iters=4096 * 40)
    stream_gbs = le.hbm_peak(eng.lib, 1 << 30, 5)
    src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(5):
        dst.copy_(src)
    ev1.record()
    torch.cuda.synchronize()
    torch_gbs = 2.0 * (1 << 30) * 5 / (ev0.elapsed_time(ev1) * 1e-3) / 1e9
    del src, dst
    copy_gbs = max(stream_gbs, torch_gbs)
    achievable = {"mfma_bf16_tflops": round(mfma_ach, 1), "mfma_bf16_tflops_sustained_20ms": round(mfma_sus, 1),
                  "hbm_copy_gbs": round(copy_gbs, 1),
                  "stream_copy_gbs": round(stream_gbs, 1), "torch_copy_gbs": round(torch_gbs, 1),
                  "method": "register-only v_mfma_f32_32x32x16_bf16 loop, 2 workgroups of 4 waves per CU "
                            "(laya_ext_mfma_loop), about 0.5 ms (burst) and about 20 ms (sustained: the clock the "
                            "chip holds under continuous MFMA load); the faster of two device copies of 1 GiB, read + write bytes: "
                            "the library's non-temporal 16-byte stream copy (laya_ext_hbm_copy) and torch's "
                            "device-to-device copy"}

    T, B, KT = batch.tokens, batch.B, int(batch.nmark.sum())
    R = KT + B
    af = attention_flops(batch.lens, cfg.d, cfg.local_attention // 2)
    kernels = {}
    gemm_flops = gemm_ms = 0.0
    for name, (ms, calls) in stages.items():
        w = stage_work(name, cfg, T, R, KT, B, elt, af)
        avg_ms = ms / calls
        entry = {"ms_per_launch": round(avg_ms, 5), "launches_per_step": calls // n_prof}
        if w is not None:
            fl, by = w
            if fl and "gemm" in name:
                entry["tflops"] = round(fl / (avg_ms * 1e-3) / 1e12, 1)
                entry["frac_mfma"] = round(fl / (avg_ms * 1e-3) / (PEAK_BF16 if elt == 2 else PEAK_FP32), 4)
                if elt == 2:
                    entry["frac_achievable_mfma"] = round(fl / (avg_ms * 1e-3) / 1e12 / mfma_ach, 4)
                if name.startswith("enc:"):
                    gemm_flops += fl * calls
                    gemm_ms += ms
            else:
                entry["gbs"] = round(by / (avg_ms * 1e-3) / 1e9, 1)
                entry["frac_hbm"] = round(by / (avg_ms * 1e-3) / PEAK_HBM, 4)
                entry["frac_achievable_hbm"] = round(by / (avg_ms * 1e-3) / 1e9 / copy_gbs, 4)
                if fl:
                    entry["tflops"] = round(fl / (avg_ms * 1e-3) / 1e12, 1)
        kernels[name] = entry
    dom = max((n for n in stages if stage_work(n, cfg, T, R, KT, B, elt, af) is not None), key=lambda n: stages[n][0])
    fl, by = stage_work(dom, cfg, T, R, KT, B, elt, af)
    dom_ms = stages[dom][0] / stages[dom][1]
    if fl and "gemm" in dom:
        ach = fl / (dom_ms * 1e-3) / 1e12
        peak = (PEAK_BF16 if elt == 2 else PEAK_FP32) / 1e12
        traffic, tsrc = measured_traffic(dom)
        roof = {"bound": "mfma", "achieved": round(ach, 1), "peak": peak, "unit": "TFLOP/s",
                "frac": round(ach / peak, 4), "traffic": traffic, "traffic_source": tsrc,
                "kernel": dom,
                "work_per_launch": "2*T*N*K = %.4g flop (T=%d valid tokens)" % (fl, T),
                "achievable_peak": round(mfma_ach, 1), "frac_of_achievable": round(ach / mfma_ach, 4)}
    else:
        ach = by / (dom_ms * 1e-3) / 1e9
        traffic, tsrc = measured_traffic(dom)
        roof = {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                "frac": round(ach / (PEAK_HBM / 1e9), 4), "traffic": traffic, "traffic_source": tsrc,
                "kernel": dom,
                "achievable_peak": round(copy_gbs, 1), "frac_of_achievable": round(ach / copy_gbs, 4)}

    cpu = None
    if not a.no_cpu_baseline:
        cpu = cpu_baseline(a.config, batch, a.cpu_budget)

    line = {
        "metric": "seqs/s & tokens/s, ModernBERT-large bf16 b32xs512, 1 GPU; GEMM MFMA util %"
                  if a.config == "c3" else "seqs/s (%s)" % batch.name,
        "value": round(seqs_s, 2), "unit": "seqs/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": precision, "data": "synthetic (seeded token ids, random-init N(0,0.02) weights)",
        "config": {"workload": batch.name, "model": cfg.name, "layers": cfg.n_layers, "d_model": cfg.d,
                   "global_batch": batch.B, "seq_len": int(cfg.max_len), "valid_tokens": T,
                   "markers": KT, "parallelism": "single GPU"},
        "tokens_per_s": round(tok_s, 1),
        "padded_slots_per_s": round(batch.B * cfg.max_len * a.steps / wall, 1),
        "abi_seqs_per_s": round(batch.B * a.steps / abi_wall, 2),
        "mfma_util_encoder_gemms": round(gemm_flops / (gemm_ms * 1e-3) / (PEAK_BF16 if elt == 2 else PEAK_FP32), 4)
        if gemm_ms else None,
        "roofline": roof,
        "cpu_baseline": cpu,
        "achievable": achievable,
        "kernels": kernels,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
