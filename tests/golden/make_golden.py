"""Write golden vectors from the reference's own PyTorch model (run in the build container only).

    python tests/golden/make_golden.py [--only tiny|large|base]

It imports the reference DecisionModel (ref/rl_common.py:81-134, built offline with
build_model(cfg, encoder_dir=...) exactly as ref/rl_agent_api.py:21-22 does) and runs it on CPU
in float32 on checkpoints written by layamd_amd.checkpoint (seeded, so the GPU side regenerates
the same weights).  Hooks capture the activations the way ref/gen_golden.py:58-71 does.

Output (data only; no reference code is copied):

  tests/golden/tiny/manifest.json + <case>/*.bin   the reference golden format
      (ref/gen_golden.py:86-105, read by src/test_parity.cpp:25-42): int32 inputs
      input_ids/attention_mask/marker_pos/marker_mask/qtype, float32 logits/act_logits, and
      for the "dump" cases float32 [n, L, D] emb/enc*/final_norm/head* (right-padded rows).
  tests/golden/<large|base>/golden.npz             full-size configs: inputs, logits, act
      logits, the bf16-autocast logits of the same model (its own drift, as ref/bf16_drift.py
      measures it), and per layer a few sampled rows plus per-layer row statistics, in fp32 and
      under the same bf16 autocast (<layer>_rows_bf16_autocast: the reference's own per-layer
      bf16 drift, the bar for the engine's bf16 path).  The autocast values depend on the host's
      bf16 GEMM kernels: another thread count sums in another order, about one bf16 ulp of a logit.
  tests/golden/<c3|c4|c5>_sample/drift.npz          a few questions of the bf16 benchmark batches
      (ModernBERT-large b32 x s512, mmBERT-base b16 x s1024, ModernBERT-large-1024 b64 varlen) run
      by the reference in fp32 and under bf16 autocast: fp32 and autocast logits and act logits,
      and per layer the reference's own bf16 drift over all valid rows, max |x_bf16 - x_fp32| /
      rms(x_fp32 row) (scalars only; the engine's fp32 side is the oracle on the GPU host).
  tests/golden/<c3|c4|c5>_full/drift.npz           the same record for every question of the
      b32 x s512, b16 x s1024 and b64 varlen batches (32, 16 and 64 questions; lengths up to 510,
      1020 and 1024).
"""
import argparse
import json
import os
import sys
import tempfile

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

from layamd_amd import checkpoint as ck  # noqa: E402
from layamd_amd import workloads as wl  # noqa: E402

REF = "/root/reference/ref"

TINY_JITTER = 0.1
# (case name, lens, nmarks, dump per-layer activations)
TINY_CASES = [
    ("mixed", [1, 39, 100], [1, 2, 5], True),
    ("long_sliding", [260], [12], True),
    ("multi_q", [218, 199, 215], [5, 3, 2], False),
    ("short", [71], [4], False),
    ("full_ctx", [320], [3], False),
]
SAMPLE_ROWS = [0, 1, 63, 127]


def load_reference_model(model_dir):
    sys.path.insert(0, REF)
    from rl_common import build_model  # the reference's own model builder
    from safetensors.torch import load_file
    with open(os.path.join(model_dir, "rl_agent_config.json")) as f:
        cfg = json.load(f)
    model = build_model(cfg, encoder_dir=os.path.join(model_dir, "encoder"))
    model.load_state_dict(load_file(os.path.join(model_dir, "model.safetensors")), strict=True)
    model.float().eval()
    return model


def hooks(model, acts):
    hs = []

    def cap(name):
        def fn(mod, inp, out):
            t = out[0] if isinstance(out, tuple) else out
            if torch.is_tensor(t):
                acts[name] = t.detach().float().cpu().numpy()
        return fn
    enc = model.encoder
    hs.append(enc.embeddings.register_forward_hook(cap("emb")))
    for i, lyr in enumerate(enc.layers):
        hs.append(lyr.register_forward_hook(cap("enc%d" % i)))
    hs.append(enc.final_norm.register_forward_hook(cap("final_norm")))
    for i, lyr in enumerate(model.head.layers):
        hs.append(lyr.register_forward_hook(cap("head%d" % i)))
    return hs


def run(model, batch, acts):
    ids, att, mpos, mmask, qt = batch.padded()
    acts.clear()
    with torch.no_grad():
        logits, act = model(torch.as_tensor(ids), torch.as_tensor(att), torch.as_tensor(mpos),
                            torch.as_tensor(mmask), torch.as_tensor(qt))
    return (ids, att, mpos, mmask, qt), logits.float().numpy(), act.float().numpy()


def tiny(out_root, work):
    cfg = ck.PRESETS["tiny"]
    mdir = ck.write_checkpoint(os.path.join(work, "tiny"), cfg, seed=0, ln_jitter=TINY_JITTER)
    model = load_reference_model(mdir)
    acts = {}
    hs = hooks(model, acts)
    out = os.path.join(out_root, "tiny")
    manifest = {"model": {"preset": "tiny", "seed": 0, "ln_jitter": TINY_JITTER, "std": 0.02, "dtype": "F32"},
                "cases": []}
    for ci, (name, lens, nm, dump) in enumerate(TINY_CASES):
        b = wl.make_batch(cfg, lens, nm, seed=100 + ci, dtype="fp32", name=name)
        (ids, att, mpos, mmask, qt), logits, act = run(model, b, acts)
        cdir = os.path.join(out, name)
        os.makedirs(cdir, exist_ok=True)
        rec = {"name": name, "seed": 100 + ci, "shapes": {}}

        def save(fn, arr, dt=np.float32):
            arr = np.ascontiguousarray(np.asarray(arr).astype(dt))
            arr.tofile(os.path.join(cdir, fn + ".bin"))
            rec["shapes"][fn] = list(arr.shape)
        save("input_ids", ids, np.int32)
        save("attention_mask", att, np.int32)
        save("marker_pos", mpos, np.int32)
        save("marker_mask", mmask, np.int32)
        save("qtype", qt, np.int32)
        save("logits", logits)
        save("act_logits", act)
        if dump:
            for k in ["emb"] + ["enc%d" % i for i in range(cfg.n_layers)] + ["final_norm"] + \
                     ["head%d" % i for i in range(cfg.head_layers)]:
                save(k, acts[k])
        rec["seq_lens"] = [int(x) for x in att.sum(-1)]
        manifest["cases"].append(rec)
        print("[golden] tiny/%-13s lens=%s K=%s" % (name, rec["seq_lens"], nm), flush=True)
    for h in hs:
        h.remove()
    with open(os.path.join(out, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1)


def full_size(out_root, work, preset, batch_fn, tag):
    cfg = ck.PRESETS[preset]
    mdir = ck.write_checkpoint(os.path.join(work, preset), cfg, seed=0)
    model = load_reference_model(mdir)
    acts = {}
    hs = hooks(model, acts)
    b = batch_fn()
    (ids, att, mpos, mmask, qt), logits, act = run(model, b, acts)
    rows = [r for r in SAMPLE_ROWS if r < int(b.lens[0])]
    rec = {"input_ids": ids.astype(np.int32), "attention_mask": att.astype(np.int32),
           "marker_pos": mpos.astype(np.int32), "marker_mask": mmask.astype(np.int32),
           "qtype": qt.astype(np.int32), "logits": logits, "act_logits": act,
           "sample_rows": np.array(rows, np.int32)}
    names = ["emb"] + ["enc%d" % i for i in range(cfg.n_layers)] + ["final_norm"] + \
            ["head%d" % i for i in range(cfg.head_layers)]
    for k in names:
        a = acts[k][0, :int(b.lens[0])]
        rec[k + "_rows"] = a[rows].astype(np.float32)
        rec[k + "_stats"] = np.array([a.mean(), np.abs(a).max(), np.sqrt((a.astype(np.float64) ** 2).sum())], np.float64)
    acts.clear()
    with torch.no_grad(), torch.autocast("cpu", dtype=torch.bfloat16):
        l16, a16 = model(torch.as_tensor(ids), torch.as_tensor(att), torch.as_tensor(mpos),
                         torch.as_tensor(mmask), torch.as_tensor(qt))
    for h in hs:
        h.remove()
    rec["logits_bf16_autocast"] = l16.float().numpy()
    rec["act_logits_bf16_autocast"] = a16.float().numpy()
    for k in names:
        rec[k + "_rows_bf16_autocast"] = acts[k][0, :int(b.lens[0])][rows].astype(np.float32)
    os.makedirs(os.path.join(out_root, tag), exist_ok=True)
    np.savez(os.path.join(out_root, tag, "golden.npz"), **rec)
    with open(os.path.join(out_root, tag, "manifest.json"), "w") as f:
        json.dump({"model": {"preset": preset, "seed": 0, "ln_jitter": 0.0, "std": 0.02, "dtype": "F32"},
                   "batch": b.name, "lens": [int(x) for x in b.lens], "nmark": [int(x) for x in b.nmark],
                   "layers": names}, f, indent=1)
    print("[golden] %s: lens=%s logits=%s" % (tag, list(b.lens), logits.tolist()), flush=True)


def batch_drift(out_root, work, preset, batch, tag):
    """The reference's own bf16-autocast drift on a few questions of a benchmark batch."""
    cfg = ck.PRESETS[preset]
    mdir = ck.write_checkpoint(os.path.join(work, preset), cfg, seed=0)
    model = load_reference_model(mdir)
    acts, acts16 = {}, {}
    hs = hooks(model, acts)
    _, logits, act = run(model, batch, acts)
    fp32 = {k: v.copy() for k, v in acts.items()}
    ids, att, mpos, mmask, qt = batch.padded()
    acts.clear()
    with torch.no_grad(), torch.autocast("cpu", dtype=torch.bfloat16):
        l16, a16 = model(torch.as_tensor(ids), torch.as_tensor(att), torch.as_tensor(mpos),
                         torch.as_tensor(mmask), torch.as_tensor(qt))
    for h in hs:
        h.remove()
    names = ["emb"] + ["enc%d" % i for i in range(cfg.n_layers)] + ["final_norm"] + \
            ["head%d" % i for i in range(cfg.head_layers - 1)]
    drift = np.zeros((len(names), batch.B))
    for li, k in enumerate(names):
        for i in range(batch.B):
            a = fp32[k][i, :int(batch.lens[i])].astype(np.float64)
            b = acts[k][i, :int(batch.lens[i])].astype(np.float64)
            rms = np.sqrt((a ** 2).mean(1))
            drift[li, i] = (np.abs(b - a).max(1) / rms).max()
    rec = {"lens": np.asarray(batch.lens, np.int32), "nmark": batch.nmark, "layers": np.array(names),
           "rel_drift_bf16_autocast": drift, "logits": logits, "act_logits": act,
           "logits_bf16_autocast": l16.float().numpy(), "act_logits_bf16_autocast": a16.float().numpy()}
    os.makedirs(os.path.join(out_root, tag), exist_ok=True)
    np.savez(os.path.join(out_root, tag, "drift.npz"), **rec)
    print("[golden] %s: lens=%s worst layer drift %.4f" % (tag, list(batch.lens), drift.max()), flush=True)


# questions of the bf16 benchmark batches whose reference bf16 drift is recorded
DRIFT_SAMPLES = {"c3_sample": ("large", "c3", [0, 1, 2, 3]), "c4_sample": ("base", "c4", [11, 15]),
                 "c5_sample": ("large1024", "c5", [50, 17, 24]),
                 # every question of the benchmark batches (b32 x s512, b16 x s1024, b64 varlen)
                 "c3_full": ("large", "c3", list(range(32))), "c4_full": ("base", "c4", list(range(16))),
                 "c5_full": ("large1024", "c5", list(range(64)))}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--only", default="")
    ap.add_argument("--work", default=os.path.join(tempfile.gettempdir(), "laya_golden_ckpt"))
    ap.add_argument("--out", default=HERE, help="output root (default: next to this script)")
    a = ap.parse_args()
    torch.set_grad_enabled(False)
    if a.only in ("", "tiny"):
        tiny(a.out, a.work)
    if a.only in ("", "large"):
        full_size(a.out, a.work, "large", lambda: wl.c1(0), "large")
    if a.only in ("", "base"):
        cfg = ck.PRESETS["base"]
        full_size(a.out, a.work, "base", lambda: wl.make_batch(cfg, [200], [4], seed=7, dtype="fp32",
                                                               name="base-b1s200"), "base")
    for tag, (preset, wname, pick) in DRIFT_SAMPLES.items():
        if a.only in ("", tag):
            batch_drift(a.out, a.work, preset, wl.CONFIGS[wname](0).subset(pick), tag)


if __name__ == "__main__":
    main()
