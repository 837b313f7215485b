"""The engine as the reference's callers use it, on the GPU, through the C ABI:

  * the reference server's warm-up (server/laya_server.py:52-56: laya_tune_all, then one call per
    length 64, 128, ..., max_len) followed by mixed single-question and batched traffic: warmed
    shapes replay their graphs without capturing, every answer equals the eager engine's bit for
    bit, and a cache miss's cost (eager run + capture + instantiate) is measured;
  * the graph cache limit (512 graphs, src/engine.hip:477): calls beyond it run eagerly and stay
    correct;
  * laya_tune_all at the default capacity (65536 rows), timed;
  * checkpoints stored as F16, BF16 and F32 (src/engine.hip:115-129): a BF16 file gives exactly the
    results of an F32 file holding the same values, in both engines; an F16 file on the fp32 engine
    matches the CPU oracle run on the F16-rounded weights within the fp32 bars;
  * the C++ tools (laya-parity on the reference golden format, laya-bench's latency table), which
    call the library as any C caller of laya_api.h would.
"""
import os
import subprocess
import sys
import time

import numpy as np
import pytest

from conftest import GOLDEN, checkpoint_dir
from layamd_amd import checkpoint as ck
from layamd_amd import engine as le
from layamd_amd import workloads as wl

pytestmark = pytest.mark.gpu

ENV = {"LAYA_MAX_TOKENS": 8192, "LAYA_DUMP_DIR": None, "LAYA_PROFILE": None, "LAYA_GRAPHS": 1, "LAYA_TUNE": 1,
       "LAYA_ATTN_QTILE": None, "LAYA_GEMM_CFG": None, "LAYA_GEMM_SPLIT": None, "LAYA_MAX_GRAPHS": None,
       "LAYA_PASS_TOKENS": None, "LAYA_MAX_SEQS": None, "LAYA_MAX_GATHERED": None, "LAYA_LN_FOLD": None,
       "LAYA_LATENCY": None}


def make_engine(model_dir, precision, **env):
    return le.Engine(None, model_dir, precision=precision, env=dict(ENV, **env))


def same(a, b):
    return np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_reference_warmup_then_traffic():
    """ModernBERT-large bf16: the server's warm-up, then 24 single questions of random lengths
    (<= 64 options: the warmed marker bucket) that must all replay warmed graphs, then batched
    requests; every answer equals the eager (graph-free) engine's."""
    cfg = ck.PRESETS["large"]
    d = checkpoint_dir("large")
    e = make_engine(d, "bf16")
    eager = make_engine(d, "bf16", LAYA_GRAPHS=0)
    t0 = time.time()
    e.tune_all()
    t_tune = time.time() - t0
    t0 = time.time()
    for n in range(64, cfg.max_len + 1, 64):                # server/laya_server.py:52-56
        e.forward_batch([[cfg.cls_id] * n], [[1, 2]], [0])
    t_warm = time.time() - t0
    g0, c0, _, _ = e.stats()
    print("warm-up: tune_all %.2f s, %d lengths %.2f s, %d graphs" % (t_tune, cfg.max_len // 64, t_warm, g0))
    assert g0 == cfg.max_len // 64
    rs = np.random.RandomState(7)
    lat = []
    for i in range(24):
        L = int(rs.randint(1, cfg.max_len + 1))
        k = int(rs.randint(1, 65))
        b = wl.make_batch(cfg, [L], [k], seed=100 + i)
        t = time.perf_counter()
        r = e.forward_flat(*b.flat())
        lat.append(1e3 * (time.perf_counter() - t))
        assert same(r, eager.forward_flat(*b.flat())), (L, k)
    assert e.stats()[1] == c0, "a warmed single-question shape captured a new graph"
    print("single questions after warm-up: p50 %.2f ms, max %.2f ms over %d calls" % (np.median(lat), max(lat), len(lat)))
    # batched traffic: new buckets (rows, questions, marker rows) are run eagerly, then captured
    miss, hit = [], []
    for i in range(6):
        B = int(rs.randint(2, 9))
        lens = rs.randint(16, cfg.max_len + 1, B)
        b = wl.make_batch(cfg, lens, rs.randint(2, 6, B), seed=200 + i)
        n_before = e.stats()[1]
        t = time.perf_counter()
        r1 = e.forward_flat(*b.flat())
        t1 = 1e3 * (time.perf_counter() - t)
        t = time.perf_counter()
        r2 = e.forward_flat(*b.flat())
        t2 = 1e3 * (time.perf_counter() - t)
        assert same(r1, r2) and same(r1, eager.forward_flat(*b.flat()))
        if e.stats()[1] > n_before:
            miss.append(t1)
            hit.append(t2)
    print("batched requests: first call of a new bucket (eager + capture) %s ms, replay %s ms"
          % (np.round(miss, 2).tolist(), np.round(hit, 2).tolist()))


def test_graph_cache_limit():
    """At most LAYA_MAX_GRAPHS graphs (default 512, the reference's limit) are kept; the 513th and
    later buckets run eagerly, give the eager engine's bits, and evict nothing."""
    cfg = ck.PRESETS["tiny"]
    d = checkpoint_dir("tiny")
    e = make_engine(d, "bf16", LAYA_MAX_TOKENS=4096)
    eager = make_engine(d, "bf16", LAYA_MAX_TOKENS=4096, LAYA_GRAPHS=0)
    first = None
    t0 = time.time()
    # 520 buckets (rows, questions, marker rows): 1..260 one-token questions with one option each
    # (64 marker rows) and with 64 options each (64 B marker rows)
    for n, (B, k) in enumerate([(B, 1) for B in range(1, 261)] + [(B, 64) for B in range(1, 261)]):
        b = wl.make_batch(cfg, [1] * B, [k] * B, seed=n)
        r = e.forward_flat(*b.flat())
        if n == 0:
            first = (b, r)
        if n in (0, 259, 510, 511, 512, 513, 519):
            assert same(r, eager.forward_flat(*b.flat())), n
    g, c, _, _ = e.stats()
    print("520 buckets in %.1f s: %d graphs cached, %d captured" % (time.time() - t0, g, c))
    assert g == 512 and c == 512
    assert same(e.forward_flat(*first[0].flat()), first[1])     # still replays the first graph
    small = make_engine(d, "fp32", LAYA_MAX_GRAPHS=2)
    for B in (1, 2, 3, 4):
        b = wl.make_batch(cfg, [40] * B, [2] * B, seed=B)
        assert same(small.forward_flat(*b.flat()), small.forward_flat(*b.flat()))
    assert small.stats()[:2] == (2, 2)


def test_tune_all_default_capacity():
    """laya_tune_all at the default capacity (65536 rows: 88 row buckets of every GEMM), timed;
    the tuned engine gives the untuned engine's bits."""
    d = checkpoint_dir("large")
    e = make_engine(d, "bf16", LAYA_MAX_TOKENS=None)
    t0 = time.time()
    e.tune_all()
    dt = time.time() - t0
    g, c, plans, buckets = e.stats()
    print("tune_all at 65536 rows: %.1f s, %d GEMM plans over %d row buckets" % (dt, plans, buckets))
    assert buckets >= 88
    b = wl.c3(0).subset(list(range(6)))
    assert same(e.forward_flat(*b.flat()), make_engine(d, "bf16", LAYA_TUNE=0).forward_flat(*b.flat()))


def _f32_copy(preset, dtype, **kw):
    """(dir of the dtype file, dir of an F32 file holding exactly its values)."""
    return ck.cached_checkpoint(preset, dtype=dtype, **kw), ck.cached_checkpoint(preset, dtype="F32", round_to=dtype, **kw)


@pytest.mark.parametrize("dtype", ["BF16", "F16"])
def test_checkpoint_dtypes_tiny(dtype):
    """Tiny model (LayerNorm weights and biases perturbed so every parameter matters): an F16 or BF16
    file equals the F32 file of the same values in both engines, bit for bit; the fp32 engine on it
    matches the oracle on the rounded weights."""
    from oracle import model as om
    dfile, df32 = _f32_copy("tiny", dtype, ln_jitter=0.1)
    b = wl.make_batch(ck.PRESETS["tiny"], [5, 64, 129, 320, 1], [2, 3, 12, 4, 1], seed=9)
    for prec in ("fp32", "bf16"):
        assert same(make_engine(dfile, prec).forward_flat(*b.flat()), make_engine(df32, prec).forward_flat(*b.flat())), prec
    cfg, W = ck.load_checkpoint(dfile)
    lo, ac = make_engine(dfile, "fp32").forward_flat(*b.flat())
    ref_lo, ref_ac = om.run_batch(om.Weights(W), ck.PRESETS["tiny"], b)
    assert np.abs(lo - ref_lo).max() < 1e-4
    assert (np.abs(ac - ref_ac) / np.maximum(1.0, np.abs(ref_ac))).max() < 1e-3


def test_checkpoint_dtypes_large():
    """ModernBERT-large at b1 x s128: the BF16 file equals the F32 file of its values in the bf16
    engine bit for bit; the fp32 engine on the F16 file matches the oracle on the F16 weights
    (probabilities within 1e-4, act logits within 1e-3)."""
    import torch
    from oracle import model as om
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    b = wl.c1(0)
    dfile, df32 = _f32_copy("large", "BF16")
    assert same(make_engine(dfile, "bf16").forward_flat(*b.flat()), make_engine(df32, "bf16").forward_flat(*b.flat()))
    d16 = ck.cached_checkpoint("large", dtype="F16")
    cfg, W = ck.load_checkpoint(d16)
    lo, ac = make_engine(d16, "fp32").forward_flat(*b.flat())
    ref_lo, ref_ac = om.run_batch(om.Weights(W), ck.PRESETS["large"], b)
    p = lambda z: np.exp(z - z.max()) / np.exp(z - z.max()).sum()
    assert np.abs(p(lo) - p(ref_lo)).max() < 1e-4
    assert (np.abs(ac - ref_ac) / np.maximum(1.0, np.abs(ref_ac))).max() < 1e-3


def _tool(name):
    exe = os.path.join(os.path.dirname(le.DEFAULT_LIB), name)
    assert os.path.exists(exe), "%s not built (python -m layamd_amd.build)" % exe
    return exe


@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_cpp_parity_tool_on_golden_format(precision):
    """laya-parity, a C++ program calling only laya_api.h, reads the reference golden format
    (tests/golden/tiny) and passes: fp32 at the fp32 bars, bf16 at the reference tool's bars."""
    env = dict(os.environ, LAYA_PRECISION=precision, LAYA_MAX_TOKENS="4096")
    tol = ["--prob-tol", "1e-4", "--act-tol", "1e-3", "--logit-tol", "1e-4"] if precision == "fp32" else []
    r = subprocess.run([_tool("laya-parity"), checkpoint_dir("tiny"), os.path.join(GOLDEN, "tiny")] + tol, env=env,
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=300)
    print(r.stdout[-3000:])
    assert r.returncode == 0
    assert "questions pass" in r.stdout


def test_cpp_latency_tool():
    """laya-bench, the ABI latency table (p50 per laya_forward_batch call, host work included) on
    ModernBERT-large bf16."""
    env = dict(os.environ, LAYA_PRECISION="bf16", LAYA_MAX_TOKENS="16384")
    r = subprocess.run([_tool("laya-bench"), checkpoint_dir("large"), "--iters", "20"], env=env,
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=600)
    print(r.stdout[-4000:])
    assert r.returncode == 0 and "batched" in r.stdout


def _with_layer0_attn_norm(src_dir, out_dir, w):
    """A copy of the checkpoint in src_dir that also carries encoder.layers.0.attn_norm.weight = w,
    the tensor the reference engine treats as optional (src/engine.hip:154-155, 415)."""
    import shutil
    os.makedirs(os.path.join(out_dir, "encoder"), exist_ok=True)
    shutil.copy(os.path.join(src_dir, "encoder", "config.json"), os.path.join(out_dir, "encoder", "config.json"))
    shutil.copy(os.path.join(src_dir, "rl_agent_config.json"), os.path.join(out_dir, "rl_agent_config.json"))
    _, W = ck.load_checkpoint(src_dir)
    W["encoder.layers.0.attn_norm.weight"] = w
    names = list(W)
    ck.write_safetensors(os.path.join(out_dir, "model.safetensors"), [(n, W[n].shape) for n in names],
                         lambda i: W[names[i]], "F32")
    return out_dir


def test_layer0_attn_norm_with_and_without_fold(tmp_path):
    """A checkpoint with a layer-0 attn_norm (weight 2 + 0.5 N(0,1)): the weight is applied once, by
    the explicit LayerNorm after the embeddings, with the LayerNorm fold on or off.  The first
    layer's output (LAYA_DUMP_DIR) of the fp32 engine matches the fp32 oracle, which applies that
    LayerNorm too, and both bf16 engines stay within the tiny model's bf16 bar (2.5e-2 of the row
    RMS); leaving the LayerNorm out or applying its weight twice moves that output by more than 3x
    the bar, so the check sees either mistake.  Logits: fp32 bars, and 2e-3 for bf16."""
    import tempfile
    from oracle import model as om
    tiny = ck.PRESETS["tiny"]
    D = tiny.d
    w = (2.0 + 0.5 * np.random.default_rng(5).standard_normal(D)).astype(np.float32)
    d = _with_layer0_attn_norm(checkpoint_dir("tiny"), str(tmp_path / "l0norm"), w)
    cfg, W = ck.load_checkpoint(d)
    b = wl.make_batch(tiny, [5, 64, 129, 320], [2, 3, 12, 4], seed=11)
    ids, att, mp, mm, qt = b.padded()
    valid = att.astype(bool)

    def oracle_enc0(Wd):
        cap = {}
        lo, ac = om.forward(om.Weights(Wd), tiny, ids, att, mp, mm.astype(bool), qt, capture=cap)
        return cap["enc0"].numpy().astype(np.float64), lo.numpy(), ac.numpy()
    ref0, ref_lo_pad, ref_ac = oracle_enc0(W)
    ref_lo = np.concatenate([ref_lo_pad[i, :b.nmark[i]] for i in range(b.B)])
    rms = np.sqrt((ref0 ** 2).mean(-1))
    rel = lambda a: float((np.abs(a - ref0).max(-1) / rms)[valid].max())
    bar = 2.5e-2
    wrong = {"none": dict(W), "twice": dict(W, **{"encoder.layers.0.attn_norm.weight": w * w})}
    del wrong["none"]["encoder.layers.0.attn_norm.weight"]
    for k, Wd in wrong.items():
        r = rel(oracle_enc0(Wd)[0])
        print("oracle with the layer-0 LayerNorm %s: enc0 moves %.4f of the row RMS" % (k, r))
        assert r > 3 * bar, k
    lens = b.lens
    soff = np.concatenate([[0], np.cumsum((lens + 7) // 8 * 8)])

    def engine_enc0(prec, **env):
        with tempfile.TemporaryDirectory() as dd:
            lo, ac = make_engine(d, prec, LAYA_DUMP_DIR=dd, LAYA_GRAPHS=0, **env).forward_flat(*b.flat())
            got = np.fromfile(os.path.join(dd, "enc0.bin"), dtype=np.float32).reshape(-1, D)
        e0 = np.zeros_like(ref0)
        for i in range(b.B):
            e0[i, :lens[i]] = got[soff[i]:soff[i] + lens[i]]
        return e0, lo, ac
    e0, lo32, ac32 = engine_enc0("fp32")
    print("fp32: enc0 %.2e of the row RMS, max|dlogit| %.2e" % (rel(e0), np.abs(lo32 - ref_lo).max()))
    assert rel(e0) < 1e-4
    assert np.abs(lo32 - ref_lo).max() < 1e-4
    assert (np.abs(ac32 - ref_ac) / np.maximum(1.0, np.abs(ref_ac))).max() < 1e-3
    out = {}
    for fold in (0, 1):
        e0, lo, ac = engine_enc0("bf16", LAYA_LN_FOLD=fold)
        print("bf16 fold %d: enc0 %.4f of the row RMS, max|dlogit| %.2e" % (fold, rel(e0), np.abs(lo - ref_lo).max()))
        assert rel(e0) < bar, fold
        assert np.abs(lo - ref_lo).max() < 2e-3, fold
        out[fold] = lo
    assert np.abs(out[0] - out[1]).max() < 2e-3


def test_max_tokens_capped_to_32bit_offsets(capfd):
    """LAYA_MAX_TOKENS beyond what the kernels' 32-bit buffer offsets reach is capped at load, with a
    message, and the engine still answers correctly."""
    d = checkpoint_dir("tiny")
    b = wl.make_batch(ck.PRESETS["tiny"], [5, 64], [2, 3], seed=3)
    ref = make_engine(d, "bf16").forward_flat(*b.flat())
    e = make_engine(d, "bf16", LAYA_MAX_TOKENS=2000000000, LAYA_MAX_GATHERED=2000000000)
    err = capfd.readouterr().err
    assert "exceeds what 32-bit buffer offsets reach" in err
    assert same(e.forward_flat(*b.flat()), ref)


def test_latency_mode_split_k():
    """LAYA_LATENCY=1 (bf16): the residual GEMMs over all rows split K into chunks of 4 stages of 64
    (encoder out-projection K = 1024: 4 chunks; MLP down-projection K = 2624: 10 chunks of 4 stages
    and one of 1; the first head layer's FFN down-projection K = 4096: 16), whatever the pass's size.
      * ModernBERT-large b1 x s128: logits and act logits within the bf16 budget of the reference's
        fp32 model (tests/golden/large), as the default engine;
      * a question's bits do not depend on its batch: alone, and as the third of four questions,
        it gives the same logits and act logits; graph replays give the eager pass's bits; the
        LayerNorm that adds a split GEMM's partial products (when they fit the workspace) gives
        the bits of the GEMM's own reduction;
      * pass times (device, graph replay) with and without the mode at 1 x 128, 1 x 512 and
        4 x 512 tokens are printed."""
    import json
    g = np.load(os.path.join(GOLDEN, "large", "golden.npz"))
    d = checkpoint_dir("large")
    lat = make_engine(d, "bf16", LAYA_LATENCY=1)
    eager = make_engine(d, "bf16", LAYA_LATENCY=1, LAYA_GRAPHS=0)
    b = wl.c1(0)
    lens, ids, nm, mk, qt = b.flat()
    lo, ac = lat.forward_flat(lens, ids, nm, mk, qt)
    gl, g16 = g["logits"][0, :nm[0]], g["logits_bf16_autocast"][0, :nm[0]]
    dl, dl_up = float(np.abs(lo - gl).max()), float(np.abs(g16 - gl).max())
    da, da_up = float(np.abs(ac - g["act_logits"]).max()), float(np.abs(g["act_logits_bf16_autocast"] - g["act_logits"]).max())
    print("latency mode, large c1: dlogit %.5f (reference bf16 %.5f), dact %.5f (reference bf16 %.5f)" % (dl, dl_up, da, da_up))
    assert dl <= 2.0 * dl_up + 1e-3 and da <= 2.0 * da_up + 1e-3
    default = make_engine(d, "bf16").forward_flat(lens, ids, nm, mk, qt)
    print("latency vs default engine: max|dlogit| %.2e" % np.abs(lo - default[0]).max())
    # batch independence and graph replay
    cfg = ck.PRESETS["large"]
    four = wl.make_batch(cfg, [512, 77, 128, 300], [4, 3, 4, 5], seed=21)
    one = four.subset([2])
    lo4, ac4 = lat.forward_flat(*four.flat())
    lo1, ac1 = lat.forward_flat(*one.flat())
    moff = np.concatenate([[0], np.cumsum(four.nmark)])
    assert np.array_equal(lo4[moff[2]:moff[3]], lo1) and np.array_equal(ac4.reshape(4, -1)[2], ac1.reshape(-1))
    assert same(lat.forward_flat(*four.flat()), (lo4, ac4))
    assert same(eager.forward_flat(*four.flat()), (lo4, ac4))
    # the partial products are added by the LayerNorm that follows each split GEMM; with per-layer
    # dumps the GEMMs reduce them themselves (so that the dumped x is whole): the same bits
    import tempfile
    with tempfile.TemporaryDirectory() as dd:
        assert same(make_engine(d, "bf16", LAYA_LATENCY=1, LAYA_DUMP_DIR=dd).forward_flat(*four.flat()), (lo4, ac4))
    assert np.isfinite(lo4).all() and np.isfinite(ac4).all()
    # pass times, device-side graph replays
    times = {}
    for tag, e in (("default", make_engine(d, "bf16")), ("latency", lat)):
        for shape in ((1, 128), (1, 512), (4, 512)):
            bb = wl.make_batch(cfg, [shape[1]] * shape[0], [4] * shape[0], seed=5)
            e.forward_flat(*bb.flat())
            e.forward_flat(*bb.flat())
            times[(tag, shape)] = e.replay(20) / 20
    print("pass ms (graph replay):", json.dumps({"%s %dx%d" % (t, s[0], s[1]): round(v, 3) for (t, s), v in times.items()}))
