"""Pins the CPU oracle (oracle/model.py) before it is trusted as the engine's checker.

  * golden vectors written by the reference's own DecisionModel (tests/golden/make_golden.py):
    tiny model in full (every layer, every case), ModernBERT-large C1 and the mmBERT-base shape
    on sampled rows;
  * closed forms: zero weights give logits == scorer bias; one key gives attention == V; one
    marker gives act features [1, 1, 0, 2/255];
  * brute force: masked attention by explicit loops, sliding window included;
  * invariants: RoPE keeps each (d, d + 32) pair's norm; batch composition, padding and order
    never change a question's outputs;
  * sensitivity: plausible mistakes planted in the oracle (window off by one, RoPE halves
    swapped, wrong GELU, missing type embedding) make the golden check fail.
"""
import json
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN, read_tiny_case, tiny_cases
from layamd_amd import checkpoint as ck
from layamd_amd import rng
from layamd_amd import workloads as wl
from oracle import model as om

TINY_JITTER = 0.1


@pytest.fixture(scope="module")
def tiny_w():
    return om.Weights(ck.generate_weights(ck.PRESETS["tiny"], 0, ln_jitter=TINY_JITTER))


def run_case(W, c, capture=None, cfg=None):
    with torch.no_grad():
        return om.forward(W, cfg or ck.PRESETS["tiny"], c["input_ids"], c["attention_mask"], c["marker_pos"],
                          c["marker_mask"].astype(bool), c["qtype"], capture)


def case_error(W, c, cfg=None):
    cap = {}
    lo, ac = run_case(W, c, cap, cfg)
    att = c["attention_mask"].astype(bool)
    e = max(np.abs(lo.numpy() - c["logits"]).max(), np.abs(ac.numpy() - c["act_logits"]).max())
    for k in cap:
        if k in c:
            e = max(e, np.abs(cap[k].numpy()[att] - c[k][att]).max())
    return float(e)


# ---------------------------------------------------------------- known answers of the generator
def test_splitmix64_known_answer():
    # first output of splitmix64 seeded with 0 (Steele, Lea & Flood 2014 reference generator)
    assert int(rng.u64(np.uint64(0), 0, 1)[0]) == 0xE220A8397B1DCDAF
    assert int(rng.u64(np.uint64(0), 1, 1)[0]) == 0x6E789E6AA1B965F4


def test_normal_generator_c_matches_numpy():
    key = rng.stream_key(7, 3)
    n = 100003
    c = rng.normal(key, n, 0.02)
    saved = rng._HOST
    try:
        rng._HOST = False
        p = rng.normal(key, n, 0.02)
    finally:
        rng._HOST = saved
    assert np.array_equal(c, p)
    assert abs(float(c.std()) - 0.02) < 3e-4 and abs(float(c.mean())) < 3e-4


# ---------------------------------------------------------------- reference golden vectors
@pytest.mark.parametrize("case", [c["name"] for c in tiny_cases()])
def test_oracle_matches_reference_tiny(tiny_w, case):
    c = read_tiny_case(next(x for x in tiny_cases() if x["name"] == case))
    assert case_error(tiny_w, c) < 1e-5


@pytest.mark.parametrize("tag", ["large", "base"])
def test_oracle_matches_reference_full_size(tag):
    g = np.load(os.path.join(GOLDEN, tag, "golden.npz"))
    man = json.load(open(os.path.join(GOLDEN, tag, "manifest.json")))
    cfg = ck.PRESETS[man["model"]["preset"]]
    W = om.Weights(ck.generate_weights(cfg, man["model"]["seed"]))
    cap = {}
    with torch.no_grad():
        lo, ac = om.forward(W, cfg, g["input_ids"], g["attention_mask"], g["marker_pos"], g["marker_mask"].astype(bool),
                            g["qtype"], cap)
    assert np.abs(lo.numpy() - g["logits"]).max() < 1e-5
    assert np.abs(ac.numpy() - g["act_logits"]).max() < 1e-5
    rows = g["sample_rows"]
    for name in man["layers"]:
        got = cap[name][0].numpy()[rows]
        assert np.abs(got - g[name + "_rows"]).max() < 1e-4, name


@pytest.mark.slow
@pytest.mark.parametrize("tag,preset,make", [("c3_full", "large", wl.c3), ("c4_full", "base", wl.c4),
                                             ("c5_full", "large1024", wl.c5)])
def test_oracle_matches_reference_whole_batches(tag, preset, make):
    """Every question of the b32 x s512 (ModernBERT-large), b16 x s1024 (mmBERT-base) and
    b64 varlen (ModernBERT-large at 1024 positions) batches, one question per forward as the
    engine packs them (no padding), against the logits and act logits the reference's fp32
    DecisionModel gave on the padded batch (tests/golden/<tag>/drift.npz)."""
    g = np.load(os.path.join(GOLDEN, tag, "drift.npz"))
    b = make(0)
    assert list(g["lens"]) == list(b.lens)
    cfg = ck.PRESETS[preset]
    W = om.Weights(ck.generate_weights(cfg, 0))
    lo, ac = om.run_per_question(W, cfg, b)
    ref = np.concatenate([g["logits"][i, :b.nmark[i]] for i in range(b.B)])
    assert np.abs(lo - ref).max() < 1e-5
    assert np.abs(ac.reshape(b.B, -1) - g["act_logits"]).max() < 1e-5


# ---------------------------------------------------------------- closed forms and brute force
def test_zero_weights_give_scorer_bias():
    cfg = ck.PRESETS["tiny"]
    Wd = ck.generate_weights(cfg, 1, ln_jitter=0.0)
    for k in Wd:
        if k not in ("scorer.3.bias",) and not k.endswith("norm.weight") and "norm1.weight" not in k \
                and "norm2.weight" not in k and k != "scorer.0.weight" and k != "temperature":
            Wd[k] = np.zeros_like(Wd[k])
    b = wl.make_batch(cfg, [7, 30], [3, 2], seed=2)
    lo, _ = om.run_batch(om.Weights(Wd), cfg, b)
    assert np.allclose(lo, Wd["scorer.3.bias"][0], atol=0, rtol=0)


def test_single_key_attention_is_v():
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(2, 3, 1, 64, generator=g, dtype=torch.float64) for _ in range(3))
    out = om.attention(q, k, v, torch.ones(2, 1, 1, 1, dtype=torch.bool))
    assert torch.equal(out, v)


def test_attention_brute_force_with_sliding_window():
    g = torch.Generator().manual_seed(1)
    n, H, L, d = 2, 2, 150, 64
    q, k, v = (torch.randn(n, H, L, d, generator=g, dtype=torch.float64) for _ in range(3))
    att = torch.ones(n, L, dtype=torch.long)
    att[1, 100:] = 0
    m_glob, m_slide = om.encoder_masks(att, 128)
    for mask, window in ((m_glob, None), (m_slide, 64)):
        fast = om.attention(q, k, v, mask)
        for b in range(n):
            valid = int(att[b].sum())
            for i in range(0, valid, 37):
                for h in range(H):
                    keys = [j for j in range(valid) if window is None or abs(i - j) <= window]
                    s = torch.stack([q[b, h, i] @ k[b, h, j] / 8.0 for j in keys])
                    p = torch.softmax(s, 0)
                    ref = sum(p[t] * v[b, h, j] for t, j in enumerate(keys))
                    assert torch.allclose(fast[b, h, i], ref, atol=1e-12)


def test_single_marker_act_features(tiny_w):
    cfg = ck.PRESETS["tiny"]
    b = wl.make_batch(cfg, [40, 25], [1, 3], seed=4)
    ids, att, mpos, mmask, qt = b.padded()
    cap = {}
    with torch.no_grad():
        lo, act = om.forward(tiny_w, cfg, ids, att, mpos, mmask, qt, cap)
        pooled = cap["head%d" % (cfg.head_layers - 1)][0, 0]
        feats = torch.tensor([1.0, 1.0, 0.0, 2.0 / 255.0])
        hid = torch.nn.functional.gelu(torch.cat([pooled, feats]) @ tiny_w["act_head.0.weight"].T + tiny_w["act_head.0.bias"])
        ref = hid @ tiny_w["act_head.2.weight"].T + tiny_w["act_head.2.bias"]
    assert torch.allclose(act[0], ref, atol=1e-6)


def test_rope_preserves_pair_norms():
    cos, sin = om.rope_tables(160000.0, 64, 300, torch.float64)
    x = torch.randn(300, 64, dtype=torch.float64)
    y = x * cos + om.rotate_half(x) * sin
    n_in = x[:, :32] ** 2 + x[:, 32:] ** 2
    n_out = y[:, :32] ** 2 + y[:, 32:] ** 2
    assert torch.allclose(n_in, n_out, rtol=1e-12, atol=1e-12)
    assert torch.equal(y[0], x[0])           # position 0 is the identity


def test_batch_padding_and_order_invariance(tiny_w):
    cfg = ck.PRESETS["tiny"]
    b = wl.make_batch(cfg, [3, 200, 64, 129], [2, 5, 1, 7], seed=9)
    lo_b, ac_b = om.run_batch(tiny_w, cfg, b)
    lo_q, ac_q = om.run_per_question(tiny_w, cfg, b)
    assert np.allclose(lo_b, lo_q, atol=2e-6) and np.allclose(ac_b, ac_q, atol=2e-6)
    perm = [2, 0, 3, 1]
    lo_p, ac_p = om.run_batch(tiny_w, cfg, b.subset(perm))
    offs = np.concatenate([[0], np.cumsum(b.nmark)])
    exp = np.concatenate([lo_b[offs[i]:offs[i + 1]] for i in perm])
    assert np.allclose(lo_p, exp, atol=2e-6) and np.allclose(ac_p, ac_b[perm], atol=2e-6)


# ---------------------------------------------------------------- the goldens catch plausible mistakes
def _mut_window(orig):
    def f(att, window):
        g, s = orig(att, window)
        n, L = att.shape
        i = torch.arange(L)
        band = (i[:, None] - i[None, :]).abs() < window // 2          # exclusive instead of inclusive
        return g, g & band[None, None]
    return f


def _mut_rotate(x):
    h = x.shape[-1] // 2
    return torch.cat((x[..., h:], -x[..., :h]), dim=-1)                 # sign on the wrong half


def test_gelu_is_the_erf_form():
    """The golden inputs keep pre-activations small, where erf and tanh GELU agree to ~1e-6, so
    the activation is pinned here directly: exact erf GELU (HF ACT2FN["gelu"], nn.GELU())."""
    import math
    x = torch.linspace(-6, 6, 241, dtype=torch.float64)
    ref = torch.tensor([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in x.tolist()], dtype=torch.float64)
    assert torch.allclose(om.F.gelu(x), ref, atol=1e-12)
    assert (om.F.gelu(x, approximate="tanh") - ref).abs().max() > 1e-4


@pytest.mark.parametrize("mutation", ["window_off_by_one", "rotate_half_sign", "relu_for_gelu", "no_type_emb"])
def test_golden_detects_planted_mistake(tiny_w, monkeypatch, mutation):
    c = read_tiny_case(next(x for x in tiny_cases() if x["name"] == "long_sliding"))
    assert case_error(tiny_w, c) < 1e-5
    if mutation == "window_off_by_one":
        monkeypatch.setattr(om, "encoder_masks", _mut_window(om.encoder_masks))
    elif mutation == "rotate_half_sign":
        monkeypatch.setattr(om, "rotate_half", _mut_rotate)
    elif mutation == "relu_for_gelu":
        monkeypatch.setattr(om.F, "gelu", torch.relu)
    else:
        W = om.Weights({})
        W.w = dict(tiny_w.w)
        W.w["type_emb.weight"] = torch.zeros_like(W.w["type_emb.weight"])
        tiny_w = W
    assert case_error(tiny_w, c) > 1e-4
