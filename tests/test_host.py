"""Host logic of the engine on the CPU: the C++ packer (pack.cpp), config parser and safetensors
loader (model.cpp), through liblaya_host.so.  Validation semantics follow the reference's
Engine::forward_batch (src/engine.hip:491-496)."""
import ctypes
import json
import os
import tempfile

import numpy as np
import pytest
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from layamd_amd import checkpoint as ck
from layamd_amd import engine as le
from layamd_amd import workloads as wl


@pytest.fixture(scope="module")
def host():
    if not os.path.exists(le.HOST_LIB):
        from layamd_amd import build
        build.build()
    L = ctypes.CDLL(le.HOST_LIB)
    IP = ctypes.POINTER(ctypes.c_int)
    L.laya_host_plan.argtypes = [ctypes.c_int, IP, IP, IP, IP, IP] + [ctypes.c_int] * 9 + [IP] * 8
    L.laya_host_plan.restype = ctypes.c_int
    L.laya_host_config.argtypes = [ctypes.c_char_p, IP, ctypes.POINTER(ctypes.c_float), ctypes.c_char_p, ctypes.c_int]
    L.laya_host_config.restype = ctypes.c_int
    L.laya_host_layer_is_global.argtypes = [ctypes.c_char_p, ctypes.c_int]
    L.laya_host_read_tensor.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float),
                                        ctypes.c_longlong, ctypes.POINTER(ctypes.c_longlong), IP]
    L.laya_host_read_tensor.restype = ctypes.c_longlong
    return L


def P(a):
    a = np.ascontiguousarray(a, np.int32)
    return a, a.ctypes.data_as(ctypes.POINTER(ctypes.c_int))


def plan(host, lens, ids, nm, mk, qt, max_len=512, pass_tokens=65536, max_seqs=512, max_grows=32768, vocab=0,
         pad_id=0, q_tile=64, q_tile_global=None):
    keep = [P(x if len(x) else [0]) for x in (lens, ids, nm, mk, qt)]
    args = (max_len, pass_tokens, max_seqs, max_grows, vocab, pad_id, q_tile,
            q_tile if q_tile_global is None else q_tile_global)
    n = host.laya_host_plan(len(lens), *[k[1] for k in keep], *args, -1, *([None] * 8))
    if n < 0:
        return None
    out = []
    T = int(np.sum((np.asarray(lens) + 7) // 8 * 8)) + 64
    R = int(np.sum(nm)) + len(lens) + 64
    for w in range(n):
        dims = np.zeros(10, np.int32)
        rows = np.zeros(3 * T, np.int32)
        seqs = np.zeros(5 * len(lens) + 1, np.int32)
        tiles = np.zeros(4 * (T // 64 + len(lens)), np.int32)
        gltiles = np.zeros(4 * (T // 64 + len(lens)), np.int32)
        gtiles = np.zeros(4 * (R // 64 + len(lens)), np.int32)
        gq = np.zeros(R, np.int32)
        grow = np.zeros(R, np.int32)
        bufs = [P(x)[1] for x in (dims, rows, seqs, tiles, gltiles, gtiles, gq, grow)]
        host.laya_host_plan(len(lens), *[k[1] for k in keep], *args, w, *bufs)
        first, B, Tn, valid, KT, Rn, nt, ngt, ngq, nglt = dims
        s = seqs[:5 * B + 1]
        out.append(dict(first=first, B=B, T=Tn, valid=valid, KT=KT, R=Rn,
                        ids=rows[:Tn], pos=rows[Tn:2 * Tn], seq=rows[2 * Tn:3 * Tn],
                        soff=s[:B + 1], vlen=s[B + 1:2 * B + 1], qt=s[2 * B + 1:3 * B + 1],
                        nm=s[3 * B + 1:4 * B + 1], moff=s[4 * B + 1:5 * B + 1],
                        tiles=tiles[:4 * nt].reshape(-1, 4), gltiles=gltiles[:4 * nglt].reshape(-1, 4),
                        gtiles=gtiles[:4 * ngt].reshape(-1, 4),
                        gq=gq[:ngq], grow=grow[:Rn]))
    return out


def test_validation_minus_one(host):
    ok = ([3], [1, 5, 2], [1], [0], [0])
    assert plan(host, *ok) is not None
    assert plan(host, [0], [], [1], [0], [0]) is None                       # len < 1
    assert plan(host, [513], [5] * 513, [1], [0], [0]) is None              # len > max_len
    assert plan(host, [3], [1, 5, 2], [0], [], [0]) is None                 # nmark < 1
    assert plan(host, [3], [1, 5, 2], [256], [0] * 256, [0]) is None        # nmark > 255
    assert plan(host, [3], [1, 5, 2], [1], [3], [0]) is None                # marker >= len
    assert plan(host, [3], [1, 5, 2], [1], [-1], [0]) is None               # marker < 0
    assert plan(host, [3], [1, 5, 2], [1], [0], [3]) is None                # qtype
    assert plan(host, [3], [1, 5, 2], [1], [0], [0], vocab=5) is None       # token id >= vocab
    assert plan(host, [3], [1, 4, 2], [1], [0], [0], vocab=5) is not None
    assert plan(host, [], [], [], [], []) == []                            # empty call: no pass


def up64(x):
    return (int(x) + 63) // 64 * 64


@pytest.mark.parametrize("q_tile,q_tile_global", [(64, 64), (64, 128), (128, 128)])
def test_layout_of_a_pass(host, q_tile, q_tile_global):
    cfg = ck.PRESETS["tiny"]
    b = wl.make_batch(cfg, [1, 64, 65, 200, 17, 128, 129, 256], [1, 3, 255, 12, 2, 1, 4, 2], seed=1)
    (p,) = plan(host, *b.flat(), max_len=320, pad_id=cfg.pad_id, q_tile=q_tile, q_tile_global=q_tile_global)
    check_layout(b, p, cfg.pad_id, q_tile, q_tile_global)


def check_layout(b, p, pad_id, q_tile, q_tile_global):
    """The layout of one pass p of the questions of batch b (every question of b in the pass)."""
    cfg = b.cfg
    rows8 = (b.lens + 7) // 8 * 8                                          # questions start on 8-row groups
    # the pass's rows are padded to a multiple of 64 (its graph bucket)
    assert p["B"] == b.B and p["T"] == up64(rows8.sum()) and p["valid"] == int(b.lens.sum())
    soff = np.concatenate([[0], np.cumsum(rows8)])
    assert np.array_equal(p["soff"], soff)
    tail = slice(soff[-1], p["T"])                                         # bucket padding rows
    assert np.all(p["ids"][tail] == pad_id) and np.all(p["pos"][tail] == 0) and np.all(p["seq"][tail] == b.B - 1)
    for i in range(b.B):
        r = slice(soff[i], soff[i + 1])
        assert np.array_equal(p["ids"][r][:b.lens[i]], b.ids[i])
        assert np.all(p["ids"][r][b.lens[i]:] == pad_id)                   # padding rows: pad token
        assert np.array_equal(p["pos"][r], np.arange(rows8[i]))
        assert np.all(p["seq"][r] == i)
        assert soff[i] % 8 == 0
    # encoder tiles (sliding-window layers: <= q_tile queries; global layers: <= q_tile_global):
    # every valid row of every question exactly once, inside its question, a full tile unless it
    # holds the question's last row, longest questions first; each list is padded with empty tiles
    # to the bucket's capacity T / 64 + B
    valid_rows = np.concatenate([np.arange(soff[i], soff[i] + b.lens[i]) for i in range(b.B)])
    for key, qtl in (("tiles", q_tile), ("gltiles", q_tile_global)):
        assert len(p[key]) == p["T"] // 64 + b.B
        real = p[key][p[key][:, 2] > 0]
        assert np.all(p[key][len(real):] == 0)
        assert np.all(np.diff(b.lens[real[:, 0]]) <= 0)
        cover = np.zeros(p["T"], int)
        for seq, q0, nq, _ in real:
            assert 1 <= nq <= qtl and q0 % qtl == 0 and q0 + nq <= b.lens[seq]
            assert nq == qtl or q0 + nq == b.lens[seq]
            cover[soff[seq] + q0: soff[seq] + q0 + nq] += 1
        assert np.all(cover[valid_rows] == 1) and cover.sum() == p["valid"]
    # gathered rows: markers in question order, padded with row 0 to a multiple of 64, then one CLS
    # row per question
    nmk = int(b.nmark.sum())
    KT = up64(nmk)
    assert p["KT"] == KT and p["R"] == KT + b.B
    mk = np.concatenate(b.markers)
    moff = np.concatenate([[0], np.cumsum(b.nmark)])
    assert np.array_equal(p["moff"], moff[:-1])
    assert np.all(p["grow"][nmk:KT] == 0)
    for i in range(b.B):
        assert np.array_equal(p["grow"][moff[i]:moff[i + 1]], soff[i] + mk[moff[i]:moff[i + 1]])
        assert p["grow"][KT + i] == soff[i]
    assert len(p["gtiles"]) == p["R"] // 64 + b.B
    greal = p["gtiles"][p["gtiles"][:, 2] > 0]
    assert np.all(p["gtiles"][len(greal):] == 0)
    seen = np.zeros(p["R"], int)
    for seq, start, nq, _ in greal:
        assert 1 <= nq <= 64
        for gi in p["gq"][start:start + nq]:
            seen[gi] += 1
            assert soff[seq] <= p["grow"][gi] < soff[seq] + b.lens[seq]
    assert np.all(seen[:nmk] == 1) and np.all(seen[nmk:KT] == 0) and np.all(seen[KT:] == 1)
    del cfg


@settings(max_examples=80, deadline=None, suppress_health_check=[HealthCheck.function_scoped_fixture])
@given(data=st.data())
def test_layout_properties_of_random_batches(host, data):
    """The layout invariants of test_layout_of_a_pass on random batches (1-12 questions of 1-320
    tokens, 1-255 markers, both query tilings), planned into one pass or, under tighter row,
    question and gathered-row caps, several: the passes take the questions in order, each within
    its caps, and each pass's layout holds for its own questions."""
    cfg = ck.PRESETS["tiny"]
    n = data.draw(st.integers(1, 12), label="questions")
    lens = data.draw(st.lists(st.integers(1, 320), min_size=n, max_size=n), label="lens")
    nm = data.draw(st.lists(st.integers(1, 255), min_size=n, max_size=n), label="markers")
    q_tile, q_tile_global = data.draw(st.sampled_from([(64, 64), (64, 128), (128, 128)]), label="tiles")
    rows_cap = data.draw(st.sampled_from([320, 640, 1024, 65536]), label="pass_tokens")
    seqs_cap = data.draw(st.sampled_from([1, 3, 512]), label="max_seqs")
    grows_cap = data.draw(st.sampled_from([257, 512, 32768]), label="max_grows")
    b = wl.make_batch(cfg, lens, nm, seed=data.draw(st.integers(0, 1000), label="seed"))
    ps = plan(host, *b.flat(), max_len=320, pad_id=cfg.pad_id, pass_tokens=rows_cap, max_seqs=seqs_cap,
              max_grows=grows_cap, q_tile=q_tile, q_tile_global=q_tile_global)
    assert ps is not None
    nxt = 0
    for p in ps:
        assert p["first"] == nxt and p["B"] >= 1
        sub = b.subset(range(nxt, nxt + p["B"]))
        rows8 = int(np.sum((sub.lens + 7) // 8 * 8))
        assert p["B"] <= seqs_cap and (p["B"] == 1 or rows8 <= rows_cap)
        assert p["B"] == 1 or up64(int(sub.nmark.sum())) + p["B"] <= max(grows_cap, 257)
        check_layout(sub, p, cfg.pad_id, q_tile, q_tile_global)
        nxt += p["B"]
    assert nxt == n


def test_pass_splitting(host):
    cfg = ck.PRESETS["tiny"]
    lens = [300, 200, 150, 10, 320, 64, 5]
    b = wl.make_batch(cfg, lens, [2, 3, 4, 5, 6, 7, 8], seed=2)

    def greedy(rows, seqs):                  # questions in order while the pass still fits
        out, cur, t = [], [], 0
        for i, L in enumerate(lens):
            L8 = (L + 7) // 8 * 8
            if cur and (t + L8 > rows or len(cur) == seqs):
                out.append(cur)
                cur, t = [], 0
            cur.append(i)
            t += L8
        return out + [cur]
    for rows, seqs in ((640, 3), (400, 512), (320, 2)):
        ps = plan(host, *b.flat(), max_len=320, pass_tokens=rows, max_seqs=seqs)
        exp = greedy(rows, seqs)
        assert [p["first"] for p in ps] == [g[0] for g in exp]
        assert [p["B"] for p in ps] == [len(g) for g in exp]
        assert all(p["T"] <= up64(rows) for p in ps)
    assert [p["B"] for p in plan(host, *b.flat(), max_len=320, pass_tokens=640, max_seqs=3)] == [2, 3, 2]
    assert [p["B"] for p in plan(host, *b.flat(), max_len=320, pass_tokens=320)] == [1, 1, 2, 1, 2]
    # gathered-row cap: marker rows padded to 64 plus one CLS row per question fit max_grows (at
    # least 257, one question of 255 markers)
    nm = [100, 90, 60, 5, 255, 64, 8]
    b = wl.make_batch(cfg, lens, nm, seed=2)
    ps = plan(host, *b.flat(), max_len=320, max_grows=128)
    assert all(p["R"] <= 257 for p in ps) and sum(p["B"] for p in ps) == 7
    # 100 + 90 -> 192 rows + 2 CLS; + 60 -> 256 + 3 > 257; 60 + 5 -> 128 + 2; + 255 > 257; 255 alone;
    # 64 + 8 -> 128 + 2
    assert [p["B"] for p in ps] == [2, 2, 1, 2]


def test_config_parsing_matches_checkpoint(host, tiny_ckpt):
    out = np.zeros(16, np.int32)
    f = np.zeros(6, np.float32)
    err = ctypes.create_string_buffer(256)
    assert host.laya_host_config(tiny_ckpt.encode(), P(out)[1], f.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                 err, 256) == 0
    c = ck.PRESETS["tiny"]
    assert list(out) == [c.n_layers, c.d, c.n_heads, c.head_dim, c.intermediate, c.vocab, c.max_len, c.head_max_len,
                         c.head_layers, c.n_act, c.local_attention, c.pad_id, c.cls_id, c.sep_id, c.mask_id,
                         sum(c.is_global(i) for i in range(c.n_layers))]
    assert np.allclose(f, [c.norm_eps, c.rope_theta_global, c.rope_theta_local, 1, 1, 1])
    assert [host.laya_host_layer_is_global(tiny_ckpt.encode(), i) for i in range(4)] == [1, 0, 0, 1]
    assert host.laya_host_config(b"/nonexistent", P(out)[1], f.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                 err, 256) == -1
    assert b"cannot open" in err.value


def test_config_defaults_and_global_every(host):
    with tempfile.TemporaryDirectory() as d:
        os.makedirs(os.path.join(d, "encoder"))
        json.dump({"num_hidden_layers": 7, "hidden_size": 256, "num_attention_heads": 4, "intermediate_size": 64,
                   "vocab_size": 99, "global_attn_every_n_layers": 2, "global_rope_theta": 5000.0},
                  open(os.path.join(d, "encoder", "config.json"), "w"))
        out = np.zeros(16, np.int32)
        f = np.zeros(6, np.float32)
        err = ctypes.create_string_buffer(256)
        assert host.laya_host_config(d.encode(), P(out)[1], f.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), err,
                                     256) == 0
        assert out[6] == 512 and out[8] == 2 and out[9] == 2      # agent config absent: reference defaults
        assert [host.laya_host_layer_is_global(d.encode(), i) for i in range(7)] == [1, 0, 1, 0, 1, 0, 1]
        assert f[1] == 5000.0 and f[2] == 10000.0


@pytest.mark.parametrize("dtype", ["F32", "BF16", "F16"])
def test_safetensors_reader(host, dtype):
    rs = np.random.RandomState(0)
    ts = [("a.weight", (3, 5)), ("b", (7,)), ("c.bias", (2, 2, 2))]
    vals = [rs.randn(*s).astype(np.float32) for _, s in ts]
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "m.safetensors")
        ck.write_safetensors(path, ts, lambda i: vals[i], dtype)
        py = ck.read_safetensors(path)
        for (name, shape), v in zip(ts, vals):
            out = np.zeros(int(np.prod(shape)), np.float32)
            sh = np.zeros(8, np.int64)
            nd = ctypes.c_int()
            n = host.laya_host_read_tensor(path.encode(), name.encode(), out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                           out.size, sh.ctypes.data_as(ctypes.POINTER(ctypes.c_longlong)), ctypes.byref(nd))
            assert n == out.size and tuple(sh[:nd.value]) == shape
            assert np.array_equal(out.reshape(shape), py[name])
            exp = {"F32": v, "BF16": ck.bf16_bits_to_f32(ck.to_bf16_bits(v)).reshape(shape),
                   "F16": v.astype(np.float16).astype(np.float32)}[dtype]
            assert np.array_equal(out.reshape(shape), exp)
        assert host.laya_host_read_tensor(path.encode(), b"missing", None, 0, None, None) == -1


def test_bf16_rounding_is_nearest_even():
    x = np.array([1.0, 1.00390625, 1.005859375, -2.5, 3.0e38], np.float32)   # 1+2^-8 is a tie -> even
    b = ck.bf16_bits_to_f32(ck.to_bf16_bits(x))
    assert list(b[:4]) == [1.0, 1.0, 1.0078125, -2.5]


def test_checkpoint_generation_is_deterministic(tiny_ckpt):
    cfg, W = ck.load_checkpoint(tiny_ckpt)
    W2 = ck.generate_weights(ck.PRESETS["tiny"], 0, ln_jitter=0.1)
    assert set(W) == set(W2)
    assert all(np.array_equal(W[k], W2[k]) for k in W)
    assert cfg.n_layers == 4 and cfg.max_len == 320
