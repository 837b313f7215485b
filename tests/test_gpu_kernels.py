"""Kernel-level parity on the GPU, through the library's C-ABI measurement hooks (laya_ext.h):

  * the MFMA GEMM at the encoder microbenchmark shapes (K x N in 1024x3072, 1024x1024, 1024x5248,
    2624x1024; M = 512 and 16384; bf16 and fp32 operands, fp32 accumulate) against an fp64 CPU
    product, as the reference checks its GEMM at the layer shapes against a library
    (bench/probes/wgemm_bench.cpp:29-57);
  * the attention kernels (bf16 k_attention_bf16, the benchmarked one, and the fp32 k_attention)
    in the engine's packed layout against fp64 masked softmax attention: sliding windows (+-64
    keys, inclusive, HF masking_utils.py:141-151) and global attention, lengths on both sides of
    the 64-key block and window edges, the ModernBERT-large b32 x s512 and mmBERT-base b16 x s1024
    length mixes, 64- and 128-query tiles, gathered queries (the decision head's last layer), and
    empty tiles (skipped).

Error bounds (stated per test, derived from the arithmetic, not fitted):
  GEMM, fp32 accumulate of K products: |err| <= 8 * 2^-24 * sqrt(K) * (|A| |W|^T) elementwise
    (a random-walk bound with margin; a dropped K chunk or a wrong row is off by O(|C|)); the bf16
    store adds its rounding, 2^-8 |C|.
  bf16 attention: probabilities are rounded to bf16 (relative 2^-8) before P V and the row sum, so
    the output is an exact weighted average with weights off by at most 2 * 2^-8 relative (to first
    order; 2% margin below): |err| <= 2^-7 * (P |V|) + 2^-8 |O| (the bf16 output rounding) + 1e-6.
  fp32 attention: |err| <= 1e-5 * (P |V|) + 1e-5 |O| + 1e-6.
  Uniform scores (Q = 0): every visible key has probability exactly 1 / n, so the output is the
    mean of exactly the visible keys' V rows; one key too many or too few at a window edge moves
    it by about |V| / 129, against a bound of 2^-8 |O| + 2^-16.
"""
import numpy as np
import pytest

from layamd_amd import checkpoint as ck
from layamd_amd import engine as le
from layamd_amd import workloads as wl

pytestmark = pytest.mark.gpu

U32 = 2.0 ** -24

# ---------------------------------------------------------------- GEMM at the encoder shapes
C2_SHAPES = [(1024, 3072), (1024, 1024), (1024, 5248), (2624, 1024)]      # (K, N)


def _sample_rows(M, n=48, seed=0):
    """All rows of a small M; for a large M, the tile edges of every tile shape plus seeded rows."""
    if M <= 1024:
        return np.arange(M)
    edges = [0, 1, 127, 128, 159, 160, 191, 192, 255, 256, 8191, 8192, M - 257, M - 256, M - 129, M - 2, M - 1]
    rs = np.random.RandomState(seed).randint(0, M, n)
    return np.unique(np.concatenate([edges, rs]))


@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
@pytest.mark.parametrize("M", [512, 16384])
@pytest.mark.parametrize("K,N", C2_SHAPES)
def test_gemm_encoder_shapes(dtype, M, K, N):
    """C = A W^T (store) and X += A W^T (fp32 residual) with the planner's tile choice, A ~ N(0,1)
    and W ~ N(0,0.02) in the operand type, checked row by row against an fp64 product."""
    import torch
    lib = le.load_library()
    prev = le.gemm_config(lib, -1)
    try:
        gen = torch.Generator(device="cuda").manual_seed(M + 7 * N + K)
        tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
        A = torch.randn(M, K, generator=gen, device="cuda").to(tdt)
        W = (torch.randn(N, K, generator=gen, device="cuda") * 0.02).to(tdt)
        X0 = torch.randn(M, N, generator=gen, device="cuda")
        C = torch.full((M, N), float("nan"), dtype=tdt, device="cuda")
        le.gemm(lib, A, W, C)
        X = X0.clone()
        le.gemm(lib, A, W, X, residual=True)
        torch.cuda.synchronize()
    finally:
        le.gemm_config(lib, prev)
    rows = _sample_rows(M)
    a = A[rows].double().cpu().numpy()
    w = W.double().cpu().numpy()
    ref = a @ w.T
    acc_tol = 8 * U32 * np.sqrt(K) * (np.abs(a) @ np.abs(w).T)
    x_err = np.abs(X[rows].double().cpu().numpy() - X0[rows].double().cpu().numpy() - ref)
    x_tol = acc_tol + U32 * np.abs(X[rows].double().cpu().numpy()) + 1e-7
    assert np.all(x_err <= x_tol), (float(x_err.max()), float((x_err / x_tol).max()))
    c = C[rows].double().cpu().numpy()
    assert np.isfinite(c).all()
    c_tol = acc_tol + (2.0 ** -8 if dtype == "bf16" else U32) * np.abs(ref) + 1e-7
    c_err = np.abs(c - ref)
    assert np.all(c_err <= c_tol), (float(c_err.max()), float((c_err / c_tol).max()))


@pytest.mark.parametrize("M,K,N,ks", [(512, 1024, 1024, 3), (160, 2624, 1024, 7), (160, 2624, 1024, 11),
                                       (512, 4096, 1024, 16), (512, 1024, 3072, 4)])
def test_gemm_split_k_chunks(M, K, N, ks):
    """bf16 split-K (laya_ext_gemm_ksplit): K in chunks of ceil(K / 64 / ks) whole 64-deep stages,
    the last one shorter when ks does not divide the stage count (K = 1024 in 3 chunks of 6, 6 and
    4 stages; K = 2624, 41 stages, in 7 chunks of 6 and one of 5, or 11 of 4 and one of 1), partial
    products summed in chunk order: the store and the fp32 residual update against an fp64 product
    with the same bound as the unsplit GEMM (a chunk dropped or read twice is off by O(|C|))."""
    import torch
    lib = le.load_library()
    ws = torch.empty(16 << 20, dtype=torch.float32, device="cuda")
    prev = le.gemm_ksplit(lib, ks, ws)
    try:
        gen = torch.Generator(device="cuda").manual_seed(M + 3 * N + K + ks)
        A = torch.randn(M, K, generator=gen, device="cuda").to(torch.bfloat16)
        W = (torch.randn(N, K, generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
        X0 = torch.randn(M, N, generator=gen, device="cuda")
        C = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
        le.gemm(lib, A, W, C)
        X = X0.clone()
        le.gemm(lib, A, W, X, residual=True)
        torch.cuda.synchronize()
    finally:
        le.gemm_ksplit(lib, prev)
    a, w = A.double().cpu().numpy(), W.double().cpu().numpy()
    ref = a @ w.T
    acc_tol = 8 * U32 * np.sqrt(K) * (np.abs(a) @ np.abs(w).T)
    xn = X.double().cpu().numpy()
    x_err = np.abs(xn - X0.double().cpu().numpy() - ref)
    assert np.all(x_err <= acc_tol + U32 * np.abs(xn) + 1e-7), float(x_err.max())
    c_err = np.abs(C.double().cpu().numpy() - ref)
    assert np.all(c_err <= acc_tol + 2.0 ** -8 * np.abs(ref) + 1e-7), float(c_err.max())


# ---------------------------------------------------------------- attention kernels
def _up(x, a):
    return (int(x) + a - 1) // a * a


class Packed:
    """Questions packed as the engine packs them: question b owns rows soff[b] .. soff[b] + len - 1,
    soff a multiple of 8; V^T [H*64][ldv] with column = row and 64 columns of slack."""

    def __init__(self, lens, H, dtype, seed, qzero=False, qscale=1.0, kramp=0.0):
        import torch
        self.lens = [int(x) for x in lens]
        self.H, self.D = H, 64 * H
        self.soff = np.concatenate([[0], np.cumsum([_up(L, 8) for L in self.lens])]).astype(np.int32)
        self.rows = _up(self.soff[-1], 64)
        ldv = _up(self.rows + 64, 64)
        g = torch.Generator(device="cpu").manual_seed(seed)
        tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
        q = torch.zeros(self.rows, self.D) if qzero else torch.randn(self.rows, self.D, generator=g) * qscale
        k = torch.randn(self.rows, self.D, generator=g)
        if kramp:
            # key j of a question scaled by 1 + kramp j / len: later keys score ever higher
            ramp = torch.ones(self.rows)
            for b, L in enumerate(self.lens):
                ramp[self.soff[b]:self.soff[b] + L] = 1.0 + kramp * torch.arange(L) / L
            k = k * ramp[:, None]
        v = torch.randn(self.rows, self.D, generator=g)
        self.q, self.k, self.v = (t.to(tdt) for t in (q, k, v))
        vt = torch.zeros(self.D, ldv, dtype=tdt)
        vt[:, :self.rows] = self.v.T
        self.dq, self.dk, self.dvt = self.q.cuda(), self.k.cuda(), vt.cuda()
        self.qd, self.kd, self.vd = (t.double().numpy() for t in (self.q, self.k, self.v))
        self.dsoff = torch.as_tensor(self.soff).cuda()
        self.dvlen = torch.as_tensor(np.array(self.lens, np.int32)).cuda()
        self.dtype = dtype

    def encoder_tiles(self, qtile, n_empty=3):
        t = [(b, q0, min(qtile, L - q0), 0) for b, L in enumerate(self.lens) for q0 in range(0, L, qtile)]
        t.sort(key=lambda x: -self.lens[x[0]])                       # longest first, as the packer orders them
        return np.array(t + [(0, 0, 0, 0)] * n_empty, np.int32)

    def run(self, tiles, window_half, qtile=64, gq=None, grow=None, out_rows=None):
        import torch
        lib = le.load_library()
        O = torch.full((out_rows or self.rows, self.D), float("nan"), dtype=self.dq.dtype, device="cuda")
        dt = lambda a: torch.as_tensor(a).cuda() if a is not None else None
        le.attention(lib, 1 if self.dtype == "bf16" else 0, self.dq, self.dk, self.dvt, O, dt(tiles), self.dsoff,
                     self.dvlen, self.H, window_half, 0.125, qtile=qtile, gq=dt(gq), grow=dt(grow))
        torch.cuda.synchronize()
        return O.double().cpu().numpy()

    def reference(self, b, pos, window_half):
        """fp64 output rows [len(pos), D] of question b's queries at positions pos, and the
        per-element bound P |V|."""
        s0, L = self.soff[b], self.lens[b]
        q = self.qd[s0 + np.asarray(pos)].reshape(len(pos), self.H, 64).transpose(1, 0, 2)
        k = self.kd[s0:s0 + L].reshape(L, self.H, 64).transpose(1, 0, 2)
        v = self.vd[s0:s0 + L].reshape(L, self.H, 64).transpose(1, 0, 2)
        s = q @ k.transpose(0, 2, 1) * 0.125
        if window_half > 0:
            band = np.abs(np.asarray(pos)[:, None] - np.arange(L)[None, :]) <= window_half
            s = np.where(band[None], s, -np.inf)
        p = np.exp(s - s.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        o = (p @ v).transpose(1, 0, 2).reshape(len(pos), self.D)
        pv = (p @ np.abs(v)).transpose(1, 0, 2).reshape(len(pos), self.D)
        return o, pv


def _check(pk, got_rows, b, pos, window_half, uniform):
    ref, pv = pk.reference(b, pos, window_half)
    got = got_rows
    assert np.isfinite(got).all()
    if uniform:
        tol = (2.0 ** -8 if pk.dtype == "bf16" else 1e-6) * np.abs(ref) + 2.0 ** -16
    elif pk.dtype == "bf16":
        tol = 1.02 * (2.0 ** -7 * pv + 2.0 ** -8 * np.abs(ref)) + 1e-6
    else:
        tol = 1e-5 * pv + 1e-5 * np.abs(ref) + 1e-6
    err = np.abs(got - ref)
    bad = err > tol
    assert not bad.any(), ("question", b, "len", pk.lens[b], "worst err/tol", float((err / tol).max()))
    return float((err / tol).max())


EDGE_LENS = [1, 2, 63, 64, 65, 127, 128, 129, 130, 191, 192, 193, 256, 320]


@pytest.mark.parametrize("dtype,qtile", [("bf16", 64), ("bf16", 128), ("fp32", 64)])
@pytest.mark.parametrize("window_half", [64, 0])
@pytest.mark.parametrize("uniform", [False, True])
def test_attention_edges(dtype, qtile, window_half, uniform):
    """Lengths on both sides of the 64-key blocks and the +-64 window, two heads, every query."""
    pk = Packed(EDGE_LENS, 2, dtype, seed=11, qzero=uniform)
    got = pk.run(pk.encoder_tiles(qtile), window_half, qtile)
    worst = 0.0
    for b, L in enumerate(pk.lens):
        worst = max(worst, _check(pk, got[pk.soff[b]:pk.soff[b] + L], b, np.arange(L), window_half, uniform))
    print("attention edges %s q%d w%d uniform=%s: worst err/bound %.3f" % (dtype, qtile, window_half, uniform, worst))


@pytest.mark.parametrize("dtype,qtile", [("bf16", 64), ("bf16", 128), ("fp32", 64)])
@pytest.mark.parametrize("window_half", [64, 0])
def test_attention_wide_score_range(dtype, qtile, window_half):
    """Scores spread far wider than the random inputs' (Q x 4, keys growing in scale along each
    question), so that a query's running maximum jumps by many times the bf16 kernel's trailing
    threshold (2^8 in probability) from block to block and its output and sum are rescaled often,
    with probabilities of earlier blocks underflowing; every query of every question."""
    pk = Packed(EDGE_LENS + [511, 700], 2, dtype, seed=14, qscale=4.0, kramp=2.0)
    got = pk.run(pk.encoder_tiles(qtile), window_half, qtile)
    worst = 0.0
    for b, L in enumerate(pk.lens):
        worst = max(worst, _check(pk, got[pk.soff[b]:pk.soff[b] + L], b, np.arange(L), window_half, False))
    print("attention wide scores %s q%d w%d: worst err/bound %.3f" % (dtype, qtile, window_half, worst))


@pytest.mark.parametrize("workload,dtype,qtile", [("c3", "bf16", 64), ("c3", "bf16", 128), ("c4", "bf16", 64),
                                                  ("c3", "fp32", 64)])
@pytest.mark.parametrize("window_half", [64, 0])
def test_attention_workload_lengths(workload, dtype, qtile, window_half):
    """The b32 x s512 length mix with 16 heads (ModernBERT-large) and the b16 x s1024 mix with 12
    heads (mmBERT-base), sliding and global; every query of every question, 4 heads checked."""
    batch = wl.CONFIGS[workload](0)
    pk = Packed(batch.lens, batch.cfg.n_heads, dtype, seed=12)
    got = pk.run(pk.encoder_tiles(qtile), window_half, qtile)
    heads = [0, 5, pk.H // 2, pk.H - 1]
    cols = np.concatenate([np.arange(64 * h, 64 * h + 64) for h in heads])
    worst = 0.0
    for b, L in enumerate(pk.lens):
        ref, pv = pk.reference(b, np.arange(L), window_half)
        g = got[pk.soff[b]:pk.soff[b] + L][:, cols]
        ref, pv = ref[:, cols], pv[:, cols]
        tol = (1.02 * (2.0 ** -7 * pv + 2.0 ** -8 * np.abs(ref)) + 1e-6) if dtype == "bf16" else \
            (1e-5 * pv + 1e-5 * np.abs(ref) + 1e-6)
        err = np.abs(g - ref)
        assert np.isfinite(g).all() and np.all(err <= tol), (b, L, float((err / tol).max()))
        worst = max(worst, float((err / tol).max()))
    print("attention %s %s q%d w%d: worst err/bound %.3f" % (workload, dtype, qtile, window_half, worst))


@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
def test_attention_gathered_queries(dtype):
    """The decision head's last layer: queries are gathered rows (each question's markers, then its
    CLS row) attending to all of their question's keys; outputs go to the gathered row.  One
    question has 255 markers (five gathered tiles)."""
    lens = [200, 37, 512, 1, 129, 300]
    nmark = [4, 3, 255, 1, 12, 64]
    pk = Packed(lens, 4, dtype, seed=13)
    marks = [wl.spread_markers(L, k) for L, k in zip(lens, nmark)]
    KT = _up(sum(nmark), 64)
    R = KT + len(lens)
    grow = np.zeros(R, np.int32)
    gq, gtiles, moff = [], [], 0
    for b, (L, m) in enumerate(zip(lens, marks)):
        grow[moff:moff + len(m)] = pk.soff[b] + m
        grow[KT + b] = pk.soff[b]
        ids = list(range(moff, moff + len(m))) + [KT + b]
        for s in range(0, len(ids), 64):
            gtiles.append((b, len(gq), min(64, len(ids) - s), 0))
            gq.extend(ids[s:s + 64])
        moff += len(m)
    gtiles += [(0, 0, 0, 0)] * 2
    got = pk.run(np.array(gtiles, np.int32), 0, 64, gq=np.array(gq, np.int32), grow=grow, out_rows=R)
    moff = 0
    for b, m in enumerate(marks):
        pos = list(m) + [0]
        rows = list(range(moff, moff + len(m))) + [KT + b]
        _check(pk, got[rows], b, np.array(pos), 0, False)
        moff += len(m)


def test_attention_rejects_bad_arguments():
    """The hook refuses what the kernels cannot take (128-query tiles in fp32 or gathered mode,
    misaligned strides) before launching anything."""
    import ctypes
    import torch
    lib = le.load_library()
    pk = Packed([70], 1, "fp32", seed=1)
    tiles = torch.as_tensor(pk.encoder_tiles(64)).cuda()
    O = torch.zeros(pk.rows, pk.D, device="cuda")
    with pytest.raises(ValueError):
        le.attention(lib, 0, pk.dq, pk.dk, pk.dvt, O, tiles, pk.dsoff, pk.dvlen, 1, 64, 0.125, qtile=128)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.laya_ext_attention(0, pk.dq.data_ptr(), pk.dk.data_ptr(), 63, pk.rows, pk.dvt.data_ptr(), pk.dvt.shape[1],
                                O.data_ptr(), 64, tiles.data_ptr(), tiles.shape[0], 64, 1, pk.dsoff.data_ptr(),
                                pk.dvlen.data_ptr(), None, None, 64, 0.125, st)
    assert rc == -1
