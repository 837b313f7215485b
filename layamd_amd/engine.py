"""ctypes binding of liblaya.so, shaped like the reference server's binding.

`Engine(lib_path, model_dir)` and `Engine.forward_batch(seqs, markers, qtypes)` have the same
names, arguments, return values and error behaviour as the reference's server-side class
(server/laya_server.py:18-50): one `laya_forward_batch` call per request batch, ValueError when
the engine rejects the batch, per-question logits arrays plus an [B, n_act] act array.  The
`forward_flat` variant takes the ABI's flat arrays directly (numpy), and the `laya_ext_*`
measurement hooks are exposed for the benchmark.

The library is the in-tree build (layamd_amd/liblaya.so, or $LAYA_LIB).  There is no fallback:
a missing library raises.
"""
import ctypes
import importlib.util
import os
import sys
from typing import List, Optional

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
DEFAULT_LIB = os.path.join(PKG, "liblaya.so")
HOST_LIB = os.path.join(PKG, "liblaya_host.so")

ABI_SYMBOLS = ["laya_create", "laya_forward_batch", "laya_forward", "laya_n_act", "laya_max_len",
               "laya_max_markers", "laya_temperature", "laya_prof_report", "laya_prof_reset", "laya_tune_all"]
EXT_SYMBOLS = ["laya_ext_prof_enable", "laya_ext_prof_stage", "laya_ext_replay", "laya_ext_precision", "laya_ext_gemm",
               "laya_ext_gemm_config", "laya_ext_gemm_split", "laya_ext_gemm_ksplit", "laya_ext_mfma_loop",
               "laya_ext_stats", "laya_ext_attention", "laya_ext_gemm_splitk_static", "laya_ext_hbm_copy",
               "laya_ext_prof_sequence"]
# every environment variable laya_create reads; Engine() sets the ones it is given for the duration
# of laya_create only
ENV_KNOBS = ["LAYA_PRECISION", "LAYA_MAX_TOKENS", "LAYA_PASS_TOKENS", "LAYA_MAX_SEQS", "LAYA_MAX_GATHERED",
             "LAYA_ATTN_QTILE", "LAYA_GRAPHS", "LAYA_MAX_GRAPHS", "LAYA_TUNE", "LAYA_GEMM_CFG", "LAYA_GEMM_SPLIT",
             "LAYA_PROFILE", "LAYA_DUMP_DIR", "LAYA_VERBOSE", "LAYA_LN_FOLD", "LAYA_LATENCY"]

_IP = ctypes.POINTER(ctypes.c_int)
_FP = ctypes.POINTER(ctypes.c_float)


def lib_path() -> str:
    return os.environ.get("LAYA_LIB", DEFAULT_LIB)


def load_library(path: Optional[str] = None) -> ctypes.CDLL:
    """Loads liblaya.so and declares every exported signature (no GPU work happens here).

    When PyTorch is installed it is imported first.  Both name the same HIP runtime library
    (SONAME libamdhip64.so.7), so liblaya.so then binds to the runtime instance torch loaded and
    the two share the device, streams and memory.  Loaded the other way round, torch brings a second
    instance of the runtime, and the library's instance sees no device."""
    path = path or lib_path()
    if not os.path.exists(path):
        raise FileNotFoundError("liblaya.so not built at %s (run python -m layamd_amd.build)" % path)
    if "torch" not in sys.modules and importlib.util.find_spec("torch") is not None:
        import torch  # noqa: F401
    L = ctypes.CDLL(path)
    L.laya_create.restype = ctypes.c_void_p
    L.laya_create.argtypes = [ctypes.c_char_p]
    L.laya_forward_batch.restype = ctypes.c_int
    L.laya_forward_batch.argtypes = [ctypes.c_void_p, ctypes.c_int, _IP, _IP, _IP, _IP, _IP, _FP, _FP]
    L.laya_forward.restype = None
    L.laya_forward.argtypes = [ctypes.c_void_p, _IP, ctypes.c_int, ctypes.c_int, _IP, ctypes.c_int, ctypes.c_int, _FP, _FP]
    for f in ("laya_n_act", "laya_max_len", "laya_max_markers"):
        getattr(L, f).argtypes = [ctypes.c_void_p]
        getattr(L, f).restype = ctypes.c_int
    L.laya_temperature.argtypes = [ctypes.c_void_p, ctypes.c_int]
    L.laya_temperature.restype = ctypes.c_float
    L.laya_prof_report.argtypes = [ctypes.c_void_p, ctypes.c_int]
    L.laya_prof_report.restype = None
    L.laya_prof_reset.argtypes = [ctypes.c_void_p]
    L.laya_prof_reset.restype = None
    L.laya_tune_all.argtypes = [ctypes.c_void_p]
    L.laya_tune_all.restype = None
    L.laya_ext_prof_enable.argtypes = [ctypes.c_void_p, ctypes.c_int]
    L.laya_ext_prof_enable.restype = ctypes.c_int
    L.laya_ext_prof_stage.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_char_p, ctypes.c_int,
                                      ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_longlong)]
    L.laya_ext_prof_stage.restype = ctypes.c_int
    L.laya_ext_prof_sequence.argtypes = [ctypes.c_void_p, _IP, ctypes.c_int]
    L.laya_ext_prof_sequence.restype = ctypes.c_int
    L.laya_ext_replay.argtypes = [ctypes.c_void_p, ctypes.c_int, _FP]
    L.laya_ext_replay.restype = ctypes.c_int
    L.laya_ext_precision.argtypes = [ctypes.c_void_p]
    L.laya_ext_precision.restype = ctypes.c_char_p
    L.laya_ext_gemm.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                ctypes.c_void_p, ctypes.c_int, _FP]
    L.laya_ext_gemm.restype = ctypes.c_int
    L.laya_ext_gemm_config.argtypes = [ctypes.c_int]
    L.laya_ext_gemm_config.restype = ctypes.c_int
    L.laya_ext_gemm_split.argtypes = [ctypes.c_int, ctypes.c_int]
    L.laya_ext_gemm_split.restype = ctypes.c_int
    L.laya_ext_gemm_ksplit.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t]
    L.laya_ext_gemm_ksplit.restype = ctypes.c_int
    L.laya_ext_mfma_loop.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                     ctypes.POINTER(ctypes.c_double)]
    L.laya_ext_mfma_loop.restype = ctypes.c_int
    L.laya_ext_hbm_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    L.laya_ext_hbm_copy.restype = ctypes.c_int
    L.laya_ext_stats.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_longlong), ctypes.c_int]
    L.laya_ext_stats.restype = ctypes.c_int
    L.laya_ext_attention.argtypes = ([ctypes.c_int] + [ctypes.c_void_p] * 2 + [ctypes.c_int] * 2 + [ctypes.c_void_p, ctypes.c_int,
                                     ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int] + [ctypes.c_void_p] * 4 + [ctypes.c_int, ctypes.c_float, ctypes.c_void_p])
    L.laya_ext_attention.restype = ctypes.c_int
    L.laya_ext_gemm_splitk_static.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                              ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                              ctypes.c_int, ctypes.c_void_p]
    L.laya_ext_gemm_splitk_static.restype = ctypes.c_int
    return L


def gemm(lib, A, W, C, bias=None, act=0, residual=False, stream=None, iters=1):
    """Runs the engine GEMM on torch device tensors (A [M,K], W [N,K], C [M,N]); returns total ms."""
    import torch
    dtype = 1 if A.dtype == torch.bfloat16 else 0
    ms = ctypes.c_float()
    st = stream if stream is not None else torch.cuda.current_stream().cuda_stream
    rc = lib.laya_ext_gemm(dtype, 1 if residual else 0, A.data_ptr(), W.data_ptr(), C.data_ptr(),
                           bias.data_ptr() if bias is not None else None, act, A.shape[0], W.shape[0], A.shape[1],
                           ctypes.c_void_p(st), iters, ctypes.byref(ms))
    if rc != 0:
        raise ValueError("gemm shape rejected: M=%d N=%d K=%d" % (A.shape[0], W.shape[0], A.shape[1]))
    return ms.value


def gemm_config(lib, cfg: int) -> int:
    """Pins the bf16 GEMM tile configuration (-1: planner, 0..8: see laya_ext.h); returns the previous."""
    prev = lib.laya_ext_gemm_config(cfg)
    if prev == -2:
        raise ValueError("invalid GEMM configuration %d" % cfg)
    return prev


def gemm_split(lib, split_rows: int, cfg_tail: int = -1):
    """Row split for pinned bf16 launches: rows [split_rows, M) in a second launch with cfg_tail."""
    if lib.laya_ext_gemm_split(split_rows, cfg_tail) != 0:
        raise ValueError("invalid GEMM split %d / %d" % (split_rows, cfg_tail))


def mfma_peak(lib, blocks_per_cu: int = 2, iters: int = 4096) -> float:
    """The chip's achievable bf16 MFMA rate in TFLOP/s (register-only MFMA loop on every CU)."""
    import torch
    ncu = torch.cuda.get_device_properties(0).multi_processor_count
    blocks = ncu * blocks_per_cu
    out = torch.empty(blocks * 256, dtype=torch.float32, device="cuda")
    flops = ctypes.c_double()
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def launch():
        if lib.laya_ext_mfma_loop(ctypes.c_void_p(out.data_ptr()), blocks, iters, st, ctypes.byref(flops)) != 0:
            raise RuntimeError("mfma loop rejected")

    launch()                                             # warm-up: the clock settles under load
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    launch()
    b.record()
    torch.cuda.synchronize()
    return flops.value / (a.elapsed_time(b) * 1e-3) / 1e12


def hbm_copy(lib, src, dst) -> None:
    """Launches the library's HBM copy of torch device tensor src into dst (same byte size, on the
    current stream); raises ValueError when the library rejects it."""
    import torch
    nbytes = src.numel() * src.element_size()
    if dst.numel() * dst.element_size() != nbytes:
        raise ValueError("hbm_copy: sizes differ")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if lib.laya_ext_hbm_copy(ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()), nbytes, st) != 0:
        raise ValueError("hbm_copy rejected")


def hbm_peak(lib, nbytes: int = 1 << 30, iters: int = 5) -> float:
    """The chip's achievable HBM rate in GB/s: bytes read plus bytes written per second by the
    library's stream copy over two buffers of nbytes, iters launches back to back."""
    import torch
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    hbm_copy(lib, src, dst)                                # warm-up
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(iters):
        hbm_copy(lib, src, dst)
    b.record()
    torch.cuda.synchronize()
    return 2.0 * nbytes * iters / (a.elapsed_time(b) * 1e-3) / 1e9


def gemm_ksplit(lib, ks: int, ws=None) -> int:
    """Split-K factor for later bf16 GEMM hook calls (0: none) with workspace ws (a torch device
    tensor); returns the previous factor."""
    prev = lib.laya_ext_gemm_ksplit(ks, ws.data_ptr() if ws is not None else None,
                                    ws.numel() * ws.element_size() if ws is not None else 0)
    if prev == -2:
        raise ValueError("invalid split-K factor %d" % ks)
    return prev


def _ptr(a: np.ndarray, ct):
    return a.ctypes.data_as(ctypes.POINTER(ct))


def attention(lib, dtype: int, Q, K, Vt, O, tiles, soff, vlen, H: int, window_half: int, scale: float, qtile: int = 64,
              gq=None, grow=None, stream=None):
    """The engine's attention kernel on torch device tensors in the packed layout of laya_ext.h
    (Q, K [rows, ldqk]; Vt [H*64, ldv]; O [.., ldo]; tiles int32 [n, 4]; soff, vlen int32)."""
    import torch
    st = stream if stream is not None else torch.cuda.current_stream().cuda_stream
    ptr = lambda t: t.data_ptr() if t is not None else None
    rc = lib.laya_ext_attention(dtype, Q.data_ptr(), K.data_ptr(), Q.shape[1], Q.shape[0], Vt.data_ptr(), Vt.shape[1],
                                O.data_ptr(), O.shape[1], tiles.data_ptr(), tiles.shape[0], qtile, H, soff.data_ptr(),
                                vlen.data_ptr(), ptr(gq), ptr(grow), window_half, scale, ctypes.c_void_p(st))
    if rc != 0:
        raise ValueError("attention arguments rejected")


class Engine:
    """One engine handle (not thread-safe; the engine lives until the process exits).

    precision and env set LAYA_* variables (None: unset) for the duration of laya_create only: the
    engine reads its configuration there, and the caller's environment is restored afterwards, so
    one engine's settings never leak into the next."""

    def __init__(self, lib_path_: Optional[str], model_dir: str, precision: Optional[str] = None, env=None):
        want = dict(env or {})
        if precision is not None:
            want["LAYA_PRECISION"] = precision
        saved = {k: os.environ.get(k) for k in want}
        self.lib = L = load_library(lib_path_)
        try:
            for k, v in want.items():
                if v is None:
                    os.environ.pop(k, None)
                else:
                    os.environ[k] = str(v)
            self.h = L.laya_create(model_dir.encode())
        finally:
            for k, v in saved.items():
                if v is None:
                    os.environ.pop(k, None)
                else:
                    os.environ[k] = v
        if not self.h:
            raise RuntimeError("laya_create failed for %s" % model_dir)
        self.n_act = L.laya_n_act(self.h)
        self.max_markers = L.laya_max_markers(self.h)
        self.max_len = L.laya_max_len(self.h)
        self.precision = L.laya_ext_precision(self.h).decode()

    # --- the reference server's call shape (server/laya_server.py:33-50)
    def forward_batch(self, seqs: List[List[int]], markers: List[List[int]], qtypes: List[int]):
        """Questions as Python lists (token ids, marker positions, qtype each), all in one
        laya_forward_batch call.  Returns one logits array per question and the [B, n_act] act
        logits; raises ValueError when the engine rejects the batch."""
        def cat(lists):
            return np.fromiter((v for l in lists for v in l), np.int32) if lists else np.zeros(0, np.int32)
        nmark = np.fromiter(map(len, markers), np.int32, len(markers))
        logits, act = self.forward_flat(np.fromiter(map(len, seqs), np.int32, len(seqs)), cat(seqs), nmark,
                                        cat(markers), np.asarray(qtypes, np.int32))
        return np.split(logits, np.cumsum(nmark)[:-1]) if len(nmark) else [], act

    # --- flat numpy arrays, exactly the ABI's arguments
    def forward_flat(self, lens, ids, nmark, markers, qtypes):
        lens = np.ascontiguousarray(lens, np.int32)
        ids = np.ascontiguousarray(ids, np.int32)
        nmark = np.ascontiguousarray(nmark, np.int32)
        markers = np.ascontiguousarray(markers, np.int32)
        qtypes = np.ascontiguousarray(qtypes, np.int32)
        B = len(lens)
        logits = np.zeros(max(1, int(nmark.sum()) if B else 0), np.float32)
        act = np.zeros(max(1, B * self.n_act), np.float32)
        rc = self.lib.laya_forward_batch(self.h, B, _ptr(lens, ctypes.c_int), _ptr(ids, ctypes.c_int),
                                         _ptr(nmark, ctypes.c_int), _ptr(markers, ctypes.c_int),
                                         _ptr(qtypes, ctypes.c_int), _ptr(logits, ctypes.c_float),
                                         _ptr(act, ctypes.c_float))
        if rc != 0:
            raise ValueError("laya_forward_batch returned %d: a length, marker count, marker position, qtype or "
                             "token id is outside the engine's limits" % rc)
        return logits[:int(nmark.sum())], act[:B * self.n_act].reshape(B, self.n_act)

    def forward_rc(self, lens, ids, nmark, markers, qtypes) -> int:
        """Raw return code of laya_forward_batch (for validation tests)."""
        lens = np.ascontiguousarray(lens, np.int32)
        ids = np.ascontiguousarray(ids if len(ids) else [0], np.int32)
        nmark = np.ascontiguousarray(nmark, np.int32)
        markers = np.ascontiguousarray(markers if len(markers) else [0], np.int32)
        qtypes = np.ascontiguousarray(qtypes, np.int32)
        logits = np.zeros(max(1, int(np.maximum(nmark, 0).sum())), np.float32)
        act = np.zeros(max(1, len(lens) * self.n_act), np.float32)
        return self.lib.laya_forward_batch(self.h, len(lens), _ptr(lens, ctypes.c_int), _ptr(ids, ctypes.c_int),
                                           _ptr(nmark, ctypes.c_int), _ptr(markers, ctypes.c_int),
                                           _ptr(qtypes, ctypes.c_int), _ptr(logits, ctypes.c_float),
                                           _ptr(act, ctypes.c_float))

    def forward_one(self, ids, markers, qtype: int):
        """laya_forward (single question)."""
        ids = np.ascontiguousarray(ids, np.int32)
        markers = np.ascontiguousarray(markers, np.int32)
        logits = np.zeros(len(markers), np.float32)
        act = np.zeros(self.n_act, np.float32)
        self.lib.laya_forward(self.h, _ptr(ids, ctypes.c_int), len(ids), len(ids), _ptr(markers, ctypes.c_int),
                              len(markers), int(qtype), _ptr(logits, ctypes.c_float), _ptr(act, ctypes.c_float))
        return logits, act

    def temperature(self, qtype: int) -> float:
        return float(self.lib.laya_temperature(self.h, qtype))

    def tune_all(self):
        self.lib.laya_tune_all(self.h)

    # --- measurement hooks
    def prof_enable(self, on: bool) -> bool:
        return bool(self.lib.laya_ext_prof_enable(self.h, 1 if on else 0))

    def prof_reset(self):
        self.lib.laya_prof_reset(self.h)

    def prof_report(self, iters: int = 1):
        self.lib.laya_prof_report(self.h, iters)

    def prof_stages(self):
        out, i = {}, 0
        name = ctypes.create_string_buffer(64)
        ms, calls = ctypes.c_double(), ctypes.c_longlong()
        while self.lib.laya_ext_prof_stage(self.h, i, name, 64, ctypes.byref(ms), ctypes.byref(calls)) == 0:
            out[name.value.decode()] = (ms.value, calls.value)
            i += 1
        return out

    def prof_sequence(self):
        """Stage name of every kernel launch of the last profiled pass, in launch order."""
        names = list(self.prof_stages())
        n = self.lib.laya_ext_prof_sequence(self.h, None, 0)
        buf = (ctypes.c_int * max(n, 1))()
        self.lib.laya_ext_prof_sequence(self.h, buf, n)
        return [names[buf[i]] for i in range(n)]

    def stats(self):
        """(graphs cached, graphs captured, tuned GEMM plans, tuned pass buckets)."""
        out = (ctypes.c_longlong * 4)()
        if self.lib.laya_ext_stats(self.h, out, 4) != 0:
            raise RuntimeError("laya_ext_stats failed")
        return tuple(int(x) for x in out)

    def replay(self, iters: int) -> float:
        ms = ctypes.c_float()
        if self.lib.laya_ext_replay(self.h, iters, ctypes.byref(ms)) != 0:
            raise RuntimeError("no pass to replay")
        return ms.value
