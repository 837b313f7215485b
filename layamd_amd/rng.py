"""Counter-based random numbers shared by the weight generator and the workload generators.

Every draw is a pure function of (stream key, index), so a tensor's values do not depend on the
order in which tensors are generated, on numpy's or torch's RNG implementations, or on chunking.

    u64(key, i)   = splitmix64_mix(key + (i + 1) * 0x9E3779B97F4A7C15)
    uniform(key,i) = (u64 >> 11 + 0.5) * 2^-53                      in (0, 1)
    normal(key,i)  = sqrt(-2 ln u1) * cos(2 pi u2)                   Box-Muller on one u64:
                     u1 = ((u64 >> 32) + 0.5) * 2^-32, u2 = ((u64 & 0xffffffff) + 0.5) * 2^-32
    stream key     = splitmix64_mix(seed * 0x9E3779B97F4A7C15 + stream_id + 1)

splitmix64 is Steele, Lea and Flood, "Fast splittable pseudorandom number generators" (OOPSLA
2014); Box-Muller is Box and Muller (1958).  All arithmetic is unsigned 64-bit with wrap-around.

The normal draws run in C++ (liblaya_host.so, laya_host_normal: the same definition, written in
place and multithreaded) when that library is built; the numpy code below is the fallback and
the readable statement of the algorithm.  Both use IEEE double log/sqrt/cos before the final
rounding to float32; every golden fixture was generated through the C++ routine.
"""
import ctypes
import os

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 22


def mix64(z):
    """splitmix64 output function on a uint64 array (wrap-around arithmetic)."""
    z = np.asarray(z, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def stream_key(seed: int, stream_id: int) -> np.uint64:
    with np.errstate(over="ignore"):
        base = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) * GOLDEN + np.uint64(stream_id + 1)
    return np.uint64(mix64(np.array([base], dtype=np.uint64))[0])


def u64(key: np.uint64, start: int, n: int) -> np.ndarray:
    idx = np.arange(start + 1, start + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return mix64(np.uint64(key) + idx * GOLDEN)


def uniform(key, n: int, start: int = 0) -> np.ndarray:
    z = u64(key, start, n)
    return ((z >> np.uint64(11)).astype(np.float64) + 0.5) * (2.0 ** -53)


_HOST = None


def _host():
    global _HOST
    if _HOST is None:
        path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "liblaya_host.so")
        _HOST = False
        if os.path.exists(path):
            lib = ctypes.CDLL(path)
            lib.laya_host_normal.argtypes = [ctypes.c_uint64, ctypes.c_longlong, ctypes.c_longlong, ctypes.c_double,
                                             ctypes.c_void_p, ctypes.c_int]
            lib.laya_host_normal.restype = None
            _HOST = lib
    return _HOST


def normal(key, n: int, std: float = 1.0, dtype=np.float32, out=None) -> np.ndarray:
    """n standard-normal draws scaled by std (float32)."""
    if out is None:
        out = np.empty(n, dtype=dtype)
    lib = _host()
    if lib and out.dtype == np.float32 and out.flags.c_contiguous:
        lib.laya_host_normal(int(key), 0, n, float(std), out.ctypes.data, min(16, os.cpu_count() or 1))
        return out
    for s in range(0, n, _CHUNK):
        m = min(_CHUNK, n - s)
        z = u64(key, s, m)
        u1 = ((z >> np.uint64(32)).astype(np.float64) + 0.5) * (2.0 ** -32)
        u2 = ((z & np.uint64(0xFFFFFFFF)).astype(np.float64) + 0.5) * (2.0 ** -32)
        out[s:s + m] = (np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2) * std).astype(dtype)
    return out


def randint(key, n: int, lo: int, hi: int, start: int = 0) -> np.ndarray:
    """Uniform integers in [lo, hi) via floor(uniform * (hi - lo))."""
    u = uniform(key, n, start)
    v = lo + np.floor(u * (hi - lo)).astype(np.int64)
    return np.minimum(v, hi - 1)
