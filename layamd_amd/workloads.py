"""Seeded synthetic question batches for the engine's benchmark and parity configurations.

A question is (token ids, marker positions, qtype), the unit `laya_forward_batch` takes
(src/laya_api.h:6-9 of the reference).  Token ids are uniform in [5, vocab) with CLS first and
SEP last; qtype is uniform in {0, 1, 2}.  Markers are spread over the sequence with
`spread_markers`.  All draws come from layamd_amd.rng streams keyed by (seed, purpose).
"""
import dataclasses
import math
from typing import List, Optional

import numpy as np

from . import rng
from .checkpoint import ModelConfig, PRESETS

_S_LENS, _S_IDS, _S_QT, _S_NM = 1001, 1002, 1003, 1004


@dataclasses.dataclass
class Batch:
    cfg: ModelConfig
    lens: np.ndarray            # [B] int32
    ids: List[np.ndarray]       # per question, int32
    markers: List[np.ndarray]   # per question, int32 positions in [0, len)
    qtypes: np.ndarray          # [B] int32
    dtype: str = "bf16"
    name: str = ""

    @property
    def B(self) -> int:
        return len(self.lens)

    @property
    def tokens(self) -> int:
        return int(np.sum(self.lens))

    @property
    def nmark(self) -> np.ndarray:
        return np.array([len(m) for m in self.markers], dtype=np.int32)

    def flat(self):
        """Arguments of laya_forward_batch: lens, concatenated ids, nmark, concatenated markers, qtypes."""
        return (np.ascontiguousarray(self.lens, np.int32),
                np.ascontiguousarray(np.concatenate(self.ids), np.int32),
                self.nmark,
                np.ascontiguousarray(np.concatenate(self.markers), np.int32),
                np.ascontiguousarray(self.qtypes, np.int32))

    def padded(self):
        """Right-padded batch as ref/rl_common.py:265-293 (collate_items) builds it."""
        n, L = self.B, int(max(self.lens))
        kmax = int(max(len(m) for m in self.markers))
        ids = np.full((n, L), self.cfg.pad_id, np.int64)
        att = np.zeros((n, L), np.int64)
        mpos = np.zeros((n, kmax), np.int64)
        mmask = np.zeros((n, kmax), bool)
        for i in range(n):
            ids[i, :self.lens[i]] = self.ids[i]
            att[i, :self.lens[i]] = 1
            k = len(self.markers[i])
            mpos[i, :k] = self.markers[i]
            mmask[i, :k] = True
        return ids, att, mpos, mmask, np.asarray(self.qtypes, np.int64)

    def subset(self, idx) -> "Batch":
        idx = list(idx)
        return Batch(self.cfg, self.lens[idx], [self.ids[i] for i in idx], [self.markers[i] for i in idx],
                     self.qtypes[idx], self.dtype, self.name + "[sub]")


def spread_markers(length: int, k: int) -> np.ndarray:
    """k marker positions inside [0, length): 1 + j*floor((length-2)/k) when they fit, otherwise
    positions cycling through 1..length-1 (markers may repeat; the ABI only bounds them)."""
    if length <= 1:
        return np.zeros(k, np.int32)
    if length - 2 >= k:
        step = (length - 2) // k
        return np.array([1 + j * step for j in range(k)], np.int32)
    return np.array([1 + (j % (length - 1)) for j in range(k)], np.int32)


def make_ids(cfg: ModelConfig, length: int, key, start: int) -> np.ndarray:
    body = rng.randint(key, length, 5, cfg.vocab, start=start).astype(np.int32)
    body[0] = cfg.cls_id
    if length > 1:
        body[-1] = cfg.sep_id
    return body


def make_batch(cfg: ModelConfig, lens, nmarks, seed: int = 0, dtype: str = "bf16", name: str = "",
               qtypes: Optional[np.ndarray] = None) -> Batch:
    lens = np.asarray(lens, np.int32)
    kid = rng.stream_key(seed, _S_IDS)
    ids, marks, off = [], [], 0
    for L, K in zip(lens, nmarks):
        ids.append(make_ids(cfg, int(L), kid, off))
        off += int(L)
        marks.append(spread_markers(int(L), int(K)))
    if qtypes is None:
        qtypes = rng.randint(rng.stream_key(seed, _S_QT), len(lens), 0, 3).astype(np.int32)
    return Batch(cfg, lens, ids, marks, np.asarray(qtypes, np.int32), dtype, name)


def c1(seed: int = 0) -> Batch:
    """ModernBERT-large + head, fp32, batch 1, seq 128, 4 markers."""
    return make_batch(PRESETS["large"], [128], [4], seed, "fp32", "c1-large-fp32-b1s128")


def c3(seed: int = 0) -> Batch:
    """ModernBERT-large + head, bf16, batch 32, lengths uniform in [32, 512], 4 markers."""
    cfg = PRESETS["large"]
    lens = rng.randint(rng.stream_key(seed, _S_LENS), 32, 32, 513)
    return make_batch(cfg, lens, [4] * 32, seed, "bf16", "c3-large-bf16-b32s512")


def c4(seed: int = 0) -> Batch:
    """mmBERT-base-shaped + head, bf16, batch 16, lengths uniform in [64, 1024], 4 markers."""
    cfg = PRESETS["base"]
    lens = rng.randint(rng.stream_key(seed, _S_LENS), 16, 64, 1025)
    return make_batch(cfg, lens, [4] * 16, seed, "bf16", "c4-base-bf16-b16s1024")


def c5(seed: int = 0) -> Batch:
    """ModernBERT-large (1024 context) + head, bf16, batch 64, lengths log-uniform on [16, 1024];
    8 questions per sequence with 2-5 options each, passed as one marker list per sequence."""
    cfg = PRESETS["large1024"]
    u = rng.uniform(rng.stream_key(seed, _S_LENS), 64)
    lens = np.minimum(1024, np.floor(np.exp(math.log(16) + u * (math.log(1025) - math.log(16))))).astype(np.int32)
    opts = rng.randint(rng.stream_key(seed, _S_NM), 64 * 8, 2, 6).reshape(64, 8)
    return make_batch(cfg, lens, opts.sum(1), seed, "bf16", "c5-large-bf16-b64s1024-varlen")


CONFIGS = {"c1": c1, "c3": c3, "c4": c4, "c5": c5}
