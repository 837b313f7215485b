import json
import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

from layamd_amd import checkpoint as ck  # noqa: E402

GOLDEN = os.path.join(REPO, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP engine through the C ABI)")
    config.addinivalue_line("markers", "slow: full-size model on the CPU (tens of seconds)")


def golden_model(tag):
    with open(os.path.join(GOLDEN, tag, "manifest.json")) as f:
        return json.load(f)["model"]


def checkpoint_dir(tag):
    """Writes (once) the seeded checkpoint a golden set was generated from and returns its dir."""
    m = golden_model(tag)
    return ck.cached_checkpoint(m["preset"], seed=m["seed"], std=m["std"], ln_jitter=m["ln_jitter"], dtype=m["dtype"])


def read_tiny_case(case):
    d = os.path.join(GOLDEN, "tiny", case["name"])
    sh = case["shapes"]
    out = {}
    for n, s in sh.items():
        dt = np.int32 if n in ("input_ids", "attention_mask", "marker_pos", "marker_mask", "qtype") else np.float32
        out[n] = np.fromfile(os.path.join(d, n + ".bin"), dtype=dt).reshape(s)
    return out


def tiny_cases():
    with open(os.path.join(GOLDEN, "tiny", "manifest.json")) as f:
        return json.load(f)["cases"]


def unpad_case(c):
    """Golden padded case -> ABI arguments (as src/test_parity.cpp:44-51 of the reference does)."""
    att, ids, mm, mp = c["attention_mask"], c["input_ids"], c["marker_mask"], c["marker_pos"]
    lens = att.sum(1).astype(np.int32)
    nm = mm.sum(1).astype(np.int32)
    flat_ids = np.concatenate([ids[i, :lens[i]] for i in range(len(lens))]).astype(np.int32)
    flat_mk = np.concatenate([mp[i, :nm[i]] for i in range(len(lens))]).astype(np.int32)
    return lens, flat_ids, nm, flat_mk, c["qtype"].astype(np.int32)


@pytest.fixture(scope="session")
def tiny_ckpt():
    return checkpoint_dir("tiny")
