"""Laya checkpoint layout: model presets, the tensor-name contract and a seeded writer.

A Laya model directory holds (reference: src/engine.hip:141-176, src/laya.cpp:5-41)

    <dir>/encoder/config.json      ModernBERT config (HF key names)
    <dir>/rl_agent_config.json     max_len, head_max_len, head_layers, act_costs, temperature
    <dir>/model.safetensors        DecisionModel state dict (ref/rl_common.py:81-97)

`write_checkpoint` produces such a directory from a counter-based RNG (layamd_amd.rng), so the
same seed gives bit-identical weights on every machine.  Linear and embedding weights and linear
biases are N(0, 0.02); LayerNorm weights are 1 and LayerNorm biases 0 unless `ln_jitter` is set,
in which case they become 1 + N(0, ln_jitter) and N(0, 0.02) so that a dropped LayerNorm weight
or bias changes the output.  Each tensor draws from its own stream, keyed by its position in
`tensor_specs` (a fixed order), so no tensor depends on another's size.
"""
import dataclasses
import hashlib
import json
import os
import struct
from typing import Dict, List, Optional, Tuple

import numpy as np

from . import rng


@dataclasses.dataclass(frozen=True)
class ModelConfig:
    name: str
    n_layers: int
    d: int
    n_heads: int
    intermediate: int
    vocab: int
    max_len: int = 512
    head_max_len: int = 192
    head_layers: int = 2
    n_act: int = 2
    local_attention: int = 128
    global_every: int = 3
    norm_eps: float = 1e-5
    rope_theta_global: float = 160000.0
    rope_theta_local: float = 10000.0
    pad_id: int = 50283
    cls_id: int = 50281
    sep_id: int = 50282
    mask_id: int = 50284

    @property
    def head_dim(self) -> int:
        return self.d // self.n_heads

    @property
    def head_ffn(self) -> int:
        return 4 * self.d

    def is_global(self, layer: int) -> bool:
        return layer % self.global_every == 0

    def with_(self, **kw) -> "ModelConfig":
        return dataclasses.replace(self, **kw)


PRESETS: Dict[str, ModelConfig] = {
    # ModernBERT-large encoder as used by laya-en (docs/architecture.md:54 of the reference)
    "large": ModelConfig("large", 28, 1024, 16, 2624, 50368, max_len=512, head_max_len=192),
    # same encoder with the 1024-token context of the typed-decisions checkpoint
    "large1024": ModelConfig("large1024", 28, 1024, 16, 2624, 50368, max_len=1024, head_max_len=256),
    # mmBERT-base-shaped encoder (laya-multi)
    "base": ModelConfig("base", 22, 768, 12, 1152, 256000, max_len=1024, head_max_len=256),
    # small model with every structural feature (global + sliding layers, window < max_len)
    "tiny": ModelConfig("tiny", 4, 128, 2, 192, 512, max_len=320, head_max_len=96,
                        pad_id=0, cls_id=1, sep_id=2, mask_id=3),
}


def encoder_config_json(c: ModelConfig) -> dict:
    """HF ModernBertConfig keys (read by both the engine and transformers' AutoConfig)."""
    return {
        "architectures": ["ModernBertModel"],
        "model_type": "modernbert",
        "hidden_size": c.d,
        "num_hidden_layers": c.n_layers,
        "num_attention_heads": c.n_heads,
        "intermediate_size": c.intermediate,
        "vocab_size": c.vocab,
        "hidden_activation": "gelu",
        "max_position_embeddings": 8192,
        "norm_eps": c.norm_eps,
        "norm_bias": False,
        "attention_bias": False,
        "mlp_bias": False,
        "local_attention": c.local_attention,
        "global_attn_every_n_layers": c.global_every,
        "layer_types": ["full_attention" if c.is_global(i) else "sliding_attention" for i in range(c.n_layers)],
        "rope_parameters": {
            "full_attention": {"rope_type": "default", "rope_theta": c.rope_theta_global},
            "sliding_attention": {"rope_type": "default", "rope_theta": c.rope_theta_local},
        },
        "pad_token_id": c.pad_id,
        "cls_token_id": c.cls_id,
        "sep_token_id": c.sep_id,
        "bos_token_id": c.cls_id,
        "eos_token_id": c.sep_id,
        "mask_token_id": c.mask_id,
        "position_embedding_type": "absolute",
        "attention_dropout": 0.0,
        "embedding_dropout": 0.0,
        "mlp_dropout": 0.0,
        "torch_dtype": "float32",
    }


def agent_config_json(c: ModelConfig) -> dict:
    return {
        "encoder": "random-init-" + c.name,
        "max_len": c.max_len,
        "head_max_len": c.head_max_len,
        "head_layers": c.head_layers,
        "act_costs": [0.0] * (c.n_act - 1),
        "temperature": [1.0, 1.0, 1.0],
        "temperature_by_options": {},
        "amp_dtype": "bf16",
    }


# kinds: "w" linear/embedding weight, "b" linear bias, "lnw" LayerNorm weight, "lnb" LayerNorm bias,
# "temp" the temperature buffer
def tensor_specs(c: ModelConfig) -> List[Tuple[str, Tuple[int, ...], str]]:
    """The checkpoint tensor-name contract (src/engine.hip:147-176; ref/rl_common.py:87-97)."""
    D, I, FF, V = c.d, c.intermediate, c.head_ffn, c.vocab
    s: List[Tuple[str, Tuple[int, ...], str]] = [
        ("encoder.embeddings.tok_embeddings.weight", (V, D), "w"),
        ("encoder.embeddings.norm.weight", (D,), "lnw"),
    ]
    for i in range(c.n_layers):
        p = "encoder.layers.%d." % i
        if i > 0:
            s.append((p + "attn_norm.weight", (D,), "lnw"))
        s += [(p + "attn.Wqkv.weight", (3 * D, D), "w"),
              (p + "attn.Wo.weight", (D, D), "w"),
              (p + "mlp_norm.weight", (D,), "lnw"),
              (p + "mlp.Wi.weight", (2 * I, D), "w"),
              (p + "mlp.Wo.weight", (D, I), "w")]
    s += [("encoder.final_norm.weight", (D,), "lnw"), ("type_emb.weight", (3, D), "w")]
    for i in range(c.head_layers):
        p = "head.layers.%d." % i
        s += [(p + "self_attn.in_proj_weight", (3 * D, D), "w"),
              (p + "self_attn.in_proj_bias", (3 * D,), "b"),
              (p + "self_attn.out_proj.weight", (D, D), "w"),
              (p + "self_attn.out_proj.bias", (D,), "b"),
              (p + "linear1.weight", (FF, D), "w"),
              (p + "linear1.bias", (FF,), "b"),
              (p + "linear2.weight", (D, FF), "w"),
              (p + "linear2.bias", (D,), "b"),
              (p + "norm1.weight", (D,), "lnw"),
              (p + "norm1.bias", (D,), "lnb"),
              (p + "norm2.weight", (D,), "lnw"),
              (p + "norm2.bias", (D,), "lnb")]
    s += [("scorer.0.weight", (D,), "lnw"), ("scorer.0.bias", (D,), "lnb"),
          ("scorer.1.weight", (D, D), "w"), ("scorer.1.bias", (D,), "b"),
          ("scorer.3.weight", (1, D), "w"), ("scorer.3.bias", (1,), "b"),
          ("act_head.0.weight", (256, D + 4), "w"), ("act_head.0.bias", (256,), "b"),
          ("act_head.2.weight", (c.n_act, 256), "w"), ("act_head.2.bias", (c.n_act,), "b"),
          ("temperature", (3,), "temp")]
    return s


def gen_tensor(kind: str, shape, key, std: float = 0.02, ln_jitter: float = 0.0) -> np.ndarray:
    n = int(np.prod(shape))
    if kind in ("w", "b"):
        a = rng.normal(key, n, std)
    elif kind == "lnw":
        a = np.ones(n, np.float32) if ln_jitter == 0 else (1.0 + rng.normal(key, n, ln_jitter)).astype(np.float32)
    elif kind == "lnb":
        a = np.zeros(n, np.float32) if ln_jitter == 0 else rng.normal(key, n, std)
    elif kind == "temp":
        a = np.ones(n, np.float32)
    else:
        raise ValueError(kind)
    return a.reshape(shape)


def generate_weights(c: ModelConfig, seed: int = 0, std: float = 0.02, ln_jitter: float = 0.0) -> Dict[str, np.ndarray]:
    out = {}
    for idx, (name, shape, kind) in enumerate(tensor_specs(c)):
        out[name] = gen_tensor(kind, shape, rng.stream_key(seed, idx), std, ln_jitter)
    return out


_ST_DT = {"F32": (np.float32, 4), "BF16": (np.uint16, 2), "F16": (np.float16, 2)}


def to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    r = ((u >> 16) & 1) + 0x7FFF
    return ((u + r) >> 16).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def write_safetensors(path: str, specs: List[Tuple[str, Tuple[int, ...]]], produce, dtype: str = "F32"):
    """Stream tensors into a safetensors file: header first (8-byte LE length + JSON), then data.

    produce(i) returns tensor i as float32; it is converted to `dtype` on the way out."""
    _, esz = _ST_DT[dtype]
    header, off = {}, 0
    for name, shape in specs:
        nb = int(np.prod(shape)) * esz
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + nb]}
        off += nb
    header["__metadata__"] = {"format": "pt"}
    hb = json.dumps(header, separators=(",", ":")).encode()
    hb += b" " * ((8 - len(hb) % 8) % 8)
    tmp = path + ".tmp"
    with open(tmp, "wb") as f:
        f.write(struct.pack("<Q", len(hb)))
        f.write(hb)
        for i, (name, shape) in enumerate(specs):
            a = np.asarray(produce(i), dtype=np.float32).reshape(-1)
            if dtype == "F32":
                f.write(a.tobytes())
            elif dtype == "BF16":
                f.write(to_bf16_bits(a).tobytes())
            else:
                f.write(a.astype(np.float16).tobytes())
    os.replace(tmp, path)


def read_safetensors(path: str) -> Dict[str, np.ndarray]:
    """Minimal reader (float32 output) used by the oracle side; never executes file content."""
    with open(path, "rb") as f:
        hlen = struct.unpack("<Q", f.read(8))[0]
        header = json.loads(f.read(hlen))
    mm = np.memmap(path, dtype=np.uint8, mode="r", offset=8 + hlen)
    out = {}
    for name, meta in header.items():
        if name == "__metadata__":
            continue
        a, b = meta["data_offsets"]
        raw = mm[a:b]
        if meta["dtype"] == "F32":
            t = np.frombuffer(raw, dtype=np.float32)
        elif meta["dtype"] == "BF16":
            t = bf16_bits_to_f32(np.frombuffer(raw, dtype=np.uint16))
        elif meta["dtype"] == "F16":
            t = np.frombuffer(raw, dtype=np.float16).astype(np.float32)
        else:
            raise ValueError("unsupported dtype %s" % meta["dtype"])
        out[name] = t.reshape(meta["shape"])
    return out


def checkpoint_id(c: ModelConfig, seed: int, std: float, ln_jitter: float, dtype: str,
                  round_to: Optional[str] = None) -> str:
    key = [dataclasses.asdict(c), seed, std, ln_jitter, dtype] + ([round_to] if round_to else [])
    h = hashlib.sha1(json.dumps(key).encode()).hexdigest()[:10]
    return "%s-s%d-%s" % (c.name, seed, h)


def round_values(a: np.ndarray, round_to: Optional[str]) -> np.ndarray:
    """float32 values rounded to the nearest BF16 or F16 value (None: unchanged)."""
    if round_to == "BF16":
        return bf16_bits_to_f32(to_bf16_bits(a)).reshape(a.shape)
    if round_to == "F16":
        return a.astype(np.float16).astype(np.float32)
    if round_to is None:
        return a
    raise ValueError(round_to)


def write_checkpoint(out_dir: str, c: ModelConfig, seed: int = 0, std: float = 0.02, ln_jitter: float = 0.0,
                     dtype: str = "F32", round_to: Optional[str] = None) -> str:
    """Write a Laya model directory; skipped when a complete one with the same id exists.  With
    round_to ("BF16" or "F16") every value is first rounded to that type, so an F32 file can hold
    exactly the weights of a BF16 or F16 file."""
    stamp = os.path.join(out_dir, "CHECKPOINT_ID")
    cid = checkpoint_id(c, seed, std, ln_jitter, dtype, round_to)
    if os.path.exists(stamp) and open(stamp).read().strip() == cid:
        return out_dir
    os.makedirs(os.path.join(out_dir, "encoder"), exist_ok=True)
    with open(os.path.join(out_dir, "encoder", "config.json"), "w") as f:
        json.dump(encoder_config_json(c), f, indent=1)
    with open(os.path.join(out_dir, "rl_agent_config.json"), "w") as f:
        json.dump(agent_config_json(c), f, indent=1)
    specs = tensor_specs(c)
    write_safetensors(os.path.join(out_dir, "model.safetensors"), [(n, s) for n, s, _ in specs],
                      lambda i: round_values(gen_tensor(specs[i][2], specs[i][1], rng.stream_key(seed, i), std,
                                                        ln_jitter), round_to),
                      dtype)
    with open(stamp, "w") as f:
        f.write(cid + "\n")
    return out_dir


def load_checkpoint(model_dir: str) -> Tuple[ModelConfig, Dict[str, np.ndarray]]:
    """Read a Laya directory back into (ModelConfig, float32 weights)."""
    with open(os.path.join(model_dir, "encoder", "config.json")) as f:
        e = json.load(f)
    a = {}
    p = os.path.join(model_dir, "rl_agent_config.json")
    if os.path.exists(p):
        with open(p) as f:
            a = json.load(f)
    rp = e.get("rope_parameters", {})
    every = e.get("global_attn_every_n_layers", 3)
    c = ModelConfig(
        name=os.path.basename(os.path.normpath(model_dir)),
        n_layers=e["num_hidden_layers"], d=e["hidden_size"], n_heads=e["num_attention_heads"],
        intermediate=e["intermediate_size"], vocab=e["vocab_size"],
        max_len=a.get("max_len", 512), head_max_len=a.get("head_max_len", 192),
        head_layers=a.get("head_layers", 2), n_act=len(a.get("act_costs", [0])) + 1,
        local_attention=e.get("local_attention", 128), global_every=every,
        norm_eps=e.get("norm_eps", e.get("layer_norm_eps", 1e-5)),
        rope_theta_global=rp.get("full_attention", {}).get("rope_theta", 160000.0),
        rope_theta_local=rp.get("sliding_attention", {}).get("rope_theta", 10000.0),
        pad_id=e.get("pad_token_id", 50283), cls_id=e.get("cls_token_id", 50281),
        sep_id=e.get("sep_token_id", 50282), mask_id=e.get("mask_token_id", 50284))
    lt = e.get("layer_types")
    if lt is not None:
        exp = ["full_attention" if c.is_global(i) else "sliding_attention" for i in range(c.n_layers)]
        if list(lt) != exp:
            raise ValueError("layer_types other than every-%d-th global are not supported" % every)
    return c, read_safetensors(os.path.join(model_dir, "model.safetensors"))


def cache_root() -> str:
    import tempfile
    return os.environ.get("LAYA_CKPT_CACHE", os.path.join(tempfile.gettempdir(), "laya_ckpt"))


def cached_checkpoint(preset: str, seed: int = 0, std: float = 0.02, ln_jitter: float = 0.0, dtype: str = "F32",
                      round_to: Optional[str] = None) -> str:
    """Seeded checkpoint of a preset under $LAYA_CKPT_CACHE (default /tmp/laya_ckpt), written once."""
    c = PRESETS[preset]
    d = os.path.join(cache_root(), checkpoint_id(c, seed, std, ln_jitter, dtype, round_to))
    return write_checkpoint(d, c, seed=seed, std=std, ln_jitter=ln_jitter, dtype=dtype, round_to=round_to)
