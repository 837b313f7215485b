"""CPU restatement of the Laya decision model forward pass (test infrastructure only).

This module is the oracle the HIP engine is checked against.  Only tests/, the smoke check in
__graft_entry__.py and bench.py's CPU-baseline leg may import it; the engine never calls it.

It restates, in plain torch tensor algebra (float32 or float64, CPU):

  * DecisionModel.forward                  ref/rl_common.py:100-124
      - encoder (HF ModernBertModel)        transformers modeling_modernbert.py:52-71 (embeddings),
                                            :136-163 (RoPE tables), :188-219 (rotate_half),
                                            :262-301 (attention), :89-91 (GeGLU MLP),
                                            :318-333 (pre-norm layer), :434-478 (model)
      - sliding-window mask                 transformers masking_utils.py:141-151 (|i-j| <= w/2)
      - type embedding                      ref/rl_common.py:104
      - decision head layers                torch nn.TransformerEncoderLayer, norm_first=True
                                            (torch/nn/modules/transformer.py:944-950, ReLU FFN)
      - scorer, -1e4 masking, act features  ref/rl_common.py:112-123
  * the padded batch layout                 ref/rl_common.py:265-293 (collate_items)

Per-layer activations are captured under the names the reference's golden generator uses
(ref/gen_golden.py:58-71): emb, enc0..enc{L-1}, final_norm, head0..head{H-1}.

Pinning (tests/test_oracle.py): golden vectors written by the reference DecisionModel itself
(tests/golden/make_golden.py) at the tiny and full ModernBERT-large shapes; closed forms
(zero weights -> scorer bias, one-token attention = V, K=1 act features); invariants (RoPE
preserves pair norms, batch-composition and permutation invariance, padding never changes valid
rows); brute-force attention on tiny sizes.

One deliberate difference: when every question of a batch has a single marker the reference's
p.topk(2) fails on a width-1 tensor; this restatement pads p with a zero column, which gives the
engine's definition (second-best probability 0).
"""
import math
from typing import Dict, Optional

import numpy as np
import torch
import torch.nn.functional as F


def _t(w, dtype):
    return w if isinstance(w, torch.Tensor) and w.dtype == dtype else torch.as_tensor(np.require(w, requirements='W')).to(dtype)


class Weights:
    """Weights dict (numpy float32 from layamd_amd.checkpoint) as torch tensors of one dtype."""

    def __init__(self, weights: Dict[str, np.ndarray], dtype=torch.float32):
        self.dtype = dtype
        self.w = {k: _t(v, dtype) for k, v in weights.items()}

    def __getitem__(self, k):
        return self.w[k]

    def get(self, k):
        return self.w.get(k)


def rope_tables(theta: float, head_dim: int, length: int, dtype):
    """cos/sin [length, head_dim] as HF computes them (modeling_modernbert.py:136-163): inverse
    frequencies theta^(-2i/d) and their products with the positions, in float32 (or float64)."""
    ct = torch.float64 if dtype == torch.float64 else torch.float32
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).to(ct) / head_dim))
    pos = torch.arange(length, dtype=ct)
    freqs = pos[:, None] * inv_freq[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def attention(q, k, v, allowed):
    """softmax(q k^T / sqrt(d) masked) v for q,k,v [n,H,L,d]; allowed [n,1|H,L,L] bool."""
    s = torch.matmul(q, k.transpose(-1, -2)) * (q.shape[-1] ** -0.5)
    # a finite floor (as HF's SDPA masks use) keeps fully masked padding rows finite, so their
    # values never turn into NaN when multiplied by a zero probability in a valid row
    s = s.masked_fill(~allowed, torch.finfo(s.dtype).min)
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, v)


def encoder_masks(att: torch.Tensor, window: int):
    """Global mask: key j valid.  Sliding mask: key valid and |i-j| <= window//2 (inclusive)."""
    n, L = att.shape
    key_ok = att.bool()[:, None, None, :].expand(n, 1, L, L)
    i = torch.arange(L)
    band = (i[:, None] - i[None, :]).abs() <= window // 2
    return key_ok, key_ok & band[None, None]


def forward(W: Weights, cfg, input_ids, attention_mask, marker_pos, marker_mask, qtype,
            capture: Optional[Dict[str, torch.Tensor]] = None):
    """DecisionModel.forward on a right-padded batch.  Returns (logits [n,kmax], act [n,n_act])."""
    dt = W.dtype
    ids = torch.as_tensor(input_ids, dtype=torch.long)
    att = torch.as_tensor(attention_mask, dtype=torch.long)
    mpos = torch.as_tensor(marker_pos, dtype=torch.long)
    mmask = torch.as_tensor(marker_mask, dtype=torch.bool)
    qt = torch.as_tensor(qtype, dtype=torch.long)
    n, L = ids.shape
    D, H, HD, eps = cfg.d, cfg.n_heads, cfg.head_dim, cfg.norm_eps
    cap = capture if capture is not None else {}

    def ln(x, w, b=None):
        return F.layer_norm(x, (D,), w, b, eps)

    x = ln(W["encoder.embeddings.tok_embeddings.weight"][ids], W["encoder.embeddings.norm.weight"])
    cap["emb"] = x
    cos_g, sin_g = rope_tables(cfg.rope_theta_global, HD, L, dt)
    cos_l, sin_l = rope_tables(cfg.rope_theta_local, HD, L, dt)
    m_glob, m_slide = encoder_masks(att, cfg.local_attention)
    for i in range(cfg.n_layers):
        p = "encoder.layers.%d." % i
        glob = cfg.is_global(i)
        # layer 0 has no attn_norm in HF ModernBERT (Identity); the reference engine applies one
        # when a checkpoint carries it (src/engine.hip:154-155, 415)
        h = ln(x, W[p + "attn_norm.weight"]) if (i > 0 or W.get(p + "attn_norm.weight") is not None) else x
        qkv = (h @ W[p + "attn.Wqkv.weight"].T).view(n, L, 3, H, HD)
        q, k, v = (qkv[:, :, j].transpose(1, 2) for j in range(3))
        c, s = (cos_g, sin_g) if glob else (cos_l, sin_l)
        q = q * c + rotate_half(q) * s
        k = k * c + rotate_half(k) * s
        o = attention(q, k, v, m_glob if glob else m_slide).transpose(1, 2).reshape(n, L, D)
        x = x + o @ W[p + "attn.Wo.weight"].T
        h = ln(x, W[p + "mlp_norm.weight"])
        a, g = (h @ W[p + "mlp.Wi.weight"].T).chunk(2, dim=-1)
        x = x + (F.gelu(a) * g) @ W[p + "mlp.Wo.weight"].T
        cap["enc%d" % i] = x
    x = ln(x, W["encoder.final_norm.weight"])
    cap["final_norm"] = x
    x = x + W["type_emb.weight"][qt][:, None, :]
    key_ok = att.bool()[:, None, None, :].expand(n, 1, L, L)
    for i in range(cfg.head_layers):
        p = "head.layers.%d." % i
        h = ln(x, W[p + "norm1.weight"], W[p + "norm1.bias"])
        qkv = h @ W[p + "self_attn.in_proj_weight"].T + W[p + "self_attn.in_proj_bias"]
        q, k, v = (t.view(n, L, H, HD).transpose(1, 2) for t in qkv.chunk(3, dim=-1))
        o = attention(q, k, v, key_ok).transpose(1, 2).reshape(n, L, D)
        x = x + o @ W[p + "self_attn.out_proj.weight"].T + W[p + "self_attn.out_proj.bias"]
        h = ln(x, W[p + "norm2.weight"], W[p + "norm2.bias"])
        f = torch.relu(h @ W[p + "linear1.weight"].T + W[p + "linear1.bias"])
        x = x + f @ W[p + "linear2.weight"].T + W[p + "linear2.bias"]
        cap["head%d" % i] = x
    m = torch.gather(x, 1, mpos.clamp(min=0)[:, :, None].expand(-1, -1, D))
    h = ln(m, W["scorer.0.weight"], W["scorer.0.bias"])
    h = F.gelu(h @ W["scorer.1.weight"].T + W["scorer.1.bias"])
    logits = (h @ W["scorer.3.weight"].T + W["scorer.3.bias"]).squeeze(-1)
    logits = logits.masked_fill(~mmask, -1e4)
    pr = torch.softmax(logits, -1)
    kk = mmask.sum(-1).clamp(min=2).to(dt)
    ent = -(pr * torch.log(pr.clamp_min(1e-9))).sum(-1) / torch.log(kk)
    if pr.shape[-1] < 2:
        pr = torch.cat([pr, torch.zeros_like(pr)], -1)
    top2 = pr.topk(2, -1).values
    feats = torch.stack([top2[:, 0], top2[:, 0] - top2[:, 1], ent, kk / 255.0], -1)
    z = torch.cat([x[:, 0], feats], -1)
    hid = F.gelu(z @ W["act_head.0.weight"].T + W["act_head.0.bias"])
    act = hid @ W["act_head.2.weight"].T + W["act_head.2.bias"]
    return logits, act


@torch.no_grad()
def run_batch(W: Weights, cfg, batch, capture=None):
    """Oracle outputs for a layamd_amd.workloads.Batch, unpadded to the ABI's output layout:
    logits concatenated per question (sum(nmark)), act [B, n_act]."""
    ids, att, mpos, mmask, qt = batch.padded()
    logits, act = forward(W, cfg, ids, att, mpos, mmask, qt, capture)
    flat = np.concatenate([logits[i, :len(batch.markers[i])].double().numpy() for i in range(batch.B)])
    return flat, act.double().numpy()


@torch.no_grad()
def run_per_question(W: Weights, cfg, batch, capture_rows=False):
    """Runs each question alone (no padding): the engine's packing semantics.  With capture_rows,
    also returns per-question dicts of captured activations [len, D]."""
    logits, acts, caps = [], [], []
    for i in range(batch.B):
        sub = batch.subset([i])
        cap = {} if capture_rows else None
        lo, ac = run_batch(W, cfg, sub, cap)
        logits.append(lo)
        acts.append(ac[0])
        if capture_rows:
            caps.append({k: v[0].double().numpy() for k, v in cap.items()})
    out = (np.concatenate(logits), np.stack(acts))
    return out + (caps,) if capture_rows else out

