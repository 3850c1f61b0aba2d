"""Oracle: torch-CPU float32 port of the block, the timed CPU baseline of bench.py.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). The reference's own CPU path (the MLX CPU
backend) cannot run here: MLX is not installed, the reference needs Python >= 3.13, and its
sources never travel to the GPU box. This port follows the same algorithm as the reference's
qwen35_moe (src/quanta/qwen35/moe.py:154-202) in torch on the host cores:
  fp32 router + softmax/sigmoid(+bias, groups) + top-k + renorm   (moe.py:36-56)
  stable permute by expert                                          (modeling/moe.py:81-85)
  per expert: dequant s*q+b of its int4 g64 stack, matmul, SwiGLU   (moe.py:85-124)
  per expert down projection, fp32 weighted combine                 (moe.py:191)
  bf16 shared expert with the sigmoid gate, bf16 output             (moe.py:145-151,201-202)
  (an int8 shared expert dequantized to bf16 first, as the loader does: artifact.py:105-115)
Only the experts a batch routes to are dequantized, as gather_qmm only reads those.
"""

from __future__ import annotations

import torch


def _dequant(packed: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """[rows, K/8] int32 words + [rows, K/64] bf16 -> float32 [rows, K]."""
    rows, nw = packed.shape
    shifts = torch.arange(0, 32, 4, dtype=torch.int32)
    q = ((packed[:, :, None] >> shifts) & 0xF).reshape(rows, nw * 8).to(torch.float32)
    s = scale.to(torch.float32).repeat_interleave(64, dim=1)
    b = bias.to(torch.float32).repeat_interleave(64, dim=1)
    return torch.addcmul(b, s, q)


def _dequant8(t: dict) -> torch.Tensor:
    """int8 triplet {packed [rows, K/4] int32, scale/bias [rows, K/g] bf16} -> bf16 [rows, K],
    bf16(fp32(s*q + b)) (s*q is exact in fp32)."""
    packed = t["packed"]
    rows, nw = packed.shape
    shifts = torch.arange(0, 32, 8, dtype=torch.int32)
    q = ((packed[:, :, None] >> shifts) & 0xFF).reshape(rows, nw * 4).to(torch.float32)
    g = int(t.get("group_size", 64))
    s = t["scale"].to(torch.float32).repeat_interleave(g, dim=1)
    b = t["bias"].to(torch.float32).repeat_interleave(g, dim=1)
    return torch.addcmul(b, s, q).to(torch.bfloat16)


def load_shared(p: dict) -> dict:
    """The layer as the reference's loader hands it to the block: an int8 shared expert (the
    bake's format, src/quanta/qwen35/bake.py:150-151) dequantized to bf16 once
    (src/quanta/qwen35/artifact.py:105-115, 171-184); other entries unchanged."""
    q = dict(p)
    for key in ("shared_gate_proj", "shared_up_proj", "shared_down_proj"):
        if isinstance(q.get(key), dict):
            q[key] = _dequant8(q[key])
    return q


def route(x: torch.Tensor, gate: torch.Tensor, cfg, k: int, bias=None):
    logits = x.to(torch.float32) @ gate.to(torch.float32).T
    if cfg.scoring_func == "softmax":
        scores = torch.softmax(logits, dim=-1)
        choice = scores if bias is None else scores + bias
    else:
        scores = torch.sigmoid(logits)
        choice = scores + (bias if bias is not None else 0.0)
    if cfg.n_group > 1:
        n, e = choice.shape
        g = choice.view(n, cfg.n_group, e // cfg.n_group).topk(2, dim=-1).values.sum(-1)
        keep = torch.zeros_like(g).scatter_(1, g.topk(cfg.topk_group, dim=-1).indices, 1.0)
        mask = keep.repeat_interleave(e // cfg.n_group, dim=1).bool()
        choice = choice.masked_fill(~mask, float("-inf"))
    idx = choice.topk(k, dim=-1).indices
    w = scores.gather(1, idx)
    # a sigmoid + correction-bias router (MoEGate) keeps a single expert's score
    # (src/quanta/modeling/moe.py:41); qwen35_route renormalises it too (moe.py:53-54)
    moegate = cfg.scoring_func == "sigmoid" and bias is not None
    if cfg.norm_topk_prob and (k > 1 or not moegate):
        w = w / (w.sum(-1, keepdim=True) + 1e-20)
    return idx, w * cfg.routed_scaling_factor


def moe_forward(x: torch.Tensor, p: dict, cfg, k: int | None = None) -> torch.Tensor:
    """x [N, H] bf16 (CPU) -> y [N, H] bf16. `p` uses the reference keys with packed triplets."""
    k = cfg.num_experts_per_tok if k is None else k
    n, H = x.shape
    I = cfg.moe_intermediate_size
    bias = p.get("e_score_correction_bias")
    idx, w = route(x, p["gate"], cfg, k, None if bias is None else bias.to(torch.float32))
    exp = idx.reshape(-1)
    order = torch.argsort(exp, stable=True)
    tok = order // k
    exp_s = exp[order]
    uniq, counts = torch.unique_consecutive(exp_s, return_counts=True)
    xf = x.to(torch.float32)
    gu, dn = p["experts_gate_up"], p["experts_down"]
    d_sorted = torch.empty(n * k, H, dtype=torch.float32)
    start = 0
    for e, c in zip(uniq.tolist(), counts.tolist()):
        rows = tok[start:start + c]
        wg = _dequant(gu["packed"][e], gu["scale"][e], gu["bias"][e])
        g_u = (xf[rows] @ wg.T).to(torch.bfloat16).to(torch.float32)
        h = (torch.nn.functional.silu(g_u[:, :I]) * g_u[:, I:]).to(torch.bfloat16).to(torch.float32)
        wd = _dequant(dn["packed"][e], dn["scale"][e], dn["bias"][e])
        d_sorted[start:start + c] = (h @ wd.T).to(torch.bfloat16).to(torch.float32)
        start += c
    d = torch.empty_like(d_sorted)
    d[order] = d_sorted
    y = (d.view(n, k, H) * w[:, :, None]).sum(1)
    if p.get("shared_gate_proj") is not None:
        p = load_shared(p)
        xb = x.to(torch.bfloat16)
        hs = torch.nn.functional.silu(xb @ p["shared_gate_proj"].T) * (xb @ p["shared_up_proj"].T)
        out = (hs @ p["shared_down_proj"].T).to(torch.float32)
        if p.get("shared_expert_gate") is not None:
            out = out * torch.sigmoid(xf @ p["shared_expert_gate"].to(torch.float32).T)
        y = y + out
    return y.to(torch.bfloat16)
