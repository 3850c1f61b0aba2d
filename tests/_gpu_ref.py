"""Test helper: the oracle's block arithmetic restated in float64 torch on the GPU, so full-size
parity can compare every token (the numpy oracle finishes only a few tokens of c2/c4 in seconds).

It follows oracle/moe.py step for step, with the same rounding points:
  weights   s*q + b exact in float64 (oracle/quant.py dequant_exact, int4 g64 LSB-first words);
  gate_up   bf16(x . W_gu^T)                         (oracle gather_qmm, rounded output)
  h         bf16(silu(g) * u) on the bf16 g, u       (oracle swiglu / glu)
  down      bf16(h . W_dn^T)                         (oracle gather_qmm)
  combine   sum_s w[t,s] * d[t,s] in float64         (oracle combine)
  shared    bf16 chain times sigmoid(x . gate)       (oracle shared_expert)
and returns the unrounded float64 y, as the oracle's `y_exact`. bf16 rounding goes through
float32 first, as oracle/quant.py round_bf16 does. It is test infrastructure only, and every test
that uses it checks it against the oracle on sampled tokens (pin_to_oracle) before trusting it.
"""

from __future__ import annotations

import numpy as np
import torch


def round_bf16(t: torch.Tensor) -> torch.Tensor:
    """float64 -> float32 (RNE) -> bf16 (RNE) -> float64, as oracle.quant.round_bf16."""
    return t.to(torch.float32).to(torch.bfloat16).to(torch.float64)


def dequant_exact(packed: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor,
                  group_size: int = 64) -> torch.Tensor:
    """[rows, K/8] int4 words + [rows, K/g] bf16 -> float64 [rows, K] = s*q + b (code 8w+j in
    nibble j of word w)."""
    rows, nw = packed.shape
    shifts = torch.arange(0, 32, 4, dtype=torch.int32, device=packed.device)
    q = ((packed.to(torch.int32)[:, :, None] >> shifts) & 0xF).reshape(rows, nw * 8)
    s = scale.to(torch.float64).repeat_interleave(group_size, dim=1)
    b = bias.to(torch.float64).repeat_interleave(group_size, dim=1)
    return s * q.to(torch.float64) + b


def shared_weight(v) -> torch.Tensor:
    """A shared-expert projection in float64: bf16 as given, or an int8 triplet dequantized to
    bf16 (oracle.moe.shared_weight: fp32(s*q + b) rounded to bf16; s*q is exact in float64 and in
    float32, so rounding the exact float64 sum to float32 then bf16 gives the same bits)."""
    if not isinstance(v, dict):
        return v.to(torch.float64)
    pk, sc, bi = v["packed"], v["scale"], v["bias"]
    rows, nw = pk.shape
    shifts = torch.arange(0, 32, 8, dtype=torch.int32, device=pk.device)
    q = ((pk.to(torch.int32)[:, :, None] >> shifts) & 0xFF).reshape(rows, nw * 4)
    gs = int(v.get("group_size", 64))
    s = sc.to(torch.float64).repeat_interleave(gs, dim=1)
    b = bi.to(torch.float64).repeat_interleave(gs, dim=1)
    return round_bf16(s * q.to(torch.float64) + b)


def _silu(v: torch.Tensor) -> torch.Tensor:
    return v / (1.0 + torch.exp(-v))


def block_reference(p: dict, cfg, x: torch.Tensor, idx: np.ndarray, w: np.ndarray) -> torch.Tensor:
    """float64 y_exact [N, H] of the block for bf16 x [N, H] on the GPU, given the routing
    (idx [N, k] expert ids, w [N, k] weights, float64)."""
    act = str(getattr(cfg, "hidden_act", "silu"))
    if act != "silu" or float(getattr(cfg, "swiglu_limit", 0.0) or 0.0) > 0:
        raise NotImplementedError("block_reference restates the plain SwiGLU only")
    dev = x.device
    N, H = x.shape
    I = cfg.moe_intermediate_size
    gu, dn = p["experts_gate_up"], p["experts_down"]
    gs_gu, gs_dn = int(gu.get("group_size", 64)), int(dn.get("group_size", 64))
    assert int(gu.get("bits", 4)) == 4 and int(dn.get("bits", 4)) == 4
    x64 = x.to(torch.float64)
    idx_t = torch.as_tensor(idx, dtype=torch.int64, device=dev)
    w_t = torch.as_tensor(w, dtype=torch.float64, device=dev)
    k = idx_t.shape[1]
    flat = idx_t.reshape(-1)
    tok = torch.arange(N, device=dev).repeat_interleave(k)
    d = torch.empty(N * k, H, dtype=torch.float64, device=dev)
    for e in torch.unique(flat).tolist():
        sel = (flat == e).nonzero().reshape(-1)
        wg = dequant_exact(gu["packed"][e], gu["scale"][e], gu["bias"][e], gs_gu)
        g_u = round_bf16(x64[tok[sel]] @ wg.T)
        del wg
        h = round_bf16(_silu(g_u[:, :I]) * g_u[:, I:])
        wd = dequant_exact(dn["packed"][e], dn["scale"][e], dn["bias"][e], gs_dn)
        d[sel] = round_bf16(h @ wd.T)
        del wd
    y = (d.reshape(N, k, H) * w_t[:, :, None]).sum(dim=1)
    if p.get("shared_gate_proj") is not None:
        wg, wu, wd = (shared_weight(p[k]) for k in ("shared_gate_proj", "shared_up_proj",
                                                    "shared_down_proj"))
        g = round_bf16(x64 @ wg.T)
        u = round_bf16(x64 @ wu.T)
        hs = round_bf16(_silu(g) * u)
        out = round_bf16(hs @ wd.T)
        if p.get("shared_expert_gate") is not None:
            sg = torch.sigmoid(x64 @ p["shared_expert_gate"].to(torch.float64).reshape(-1))
            out = out * sg[:, None]
        y = y + out
    return y


def pin_to_oracle(y_ref: np.ndarray, want: np.ndarray, what: str) -> None:
    """The GPU restatement agrees with the numpy oracle on the sampled tokens: both evaluate the
    same float64 expressions with the same bf16 rounding points, so they differ only where a
    float64 summation-order difference moves a value across a bf16 rounding boundary (a few
    elements at most). A dropped term, a wrong index or a transposed operand fails this."""
    d = np.abs(y_ref - want)
    scale = max(1.0, float(np.max(np.abs(want))))
    rel = float(np.linalg.norm(y_ref - want) / max(np.linalg.norm(want), 1e-30))
    frac_exact = float(np.mean(d <= 1e-12 * scale))
    print(f"[pin] {what}: GPU float64 reference vs oracle: max {float(d.max()):.3e}, rel_l2 "
          f"{rel:.3e}, {100 * frac_exact:.2f}% of elements equal", flush=True)
    assert rel <= 1e-5 and float(d.max()) <= 1e-3 * scale and frac_exact >= 0.99, what
