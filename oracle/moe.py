"""Oracle: float64 restatement of the quantized sparse-MoE block.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Arrays holding bf16 data are float64 arrays whose values are exactly representable in bf16.
Every function cites the reference lines it restates. The bf16 materialisation points of the
reference's dtype flow are kept (`round_bf16` where MLX produces a bf16 array):
  gu = bf16(x . deq(W_gu)^T)       (gather_qmm output follows the bf16 scale dtype)
  h  = bf16(silu(g) * u)           (bf16 elementwise ops; here one rounding)
  d  = bf16(h . deq(W_d)^T)
  routed = sum_s f32(d) * w        (float32 combine; here float64)
  shared = bf16 SwiGLU chain, times sigmoid(x_f32 . g_f32)
  y = bf16(routed + shared)
The GPU path keeps float32 accumulators at the same points, so results agree to bf16
rounding, which the BASELINE tolerances (max-abs 2e-2, rel-L2 5e-3) bound.
"""

from __future__ import annotations

import numpy as np

from oracle.quant import (bf16_bits_to_f32, dequant_bf16_bits, dequant_exact, dequant_float,
                          round_bf16)


def _silu(v: np.ndarray) -> np.ndarray:
    """silu(x) = x * sigmoid(x) (`src/quanta/qwen35/moe.py:32-33`)."""
    return v / (1.0 + np.exp(-v))


def _sigmoid(v: np.ndarray) -> np.ndarray:
    return 1.0 / (1.0 + np.exp(-v))


# ----------------------------------------------------------------------------- layer norm


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """The decoder layer's post_attention_layernorm in front of the block
    (`src/quanta/qwen35/model.py:104-105`): w * (x * rsqrt(mean(x^2) + eps)) over the last dim, as
    the reference restates its norms (`src/quanta/qwen35/attention.py:113-117`,
    `src/quanta/qwen35/mtp.py:40-42`: fp32 math, one rounding to the input dtype). Here in
    float64 and unrounded; `w` is nn.RMSNorm's resident weight (checkpoint weight + 1,
    `src/quanta/qwen35/runtime.py:57-63`). MLX's own reduction order inside mx.fast.rms_norm is
    parity unpinned at the MLX boundary (a last-bit difference in bf16 at most)."""
    r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return w * (x * r)


def residual_add(x: np.ndarray, block_out_bf16: np.ndarray) -> np.ndarray:
    """x + mlp(...) of the decoder layer (`src/quanta/qwen35/model.py:104-105`): both bf16, the
    sum rounded once to bf16 (an fp32 add of two bf16 values then RNE)."""
    return round_bf16(x + block_out_bf16)


# ----------------------------------------------------------------------------- routing


def topk_canonical(choice: np.ndarray, k: int) -> np.ndarray:
    """Top-k indices per row in this build's canonical order: value descending, id ascending
    on ties. `mx.argpartition(-s, k-1)[:, :k]` (`src/quanta/qwen35/moe.py:52`) returns the same
    SET in an unspecified order (parity unpinned at the MLX boundary for the order); the
    reference's own routing gate compares sets (`parity/glm_moe_test.py:98-102`)."""
    n, e = choice.shape
    ids = np.broadcast_to(np.arange(e), choice.shape)
    order = np.lexsort((ids, -choice), axis=-1)
    return order[:, :k]


def group_limit(choice: np.ndarray, n_group: int, topk_group: int) -> np.ndarray:
    """Group-limited selection mask (DeepSeek-V3 `noaux_tc`).

    Follows transformers 5.15.0 `models/deepseek_v3/modeling_deepseek_v3.py:149-164` (the
    reference asserts n_group == 1, `src/quanta/modeling/moe.py:34`): group score = sum of the
    two largest choice values in each of the n_group contiguous expert groups; keep the
    topk_group best groups (canonical order on ties); every expert outside them gets -inf.
    """
    n, e = choice.shape
    g = choice.reshape(n, n_group, e // n_group)
    top2 = np.sort(g, axis=-1)[..., -2:].sum(axis=-1)
    gidx = topk_canonical(top2, topk_group)
    keep = np.zeros((n, n_group), dtype=bool)
    np.put_along_axis(keep, gidx, True, axis=-1)
    mask = np.repeat(keep, e // n_group, axis=-1)
    return np.where(mask, choice, -np.inf)


def route(x: np.ndarray, wr: np.ndarray, *, k: int, scoring: str = "softmax",
          norm_topk: bool = True, bias: np.ndarray | None = None, n_group: int = 1,
          topk_group: int = 1, scale: float = 1.0, norm_single: bool = True):
    """Router -> (idx [N,k] int32, w [N,k] float64, logits, scores).

    softmax (`src/quanta/qwen35/moe.py:47-55`): logits = x . Wr^T in float (here float64),
    scores = softmax(logits); top-k of scores; w = scores[idx]; if norm_topk,
    w /= sum(w) + 1e-20.
    sigmoid + correction bias (`src/quanta/modeling/moe.py:36-43`, `src/quanta/glm/moe.py:48-55`):
    scores = sigmoid(logits); select by scores + bias (optionally group-limited); weights are
    the bias-free scores, renormalised, then times `scale` (routed_scaling_factor).
    sqrtsoftplus (DeepSeek-V4, `src/quanta/dsv4/moe.py:37-57`): scores = sqrt(log(1 + e^logits)),
    then as sigmoid.
    Renormalisation at k = 1: qwen35_route divides a single weight by itself too
    (`src/quanta/qwen35/moe.py:53-54`, norm_single=True); the MoEGate routers keep a single
    expert's score (`topk > 1 and norm_topk_prob`, `src/quanta/modeling/moe.py:41`,
    `src/quanta/glm/moe.py:53`, norm_single=False).
    """
    logits = x.astype(np.float64) @ wr.astype(np.float64).T
    if scoring == "softmax":
        m = logits.max(axis=-1, keepdims=True)
        p = np.exp(logits - m)
        scores = p / p.sum(axis=-1, keepdims=True)
    elif scoring == "sigmoid":
        scores = _sigmoid(logits)
    elif scoring == "sqrtsoftplus":
        scores = np.sqrt(np.logaddexp(0.0, logits))
    else:
        raise ValueError(scoring)
    choice = scores + bias[None, :].astype(np.float64) if bias is not None else scores.copy()
    if n_group > 1:
        choice = group_limit(choice, n_group, topk_group)
    idx = topk_canonical(choice, k)
    w = np.take_along_axis(scores, idx, axis=-1)
    if norm_topk and (k > 1 or norm_single):
        w = w / (w.sum(axis=-1, keepdims=True) + 1e-20)
    w = w * scale
    return idx.astype(np.int32), w, logits, scores, choice


def route_margin(choice: np.ndarray, k: int) -> np.ndarray:
    """Per-row gap between the k-th and (k+1)-th largest choice values (inf when k == E).
    Rows whose gap is below the float32 evaluation error of the logits can legitimately
    select a different k-th expert on the GPU; tests report and exclude them."""
    s = -np.sort(-choice, axis=-1)
    if k >= choice.shape[1]:
        return np.full(choice.shape[0], np.inf)
    return s[:, k - 1] - s[:, k]


# ----------------------------------------------------------------------------- permute


def permute(idx: np.ndarray, n_experts: int):
    """Stable sort of the flattened (token, slot) list by expert id.

    Restates `order = argsort(exp)` / `inv = argsort(order)` (`src/quanta/modeling/moe.py:81-85`,
    `src/quanta/dsv4/moe.py:68,107-110`; MLX argsort is stable per `dsv4/moe.py:68`).
    Returns counts[E], offsets[E+1], order[mc] (sorted position -> slot), inv[mc]
    (slot -> sorted position).
    """
    exp = np.asarray(idx).reshape(-1).astype(np.int64)
    order = np.argsort(exp, kind="stable")
    inv = np.empty_like(order)
    inv[order] = np.arange(order.size)
    counts = np.bincount(exp, minlength=n_experts)
    offsets = np.concatenate([[0], np.cumsum(counts)])
    return (counts.astype(np.int32), offsets.astype(np.int32), order.astype(np.int32),
            inv.astype(np.int32))


# ----------------------------------------------------------------------------- expert math


def gather_qmm(xrows: np.ndarray, experts: np.ndarray, packed: np.ndarray, scale: np.ndarray,
               bias: np.ndarray, in_features: int, *, round_out: bool = True,
               round_weights: bool = False, group_size: int = 64, bits: int = 4) -> np.ndarray:
    """y[m] = x[m] . (s*q + b)[experts[m]]^T per row, float64, rounded to bf16.

    Restates `mx.gather_qmm(x, packed, scale, bias, rhs_indices=exp, transpose=True)`
    (`src/quanta/qwen35/moe.py:117-123`): the weight stack is [E, out, in] affine int4 with
    bf16 scale/bias per 64 along `in`; output dtype follows the bf16 scale dtype.
    Default: the exact affine weight (the fused matrix-vector form, sum x*(s*q+b) with float
    accumulation). `round_weights=True` is the large-batch form that first dequantizes each
    weight to bf16 and then multiplies (the tile-dequant matmul form); both are bf16-accurate
    and differ by the bf16 rounding of the weights (parity unpinned at the MLX boundary as to
    which form MLX picks for a given batch size).
    """
    experts = np.asarray(experts).reshape(-1)
    out = np.zeros((xrows.shape[0], packed.shape[1]), dtype=np.float64)
    for e in np.unique(experts):
        sel = experts == e
        w = dequant_exact(packed[e], scale[e], bias[e], in_features, bits=bits,
                          group_size=group_size)
        if round_weights:
            w = round_bf16(w)
        out[sel] = xrows[sel].astype(np.float64) @ w.T
    return round_bf16(out) if round_out else out


def gather_mm(xrows: np.ndarray, experts: np.ndarray, stack: np.ndarray) -> np.ndarray:
    """bf16 sibling (`mx.gather_mm`, `src/quanta/qwen35/moe.py:66-82`): y[m] = x[m] . W[e]^T."""
    experts = np.asarray(experts).reshape(-1)
    out = np.zeros((xrows.shape[0], stack.shape[1]), dtype=np.float64)
    for e in np.unique(experts):
        sel = experts == e
        out[sel] = xrows[sel].astype(np.float64) @ stack[e].astype(np.float64).T
    return round_bf16(out)


def glu(g: np.ndarray, u: np.ndarray, act: str = "silu", alpha: float = 1.702,
        limit: float = 0.0) -> np.ndarray:
    """The gated activation on bf16 gate/up values, unrounded:
      "silu"       silu(g) * u (`src/quanta/qwen35/moe.py:59-63`), clamped when limit > 0 as
                   g = min(g, L), u = clip(u, -L, L) (`src/quanta/dsv4/moe.py:74-77`);
      "swigluoai"  g = min(g, L), u = clip(u, -L, L), (u + 1) * g * sigmoid(alpha * g)
                   (`src/quanta/minimax/model_m3.py:112-128`, transformers GptOssExperts)."""
    if limit > 0:
        g = np.minimum(g, limit)
        u = np.clip(u, -limit, limit)
    if act == "swigluoai":
        return (u + 1.0) * (g * _sigmoid(alpha * g))
    if act != "silu":
        raise ValueError(f"unknown act {act!r}")
    return _silu(g) * u


def swiglu(gu: np.ndarray, inter: int, act: str = "silu", alpha: float = 1.702,
           limit: float = 0.0) -> np.ndarray:
    """SwiGLU on the fused gate|up activation (`src/quanta/qwen35/moe.py:59-63`):
    gate = first `inter` columns, up = the rest; h = bf16(glu(g, u)) (the MiniMax M3 split is
    the same, `src/quanta/minimax/model_m3.py:407-408`)."""
    g = gu[:, :inter]
    u = gu[:, inter:]
    return round_bf16(glu(g, u, act, alpha, limit))


def awq_divide(x: np.ndarray, s: np.ndarray) -> np.ndarray:
    """bf16(fp32(x / s)) for bf16-valued x and s: the fp32 division rounded once to bf16 by the
    matmul's bf16 input (`src/quanta/dsv4/moe.py:112-137`). The float64 quotient of two bf16
    values rounds to fp32 as the correctly rounded fp32 division does (an 8-bit by 8-bit quotient
    is never an fp32 rounding midpoint), so round_bf16's fp32 step is that division."""
    return round_bf16(x / s)


def awq_expert_rows(xrows: np.ndarray, exp: np.ndarray, p: dict, inter: int, hdim: int, *,
                    act: str = "silu", alpha: float = 1.702, limit: float = 0.0,
                    round_weights: bool = False, group_size: int = 64, bits: int = 4):
    """DeepSeek-V4's packed routed SwiGLU with activation-aware scales
    (`src/quanta/dsv4/moe.py:112-137`): g = qmm(bf16(x / s_w1[e])), u = qmm(bf16(x / s_w3[e])),
    both bf16; h = bf16(glu(g, u) / s_w2[e]) with the gated activation unrounded. The fused
    gate_up stack holds w1 in rows [0, I) and w3 in rows [I, 2I). Returns (gu [M, 2I], h)."""
    exp = np.asarray(exp).reshape(-1)
    s_gu, s_dn = p["gu_awq"], p["dn_awq"]
    outs = []
    for half in (0, 1):
        rows = slice(half * inter, (half + 1) * inter)
        xs = awq_divide(xrows, s_gu[exp, half])
        outs.append(gather_qmm(xs, exp, p["gu_packed"][:, rows], p["gu_scale"][:, rows],
                               p["gu_bias"][:, rows], hdim, round_weights=round_weights,
                               group_size=group_size, bits=bits))
    g, u = outs
    h = awq_divide(glu(g, u, act, alpha, limit), s_dn[exp])
    return np.concatenate([g, u], axis=1), h


def mixed_proj(xrows: np.ndarray, exp: np.ndarray, m: dict, proj: str, in_features: int) -> np.ndarray:
    """One projection over routed rows whose experts have per-(expert, projection) widths
    (`src/quanta/modeling/quantized.py:53-66`): row r uses expert e = exp[r]'s width
    b = pbits[proj][e] and its slot pslot[proj][e] in the width-b stack; y = bf16(x . W^T).
    `m`: {"stacks": {proj: {bits: (packed, scale, bias[, group_size])}}, "pbits": {proj: [E]},
    "pslot": {proj: [E]}, "group_size": g}; a stack's own group size, when given, overrides g."""
    exp = np.asarray(exp).reshape(-1)
    pb = np.asarray(m["pbits"][proj])[exp]
    ps = np.asarray(m["pslot"][proj])[exp]
    out = None
    for bits, st in sorted(m["stacks"][proj].items()):
        packed, scale, bias = st[:3]
        gs = st[3] if len(st) > 3 else m["group_size"]
        sel = pb == bits
        if not sel.any():
            continue
        o = gather_qmm(xrows[sel], ps[sel], packed, scale, bias, in_features,
                       group_size=gs, bits=bits)
        if out is None:
            out = np.zeros((exp.size, o.shape[1]))
        out[sel] = o
    return out


def combine(d: np.ndarray, w: np.ndarray) -> np.ndarray:
    """routed[t] = sum_s d[t*k+s] * w[t,s] (`src/quanta/qwen35/moe.py:191`), float64."""
    n, k = w.shape
    return (d.reshape(n, k, -1) * w[:, :, None]).sum(axis=1)


def shared_weight(v) -> np.ndarray:
    """A shared-expert projection as the reference's loader hands it to the block: bf16 values as
    given, or the bake's int8 triplet (`src/quanta/qwen35/bake.py:106-110, 150-151`: a dict
    {packed uint32 [out, in/4], scale, bias: bf16 bits [out, in/g], group_size, bits: 8})
    dequantized to bf16 (`src/quanta/qwen35/artifact.py:105-115`, read by `moe()` at
    :171-184), under the dequant convention of oracle.quant.dequant_bf16_bits."""
    if not isinstance(v, dict):
        return v
    if int(v.get("bits", 8)) != 8:
        raise ValueError("shared expert triplets are int8")
    packed = np.asarray(v["packed"])
    in_features = packed.shape[-1] * 4
    bits = dequant_bf16_bits(packed, np.asarray(v["scale"]), np.asarray(v["bias"]), in_features,
                             bits=8, group_size=int(v.get("group_size", 64)))
    return bf16_bits_to_f32(bits).astype(np.float64)


def shared_expert(x: np.ndarray, wg: np.ndarray, wu: np.ndarray, wd: np.ndarray,
                  gate: np.ndarray | None, act: str = "silu", alpha: float = 1.702,
                  limit: float = 0.0):
    """Shared SwiGLU expert (`src/quanta/qwen35/moe.py:145-151`): bf16 chain
    out = bf16(bf16(silu(bf16(x Wg^T)) * bf16(x Wu^T)) Wd^T), then times
    sg = sigmoid(x_f32 . g_f32) when a gate is given (Qwen); DeepSeek/GLM shared experts are
    ungated (`src/quanta/glm/moe.py:83-84`). Returns (scaled float64 out, out bf16, sg)."""
    x = x.astype(np.float64)
    g = round_bf16(x @ wg.astype(np.float64).T)
    u = round_bf16(x @ wu.astype(np.float64).T)
    h = round_bf16(glu(g, u, act, alpha, limit))
    out = round_bf16(h @ wd.astype(np.float64).T)
    if gate is None:
        return out, out, None
    sg = _sigmoid(x @ gate.astype(np.float64).reshape(-1))
    return out * sg[:, None], out, sg


# ----------------------------------------------------------------------------- the block


def moe_forward(x: np.ndarray, p: dict, *, k: int, inter: int, scoring: str = "softmax",
                norm_topk: bool = True, n_group: int = 1, topk_group: int = 1,
                scale: float = 1.0, round_weights: bool = False, act: str = "silu",
                alpha: float = 1.702, limit: float = 0.0, group_size: int = 64, bits: int = 4,
                down_bits: int | None = None, norm_single: bool = True):
    """Whole block y = bf16(routed + shared) for x [N, H] (`src/quanta/qwen35/moe.py:154-202`).

    `p` keys (numpy, bf16 data as float64 values, int4 stacks as uint32/uint16 bit arrays):
      gate [E,H]; gu_packed [E,2I,H/8], gu_scale/gu_bias [E,2I,H/64] (bf16 bits);
      dn_packed [E,H,I/8], dn_scale/dn_bias [E,H,I/64]; optional e_score_correction_bias [E];
      optional shared_gate_proj [Is,H], shared_up_proj [Is,H], shared_down_proj [H,Is] (bf16
      values, or int8 triplets, see shared_weight), shared_expert_gate [1,H]; optional gu_awq [E,2,H] and dn_awq [E,I] (bf16 values): the
      activation-aware scales of DeepSeek-V4's packed experts (see awq_expert_rows); or, in
      place of the gu_/dn_ stacks, "mixed" (per-(expert, projection) widths, see mixed_proj).
    Returns (y bf16-valued float64 [N,H], dict of intermediates).
    """
    n, hdim = x.shape
    idx, w, logits, scores, choice = route(
        x, p["gate"], k=k, scoring=scoring, norm_topk=norm_topk,
        bias=p.get("e_score_correction_bias"), n_group=n_group, topk_group=topk_group,
        scale=scale, norm_single=norm_single)
    exp = idx.reshape(-1)
    tok = np.repeat(np.arange(n), k)
    if p.get("mixed") is not None:
        # Kimi's QuantizedSparseMoE (`src/quanta/modeling/quantized.py:68-84`): gate and up by
        # width, h = silu(g) * u (rounded once to bf16 here), down by width
        g = mixed_proj(x[tok], exp, p["mixed"], "gate", hdim)
        u = mixed_proj(x[tok], exp, p["mixed"], "up", hdim)
        gu = np.concatenate([g, u], axis=1)
        h = swiglu(gu, inter, act, alpha, limit)
    elif p.get("gu_awq") is not None:
        gu, h = awq_expert_rows(x[tok], exp, p, inter, hdim, act=act, alpha=alpha, limit=limit,
                                round_weights=round_weights, group_size=group_size, bits=bits)
    else:
        gu = gather_qmm(x[tok], exp, p["gu_packed"], p["gu_scale"], p["gu_bias"], hdim,
                        round_weights=round_weights, group_size=group_size, bits=bits)
        h = swiglu(gu, inter, act, alpha, limit)
    if p.get("mixed") is not None:
        d = mixed_proj(h, exp, p["mixed"], "down", inter)
    else:
        d = gather_qmm(h, exp, p["dn_packed"], p["dn_scale"], p["dn_bias"], inter,
                       round_weights=round_weights, group_size=group_size,
                       bits=bits if down_bits is None else down_bits)
    routed = combine(d, w)
    y = routed.copy()
    sh = None
    if p.get("shared_gate_proj") is not None:
        sh, sh_out, sg = shared_expert(x, shared_weight(p["shared_gate_proj"]),
                                       shared_weight(p["shared_up_proj"]),
                                       shared_weight(p["shared_down_proj"]),
                                       p.get("shared_expert_gate"), act, alpha, limit)
        y = y + sh
    inter_d = dict(idx=idx, w=w, logits=logits, scores=scores, choice=choice, gu=gu, h=h, d=d,
                   routed=routed, shared=sh, y_exact=y)
    return round_bf16(y), inter_d


def moe_dense_reference(x: np.ndarray, idx: np.ndarray, w: np.ndarray, gu_dense: np.ndarray,
                        dn_dense: np.ndarray, inter: int) -> np.ndarray:
    """Run-every-expert oracle (`src/quanta/qwen35/moe.py:127-142`): every expert on every
    token, combined with the routing weight scattered onto the chosen experts (0 elsewhere).
    `gu_dense` [E,2I,H] / `dn_dense` [E,H,I] are dequantized float64 stacks. Unrounded float64
    throughout; this is the cross-check for the sparse gather path, not a bf16 flow."""
    n = x.shape[0]
    e = gu_dense.shape[0]
    gu = np.einsum("nh,eoh->neo", x.astype(np.float64), gu_dense)
    hh = _silu(gu[..., :inter]) * gu[..., inter:]
    d = np.einsum("nei,ehi->neh", hh, dn_dense)
    gates = np.zeros((n, e))
    rows = np.repeat(np.arange(n), idx.shape[1])
    gates[rows, idx.reshape(-1)] = w.reshape(-1)
    return (d * gates[:, :, None]).sum(axis=1)


# ----------------------------------------------------------------------------- reference dtypes


def round_to(v: np.ndarray, dt: str) -> np.ndarray:
    """v materialised in dtype dt: "f32" (float32 round to nearest even) or "bf16"."""
    if dt == "bf16":
        return round_bf16(v)
    if dt == "f32":
        return np.asarray(v, dtype=np.float64).astype(np.float32).astype(np.float64)
    raise ValueError(f"unknown dtype {dt!r}")


def moe_forward_general(x: np.ndarray, p: dict, *, k: int, inter: int, x_dtype: str = "f32",
                        dense_all: bool = False, scoring: str = "softmax", norm_topk: bool = True,
                        n_group: int = 1, topk_group: int = 1, scale: float = 1.0,
                        act: str = "silu", alpha: float = 1.702, limit: float = 0.0,
                        norm_single: bool = True):
    """The block at the reference's own dtype flow, for float32 or bf16 data
    (`src/quanta/qwen35/moe.py:36-56, 66-124, 145-151, 154-202`):
      logits = f32(x) @ f32(gate)^T, routing as `route`
      routed experts in dtype T: dense stacks' dtype (x cast to it, :77), or for packed codes the
        promotion of x's and the scales' dtypes (the qmm output follows the scale dtype, :98-104;
        float32 if either is float32)
      gu = T(x_T . W^T); h = T(glu(g, u)); d = T(h . W_d^T)   (one rounding per op here)
      routed = sum_s d * w (float32 in the reference, float64 here)
      shared = T_s(T_s(glu(T_s(x_s Wg^T), T_s(x_s Wu^T))) Wd^T) * sigmoid(x . g), x_s = x cast to
        the shared weights' dtype T_s (:145-151)
      y = cast to x's dtype (routed + shared) (:201-202)
    With `dense_all` every expert runs on every token and the combine weights are the routing
    weights scattered onto the chosen experts, zero elsewhere (the sparse=False oracle, :127-142).

    `p` keys: gate [E,H]; packed experts: gu_packed, dn_packed (uint32 words), gu_scale, gu_bias,
    dn_scale, dn_bias (float arrays holding float32 or bf16 values), "bits", "group_size",
    "sb_dtype"; or dense experts: gu_dense [E,2I,H], dn_dense [E,H,I] and "expert_dtype";
    optional shared_gate_proj/shared_up_proj [Is,H], shared_down_proj [H,Is], "shared_dtype",
    shared_expert_gate [1,H]; optional e_score_correction_bias [E]. Float arrays hold values
    exactly representable in their stated dtypes. Returns (y float64 in x's dtype, dict).
    """
    n, hdim = x.shape
    idx, w, logits, scores, choice = route(
        x, p["gate"], k=k, scoring=scoring, norm_topk=norm_topk,
        bias=p.get("e_score_correction_bias"), n_group=n_group, topk_group=topk_group,
        scale=scale, norm_single=norm_single)
    packed = "gu_packed" in p
    if packed:
        T = "f32" if "f32" in (x_dtype, p["sb_dtype"]) else "bf16"
        bits, gs = int(p["bits"]), int(p["group_size"])
    else:
        T = p["expert_dtype"]
    E = p["gate"].shape[0]
    if dense_all:
        if packed:
            raise ValueError("the run-every-expert form takes dense stacks")
        ks = E
        exp = np.tile(np.arange(E), n)
        wk = np.zeros((n, E))
        wk[np.repeat(np.arange(n), k), idx.reshape(-1)] = w.reshape(-1)
    else:
        ks, exp, wk = k, idx.reshape(-1), w
    tok = np.repeat(np.arange(n), ks)
    xr = round_to(x[tok].astype(np.float64), T)

    def weight(proj: str, e: int, in_features: int) -> np.ndarray:
        if packed:
            return dequant_float(p[f"{proj}_packed"][e], p[f"{proj}_scale"][e], p[f"{proj}_bias"][e],
                                 in_features, bits=bits, group_size=gs)
        return np.asarray(p[f"{proj}_dense"][e], dtype=np.float64)

    gu = np.zeros((n * ks, 2 * inter))
    for e in np.unique(exp):
        sel = exp == e
        gu[sel] = xr[sel] @ weight("gu", e, hdim).T
    gu = round_to(gu, T)
    h = round_to(glu(gu[:, :inter], gu[:, inter:], act, alpha, limit), T)
    d = np.zeros((n * ks, hdim))
    for e in np.unique(exp):
        sel = exp == e
        d[sel] = h[sel] @ weight("dn", e, inter).T
    d = round_to(d, T)
    routed = combine(d, wk)
    y = routed.copy()
    sh = None
    if p.get("shared_gate_proj") is not None:
        S = p["shared_dtype"]
        xs = round_to(x.astype(np.float64), S)
        g = round_to(xs @ np.asarray(p["shared_gate_proj"], dtype=np.float64).T, S)
        u = round_to(xs @ np.asarray(p["shared_up_proj"], dtype=np.float64).T, S)
        hh = round_to(glu(g, u, act, alpha, limit), S)
        out = round_to(hh @ np.asarray(p["shared_down_proj"], dtype=np.float64).T, S)
        sgw = p.get("shared_expert_gate")
        sh = out if sgw is None else out * _sigmoid(x.astype(np.float64) @ np.asarray(sgw, dtype=np.float64).reshape(-1))[:, None]
        y = y + sh
    inter_d = dict(idx=idx, w=w, logits=logits, scores=scores, choice=choice, gu=gu, h=h, d=d,
                   routed=routed, shared=sh, y_exact=y, routed_dtype=T)
    return round_to(y, x_dtype), inter_d
