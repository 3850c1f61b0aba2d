"""The quantized sparse-MoE block on MI355X: the reference's Python surface over the HIP C ABI.

Mirrors `qwen35_moe` / `qwen35_route` (src/quanta/qwen35/moe.py:36-56,154-202) and
`Qwen35MoEModule` (src/quanta/qwen35/model.py:28-70): same parameter-dict keys, same
`sparse` / `token_chunk` / `topk_override` arguments, same fail-loud errors (ValueError for a bad
`topk_override`, ValueError for the dense oracle on packed experts), packed-dict auto-detection,
fp32 combine, sigmoid-gated shared expert and bf16 output. It adds the DeepSeek/GLM router fields
(`scoring_func="sigmoid"`, `e_score_correction_bias`, `n_group`/`topk_group`,
`routed_scaling_factor`; src/quanta/modeling/moe.py:33-44, src/quanta/glm/moe.py:44-55).

All compute runs in the HIP kernels of `_qmoe.so`; there is no CPU path. Weights are converted
once into the MFMA-tiled layouts the kernels stream (cached per source tensor for the functional
API; held directly by the module).
"""

from __future__ import annotations

import ctypes
import math
import weakref
from dataclasses import dataclass

import torch
from torch.utils.weak import WeakIdKeyDictionary

from quanta_amd import _lib as L
from quanta_amd import ops


# ----------------------------------------------------------------------------------- config


@dataclass(frozen=True)
class MoEConfig:
    """MoE fields of `Qwen35Config` (src/quanta/qwen35/config.py:125-130) plus the DeepSeek/GLM
    router fields. Any object exposing these attribute names works where a config is taken."""

    hidden_size: int
    num_experts: int
    num_experts_per_tok: int
    moe_intermediate_size: int
    shared_expert_intermediate_size: int = 0
    scoring_func: str = "softmax"
    norm_topk_prob: bool = True
    n_group: int = 1
    topk_group: int = 1
    routed_scaling_factor: float = 1.0
    norm_eps: float = 1e-6
    hidden_act: str = "silu"
    swiglu_alpha: float = 1.702
    swiglu_limit: float = 0.0
    # renormalise a single routed expert's weight (k = 1) when norm_topk_prob is set; None picks
    # the reference router's own rule (see norm_mode)
    norm_topk_single: bool | None = None

    @property
    def moe_gate_up_out(self) -> int:
        """Stacked gate_up output width = 2 * moe_intermediate_size (config.py:223-225)."""
        return 2 * self.moe_intermediate_size

    @property
    def has_shared_expert(self) -> bool:
        return self.shared_expert_intermediate_size > 0


def _cfg(cfg, name, default=None):
    v = getattr(cfg, name, default)
    return default if v is None else v


def norm_mode(cfg, scoring: str, has_bias: bool) -> int:
    """QMOE_NORM_* mode of the router's renormalisation.

    qwen35_route renormalises whenever norm_topk_prob is set, a single expert included
    (src/quanta/qwen35/moe.py:53-54). The MoEGate routers, which select on sigmoid scores plus
    e_score_correction_bias, renormalise only when more than one expert is kept
    (src/quanta/modeling/moe.py:41-42, src/quanta/glm/moe.py:53-54, src/quanta/minimax/moe.py:54-55).
    DeepSeek-V4 renormalises its sqrt-softplus scores whatever norm_topk_prob says
    (src/quanta/dsv4/moe.py:54-55). `cfg.norm_topk_single`, when set, overrides the k = 1 rule."""
    if scoring == "sqrtsoftplus":
        return L.NORM_ALWAYS
    if not bool(_cfg(cfg, "norm_topk_prob", True)):
        return L.NORM_NONE
    single = getattr(cfg, "norm_topk_single", None)
    if single is None:
        single = not (scoring == "sigmoid" and has_bias)
    return L.NORM_ALWAYS if single else L.NORM_MULTI


# ----------------------------------------------------------------------------------- tiled experts


class TiledExperts(dict):
    """A routed expert stack resident in the MFMA-tiled layout.

    Keys: "format" ("int4_g64" | "int6_g64" | "int3_g64" | "bf16"), "codes" (tiled int4 / int6 /
    int3 words or tiled bf16), "sb" (tiled scale+bias of the quantized formats), "shape"
    (E, rows, K), "group_size", "bits", "awq_scale" (bf16 per-input-channel activation scales, or
    None) and "rexp" (int3/int4/int6: int8 [E, rows] per-row power-of-two exponents of the
    prefill kernels' fp16 dequant, or None). Produced from the reference's packed triplet
    {packed, scale, bias, group_size, bits} (src/quanta/qwen35/artifact.py:199-203; DeepSeek-V4's
    packed experts add awq_scale, src/quanta/dsv4/artifact.py:252-290) or from a bf16
    [E, rows, K] stack.
    """

    @property
    def is_packed(self) -> bool:
        return self["format"] in ("int4_g64", "int6_g64", "int3_g64")


def tile_experts_packed(d: dict) -> TiledExperts:
    """Reference packed triplet -> TiledExperts. Fails loud unless bits is 3, 4 or 6 and group_size
    is 64 or 128 (the kernels' formats: 128-column groups are tiled as two 64-column halves with
    the same scale and bias; int6 is MiniMax M3's expert format, src/quanta/minimax/
    model_m3.py:414-450; int3 Kimi's gate/up width, src/quanta/modeling/quantized.py:4-7; the
    manifest is the source of truth, src/quanta/qwen35/artifact.py:194)."""
    if isinstance(d, TiledExperts):
        return d
    bits, gs = int(d["bits"]), int(d["group_size"])
    if bits not in (3, 4, 6) or gs not in (64, 128):
        raise ValueError(f"packed experts must be affine int3, int4 or int6 with group_size 64 or "
                         f"128 (got bits={bits}, group_size={gs})")
    packed, scale, bias = d["packed"], d["scale"], d["bias"]
    if scale.dtype != torch.bfloat16 or bias.dtype != torch.bfloat16:
        raise TypeError("packed experts need bf16 scale and bias")
    if packed.dim() != 3:
        raise ValueError("packed experts must be a stacked [E, out, in*bits/32] tensor")
    E, rows, W = packed.shape
    tile = {4: ops.tile_int4, 6: ops.tile_int6, 3: ops.tile_int3}[bits]
    codes, sb = tile(packed.contiguous(), scale.contiguous(), bias.contiguous(), group_size=gs)
    # the prefill kernels' fp16 dequant: per-row power-of-two exponents keep any row's weights
    # in fp16's normal range
    rexp = ops.row_exponents(scale.contiguous(), bias.contiguous(), bits=bits, group_size=gs)
    awq = d.get("awq_scale")
    if awq is not None:
        awq = awq.to(device=packed.device, dtype=torch.bfloat16).contiguous()
    return TiledExperts(format=f"int{bits}_g64", codes=codes, sb=sb, shape=(E, rows, W * 32 // bits),
                        group_size=gs, bits=bits, awq_scale=awq, rexp=rexp)


def tile_experts_bf16(stack: torch.Tensor) -> TiledExperts:
    """bf16 expert stack [E, rows, K] -> TiledExperts (format "bf16")."""
    if isinstance(stack, TiledExperts):
        return stack
    if stack.dtype != torch.bfloat16:
        raise TypeError(f"bf16 expert stacks only (got {stack.dtype})")
    if stack.dim() != 3:
        raise ValueError("expert stack must be [E, out, in]")
    return TiledExperts(format="bf16", codes=ops.tile_bf16(stack.contiguous()), sb=None,
                        shape=tuple(stack.shape), group_size=0, bits=16)


PROJS = ("gate", "up", "down")
# router score functions: Qwen softmax; DeepSeek-V3/GLM sigmoid; DeepSeek-V4 sqrt(softplus)
# (src/quanta/dsv4/moe.py:37-57)
_SCORING = {"softmax": L.SCORE_SOFTMAX, "sigmoid": L.SCORE_SIGMOID, "sqrtsoftplus": L.SCORE_SQRTSOFTPLUS}


class MixedExperts(dict):
    """Routed experts whose widths vary per (expert, projection), resident: "stacks" is a list of
    (projection, TiledExperts, expert map [E] int32 on the device: the expert's slot in that
    stack or -1), "n_experts" E; projection "gate_up" when gate and up are fused per width.
    Built by tile_experts_mixed."""


def tile_experts_mixed(stacks: dict, pbits: dict, pslot: dict, *, group_size: int = 128) -> MixedExperts:
    """Kimi's per-(expert, projection) widths (QuantizedSparseMoE.set_experts,
    src/quanta/modeling/quantized.py:40-51) -> MixedExperts. `stacks[proj][bits]` is the packed
    stack {packed, scale, bias} of that projection and width ("gate", "up" [E_w, I, H], "down"
    [E_w, H, I]); `pbits[proj]` / `pslot[proj]` [E]: each expert's width and its slot in that
    width's stack. Checked here, on the host: every expert's width has a stack and its slot lies
    in it (the kernels read the maps without checks)."""
    if isinstance(stacks, MixedExperts):
        return stacks
    out, E = [], None
    # every expert's gate and up of one width and slot: fuse them per width (gate rows first),
    # so gate_up runs as the uniform stacks do, SwiGLU in the matmul's epilogue
    host = lambda v: torch.as_tensor(v).to("cpu", torch.int64).reshape(-1)
    gsz = lambda st: int(st.get("group_size", group_size))
    fuse = (set(stacks["gate"]) == set(stacks["up"]) and
            torch.equal(host(pbits["gate"]), host(pbits["up"])) and
            torch.equal(host(pslot["gate"]), host(pslot["up"])) and
            all(stacks["gate"][b]["packed"].shape == stacks["up"][b]["packed"].shape and
                gsz(stacks["gate"][b]) == gsz(stacks["up"][b]) for b in stacks["gate"]))
    if fuse:
        stacks = dict(stacks, gate_up={b: dict({key: torch.cat([stacks["gate"][b][key], stacks["up"][b][key]], dim=1)
                                                for key in ("packed", "scale", "bias")},
                                               group_size=gsz(stacks["gate"][b]))
                                       for b in stacks["gate"]})
        pbits, pslot = dict(pbits, gate_up=pbits["gate"]), dict(pslot, gate_up=pslot["gate"])
    for proj in (("gate_up", "down") if fuse else PROJS):
        pb = torch.as_tensor(pbits[proj]).to("cpu", torch.int64).reshape(-1)
        ps = torch.as_tensor(pslot[proj]).to("cpu", torch.int64).reshape(-1)
        if E is None:
            E = pb.numel()
        if pb.numel() != E or ps.numel() != E:
            raise ValueError(f"pbits/pslot[{proj!r}] must have one entry per expert ({E})")
        have = {int(b) for b in stacks[proj]}
        missing = sorted(set(pb.tolist()) - have)
        if missing:
            raise ValueError(f"{proj}: experts of width {missing} have no stack")
        for bits in sorted(have):
            st = stacks[proj][bits]
            te = tile_experts_packed(dict(st, bits=bits, group_size=int(st.get("group_size", group_size))))
            mine = pb == bits
            if bool(mine.any()) and (int(ps[mine].min()) < 0 or int(ps[mine].max()) >= te["shape"][0]):
                raise ValueError(f"{proj}: slots of width {bits} outside its stack of {te['shape'][0]}")
            emap = torch.where(mine, ps, torch.full_like(ps, -1)).to(torch.int32).to(te["codes"].device)
            out.append((proj, te, emap))
    return MixedExperts(stacks=out, n_experts=E)


def _is_packed(v) -> bool:
    """Auto-detection of packed experts, as the reference does with isinstance(dict)
    (src/quanta/qwen35/moe.py:181)."""
    if isinstance(v, TiledExperts):
        return v.is_packed
    return isinstance(v, dict)


# ----------------------------------------------------------------------------------- resident forms

# The resident (tiled) forms the kernels read are derived once per layer and memoised on the
# caller's own tensors: each memo entry hangs off an "anchor" tensor of the layer (the router
# gate, a native expert stack, the shared gate_proj) through a weak key, so it lives exactly as
# long as the layer's weights do. There is no size limit to overflow at model scale (a 60-layer
# decode loop hits on every call), and a dropped layer takes its entries with it. An entry is
# reused only while every source it was built from is the same object at the same version.
# (keyed by tensor identity: a plain WeakKeyDictionary would compare tensors with ==)
_MEMO: "WeakIdKeyDictionary" = WeakIdKeyDictionary()


def _leaves(o, out: list) -> list:
    """Flatten a parameter value into identity leaves (tensors, arrays, resident forms) and value
    leaves (keys, bits, group sizes, shapes)."""
    if isinstance(o, (torch.Tensor, TiledExperts, MixedExperts)) or type(o).__name__ == "ndarray":
        out.append(o)
    elif isinstance(o, dict):
        for k in sorted(o, key=str):
            out.append(("k", str(k)))
            _leaves(o[k], out)
    elif isinstance(o, (list, tuple)):
        out.append(("n", len(o)))
        for v in o:
            _leaves(v, out)
    else:
        out.append(("v", o))
    return out


def _version(o) -> int:
    return o._version if isinstance(o, torch.Tensor) else 0


def _signature(sources) -> tuple:
    sig = []
    for leaf in _leaves(list(sources), []):
        if isinstance(leaf, tuple):
            sig.append(leaf)
        else:
            sig.append((weakref.ref(leaf), _version(leaf)))
    return tuple(sig)


def _matches(sig: tuple, sources) -> bool:
    leaves = _leaves(list(sources), [])
    if len(leaves) != len(sig):
        return False
    for leaf, want in zip(leaves, sig):
        if isinstance(leaf, tuple):
            if leaf != want:
                return False
        elif not (isinstance(want[0], weakref.ref) and want[0]() is leaf and want[1] == _version(leaf)):
            return False
    return True


def _memo(anchor: torch.Tensor, kind, sources, build):
    """The value `build()` derives from `sources`, memoised on `anchor` (a weak key). The value
    must not hold `anchor` itself, or the entry would keep its own key alive."""
    entries = _MEMO.get(anchor)
    if entries is None:
        entries = _MEMO[anchor] = {}
    hit = entries.get(kind)
    if hit is not None and _matches(hit[0], sources):
        return hit[1]
    value = build()
    entries[kind] = (_signature(sources), value)
    return value


def clear_cache() -> None:
    """Drop every memoised resident form (they are rebuilt on the next call)."""
    _MEMO.clear()


def resident_experts(v):
    """The resident (tiled) form of an expert stack: a packed triplet dict or a bf16 [E, out, in]
    stack, converted once (memoised on the native tensors); a TiledExperts is returned as is."""
    if v is None or isinstance(v, TiledExperts):
        return v
    if isinstance(v, dict):
        return _memo(v["packed"], "tiled", (v,), lambda: tile_experts_packed(v))
    return _memo(v, "tiled16", (v,), lambda: tile_experts_bf16(v))


def resident_params(p: dict) -> dict:
    """A copy of the parameter dict `p` whose expert stacks are their resident tiled forms. A
    caller that keeps this dict and drops its native triplets holds each layer once on the GPU
    (the module's set_experts_packed does the same). Other entries are passed through."""
    q = dict(p)
    for key in ("experts_gate_up", "experts_down"):
        if q.get(key) is not None:
            q[key] = resident_experts(q[key])
    return q


# ----------------------------------------------------------------------------------- prepare


@dataclass
class Prepared:
    """Everything one qmoe_forward call needs, with the tensors kept alive."""

    cfg: L.QmoeConfig
    weights: L.QmoeWeights
    keep: tuple
    router_tiled: torch.Tensor | None
    router_f32: torch.Tensor | None
    shared_gate_f32: torch.Tensor | None
    gu: TiledExperts
    dn: TiledExperts
    sh_gu: torch.Tensor | None
    sh_dn: torch.Tensor | None
    bias: torch.Tensor | None
    mixed: L.QmoeMixed | None = None
    sh_gu_sb: torch.Tensor | None = None   # int8 shared expert: tiled scale/bias
    sh_dn_sb: torch.Tensor | None = None


def _prepare_router(gate: torch.Tensor, sgate: torch.Tensor | None, E: int, H: int):
    """Router weight [E, H] (+ optional shared-expert gate [1, H]) -> resident form.

    bf16 router (the artifact dtype, src/quanta/qwen35/bake.py:147-148): one tiled bf16 matrix
    whose row E is the shared gate, padded to a multiple of 256 rows; its logits come from the
    bf16 MFMA path (bf16 x bf16 products are exact in fp32). fp32 router (or fp32 gate): kept
    fp32 row-major for the fp32 VALU logits kernel, preserving xf.f32 @ gate.f32.T exactly."""
    if gate.shape != (E, H):
        raise ValueError(f"gate must be [{E}, {H}] (got {tuple(gate.shape)})")
    gated = sgate is not None
    if gate.dtype == torch.bfloat16 and (not gated or sgate.dtype == torch.bfloat16):
        rows = int(math.ceil((E + (1 if gated else 0)) / 256.0)) * 256
        full = torch.zeros(rows, H, dtype=torch.bfloat16, device=gate.device)
        full[:E] = gate
        if gated:
            full[E] = sgate.reshape(H)
        return ("bf16", ops.tile_bf16(full), rows, None)
    wr = gate.to(torch.float32).contiguous()
    if wr is gate:   # an fp32 gate: its own copy, so the memo entry does not hold its weak key
        wr = gate.clone()
    sg = sgate.to(torch.float32).reshape(H).contiguous() if gated else None
    return ("f32", wr, E + 1, sg)


def _prepare_shared(p: dict, H: int, Is: int):
    """Shared expert -> (format, gate|up tiles, their sb, down tiles, their sb). bf16 [Is, H] /
    [H, Is] matrices tile as bf16. int8 triplets {packed, scale, bias, group_size, bits: 8}, the
    bake's shared-expert format (src/quanta/qwen35/bake.py:106-110, 150-151), stay int8: the
    kernels dequantize them in registers to the bf16 weights the reference's loader makes of them
    (src/quanta/qwen35/artifact.py:105-115), so the outputs are those of the dequantized bf16
    matrices, at half the bytes read."""
    names = ("shared_gate_proj", "shared_up_proj", "shared_down_proj")
    wg, wu, wd = (p[nm] for nm in names)
    quant = [isinstance(t, dict) for t in (wg, wu, wd)]
    if any(quant) and not all(quant):
        raise ValueError("shared expert: gate, up and down must all be int8 triplets or all bf16")
    if all(quant):
        for t, nm in zip((wg, wu, wd), names):
            if int(t.get("bits", 8)) != 8:
                raise ValueError(f"{nm}: a quantized shared expert must be int8 (bits 8), as baked")
        gs = int(wg.get("group_size", 64))
        if any(int(t.get("group_size", 64)) != gs for t in (wu, wd)) or gs not in (64, 128):
            raise ValueError("shared expert: one group size (64 or 128) for gate, up and down")
        if (tuple(wg["packed"].shape) != (Is, H // 4) or tuple(wu["packed"].shape) != (Is, H // 4)
                or tuple(wd["packed"].shape) != (H, Is // 4)):
            raise ValueError("shared expert int8 shapes must be gate/up [Is, H/4] and down [H, Is/4] words")
        cat = [torch.cat([wg[k], wu[k]], dim=0).contiguous() for k in ("packed", "scale", "bias")]
        gu_c, gu_sb = ops.tile_int8(*cat, group_size=gs)
        dn_c, dn_sb = ops.tile_int8(wd["packed"].contiguous(), wd["scale"].contiguous(),
                                    wd["bias"].contiguous(), group_size=gs)
        return "int8", gu_c, gu_sb, dn_c, dn_sb
    for t, nm in zip((wg, wu, wd), names):
        if t.dtype != torch.bfloat16:
            raise TypeError(f"{nm} must be bf16 or an int8 triplet (the shared expert runs in bf16)")
    if wg.shape != (Is, H) or wu.shape != (Is, H) or wd.shape != (H, Is):
        raise ValueError("shared expert shapes must be gate/up [Is, H] and down [H, Is]")
    gu = torch.cat([wg, wu], dim=0).contiguous()
    return "bf16", ops.tile_bf16(gu), None, ops.tile_bf16(wd.contiguous()), None


def _anchor(v) -> torch.Tensor:
    """The tensor a memo entry of parameter value `v` hangs off (a triplet's packed codes)."""
    return v["packed"] if isinstance(v, dict) else v


def gated_activation(cfg) -> tuple[int, float, float]:
    """(act, alpha, limit) of the experts' SwiGLU from the config: `hidden_act` "silu" is the
    Qwen SwiGLU (src/quanta/qwen35/moe.py:59-63), clamped by `swiglu_limit` > 0 as DeepSeek-V4
    does (src/quanta/dsv4/moe.py:74-77); "swigluoai" is the clamped SwiGLU-OAI of MiniMax M3
    (src/quanta/minimax/model_m3.py:112-128; `swiglu_alpha`, `swiglu_limit`)."""
    act = str(_cfg(cfg, "hidden_act", "silu"))
    limit = float(_cfg(cfg, "swiglu_limit", 0.0) or 0.0)
    alpha = float(_cfg(cfg, "swiglu_alpha", 1.702))
    inf = float("inf")
    if act == "swigluoai":
        return L.ACT_SWIGLU_OAI, alpha, (limit if limit > 0 else inf)
    if act in ("silu", "swish"):
        return (L.ACT_SILU_CLAMP, 1.0, limit) if limit > 0 else (L.ACT_SILU, 1.0, inf)
    raise ValueError(f"hidden_act {act!r} not supported (silu | swigluoai)")


# parameter-dict keys and config fields a prepared block depends on
_PARAM_KEYS = ("gate", "experts_gate_up", "experts_down", "experts_mixed", "shared_gate_proj",
               "shared_up_proj", "shared_down_proj", "shared_expert_gate", "e_score_correction_bias")
_CFG_FIELDS = ("hidden_size", "num_experts", "num_experts_per_tok", "moe_intermediate_size",
               "shared_expert_intermediate_size", "scoring_func", "norm_topk_prob", "n_group",
               "topk_group", "routed_scaling_factor", "hidden_act", "swiglu_alpha", "swiglu_limit",
               "norm_topk_single")


def prepare(p: dict, cfg, *, topk: int | None = None, regime: int = L.REGIME_AUTO) -> Prepared:
    """Resolve the parameter dict `p` (reference keys, src/quanta/qwen35/moe.py:159-161) into the
    resident kernel form. The result is memoised per layer on p["gate"], and each weight's tiled
    form on that weight, so a model's layers are converted once however many there are."""
    sig = tuple(getattr(cfg, f, None) for f in _CFG_FIELDS)
    sources = [p.get(k) for k in _PARAM_KEYS]
    return _memo(p["gate"], ("block", topk, regime, sig), sources,
                 lambda: _build_prepared(p, cfg, topk=topk, regime=regime))


def _build_prepared(p: dict, cfg, *, topk: int | None, regime: int) -> Prepared:
    H = int(_cfg(cfg, "hidden_size"))
    E = int(_cfg(cfg, "num_experts"))
    I = int(_cfg(cfg, "moe_intermediate_size"))
    Is = int(_cfg(cfg, "shared_expert_intermediate_size", 0))
    k = int(topk if topk is not None else _cfg(cfg, "num_experts_per_tok"))
    scoring = str(_cfg(cfg, "scoring_func", "softmax"))
    if scoring not in _SCORING:
        raise ValueError(f"scoring_func {scoring!r} not supported (softmax | sigmoid | sqrtsoftplus)")

    if p.get("experts_mixed") is not None:
        return _prepare_mixed(p, cfg, topk=topk, regime=regime)
    gu_src, dn_src = p["experts_gate_up"], p["experts_down"]
    packed = _is_packed(gu_src)
    if packed != _is_packed(dn_src):
        raise ValueError("experts_gate_up and experts_down must both be packed or both bf16")
    gu, dn = resident_experts(gu_src), resident_experts(dn_src)
    if tuple(gu["shape"]) != (E, 2 * I, H) or tuple(dn["shape"]) != (E, H, I):
        raise ValueError(f"expert stacks must be gate_up [{E},{2 * I},{H}] and down [{E},{H},{I}] "
                         f"(got {gu['shape']} and {dn['shape']})")

    has_shared = Is > 0 and p.get("shared_gate_proj") is not None
    sgate = p.get("shared_expert_gate") if has_shared else None
    gate = p["gate"]
    rkind, rw, rrows, sg32 = _memo(gate, ("router", sgate is not None), (gate, sgate),
                                   lambda: _prepare_router(gate, sgate, E, H))
    sh_fmt, sh_gu, sh_gu_sb, sh_dn, sh_dn_sb = "bf16", None, None, None, None
    if has_shared:
        shw = (p["shared_gate_proj"], p["shared_up_proj"], p["shared_down_proj"])
        sh_fmt, sh_gu, sh_gu_sb, sh_dn, sh_dn_sb = _memo(_anchor(shw[0]), "shared", shw,
                                                         lambda: _prepare_shared(p, H, Is))
    bias = p.get("e_score_correction_bias")
    if bias is not None:
        bias = bias.to(torch.float32).reshape(E).contiguous()

    c = L.QmoeConfig()
    c.hidden, c.n_experts, c.top_k, c.inter = H, E, k, I
    c.shared_inter = Is if has_shared else 0
    c.scoring = _SCORING[scoring]
    c.norm_topk = norm_mode(cfg, scoring, bias is not None)
    c.n_group = int(_cfg(cfg, "n_group", 1))
    c.topk_group = int(_cfg(cfg, "topk_group", 1))
    c.routed_scale = float(_cfg(cfg, "routed_scaling_factor", 1.0))
    fmts = {"int4_g64": L.FMT_INT4_G64, "int6_g64": L.FMT_INT6_G64, "int3_g64": L.FMT_INT3_G64,
            "bf16": L.FMT_BF16}
    # gate_up and down may differ in width (Kimi: gate/up int3, down int4,
    # src/quanta/modeling/quantized.py:4-7)
    c.expert_format, c.down_format = fmts[gu["format"]], fmts[dn["format"]]
    c.router_format = L.ROUTER_BF16_TILED if rkind == "bf16" else L.ROUTER_F32
    c.router_rows = rrows
    c.shared_gated = int(sgate is not None)
    c.shared_format = L.FMT_INT8_G64 if sh_fmt == "int8" else L.FMT_BF16
    c.regime = regime
    c.act, c.act_alpha, c.act_limit = gated_activation(cfg)
    # DeepSeek-V4's activation-aware scales (src/quanta/dsv4/moe.py:112-137): gate and up
    # scales of the fused gate_up stack as [E, 2, H] (w1 row 0, w3 row 1), down [E, I]
    awq_gu, awq_dn = gu.get("awq_scale"), dn.get("awq_scale")
    if (awq_gu is None) != (awq_dn is None):
        raise ValueError("awq_scale must be given on both experts_gate_up and experts_down")
    if awq_gu is not None:
        if tuple(awq_gu.shape) != (E, 2, H) or tuple(awq_dn.shape) != (E, I):
            raise ValueError(f"awq_scale must be gate_up [{E}, 2, {H}] and down [{E}, {I}] "
                             f"(got {tuple(awq_gu.shape)} and {tuple(awq_dn.shape)})")
        c.awq = 1

    w = L.QmoeWeights()
    w.router_w = rw.data_ptr()
    w.router_bias = bias.data_ptr() if bias is not None else None
    w.shared_gate_w = sg32.data_ptr() if sg32 is not None else None
    # (codes None: the shape-only placeholder of a mixed-width layer, see _prepare_mixed)
    w.gu_codes = gu["codes"].data_ptr() if gu["codes"] is not None else None
    w.gu_sb = gu["sb"].data_ptr() if gu["sb"] is not None else None
    w.dn_codes = dn["codes"].data_ptr() if dn["codes"] is not None else None
    w.dn_sb = dn["sb"].data_ptr() if dn["sb"] is not None else None
    w.sh_gu = sh_gu.data_ptr() if sh_gu is not None else None
    w.sh_dn = sh_dn.data_ptr() if sh_dn is not None else None
    w.sh_gu_sb = sh_gu_sb.data_ptr() if sh_gu_sb is not None else None
    w.sh_dn_sb = sh_dn_sb.data_ptr() if sh_dn_sb is not None else None
    w.awq_gu = awq_gu.data_ptr() if awq_gu is not None else None
    w.awq_dn = awq_dn.data_ptr() if awq_dn is not None else None
    gu_rexp, dn_rexp = gu.get("rexp"), dn.get("rexp")
    w.gu_rexp = gu_rexp.data_ptr() if gu_rexp is not None else None
    w.dn_rexp = dn_rexp.data_ptr() if dn_rexp is not None else None
    keep = (rw, bias, sg32, gu, dn, sh_gu, sh_dn, sh_gu_sb, sh_dn_sb, awq_gu, awq_dn)
    return Prepared(c, w, keep, rw if rkind == "bf16" else None, rw if rkind == "f32" else None,
                    sg32, gu, dn, sh_gu, sh_dn, bias, sh_gu_sb=sh_gu_sb, sh_dn_sb=sh_dn_sb)


def _prepare_mixed(p: dict, cfg, *, topk, regime) -> Prepared:
    """prepare() for p["experts_mixed"] (MixedExperts, or the reference's (stacks, pbits, pslot)
    as a dict with those keys): the rest of the block as for uniform stacks, the routed experts
    through qmoe_forward_mixed."""
    H, E = int(_cfg(cfg, "hidden_size")), int(_cfg(cfg, "num_experts"))
    I = int(_cfg(cfg, "moe_intermediate_size"))
    src = p["experts_mixed"]
    mx = src if isinstance(src, MixedExperts) else _memo(
        p["gate"], "mixed", (src,),
        lambda: tile_experts_mixed(src["stacks"], src["pbits"], src["pslot"],
                                   group_size=int(src.get("group_size", 128))))
    if mx["n_experts"] != E:
        raise ValueError(f"mixed experts: {mx['n_experts']} experts for a {E}-expert config")
    if len(mx["stacks"]) > L.MAX_STACKS:
        raise ValueError(f"mixed experts: at most {L.MAX_STACKS} (projection, width) stacks")
    m = L.QmoeMixed()
    m.n_stacks = len(mx["stacks"])
    fmts = {"int4_g64": L.FMT_INT4_G64, "int6_g64": L.FMT_INT6_G64, "int3_g64": L.FMT_INT3_G64}
    proj_id = {"gate": L.PROJ_GATE, "up": L.PROJ_UP, "down": L.PROJ_DOWN, "gate_up": L.PROJ_GATE_UP}
    for i, (proj, te, emap) in enumerate(mx["stacks"]):
        want = {"down": (H, I), "gate_up": (2 * I, H)}.get(proj, (I, H))
        if tuple(te["shape"][1:]) != want:
            raise ValueError(f"mixed experts: {proj} stacks must be [E_w, {want[0]}, {want[1]}] "
                             f"(got {tuple(te['shape'])})")
        m.stacks[i] = L.QmoeStack(proj_id[proj], fmts[te["format"]], te["codes"].data_ptr(),
                                  te["sb"].data_ptr(), emap.data_ptr(),
                                  te["rexp"].data_ptr() if te.get("rexp") is not None else None)
    # the rest of the block: a placeholder uniform stack pair supplies nothing but the shapes
    q = {kk: v for kk, v in p.items() if kk != "experts_mixed"}
    q["experts_gate_up"] = TiledExperts(format="int4_g64", codes=None, sb=None, shape=(E, 2 * I, H),
                                        group_size=64, bits=4)
    q["experts_down"] = TiledExperts(format="int4_g64", codes=None, sb=None, shape=(E, H, I),
                                     group_size=64, bits=4)
    pr = _build_prepared(q, cfg, topk=topk, regime=regime)
    pr.cfg.mixed = 1
    pr.mixed = m
    pr.keep = pr.keep + (mx,)
    return pr


# ----------------------------------------------------------------------------------- routing


def _dense_regime(n: int, hidden: int) -> int:
    """Regime of the dense (router / shared expert) matmuls, as qmoe_forward picks it."""
    return L.REGIME_LARGE if (n > 256 and hidden % 256 == 0) else L.REGIME_SMALL


def _router_logits(xf: torch.Tensor, pr: Prepared) -> torch.Tensor:
    c = pr.cfg
    if c.router_format == L.ROUTER_F32:
        return ops.router_logits_f32(xf, pr.router_f32, pr.shared_gate_f32)
    n = xf.shape[0]
    regime = _dense_regime(n, c.hidden)
    return ops.grouped_qmm(xf, K=c.hidden, n_rows=c.router_rows, weight_format=L.FMT_BF16,
                           codes=pr.router_tiled, sb=None, epilogue=L.EPI_F32, out_rows=n,
                           regime=regime, dense_rows=n)


def _topk(logits: torch.Tensor, pr: Prepared, k: int):
    c = pr.cfg
    return ops.router_topk(logits, c.n_experts, k, scoring=c.scoring, bias=pr.bias,
                           n_group=c.n_group, topk_group=c.topk_group, norm_topk=c.norm_topk,
                           routed_scale=c.routed_scale, has_shared_gate=bool(c.shared_gated))


def qwen35_route(xf: torch.Tensor, gate_w: torch.Tensor, cfg, *, topk_override: int | None = None,
                 e_score_correction_bias: torch.Tensor | None = None):
    """Top-k routing -> (idx [N,k] int32, w [N,k] fp32), on the GPU.

    Mirrors `qwen35_route` (src/quanta/qwen35/moe.py:36-56): fp32 logits, softmax (or sigmoid)
    scores, top-k, gathered scores renormalised with +1e-20 when norm_topk_prob. Returned in the
    canonical order (score descending, id ascending); the reference's argpartition gives the
    same set unordered. With the DeepSeek/GLM fields it is MoEGate.__call__
    (src/quanta/modeling/moe.py:33-44): selection by sigmoid + bias, optional groups, scaling.
    """
    if xf.dtype != torch.bfloat16:
        raise TypeError("qwen35_route: x must be bf16")
    E, H = int(_cfg(cfg, "num_experts")), int(_cfg(cfg, "hidden_size"))
    k = topk_override if topk_override is not None else int(_cfg(cfg, "num_experts_per_tok"))
    kind, rw, rows, _ = _memo(gate_w, ("router", False), (gate_w, None),
                              lambda: _prepare_router(gate_w, None, E, H))
    xf = xf.contiguous()
    n = xf.shape[0]
    if kind == "f32":
        logits = ops.router_logits_f32(xf, rw, None)
    else:
        logits = ops.grouped_qmm(xf, K=H, n_rows=rows, weight_format=L.FMT_BF16, codes=rw, sb=None,
                                 epilogue=L.EPI_F32, out_rows=n, regime=_dense_regime(n, H),
                                 dense_rows=n)
    sname = str(_cfg(cfg, "scoring_func", "softmax"))
    scoring = _SCORING[sname]
    bias = None if e_score_correction_bias is None else e_score_correction_bias.float().reshape(E).contiguous()
    idx, w, _ = ops.router_topk(logits, E, k, scoring=scoring, bias=bias,
                                n_group=int(_cfg(cfg, "n_group", 1)),
                                topk_group=int(_cfg(cfg, "topk_group", 1)),
                                norm_topk=norm_mode(cfg, sname, bias is not None),
                                routed_scale=float(_cfg(cfg, "routed_scaling_factor", 1.0)))
    return idx, w


# ----------------------------------------------------------------------------------- the block


def _routed_dense(xf: torch.Tensor, pr: Prepared, k: int) -> torch.Tensor:
    """Run-every-expert path (`sparse=False`, bf16 stacks only; src/quanta/qwen35/moe.py:127-142):
    every expert runs on every token and the combine uses the routing weight scattered onto the
    chosen experts (0 elsewhere). Built from the op-level entry points."""
    c = pr.cfg
    n, E = xf.shape[0], c.n_experts
    logits = _router_logits(xf, pr)
    idx, w, sg = _topk(logits, pr, k)
    idx_all = torch.arange(E, dtype=torch.int32, device=xf.device).repeat(n, 1).contiguous()
    w_all = torch.zeros(n, E, dtype=torch.float32, device=xf.device)
    w_all.scatter_(1, idx.long(), w)
    regime = L.REGIME_SMALL if (n * E <= 256 * 16 or c.hidden % 256) else L.REGIME_LARGE
    m_tile = L.SMALL_M_TILE if regime == L.REGIME_SMALL else L.LARGE_M_TILE
    counts, offsets, tile_off, sorted_slot, inv, tile_map = ops.permute(idx_all, E, m_tile)
    fmt = c.expert_format
    h = ops.grouped_qmm(xf, K=c.hidden, n_rows=2 * c.inter, weight_format=fmt,
                        codes=pr.gu["codes"], sb=pr.gu["sb"], epilogue=L.EPI_SWIGLU,
                        out_rows=n * E, regime=regime, slot_of=sorted_slot, slot_div=E,
                        n_slots=n * E, offsets=offsets, tile_off=tile_off, tile_map=tile_map,
                        n_experts=E, glu=c.act, glu_alpha=c.act_alpha, glu_limit=c.act_limit)
    d = ops.grouped_qmm(h, K=c.inter, n_rows=c.hidden, weight_format=fmt, codes=pr.dn["codes"],
                        sb=pr.dn["sb"], epilogue=L.EPI_BF16, out_rows=n * E, regime=regime,
                        n_slots=n * E, offsets=offsets, tile_off=tile_off, tile_map=tile_map,
                        n_experts=E)
    sh_out = None
    if c.shared_inter > 0:
        # (int8 shared weights: the small regime, which dequantizes them in registers)
        sfmt = c.shared_format
        sreg = L.REGIME_SMALL if sfmt == L.FMT_INT8_G64 else _dense_regime(n, c.hidden)
        sh_h = ops.grouped_qmm(xf, K=c.hidden, n_rows=2 * c.shared_inter, weight_format=sfmt,
                               codes=pr.sh_gu, sb=pr.sh_gu_sb, epilogue=L.EPI_SWIGLU, out_rows=n,
                               regime=sreg, dense_rows=n, glu=c.act, glu_alpha=c.act_alpha,
                               glu_limit=c.act_limit)
        sh_out = ops.grouped_qmm(sh_h, K=c.shared_inter, n_rows=c.hidden, weight_format=sfmt,
                                 codes=pr.sh_dn, sb=pr.sh_dn_sb, epilogue=L.EPI_BF16, out_rows=n,
                                 regime=sreg, dense_rows=n)
    return ops.combine(d, inv, w_all, sh_out, sg)


# --------------------------------------------------------- the reference's own dtypes and groups

_SHARED_KEYS = ("shared_gate_proj", "shared_up_proj", "shared_down_proj")


def _fast_packed(d) -> bool:
    """Whether a packed triplet is one of the fast path's formats (bf16 scale/bias, int3/4/6,
    groups of 64 or 128)."""
    if isinstance(d, TiledExperts):
        return True
    return (int(d["bits"]) in (3, 4, 6) and int(d["group_size"]) in (64, 128)
            and d["scale"].dtype == torch.bfloat16 and d["bias"].dtype == torch.bfloat16)


def needs_general(x: torch.Tensor, p: dict, cfg) -> bool:
    """Whether the block must run at the reference's own dtypes (qmoe_forward_general): float32
    activations, float32 (or otherwise non-bf16) expert or shared weights, packed groups other
    than 64/128, code widths other than 3/4/6, or dimensions the tiled kernels do not take
    (hidden, moe_intermediate or shared_intermediate not a multiple of 128) -- all of which the
    reference's block accepts (src/quanta/qwen35/moe.py:98-104: the qmm output follows the
    scale dtype; parity/qwen35_forward_test.py:213-271 runs float32, group 32, hidden 32)."""
    if p.get("experts_mixed") is not None:
        return False
    if x.dtype != torch.bfloat16:
        return True
    H, I = int(_cfg(cfg, "hidden_size")), int(_cfg(cfg, "moe_intermediate_size"))
    Is = int(_cfg(cfg, "shared_expert_intermediate_size", 0))
    if H % 128 or I % 128 or (Is > 0 and Is % 128):
        return True
    for v in (p["experts_gate_up"], p["experts_down"]):
        if isinstance(v, dict):
            if not _fast_packed(v):
                return True
        elif v.dtype != torch.bfloat16:
            return True
    if Is > 0 and p.get("shared_gate_proj") is not None:
        if any(isinstance(p[k], torch.Tensor) and p[k].dtype != torch.bfloat16 for k in _SHARED_KEYS):
            return True
    return False


def _gen_tensor(t: torch.Tensor, shape: tuple, name: str) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a tensor")
    if tuple(t.shape) != shape:
        raise ValueError(f"{name} must be {list(shape)} (got {list(t.shape)})")
    ops.dtype_code(t.dtype, name)
    return t.contiguous()


def _gen_experts(v, rows: int, K: int, E: int, name: str):
    """(packed?, dtype code, bits, group_size, tensors) of one routed stack for the general path."""
    if isinstance(v, TiledExperts):
        raise TypeError(f"{name}: this block needs the native packed triplet (the tiled resident "
                        "form serves bf16 activations with bf16 scales only)")
    if isinstance(v, dict):
        if v.get("awq_scale") is not None:
            raise ValueError(f"{name}: activation-aware scales need bf16 activations and bf16 scales")
        bits, gs = int(v["bits"]), int(v["group_size"])
        if bits not in (2, 3, 4, 5, 6, 8) or gs not in (32, 64, 128) or K % gs or (K * bits) % 32:
            raise ValueError(f"{name}: packed experts must be 2..6 or 8 bits with group_size 32, 64 "
                             f"or 128 dividing the in-features (got bits={bits}, group_size={gs})")
        words = v["packed"]
        if words.dtype == torch.uint32:
            words = words.view(torch.int32)
        if words.dtype != torch.int32 or tuple(words.shape) != (E, rows, K * bits // 32):
            raise ValueError(f"{name}: packed must be uint32 [{E}, {rows}, {K * bits // 32}]")
        for part in ("scale", "bias"):
            if tuple(v[part].shape) != (E, rows, K // gs):
                raise ValueError(f"{name}.{part} {list(v[part].shape)} does not match group_size "
                                 f"{gs} (expected {[E, rows, K // gs]})")
        sc = _gen_tensor(v["scale"], (E, rows, K // gs), f"{name}.scale")
        bi = _gen_tensor(v["bias"], (E, rows, K // gs), f"{name}.bias")
        if sc.dtype != bi.dtype:
            raise TypeError(f"{name}: scale and bias must share a dtype")
        return True, ops.dtype_code(sc.dtype, name), bits, gs, (words.contiguous(), sc, bi)
    st = _gen_tensor(v, (E, rows, K), name)
    return False, ops.dtype_code(st.dtype, name), 0, 0, (st,)


def _shared_dense(p: dict):
    """The shared expert's three matrices as dense tensors: int8 triplets are dequantized (once,
    memoised) to the bf16 weights the reference's loader makes of them
    (src/quanta/qwen35/artifact.py:105-115)."""
    wg, wu, wd = (p[k] for k in _SHARED_KEYS)
    if not isinstance(wg, dict):
        return wg, wu, wd

    def build():
        return tuple(ops.dequant(t["packed"].contiguous(), t["scale"].contiguous(),
                                 t["bias"].contiguous(), bits=int(t.get("bits", 8)),
                                 group_size=int(t.get("group_size", 64))) for t in (wg, wu, wd))
    return _memo(_anchor(wg), "shared_dense", (wg, wu, wd), build)


def _general_call(x: torch.Tensor, p: dict, cfg, topk: int, dense_all: bool, token_chunk: int):
    """qwen35_moe at the reference's own dtypes through qmoe_forward_general."""
    H, E = int(_cfg(cfg, "hidden_size")), int(_cfg(cfg, "num_experts"))
    I = int(_cfg(cfg, "moe_intermediate_size"))
    Is = int(_cfg(cfg, "shared_expert_intermediate_size", 0))
    scoring = str(_cfg(cfg, "scoring_func", "softmax"))
    if scoring not in _SCORING:
        raise ValueError(f"scoring_func {scoring!r} not supported (softmax | sigmoid | sqrtsoftplus)")
    if p.get("experts_mixed") is not None:
        raise TypeError("mixed-width experts need bf16 activations")
    c, w = L.QmoeGeneralConfig(), L.QmoeGeneralWeights()
    c.hidden, c.n_experts, c.top_k, c.inter = H, E, topk, I
    c.x_dtype = ops.dtype_code(x.dtype, "x")
    gate = _gen_tensor(p["gate"], (E, H), "gate")
    c.gate_dtype = ops.dtype_code(gate.dtype, "gate")
    gpk, gdt, gbits, ggs, gts = _gen_experts(p["experts_gate_up"], 2 * I, H, E, "experts_gate_up")
    dpk, ddt, dbits, dgs, dts = _gen_experts(p["experts_down"], H, I, E, "experts_down")
    if (gpk, gdt, gbits, ggs) != (dpk, ddt, dbits, dgs):
        raise ValueError("experts_gate_up and experts_down must share one format (packed or dense, "
                         "dtype, bits and group_size) on this path")
    c.experts_packed, c.expert_dtype, c.bits, c.group_size = int(gpk), gdt, gbits, ggs
    c.dense_all = int(dense_all)
    keep = [gate, *gts, *dts]
    w.gate = gate.data_ptr()
    if gpk:
        w.gu, w.gu_scale, w.gu_bias = (t.data_ptr() for t in gts)
        w.dn, w.dn_scale, w.dn_bias = (t.data_ptr() for t in dts)
    else:
        w.gu, w.dn = gts[0].data_ptr(), dts[0].data_ptr()
    has_shared = Is > 0 and p.get("shared_gate_proj") is not None
    if has_shared:
        wg, wu, wd = _shared_dense(p)
        wg = _gen_tensor(wg, (Is, H), "shared_gate_proj")
        wu = _gen_tensor(wu, (Is, H), "shared_up_proj")
        wd = _gen_tensor(wd, (H, Is), "shared_down_proj")
        if not wg.dtype == wu.dtype == wd.dtype:
            raise TypeError("shared expert: gate, up and down must share a dtype")
        c.shared_inter, c.shared_dtype = Is, ops.dtype_code(wg.dtype, "shared_gate_proj")
        w.sh_gate, w.sh_up, w.sh_down = wg.data_ptr(), wu.data_ptr(), wd.data_ptr()
        keep += [wg, wu, wd]
        sg = p.get("shared_expert_gate")
        if sg is not None:
            sg = _gen_tensor(sg.reshape(1, H), (1, H), "shared_expert_gate")
            c.shared_gated, c.shared_gate_dtype = 1, ops.dtype_code(sg.dtype, "shared_expert_gate")
            w.sh_expert_gate = sg.data_ptr()
            keep.append(sg)
    bias = p.get("e_score_correction_bias")
    if bias is not None:
        bias = bias.to(device=x.device, dtype=torch.float32).reshape(E).contiguous()
        w.router_bias = bias.data_ptr()
        keep.append(bias)
    c.scoring = _SCORING[scoring]
    c.norm_topk = norm_mode(cfg, scoring, bias is not None)
    c.n_group = int(_cfg(cfg, "n_group", 1))
    c.topk_group = int(_cfg(cfg, "topk_group", 1))
    c.routed_scale = float(_cfg(cfg, "routed_scaling_factor", 1.0))
    c.act, c.act_alpha, c.act_limit = gated_activation(cfg)
    b, s, _ = x.shape
    n = b * s
    xf = x.reshape(n, H).contiguous()
    y = torch.empty_like(xf)
    chunk = min(token_chunk if token_chunk and token_chunk > 0 else n, 65535)
    ws = None
    for c0 in range(0, n, chunk):
        c1 = min(c0 + chunk, n)
        ops.forward_general(c, w, xf[c0:c1], out=y[c0:c1], ws=ws)
    del keep
    return y.reshape(b, s, H)


def qwen35_moe(x: torch.Tensor, p: dict, cfg, *, sparse: bool = True, token_chunk: int = 8192,
               topk_override: int | None = None, regime: int = L.REGIME_AUTO) -> torch.Tensor:
    """Full MoE block: routed top-k experts + gated shared expert. `x` [B,S,H] -> [B,S,H].

    Mirrors `qwen35_moe` (src/quanta/qwen35/moe.py:154-202). `p` keys: gate [E,H];
    experts_gate_up / experts_down as packed triplet dicts {packed, scale, bias, group_size, bits}
    (int4 g64; or TiledExperts) or bf16 stacks [E,2I,H] / [E,H,I]; shared_gate_proj,
    shared_up_proj [Is,H]; shared_down_proj [H,Is] in bf16, or all three as the bake's int8
    triplets (same outputs as their bf16 dequant, half the bytes read); shared_expert_gate [1,H]
    (omit it for an ungated DeepSeek/GLM shared expert); optional e_score_correction_bias [E].
    `sparse=False` is the run-every-expert oracle and, as in the reference, refuses packed experts.
    Tokens beyond `token_chunk` are processed chunk by chunk (output-equivalent).

    bf16 activations over the formats above run the tiled MFMA kernels (qmoe_forward). Anything
    else the reference's block takes -- float32 activations, float32 weights or scale/bias, packed
    groups of 32 or code widths 2..8, dimensions that are not multiples of 128 -- runs
    qmoe_forward_general at the reference's own dtype flow (see `needs_general`).
    """
    if x.dim() != 3:
        raise ValueError("x must be [B, S, hidden]")
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"x must be bf16 or float32 (got {x.dtype})")
    b, s, hidden = x.shape
    n = b * s
    k_max = int(_cfg(cfg, "num_experts_per_tok"))
    topk = topk_override if topk_override is not None else k_max
    if topk < 1 or topk > k_max:
        raise ValueError(f"topk_override {topk_override} must be in [1, {k_max}]")
    packed = p.get("experts_mixed") is not None or _is_packed(p["experts_gate_up"])
    if not sparse and packed:
        raise ValueError("qwen35_moe(sparse=False) is the bf16 dense oracle; packed int4 experts "
                         "require sparse=True (gather_qmm). Refusing to dequant silently.")
    if needs_general(x, p, cfg):
        if n == 0:
            return x.clone()
        return _general_call(x, p, cfg, topk, not sparse, token_chunk)
    pr = prepare(p, cfg, topk=topk, regime=regime)
    xf = x.reshape(n, hidden).contiguous()
    if n == 0:
        return x.clone()
    if not sparse:
        return _routed_dense(xf, pr, topk).reshape(b, s, hidden)
    chunk = token_chunk if token_chunk and token_chunk > 0 else n
    chunk = min(chunk, 65535)
    y = torch.empty_like(xf)
    ws = torch.empty(max(ops.forward_workspace(pr.cfg, min(n, chunk)), 1), dtype=torch.uint8,
                     device=x.device)
    for c0 in range(0, n, chunk):
        c1 = min(c0 + chunk, n)
        ops.forward(pr.cfg, pr.weights, xf[c0:c1], out=y[c0:c1], ws=ws, mixed=pr.mixed)
    return y.reshape(b, s, hidden)


def qwen35_moe_residual(x: torch.Tensor, p: dict, cfg, norm_weight: torch.Tensor, *,
                        eps: float | None = None, sparse: bool = True, token_chunk: int = 8192,
                        topk_override: int | None = None,
                        regime: int = L.REGIME_AUTO) -> torch.Tensor:
    """The decoder layer's MoE half, x + qwen35_moe(post_attention_layernorm(x)), as one call.

    Mirrors `x = x + self.mlp(self.post_attention_layernorm(x), ...)`
    (src/quanta/qwen35/model.py:104-105; src/quanta/qwen35/batched_runtime.py:304-306).
    `norm_weight` [H] bf16 is nn.RMSNorm's resident weight (the checkpoint weight + 1,
    src/quanta/qwen35/runtime.py:57-63); `eps` defaults to the config's `norm_eps`. The norm is
    fp32 math rounded once to bf16 (the reference's own restatement, src/quanta/qwen35/
    attention.py:113-117), the block runs on the normalised rows, and the bf16 residual add is
    fused into the block's combine: y = bf16(x + bf16(block)). `sparse=False` runs the same norm
    and add around the run-every-expert oracle path.
    """
    if x.dim() != 3:
        raise ValueError("x must be [B, S, hidden]")
    if x.dtype != torch.bfloat16:
        raise TypeError(f"x must be bf16 (got {x.dtype}); the block computes on bf16 activations")
    b, s, hidden = x.shape
    if norm_weight.dtype != torch.bfloat16 or tuple(norm_weight.shape) != (hidden,):
        raise ValueError("norm_weight must be bf16 [hidden]")
    eps = float(_cfg(cfg, "norm_eps", 1e-6) if eps is None else eps)
    n = b * s
    if not sparse or n == 0:
        xf = x.reshape(n, hidden).contiguous()
        xn = ops.rmsnorm(xf, norm_weight.contiguous(), eps) if n else xf
        y = qwen35_moe(xn.reshape(b, s, hidden), p, cfg, sparse=sparse, token_chunk=token_chunk,
                       topk_override=topk_override, regime=regime)
        return (x.float() + y.float()).to(torch.bfloat16)
    k_max = int(_cfg(cfg, "num_experts_per_tok"))
    topk = topk_override if topk_override is not None else k_max
    if topk < 1 or topk > k_max:
        raise ValueError(f"topk_override {topk_override} must be in [1, {k_max}]")
    pr = prepare(p, cfg, topk=topk, regime=regime)
    xf = x.reshape(n, hidden).contiguous()
    nw = norm_weight.contiguous()
    chunk = token_chunk if token_chunk and token_chunk > 0 else n
    chunk = min(chunk, 65535)
    y = torch.empty_like(xf)
    ws = torch.empty(max(ops.forward_residual_workspace(pr.cfg, min(n, chunk)), 1),
                     dtype=torch.uint8, device=x.device)
    for c0 in range(0, n, chunk):
        c1 = min(c0 + chunk, n)
        ops.forward_residual(pr.cfg, pr.weights, xf[c0:c1], nw, eps, out=y[c0:c1], ws=ws)
    return y.reshape(b, s, hidden)


class Qwen35MoEModule(torch.nn.Module):
    """Module wrapper over :func:`qwen35_moe` holding the router, expert and shared params
    (src/quanta/qwen35/model.py:28-70).

    Differences, both from holding tensors eagerly on a GPU: the routed expert stacks start as
    None (the reference's `mx.zeros` stacks are lazy and never materialised before the loader
    sets them), and `set_experts` / `set_experts_packed` convert the stacks once into the
    resident MFMA-tiled layout (`TiledExperts`, still a dict for packed experts) instead of
    holding the caller's arrays, so a layer is resident once, not twice.
    """

    def __init__(self, cfg, *, device: torch.device | str | None = None,
                 dtype: torch.dtype = torch.bfloat16) -> None:
        super().__init__()
        self.cfg = cfg
        dev = torch.device(device) if device is not None else torch.device("cuda")
        h, e = int(_cfg(cfg, "hidden_size")), int(_cfg(cfg, "num_experts"))
        si = int(_cfg(cfg, "shared_expert_intermediate_size", 0))
        self.gate = torch.zeros(e, h, dtype=dtype, device=dev)
        self.experts_gate_up = None
        self.experts_down = None
        self.experts_mixed = None
        self.shared_gate_proj = torch.zeros(si, h, dtype=dtype, device=dev)
        self.shared_up_proj = torch.zeros(si, h, dtype=dtype, device=dev)
        self.shared_down_proj = torch.zeros(h, si, dtype=dtype, device=dev)
        self.shared_expert_gate = torch.zeros(1, h, dtype=dtype, device=dev)
        self.e_score_correction_bias = None
        self.token_chunk = 8192

    def set_experts(self, gate_up: torch.Tensor, down: torch.Tensor) -> None:
        """Expert stacks [E,2I,H] / [E,H,I] (src/quanta/qwen35/model.py:46-47): bf16 stacks are
        converted once to the tiled resident layout; float32 stacks are held as given (the
        reference-dtype path reads them natively)."""
        if gate_up.dtype == torch.bfloat16 and down.dtype == torch.bfloat16:
            gate_up, down = tile_experts_bf16(gate_up), tile_experts_bf16(down)
        self.experts_gate_up, self.experts_down = gate_up, down
        self.experts_mixed = None

    def set_experts_packed(self, gate_up: dict, down: dict) -> None:
        """Packed triplets {packed, scale, bias, group_size, bits} (src/quanta/qwen35/
        model.py:49-55). The tiled kernels' formats (bf16 scale/bias, int3/int4/int6, groups of
        64/128) are converted once to the tiled resident layout; other triplets (float32 scales,
        group 32, other widths) are held as given for the reference-dtype path."""
        if _fast_packed(gate_up) and _fast_packed(down):
            gate_up, down = tile_experts_packed(gate_up), tile_experts_packed(down)
        self.experts_gate_up, self.experts_down = gate_up, down
        self.experts_mixed = None

    def set_experts_mixed(self, stacks: dict, pbits: dict, pslot: dict, *, group_size: int = 128) -> None:
        """Widths per (expert, projection), as QuantizedSparseMoE.set_experts(stacks, pbits, pslot)
        (src/quanta/modeling/quantized.py:40-51); converted once to tiled stacks."""
        self.experts_mixed = tile_experts_mixed(stacks, pbits, pslot, group_size=group_size)
        self.experts_gate_up = self.experts_down = None

    def _params(self) -> dict:
        if self.experts_mixed is None and (self.experts_gate_up is None or self.experts_down is None):
            raise ValueError("experts not set: call set_experts, set_experts_packed or set_experts_mixed first")
        experts = ({"experts_mixed": self.experts_mixed} if self.experts_mixed is not None else
                   {"experts_gate_up": self.experts_gate_up, "experts_down": self.experts_down})
        p = {
            "gate": self.gate,
            **experts,
            "shared_gate_proj": self.shared_gate_proj,
            "shared_up_proj": self.shared_up_proj,
            "shared_down_proj": self.shared_down_proj,
            "shared_expert_gate": self.shared_expert_gate,
        }
        if self.e_score_correction_bias is not None:
            p["e_score_correction_bias"] = self.e_score_correction_bias
        return p

    def forward(self, x: torch.Tensor, *, sparse: bool = True,
                topk_override: int | None = None) -> torch.Tensor:
        return qwen35_moe(x, self._params(), self.cfg, sparse=sparse, token_chunk=self.token_chunk,
                          topk_override=topk_override)

    def forward_residual(self, x: torch.Tensor, norm_weight: torch.Tensor, *,
                         eps: float | None = None, sparse: bool = True,
                         topk_override: int | None = None) -> torch.Tensor:
        """x + self(post_attention_layernorm(x)) in one call (:func:`qwen35_moe_residual`)."""
        return qwen35_moe_residual(x, self._params(), self.cfg, norm_weight, eps=eps, sparse=sparse,
                                   token_chunk=self.token_chunk, topk_override=topk_override)
