"""Shared helpers for the GPU parity tests: numpy <-> torch conversion of bf16/word data and the
tolerance metrics the BASELINE parity gates use."""

from __future__ import annotations

import numpy as np
import torch

from oracle import quant as oq

# BASELINE parity gates for the bf16 layer output
MAX_ABS = 2e-2
REL_L2 = 5e-3


def bf16_dev(bits: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(dev)


def words_dev(words: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(words).view(np.int32)).to(dev)


def bits_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().view(torch.int16).numpy().astype(np.uint16)


def f64(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def words_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().numpy().view(np.uint32)


def metrics(got: np.ndarray, want: np.ndarray) -> tuple[float, float]:
    """(max-abs error scaled by max(1, max|want|), relative L2 error).

    The max-abs gate is absolute for outputs up to magnitude 1 and relative to the output's
    largest magnitude beyond that, as the reference's own bf16 gates measure it
    (`_relmax` = max|a-b| / max|b|, parity/bf16_scale_g64_test.py:24-25): one bf16 ulp of an
    output of magnitude 8 is already 0.031, so a purely absolute 2e-2 bound would reject
    correctly rounded results."""
    want = want.astype(np.float64)
    d = got.astype(np.float64) - want
    scale = max(1.0, float(np.max(np.abs(want)))) if want.size else 1.0
    max_abs = float(np.max(np.abs(d))) / scale if d.size else 0.0
    rel = float(np.linalg.norm(d) / max(np.linalg.norm(want), 1e-30))
    return max_abs, rel


def raw_max_abs(got, want) -> float:
    """The unscaled max |got - want|, reported beside the scaled gate figure."""
    d = np.asarray(got, np.float64) - np.asarray(want, np.float64)
    return float(np.max(np.abs(d))) if d.size else 0.0


# Below these output magnitudes the raw (unscaled) max-abs gate, |got - want| <= max_abs, is
# asserted as well. The bf16 output carries half an ulp of rounding, and the reference's bf16
# intermediates (gate/up, h, d) flip to the neighbouring bf16 value wherever float32 and float64
# evaluation straddle a rounding boundary, each flip moving the output by up to an ulp of that
# intermediate. Below 2 an ulp is 2^-7, so a correct result sits far inside 2e-2 even with
# flips; below 4 (ulp 2^-6) it still does at the BASELINE shapes and inputs (x ~ N(0,1), weights
# N(0,0.02); _full_parity passes raw_peak=4), while the stress layers of the format tests (x
# scaled by 4) can sum two flips to 1.5 ulps there. Above, the gate scales with max|want|.
RAW_GATE_PEAK = 2.0
RAW_GATE_PEAK_BASELINE = 4.0


def assert_close(got, want, what="", max_abs=MAX_ABS, rel_l2=REL_L2, want_rounded=False,
                 raw_peak=RAW_GATE_PEAK):
    """`want` should be the oracle's unrounded (float64) result: the GPU's bf16 output then
    carries exactly one rounding, not two. want_rounded: `want` is itself a bf16 output (another
    path of this build), which caps the raw gate at RAW_GATE_PEAK.

    Asserts the scaled max-abs and relative-L2 gates always, and the raw max-abs gate (the
    north-star bound as written) whenever max|want| lies below raw_peak."""
    ma, rl = metrics(got, want)
    raw = raw_max_abs(got, want)
    peak = float(np.max(np.abs(want))) if np.size(want) else 0.0
    raw_on = peak < (min(raw_peak, RAW_GATE_PEAK) if want_rounded else raw_peak)
    print(f"[parity] {what}: max_abs(scaled)={ma:.3e} max_abs(raw)={raw:.3e} max|want|={peak:.3g} "
          f"rel_l2={rl:.3e} raw_gate={'on' if raw_on else 'off'}", flush=True)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    assert ma <= max_abs and rl <= rel_l2, f"{what}: max_abs={ma:.3e} rel_l2={rl:.3e}"
    if raw_on:
        assert raw <= max_abs, f"{what}: raw max_abs={raw:.3e} > {max_abs:g} (max|want|={peak:.3g})"


def oracle_params_from_torch(p: dict) -> dict:
    """Reference-keyed torch parameter dict (any device) -> the oracle's numpy parameters."""
    out = {"gate": f64(p["gate"])}
    for pre, key in (("gu", "experts_gate_up"), ("dn", "experts_down")):
        out[f"{pre}_packed"] = words_np(p[key]["packed"])
        out[f"{pre}_scale"] = bits_np(p[key]["scale"])
        out[f"{pre}_bias"] = bits_np(p[key]["bias"])
    for k in ("shared_gate_proj", "shared_up_proj", "shared_down_proj", "shared_expert_gate"):
        v = p.get(k)
        if isinstance(v, dict):   # the bake's int8 shared-expert triplet
            out[k] = {"packed": words_np(v["packed"]), "scale": bits_np(v["scale"]),
                      "bias": bits_np(v["bias"]), "group_size": int(v.get("group_size", 64)),
                      "bits": int(v.get("bits", 8))}
        elif v is not None:
            out[k] = f64(v)
    if p.get("e_score_correction_bias") is not None:
        out["e_score_correction_bias"] = f64(p["e_score_correction_bias"])
    for pre, key in (("gu", "experts_gate_up"), ("dn", "experts_down")):
        if p[key].get("awq_scale") is not None:
            out[f"{pre}_awq"] = f64(p[key]["awq_scale"])
    return out


def near_tie_rows(margin: np.ndarray, logits_scale: np.ndarray, tol: float = 1e-5) -> np.ndarray:
    """Rows whose top-k boundary gap is within float32 evaluation error of the router logits."""
    return margin <= tol * np.maximum(logits_scale, 1.0)


def route_sets_equal(a: np.ndarray, b: np.ndarray) -> bool:
    return all(set(x) == set(y) for x, y in zip(a.tolist(), b.tolist()))


__all__ = ["bf16_dev", "words_dev", "bits_np", "f64", "words_np", "metrics", "raw_max_abs", "assert_close",
           "oracle_params_from_torch", "near_tie_rows", "route_sets_equal", "oq"]
