"""CPU tier: the C-ABI library loads, exports every symbol include/quanta_moe.h declares, and
rejects bad arguments before touching the GPU (each call below fails validation, so no HIP work
is enqueued and nothing is dereferenced)."""

from __future__ import annotations

import ctypes

import pytest

from quanta_amd import _lib as L


def test_library_loads_and_abi_version():
    lib = L.load()
    assert lib.qmoe_abi_version() == L.ABI_VERSION == 10


def test_every_header_symbol_is_exported_and_bound():
    lib = L.load()
    declared = L.header_symbols()
    assert declared, "no symbols parsed from the header"
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in include/quanta_moe.h but not exported"
    assert sorted(L.SIGNATURES) == declared, "ctypes signature table out of sync with the header"


def test_struct_layouts_match_header_field_order():
    text = L.HEADER.read_text()
    for struct, name in ((L.QmoeConfig, "qmoe_config_t"), (L.QmoeWeights, "qmoe_weights_t")):
        body = text.split("typedef struct {", 1)[1] if name == "qmoe_config_t" else \
            text.split("typedef struct {", 2)[2]
        body = body.split("}", 1)[0]
        for fname, _ in struct._fields_:
            assert f" {fname};" in body, f"{name}.{fname} missing from header"


def _last_error() -> str:
    return L.load().qmoe_last_error().decode()


_DUMMY = ctypes.c_void_p(16)   # never dereferenced: each call fails validation first


@pytest.mark.parametrize("call, fragment", [
    (lambda lib: lib.qmoe_dequant(None, None, None, 4, 128, 5, 64, None, None), "bits 3, 4, 6 or 8"),
    (lambda lib: lib.qmoe_tile_int3(None, None, None, 1, 16, 96, 64, None, None, None), "in_features % 128"),
    (lambda lib: lib.qmoe_tile_int6(None, None, None, 1, 16, 100, 64, None, None, None), "in_features % 128"),
    (lambda lib: lib.qmoe_dequant(None, None, None, 4, 100, 4, 64, None, None), "in_features"),
    (lambda lib: lib.qmoe_tile_int4(None, None, None, 1, 15, 128, 64, None, None, None), "rows % 16"),
    (lambda lib: lib.qmoe_tile_bf16(None, 1, 16, 33, None, None), "in_features % 32"),
    (lambda lib: lib.qmoe_permute(None, 0, 2, 16, 16, None, None, None, None, None, None, 0, None),
     "N,k"),
    (lambda lib: lib.qmoe_permute(None, 4, 2, 2000, 16, None, None, None, None, None, None, 0, None),
     "E <= 1024"),
    (lambda lib: lib.qmoe_router_topk(None, 16, None, 4, 16, 17, 0, 1, 1, 1, 1.0, 0, None, None, None,
                                      None), "k <= min"),
    (lambda lib: lib.qmoe_router_topk(None, 16, None, 4, 16, 2, 0, 3, 1, 1, 1.0, 0, None, None, None,
                                      None), "n_group"),
    (lambda lib: lib.qmoe_router_topk(None, 16, None, 4, 16, 8, 1, 8, 2, 1, 1.0, 0, None, None, None,
                                      None), "kept groups"),
    (lambda lib: lib.qmoe_combine(None, None, None, 4, 2, 100, None, None, None, None), "H % 8"),
    (lambda lib: lib.qmoe_grouped_qmm(None, 1, None, 1, 1, None, None, None, 1, 1, 128, 16, 0, None,
                                      None, None, 0, 0, 1.0, 0.0, None, 16, 1, None, 0, None),
     "null pointer"),
    (lambda lib: lib.qmoe_grouped_qmm(_DUMMY, 1, None, 1, 1, None, None, None, 1, 1, 128, 32, 1,
                                      _DUMMY, None, None, 0, 2, 1.0, 0.0, _DUMMY, 16, 1, None, 0,
                                      None), "act_limit"),
    (lambda lib: lib.qmoe_grouped_qmm(_DUMMY, 1, None, 1, 1, None, None, None, 1, 1, 128, 32, 1,
                                      _DUMMY, None, None, 0, 5, 1.0, 7.0, _DUMMY, 16, 1, None, 0,
                                      None), "unknown act"),
    (lambda lib: lib.qmoe_grouped_qmm(_DUMMY, 1, None, 1, 1, None, None, None, 1, 1, 128, 256, 0,
                                      _DUMMY, _DUMMY, None, 1, 0, 1.0, 0.0, _DUMMY, 256, 2, None,
                                      0, None), "need row_exp"),
    (lambda lib: lib.qmoe_row_exponents(None, None, 1, 16, 128, 4, 64, None, None), "null pointer"),
    (lambda lib: lib.qmoe_forward_noalloc(None, None, None, 1, None, None), "null pointer"),
    (lambda lib: lib.qmoe_row_exponents(_DUMMY, _DUMMY, 1, 16, 100, 4, 64, _DUMMY, None),
     "group_size"),
    (lambda lib: lib.qmoe_dequant(None, None, None, 4, 128, 4, 32, None, None), "group_size 64 or 128"),
    (lambda lib: lib.qmoe_tile_int4(None, None, None, 1, 16, 128, 32, None, None, None), "64 or 128"),
    (lambda lib: lib.qmoe_tile_int8(None, None, None, 1, 16, 96, 64, None, None, None), "in_features % 64"),
    (lambda lib: lib.qmoe_tile_int8(None, None, None, 1, 8, 128, 64, None, None, None), "rows % 16"),
    (lambda lib: lib.qmoe_tile_int8(_DUMMY, _DUMMY, _DUMMY, 1, 16, 128, 64, None, _DUMMY, None),
     "null pointer"),
    (lambda lib: lib.qmoe_grouped_qmm(_DUMMY, 1, None, 1, 1, None, None, None, 1, 1, 128, 32, 4,
                                      _DUMMY, None, None, 1, 0, 1.0, 0.0, _DUMMY, 32, 1, None, 0,
                                      None), "quantized weights need sb"),
    (lambda lib: lib.qmoe_grouped_qmm(_DUMMY, 1, None, 1, 1, None, None, None, 1, 1, 128, 32, 5,
                                      _DUMMY, _DUMMY, None, 1, 0, 1.0, 0.0, _DUMMY, 32, 1, None, 0,
                                      None), "bad weight_format"),
])
def test_invalid_arguments_rejected(call, fragment):
    rc = call(L.load())
    assert rc == L.QMOE_EINVAL
    assert fragment in _last_error()


def test_forward_rejects_bad_config():
    lib = L.load()
    cfg = L.QmoeConfig(hidden=100, n_experts=16, top_k=2, inter=128, shared_inter=0, scoring=0,
                       norm_topk=1, n_group=1, topk_group=1, routed_scale=1.0, expert_format=0,
                       router_format=1, router_rows=0, shared_gated=0, regime=0)
    w = L.QmoeWeights()
    dummy = ctypes.c_void_p(16)
    rc = lib.qmoe_forward(ctypes.byref(cfg), ctypes.byref(w), dummy, 4, dummy, dummy, 1 << 20, None)
    assert rc == L.QMOE_EINVAL and "hidden % 128" in _last_error()
    assert lib.qmoe_forward_workspace(ctypes.byref(cfg), 0) == 0


def test_workspace_grows_with_tokens():
    lib = L.load()
    cfg = L.QmoeConfig(hidden=4096, n_experts=512, top_k=10, inter=1024, shared_inter=1024,
                       scoring=0, norm_topk=1, n_group=1, topk_group=1, routed_scale=1.0,
                       expert_format=0, router_format=0, router_rows=640, shared_gated=1, regime=0)
    a = lib.qmoe_forward_workspace(ctypes.byref(cfg), 1)
    b = lib.qmoe_forward_workspace(ctypes.byref(cfg), 128)
    assert 0 < a < b
    # h (mc*I bf16) + d (mc*H bf16) dominate
    assert b >= 128 * 10 * (1024 + 4096) * 2
    # the residual entry adds the normalised rows (N*H bf16, 256-byte aligned) after them
    for n in (1, 3, 128):
        assert (lib.qmoe_forward_residual_workspace(ctypes.byref(cfg), n)
                == lib.qmoe_forward_workspace(ctypes.byref(cfg), n) + (n * 4096 * 2 + 255) // 256 * 256)
    assert lib.qmoe_forward_residual_workspace(ctypes.byref(cfg), 0) == 0


def test_ops_refuse_cpu_tensors():
    import torch
    from quanta_amd import ops

    with pytest.raises(ValueError, match="GPU tensor"):
        ops.tile_bf16(torch.zeros(16, 32, dtype=torch.bfloat16))


def test_forward_rejects_mixed_bf16_and_unknown_down_format():
    lib = L.load()
    base = dict(hidden=512, n_experts=16, top_k=2, inter=128, shared_inter=0, scoring=0, norm_topk=1,
                n_group=1, topk_group=1, routed_scale=1.0, router_format=1, router_rows=0,
                shared_gated=0, regime=0)
    w = L.QmoeWeights()
    dummy = ctypes.c_void_p(16)
    for ef, df, frag in ((L.FMT_INT3_G64, L.FMT_BF16, "both be quantized or both bf16"),
                         (L.FMT_INT4_G64, 7, "down_format must be"),
                         (L.FMT_INT3_G64, L.FMT_INT4_G64, None)):
        cfg = L.QmoeConfig(expert_format=ef, down_format=df, **base)
        if frag is None:   # a valid mix, in either regime: the workspace query accepts it
            assert lib.qmoe_forward_workspace(ctypes.byref(cfg), 4) > 0
            cfg.regime = L.REGIME_LARGE
            assert lib.qmoe_forward_workspace(ctypes.byref(cfg), 4) > 0
            continue
        rc = lib.qmoe_forward(ctypes.byref(cfg), ctypes.byref(w), dummy, 4, dummy, dummy, 1 << 20, None)
        assert rc == L.QMOE_EINVAL and frag in _last_error(), _last_error()


def test_forward_large_int4_needs_row_exponents():
    """The prefill kernels' fp16 dequant scales each weight row by its exponent (row_exponents):
    an int4 call that reaches the large regime without them is rejected before any launch."""
    lib = L.load()
    cfg = L.QmoeConfig(hidden=512, n_experts=16, top_k=2, inter=256, shared_inter=0, scoring=0,
                       norm_topk=1, n_group=1, topk_group=1, routed_scale=1.0, expert_format=0,
                       router_format=1, router_rows=0, shared_gated=0, regime=L.REGIME_LARGE)
    w = L.QmoeWeights()
    dummy = ctypes.c_void_p(16)
    for f in ("router_w", "gu_codes", "gu_sb", "dn_codes", "dn_sb"):
        setattr(w, f, dummy.value)
    rc = lib.qmoe_forward(ctypes.byref(cfg), ctypes.byref(w), dummy, 4, dummy, dummy, 1 << 20, None)
    assert rc == L.QMOE_EINVAL and "gu_rexp and dn_rexp" in _last_error(), _last_error()


def test_forward_rejects_bad_shared_format():
    """shared_format must be named (bf16 or int8 g64); an int8 shared expert needs its scale/bias
    arrays; the large-M regime's expanded bf16 copy is part of the workspace."""
    lib = L.load()
    base = dict(hidden=512, n_experts=16, top_k=2, inter=128, shared_inter=256, scoring=0,
                norm_topk=1, n_group=1, topk_group=1, routed_scale=1.0, router_format=1,
                router_rows=0, shared_gated=0, regime=0, expert_format=0, down_format=0)
    dummy = ctypes.c_void_p(16)
    w = L.QmoeWeights(router_w=16, gu_codes=16, gu_sb=16, dn_codes=16, dn_sb=16, sh_gu=16, sh_dn=16)
    for fmt, frag in ((L.FMT_INT4_G64, "shared_format must be"), (L.FMT_INT6_G64, "shared_format must be"),
                      (L.FMT_INT8_G64, "needs sh_gu_sb and sh_dn_sb")):
        cfg = L.QmoeConfig(shared_format=fmt, **base)
        rc = lib.qmoe_forward(ctypes.byref(cfg), ctypes.byref(w), dummy, 4, dummy, dummy, 1 << 30, None)
        assert rc == L.QMOE_EINVAL and frag in _last_error(), _last_error()
    assert L.QmoeConfig().shared_format == L.FMT_BF16
    c16 = L.QmoeConfig(shared_format=L.FMT_BF16, **base)
    c8 = L.QmoeConfig(shared_format=L.FMT_INT8_G64, **base)
    for n in (1, 64, 256):
        assert lib.qmoe_forward_workspace(ctypes.byref(c8), n) == lib.qmoe_forward_workspace(ctypes.byref(c16), n)
    extra = 3 * 256 * 512 * 2
    assert (lib.qmoe_forward_workspace(ctypes.byref(c8), 300)
            == lib.qmoe_forward_workspace(ctypes.byref(c16), 300) + extra)


def test_forward_rejects_bad_awq_config():
    lib = L.load()
    base = dict(hidden=512, n_experts=16, top_k=2, inter=128, shared_inter=0, scoring=0, norm_topk=1,
                n_group=1, topk_group=1, routed_scale=1.0, router_format=1, router_rows=0,
                shared_gated=0)
    dummy = ctypes.c_void_p(16)
    w = L.QmoeWeights()
    for kw, frag in ((dict(expert_format=L.FMT_BF16, down_format=L.FMT_BF16, awq=1, regime=0),
                      "awq scales need quantized experts"),
                     (dict(expert_format=0, down_format=0, awq=1, regime=L.REGIME_LARGE),
                      "awq scales in the large regime need inter % 256 == 0"),
                     (dict(expert_format=0, down_format=0, awq=2, regime=0), "awq must be 0 or 1")):
        cfg = L.QmoeConfig(**kw, **base)
        rc = lib.qmoe_forward(ctypes.byref(cfg), ctypes.byref(w), dummy, 4, dummy, dummy, 1 << 20, None)
        assert rc == L.QMOE_EINVAL and frag in _last_error(), _last_error()
    # awq adds the prescaled rows [2][mc][H] and the gate|up outputs [mc][2I] to the workspace
    cfg0 = L.QmoeConfig(expert_format=0, down_format=0, awq=0, regime=0, **base)
    cfg1 = L.QmoeConfig(expert_format=0, down_format=0, awq=1, regime=0, **base)
    extra = lib.qmoe_forward_workspace(ctypes.byref(cfg1), 5) - lib.qmoe_forward_workspace(ctypes.byref(cfg0), 5)
    assert extra >= 2 * 10 * 512 * 2 + 10 * 256 * 2


def test_decode_flow_mode_switch_returns_previous():
    lib = L.load()
    assert lib.qmoe_set_decode_flow(0) == 1
    assert lib.qmoe_set_decode_flow(1) == 0
    assert lib.qmoe_set_decode_flow(2) == 1
    assert lib.qmoe_set_decode_flow(7) == 2   # unknown modes leave the mode as it was
    assert lib.qmoe_set_decode_flow(1) == 2


def _general_cfg(**kw) -> L.QmoeGeneralConfig:
    base = dict(hidden=32, n_experts=8, top_k=3, inter=64, shared_inter=64, scoring=0, norm_topk=1,
                n_group=1, topk_group=1, routed_scale=1.0, act=0, act_alpha=1.702,
                act_limit=float("inf"), x_dtype=L.DT_F32, gate_dtype=L.DT_F32, experts_packed=1,
                expert_dtype=L.DT_F32, bits=4, group_size=32, shared_dtype=L.DT_F32, shared_gated=1,
                shared_gate_dtype=L.DT_F32, dense_all=0)
    base.update(kw)
    return L.QmoeGeneralConfig(**base)


@pytest.mark.parametrize("kw, fragment", [
    (dict(bits=7), "bits must be"),
    (dict(group_size=16), "group_size must be 32, 64 or 128"),
    (dict(hidden=48), "multiples of group_size"),
    (dict(x_dtype=5), "dtypes must be"),
    (dict(experts_packed=1, dense_all=1), "dense stacks only"),
    (dict(top_k=9), "k <= min"),
    (dict(act=1, act_limit=0.0), "act_limit"),
    (dict(inter=0), "inter > 0"),
])
def test_forward_general_rejects_bad_config(kw, fragment):
    """qmoe_forward_general validates the whole configuration before it enqueues anything."""
    lib = L.load()
    cfg = _general_cfg(**kw)
    w = L.QmoeGeneralWeights(gate=16, gu=16, dn=16, gu_scale=16, gu_bias=16, dn_scale=16,
                             dn_bias=16, sh_gate=16, sh_up=16, sh_down=16, sh_expert_gate=16)
    rc = lib.qmoe_forward_general(ctypes.byref(cfg), ctypes.byref(w), _DUMMY, 4, _DUMMY, _DUMMY,
                                  1 << 24, None)
    assert rc == L.QMOE_EINVAL and fragment in _last_error(), _last_error()


def test_forward_general_null_and_workspace():
    lib = L.load()
    cfg = _general_cfg()
    w = L.QmoeGeneralWeights()
    rc = lib.qmoe_forward_general(ctypes.byref(cfg), ctypes.byref(w), _DUMMY, 4, _DUMMY, _DUMMY,
                                  1 << 24, None)
    assert rc == L.QMOE_EINVAL and "missing weights" in _last_error()
    rc = lib.qmoe_forward_general(None, ctypes.byref(w), _DUMMY, 4, _DUMMY, _DUMMY, 1 << 24, None)
    assert rc == L.QMOE_EINVAL and "null pointer" in _last_error()
    small = lib.qmoe_forward_general_workspace(ctypes.byref(cfg), 9)
    big = lib.qmoe_forward_general_workspace(ctypes.byref(cfg), 900)
    assert 0 < small < big
    dense = _general_cfg(experts_packed=0, dense_all=1)
    # the run-every-expert form holds E slots per token instead of k
    assert lib.qmoe_forward_general_workspace(ctypes.byref(dense), 9) > small
    w = L.QmoeGeneralWeights(gate=16, gu=16, dn=16, gu_scale=16, gu_bias=16, dn_scale=16,
                             dn_bias=16, sh_gate=16, sh_up=16, sh_down=16, sh_expert_gate=16)
    rc = lib.qmoe_forward_general(ctypes.byref(cfg), ctypes.byref(w), _DUMMY, 9, _DUMMY, _DUMMY,
                                  small - 1, None)
    assert rc == L.QMOE_EINVAL and "workspace too small" in _last_error()


def test_struct_offsets_match_the_c_compiler(tmp_path):
    """Every ctypes struct has the C compiler's field offsets and size for the header's struct."""
    import shutil
    import subprocess

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    structs = [(L.QmoeConfig, "qmoe_config_t"), (L.QmoeWeights, "qmoe_weights_t"),
               (L.QmoeStack, "qmoe_stack_t"), (L.QmoeMixed, "qmoe_mixed_t"),
               (L.QmoeGeneralConfig, "qmoe_general_config_t"),
               (L.QmoeGeneralWeights, "qmoe_general_weights_t")]
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{L.HEADER}"', "int main(void) {"]
    for st, cname in structs:
        lines.append(f'  printf("{cname} %zu\\n", sizeof({cname}));')
        for fname, _ in st._fields_:
            lines.append(f'  printf("{cname}.{fname} %zu\\n", offsetof({cname}, {fname}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "offsets.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "offsets"
    subprocess.run([gcc, "-std=c11", str(src), "-o", str(exe)], check=True)
    out = dict(line.rsplit(" ", 1) for line in subprocess.run(
        [str(exe)], check=True, capture_output=True, text=True).stdout.splitlines())
    for st, cname in structs:
        assert int(out[cname]) == ctypes.sizeof(st), cname
        for fname, _ in st._fields_:
            assert int(out[f"{cname}.{fname}"]) == getattr(st, fname).offset, f"{cname}.{fname}"


@pytest.mark.parametrize("args, fragment", [
    (dict(H=100), "H % 8"),
    (dict(k=17), "k <= min"),
    (dict(wr_is_f32=2), "wr_is_f32"),
    (dict(N=0), "0 < N"),
    (dict(ws_bytes=16), "workspace too small"),
    (dict(norm_topk=3), "norm_topk"),
    (dict(x=ctypes.c_void_p(24)), "16-byte aligned"),
])
def test_router_one_call_validation(args, fragment):
    lib = L.load()
    a = dict(x=ctypes.c_void_p(256), wr=ctypes.c_void_p(256), wr_is_f32=0, sg=None, bias=None, N=4,
             H=256, E=16, k=2, scoring=0, n_group=1, topk_group=1, norm_topk=1, scale=1.0,
             idx=_DUMMY, w=_DUMMY, sg_out=None, ws=_DUMMY, ws_bytes=1 << 20)
    a.update(args)
    rc = lib.qmoe_router(a["x"], a["wr"], a["wr_is_f32"], a["sg"], a["bias"], a["N"], a["H"], a["E"],
                         a["k"], a["scoring"], a["n_group"], a["topk_group"], a["norm_topk"],
                         a["scale"], a["idx"], a["w"], a["sg_out"], a["ws"], a["ws_bytes"], None)
    assert rc == L.QMOE_EINVAL and fragment in _last_error(), _last_error()
    assert lib.qmoe_router_workspace(4, 16) >= 4 * 17 * 4
