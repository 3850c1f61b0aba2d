"""torch-facing wrappers of the C ABI (one function per entry point of include/quanta_moe.h).

Tensors must be CUDA (HIP) tensors, contiguous, with the dtypes each function names. bf16 data is
passed as torch.bfloat16; packed int4 words as torch.int32 (or torch.uint32) holding the uint32
bit patterns. Every call enqueues on torch's current stream of the tensor's device and returns
without synchronising. Argument errors raise ValueError; HIP launch errors raise RuntimeError.
"""

from __future__ import annotations

import ctypes

import torch

from quanta_amd import _lib as L


def _stream(dev: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _p(t: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _need(t: torch.Tensor, dtypes, name: str) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name}: must be a GPU tensor (no CPU fallback exists)")
    if not isinstance(dtypes, tuple):
        dtypes = (dtypes,)
    if t.dtype not in dtypes:
        raise TypeError(f"{name}: dtype {t.dtype} not in {dtypes}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")
    return t


def _words(t: torch.Tensor, name: str) -> torch.Tensor:
    _need(t, (torch.int32, torch.uint32), name)
    return t.view(torch.int32) if t.dtype == torch.uint32 else t


# ------------------------------------------------------------------------------- formats


def dequant(packed: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor, *, bits: int = 4,
            group_size: int = 64) -> torch.Tensor:
    """Native affine int4 (or int6 / int8, bits=6 / 8) stack [..., rows, K*bits/32], group 64 or 128 ->
    bf16 [..., rows, K] (bit-exact: bf16(fma(s, q, b)))."""
    packed = _words(packed, "packed")
    _need(scale, torch.bfloat16, "scale")
    _need(bias, torch.bfloat16, "bias")
    if bits not in (3, 4, 6, 8):
        raise ValueError("dequant: bits must be 3, 4, 6 or 8")
    if (packed.shape[-1] * 32) % bits:
        raise ValueError("dequant: packed words do not hold a whole number of codes")
    K = packed.shape[-1] * 32 // bits
    if scale.shape != bias.shape or scale.shape[:-1] != packed.shape[:-1] or scale.shape[-1] * group_size != K:
        raise ValueError("dequant: shape mismatch between packed words and scale/bias")
    rows = packed.numel() // packed.shape[-1]
    out = torch.empty(*packed.shape[:-1], K, dtype=torch.bfloat16, device=packed.device)
    L.check(L.load().qmoe_dequant(_p(packed), _p(scale), _p(bias), rows, K, bits, group_size,
                                  _p(out), _stream(packed.device)), "qmoe_dequant")
    return out


def tile_int4(packed: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor, *,
              group_size: int = 64) -> tuple[torch.Tensor, torch.Tensor]:
    """Native stack [E, rows, K/8] (+ scale/bias [E, rows, K/group_size], group 64 or 128) ->
    MFMA-tiled (codes, sb); sb holds one (scale, bias) per 64 columns either way."""
    packed = _words(packed, "packed")
    _need(scale, torch.bfloat16, "scale")
    _need(bias, torch.bfloat16, "bias")
    if packed.dim() == 2:
        packed, scale, bias = packed[None], scale[None], bias[None]
    if packed.dim() != 3:
        raise ValueError("tile_int4: expected [E, rows, K/8]")
    E, rows, W = packed.shape
    K = W * 8
    if group_size not in (64, 128):
        raise ValueError("tile_int4: group_size must be 64 or 128")
    if scale.shape != (E, rows, K // group_size) or bias.shape != scale.shape:
        raise ValueError(f"tile_int4: scale/bias must be [E, rows, K/{group_size}]")
    codes = torch.empty(E * rows * W, dtype=torch.int32, device=packed.device)
    sb = torch.empty(E * rows * (K // 64) * 2, dtype=torch.bfloat16, device=packed.device)
    L.check(L.load().qmoe_tile_int4(_p(packed), _p(scale), _p(bias), E, rows, K, group_size,
                                    _p(codes), _p(sb), _stream(packed.device)), "qmoe_tile_int4")
    return codes, sb


def row_exponents(scale: torch.Tensor, bias: torch.Tensor, *, bits: int = 4,
                  group_size: int = 64) -> torch.Tensor:
    """Per weight row of a native stack's scale/bias [E, rows, K/group_size] (bf16): the int8
    power-of-two exponent the prefill kernels scale the row's fp16 weights by
    (qmoe_row_exponents)."""
    _need(scale, torch.bfloat16, "scale")
    _need(bias, torch.bfloat16, "bias")
    if scale.dim() == 2:
        scale, bias = scale[None], bias[None]
    if scale.dim() != 3 or bias.shape != scale.shape:
        raise ValueError("row_exponents: scale/bias must be [E, rows, groups]")
    E, rows, G = scale.shape
    out = torch.empty(E, rows, dtype=torch.int8, device=scale.device)
    L.check(L.load().qmoe_row_exponents(_p(scale), _p(bias), E, rows, G * group_size, bits,
                                        group_size, _p(out), _stream(scale.device)),
            "qmoe_row_exponents")
    return out


def _tile_narrow(packed: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor, bits: int,
                 group_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Native int3/int6/int8 stack [E, rows, K*bits/32] (+ scale/bias [E, rows, K/group_size]) ->
    the tiled layout of the decode kernel (codes: the same byte count; int3/int6 the planes of the
    code bits per tile superblock, int8 one byte per weight in the bf16 tiling's order; sb as
    tile_int4)."""
    packed = _words(packed, "packed")
    _need(scale, torch.bfloat16, "scale")
    _need(bias, torch.bfloat16, "bias")
    if packed.dim() == 2:
        packed, scale, bias = packed[None], scale[None], bias[None]
    if packed.dim() != 3:
        raise ValueError(f"tile_int{bits}: expected [E, rows, K*{bits}/32]")
    E, rows, W = packed.shape
    if (W * 32) % bits:
        raise ValueError(f"tile_int{bits}: packed words do not hold a whole number of codes")
    K = W * 32 // bits
    if group_size not in (64, 128):
        raise ValueError(f"tile_int{bits}: group_size must be 64 or 128")
    if scale.shape != (E, rows, K // group_size) or bias.shape != scale.shape:
        raise ValueError(f"tile_int{bits}: scale/bias must be [E, rows, K/{group_size}]")
    if packed.data_ptr() % 16:   # (the int8 tiling reads 8-byte pieces of the rows)
        packed = packed.clone()
    codes = torch.empty(E * rows * W, dtype=torch.int32, device=packed.device)
    sb = torch.empty(E * rows * (K // 64) * 2, dtype=torch.bfloat16, device=packed.device)
    fn = {6: L.load().qmoe_tile_int6, 3: L.load().qmoe_tile_int3, 8: L.load().qmoe_tile_int8}[bits]
    L.check(fn(_p(packed), _p(scale), _p(bias), E, rows, K, group_size, _p(codes), _p(sb),
               _stream(packed.device)), f"qmoe_tile_int{bits}")
    return codes, sb


def tile_int6(packed: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor, *,
              group_size: int = 64) -> tuple[torch.Tensor, torch.Tensor]:
    """Native int6 stack -> the decode kernel's tiled int6 layout (qmoe_tile_int6)."""
    return _tile_narrow(packed, scale, bias, 6, group_size)


def tile_int8(packed: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor, *,
              group_size: int = 64) -> tuple[torch.Tensor, torch.Tensor]:
    """Native int8 matrix [rows, K/4] or stack [E, rows, K/4] -> the tiled int8 layout the dense
    kernels dequantize in registers (qmoe_tile_int8): the bake's int8 shared expert."""
    return _tile_narrow(packed, scale, bias, 8, group_size)


def tile_int3(packed: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor, *,
              group_size: int = 64) -> tuple[torch.Tensor, torch.Tensor]:
    """Native int3 stack -> the decode kernel's tiled int3 layout (qmoe_tile_int3)."""
    return _tile_narrow(packed, scale, bias, 3, group_size)


def dequant_tiled(codes: torch.Tensor, sb: torch.Tensor, n_mats: int, rows: int,
                  K: int) -> torch.Tensor:
    """MFMA-tiled int4 stack -> bf16 [n_mats, rows, K] (bit-identical to dequant of the native
    stack it was tiled from)."""
    codes = _words(codes, "codes")
    _need(sb, torch.bfloat16, "sb")
    if codes.numel() != n_mats * rows * K // 8 or sb.numel() != n_mats * rows * (K // 64) * 2:
        raise ValueError("dequant_tiled: sizes do not match n_mats/rows/K")
    out = torch.empty(n_mats, rows, K, dtype=torch.bfloat16, device=codes.device)
    L.check(L.load().qmoe_dequant_tiled(_p(codes), _p(sb), n_mats, rows, K, _p(out),
                                        _stream(codes.device)), "qmoe_dequant_tiled")
    return out


def tile_bf16(w: torch.Tensor) -> torch.Tensor:
    """Row-major bf16 [..., rows, K] -> MFMA-tiled flat bf16 tensor of the same size."""
    _need(w, torch.bfloat16, "w")
    rows, K = w.shape[-2], w.shape[-1]
    n = w.numel() // (rows * K)
    out = torch.empty(w.numel(), dtype=torch.bfloat16, device=w.device)
    L.check(L.load().qmoe_tile_bf16(_p(w), n, rows, K, _p(out), _stream(w.device)),
            "qmoe_tile_bf16")
    return out


# ------------------------------------------------------------------------------- block steps


def router_logits_f32(x: torch.Tensor, wr: torch.Tensor,
                      shared_gate: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 router logits [N, E+1] (column E = x . shared_gate when given, else unused)."""
    _need(x, torch.bfloat16, "x")
    _need(wr, torch.float32, "wr")
    N, H = x.shape
    E = wr.shape[0]
    if wr.shape != (E, H):
        raise ValueError("router_logits_f32: wr must be [E, H]")
    if shared_gate is not None:
        _need(shared_gate, torch.float32, "shared_gate")
        if shared_gate.numel() != H:
            raise ValueError("router_logits_f32: shared_gate must have H elements")
    out = torch.zeros(N, E + 1, dtype=torch.float32, device=x.device)
    L.check(L.load().qmoe_router_logits_f32(_p(x), _p(wr), _p(shared_gate), N, H, E, _p(out), E + 1,
                                            _stream(x.device)), "qmoe_router_logits_f32")
    return out


def router_topk(logits: torch.Tensor, n_experts: int, k: int, *, scoring: int = L.SCORE_SOFTMAX,
                bias: torch.Tensor | None = None, n_group: int = 1, topk_group: int = 1,
                norm_topk: int = L.NORM_ALWAYS, routed_scale: float = 1.0,
                has_shared_gate: bool = False):
    """Top-k over router logits [N, ld] -> (idx [N,k] int32, w [N,k] fp32, sg [N] fp32 or None).
    `norm_topk` is a QMOE_NORM_* mode (True / False mean always / never)."""
    _need(logits, torch.float32, "logits")
    N, ld = logits.shape
    if bias is not None:
        _need(bias, torch.float32, "bias")
        if bias.numel() != n_experts:
            raise ValueError("router_topk: bias must have E elements")
    idx = torch.empty(N, k, dtype=torch.int32, device=logits.device)
    w = torch.empty(N, k, dtype=torch.float32, device=logits.device)
    sg = torch.empty(N, dtype=torch.float32, device=logits.device) if has_shared_gate else None
    L.check(L.load().qmoe_router_topk(_p(logits), ld, _p(bias), N, n_experts, k, scoring, n_group,
                                      topk_group, int(norm_topk), float(routed_scale),
                                      int(has_shared_gate), _p(idx), _p(w), _p(sg),
                                      _stream(logits.device)), "qmoe_router_topk")
    return idx, w, sg


def router(x: torch.Tensor, wr: torch.Tensor, k: int, *, shared_gate: torch.Tensor | None = None,
           scoring: int = L.SCORE_SOFTMAX, bias: torch.Tensor | None = None, n_group: int = 1,
           topk_group: int = 1, norm_topk: int = L.NORM_ALWAYS, routed_scale: float = 1.0):
    """The router in one call (qmoe_router) from the gate as stored: x [N, H] bf16, wr [E, H]
    bf16 or fp32 (shared_gate [H] or [1, H] of wr's dtype, optional) -> (idx [N,k] int32,
    w [N,k] fp32, sg [N] fp32 or None)."""
    _need(x, torch.bfloat16, "x")
    _need(wr, (torch.bfloat16, torch.float32), "wr")
    N, H = x.shape
    E = wr.shape[0]
    if wr.dim() != 2 or wr.shape[1] != H:
        raise ValueError("router: wr must be [E, H]")
    if shared_gate is not None:
        _need(shared_gate, wr.dtype, "shared_gate")
        if shared_gate.numel() != H:
            raise ValueError("router: shared_gate must have H elements")
    if bias is not None:
        _need(bias, torch.float32, "bias")
        if bias.numel() != E:
            raise ValueError("router: bias must have E elements")
    lib = L.load()
    ws = torch.empty(max(int(lib.qmoe_router_workspace(N, E)), 1), dtype=torch.uint8, device=x.device)
    idx = torch.empty(N, k, dtype=torch.int32, device=x.device)
    w = torch.empty(N, k, dtype=torch.float32, device=x.device)
    sg = torch.empty(N, dtype=torch.float32, device=x.device) if shared_gate is not None else None
    L.check(lib.qmoe_router(_p(x), _p(wr), int(wr.dtype == torch.float32), _p(shared_gate), _p(bias),
                            N, H, E, k, scoring, n_group, topk_group, int(norm_topk),
                            float(routed_scale), _p(idx), _p(w), _p(sg), _p(ws), ws.numel(),
                            _stream(x.device)), "qmoe_router")
    return idx, w, sg


def permute(idx: torch.Tensor, n_experts: int, m_tile: int = L.SMALL_M_TILE):
    """Stable permute of idx [N, k] by expert -> (counts, offsets, tile_off, sorted_slot, inv,
    tile_map)."""
    _need(idx, torch.int32, "idx")
    N, k = idx.shape
    dev = idx.device
    counts = torch.empty(n_experts, dtype=torch.int32, device=dev)
    offsets = torch.empty(n_experts + 1, dtype=torch.int32, device=dev)
    tile_off = torch.empty(n_experts + 1, dtype=torch.int32, device=dev)
    sorted_slot = torch.empty(N * k, dtype=torch.int32, device=dev)
    inv = torch.empty(N * k, dtype=torch.int32, device=dev)
    max_tiles = L.mtile_upper_bound(N * k, n_experts, m_tile)
    tile_map = torch.empty(max_tiles, 4, dtype=torch.int32, device=dev)
    L.check(L.load().qmoe_permute(_p(idx), N, k, n_experts, m_tile, _p(counts), _p(offsets),
                                  _p(tile_off), _p(sorted_slot), _p(inv), _p(tile_map), max_tiles,
                                  _stream(dev)), "qmoe_permute")
    return counts, offsets, tile_off, sorted_slot, inv, tile_map


def grouped_qmm(act: torch.Tensor, *, K: int, n_rows: int, weight_format: int,
                codes: torch.Tensor, sb: torch.Tensor | None, epilogue: int, out_rows: int,
                regime: int, slot_of: torch.Tensor | None = None, slot_div: int = 1,
                n_slots: int = 0, offsets: torch.Tensor | None = None,
                tile_off: torch.Tensor | None = None, tile_map: torch.Tensor | None = None,
                n_experts: int = 1,
                dense_rows: int = 0, out: torch.Tensor | None = None,
                ws: torch.Tensor | None = None, glu: int = L.ACT_SILU, glu_alpha: float = 1.0,
                glu_limit: float = float("inf"), row_exp: torch.Tensor | None = None) -> torch.Tensor:
    """Grouped matmul over expert segments (see qmoe_grouped_qmm). Returns out [out_rows, cols]
    (bf16, or fp32 for EPI_F32); cols = n_rows/2 for SwiGLU else n_rows. `glu`, `glu_alpha`,
    `glu_limit`: the SwiGLU epilogue's gated activation (L.ACT_*). `row_exp`: int4 stacks' per-row
    exponents (row_exponents) for the large regime's fp16 dequant (required there)."""
    _need(act, torch.bfloat16, "act")
    if act.dim() != 2 or act.shape[1] != K:
        raise ValueError("grouped_qmm: act must be [rows, K]")
    if weight_format in (L.FMT_INT4_G64, L.FMT_INT6_G64, L.FMT_INT3_G64, L.FMT_INT8_G64):
        codes = _words(codes, "codes")
        _need(sb, torch.bfloat16, "sb")
    else:
        _need(codes, torch.bfloat16, "codes")
    for t, nm in ((slot_of, "slot_of"), (offsets, "offsets"), (tile_off, "tile_off"),
                  (tile_map, "tile_map")):
        if t is not None:
            _need(t, torch.int32, nm)
    if row_exp is not None:
        _need(row_exp, torch.int8, "row_exp")
        if row_exp.numel() < n_experts * n_rows:
            raise ValueError("grouped_qmm: row_exp must hold one exponent per weight row")
    cols = n_rows // 2 if epilogue == L.EPI_SWIGLU else n_rows
    dtype = torch.float32 if epilogue == L.EPI_F32 else torch.bfloat16
    if out is None:
        out = torch.zeros(out_rows, cols, dtype=dtype, device=act.device)
    else:
        _need(out, dtype, "out")
        if out.shape != (out_rows, cols):
            raise ValueError("grouped_qmm: out has the wrong shape")
    lib = L.load()
    need = int(lib.qmoe_grouped_qmm_workspace(act.shape[0], K, weight_format, regime))
    if need and (ws is None or ws.numel() < need):
        ws = torch.empty(need, dtype=torch.uint8, device=act.device)
    if tile_map is not None and offsets is not None:
        m_tile = L.SMALL_M_TILE if regime == L.REGIME_SMALL else L.LARGE_M_TILE
        if tile_map.shape[0] < L.mtile_upper_bound(n_slots, n_experts, m_tile):
            raise ValueError("grouped_qmm: tile_map was built for a different m-tile")
    L.check(lib.qmoe_grouped_qmm(_p(act), act.shape[0], _p(slot_of), slot_div, n_slots,
                                 _p(offsets), _p(tile_off), _p(tile_map), n_experts, dense_rows,
                                 K, n_rows,
                                 weight_format, _p(codes), _p(sb), _p(row_exp), epilogue, int(glu),
                                 float(glu_alpha), float(glu_limit), _p(out), cols,
                                 regime, _p(ws) if need else None, ws.numel() if need else 0,
                                 _stream(act.device)), "qmoe_grouped_qmm")
    return out


def combine(d: torch.Tensor, inv: torch.Tensor, w: torch.Tensor,
            shared_out: torch.Tensor | None = None,
            shared_gate: torch.Tensor | None = None) -> torch.Tensor:
    """y[t] = bf16(sum_s w[t,s] * d[inv[t*k+s]] + shared_gate[t] * shared_out[t])."""
    _need(d, torch.bfloat16, "d")
    _need(inv, torch.int32, "inv")
    _need(w, torch.float32, "w")
    N, k = w.shape
    H = d.shape[1]
    if shared_out is not None:
        _need(shared_out, torch.bfloat16, "shared_out")
    if shared_gate is not None:
        _need(shared_gate, torch.float32, "shared_gate")
    y = torch.empty(N, H, dtype=torch.bfloat16, device=d.device)
    L.check(L.load().qmoe_combine(_p(d), _p(inv), _p(w), N, k, H, _p(shared_out), _p(shared_gate),
                                  _p(y), _stream(d.device)), "qmoe_combine")
    return y


def forward_workspace(cfg: L.QmoeConfig, N: int) -> int:
    return int(L.load().qmoe_forward_workspace(ctypes.byref(cfg), N))


def forward(cfg: L.QmoeConfig, weights: L.QmoeWeights, x: torch.Tensor,
            out: torch.Tensor | None = None, ws: torch.Tensor | None = None,
            mixed: L.QmoeMixed | None = None) -> torch.Tensor:
    """Whole block on x [N, H] bf16 (qmoe_forward; with `mixed`, the routed experts of mixed
    widths, qmoe_forward_mixed). `ws` may be a preallocated uint8 buffer."""
    _need(x, torch.bfloat16, "x")
    N, H = x.shape
    if H != cfg.hidden:
        raise ValueError("forward: x hidden size does not match the config")
    need = forward_workspace(cfg, N)
    if ws is None or ws.numel() < need:
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
    if out is None:
        out = torch.empty(N, H, dtype=torch.bfloat16, device=x.device)
    if mixed is not None:
        L.check(L.load().qmoe_forward_mixed(ctypes.byref(cfg), ctypes.byref(weights), ctypes.byref(mixed),
                                            _p(x), N, _p(out), _p(ws), ws.numel(), _stream(x.device)),
                "qmoe_forward_mixed")
        return out
    L.check(L.load().qmoe_forward(ctypes.byref(cfg), ctypes.byref(weights), _p(x), N, _p(out),
                                  _p(ws), ws.numel(), _stream(x.device)), "qmoe_forward")
    return out


_DT = {torch.bfloat16: L.DT_BF16, torch.float32: L.DT_F32}


def dtype_code(dt: torch.dtype, name: str) -> int:
    """QMOE_DT_* of a torch dtype (bf16 or float32; anything else raises)."""
    if dt not in _DT:
        raise TypeError(f"{name}: dtype {dt} not supported (bfloat16 or float32)")
    return _DT[dt]


def forward_general(cfg: L.QmoeGeneralConfig, weights: L.QmoeGeneralWeights, x: torch.Tensor,
                    out: torch.Tensor | None = None, ws: torch.Tensor | None = None) -> torch.Tensor:
    """Whole block on x [N, H] of the config's x_dtype at the reference's own dtypes and group
    sizes (qmoe_forward_general)."""
    dt = torch.float32 if cfg.x_dtype == L.DT_F32 else torch.bfloat16
    _need(x, dt, "x")
    N, H = x.shape
    if H != cfg.hidden:
        raise ValueError("forward_general: x hidden size does not match the config")
    need = int(L.load().qmoe_forward_general_workspace(ctypes.byref(cfg), N))
    if ws is None or ws.numel() < need:
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
    if out is None:
        out = torch.empty(N, H, dtype=dt, device=x.device)
    _need(out, dt, "out")
    L.check(L.load().qmoe_forward_general(ctypes.byref(cfg), ctypes.byref(weights), _p(x), N,
                                          _p(out), _p(ws), ws.numel(), _stream(x.device)),
            "qmoe_forward_general")
    return out


def forward_noalloc(cfg: L.QmoeConfig, weights: L.QmoeWeights, x: torch.Tensor,
                    out: torch.Tensor) -> torch.Tensor:
    """Whole block on x [N, H] bf16 into `out` (qmoe_forward_noalloc): the library's fixed
    per-GPU scratch in place of a workspace, every launch on the current stream, nothing
    allocated (the caller passes `out`)."""
    _need(x, torch.bfloat16, "x")
    _need(out, torch.bfloat16, "out")
    N, H = x.shape
    if H != cfg.hidden or out.shape != x.shape:
        raise ValueError("forward_noalloc: x / out do not match the config's hidden size")
    L.check(L.load().qmoe_forward_noalloc(ctypes.byref(cfg), ctypes.byref(weights), _p(x), N,
                                          _p(out), _stream(x.device)), "qmoe_forward_noalloc")
    return out


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float,
            out: torch.Tensor | None = None) -> torch.Tensor:
    """RMSNorm rows of x [N, H] bf16 with the resident bf16 weight [H] (qmoe_rmsnorm):
    bf16(weight * (x * rsqrt(mean(x^2) + eps))) in fp32."""
    _need(x, torch.bfloat16, "x")
    _need(weight, torch.bfloat16, "weight")
    if x.dim() != 2 or weight.shape != (x.shape[1],):
        raise ValueError("rmsnorm: x must be [N, H] and weight [H]")
    if out is None:
        out = torch.empty_like(x)
    L.check(L.load().qmoe_rmsnorm(_p(x), _p(weight), x.shape[0], x.shape[1], float(eps), _p(out),
                                  _stream(x.device)), "qmoe_rmsnorm")
    return out


def forward_residual_workspace(cfg: L.QmoeConfig, N: int) -> int:
    return int(L.load().qmoe_forward_residual_workspace(ctypes.byref(cfg), N))


def forward_residual(cfg: L.QmoeConfig, weights: L.QmoeWeights, x: torch.Tensor,
                     norm_weight: torch.Tensor, eps: float, out: torch.Tensor | None = None,
                     ws: torch.Tensor | None = None) -> torch.Tensor:
    """x + block(rmsnorm(x)) on the residual rows x [N, H] bf16 (qmoe_forward_residual). `out`
    may be x itself (in-place residual update)."""
    _need(x, torch.bfloat16, "x")
    _need(norm_weight, torch.bfloat16, "norm_weight")
    N, H = x.shape
    if H != cfg.hidden or norm_weight.shape != (H,):
        raise ValueError("forward_residual: x / norm_weight do not match the config's hidden size")
    need = forward_residual_workspace(cfg, N)
    if ws is None or ws.numel() < need:
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
    if out is None:
        out = torch.empty(N, H, dtype=torch.bfloat16, device=x.device)
    L.check(L.load().qmoe_forward_residual(ctypes.byref(cfg), ctypes.byref(weights), _p(x),
                                           _p(norm_weight), float(eps), N, _p(out), _p(ws),
                                           ws.numel(), _stream(x.device)), "qmoe_forward_residual")
    return out
