"""Benchmark of the MI355X quantized sparse-MoE layer (BASELINE.json metric).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2] [--batch 32]

One step = one forward of the MoE layer (router, permute, int4 gate_up + SwiGLU, int4 down,
gated shared expert, combine) over one batch of synthetic tokens, with weights and inputs
resident in HBM. Workload: Qwen3.5-397B-A17B-shaped layer, hidden 4096,
512 experts, top-10 softmax, expert intermediate 1024, shared expert 1024, int4 g64, decode batch
32 tokens. To time HBM rather than the 256 MB Infinity Cache, the timed loop rotates over
`--layers` copies of the layer (distinct memory) and a pool of distinct input batches (so the
routed experts change every step).

Printed (one JSON line): whole-layer tokens/s (`value`), per-step time, the dominant kernel's
roofline (routed gate_up+SwiGLU: algorithmic bytes per launch / its average duration, HIP events
on the launch stream), a sweep over the other decode batches and the 4096-token prefill, the
widened rows at the headline batch (`--extra`: the block with the decoder layer's RMSNorm and
residual add, qmoe_forward_residual; the layer with int6 experts, MiniMax M3's format, and with
Kimi's widths, gate_up int3 + down int4 at group 128, each rotating two copies and each also at
the c4 prefill; and with
DeepSeek-V4's activation-aware expert scales on the int4 experts, also at the c4 prefill; with
Kimi's widths drawn per (expert, projection)), and the CPU baseline (the torch-CPU port in oracle/torch_cpu.py on the host
cores, bounded sample).

`roofline.traffic` (measured HBM bytes per launch of the dominant kernel) comes from
profiles/hbm_traffic.json, written from two rocprofv3 counter passes over `--only kernel` runs:

    rocprofv3 --pmc FETCH_SIZE --output-format csv -d F -o pmc -- python bench.py --only kernel --kernel-reps 8
    rocprofv3 --pmc WRITE_SIZE --output-format csv -d W -o pmc -- python bench.py --only kernel --kernel-reps 8
    python bench.py --write-traffic F W --kernel-reps 8

Each counter is scaled by what it reads for the 2 GiB device copy of the same run (the copy's
known read and write bytes divided by its counter values).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

HBM_PEAK_GBPS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0       # MI355X dense bf16 MFMA
METRIC = "MoE-layer tokens/sec + achieved HBM GB/s (decode) / MFMA util (prefill), int4g64"


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="c2")
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--layers", type=int, default=8, help="layer copies rotated for cold HBM")
    ap.add_argument("--pool", type=int, default=16, help="distinct input batches rotated")
    ap.add_argument("--sweep", default="1,8,128", help="extra decode batch sizes ('' = none)")
    ap.add_argument("--configs-sweep", default="c1:1,8,32,64;c3:1,16,64",
                    help="decode lines of the other BASELINE configs, 'cfg:N,N;cfg:N' ('' = none)")
    ap.add_argument("--warmup-ms", type=float, default=150.0,
                    help="each timed loop's warm-up runs at least --warmup steps and at least this "
                         "many ms of steps: the clocks settle only after ~30 ms of sustained load")
    ap.add_argument("--prefill", type=int, default=4096,
                    help="tokens of the c4 Zipf prefill line (0 = none)")
    ap.add_argument("--zipf", action="store_true",
                    help="headline workload with c4's Zipf(1.1) routing (profiling the prefill)")
    ap.add_argument("--kernel-reps", type=int, default=64)
    ap.add_argument("--extra", default="residual,int6,int3,mixed,awq",
                    help="widened rows timed at the headline batch ('' = none): residual, int6, "
                         "int3, mixed, awq")
    ap.add_argument("--shared", choices=("int8", "bf16"), default="int8",
                    help="shared-expert weights: int8 g64 as the bake stores them (dequantized in "
                         "registers to the bf16 weights the reference loads; same outputs) or bf16")
    ap.add_argument("--flow-mode", type=int, choices=(0, 1, 2), default=None,
                    help="qmoe_set_decode_flow mode: 0 chain, 1 the library's default (the dataflow "
                         "launch for one and two tokens), 2 the dataflow launch wherever it fits")
    ap.add_argument("--no-flow", action="store_true",
                    help="launch the decode stages one by one (qmoe_set_decode_flow(0)) instead of "
                         "the one dataflow launch after the router")
    ap.add_argument("--route-tail", type=int, choices=(0, 1), default=None,
                    help="qmoe_set_route_tail: 1 (the library's default) ranks and sorts decode "
                         "batches in the router launch's last workgroups, 0 uses the top-k and "
                         "permute launches")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-reps", type=int, default=3, help="batches in the CPU-baseline sample")
    ap.add_argument("--only", default="", help="profiling aid: 'layer' or 'kernel' loop only")
    ap.add_argument("--graph", action="store_true",
                    help="also time decode steps replayed from a captured HIP graph (one step per "
                         "layer copy per replay), beside the stream launches")
    ap.add_argument("--write-traffic", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="summarise two rocprofv3 counter runs into profiles/hbm_traffic.json "
                         "(the workload of --batch / --zipf: its dominant gate_up kernel)")
    return ap.parse_args()


TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "hbm_traffic.json")
COPY_BYTES = 2 << 30          # the 2 GiB device copy of the `--only kernel` run


def kernel_key(workload, regime_small):
    """Counter-CSV kernel name prefix of the routed gate_up+SwiGLU launch."""
    return "qmm_small_kernel<0, 0," if regime_small else "qmm_wide_kernel<0>"


def write_traffic(fetch_dir, write_dir, workload="c2-decode-N32", regime_small=True, reps=8):
    """Per-dispatch FETCH_SIZE / WRITE_SIZE (KiB) of the dominant kernel, scaled by the copy.
    Only the last `reps` dispatches of the kernel count: the timed kernel loop of an
    `--only kernel --kernel-reps reps` run (the layer steps before it may launch the same kernel
    over a different tile set: the hot experts alone in the hybrid prefill)."""
    import csv
    import glob

    def read(d, counter):
        f = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
        if not f:
            sys.exit(f"bench.py: no counter_collection.csv under {d}")
        kern, copy, name = [], [], None
        for r in csv.DictReader(open(f[0])):
            if r.get("Counter_Name") != counter:
                continue
            v = float(r["Counter_Value"])
            if "copyBuffer" in r["Kernel_Name"]:
                copy.append(v)
            elif kernel_key(workload, regime_small) in r["Kernel_Name"]:
                kern.append((int(r["Dispatch_Id"]), v))
                name = r["Kernel_Name"]
        if not kern or not copy:
            sys.exit(f"bench.py: {counter}: kernel or copy dispatches missing in {d}")
        kern = [v for _, v in sorted(kern)[-reps:]]
        return sum(kern) / len(kern), max(copy), name, len(kern)

    fk, fcopy, name, n1 = read(fetch_dir, "FETCH_SIZE")
    wk, wcopy, _, n2 = read(write_dir, "WRITE_SIZE")
    fs, ws = COPY_BYTES / 1024 / fcopy, COPY_BYTES / 1024 / wcopy
    rec = dict(workload=workload, kernel=name, dispatches=[n1, n2], fetch_kib=round(fk, 1),
               write_kib=round(wk, 1), copy_fetch_kib=round(fcopy, 1), copy_write_kib=round(wcopy, 1),
               fetch_scale=round(fs, 4), write_scale=round(ws, 4),
               traffic_bytes=int(round((fk * fs + wk * ws) * 1024)))
    data = {}
    if os.path.exists(TRAFFIC_FILE):
        data = json.load(open(TRAFFIC_FILE))
    data[workload] = rec
    with open(TRAFFIC_FILE, "w") as f:
        json.dump(data, f, indent=1)
        f.write("\n")
    print(json.dumps(rec))


def measured_traffic(workload):
    if not os.path.exists(TRAFFIC_FILE):
        return None
    rec = json.load(open(TRAFFIC_FILE)).get(workload)
    return rec["traffic_bytes"] if rec else None


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def main():
    args = parse()
    if args.write_traffic:
        wl = ("c4-prefill-zipf" if args.zipf else
              f"{args.config}-decode" if args.batch <= 256 else f"{args.config}-prefill") + f"-N{args.batch}"
        write_traffic(*args.write_traffic, workload=wl, regime_small=args.batch <= 256,
                      reps=args.kernel_reps)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the MoE layer on one MI355X); "
              f"--gpus {args.gpus} is not supported. Multi-GPU sharding is a design note "
              "(expert- or tensor-parallel over xGMI), not a measured path.", file=sys.stderr)
        sys.exit(2)

    import torch

    from quanta_amd import _lib as L
    from quanta_amd import ops, synth
    from quanta_amd.moe import TiledExperts, prepare, qwen35_route, tile_experts_packed

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    L.load()
    if args.no_flow:
        L.load().qmoe_set_decode_flow(0)
    elif args.flow_mode is not None:
        L.load().qmoe_set_decode_flow(args.flow_mode)
    if args.route_tail is not None:
        L.load().qmoe_set_route_tail(args.route_tail)
    dev = torch.device("cuda", 0)
    spec = synth.spec(args.config)
    cfg = spec.cfg
    H, E, k, I = cfg.hidden_size, cfg.num_experts, cfg.num_experts_per_tok, cfg.moe_intermediate_size
    Is = cfg.shared_expert_intermediate_size
    SB = 8 if args.shared == "int8" else 16   # shared-expert bits (algorithmic bytes too)

    def resident_layers(name, copies):
        """`copies` resident (tiled) copies of config `name`'s synthetic layer at distinct
        addresses, and the native layer on the host (for the CPU baseline) or None."""
        t0 = time.time()
        base = synth.make_layer(name, device=dev, shared_bits=SB)
        gu0 = TiledExperts(**tile_experts_packed(base["experts_gate_up"]))
        dn0 = TiledExperts(**tile_experts_packed(base["experts_down"]))
        native = {kk: ({q: (v.cpu() if isinstance(v, torch.Tensor) else v) for q, v in vv.items()}
                       if isinstance(vv, dict) else vv.cpu()) for kk, vv in base.items()}
        del base["experts_gate_up"], base["experts_down"]
        out = []
        for li in range(copies):
            def cp(te):
                return TiledExperts({q: (v.clone() if isinstance(v, torch.Tensor) else v) for q, v in te.items()})
            p = {kk: ({q: (t.clone() if isinstance(t, torch.Tensor) else t) for q, t in v.items()}
                      if isinstance(v, dict) else v.clone()) for kk, v in base.items()}
            p["experts_gate_up"] = gu0 if li == 0 else cp(gu0)
            p["experts_down"] = dn0 if li == 0 else cp(dn0)
            out.append(p)
        torch.cuda.synchronize()
        log(f"{name}: {copies} resident layer copies ready ({time.time() - t0:.1f}s)")
        return out, native

    layers, native = resident_layers(args.config, args.layers)
    native_cpu = None if args.no_cpu_baseline else native
    warm_runs = []
    graph_runs = []

    def warm(step, warmup):
        """At least `warmup` steps and at least --warmup-ms of steps, then a synchronize. From
        idle, the chip runs the first ~5 steps fast, the next ~100 up to 17% slower and then
        settles (a power-management transient); sustained load removes it, so the timed loop
        starts from the steady state a serving loop runs in."""
        t0 = time.perf_counter()
        n = 0
        while n < warmup or (time.perf_counter() - t0) * 1e3 < args.warmup_ms:
            for _ in range(max(warmup - n, 16)):   # enqueued back to back: sustained load
                step(n)
                n += 1
            torch.cuda.synchronize()
        warm_runs.append(n)
        return n

    def run_batch(N, steps, warmup, pool, regime=L.REGIME_AUTO, zipf=False, lays=None,
                  residual=False, cfg_=None):
        # zipf: the c4 workload (the same shape, Zipf(1.1) expert popularity through router
        # column 0 and x[:, 0] = 1.0), on the resident experts of the headline config
        # residual: the block with the layer's RMSNorm in front and the residual add fused
        src = "c4" if zipf else (cfg_ or args.config)
        c_ = synth.spec(src).cfg
        xs = [synth.make_inputs(src, N, device=dev, seed=100 + i) for i in range(pool)]
        lays = layers if lays is None else lays
        if zipf:
            lays = [dict(p, gate=synth.zipf_router(p["gate"])) for p in lays]
        preps = [prepare(p, c_, regime=regime) for p in lays]
        wsz = (ops.forward_residual_workspace if residual else ops.forward_workspace)(preps[0].cfg, N)
        ws = torch.empty(wsz, dtype=torch.uint8, device=dev)
        out = torch.empty(N, c_.hidden_size, dtype=torch.bfloat16, device=dev)
        norm_w = (1.0 + 0.1 * torch.randn(c_.hidden_size, device=dev)).to(torch.bfloat16)

        def step(i):
            pr = preps[i % len(preps)]
            if residual:
                ops.forward_residual(pr.cfg, pr.weights, xs[i % pool], norm_w, 1e-6, out=out, ws=ws)
            else:
                ops.forward(pr.cfg, pr.weights, xs[i % pool], out=out, ws=ws, mixed=pr.mixed)

        warm(step, warmup)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(steps):
            step(i)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        if args.graph and N <= 256:
            # the same steps captured once (one per layer copy, kernel launches only: the block
            # records no memset or copy) and replayed: the step time without host launch cost
            n_cap = len(preps)
            s_cap = torch.cuda.Stream()
            s_cap.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s_cap):
                for i in range(n_cap):
                    step(i)
            torch.cuda.current_stream().wait_stream(s_cap)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for i in range(n_cap):
                    step(i)
            warm(lambda i: g.replay(), max(1, warmup // n_cap))
            reps = max(1, steps // n_cap)
            e0.record()
            for _ in range(reps):
                g.replay()
            e1.record()
            torch.cuda.synchronize()
            gms = e0.elapsed_time(e1) / (reps * n_cap)
            graph_runs.append(dict(workload=f"{src}-N{N}" + ("-residual" if residual else ""),
                                   ms_per_step_stream=round(ms, 5), ms_per_step_graph=round(gms, 5)))
            log(f"graph {graph_runs[-1]}")
            del g
        # distinct experts per batch (U) for the algorithmic byte count
        us = []
        for x in xs:
            xr = ops.rmsnorm(x, norm_w, 1e-6) if residual else x
            idx, _ = qwen35_route(xr, lays[0]["gate"], c_,
                                  e_score_correction_bias=lays[0].get("e_score_correction_bias"))
            us.append(int(torch.unique(idx).numel()))
        return ms, us, xs, preps

    # ------------------------------------------------------------------ headline workload
    N = args.batch
    if args.only == "kernel":
        steps_layer = 1
    else:
        steps_layer = args.steps
    ms, us, xs, preps = run_batch(N, steps_layer, args.warmup, args.pool, zipf=args.zipf)
    U = sum(us) / len(us)
    layer_bytes = synth.algorithmic_bytes(cfg, U, N, shared_bits=SB)
    log(f"N={N}: {ms * 1e3:.1f} us/step, U={U:.1f}, layer {layer_bytes / ms / 1e6:.0f} GB/s")

    # ------------------------------------------------------------------ dominant kernel
    # routed gate_up + SwiGLU, launched alone on the real permuted inputs, rotating layers
    kern = None
    if args.only != "layer":
        regime = L.REGIME_SMALL if N <= 256 else L.REGIME_LARGE
        m_tile = L.SMALL_M_TILE if regime == L.REGIME_SMALL else L.LARGE_M_TILE
        inputs = []
        gate0 = synth.zipf_router(layers[0]["gate"]) if args.zipf else layers[0]["gate"]
        for x in xs[:4]:
            idx, _ = qwen35_route(x, gate0, cfg)
            counts, offsets, tile_off, sorted_slot, inv, tile_map = ops.permute(idx, E, m_tile)
            inputs.append((x, offsets, tile_off, sorted_slot, tile_map, int((counts > 0).sum())))
        h = torch.empty(N * k, I, dtype=torch.bfloat16, device=dev)

        def launch(i):
            pr = preps[i % len(preps)]
            x, offsets, tile_off, sorted_slot, tile_map, _ = inputs[i % len(inputs)]
            ops.grouped_qmm(x, K=H, n_rows=2 * I, weight_format=L.FMT_INT4_G64,
                            codes=pr.gu["codes"], sb=pr.gu["sb"], row_exp=pr.gu.get("rexp"),
                            epilogue=L.EPI_SWIGLU,
                            out_rows=N * k, regime=regime, slot_of=sorted_slot, slot_div=k,
                            n_slots=N * k, offsets=offsets, tile_off=tile_off, tile_map=tile_map,
                            n_experts=E, out=h)

        warm(launch, 8)
        reps = args.kernel_reps
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(reps):
            launch(i)
        e1.record()
        torch.cuda.synchronize()
        kms = e0.elapsed_time(e1) / reps
        u_k = sum(t[5] for t in inputs) / len(inputs)
        per_expert = 2 * I * H * 9 // 16                   # int4 codes + bf16 scale/bias per 64
        kbytes = u_k * per_expert + N * H * 2 + N * k * I * 2
        kern = dict(name="qmm_small_kernel<int4,swiglu,W,CPW,JPW>" if regime == L.REGIME_SMALL
                    else "act_to_f16 + qmm_wide_kernel<swiglu>", us=kms * 1e3, bytes=kbytes,
                    U=u_k, mfma=regime == L.REGIME_LARGE, flops=2 * N * k * 2 * I * H)
        log(f"gate_up kernel: {kms * 1e3:.1f} us, {kbytes / kms / 1e6:.0f} GB/s")

    # ------------------------------------------------------------------ sweep
    sweep = []
    runs = []
    if args.only == "":
        runs = [(int(v), False) for v in args.sweep.split(",") if v]
        if args.prefill > 0:
            runs.append((args.prefill, True))
    if runs:
        for n2, zipf in runs:
            st = max(100, args.steps // 4) if n2 <= 256 else max(20, args.steps // 20)
            m2, u2, _, _ = run_batch(n2, st, 3, min(args.pool, 8), zipf=zipf)
            U2 = sum(u2) / len(u2)
            b2 = synth.algorithmic_bytes(cfg, U2, n2, shared_bits=SB)
            f2 = synth.algorithmic_flops(cfg, n2)
            rec = dict(workload=f"c4-prefill-N{n2}-zipf" if zipf else f"{args.config}-N{n2}",
                       N=n2, ms_per_step=round(m2, 5), tokens_per_s=round(n2 / (m2 / 1e3), 1),
                       distinct_experts=round(U2, 1), hbm_gbps=round(b2 / m2 / 1e6, 1),
                       hbm_frac=round(b2 / m2 / 1e6 / HBM_PEAK_GBPS, 4),
                       tflops=round(f2 / m2 / 1e9, 2),
                       mfma_frac=round(f2 / m2 / 1e9 / BF16_PEAK_TFLOPS, 4))
            sweep.append(rec)
            log(f"sweep {rec}")

    # ------------------------------------------------------------------ other BASELINE configs
    # decode lines of configs 1 (Qwen3.6-35B-A3B shape) and 3 (DeepSeek-style sigmoid, groups),
    # each on its own resident copies: enough of them that a step's weights come from HBM
    if args.only == "" and args.configs_sweep:
        for part in args.configs_sweep.split(";"):
            name, ns = part.split(":")
            c_ = synth.spec(name).cfg
            layer_mb = synth.algorithmic_bytes(c_, c_.num_experts, 0, shared_bits=SB) / 2**20
            copies = max(2, min(8, int(2048 // layer_mb) + 1))
            lays_c, _ = resident_layers(name, copies)
            for n2 in (int(v) for v in ns.split(",") if v):
                m2, u2, _, _ = run_batch(n2, max(100, args.steps // 4), 3, min(args.pool, 8),
                                         lays=lays_c, cfg_=name)
                U2 = sum(u2) / len(u2)
                b2 = synth.algorithmic_bytes(c_, U2, n2, shared_bits=SB)
                rec = dict(workload=f"{name}-N{n2}", N=n2, ms_per_step=round(m2, 5),
                           tokens_per_s=round(n2 / (m2 / 1e3), 1), distinct_experts=round(U2, 1),
                           hbm_gbps=round(b2 / m2 / 1e6, 1),
                           hbm_frac=round(b2 / m2 / 1e6 / HBM_PEAK_GBPS, 4), layer_copies=copies)
                sweep.append(rec)
                log(f"sweep {rec}")
            del lays_c
            torch.cuda.empty_cache()

    # ------------------------------------------------------------------ widened rows
    # the block with the decoder layer's norm and residual add (qmoe_forward_residual), and the
    # layer with int6 experts (MiniMax M3's format), at the headline batch
    if args.only == "" and N <= 256:
        def record(name, m2, u2, extra_bytes=0, per_expert_bytes=0, **fmt):
            U2 = sum(u2) / len(u2)
            b2 = (synth.algorithmic_bytes(cfg, U2, N, shared_bits=SB, **fmt) + extra_bytes
                  + U2 * per_expert_bytes)
            rec = dict(workload=name, N=N, ms_per_step=round(m2, 5),
                       tokens_per_s=round(N / (m2 / 1e3), 1), distinct_experts=round(U2, 1),
                       hbm_gbps=round(b2 / m2 / 1e6, 1), hbm_frac=round(b2 / m2 / 1e6 / HBM_PEAK_GBPS, 4))
            sweep.append(rec)
            log(f"sweep {rec}")

        if "residual" in args.extra:
            # (the same steps, warm-up and input pool as the headline loop, so the two lines
            # differ only by the norm and the residual add)
            m2, u2, _, _ = run_batch(N, args.steps, args.warmup, args.pool, residual=True)
            record(f"{args.config}-N{N}-residual", m2, u2, extra_bytes=2 * H)
        # int6: MiniMax M3's experts; int3: Kimi's widths (gate_up int3 + down int4, group 128).
        # Two copies suffice to stream from HBM: one step touches U experts x 6-10 MB.
        for tag, fmt in (("int6", dict(bits=6)), ("int3", dict(bits=3, down_bits=4, group_size=128))):
            if tag not in args.extra:
                continue
            lays_f = []
            for li in range(2):
                pf = synth.make_layer(args.config, device=dev, layer=li, shared_bits=SB, **fmt)
                pf["experts_gate_up"] = TiledExperts(**tile_experts_packed(pf["experts_gate_up"]))
                pf["experts_down"] = TiledExperts(**tile_experts_packed(pf["experts_down"]))
                lays_f.append(pf)
            torch.cuda.synchronize()
            m2, u2, _, _ = run_batch(N, max(100, args.steps // 4), 3, min(args.pool, 8), lays=lays_f)
            record(f"{args.config}-N{N}-{tag}", m2, u2, **fmt)
            if args.prefill > 0:
                # the same layers at the c4 prefill (Zipf routing): the large regime, hot experts
                # on the 256-row prefill kernel; FLOPs as the int4 prefill line
                n3 = args.prefill
                m3, _, _, _ = run_batch(n3, max(20, args.steps // 20), 3, min(args.pool, 8),
                                        zipf=True, lays=lays_f)
                f3 = synth.algorithmic_flops(cfg, n3)
                rec = dict(workload=f"c4-prefill-N{n3}-zipf-{tag}", N=n3, ms_per_step=round(m3, 5),
                           tokens_per_s=round(n3 / (m3 / 1e3), 1), tflops=round(f3 / m3 / 1e9, 2),
                           mfma_frac=round(f3 / m3 / 1e9 / BF16_PEAK_TFLOPS, 4))
                sweep.append(rec)
                log(f"sweep {rec}")
            del lays_f
        if "mixed" in args.extra:
            # Kimi's per-(expert, projection) widths, int3 or int4 at group 128 drawn per expert
            # and projection: one launch per (projection, width); two copies
            from quanta_amd.moe import tile_experts_mixed
            lays_m, be = [], 0.0
            for li in range(2):
                src = synth.make_mixed_experts(args.config, device=dev, seed=li)
                be = synth.mixed_expert_bytes(src, cfg)
                pm = {kk: v for kk, v in layers[li].items() if not kk.startswith("experts_")}
                pm["experts_mixed"] = tile_experts_mixed(src["stacks"], src["pbits"], src["pslot"])
                del src
                lays_m.append(pm)
            torch.cuda.synchronize()
            m2, u2, _, _ = run_batch(N, max(100, args.steps // 4), 3, min(args.pool, 8), lays=lays_m)
            # bytes: the int4-g64 figure with the mixed layer's mean bytes per expert in its place
            be4 = 3 * cfg.moe_intermediate_size * H * 36 / 64
            record(f"{args.config}-N{N}-mixed34", m2, u2, per_expert_bytes=be - be4)
            if args.prefill > 0:
                # the same layers at the c4 prefill (Zipf routing): each (projection, width)
                # stack's launch on the prefill kernels over the hot experts' m-tiles
                n3 = args.prefill
                m3, _, _, _ = run_batch(n3, max(20, args.steps // 20), 3, min(args.pool, 8),
                                        zipf=True, lays=lays_m)
                f3 = synth.algorithmic_flops(cfg, n3)
                rec = dict(workload=f"c4-prefill-N{n3}-zipf-mixed34", N=n3,
                           ms_per_step=round(m3, 5), tokens_per_s=round(n3 / (m3 / 1e3), 1),
                           tflops=round(f3 / m3 / 1e9, 2),
                           mfma_frac=round(f3 / m3 / 1e9 / BF16_PEAK_TFLOPS, 4))
                sweep.append(rec)
                log(f"sweep {rec}")
            del lays_m
        if "awq" in args.extra:
            # DeepSeek-V4's activation-aware scales on the int4 experts: each routed row's
            # activation divided per input channel before gate, up and down (bf16 scales [E,2,H]
            # and [E,I], read per distinct expert)
            lays_a = []   # the resident int4 layer copies, with scales
            for li, pl in enumerate(layers):
                pa = dict(pl)
                g = torch.Generator(device="cpu").manual_seed(77 + li)
                E_, I_ = cfg.num_experts, cfg.moe_intermediate_size
                s_gu = (2.0 ** (torch.rand(E_, 2, H, generator=g) * 2 - 1)).to(torch.bfloat16).to(dev)
                s_dn = (2.0 ** (torch.rand(E_, I_, generator=g) * 2 - 1)).to(torch.bfloat16).to(dev)
                pa["experts_gate_up"] = TiledExperts(dict(pa["experts_gate_up"], awq_scale=s_gu))
                pa["experts_down"] = TiledExperts(dict(pa["experts_down"], awq_scale=s_dn))
                lays_a.append(pa)
            torch.cuda.synchronize()
            m2, u2, _, _ = run_batch(N, max(100, args.steps // 4), 3, min(args.pool, 8), lays=lays_a)
            record(f"{args.config}-N{N}-awq", m2, u2,
                   per_expert_bytes=(2 * H + cfg.moe_intermediate_size) * 2)
            if args.prefill > 0:
                # the same scaled layers at the c4 prefill (Zipf routing): the large regime, the
                # hot experts' gate_up on the prefill kernel reading fp16 copies of the prescaled
                # rows; FLOPs as the plain prefill line (the AWQ passes are elementwise)
                n3 = args.prefill
                m3, _, _, _ = run_batch(n3, max(20, args.steps // 20), 3, min(args.pool, 8),
                                        zipf=True, lays=lays_a)
                f3 = synth.algorithmic_flops(cfg, n3)
                rec = dict(workload=f"c4-prefill-N{n3}-zipf-awq", N=n3, ms_per_step=round(m3, 5),
                           tokens_per_s=round(n3 / (m3 / 1e3), 1), tflops=round(f3 / m3 / 1e9, 2),
                           mfma_frac=round(f3 / m3 / 1e9 / BF16_PEAK_TFLOPS, 4))
                sweep.append(rec)
                log(f"sweep {rec}")
            del lays_a

    # ------------------------------------------------------------------ measured copy peak
    # device-to-device copy of 2 GiB (read + write bytes), the practical HBM ceiling next to
    # the 8 TB/s vendor figure; in the `--only kernel` profiling mode it is also the copy of
    # known size that FETCH_SIZE / WRITE_SIZE counter passes are calibrated against
    copy_gbps = None
    if args.only in ("", "kernel"):
        src = torch.empty(1 << 30, dtype=torch.int16, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(10):
            dst.copy_(src)
        e1.record()
        torch.cuda.synchronize()
        copy_gbps = round(2 * src.numel() * 2 * 10 / (e0.elapsed_time(e1) * 1e6), 1)
        del src, dst
        log(f"copy bandwidth {copy_gbps} GB/s")

    # ------------------------------------------------------------------ CPU baseline
    cpu = None
    if native_cpu is not None and args.only == "":
        from oracle import torch_cpu

        # the reference's loader dequantizes an int8 shared expert to bf16 once, at load
        native_cpu = torch_cpu.load_shared(native_cpu)
        cores = len(os.sched_getaffinity(0))
        torch.set_num_threads(cores)
        xs_cpu = [x.cpu() for x in xs[:args.cpu_reps]]
        torch_cpu.moe_forward(xs_cpu[0][:2], native_cpu, cfg)      # warm-up
        t1 = time.perf_counter()
        for x in xs_cpu:
            torch_cpu.moe_forward(x, native_cpu, cfg)
        dt = time.perf_counter() - t1
        cpu = dict(value=round(N * len(xs_cpu) / dt, 2), unit="tokens/s", cores=cores, kind="port",
                   sample=f"{len(xs_cpu)} batches of {N} tokens of the {args.config} workload "
                          f"(torch-CPU fp32 port, oracle/torch_cpu.py), {dt:.1f}s")
        log(f"cpu baseline: {cpu}")

    workload = (("c4-prefill-zipf" if args.zipf else
                 f"{args.config}-decode" if N <= 256 else f"{args.config}-prefill") + f"-N{N}")
    traffic = measured_traffic(workload)
    roofline = None
    if kern is not None:
        if kern["mfma"]:
            # prefill: FLOPs of the routed gate_up per launch (2 * N*k * 2I * H) per second
            achieved = kern["flops"] / (kern["us"] * 1e-6) / 1e12
            roofline = dict(bound="mfma", achieved=round(achieved, 1), peak=BF16_PEAK_TFLOPS,
                            unit="TFLOP/s", frac=round(achieved / BF16_PEAK_TFLOPS, 4),
                            traffic=traffic, kernel=kern["name"], kernel_us=round(kern["us"], 2),
                            flops_per_launch=int(kern["flops"]), distinct_experts=round(kern["U"], 1))
        else:
            achieved = kern["bytes"] / (kern["us"] * 1e-6) / 1e9
            roofline = dict(bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBPS, unit="GB/s",
                            frac=round(achieved / HBM_PEAK_GBPS, 4), traffic=traffic,
                            kernel=kern["name"], kernel_us=round(kern["us"], 2),
                            bytes_per_launch=int(kern["bytes"]), distinct_experts=round(kern["U"], 1))
    line = {
        "metric": METRIC,
        "value": round(N / (ms / 1e3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps_layer,
        "warmup": args.warmup,
        "warmup_policy": f"at least --warmup steps and {args.warmup_ms:g} ms of steps before each "
                         "timed loop (the clocks settle ~30 ms into sustained load)",
        "warmup_steps_run": warm_runs[0] if warm_runs else None,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": workload,
                   "hidden": H, "experts": E, "top_k": k, "inter": I, "shared_inter": Is,
                   "batch_tokens": N, "weights": "int4-g64 affine, bf16 scale/bias",
                   "shared_weights": ("int8-g64 as baked, dequantized in registers to the bf16 "
                                      "weights the reference loads" if SB == 8 else "bf16"),
                   "layer_copies": args.layers, "input_pool": args.pool},
        "layer_hbm_gbps": round(layer_bytes / ms / 1e6, 1),
        "measured_copy_gbps": copy_gbps,
        "layer_hbm_frac": round(layer_bytes / ms / 1e6 / HBM_PEAK_GBPS, 4),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "sweep": sweep,
    }
    if graph_runs:
        line["graph"] = graph_runs
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
