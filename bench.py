#!/usr/bin/env python3
"""Fused-MoE layer benchmark on one MI355X (Qwen3-30B-A3B MoE shape, bf16).

A step is one MoE layer forward (fused router + align + gate_up/SwiGLU + down + k-sum) over one
batch of T synthetic tokens, inputs and weights resident in HBM. The headline workload is the
decode configuration T=64 (H=2048, E=128, top-8, I=768); the step cycles over 8 distinct
random-init layer copies so expert weights are streamed from HBM, not served from the 256 MB
Infinity Cache. The timed region replays a HIP graph of the 8 layer copies back to back (a
model's decode graph runs its MoE layers the same way), timing exactly `--steps` layer steps.

Prints ONE JSON line on stdout. Extra fields: per-stage kernel times (HIP events around each stage
launch on the launch stream), the dominant kernel's roofline, a sweep over the decode/prefill
token counts and the load-imbalance stress cases, and the CPU baseline (the torch-CPU restatement
of the reference MoE path, timed on this host's cores).
"""
import argparse
import json
import os
import sys
import time

HBM_PEAK = 8.0e12        # B/s, MI355X HBM3E
MFMA_BF16_PEAK = 2.5e15  # flop/s, MI355X dense bf16
H, E, K_TOP, I = 2048, 128, 8, 768


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def layer_bytes(T, n_touched):
    """Algorithmic HBM bytes of one layer: touched expert weights + router weight + x in/out + logits."""
    return n_touched * 3 * H * I * 2 + E * H * 2 + 2 * T * H * 2 + T * E * 2


def layer_flops(T):
    return 2 * T * H * E + 6 * T * K_TOP * H * I


def stage_bytes(T, n_touched):
    numel = T * K_TOP
    return {
        "router": T * H * 2 + E * H * 2 + numel * 8,
        "align": numel * 4,
        "gate_up": n_touched * 2 * I * H * 2 + T * H * 2 + numel * I * 2,
        "down": n_touched * H * I * 2 + numel * I * 2 + numel * H * 2,
        "combine": numel * H * 2 + T * H * 2,
    }


def stage_flops(T):
    numel = T * K_TOP
    return {"router": 2 * T * H * E, "gate_up": 2 * numel * H * 2 * I, "down": 2 * numel * I * H}


def torch_moe_layer(x, gw, w13, w2, top_k=8):
    """The same layer composed from stock PyTorch-ROCm ops on the GPU (what a framework without
    a fused MoE kernel runs): fp32 router + softmax + top-k + renormalise, assignments sorted
    by expert, per-expert hipBLASLt GEMMs with the reference's bf16 rounding points, weighted
    rows added into an fp32 output. Comparison baseline only; not a parity reference."""
    import torch
    T, H = x.shape
    I = w2.shape[-1]
    p = torch.softmax(torch.nn.functional.linear(x.float(), gw.float()), dim=-1)
    w, ids = torch.topk(p, top_k, dim=-1)
    w = w / w.sum(-1, keepdim=True)
    flat_ids = ids.reshape(-1)
    order = torch.argsort(flat_ids, stable=True)
    counts = torch.bincount(flat_ids, minlength=w13.shape[0]).tolist()
    tok = order // top_k
    out = torch.zeros(T, H, dtype=torch.float32, device=x.device)
    start = 0
    for e, c in enumerate(counts):
        if c == 0:
            continue
        sel = order[start:start + c]
        t_e = tok[start:start + c]
        h = x[t_e] @ w13[e].t()
        a = torch.nn.functional.silu(h[:, :I]) * h[:, I:]
        y = (a @ w2[e].t()).float() * w.reshape(-1)[sel, None]
        out.index_add_(0, t_e, y)
        start += c
    return out.to(x.dtype)


def torch_gpu_baseline(layer, x, T, layer_b):
    import torch
    gw, w13, w2 = layer
    for _ in range(3):
        torch_moe_layer(x, gw, w13, w2)
    torch.cuda.synchronize()
    reps, t0 = 0, time.perf_counter()
    while reps < 20 and (reps < 3 or time.perf_counter() - t0 < 3.0):
        torch_moe_layer(x, gw, w13, w2)
        reps += 1
    torch.cuda.synchronize()
    t = (time.perf_counter() - t0) / reps
    return {"us_per_layer": t * 1e6, "GBps": layer_b / t / 1e9, "reps": reps,
            "kind": "stock PyTorch-ROCm ops on the same GPU (fp32 router, sort by expert, "
                    "per-expert hipBLASLt GEMMs, index_add into fp32); the reference's Triton "
                    "kernels cannot run on the GPU box"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--tokens", type=int, default=64)
    ap.add_argument("--layers", type=int, default=8, help="distinct layer copies cycled over")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-torch-baseline", action="store_true")
    ap.add_argument("--e2e", action="store_true",
                    help="instead: the end-to-end qwen3_moe driver (64 x 512-token prompts, "
                         "256 greedy tokens, 48 random-init layers)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 1 GiB device copy (counter calibration for rocprofv3)")
    ap.add_argument("--traffic-json", default=os.path.join(
        os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic_gate_up_T64.json"),
                    help="HBM traffic per gate_up launch measured with rocprofv3 --pmc")
    ap.add_argument("--block-m", type=int, default=None,
                    help="stage timing with this tile height (0 = expert-major) instead of the plan's")
    ap.add_argument("--no-autotune", action="store_true",
                    help="keep the library's static plan table (by default the expert plans are "
                         "tuned first, as the engine does at start-up: serve.py:1692-1705)")
    ap.add_argument("--profile", action="store_true",
                    help="stage launches only (for rocprofv3 runs; the static plans, or "
                         "--block-m, without tuning launches in the trace); no sweep, no CPU leg")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested)", file=sys.stderr)
        sys.exit(2)

    import torch
    if args.e2e:
        from tinyserve_amd.e2e import run_e2e
        r = run_e2e()
        print(json.dumps({"metric": "qwen3_moe end-to-end greedy generation (random-init "
                                    "Qwen3-30B-A3B, bf16, one GPU)", "e2e": r}), flush=True)
        return
    if args.copy_calibration:
        n = 1 << 30
        src = torch.empty(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n}), flush=True)
        return
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    lib_path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tinyserve_amd",
                            "libtinyserve_moe.so")
    if not os.path.exists(lib_path):
        import __graft_entry__
        __graft_entry__.build()
    import tinyserve_amd as tsm
    from tinyserve_amd._lib import check, lib, ptr

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    g = torch.Generator(device=dev).manual_seed(0)
    L = args.layers
    log(f"allocating {L} layer copies")
    layers = []
    for _ in range(L):
        gw = (torch.randn(E, H, generator=g, device=dev) * 0.02).bfloat16()
        w13 = (torch.randn(E, 2 * I, H, generator=g, device=dev) * 0.02).bfloat16()
        w2 = (torch.randn(E, H, I, generator=g, device=dev) * 0.02).bfloat16()
        layers.append((gw, w13, w2))

    def inputs(T, seed):
        gg = torch.Generator(device=dev).manual_seed(seed)
        return [torch.randn(T, H, generator=gg, device=dev).bfloat16() for _ in range(L)]

    log("packing weights (MFMA-tiled copies)")
    packed = [tsm.pack_moe_weights(w13, w2) for (_, w13, w2) in layers]
    torch.cuda.synchronize()

    plans = None
    if not (args.no_autotune or args.profile):   # profile runs: the static plans or --block-m
        from tinyserve_amd import kernels
        log("autotuning the expert plans (both weight layouts, batches up to 8192 tokens)")
        plans = {}
        for name, (a, b), is_packed in (("packed", packed[0], True),
                                        ("reference", layers[0][1:], False)):
            table = kernels.autotune_fused_moe(a, b, K_TOP, 8192, packed=is_packed)
            plans[name] = {str(k): bm for k, (bm, _) in sorted(table.items())}
        log(json.dumps(plans))

    def forward(i, x, bias, use_packed):
        gw = layers[i][0]
        if use_packed:
            return tsm.moe_forward_packed(x, gw, *packed[i], K_TOP, True, None, bias)
        return tsm.moe_forward(x, *layers[i], K_TOP, True, None, bias)

    def time_layer(T, steps, warmup, bias=None, use_packed=True):
        """HIP-graph replays of the whole layer, cycling the layer copies: one graph holds the L
        copies back to back (as a model's decode graph runs its MoE layers), another the first
        steps % L of them, so the timed region runs exactly `steps` layer steps, each on its own
        weights, without a host graph launch per step. Returns (ms/step, mean touched experts)."""
        xs = inputs(T, 1000 + T)
        touched = []
        for i in range(L):
            _, ids, _ = tsm.moe_router(xs[i], layers[i][0], K_TOP, True, None, bias)
            touched.append(int(torch.unique(ids).numel()))
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for i in range(L):
                forward(i, xs[i], bias, use_packed)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()

        def capture(n):
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                for i in range(n):
                    forward(i, xs[i], bias, use_packed)
            return gr
        full = capture(L)
        rem = steps % L
        part = capture(rem) if rem else None
        for _ in range(max(1, (warmup + L - 1) // L)):  # at least `warmup` untimed steps
            full.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps // L):
            full.replay()
        if part is not None:
            part.replay()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        del full, part
        return ms, sum(touched) / len(touched)

    def time_stages(T, steps, warmup):
        """Per-stage kernel times: every stage is launched `steps` times back to back through the
        C ABI (cycling the layer copies, each with its own routing, permutation and
        intermediates), captured in one HIP graph whose replay is bracketed by a pair of HIP
        events on the replay stream. Returns mean ms per launch of each stage and the tile
        height."""
        xs = inputs(T, 1000 + T)
        numel = T * K_TOP
        bm = int(lib.tsm_moe_block_m(T, H, I, E, K_TOP, 1))  # 0: expert-major, no permutation
        if args.block_m is not None:
            bm = args.block_m
        mp = int(lib.tsm_moe_max_padded(numel, E, bm)) if bm else numel
        nws = int(lib.tsm_moe_align_workspace_size(numel, E, bm)) if bm else 0
        st = []
        for i in range(L):
            st.append(dict(
                w=torch.empty(T, K_TOP, dtype=torch.float32, device=dev),
                ids=torch.empty(T, K_TOP, dtype=torch.int32, device=dev),
                logits=torch.empty(T, E, dtype=torch.float32, device=dev),
                sorted_ids=torch.empty(mp, dtype=torch.int32, device=dev),
                eids=torch.empty(mp // bm if bm else 1, dtype=torch.int32, device=dev),
                total=torch.empty(1, dtype=torch.int32, device=dev),
                aws=torch.empty(max(nws, 1), dtype=torch.uint8, device=dev),
                act=torch.empty(mp, I, dtype=torch.bfloat16, device=dev),
                rows=torch.empty(numel, H, dtype=torch.bfloat16, device=dev),
                out=torch.empty(T, H, dtype=torch.bfloat16, device=dev)))
        def cur():
            return torch.cuda.current_stream().cuda_stream

        def router(i):
            c = st[i]
            check(lib.tsm_moe_router(ptr(xs[i]), ptr(layers[i][0]), 1, T, H, E, K_TOP, 1, None,
                                     None, 0, ptr(c["logits"]), ptr(c["w"]), ptr(c["ids"]), cur()), "router")

        def align(i):
            c = st[i]
            check(lib.tsm_moe_align(ptr(c["ids"]), numel, E, bm, ptr(c["sorted_ids"]),
                                    ptr(c["eids"]), ptr(c["total"]), ptr(c["aws"]), nws, cur()),
                  "align")

        def gate_up(i):
            c = st[i]
            if bm == 0:
                check(lib.tsm_moe_expert_gate_up(ptr(xs[i]), ptr(packed[i][0]), ptr(c["ids"]),
                                                 numel, K_TOP, H, I, E, 1, ptr(c["act"]),
                                                 cur()), "gate_up")
                return
            check(lib.tsm_moe_gemm_gate_up(ptr(xs[i]), ptr(packed[i][0]), ptr(c["sorted_ids"]),
                                           ptr(c["eids"]), ptr(c["total"]), numel, K_TOP, H, I,
                                           E, bm, 1, ptr(c["act"]), cur()), "gate_up")

        def down(i):
            c = st[i]
            if bm == 0:
                check(lib.tsm_moe_expert_down(ptr(c["act"]), ptr(packed[i][1]), ptr(c["w"]),
                                              ptr(c["ids"]), numel, H, I, E, 1, ptr(c["rows"]),
                                              cur()), "down")
                return
            check(lib.tsm_moe_gemm_down(ptr(c["act"]), ptr(packed[i][1]), ptr(c["w"]),
                                        ptr(c["sorted_ids"]), ptr(c["eids"]), ptr(c["total"]),
                                        numel, H, I, E, bm, 1, ptr(c["rows"]), cur()), "down")

        def combine(i):
            c = st[i]
            check(lib.tsm_moe_combine(ptr(c["rows"]), T, H, K_TOP, ptr(c["out"]), cur()),
                  "combine")

        stages = [("router", router), ("align", align), ("gate_up", gate_up), ("down", down),
                  ("combine", combine)]
        if bm == 0:
            stages = [st_ for st_ in stages if st_[0] != "align"]
        for i in range(L):
            for _, fn in stages:
                fn(i)
        torch.cuda.synchronize()
        res = {}
        for name, fn in stages:
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                for j in range(steps):
                    fn(j % L)
            for _ in range(max(1, warmup // max(steps, 1))):
                gr.replay()
            torch.cuda.synchronize()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            gr.replay()
            e1.record()
            torch.cuda.synchronize()
            res[name] = e0.elapsed_time(e1) / steps
            del gr
        return res, bm

    T = args.tokens
    log(f"stage timing T={T}")
    stages_ms, bm = time_stages(T, args.steps, args.warmup)
    if args.profile:
        print(json.dumps({"profile_run": True, "tokens": T, "stages_ms": stages_ms}), flush=True)
        return

    log(f"layer timing T={T}")
    ms, n_touched = time_layer(T, args.steps, args.warmup)
    B = layer_bytes(T, n_touched)
    F = layer_flops(T)
    t = ms * 1e-3
    sb = stage_bytes(T, n_touched)
    sf = stage_flops(T)
    if "align" not in stages_ms:
        sb.pop("align")
    dom = "gate_up"
    dom_t = stages_ms[dom] * 1e-3
    roofline = {
        "kernel": {0: "moe_expert_kernel<gate_up, packed> (gate_up GEMM + SwiGLU epilogue)",
                   16: "moe_stream_kernel<gate_up, packed> (gate_up GEMM + SwiGLU epilogue)"}.get(
                       bm, "moe_tile_kernel<gate_up> (gate_up GEMM + SwiGLU epilogue)"),
        "bound": "hbm",
        "achieved": sb[dom] / dom_t / 1e9,
        "peak": HBM_PEAK / 1e9,
        "unit": "GB/s",
        "frac": sb[dom] / dom_t / HBM_PEAK,
        "traffic": None,  # filled below from the committed rocprofv3 --pmc measurement
        "algorithmic_bytes_per_launch": sb[dom],
        "avg_launch_us": stages_ms[dom] * 1e3,
        "layer_frac_of_roofline": max(B / HBM_PEAK, F / MFMA_BF16_PEAK) / t,
    }
    try:
        tj = json.load(open(args.traffic_json))
        kname = {0: "moe_expert_kernel", 16: "moe_stream_kernel"}.get(bm, "moe_tile_kernel")
        if tj.get("tokens") == T and kname in tj.get("kernel", ""):
            roofline["traffic"] = tj["traffic_bytes"]
            roofline["traffic_source"] = os.path.relpath(args.traffic_json,
                                                         os.path.dirname(args.traffic_json) +
                                                         "/..")
    except (OSError, ValueError, KeyError):
        pass
    res = {
        "metric": "fused-MoE layer HBM GB/s, Qwen3-30B-A3B decode T=64 (bf16)",
        "value": B / t / 1e9,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (x~N(0,1), random-init weights std 0.02, seed 0)",
        "config": {"workload": f"Qwen3-30B-A3B MoE layer decode, T={T} tokens", "tokens": T,
                   "hidden": H, "experts": E, "top_k": K_TOP, "moe_intermediate": I,
                   "norm_topk_prob": True, "layer_copies": L, "block_m": bm,
                   "n_touched": n_touched,
                   # tile height per power-of-two bucket of T*top_k, installed by autotuning
                   # before any timing (null: the static table)
                   "moe_plans": plans},
        "us_per_layer": ms * 1e3,
        "tokens_per_s": T / t,
        "tflops": F / t / 1e12,
        "stages_us": {k: v * 1e3 for k, v in stages_ms.items()},
        "stages_gbps": {k: sb[k] / (stages_ms[k] * 1e-3) / 1e9 for k in sb},
        "roofline": roofline,
        "weights": "MFMA-tiled packed copy (pack_moe_weights), as SparseMoE runs by default",
    }
    ms_ref, _ = time_layer(T, args.steps, args.warmup, use_packed=False)
    res["reference_layout_us_per_layer"] = ms_ref * 1e3
    res["reference_layout_GBps"] = B / (ms_ref * 1e-3) / 1e9

    if not args.no_sweep:
        sweep = []
        for Ts in (1, 8, 64, 256, 512, 2048, 8192):
            steps = 30 if Ts <= 2048 else 12
            mss, nt = time_layer(Ts, steps, 5)
            Bs, Fs = layer_bytes(Ts, nt), layer_flops(Ts)
            ts = mss * 1e-3
            sweep.append({"tokens": Ts, "us": mss * 1e3, "GBps": Bs / ts / 1e9,
                          "TFLOPS": Fs / ts / 1e12, "frac_hbm": Bs / ts / HBM_PEAK,
                          "frac_mfma": Fs / ts / MFMA_BF16_PEAK,
                          "frac_roofline": max(Bs / HBM_PEAK, Fs / MFMA_BF16_PEAK) / ts,
                          "n_touched": nt,
                          "block_m": int(lib.tsm_moe_block_m(Ts, H, I, E, K_TOP, 1))})
            log(json.dumps(sweep[-1]))
        for kind in ("zipf", "half_empty"):
            gen = torch.Generator().manual_seed(1)
            if kind == "zipf":
                p = 1.0 / torch.arange(1, E + 1, dtype=torch.float64) ** 1.2
                p = p[torch.randperm(E, generator=gen)]
                bias = torch.log(p / p.sum()).float().to(dev)
            else:
                bias = torch.zeros(E, device=dev)
                bias[E // 2:] = float("-inf")
            mss, nt = time_layer(2048, 30, 5, bias)
            Bs, Fs = layer_bytes(2048, nt), layer_flops(2048)
            ts = mss * 1e-3
            sweep.append({"tokens": 2048, "stress": kind, "us": mss * 1e3, "GBps": Bs / ts / 1e9,
                          "TFLOPS": Fs / ts / 1e12,
                          "frac_roofline": max(Bs / HBM_PEAK, Fs / MFMA_BF16_PEAK) / ts,
                          "n_touched": nt,
                          "block_m": int(lib.tsm_moe_block_m(2048, H, I, E, K_TOP, 1))})
            log(json.dumps(sweep[-1]))
        res["sweep"] = sweep

    if not args.no_torch_baseline:
        res["torch_gpu_baseline"] = torch_gpu_baseline(layers[0], inputs(T, 1000 + T)[0], T, B)

    if not args.no_cpu_baseline:
        from oracle.moe_oracle import moe_reference, route_torch
        # Every core this process may run on, capped by the host-thread share the job is given
        # (OMP_NUM_THREADS, when the launcher sets one): the torch-CPU path is then timed on all
        # the cores it is allowed, and `cores` says how many that was.
        affinity = len(os.sched_getaffinity(0))
        share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
        threads = min(affinity, share) if share > 0 else affinity
        torch.set_num_threads(threads)
        gw, w13, w2 = (t_.cpu() for t_ in layers[0])
        x = inputs(T, 1000 + T)[0].cpu()
        reps, t0 = 0, time.perf_counter()
        while True:
            logits = (x @ gw.t()).float()
            wc, idc = route_torch(logits, K_TOP, True)
            moe_reference(x, w13, w2, wc, idc)
            reps += 1
            el = time.perf_counter() - t0
            if (el >= args.cpu_seconds and reps >= 3) or el > 4 * args.cpu_seconds:
                break
        tc = el / reps
        nt_c = int(torch.unique(idc).numel())
        res["cpu_baseline"] = {"value": layer_bytes(T, nt_c) / tc / 1e9, "unit": "GB/s",
                               "cores": threads, "host_cpus": os.cpu_count(),
                               "affinity_cpus": affinity, "kind": "port",
                               "sample": f"{reps} layer forwards at T={T} (torch-CPU bf16 "
                                         f"restatement of serve.py router + moe_reference), "
                                         f"{el:.1f} s total, {tc * 1e3:.1f} ms/layer"}
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
