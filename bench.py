"""MoE layer benchmark: Qwen3-30B-A3B-shaped quantized MoE FFN on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A "step" is one HipSparseMoEMLP.forward (router -> top-k -> dispatch -> gate/up+SwiGLU ->
down -> combine) over one batch of synthetic tokens already resident in HBM.  The headline
`value` is decode tok/s at M=1; the same JSON line carries M=2/4/8
decode, M=4096 Zipf-skewed prefill (config 3), the roofline of the dominant kernel and
the CPU baseline (the torch-CPU restatement of the reference path, timed on this host).

Weights are rotated over >= 8 device copies so decode reads come from HBM rather than the
256 MB Infinity Cache.  Only the GGUF bytes of distinct active experts count as traffic.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for p in (REPO, os.path.join(REPO, "pytorch-engine_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0     # MI355X HBM3E, published
FP16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA, published


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--copies", type=int, default=8, help="rotated weight copies (MALL defeat)")
    ap.add_argument("--prefill-steps", type=int, default=10)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    return ap.parse_args()


class Timer:
    """HIP events on the current stream."""

    def __init__(self, torch):
        self.torch = torch
        self.a = torch.cuda.Event(enable_timing=True)
        self.b = torch.cuda.Event(enable_timing=True)

    def __enter__(self):
        self.torch.cuda.synchronize()
        self.a.record()
        return self

    def __exit__(self, *exc):
        self.b.record()
        self.torch.cuda.synchronize()
        self.ms = self.a.elapsed_time(self.b)


def time_forward(torch, mods, xs, steps, warmup):
    n = len(mods)
    for i in range(warmup):
        mods[i % n](xs[i % len(xs)])
    with Timer(torch) as t:
        for i in range(steps):
            mods[i % n](xs[i % len(xs)])
    return t.ms / steps


def stage_kernel_times(torch, mods, x, steps):
    """Average duration of the gate/up and down expert kernels, measured with events
    around each launch while running the staged forward on the current stream."""
    from pgmoe import ops
    n = len(mods)
    m0 = mods[0]
    M = x.shape[0]
    mode = 0 if M <= 8 else 1
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    prep = []
    for m in mods:
        _, idx, tw = ops.router_topk(x, m.router_weight, m.router_bias, m.top_k, m.norm_topk_prob)
        prep.append((ops.dispatch(idx, m.n_experts, 64), tw))
    torch.cuda.synchronize()
    for i in range(steps + 3):
        m = mods[i % n]
        disp, tw = prep[i % n]
        e = ev[i - 3] if i >= 3 else None
        if e:
            e[0].record()
        inter = ops.expert_gateup(m.gate_exps.weights(), m.up_exps.weights(), x, m.top_k, disp, mode)
        if e:
            e[1].record()
        ops.expert_down(m.down_exps.weights(), inter, M, m.top_k, disp, tw, mode)
        if e:
            e[2].record()
    torch.cuda.synchronize()
    gu = sum(e[0].elapsed_time(e[1]) for e in ev) / steps
    dn = sum(e[1].elapsed_time(e[2]) for e in ev) / steps
    n_active = int(prep[0][0][4].cpu()[0])
    return gu, dn, n_active


def cpu_baseline(spec, lay, M, seconds):
    import numpy as np
    import torch
    import oracle
    from oracle import torch_port

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    ol = oracle.OracleLayer.from_gguf(lay.gguf, lay.config, router_bias=lay.router_bias)
    port = torch_port.PortMoE(ol)
    x = torch.from_numpy(lay.draw_x(64))
    port.forward(x[0:M], faithful=True)  # warmup
    n, t0 = 0, time.perf_counter()
    while True:
        port.forward(x[(n * M) % 64:(n * M) % 64 + M], faithful=True)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= 200:
            break
    return {"value": round(n * M / el, 3), "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"{n} forwards of M={M} tokens of the same layer (torch-CPU restatement of the "
                      f"reference CPU path, fp16 casts kept), {el:.1f} s, {cores} threads"}


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; multi-GPU figures are not produced",
                          "n_gpus": args.gpus}))
        return 2
    import numpy as np
    import torch
    import oracle
    from pgmoe import HipSparseMoEMLP
    from pgmoe.synth import CONFIGS, SyntheticLayer

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    props = torch.cuda.get_device_properties(dev)
    spec = CONFIGS["qwen3_30b_a3b"]
    log(f"[bench] device {props.name} CUs={props.multi_processor_count}; building {spec.name}")
    lay = SyntheticLayer(spec, seed=0)
    base = HipSparseMoEMLP(lay.gguf, lay.config, 0, dev)
    mods = [base] + [base.replica() for _ in range(max(0, args.copies - 1))]
    per_expert = base.active_weight_bytes(1)
    ol = oracle.OracleLayer.from_gguf(lay.gguf, lay.config)

    # correctness gate on the benchmarked layer
    x1 = lay.draw_x(1)
    got = base(torch.from_numpy(x1).to(dev)).cpu().numpy()
    logits, idx, w = ol.route(x1)
    ref = ol.forward_tokens(x1, idx, w)
    gate = {"rel_l2": oracle.rel_l2(got, ref), "max_rel": oracle.max_rel(got, ref),
            "min_topk_margin": oracle.min_topk_margin(logits, spec.top_k)}
    log(f"[bench] parity M=1: {gate}")
    if not (gate["rel_l2"] <= 1e-3 and gate["max_rel"] <= 2e-2):
        log("[bench] PARITY FAILED")
        return 1

    decode = {}
    for M in (1, 2, 4, 8):
        xs = [torch.from_numpy(lay.draw_x(M)).to(dev)]
        ms = time_forward(torch, mods, xs, args.steps, args.warmup)
        decode[M] = {"ms_per_step": ms, "tok_per_s": M / (ms * 1e-3)}
        log(f"[bench] decode M={M}: {ms * 1e3:.2f} us/layer, {M / (ms * 1e-3):.0f} tok/s")
    xk = torch.from_numpy(x1).to(dev)
    gu_ms, dn_ms, n_act = stage_kernel_times(torch, mods, xk, args.steps)
    gu_bytes = n_act * (base.gate_exps.gguf_bytes_per_mat + base.up_exps.gguf_bytes_per_mat)
    dn_bytes = n_act * base.down_exps.gguf_bytes_per_mat
    gu_gbs = gu_bytes / (gu_ms * 1e-3) / 1e9
    dn_gbs = dn_bytes / (dn_ms * 1e-3) / 1e9
    both_gbs = (gu_bytes + dn_bytes) / ((gu_ms + dn_ms) * 1e-3) / 1e9
    log(f"[bench] kernels M=1: gateup {gu_ms * 1e3:.2f} us {gu_gbs:.0f} GB/s; down {dn_ms * 1e3:.2f} us "
        f"{dn_gbs:.0f} GB/s; experts {both_gbs:.0f} GB/s ({n_act} experts)")

    prefill = None
    if not args.no_prefill:
        del mods
        torch.cuda.empty_cache()
        pspec = CONFIGS["qwen3_30b_a3b_zipf"]
        play = SyntheticLayer(pspec, seed=0)
        pm = HipSparseMoEMLP(play.gguf, play.config, 0, dev)
        pm.set_router_bias(torch.from_numpy(play.router_bias))
        pmods = [pm, pm.replica()]
        M = 4096
        xp = torch.from_numpy(play.draw_x(M)).to(dev)
        ms = time_forward(torch, pmods, [xp], args.prefill_steps, 2)
        gu_p, dn_p, n_act_p = stage_kernel_times(torch, pmods, xp, args.prefill_steps)
        P = M * pspec.top_k
        fl_gu = 2.0 * P * pspec.hidden * 2 * pspec.inter
        fl_dn = 2.0 * P * pspec.inter * pspec.hidden
        mfma = (fl_gu + fl_dn) / ((gu_p + dn_p) * 1e-3) / 1e12
        prefill = {"M": M, "ms_per_step": round(ms, 4), "tok_per_s": round(M / (ms * 1e-3), 1),
                   "gateup_ms": round(gu_p, 4), "down_ms": round(dn_p, 4),
                   "gemm_tflops": round(mfma, 2), "mfma_frac": round(mfma / FP16_PEAK_TFLOPS, 4),
                   "active_experts": n_act_p}
        log(f"[bench] prefill M=4096: {prefill}")
        del pmods, pm
        torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(spec, lay, 1, args.cpu_seconds)
        log(f"[bench] cpu baseline: {cpu}")

    ms1 = decode[1]["ms_per_step"]
    rec = {
        "metric": "MoE layer tok/s at M=1 (Qwen3-30B-A3B shape)",
        "value": round(decode[1]["tok_per_s"], 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms1, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "qwen3_30b_a3b MoE layer decode M=1: H=2048, E=128, top-8, I=768, "
                               "gate/up Q4_K, down Q6_K, fp16 activations",
                   "weight_copies": args.copies},
        "roofline": {"bound": "hbm", "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "gemv_gateup_kernel (gate+up GGUF bytes of the distinct active experts)"},
        "cpu_baseline": cpu,
        "decode": {str(k): {"tok_per_s": round(v["tok_per_s"], 1), "us_per_step": round(v["ms_per_step"] * 1e3, 2)}
                   for k, v in decode.items()},
        "kernels_m1": {"gateup_us": round(gu_ms * 1e3, 3), "gateup_gbs": round(gu_gbs, 1),
                       "down_us": round(dn_ms * 1e3, 3), "down_gbs": round(dn_gbs, 1),
                       "experts_gbs": round(both_gbs, 1), "experts_hbm_frac": round(both_gbs / HBM_PEAK_GBS, 4),
                       "active_bytes": int(gu_bytes + dn_bytes)},
        "prefill": prefill,
        "parity": {k: float(f"{v:.3e}") for k, v in gate.items()},
    }
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
