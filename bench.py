"""MoE layer benchmark: Qwen3-30B-A3B-shaped quantized MoE FFN on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A "step" is one HipSparseMoEMLP.forward (router -> top-k -> dispatch -> gate/up + SwiGLU ->
down -> combine) over one batch of synthetic tokens already resident in HBM.  The headline
`value` is decode tok/s at M = 1.  Each step runs one layer forward,
replayed from a HIP graph (one graph per weight copy, no host work inside the timed region).
The same JSON line carries M = 2 / 4 / 8 decode, the M = 4096 Zipf-skewed prefill (config
3), the roofline of the dominant kernel, and the CPU baseline.  The CPU baseline is the
torch-CPU restatement of the reference path, timed on this host.

Weights are rotated over `--copies` device copies (default 32, each with its own token
rows, so each copy routes to its own experts): one rotation reads about 780 MB of distinct
expert bytes at M = 1, three times the 256 MB Infinity Cache, so decode reads come from
HBM.  The line states those bytes (`distinct_weight_bytes_per_rotation`).  Only the GGUF
bytes of the distinct active experts count as algorithmic traffic.

Kernel durations come from pgmoe_moe_forward_timed.  Every kernel of the forward records
HIP events at its own begin and end on the stream it runs on, which is the interval a
kernel trace (rocprofv3 --kernel-trace) reports; the forwards run back to back over the
rotated copies, as in the timed graph replays.  `roofline.frac` takes the dominant
kernel's average from the committed kernel trace of this command
(profiles/trace_bench.json) and reports the live event figure beside it.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for p in (REPO, os.path.join(REPO, "pytorch-engine_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E, published
FP16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA, published
METRIC = "MoE layer tok/s at M=1 and M=4096 (Qwen3-30B-A3B shape); % HBM / MFMA roofline"
TRAFFIC_FILES = [os.path.join(REPO, "profiles", f) for f in ("traffic_dec_moe_qwen3_m1.json",
                                                               "traffic_dec_gu_qwen3_m1.json")]


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--copies", type=int, default=32, help="rotated weight copies (MALL defeat)")
    ap.add_argument("--prefill-steps", type=int, default=10)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-dense", action="store_true", help="skip the dense FFN measurement")
    ap.add_argument("--no-configs", action="store_true", help="skip the Mixtral and Qwen2 + shared configs")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--m-list", default="1,2,4,8", help="decode token counts to time (1 is the headline)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run a plain 256 MiB device copy (calibrates FETCH/WRITE_SIZE counters)")
    return ap.parse_args()


# ----------------------------------------------------------------------------- HIP events
class Hip:
    """The HIP runtime torch loaded (so events and kernels share one runtime)."""

    def __init__(self) -> None:
        path = None
        for line in open("/proc/self/maps"):
            if "libamdhip64" in line:
                path = line.split()[-1]
                break
        self.L = ctypes.CDLL(path or "libamdhip64.so")
        self.L.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.L.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.L.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.L.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def events(self, n: int):
        out = (ctypes.c_void_p * n)()
        for i in range(n):
            h = ctypes.c_void_p()
            if self.L.hipEventCreate(ctypes.byref(h)) != 0:
                raise RuntimeError("hipEventCreate failed")
            out[i] = h.value
        return out

    def elapsed_ms(self, a, b) -> float:
        f = ctypes.c_float()
        if self.L.hipEventElapsedTime(ctypes.byref(f), a, b) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return float(f.value)


# Short names of the forward's kernels (as pgmoe_moe_forward_timed reports their launches).
_KNAMES = (("router_gemm_kernel", "router"), ("router_logits_kernel", "router"), ("topk_kernel", "topk"),
           ("dispatch_count_kernel", "dispatch_count"), ("identity_dispatch_kernel", "sh_dispatch"),
           ("dispatch_kernel", "dispatch"), ("gemm_split_reduce_kernel<true>", "gemm_gateup_reduce"),
           ("gemm_split_reduce_kernel<false>", "gemm_down_reduce"), ("rowscale_kernel", "rowscale"),
           ("rowscale_block_kernel", "rowscale"),
           ("combine_kernel", "combine"), ("dec_gu_kernel", "dec_gu"), ("dec_dc_kernel", "dec_dc"),
           ("dec_dc_chunk_kernel", "dec_dc"), ("dec_down_kernel", "dec_down"))


def short_names(raw):
    """Short labels of the launches: the products by their template's GATEUP flag; after the
    shared expert's identity dispatch, its products (and its gate's router) get "sh_"."""
    out, shared = [], False
    for r in raw:
        if "gemm_kernel<" in r:
            n = "gemm_gateup" if ", true," in r else "gemm_down"
        else:
            n = next((v for k, v in _KNAMES if k in r), r)
        shared = shared or n == "sh_dispatch"
        if shared and n == "router":
            n = "gate"
        out.append("sh_" + n if shared and not n.startswith("sh_") and n != "combine" else n)
    return out


def kernel_durations(torch, hip, mods, xs, reps: int, with_names: bool = False):
    """Average duration (ms) of each kernel of the forward, over `reps` forwards that rotate
    the weight copies (copy i on its own token rows xs[i]) back to back on one stream, as
    the timed graph replays run them, from the events the kernels record themselves (and
    their names).  Two untimed forwards run first."""
    from pgmoe._lib import check, lib
    n_ev = 32
    xs = xs if isinstance(xs, (list, tuple)) else [xs] * len(mods)
    M = xs[0].shape[0]
    stream = torch.cuda.current_stream(xs[0].device).cuda_stream
    starts = [hip.events(n_ev) for _ in range(reps)]
    stops = [hip.events(n_ev) for _ in range(reps)]
    names = (ctypes.c_char_p * n_ev)()
    nl = ctypes.c_int32()
    outs = [torch.empty((M, m.hidden), dtype=torch.float32, device=xs[0].device) for m in mods]
    wss = [m._workspace(M) for m in mods]
    for i in range(2):
        mods[i % len(mods)](xs[i % len(mods)])
    for r in range(reps):
        k = r % len(mods)
        m = mods[k]
        check(lib().pgmoe_moe_forward_timed(m._layer, xs[k].data_ptr(), M, outs[k].data_ptr(), wss[k].data_ptr(),
                                            wss[k].numel(), stream, starts[r], stops[r], n_ev, ctypes.byref(nl),
                                            names), "forward_timed")
    torch.cuda.synchronize()
    names_n = min(nl.value, n_ev)
    sums = [0.0] * names_n
    for r in range(reps):
        for k in range(names_n):
            sums[k] += hip.elapsed_ms(starts[r][k], stops[r][k])
    for evs in starts + stops:
        for k in range(n_ev):
            hip.L.hipEventDestroy(evs[k])
    avg = [s / reps for s in sums]
    if with_names:
        return avg, short_names([names[k].decode() for k in range(names_n)])
    return avg


# ----------------------------------------------------------------------------- timing
def graph_step_ms(torch, mods, xs, steps: int, warmup: int) -> float:
    """Per-step time of exactly `steps` forwards replayed from HIP graphs: one graph holds
    one forward of every weight copy in turn, copy i on its own token rows xs[i] (so a
    replay is `len(mods)` steps), and a second graph of the first `steps % len(mods)`
    copies completes the count.  The timed region is bracketed by synchronizations and
    holds no host work besides the replays."""
    n = len(mods)
    xs = xs if isinstance(xs, (list, tuple)) else [xs] * n
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    outs = []

    def capture(ms):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            o = [m(xs[i]) for i, m in enumerate(ms)]
        return g, o

    with torch.cuda.stream(s):
        for i, m in enumerate(mods):
            m(xs[i])  # allocate the workspaces outside capture
        torch.cuda.synchronize()
        full, outs = capture(mods)
        rem = steps % n
        part = capture(mods[:rem])[0] if rem else None
    torch.cuda.synchronize()
    for _ in range(max(1, warmup // n)):
        full.replay()
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps // n):
        full.replay()
    if part is not None:
        part.replay()
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / steps
    full.replay()
    torch.cuda.synchronize()
    for i, (m, o) in enumerate(zip(mods, outs)):  # the replays compute what eager forwards compute
        if not torch.equal(o, m(xs[i])):
            raise RuntimeError("graph replay differs from the eager forward")
    del full, part
    return ms


def dense_section(torch, oracle, dev, steps: int, warmup: int, prefill_steps: int) -> dict:
    """The dense SwiGLU FFN (HipDenseMLP, the GGUFDenseMLP drop-in) on an 8B-class layer:
    parity against the oracle (M = 1, and a token sample of M = 4096), decode M = 1 from
    graph replays over 6 weight copies (587 MB, past the 256 MB MALL), prefill M = 4096."""
    import numpy as np
    from pgmoe import HipDenseMLP
    from pgmoe.synth import DENSE_CONFIGS, SyntheticDense
    sp = DENSE_CONFIGS["dense_8b"]
    lay = SyntheticDense(sp, seed=0)
    base = HipDenseMLP(lay.gguf, lay.config, 0, dev)
    mats = []
    for qt, proj, shp in zip(sp.qtypes, ("gate", "up", "down"),
                             ((sp.inter, sp.hidden), (sp.inter, sp.hidden), (sp.hidden, sp.inter))):
        mats.append((qt, shp[0], shp[1], np.ascontiguousarray(lay.tensor(f"ffn_{proj}.weight"))))
    parity = {}
    for M, toks in ((1, [0]), (4096, [0, 1777, 4095])):
        x = lay.draw_x(M)
        got = base(torch.from_numpy(x).to(dev)).cpu().numpy()[toks]
        ref = oracle.dense_forward(x, *mats, tokens=toks)
        parity[str(M)] = {"rel_l2": float(f"{oracle.rel_l2(got, ref):.3e}"),
                          "max_rel": float(f"{oracle.max_rel(got, ref):.3e}")}
    ok = all(v["rel_l2"] <= 1e-3 and v["max_rel"] <= 2e-2 for v in parity.values())
    mods = [base] + [base.replica() for _ in range(5)]
    x1, _ = rotation_inputs(torch, lay, None, len(mods), 1, dev)
    ms1 = graph_step_ms(torch, mods, x1, steps, warmup)
    xp = torch.from_numpy(lay.draw_x(4096)).to(dev)
    msp = eager_step_ms(torch, mods[:2], xp, prefill_steps, 2)
    wb = base.weight_bytes()
    n_copies = len(mods)
    gbs = wb / (ms1 * 1e-3) / 1e9
    fl = 2.0 * 4096 * 3 * sp.hidden * sp.inter
    tf = fl / (msp * 1e-3) / 1e12
    del mods, base
    torch.cuda.empty_cache()
    return {"workload": f"dense SwiGLU FFN H={sp.hidden} I={sp.inter}, gate/up Q4_K, down Q6_K",
            "decode_m1": {"us_per_step": round(ms1 * 1e3, 3), "tok_per_s": round(1 / (ms1 * 1e-3), 1),
                          "weight_bytes": wb, "hbm_gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                          "distinct_weight_bytes_per_rotation": wb * n_copies,
                          "timing": f"one forward per HIP graph replay, {n_copies} weight copies"},
            "prefill": {"M": 4096, "us_per_step": round(msp * 1e3, 2), "tok_per_s": round(4096 / (msp * 1e-3), 1),
                        "tflops": round(tf, 1), "mfma_frac": round(tf / FP16_PEAK_TFLOPS, 4)},
            "parity": parity, **({} if ok else {"parity_failed": True})}


def eager_step_ms(torch, mods, xs, steps: int, warmup: int) -> float:
    n = len(mods)
    xs = xs if isinstance(xs, (list, tuple)) else [xs] * n
    for i in range(warmup):
        mods[i % n](xs[i % n])
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(steps):
        mods[i % n](xs[i % n])
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps


def rotation_inputs(torch, lay, ol, n: int, M: int, dev):
    """Token rows for n rotated weight copies: copy i gets its own M rows (rows i*M.. of one
    seeded draw of n*M), so each copy routes to its own experts.  Returns the device tensors
    and, per copy, its distinct active experts (from the oracle's routing; None without a
    router)."""
    import numpy as np
    pool = lay.draw_x(M * n)
    xs_np = [np.ascontiguousarray(pool[i * M:(i + 1) * M]) for i in range(n)]
    xs = [torch.from_numpy(a).to(dev) for a in xs_np]
    acts = [len(np.unique(ol.route(a)[1])) for a in xs_np] if ol is not None else None
    return xs, acts


def copy_probe(torch) -> None:
    """A plain device copy of known size, run when the counters are being calibrated."""
    n = 256 << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"[bench] copy probe: 4 x {n} byte device copies")


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(lay, M: int, seconds: float, threads: int = 0, max_forwards: int = 400, min_forwards: int = 3):
    """The torch-CPU restatement of the reference path (oracle/torch_port.py, fp16 casts
    kept) timed on this host for a bounded sample: forwards of M tokens (after one warm-up
    forward) until `seconds` have passed and at least min_forwards ran, at most
    max_forwards; the rate is M over the median forward time."""
    import statistics
    import torch
    import oracle
    from oracle import torch_port

    cores = len(os.sched_getaffinity(0))
    nthr = threads or cores
    prev = torch.get_num_threads()
    torch.set_num_threads(nthr)
    times = []
    try:
        ol = oracle.OracleLayer.from_gguf(lay.gguf, lay.config, router_bias=lay.router_bias)
        port = torch_port.PortMoE(ol)
        pool = max(M, 64)
        x = torch.from_numpy(lay.draw_x(pool))
        port.forward(x[0:M], faithful=True)  # warm-up
        t_start = time.perf_counter()
        while True:
            o = (len(times) * M) % (pool - M + 1)
            t0 = time.perf_counter()
            port.forward(x[o:o + M], faithful=True)
            times.append(time.perf_counter() - t0)
            el = time.perf_counter() - t_start
            if len(times) >= max_forwards or (len(times) >= min_forwards and el >= seconds):
                break
    finally:
        torch.set_num_threads(prev)
    med = statistics.median(times)
    return {"value": round(M / med, 3), "unit": "tok/s", "cores": nthr, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"{len(times)} forward(s) of M={M} token(s) of the {lay.spec.name} layer, median "
                      f"{med * 1e3:.2f} ms per forward: oracle/torch_port.py, the torch-CPU restatement of the "
                      f"reference CPU path (repacked W4/W8, chunked fp32 dequant + F.linear, fp16 casts kept), "
                      f"{el:.1f} s on {nthr} of {cores} host threads"}


def routing_bit_exact(mod, M: int, idx, oracle) -> bool:
    """Whether the routing the forward just run computed itself (read back from its own
    workspace: at M <= 8 the descriptor the routed gate/up launch published) equals the
    oracle's top-k + stable dispatch: offsets, and per sorted pair its expert and token."""
    import numpy as np
    g_off, g_e, g_t, _ = (t.cpu().numpy() for t in mod.routing(M))
    r_off, r_perm, _ = oracle.dispatch(idx, mod.n_experts)
    return bool(np.array_equal(g_off, r_off) and np.array_equal(g_e, idx.reshape(-1)[r_perm])
                and np.array_equal(g_t, r_perm // idx.shape[1]))


def load_traffic(kernel: str):
    """Counter-derived HBM bytes per launch of `kernel` (a kernel-name prefix), if profiled."""
    for path in TRAFFIC_FILES:
        try:
            with open(path) as f:
                rec = json.load(f)
        except (OSError, ValueError):
            continue
        name = rec.get("kernel_pattern") or rec.get("kernel", "")
        if name.split("pgmoe::")[-1].startswith(kernel):
            rec.setdefault("source", f"{os.path.relpath(path, REPO)}: FETCH_SIZE + WRITE_SIZE of "
                                     f"{name} per dispatch, copy-calibrated")
            return rec.get("bytes_per_launch"), rec
    return None, None


def layer_flops(spec, M: int, pairs: int) -> float:
    f = 2.0 * pairs * 3 * spec.hidden * spec.inter
    if spec.shared_inter:
        f += 2.0 * M * 3 * spec.hidden * spec.shared_inter
    return f


def config_section(torch, oracle, hip, dev, name: str, m_dec: int, m_pf: int, steps: int, warmup: int,
                   pf_steps: int, cpu_seconds: float, copies: int = 3) -> dict:
    """One BASELINE config: parity gate, decode M = m_dec from graph replays over `copies`
    weight copies (HBM fraction of the active GGUF bytes), prefill M = m_pf eager (MFMA
    fraction of the grouped GEMMs and of the layer; for a shared expert also the HBM
    fraction of every byte the step reads), and the CPU baseline at M = m_dec."""
    import numpy as np
    from pgmoe import HipSparseMoEMLP
    from pgmoe.synth import CONFIGS, SyntheticLayer
    spec = CONFIGS[name]
    lay = SyntheticLayer(spec, seed=0)
    base = HipSparseMoEMLP(lay.gguf, lay.config, 0, dev)
    mods = [base] + [base.replica() for _ in range(copies - 1)]
    ol = oracle.OracleLayer.from_gguf(lay.gguf, lay.config)
    out = {"workload": f"{name}: H={spec.hidden} E={spec.n_experts} top-{spec.top_k} I={spec.inter}"
                       + (f" + shared I={spec.shared_inter}" if spec.shared_inter else "")
                       + f", GGUF types {list(spec.qtypes)}", "weight_copies": copies}
    parity = {}
    for M, toks in ((m_dec, None), (m_pf, [0, m_pf // 2, m_pf - 1])):
        xg = lay.draw_x(M)
        got = base(torch.from_numpy(xg).to(dev)).cpu().numpy()
        logits, idx, w = ol.route(xg)
        tk = np.arange(M) if toks is None else np.array(toks)
        ref = ol.forward_tokens(xg, idx, w, tokens=tk)
        parity[str(M)] = {"rel_l2": float(f"{oracle.rel_l2(got[tk], ref):.3e}"),
                          "max_rel": float(f"{oracle.max_rel(got[tk], ref):.3e}"),
                          "routing_bit_exact": routing_bit_exact(base, M, idx, oracle), "rows_checked": len(tk)}
    out["parity"] = parity
    ok = all(v["rel_l2"] <= 1e-3 and v["max_rel"] <= 2e-2 and v["routing_bit_exact"] for v in parity.values())
    # decode: every copy on its own token rows
    xs, acts = rotation_inputs(torch, lay, ol, len(mods), m_dec, dev)
    ms = graph_step_ms(torch, mods, xs, steps, warmup)
    per_exp = base.active_weight_bytes(1)
    wb = round(sum(acts) / len(acts) * per_exp) + base.shared_weight_bytes()
    kd = kernel_durations(torch, hip, mods, xs, 20)
    gbs = wb / (ms * 1e-3) / 1e9
    out["decode"] = {"M": m_dec, "us_per_step": round(ms * 1e3, 3), "tok_per_s": round(m_dec / (ms * 1e-3), 1),
                     "active_experts": round(sum(acts) / len(acts), 2), "weight_bytes": wb,
                     "hbm_gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                     "kernel_us": [round(v * 1e3, 3) for v in kd],
                     "distinct_weight_bytes_per_rotation": sum(acts) * per_exp + len(mods) * base.shared_weight_bytes(),
                     "timing": f"one forward per HIP graph replay, {copies} weight copies"}
    # prefill
    xp_np = lay.draw_x(m_pf)
    xp = torch.from_numpy(xp_np).to(dev)
    msp = eager_step_ms(torch, mods, xp, pf_steps, 2)
    kd, names = kernel_durations(torch, hip, mods, [xp] * len(mods), max(3, pf_steps // 2), with_names=True)
    _, idxp, _ = ol.route(xp_np)
    n_act_p = len(np.unique(idxp))
    fl = layer_flops(spec, m_pf, m_pf * spec.top_k)
    gemm_ms = sum(v for n, v in zip(names, kd) if "gemm" in n)
    wbp = base.active_weight_bytes(n_act_p) + base.shared_weight_bytes()
    out["prefill"] = {"M": m_pf, "us_per_step": round(msp * 1e3, 2), "tok_per_s": round(m_pf / (msp * 1e-3), 1),
                      "kernels": names, "kernel_us": [round(v * 1e3, 2) for v in kd], "flops": fl,
                      "gemm_mfma_frac": round(fl / (gemm_ms * 1e-3) / 1e12 / FP16_PEAK_TFLOPS, 4),
                      "layer_mfma_frac": round(fl / (msp * 1e-3) / 1e12 / FP16_PEAK_TFLOPS, 4),
                      "active_experts": n_act_p, "weight_bytes": wbp,
                      "layer_hbm_frac": round(wbp / (msp * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    del mods, base
    torch.cuda.empty_cache()
    if cpu_seconds > 0:
        out["cpu_baseline"] = cpu_baseline(lay, m_dec, cpu_seconds, max_forwards=50)
    if not ok:
        out["parity_failed"] = True
    return out


def load_trace_avg(kernel: str):
    """Average duration (us) of `kernel` (a name prefix) in the committed kernel-trace
    summary of this benchmark, if one is there."""
    try:
        with open(os.path.join(REPO, "profiles", "trace_bench.json")) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    for k, v in rec.get("kernels", {}).items():
        if k.split("pgmoe::")[-1].startswith(kernel):
            return v.get("avg_us")
    return None


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; multi-GPU figures are not produced",
                          "n_gpus": args.gpus}), flush=True)
        return 2
    import numpy as np
    import torch
    import oracle
    from pgmoe import HipSparseMoEMLP
    from pgmoe.synth import CONFIGS, SyntheticLayer

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    hip = Hip()
    props = torch.cuda.get_device_properties(dev)
    spec = CONFIGS["qwen3_30b_a3b"]
    log(f"[bench] device {props.name} CUs={props.multi_processor_count}; building {spec.name} "
        f"+ {args.copies - 1} weight copies")
    if args.copy_probe:
        copy_probe(torch)
    lay = SyntheticLayer(spec, seed=0)
    base = HipSparseMoEMLP(lay.gguf, lay.config, 0, dev)
    mods = [base] + [base.replica() for _ in range(max(0, args.copies - 1))]
    ol = oracle.OracleLayer.from_gguf(lay.gguf, lay.config)

    # ---- correctness gate on the benchmarked layer (M = 1 and M = 8), the routing read
    # back from the timed forward's own workspace
    gate = {}
    for M in (1, 8):
        xg = lay.draw_x(M)
        xt = torch.from_numpy(xg).to(dev)
        got = base(xt).cpu().numpy()
        logits, idx, w = ol.route(xg)
        ref = ol.forward_tokens(xg, idx, w)
        gate[M] = {"rel_l2": oracle.rel_l2(got, ref), "max_rel": oracle.max_rel(got, ref),
                   "topk_bit_exact": routing_bit_exact(base, M, idx, oracle),
                   "min_topk_margin": oracle.min_topk_margin(logits, spec.top_k)}
        log(f"[bench] parity M={M}: {gate[M]}")
        if not (gate[M]["rel_l2"] <= 1e-3 and gate[M]["max_rel"] <= 2e-2 and gate[M]["topk_bit_exact"]):
            log("[bench] PARITY FAILED")
            return 1

    # ---- decode: graph-replayed steps (headline M = 1), eager for reference
    decode = {}
    m_list = sorted({1} | {int(v) for v in args.m_list.split(",") if v})
    for M in m_list:
        # every copy on its own token rows, so each routes to its own experts
        xs, acts = rotation_inputs(torch, lay, ol, len(mods), M, dev)
        # every M is timed like the headline: --warmup untimed, then --steps timed forwards
        steps, warm = args.steps, args.warmup
        ms = graph_step_ms(torch, mods, xs, steps, warm)
        ms_eager = eager_step_ms(torch, mods, xs, max(50, steps // 4), 10)
        kd = kernel_durations(torch, hip, mods, xs, 64)
        per_exp = base.active_weight_bytes(1)
        n_act = sum(acts) / len(acts)
        ab = round(n_act * per_exp)
        decode[M] = {"us_per_step": round(ms * 1e3, 3), "tok_per_s": round(M / (ms * 1e-3), 1),
                     "steps": steps, "eager_us_per_step": round(ms_eager * 1e3, 3),
                     "active_experts": round(n_act, 3), "kernel_us": [round(v * 1e3, 3) for v in kd],
                     "active_weight_bytes": ab,
                     "distinct_weight_bytes_per_rotation": sum(acts) * per_exp,
                     "layer_hbm_frac": round(ab / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        log(f"[bench] decode M={M}: {decode[M]}")

    # dominant kernel at M = 1: the routed gate/up launch (router folded in, routing, gate/up
    # + SwiGLU).  Its algorithmic bytes are the active experts' gate and up GGUF bytes (the
    # 1 MiB fp32 router weights it also reads are reported beside them, not counted).
    d1 = decode[1]
    ku = d1["kernel_us"]
    router_bytes = spec.n_experts * spec.hidden * 4
    gu_mat = base.gate_exps.gguf_bytes_per_mat + base.up_exps.gguf_bytes_per_mat
    dom_kernel, dom_names = "dec_gu_kernel", ["dec_gu", "dec_dc"]
    dom_desc = "dec_gu_kernel (router + routing + gate/up + SwiGLU), M=1"
    dom_bytes = spec.top_k * gu_mat  # one token: top_k distinct experts every step
    ev_us = ku[0]
    trace_us = load_trace_avg("dec_gu_kernel<12, 1, 1, 2, false>")
    # frac from the committed kernel trace of this command when it holds the kernel, the
    # live event average beside it
    dom_us = trace_us if trace_us else ev_us
    dom_gbs = dom_bytes / (dom_us * 1e-6) / 1e9
    layer_gbs = d1["active_weight_bytes"] / (d1["us_per_step"] * 1e-6) / 1e9
    traffic, traffic_rec = load_traffic(dom_kernel)

    # ---- prefill M = 4096 with the Zipf router bias (config 3)
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
        xp_np = play.draw_x(M)
        xp = torch.from_numpy(xp_np).to(dev)
        got = pm(xp)
        pol = oracle.OracleLayer.from_gguf(play.gguf, play.config, router_bias=play.router_bias)
        _, pidx, pw = pol.route(xp_np)
        prouting = routing_bit_exact(pm, M, pidx, oracle)
        ptoks = np.array([0, 2047, 4095])
        pref = pol.forward_tokens(xp_np, pidx, pw, tokens=ptoks)
        pgot = got.cpu().numpy()[ptoks]
        ms = eager_step_ms(torch, pmods, xp, args.prefill_steps, 2)
        kd, names = kernel_durations(torch, hip, pmods, xp, max(3, args.prefill_steps // 2), with_names=True)
        i_gu, i_dn = names.index("gemm_gateup"), names.index("gemm_down")
        P = M * pspec.top_k
        fl_gu = 2.0 * P * pspec.hidden * 2 * pspec.inter
        fl_dn = 2.0 * P * pspec.inter * pspec.hidden
        gu_tf = fl_gu / (kd[i_gu] * 1e-3) / 1e12
        dn_tf = fl_dn / (kd[i_dn] * 1e-3) / 1e12
        both_tf = (fl_gu + fl_dn) / ((kd[i_gu] + kd[i_dn]) * 1e-3) / 1e12
        side_us = sum(v for n, v in zip(names, kd) if "gemm" not in n) * 1e3
        prefill = {"M": M, "us_per_step": round(ms * 1e3, 2), "tok_per_s": round(M / (ms * 1e-3), 1),
                   "kernel_us": [round(v * 1e3, 2) for v in kd], "kernels": names,
                   "gemm_gateup_tflops": round(gu_tf, 1), "gemm_down_tflops": round(dn_tf, 1),
                   "gemm_tflops": round(both_tf, 1), "mfma_frac": round(both_tf / FP16_PEAK_TFLOPS, 4),
                   "layer_tflops": round((fl_gu + fl_dn) / (ms * 1e-3) / 1e12, 1),
                   "layer_mfma_frac": round((fl_gu + fl_dn) / (ms * 1e-3) / 1e12 / FP16_PEAK_TFLOPS, 4),
                   "side_kernels_us": round(side_us, 2),
                   "parity": {"rel_l2": float(f"{oracle.rel_l2(pgot, pref):.3e}"),
                              "max_rel": float(f"{oracle.max_rel(pgot, pref):.3e}"),
                              "routing_bit_exact": prouting, "rows_checked": len(ptoks)}}
        log(f"[bench] prefill M=4096: {prefill}")
        del pmods, pm, got
        torch.cuda.empty_cache()
        if not (prouting and prefill["parity"]["rel_l2"] <= 1e-3 and prefill["parity"]["max_rel"] <= 2e-2):
            log("[bench] PREFILL PARITY FAILED")
            return 1

    configs = {}
    if not args.no_configs:
        for cname, m_dec, m_pf in (("mixtral_8x7b", 1, 2048), ("qwen2_57b_a14b", 1, 512)):
            configs[cname] = config_section(torch, oracle, hip, dev, cname, m_dec, m_pf, max(50, args.steps // 4),
                                            10, args.prefill_steps,
                                            0.0 if args.no_cpu_baseline else args.cpu_seconds / 2)
            log(f"[bench] {cname}: {configs[cname]}")
            if configs[cname].get("parity_failed"):
                log(f"[bench] {cname} PARITY FAILED")
                return 1

    dense = None
    if not args.no_dense:
        dense = dense_section(torch, oracle, dev, args.steps, args.warmup, args.prefill_steps)
        log(f"[bench] dense: {dense}")
        if dense.get("parity_failed"):
            log("[bench] DENSE PARITY FAILED")
            return 1

    cpu = None
    cpu_more = {}
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(lay, 1, args.cpu_seconds)
        log(f"[bench] cpu baseline: {cpu}")
        cpu_more["qwen3_m1_1thread"] = cpu_baseline(lay, 1, args.cpu_seconds / 2, threads=1)
        if not args.no_prefill:
            cpu_more["qwen3_zipf_prefill_m4096"] = cpu_baseline(play, 4096, 1.0, max_forwards=5, min_forwards=3)
        log(f"[bench] cpu baselines: {cpu_more}")

    rec = {
        "metric": METRIC,
        "value": d1["tok_per_s"],
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(d1["us_per_step"] / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "qwen3_30b_a3b MoE layer decode, M=1 token per step (H=2048, E=128, top-8, "
                               "I=768, gate/up Q4_K, down Q6_K, fp16 activations, fp32 accumulate)",
                   "weight_copies": args.copies,
                   "distinct_weight_bytes_per_rotation": d1["distinct_weight_bytes_per_rotation"],
                   "timing": "one forward per HIP graph replay, each weight copy on its own token rows"},
        "roofline": {"bound": "hbm", "achieved": round(dom_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": dom_desc, "algorithmic_bytes": dom_bytes,
                     "algorithmic_bytes_note": f"{spec.top_k} active experts x ({gu_mat:,} gate + up GGUF "
                                               "bytes); the launch also reads the fp32 router weights "
                                               f"({router_bytes:,} B), not counted",
                     "kernel_us": round(dom_us, 3),
                     "kernel_us_source": ("average of the kernel in the rocprofv3 kernel trace of this command, "
                                          "profiles/trace_bench.json" if trace_us else
                                          "HIP events the kernel records at its own begin / end (no committed "
                                          "trace holds this kernel)"),
                     "event_us": ev_us,
                     "event_us_source": "HIP events the kernel records at its own begin / end, average over 64 "
                                        "back-to-back forwards rotating the weight copies",
                     "frac_from_events": round(dom_bytes / (ev_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "router_inclusive_gbs": round((dom_bytes + router_bytes) / (dom_us * 1e-6) / 1e9, 1),
                     "traffic_source": traffic_rec.get("source") if traffic_rec else None},
        "cpu_baseline": cpu,
        "cpu_baselines_more": cpu_more or None,
        "decode": {str(k): v for k, v in decode.items()},
        "kernels_m1": {"names": dom_names, "us": ku,
                       "layer_active_gbs": round(layer_gbs, 1),
                       "layer_hbm_frac": round(layer_gbs / HBM_PEAK_GBS, 4)},
        "prefill": prefill,
        "configs": configs or None,
        "dense": dense,
        "parity": {str(M): {k: (float(f"{v:.3e}") if isinstance(v, float) else v) for k, v in g.items()}
                   for M, g in gate.items()},
    }
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
