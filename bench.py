"""MoE-layer throughput benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
                    [--workload mixtral|dsv2lite|ep128-share|mixtral-fp8|mixtral-adam]
                    [--no-cpu-baseline]

One step is one forward + backward of the MoE layer over one batch of
synthetic tokens, with inputs and weights already resident in HBM.  The
default workload is the Mixtral-8x7B layer shape (hidden 4096, 8 experts,
ffn 14336 SwiGLU, top-2 softmax router in float32, 8192 tokens, bfloat16).
Weights are random N(0, 0.02) of the architecture, drawn on the device;
tokens are N(0, 1).  The other workloads are the fine-grained layer with
shared experts and a sigmoid router with selection bias (dsv2lite), one
GPU's 16-expert share of a 128-expert top-8 layer under a Zipf(1.1)
selection prior (ep128-share), and the Mixtral shape with 16384 tokens and
fp8 experts under delayed scaling (mixtral-fp8; its step includes the end of
iteration amax-history roll).  ``--workload mixtral-adam`` instead times the
optimizer step after the layer: one fused Adam step over the Mixtral layer's
parameters, gradients and moments, against the HBM roofline.

Prints one JSON line: whole-job tokens/s, the grouped-GEMM roofline fraction
(algorithmic FLOPs / the GEMM kernels' HIP-event time / dense bf16 peak),
the permute/combine HBM fraction, a per-entry-point time breakdown, and the
CPU baseline: the float64/float32 torch restatement of the reference layer
(oracle/moe_ref.py) timed on this host's cores on a bounded token sample.
"""

from __future__ import annotations

import argparse
import ctypes
import importlib.util
import json
import os
import pathlib
import sys
import time

import torch

ROOT = pathlib.Path(__file__).resolve().parent
PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA
PEAK_HBM_GBPS = 8000.0        # MI355X HBM3E

WORKLOADS = {
    # name: (tokens, hidden, ffn, experts, top_k, score, num_shared, window, n_src, selection bias, fp8)
    "mixtral": (8192, 4096, 14336, 8, 2, "softmax", 0, None, 1, None, False),
    "dsv2lite": (16384, 2048, 1408, 64, 6, "sigmoid", 2, None, 1, "normal", False),
    "ep128-share": (32768, 2048, 768, 128, 8, "softmax", 0, (0, 16), 8, "zipf", False),
    "mixtral-fp8": (16384, 4096, 14336, 8, 2, "softmax", 0, None, 1, None, True),
}
# Workloads that start from a received buffer (the receiving side of the expert exchange) instead of
# routing their own tokens through the whole layer.
RECEIVED = {"ep128-share"}

GEMM_CALLS = ("rhp_expert_fc1_fwd", "rhp_expert_fc2_fwd", "rhp_expert_fc2_bwd", "rhp_expert_fc1_bwd", "rhp_fp8_gemm",
              "rhp_fp8_gemm_cast", "rhp_expert_fc1_fwd_gather", "rhp_expert_fc2_fwd_scatter",
              "rhp_expert_fc2_dgrad_gather", "rhp_expert_fc1_dgrad_scatter", "rhp_expert_fc1_dgrad_router")
PEAK_FP8_TFLOPS = 5000.0      # MI355X dense fp8 MFMA


def _package():
    name = "resihp_megatron_amd"
    if name in sys.modules:
        return sys.modules[name]
    pkg_dir = ROOT / "resihp-megatron_amd"
    spec = importlib.util.spec_from_file_location(name, pkg_dir / "__init__.py",
                                                  submodule_search_locations=[str(pkg_dir)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


class _HipEvent:
    """A HIP timing event created with hipEventDisableSystemFence: recording it takes a timestamp without
    the system-scope release (L2 write-back) a default event performs, which left about 10 us between
    the launches around it.  Only timestamps are read from these events."""

    _lib = None
    DISABLE_SYSTEM_FENCE = 0x20000000   # hipEventDisableSystemFence

    def __init__(self):
        if _HipEvent._lib is None:
            lib = ctypes.CDLL("libamdhip64.so")
            lib.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
            lib.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
            lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
            lib.hipEventDestroy.argtypes = [ctypes.c_void_p]
            _HipEvent._lib = lib
        self.ev = ctypes.c_void_p()
        if _HipEvent._lib.hipEventCreateWithFlags(ctypes.byref(self.ev), self.DISABLE_SYSTEM_FENCE) != 0:
            raise RuntimeError("hipEventCreateWithFlags failed")

    def record(self, stream):
        if _HipEvent._lib.hipEventRecord(self.ev, ctypes.c_void_p(stream.cuda_stream)) != 0:
            raise RuntimeError("hipEventRecord failed")

    def elapsed_time(self, end) -> float:
        ms = ctypes.c_float()
        if _HipEvent._lib.hipEventElapsedTime(ctypes.byref(ms), self.ev, end.ev) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value

    def __del__(self):
        if _HipEvent._lib is not None and self.ev:
            _HipEvent._lib.hipEventDestroy(self.ev)


class EventTimer:
    """HIP events around every C-ABI call, on the stream the call enqueues on."""

    def __init__(self):
        self.pending: dict[str, list] = {}
        self.pairs: list[tuple[str, _HipEvent, _HipEvent]] = []

    def start(self, name, stream):
        ev = _HipEvent()
        ev.record(stream)
        self.pending.setdefault(name, []).append(ev)

    def stop(self, name, stream):
        ev = _HipEvent()
        ev.record(stream)
        self.pairs.append((name, self.pending[name].pop(), ev))

    def totals_ms(self) -> dict[str, tuple[float, int]]:
        out: dict[str, tuple[float, int]] = {}
        for name, a, b in self.pairs:
            t, n = out.get(name, (0.0, 0))
            out[name] = (t + a.elapsed_time(b), n + 1)
        return out

    def union_ms(self, names) -> float:
        """Time covered by the calls of ``names``: the union of their intervals, so calls that run at
        once on two streams count once."""
        pairs = [(a, b) for n, a, b in self.pairs if n in names]
        if not pairs:
            return 0.0
        t0 = pairs[0][0]
        iv = sorted((t0.elapsed_time(a), t0.elapsed_time(b)) for a, b in pairs)
        total, cur_s, cur_e = 0.0, iv[0][0], iv[0][1]
        for s_, e_ in iv[1:]:
            if s_ > cur_e:
                total += cur_e - cur_s
                cur_s, cur_e = s_, e_
            else:
                cur_e = max(cur_e, e_)
        return total + cur_e - cur_s


def build_workload(name: str, dev: torch.device):
    T, h, f, E, k, score, S, window, n_src, bias_kind, fp8 = WORKLOADS[name]
    e0, e1 = window or (0, E)
    g = torch.Generator(device=dev).manual_seed(1234)

    def randn(*shape, std=1.0, dtype=torch.bfloat16):
        return (torch.randn(*shape, generator=g, device=dev, dtype=torch.float32) * std).to(dtype)

    router = randn(E, h, std=0.02, dtype=torch.float32).requires_grad_(True)
    fc1 = [randn(2 * f, h, std=0.02).requires_grad_(True) for _ in range(e1 - e0)]
    fc2 = [randn(h, f, std=0.02).requires_grad_(True) for _ in range(e1 - e0)]
    s1 = [randn(2 * f, h, std=0.02).requires_grad_(True) for _ in range(S)]
    s2 = [randn(h, f, std=0.02).requires_grad_(True) for _ in range(S)]
    if bias_kind == "normal":
        bias = randn(E, std=0.1, dtype=torch.float32)
    elif bias_kind == "zipf":   # selection prior of a Zipf(1.1) expert popularity: -1.1 ln(e + 1)
        bias = (-1.1 * torch.log(torch.arange(1, E + 1, dtype=torch.float64))).float().to(dev)
    else:
        bias = None
    x = randn(T, h).requires_grad_(True)
    dout = randn(T, h)
    st = None
    if fp8:
        _package()
        from resihp_megatron_amd.fp8 import Fp8State
        st = Fp8State(e1 - e0, 16, device=dev)
    return dict(T=T, h=h, f=f, E=E, k=k, score=score, S=S, e0=e0, e1=e1, n_src=n_src, router=router, fc1=fc1,
                fc2=fc2, s1=s1, s2=s2, bias=bias, x=x, dout=dout, fp8=st)


def build_received(pkg, w, dev):
    """The received buffer of the GPU holding the local window: the workload's tokens are split into
    n_src sources (even_split), routed once, and every source's rows for the local experts are laid out
    source-major, expert-major within a source, (token, slot) ascending within an expert -- the order
    the reference's dispatch exchange delivers (resihp/runtime/moe.py:193-212).  Built once, before
    timing (it stands for what the all-to-all delivers)."""
    import importlib

    K = importlib.import_module(f"{pkg.__name__}.kernels")
    T, k, E, e0, e1, n_src = w["T"], w["k"], w["E"], w["e0"], w["e1"], w["n_src"]
    with torch.no_grad():
        _, topi, _ = K.route(w["x"].detach(), w["router"].detach(), w["bias"], k, w["score"])
        plan = K.dispatch(topi, E, e0, e1, n_src)
        P = int(plan.offsets[-1].item())
        pairs = plan.perm[:P].long()
        tok = pairs // k
        expert = topi.reshape(-1).long()[pairs] - e0
        bounds = torch.tensor([(T // n_src) * (s + 1) + min(s + 1, T % n_src) for s in range(n_src)], device=dev)
        src = torch.searchsorted(bounds, tok, right=True)
        order = torch.sort(src * (e1 - e0) + expert, stable=True).indices
        recv = w["x"].detach()[tok[order]].contiguous().requires_grad_(True)
    g = torch.Generator(device=dev).manual_seed(99)
    dy = (torch.randn(P, w["h"], generator=g, device=dev)).to(torch.bfloat16)
    return recv, plan.src_counts.contiguous(), dy


def recv_step(pkg, w):
    """The receiving side of the expert exchange: expert outputs of the received rows, then the backward
    from their gradient (resihp/runtime/moe.py:213-224 and its autograd)."""
    for p in (w["recv"], *w["fc1"], *w["fc2"]):
        p.grad = None
    y = pkg.layer.expert_chunks(w["recv"], w["recv_counts"], w["fc1"], w["fc2"], "swiglu", rows=w["recv"].shape[0])
    y.backward(w["recv_dy"])


def gpu_step(pkg, w, meta):
    for p in (w["x"], w["router"], *w["fc1"], *w["fc2"], *w["s1"], *w["s2"]):
        p.grad = None
    out, counts = pkg.layer.moe_layer(meta, w["x"], w["router"], w["bias"], w["fc1"], w["fc2"], w["s1"], w["s2"],
                                      fp8=w["fp8"])
    out.backward(w["dout"])
    if w["fp8"] is not None:
        w["fp8"].finish_iteration()
    return counts


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(name: str, sample_tokens: int, reps: int = 3, received_rows: int | None = None) -> dict:
    """The float32 CPU restatement of the reference layer (oracle), fwd + bwd on a token sample.

    For a received-buffer workload (``received_rows`` = the P rows one step processes) the sample is
    the reference's receiving side instead: expert_ffn chunk by chunk (resihp/runtime/moe.py:213-223)
    over 8 sources x 16 rows of each local expert, scaled to source tokens per second by T / P.
    """
    if str(ROOT) not in sys.path:
        sys.path.insert(0, str(ROOT))
    from oracle import moe_ref as M

    T, h, f, E, k, score, S, window, n_src = WORKLOADS[name][:9]
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(5)
    times = []
    if received_rows:
        L = window[1] - window[0]
        w1 = [torch.empty(2 * f, h).normal_(0.0, 0.02, generator=g).requires_grad_(True) for _ in range(L)]
        w2 = [torch.empty(h, f).normal_(0.0, 0.02, generator=g).requires_grad_(True) for _ in range(L)]
        chunk = 16
        rows = n_src * L * chunk
        x = torch.randn(rows, h, generator=g).requires_grad_(True)
        dy = torch.randn(rows, h, generator=g)
        for i in range(reps + 1):
            for p in (x, *w1, *w2):
                p.grad = None
            t0 = time.perf_counter()
            outs = [M.expert_ffn(x[c * chunk:(c + 1) * chunk], w1[c % L], w2[c % L], "swiglu")
                    for c in range(n_src * L)]
            torch.cat(outs).backward(dy)
            dt = time.perf_counter() - t0
            if i:
                times.append(dt)
        med = sorted(times)[len(times) // 2]
        return {"value": rows / med * T / received_rows, "unit": "tokens/s", "cores": cores, "kind": "port",
                "cpu": cpu_model(),
                "sample": f"{rows} of the {received_rows} received rows ({n_src} sources x {L} experts x {chunk} "
                          f"rows), float32 torch CPU restatement of the reference's per-chunk expert_ffn, fwd+bwd, "
                          f"median of {reps} after 1 warm-up, scaled by {T} source tokens / {received_rows} rows; "
                          f"torch {torch.__version__}"}
    cfg = M.OracleConfig(hidden=h, ffn=f, num_experts=E, top_k=k, tokens=sample_tokens, act="swiglu", score=score,
                         num_shared=S, shared_ffn=f if S else 0, dtype=torch.float32)
    params = {}
    for key, (shape, _) in M.param_shapes(cfg).items():
        params[key] = torch.empty(shape, dtype=torch.float32).normal_(0.0, 0.02, generator=g).requires_grad_(True)
    x = torch.randn(sample_tokens, h, generator=g).requires_grad_(True)
    dout = torch.randn(sample_tokens, h, generator=g)
    for i in range(reps + 1):
        for p in (x, *params.values()):
            p.grad = None
        t0 = time.perf_counter()
        M.layer_forward(cfg, params, x).backward(dout)
        dt = time.perf_counter() - t0
        if i:
            times.append(dt)
    med = sorted(times)[len(times) // 2]
    return {"value": sample_tokens / med, "unit": "tokens/s", "cores": cores, "kind": "port", "cpu": cpu_model(),
            "sample": f"{sample_tokens} of {T} tokens, float32 torch CPU restatement of the reference layer, "
                      f"fwd+bwd, median of {reps} after 1 warm-up; torch {torch.__version__}"}


def adam_bench(args) -> int:
    """The optimizer step after the layer: one fused Adam step (rhp_adam_step) over the Mixtral layer's
    parameters -- router float32 [8, 4096], 8 experts' fc1 [28672, 4096] and fc2 [4096, 14336] bfloat16 --
    with their gradients and name-keyed moment state resident in HBM."""
    pkg = _package()
    import importlib

    K = importlib.import_module(f"{pkg.__name__}.kernels")
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(7)
    E, h, f = 8, 4096, 14336
    shapes = {torch.float32: [(E, h)], torch.bfloat16: [(2 * f, h)] * E + [(h, f)] * E}
    groups = {}
    for dt, shp in shapes.items():
        ps = [(torch.randn(s, generator=g, device=dev, dtype=torch.float32) * 0.02).to(dt) for s in shp]
        gs = [(torch.randn(s, generator=g, device=dev, dtype=torch.float32) * 1e-3).to(dt) for s in shp]
        groups[dt] = (ps, gs, [torch.zeros_like(x) for x in ps], [torch.zeros_like(x) for x in ps])
    n_el = {dt: sum(x.numel() for x in v[0]) for dt, v in groups.items()}
    step_no = [0]

    def step():
        step_no[0] += 1
        for ps, gs, ms, vs in groups.values():
            K.adam_step(ps, gs, ms, vs, 1e-4, (0.9, 0.95), 1e-8, 0.1, step_no[0])

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    a.record(stream)
    for _ in range(args.steps):
        step()
    b.record(stream)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms = a.elapsed_time(b) / args.steps
    elems = sum(n_el.values())
    nbytes = 14 * n_el[torch.bfloat16] + 28 * n_el[torch.float32]   # p, g, m, v read; p, m, v written
    gbps = nbytes / (ms * 1e-3) / 1e9
    result = {
        "metric": "Adam step parameters/s (Mixtral-8x7B MoE layer parameters, 1 GPU)",
        "value": elems * args.steps / elapsed, "unit": "parameters/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": elapsed * 1e3 / args.steps, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16 experts, fp32 router (moments in the parameter dtype)",
        "data": "synthetic (random parameters and gradients drawn on device)",
        "config": {"workload": f"mixtral-adam: one Adam step (lr 1e-4, betas 0.9/0.95, weight decay 0.1) over "
                               f"{elems} parameters: router fp32 [8, 4096], 8 x fc1 [28672, 4096] and 8 x fc2 "
                               f"[4096, 14336] bf16", "parameters": elems},
        "roofline": {"bound": "hbm", "achieved": gbps, "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": gbps / PEAK_HBM_GBPS, "traffic": None, "kernel": "adam_kernel",
                     "algorithmic": "14 bytes per bf16 parameter, 28 per fp32 (each array read or written once)"},
    }
    if not args.no_cpu_baseline:
        if str(ROOT) not in sys.path:
            sys.path.insert(0, str(ROOT))
        import numpy as np
        from oracle import adam_c

        n = 1 << 24
        rng = np.random.default_rng(0)
        bits = lambda x: (x.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)  # noqa: E731
        hp, hg = bits(rng.standard_normal(n) * 0.02), bits(rng.standard_normal(n) * 1e-3)
        hm, hv = np.zeros(n, np.uint16), np.zeros(n, np.uint16)
        times = []
        for i in range(4):
            c0 = time.perf_counter()
            adam_c.adam_step(hp, hg, hm, hv, 1e-4, (0.9, 0.95), 1e-8, 0.1, i + 1)
            if i:
                times.append(time.perf_counter() - c0)
        med = sorted(times)[len(times) // 2]
        result["cpu_baseline"] = {"value": n / med, "unit": "parameters/s", "cores": 1, "kind": "port",
                                  "cpu": cpu_model(),
                                  "sample": f"{n} bf16 parameters, C oracle of the same update (one thread), "
                                            f"median of 3 after 1 warm-up"}
    print(json.dumps(result), flush=True)
    return 0


def copy_probe(nbytes: int) -> int:
    """A plain device copy of a known size: profiled with FETCH_SIZE / WRITE_SIZE, it converts those
    counters into bytes (each copy reads and writes ``nbytes``)."""
    a = torch.ones(nbytes // 2, dtype=torch.bfloat16, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes": nbytes, "copies": 3}), flush=True)
    return 0


def dense_probe(reps: int) -> int:
    """The vendor library (hipBLASLt through torch.mm) on the dense products of the Mixtral-shape layer:
    each of the six expert products once with all 16384 routed rows in one matrix (the weight gradients
    then reduce over all rows) and once per expert on 2048 rows, bf16, 2-D products only.  Prints one
    JSON line per product with its TFLOP/s; run under rocprofv3 it names the library's kernels and
    gives their counters beside those of the grouped kernels."""
    dev = torch.device("cuda:0")
    P, h, f, E = 16384, 4096, 14336, 8
    g = torch.Generator(device=dev).manual_seed(3)

    def rnd(*shape, std=1.0):
        return (torch.randn(*shape, generator=g, device=dev, dtype=torch.float32) * std).to(torch.bfloat16)

    x, w1, w2 = rnd(P, h), rnd(2 * f, h, std=0.02), rnd(h, f, std=0.02)
    act, dy, dh = rnd(P, f), rnd(P, h), rnd(P, 2 * f)
    products = {   # name: (left, right, FLOP); right operands of the forms the layer's products read
        "fc1_fwd": (lambda a, r: torch.mm(a, w1.t()), x, 2 * P * h * 2 * f),
        "fc2_fwd": (lambda a, r: torch.mm(a, w2.t()), act, 2 * P * f * h),
        "fc2_dgrad": (lambda a, r: torch.mm(a, w2), dy, 2 * P * h * f),
        "fc2_wgrad": (lambda a, r: torch.mm(a.t(), r), dy, 2 * P * h * f),
        "fc1_dgrad": (lambda a, r: torch.mm(a, w1), dh, 2 * P * 2 * f * h),
        "fc1_wgrad": (lambda a, r: torch.mm(a.t(), r), dh, 2 * P * 2 * f * h),
    }
    right = {"fc2_wgrad": act, "fc1_wgrad": x}
    stream = torch.cuda.current_stream(dev)
    for name, (fn, a, flop) in products.items():
        r = right.get(name)
        for split in (1, E):
            rows = P // split

            def run():
                for e in range(split):
                    sl = slice(e * rows, (e + 1) * rows)
                    fn(a[sl], r[sl] if r is not None else None)

            for _ in range(3):
                run()
            torch.cuda.synchronize()
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0.record(stream)
            for _ in range(reps):
                run()
            t1.record(stream)
            torch.cuda.synchronize()
            ms = t0.elapsed_time(t1) / reps
            print(json.dumps({"dense_probe": name, "rows_per_product": rows, "products": split, "ms": round(ms, 4),
                              "tflops": round(flop / (ms * 1e-3) / 1e12, 1),
                              "frac_of_2500": round(flop / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}), flush=True)
    return 0


def gemm_traffic(workload: str) -> float | None:
    """HBM bytes per step of the grouped GEMM launches, from profiles/gemm_traffic_<workload>.json
    (rocprofv3 FETCH_SIZE + WRITE_SIZE, calibrated on a plain copy), when it was measured."""
    path = ROOT / "profiles" / f"gemm_traffic_{workload}.json"
    if not path.exists():
        return None
    return float(json.loads(path.read_text())["hbm_bytes_per_step"])


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="mixtral", choices=sorted(WORKLOADS) + ["mixtral-adam"])
    ap.add_argument("--cpu-sample", type=int, default=256)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="only copy BYTES bytes on the device three times (calibrates HBM byte counters)")
    ap.add_argument("--dense-probe", type=int, default=0, metavar="REPS",
                    help="only time the vendor library's dense products of the Mixtral-shape layer (REPS each)")
    args = ap.parse_args()
    if args.copy_probe:
        return copy_probe(args.copy_probe)
    if args.dense_probe:
        return dense_probe(args.dense_probe)
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs the MoE layer on one GPU; multi-GPU expert parallelism "
                                   "(the all-to-all dispatch) is not part of it", "n_gpus": args.gpus}))
        return 2
    if args.workload == "mixtral-adam":
        return adam_bench(args)
    pkg = _package()
    import importlib

    importlib.import_module(f"{pkg.__name__}.layer")
    kernels = importlib.import_module(f"{pkg.__name__}.kernels")
    dev = torch.device("cuda:0")
    w = build_workload(args.workload, dev)
    T, h, f, E, k = w["T"], w["h"], w["f"], w["E"], w["k"]
    meta = pkg.layer.LayerMeta(num_experts=E, top_k=k, ffn=f, act="swiglu", score=w["score"],
                               num_shared=w["S"], shared_ffn=f if w["S"] else 0, e0=w["e0"], e1=w["e1"],
                               n_src=w["n_src"])
    received = args.workload in RECEIVED
    if received:
        w["recv"], w["recv_counts"], w["recv_dy"] = build_received(pkg, w, dev)
        step = lambda: recv_step(pkg, w)  # noqa: E731
        P = w["recv"].shape[0]
    else:
        step = lambda: gpu_step(pkg, w, meta)  # noqa: E731
    counts = None
    if w["fp8"] is not None:
        # Delayed scaling from seeded prior amax values: two calibration steps from the reference's initial
        # histories (ones), each seeding every 16-step history from the amax it recorded (spread +-25 %,
        # seeded), so the timed steps run with scales of the tensors' real ranges.
        st = w["fp8"]
        for c in range(2):
            step()
            st.seed_history({i: float(a) for i, a in enumerate(st.history[:, 0].tolist())}, seed=100 + c)
    for _ in range(args.warmup):
        counts = step()
    torch.cuda.synchronize()
    if not received:
        # Routed pairs on this GPU (the routing is the same every step: same tokens and router).
        P = int(counts[w["e0"]:w["e1"]].sum().item()) if counts is not None else T * k

    timer = EventTimer()
    kernels.set_timer(timer)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    kernels.set_timer(None)

    per = {name: (ms / args.steps, n // args.steps) for name, (ms, n) in timer.totals_ms().items()}
    fp8 = w["fp8"] is not None
    S = w["S"]
    peak = PEAK_FP8_TFLOPS if fp8 else PEAK_BF16_TFLOPS
    gemm_flops = 18.0 * (P + S * T) * h * f          # SwiGLU: fwd 6 P h f + bwd 12 P h f
    gemm_ms = timer.union_ms(GEMM_CALLS) / args.steps
    gemm_tflops = gemm_flops / (gemm_ms * 1e-3) / 1e12
    s = 2  # bf16 bytes
    if received:   # the products read and write received rows through the plan's row map; two row gathers a
        # step make the expert-major copies the weight gradients read (inputs, output gradients)
        row_bytes = {"rhp_gather_rows": 2 * (2 * P * h * s + 4 * P)}
    else:          # algorithmic HBM bytes per step of the row kernels (token-major permute); with fp8
        # experts the permute and the combine backward write 1-byte codes instead of bf16 rows
        c = 1 if fp8 else s
        row_bytes = {
            "rhp_permute_fp8" if fp8 else "rhp_permute": T * h * s + P * h * c + 4 * P,
            "rhp_combine": P * h * s + 2 * T * h * s + 8 * P + S * T * h * s,
            "rhp_combine_bwd_fp8" if fp8 else "rhp_combine_bwd": T * h * s + P * h * s + P * h * c + 8 * P,
            "rhp_token_bwd": 2 * T * h * s + P * h * s + 12 * P + S * T * h * s,
        }
    row_ms = sum(per.get(n, (0.0, 0))[0] for n in row_bytes)
    row_gbps = sum(row_bytes.values()) / (row_ms * 1e-3) / 1e9 if row_ms else None
    ms_step = elapsed * 1e3 / args.steps
    result = {
        "metric": "MoE-layer tokens/s fwd+bwd (Mixtral shape, 1 GPU)" if args.workload == "mixtral"
        else f"MoE-layer tokens/s fwd+bwd ({args.workload}, 1 GPU)",
        "value": T * args.steps / elapsed,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8 (e4m3 fwd, e5m2 grads) with bf16 outputs" if fp8 else "bf16",
        "data": "synthetic (N(0,1) tokens, random N(0,0.02) weights of the layer shape, drawn on device)",
        "config": {"workload": (f"{args.workload}: the local experts [{w['e0']}, {w['e1']}) of a {E}-expert top-{k} "
                                f"layer (hidden={h}, ffn={f} SwiGLU, bf16) on the {P} rows received from "
                                f"{w['n_src']} sources of {T // w['n_src']} tokens ({T} source tokens, {w['score']} "
                                f"router with a Zipf(1.1) selection prior): regroup, expert FFN, return, fwd+bwd")
                   if received else
                   (f"{args.workload} MoE layer: tokens={T}, hidden={h}, ffn={f} SwiGLU, experts={E}, "
                    f"local experts [{w['e0']}, {w['e1']}), top_k={k} {w['score']} router (fp32), "
                    f"shared experts={S}, "
                    f"{'fp8 experts (e4m3 fwd, e5m2 grads, 16-step amax histories seeded from two calibration steps)' if fp8 else 'bf16'}"
                    f", fwd+bwd"),
                   "tokens": T, "hidden": h, "ffn": f, "experts": E, "top_k": k, "local_experts": w["e1"] - w["e0"],
                   "routed_pairs": P, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": gemm_tflops, "peak": peak, "unit": "TFLOP/s",
                     "frac": gemm_tflops / peak, "traffic": gemm_traffic(args.workload),
                     "traffic_source": f"profiled constant: rocprofv3 FETCH_SIZE + WRITE_SIZE of the same launches, "
                                       f"copy-calibrated, from profiles/gemm_traffic_{args.workload}.json (not "
                                       f"measured in this run)" if gemm_traffic(args.workload) else None,
                     "kernel": "grouped expert GEMMs (fc1/fc2 fwd, dgrad, wgrad)",
                     "algorithmic": f"18*(P + S*T)*h*f = {gemm_flops:.4g} FLOP per step, P = {P} routed pairs"},
        "rows_roofline": {"bound": "hbm", "achieved": row_gbps, "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                          "frac": (row_gbps / PEAK_HBM_GBPS) if row_gbps else None,
                          "kernel": "two row gathers (expert-major inputs and output gradients, side stream)"
                          if received else "permute + combine + combine_bwd + token_bwd"},
        "breakdown_ms": {n: round(v[0], 4) for n, v in sorted(per.items())},
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args.workload, args.cpu_sample, received_rows=P if received else None)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
