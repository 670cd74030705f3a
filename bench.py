"""MoE-layer fwd+bwd throughput on one MI355X (BASELINE.json metric).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c3]
                    [--no-cpu-baseline]

Workload (default): the full MoE layer training step
at T=32768 tokens, d=2048, E=128 routed experts, top-8, SwiGLU f=768, plus a
shared SwiGLU expert of width 1536, bf16 parameters and activations, synthetic
seeded inputs (x ~ N(0,1), upstream grad ~ N(0,1), random-init weights). A step
is one forward and one full backward of the layer (gate, shared expert, routed
experts, combine; dX, grouped dW, gate grads). Inputs are resident in HBM before
the timed region.

Prints ONE JSON line. ``roofline`` covers the dominant grouped-GEMM launch,
timed live with HIP events on the stream it runs on; ``cpu_baseline`` times the
reference layer as eager torch (float32) on a bounded sample of the same workload,
under ``numpy_oracle`` the numpy oracle (float32) on the same sample, and, under
``c1_fwd_torch_eager``, the reference forward as eager torch at BASELINE.json's
CPU config C1. ``--dense-gemm`` times the grouped GEMM kernel as a plain dense GEMM
beside hipBLASLt instead.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.join(ROOT, "architecture-zarelga-superposition_amd")
for _p in (ROOT, PKG_ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "MoE-layer tokens/s fwd+bwd on 1 MI355X; grouped-GEMM MFMA util %"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E

WORKLOADS = {
    # name: (T, d, E, k, f, shared_width (0: n_shared_experts = 0), backward)
    "c2": (16384, 1024, 64, 8, 512, 0, False),
    "c3": (32768, 2048, 128, 8, 768, 1536, True),
    "c4": (8192, 7168, 256, 8, 2048, 2048, True),
    "c5": (512, 2048, 128, 8, 768, 0, False),
}

GEMM_OPS = ("glu_w1_forward", "scatter2scatter", "glu_w2_backward_dh", "group_bwd_w")

# HBM-side bytes per launch at C3 (L2 -> memory fabric reads and writes), from two
# rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE) over this script, each scaled by what
# the same counter reads for a plain 1 GiB copy (reads x 2.000, writes x 1.000); the
# commands and raw counts are in TRAFFIC_C3_PROFILE. They hold for the GEMM sources
# they were measured on (TRAFFIC_C3_GEMM_SHA256, the sha256 of TRAFFIC_C3_SOURCES read
# one after the other): when those differ, the line reports traffic null and says why.
TRAFFIC_C3_PROFILE = "profiles/grouped_gemm_c3_hbm_bytes.md"
TRAFFIC_C3_SOURCES = ("gemm.hip", "zmoe_internal.h")  # what the grouped GEMM kernels compile from
TRAFFIC_C3_GEMM_SHA256 = "d38eed6a4335a73af29503a97c1226584f471d8cc58f3fd5205c9aaf7c53e814"
TRAFFIC_C3 = {
    "glu_w1_forward#0": 6035677760,
    "scatter2scatter#0": 2891170624,
    "glu_w2_backward_dh#0": 2458364202,
    "scatter2scatter#1": 5833844736,
    "group_bwd_w#0": 2165850346,
    "group_bwd_w#1": 3661097280,
}
ROW_OPS = ("route_topk", "flatten_sort_count", "combine", "combine_backward", "combine_backward_scale",
           "swiglu_backward_gates", "sum_k")


def gemm_flops(name: str, launch: int, T, d, k, f) -> float:
    """Algorithmic flops of the n-th launch of ``name`` within one step."""
    R = T * k
    big, small = 2.0 * R * d * 2 * f, 2.0 * R * d * f
    if name == "glu_w1_forward":
        return big
    if name == "glu_w2_backward_dh":
        return small
    # scatter2scatter: W2 forward then W1 input grad; group_bwd_w: dW2 then dW1
    return small if launch % 2 == 0 else big


def row_bytes(name: str, T, d, E, k, f=0) -> float:
    """Algorithmic HBM bytes of one launch (bf16 rows, fp32 gates, int64 ids).

    The layer's combine also reads the shared expert's output [T, d] as its addend.
    """
    R = T * k
    return {
        "route_topk": T * E * 2 + E * 4 + R * (8 + 4 + 4),
        "flatten_sort_count": R * 8 * 2 + R * 8 * 2 + R * 4,
        "combine": R * d * 2 + R * 4 + T * d * 2 + T * d * 2,
        "combine_backward": R * d * 2 + T * d * 2 + R * (4 + 4 + 4) + R * d * 2,
        "combine_backward_scale": T * d * 2 + R * (4 + 4) + R * d * 2,   # without Y: no gate dots
        "swiglu_backward_gates": R * f * 2 + 2 * R * 2 * f * 2 + R * (4 + 8 + 4),  # dA, H, dH; scales, slots, d_gates
        "sum_k": R * d * 2 + T * d * 2,
    }[name]


def zipf_bias(logits, k: int, s: float = 1.1, seed: int = 0):
    """Selection bias that skews expert popularity towards Zipf(s) (BASELINE.json C4).

    b_e = c * log(rank_e ** -s) for a seeded random ranking of the experts; c is the
    value on a log grid (refined once) whose realised top-k counts on ``logits`` are
    closest to Zipf(s) over the ranks in Kolmogorov-Smirnov distance. Returns
    (bias [E] fp32 on the logits' device, c, KS distance).
    """
    import torch

    from zmoe import ops

    E = logits.shape[1]
    g = torch.Generator()
    g.manual_seed(seed)
    rank = torch.randperm(E, generator=g) + 1                    # rank of expert e (1 = most popular)
    base = (-s * torch.log(rank.double())).float()
    pmf = rank.double().sort().values.pow(-s)
    target = torch.cumsum(pmf / pmf.sum(), 0)
    order = torch.argsort(rank)                                   # experts by rank

    def ks(c: float) -> float:
        idx, _, _ = ops.route_topk(logits, (c * base).to(logits.device), k)
        counts = torch.bincount(idx.view(-1), minlength=E).double().cpu()[order]
        return float((torch.cumsum(counts / counts.sum(), 0) - target).abs().max())

    grid = [0.0] + [10 ** (x / 8.0) for x in range(-24, 9)]       # 1e-3 .. ~10
    best = min(grid, key=ks)
    fine = [best * (1 + x / 10.0) for x in range(-5, 6)]
    best = min(fine, key=ks)
    return (best * base).to(logits.device), best, ks(best)


def build_layer(T, d, E, k, f, fs, dev, seed=0, fp32_params=False):
    """The MoE layer at the workload's shape: bf16 parameters, or with ``fp32_params`` fp32
    master weights (run under bf16 autocast, the reference's training mode)."""
    import torch

    from modeling.model_config import ModelConfig
    from modeling.moe_layer import MoELayer

    ns = fs // f if fs else 0
    if ns * f != fs:
        raise ValueError("shared width must be a multiple of f")
    torch.manual_seed(seed)
    cfg = ModelConfig(hidden_size=d, intermediate_size=f, n_experts=E + ns, n_shared_experts=ns,
                      n_experts_per_token=k)
    layer = MoELayer(cfg).to(dev)
    if not fp32_params:
        layer = layer.to(torch.bfloat16)
    layer.gate.expert_biases.data = layer.gate.expert_biases.data.float()
    return layer


def cpu_baseline(T, d, E, k, f, fs, backward=True, budget_s=20.0, sample_T=1024):
    """Time the numpy oracle (float32) fwd (+bwd) on ``sample_T`` tokens of the workload."""
    import numpy as np

    import oracle as O

    try:
        from threadpoolctl import threadpool_info

        threads = max((i.get("num_threads", 1) for i in threadpool_info()), default=1)
    except Exception:  # pragma: no cover - informational only
        threads = len(os.sched_getaffinity(0))
    O.set_precision(np.float32)
    rng = np.random.default_rng(0)
    std = np.float32(1.0 / np.sqrt(d))
    x = rng.standard_normal((sample_T, d), dtype=np.float32)
    dout = rng.standard_normal((sample_T, d), dtype=np.float32)
    Wg = rng.standard_normal((E, d), dtype=np.float32) * std
    W1 = rng.standard_normal((E, 2 * f, d), dtype=np.float32) * std
    W2 = rng.standard_normal((E, d, f), dtype=np.float32) * std
    shared = None
    if fs:
        shared = tuple(rng.standard_normal(s, dtype=np.float32) * std for s in ((fs, d), (fs, d), (d, fs)))
    orc = O.MoELayerOracle(Wg, np.zeros(E, np.float32), W1, W2, k, shared=shared)
    times = []
    t_start = time.perf_counter()
    for i in range(6):
        t0 = time.perf_counter()
        orc.forward(x)
        if backward:
            orc.backward(dout)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s and i >= 1:
            break
    O.set_precision(np.float64)
    timed = times[1:] if len(times) > 1 else times
    sec = sum(timed) / len(timed)
    return {
        "value": sample_T / sec,
        "unit": "tokens/s",
        "cores": int(threads),
        "kind": "port",
        "sample": (f"numpy oracle (float32) MoE layer {'fwd+bwd' if backward else 'fwd'} on {sample_T} tokens "
                   f"of the same shape "
                   f"(d={d}, E={E}, k={k}, f={f}, shared={fs}); mean of {len(timed)} steps after 1 warmup, "
                   f"{sec:.2f} s/step"),
    }


def cpu_baseline_torch(T, d, E, k, f, fs, backward=True, budget_s=12.0, sample_T=1024):
    """Time the reference layer as eager torch (float32, oracle/torch_eager.py) fwd (+bwd) on
    ``sample_T`` tokens of the workload's shape, on the host cores."""
    import torch

    from oracle.torch_eager import moe_forward, moe_step

    g = torch.Generator().manual_seed(0)
    std = d ** -0.5
    x = torch.randn(sample_T, d, generator=g)
    dout = torch.randn(sample_T, d, generator=g)
    Wg = torch.randn(E, d, generator=g) * std
    W1 = torch.randn(E, 2 * f, d, generator=g) * std
    W2 = torch.randn(E, d, f, generator=g) * std
    shared = tuple(torch.randn(s, generator=g) * std for s in ((fs, d), (fs, d), (d, fs))) if fs else None
    bias = torch.zeros(E)

    def run():
        if backward:
            moe_step(x, Wg, bias, W1, W2, k, dout, shared=shared)
        else:
            moe_forward(x, Wg, bias, W1, W2, k, shared=shared)

    run()  # warmup
    times = []
    t_start = time.perf_counter()
    while len(times) < 20 and (time.perf_counter() - t_start < budget_s or len(times) < 2):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    sec = sorted(times)[len(times) // 2]
    return {
        "value": sample_T / sec,
        "unit": "tokens/s",
        "cores": int(torch.get_num_threads()),
        "kind": "port",
        "sample": (f"the reference layer as eager torch (float32, oracle/torch_eager.py) "
                   f"{'fwd+bwd' if backward else 'fwd'} on {sample_T} tokens of the same shape (d={d}, E={E}, "
                   f"k={k}, f={f}, shared={fs}); median of {len(times)} steps after 1 warmup, {sec:.3f} s/step"),
    }


def cpu_baseline_c1(budget_s=8.0):
    """Time the reference forward as eager torch (float32) at C1
    (T=2048, d=256, E=8, top-2, SwiGLU f=512, no shared expert), on the host cores."""
    import torch

    from oracle.torch_eager import c1_inputs, moe_forward

    x, Wg, bias, W1, W2 = c1_inputs()
    moe_forward(x, Wg, bias, W1, W2, 2)  # warmup
    times = []
    t_start = time.perf_counter()
    while len(times) < 50 and (time.perf_counter() - t_start < budget_s or len(times) < 3):
        t0 = time.perf_counter()
        moe_forward(x, Wg, bias, W1, W2, 2)
        times.append(time.perf_counter() - t0)
    sec = sorted(times)[len(times) // 2]
    return {
        "value": x.shape[0] / sec,
        "unit": "tokens/s",
        "cores": int(torch.get_num_threads()),
        "kind": "port",
        "sample": (f"C1 forward (fp32, T=2048 d=256 E=8 k=2 SwiGLU f=512, no shared expert) as eager torch "
                   f"(oracle/torch_eager.py); median of {len(times)} runs after 1 warmup, {1e3 * sec:.1f} ms/run"),
    }


def traffic_c3(name):
    """(bytes, source note) of the dominant launch's measured HBM traffic at C3."""
    import hashlib

    h = hashlib.sha256()
    for src in TRAFFIC_C3_SOURCES:
        with open(os.path.join(PKG_ROOT, "csrc", src), "rb") as fh:
            h.update(fh.read())
    sha = h.hexdigest()
    what = " + ".join("csrc/" + s for s in TRAFFIC_C3_SOURCES)
    if TRAFFIC_C3_GEMM_SHA256 is None or sha != TRAFFIC_C3_GEMM_SHA256:
        return None, f"not measured for this {what} (sha256 {sha[:12]}); {TRAFFIC_C3_PROFILE} is older"
    return TRAFFIC_C3.get(name), f"{TRAFFIC_C3_PROFILE} ({what} sha256 {sha[:12]})"


COPY_PROBE_BYTES = 1 << 30  # device-to-device copy used to calibrate FETCH_SIZE / WRITE_SIZE


def copy_probe() -> int:
    """Three 1 GiB device copies (run under rocprofv3 --pmc to calibrate the byte counters)."""
    import torch

    src = torch.empty(COPY_PROBE_BYTES, dtype=torch.uint8, device="cuda")
    src.fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"copy probe: 3 x {COPY_PROBE_BYTES} bytes", flush=True)
    return 0


def pmc_summary(path: str) -> int:
    """Mean of each counter per dispatch, by kernel, in dispatch order of first appearance,
    from the run_counter_collection.csv files under ``path`` (rocprofv3 --pmc output)."""
    import csv
    import glob

    files = sorted(glob.glob(os.path.join(path, "**", "*counter_collection.csv"), recursive=True))
    if not files:
        print(f"no counter_collection.csv under {path}", file=sys.stderr)
        return 1
    rows = {}
    for fn in files:
        with open(fn) as fh:
            for r in csv.DictReader(fh):
                key = (r["Kernel_Name"], r["Counter_Name"])
                d = rows.setdefault(key, {"first": int(r.get("Dispatch_Id", 0) or 0), "v": {}})
                d["v"][r.get("Dispatch_Id", len(d["v"]))] = d["v"].get(r.get("Dispatch_Id", len(d["v"])), 0.0) + float(
                    r["Counter_Value"])
    print(f"{'counter':12s} {'dispatches':>10s} {'mean/dispatch':>16s}  kernel")
    for (kern, ctr), d in sorted(rows.items(), key=lambda kv: kv[1]["first"]):
        vals = list(d["v"].values())
        print(f"{ctr:12s} {len(vals):10d} {sum(vals) / len(vals):16.1f}  {kern[:110]}")
    _pmc_clock_mfma(path, rows)
    return 0


def _pmc_clock_mfma(path: str, rows: dict) -> None:
    """With GRBM_GUI_ACTIVE and SQ_VALU_MFMA_BUSY_CYCLES collected beside --kernel-trace: the
    core clock each kernel ran at (GRBM_GUI_ACTIVE is summed over the 8 XCDs) and the fraction
    of the 1024 SIMDs' cycles in which the MFMA pipe was busy, at that clock."""
    import csv
    import glob

    traces = sorted(glob.glob(os.path.join(path, "**", "*kernel_trace.csv"), recursive=True))
    if not traces:
        return
    dur = {}
    for fn in traces:
        with open(fn) as fh:
            for r in csv.DictReader(fh):
                dur[(r["Kernel_Name"], r["Dispatch_Id"])] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
    kernels = {k for k, c in rows if c == "SQ_VALU_MFMA_BUSY_CYCLES"}
    out = []
    for kern in kernels:
        gui, busy = rows.get((kern, "GRBM_GUI_ACTIVE")), rows[(kern, "SQ_VALU_MFMA_BUSY_CYCLES")]
        if gui is None:
            continue
        ids = [i for i in busy["v"] if (kern, i) in dur and i in gui["v"]]
        if not ids or sum(busy["v"][i] for i in ids) < 1e6 * len(ids):
            continue
        ns = sum(dur[(kern, i)] for i in ids) / len(ids)
        cyc = sum(gui["v"][i] for i in ids) / len(ids) / 8            # per XCD
        mf = sum(busy["v"][i] for i in ids) / len(ids)
        out.append((busy["first"], kern, len(ids), ns, cyc, mf))
    if not out:
        return
    print(f"\n{'dispatches':>10s} {'avg ms':>8s} {'clock GHz':>9s} {'MFMA busy':>9s} {'MFMA ops/disp':>13s}  kernel")
    for _, kern, n, ns, cyc, mf in sorted(out):
        print(f"{n:10d} {ns / 1e6:8.3f} {cyc / ns:9.3f} {mf / (1024 * cyc):9.3f} {mf / 32:13.4g}  {kern[:90]}")


def ns_flops(m: int, n: int, steps: int, executed: bool = False) -> float:
    """Newton-Schulz GEMM flops for one m x n matrix (m <= n): X X^T, (cA) A, B X per step.

    executed=True counts what the kernels run: the two symmetric products only compute the
    256 x 256 tiles on or above the diagonal (nm (nm + 1) / 2 of nm^2 tiles)."""
    m, n = min(m, n), max(m, n)
    nm = -(-m // 256)
    sym = nm * (nm + 1) / 2 / (nm * nm) if executed else 1.0
    return steps * (sym * 2.0 * m * m * n + sym * 2.0 * m * m * m + 2.0 * m * m * n)


def muon_bench(args) -> int:
    """Newton-Schulz (optimizer/muon.py:6-32, 5 steps) over the routed-expert weight stacks of
    one C3 MoE layer (W1 [128, 1536, 2048], W2 [128, 2048, 768]), as the MuonMD step runs it
    on 3-D expert weights (muon.py:449). Prints one JSON line; also times the same bf16
    arithmetic through torch's batched matmuls (hipBLASLt) for comparison."""
    import torch

    from zmoe import ops

    dev = torch.device("cuda:0")
    E, d, f, steps = 128, 2048, 768, 5
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    stacks = [torch.randn(E, 2 * f, d, device=dev, generator=g), torch.randn(E, d, f, device=dev, generator=g)]
    flops = sum(E * ns_flops(G.shape[1], G.shape[2], steps) for G in stacks)
    flops_exec = sum(E * ns_flops(G.shape[1], G.shape[2], steps, executed=True) for G in stacks)
    a, b, c = ops.NS_COEFFS

    def torch_ns(G):
        # every batched-matmul operand is made contiguous: bf16 bmm on a transposed view
        # (the .mT of a tall stack keeps its transposed strides through the elementwise
        # ops) is avoided on this platform
        X = G.bfloat16()
        if G.size(-2) > G.size(-1):
            X = X.mT.contiguous()
        X = X / (X.norm(dim=(-2, -1), keepdim=True) + 1e-7)
        for _ in range(steps):
            A = X @ X.mT.contiguous()
            B = b * A + c * A @ A
            X = a * X + B @ X
        return X.mT if G.size(-2) > G.size(-1) else X

    def timed(fn, reps):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        return 1000.0 * (time.perf_counter() - t0) / reps

    reps = max(1, args.steps // 4)
    print("muon bench: zmoe_newton_schulz5 on the two stacks", file=sys.stderr, flush=True)
    ms = timed(lambda: [ops.newton_schulz5(G, steps) for G in stacks], reps)
    print("muon bench: torch bf16 batched matmuls on the two stacks", file=sys.stderr, flush=True)
    ms_torch = timed(lambda: [torch_ns(G) for G in stacks], reps)
    tf = flops / (ms * 1e-3) / 1e12
    tf_exec = flops_exec / (ms * 1e-3) / 1e12
    out = {
        "metric": "MuonMD Newton-Schulz (5 steps) over one C3 layer's routed-expert stacks, "
                  "reference-equivalent TFLOP/s (full products counted)",
        "value": tf, "unit": "TFLOP/s", "n_gpus": 1, "steps": reps, "warmup": 2, "ms_per_step": ms,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) stacks)",
        "config": {"workload": "muon-ns: W1 [128,1536,2048] + W2 [128,2048,768] (transposed to [128,768,2048]), 5 steps",
                   "flops": flops, "flops_executed": flops_exec},
        "roofline": {"bound": "mfma", "achieved": tf_exec, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": tf_exec / PEAK_BF16_TFLOPS, "traffic": None},
        "torch_bf16_bmm_ms": ms_torch, "speedup_vs_torch": ms_torch / ms,
    }
    print(json.dumps(out), flush=True)
    return 0


def dense_gemm_bench(args) -> int:
    """The grouped GEMM kernel run as a plain dense GEMM (one expert, no gather or scatter:
    Y = X W^T with X [M, K], W [N, K], M = 262144 = C3's routed rows, N = K = 2048), beside
    torch's matmul (hipBLASLt) on the same operands. Isolates the K loop from the grouping.
    Prints one JSON line."""
    import torch

    from zmoe import ops

    dev = torch.device("cuda:0")
    M, N, K = 262144, 2048, 2048
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    X = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
    W = (torch.randn(1, N, K, device=dev, generator=g) / K ** 0.5).to(torch.bfloat16)
    se = torch.zeros(M, dtype=torch.int64, device=dev)
    ss = torch.arange(M, dtype=torch.int64, device=dev)
    off = torch.tensor([M], dtype=torch.int64, device=dev)
    Wl = W.permute(0, 2, 1)  # the logical [E, K, N] view of the nn.Linear layout

    def ours():
        return ops.scatter2scatter(X, Wl, se, ss, 1, x_grouped=True, y_grouped=True, expert_offsets=off)

    def lib():
        return X @ W[0].T

    def timed(fn, reps):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    reps = max(5, args.steps)
    y0, y1 = ours(), lib()
    max_rel = float(((y0.float() - y1.float()).abs().max() / y1.float().abs().max()).item())
    # two rounds in alternation, best of each: the core clock drifts under sustained MFMA load,
    # and a fixed order would hand the drift to one side
    ms, ms_lib = timed(ours, reps), timed(lib, reps)
    ms, ms_lib = min(ms, timed(ours, reps)), min(ms_lib, timed(lib, reps))
    flops = 2.0 * M * N * K
    tf, tf_lib = flops / (ms * 1e-3) / 1e12, flops / (ms_lib * 1e-3) / 1e12
    out = {
        "metric": "grouped GEMM kernel as a dense bf16 GEMM (E=1, M=262144, N=K=2048), TFLOP/s",
        "value": tf, "unit": "TFLOP/s", "n_gpus": 1, "steps": reps, "warmup": 3, "ms_per_step": ms,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1))",
        "config": {"workload": "dense: Y[262144, 2048] = X[262144, 2048] W^T, W [2048, 2048] (nn.Linear layout)"},
        "roofline": {"bound": "mfma", "achieved": tf, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": tf / PEAK_BF16_TFLOPS, "traffic": None},
        "hipblaslt_ms": ms_lib, "hipblaslt_tflops": tf_lib, "ratio_to_hipblaslt": tf / tf_lib,
        "max_rel_diff_vs_hipblaslt": max_rel,
    }
    print(json.dumps(out), flush=True)
    return 0


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="c3", choices=sorted(WORKLOADS))
    ap.add_argument("--tokens", type=int, default=None, help="override the workload's token count T")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--copy-probe", action="store_true", help="run the counter-calibration copy and exit")
    ap.add_argument("--muon", action="store_true",
                    help="time the MuonMD Newton-Schulz step on the C3 routed-expert stacks instead of the layer")
    ap.add_argument("--pmc-summary", metavar="DIR", help="summarise rocprofv3 --pmc CSVs under DIR and exit")
    ap.add_argument("--dense-gemm", action="store_true",
                    help="time the grouped GEMM kernel as a plain dense GEMM beside hipBLASLt and exit")
    ap.add_argument("--autocast-fp32-params", action="store_true",
                    help="the reference's training mode (main.py:595, :746): fp32 master weights and an fp32 "
                         "input under torch.autocast(bf16); the step includes the weights' bf16 copies and "
                         "writes fp32 weight grads")
    args = ap.parse_args(argv)
    if args.pmc_summary:
        return pmc_summary(args.pmc_summary)
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(across GPUs the MoE layer would shard its experts: expert parallelism over RCCL all-to-all)", file=sys.stderr)
        return 2

    if args.copy_probe:
        return copy_probe()
    if args.muon:
        return muon_bench(args)
    if args.dense_gemm:
        return dense_gemm_bench(args)

    import torch

    from zmoe import profiling

    dev = torch.device("cuda:0")
    T, d, E, k, f, fs, backward = WORKLOADS[args.workload]
    if args.tokens:
        T = args.tokens
    amp = args.autocast_fp32_params
    layer = build_layer(T, d, E, k, f, fs, dev, fp32_params=amp)
    # the reference layer always runs a shared expert; n_shared_experts = 0 gives width f
    fs = layer.shared_experts.intermediate_size
    g = torch.Generator(device=dev)
    g.manual_seed(1234)
    x = torch.randn(1, T, d, device=dev, generator=g)
    x = (x if amp else x.to(torch.bfloat16)).requires_grad_(backward)   # fp32 residual stream under autocast
    dout = torch.randn(1, T, d, device=dev, generator=g).to(torch.bfloat16)
    skew = None
    if args.workload == "c4":  # Zipf(1.1)-skewed expert popularity through the selection bias
        with torch.no_grad():
            logits = torch.nn.functional.linear(x.detach().view(T, d).to(torch.bfloat16),
                                                layer.gate.weight.to(torch.bfloat16))
        bias, c, ks = zipf_bias(logits, k)
        layer.gate.expert_biases.data = bias
        skew = {"zipf_s": 1.1, "bias_scale": c, "ks_distance": ks}
    params = list(layer.parameters())

    def step():
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=amp):
            if backward:
                for p in params:
                    p.grad = None
                x.grad = None
                out, _ = layer(x)
            else:
                with torch.no_grad():
                    layer(x)
        if backward:
            out.backward(dout)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    def launch_times(nsteps):
        """Per-launch kernel times from HIP events recorded on the launch stream."""
        kernels = {}
        for name in GEMM_OPS:
            durs = profiling.durations_ms(name)
            if not durs:
                continue
            per_step = len(durs) // nsteps
            for j in range(per_step):
                ds = durs[j::per_step]
                fl = gemm_flops(name, j, T, d, k, f)
                avg = sum(ds) / len(ds)
                kernels[f"{name}#{j}"] = dict(avg_ms=avg, tflops=fl / (avg * 1e-3) / 1e12, flops=fl)
        for name in ROW_OPS:
            durs = profiling.durations_ms(name)
            if not durs:
                continue
            avg = sum(durs) / len(durs)
            by = row_bytes(name, T, d, E, k, f)
            kernels[name] = dict(avg_ms=avg, gbs=by / (avg * 1e-3) / 1e9, bytes=by)
        return kernels

    # the per-launch breakdown (every GEMM and row launch bracketed by events) comes from an
    # untimed pass; the timed steps carry events around the roofline kernel's op only, so the
    # step time is not inflated by ~20 event pairs per step (~1% at C3)
    nbreak = max(3, args.steps // 2)
    profiling.reset()
    profiling.enable(*GEMM_OPS, *ROW_OPS)
    for _ in range(nbreak):
        step()
    torch.cuda.synchronize()
    kernels = launch_times(nbreak)
    profiling.disable()
    gemm = {n: v for n, v in kernels.items() if "tflops" in v}
    dom_name = max(gemm, key=lambda n: gemm[n]["avg_ms"])

    profiling.reset()
    profiling.enable(dom_name.split("#")[0])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    timed = launch_times(args.steps)
    profiling.disable()
    ms_per_step = 1000.0 * elapsed / args.steps
    tokens_per_s = T / (ms_per_step / 1000.0)
    kernels[dom_name] = timed[dom_name]  # the roofline kernel as timed inside the timed region

    gemm = {n: v for n, v in kernels.items() if "tflops" in v}
    dom = gemm[dom_name]
    gemm_ms = sum(v["avg_ms"] for v in gemm.values())
    gemm_flops_total = sum(v["flops"] for v in gemm.values())
    util = gemm_flops_total / (gemm_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS

    weight_stream = None
    if not backward:
        # expert-weight streaming of the routed GEMMs (HBM-bound at small T): bytes of the
        # W1 and W2 slabs of every expert that received a token, over the two GEMMs' time
        with torch.no_grad():
            idx, _ = layer.gate(x)
        U = int(torch.unique(idx).numel())
        wbytes = U * (2 * f * d + d * f) * 2
        t_ms = sum(v["avg_ms"] for n, v in kernels.items() if n.startswith(("glu_w1_forward", "scatter2scatter")))
        weight_stream = {"experts_touched": U, "bytes": wbytes, "ms": t_ms,
                         "gbs": wbytes / (t_ms * 1e-3) / 1e9, "frac_of_hbm_peak": wbytes / (t_ms * 1e-3) / 1e9 / PEAK_HBM_GBS}

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_torch(T, d, E, k, f, fs, backward=backward, sample_T=min(1024, T))
        cpu["numpy_oracle"] = cpu_baseline(T, d, E, k, f, fs, backward=backward, sample_T=min(1024, T),
                                           budget_s=12.0)
        cpu["c1_fwd_torch_eager"] = cpu_baseline_c1()
    traffic, traffic_source = (traffic_c3(dom_name) if args.workload == "c3"
                               else (None, "measured for the c3 workload only"))

    line = {
        "metric": METRIC,
        "value": tokens_per_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) inputs and upstream grads; random-init weights)",
        "config": {
            "workload": (f"{args.workload}: MoE layer {'fwd+bwd' if backward else 'fwd'} T={T} d={d} E={E} "
                         f"k={k} SwiGLU f={f} + shared SwiGLU {fs}"),
            "tokens": T, "d_model": d, "experts": E, "top_k": k, "ffn": f, "shared_ffn": fs,
            "parallelism": "single GPU",
            "params": ("fp32 master weights, fp32 input, under torch.autocast(bf16): bf16 compute copies made "
                       "each forward, fp32 weight grads" if amp else "bf16"),
            **({"routing_skew": skew} if skew else {}),
        },
        "grouped_gemm_mfma_util_pct": 100.0 * util,
        "roofline": {
            "kernel": dom_name,
            "bound": "mfma",
            "achieved": dom["tflops"],
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": dom["tflops"] / PEAK_BF16_TFLOPS,
            "avg_ms": dom["avg_ms"],
            "traffic": traffic,
            "traffic_source": traffic_source,
        },
        "cpu_baseline": cpu,
    }
    if weight_stream:
        line["weight_streaming"] = weight_stream
    if args.verbose:
        line["kernels"] = kernels
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
