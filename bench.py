#!/usr/bin/env python3
"""Benchmark of QStream's quantized matvec hot path on one MI355X.

Metric: quant matvec HBM GB/s (% of ~8 TB/s peak) + us/call
at 7B decode shapes.  The headline workload is BASELINE.json config 1: the
2-bit+outlier FFN gate and up projections (11008x4096 each, block 64), batch-1
decode.  A step is one pass over one activation vector: one grouped GEMV
launch over gate and up that prepares x inside its workgroups.  Weights
rotate over >= 512 MiB of distinct copies in HBM so the 256 MB Infinity Cache
cannot serve them; inputs are resident in HBM before the timed region.

    python bench.py [--steps K] [--warmup W] [--config 1|headline|0|2|3|4|layer|copy]

Prints one JSON line.  `value` is algorithmic bytes per step (on-disk QSF
payload + x read once + y written, per matrix) / wall time per step, over K
steps captured once into a HIP graph and replayed between two HIP events on
the replay stream, after W untimed eager steps and at least 0.2 s of untimed
replays (the clocks settle after about 40 ms of sustained work).  For the
one-launch decode steps (configs 0 and 1) that timed region is also the
kernel's time: `roofline.kernel_us` is the region time per launch, so it
never exceeds the step.  Configs 2, 3, 4 and the layer step time their
dominant kernel by a graph of that kernel's launches alone (config 3 at
batch 8: routing + gate/up less routing alone; `roofline.timing` says
which).
`roofline.traffic` is the HBM bytes per launch measured with rocprofv3
counters (profiles/traffic.json), used only while the kernel source it was
measured on is unchanged, else null.  Configs 0 and 1 also carry
`read_floor`: one launch per step that only streams the same rotated
tensors' device bytes, timed the same way.  `cpu_baseline` times QStream's
own CPU kernel (oracle/_ref, reference release flags, 1 thread) on a
bounded sample whose weights rotate over >= 768 MiB of host copies.

The default run (`--config 1`) prints the headline line with every other
config (0, 2, 3 at batch 1 and 8, 4, the layer step) nested under
"configs", each with its roofline and cpu_baseline: about 2-4 minutes in
all (data generation and about 34 s of CPU baselines included; the GPU
timed work is under 10 s).  `--config headline` runs config 1 alone.
`--profile` runs eager launches only, for rocprofv3 counter passes;
`--no-slot` skips the PCIe-inclusive table-slot timing.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_MFMA_PEAK_TFS = 2500.0     # dense bf16 MFMA, MI355X
ROTATE_BYTES = 512 << 20
HOST_ROTATE_BYTES = 768 << 20   # CPU baselines: past the largest host LLC (EPYC: up to 512 MB L3)
METRIC = "quant matvec HBM GB/s (% of ~8 TB/s peak) + µs/call at 7B decode shapes"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------
def cfg1_data(seed=1):
    from qstream_amd import qsf_format as F
    return F.config1_matrices(seed)


def cfg0_data(seed=0):
    from qstream_amd import qsf_format as F
    return F.config0_matrix(seed)


def cfg4_data(seed=4):
    from qstream_amd import qsf_format as F
    rng = np.random.default_rng(seed)
    m, n, k, bs = 512, 14336, 4096, 64
    w = F.gaussian(rng, (n, k), 0.02)
    payload = np.frombuffer(F.quantize_matrix(w, F.Q4, bs), np.uint8)
    del w
    xb = F.bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    return payload, xb, m, n, k, bs


def cfg2_layer(seed=2):
    """One 7B decoder layer at 3-bit, block 128 (qsf_format.config2_layer);
    the 32 layers of config 2 are distinct device copies of these payloads."""
    from qstream_amd import qsf_format as F
    return F.config2_layer(seed)


def cfg3_experts(seed=3, n_exp=32, dim=2880, workers=None):
    """32 MXFP4 experts (gate, up [2880][2880], down [2880][2880]) quantised
    from N(0, 0.02) weights, one seed per matrix (qsf_format.moe_experts;
    the config-3 parity tests build the same experts).  The bytes do not
    depend on `workers`."""
    from qstream_amd import qsf_format as F
    return F.moe_experts(seed, n_exp, dim, dim, workers=workers)


def algo_bytes(mats) -> int:
    return sum(len(p) + 4 * c + 4 * r for _, p, r, c in mats)


WARM_S = 0.2     # untimed replays before the timed one (clocks settle after ~40 ms of work)


def graph_ms(torch, fn, steps):
    """Mean ms per step of `fn(i, stream)` for i < steps, captured once into a
    HIP graph and replayed between two HIP events on the replay stream.
    Untimed replays run first for at least WARM_S seconds (and at least two):
    a config-1 step measures about 10.7 us in the first 10 ms of sustained
    work and settles at 9.9-10.0 us from about 40 ms on."""
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        with torch.cuda.graph(graph, stream=cap):
            for i in range(steps):
                fn(i, cap)
    stream = torch.cuda.current_stream()
    t_warm, n_warm = time.perf_counter(), 0
    while n_warm < 2 or time.perf_counter() - t_warm < WARM_S:
        graph.replay()
        torch.cuda.synchronize()
        n_warm += 1
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    graph.replay()
    t1.record(stream)
    torch.cuda.synchronize()
    del graph
    return t0.elapsed_time(t1) / steps


def run_dense(torch, hip, qt, bs, mats, x, steps, warmup, split=False):
    """Rotating copies of `mats`.  Each step is one grouped GEMV launch that
    prepares x inside its workgroups; with split=True, a stand-alone x-prep
    launch followed by the GEMV on the prepared digits."""
    per_copy = sum(len(p) for _, p, _, _ in mats)
    n_copies = max(2, math.ceil(ROTATE_BYTES / per_copy))
    copies = [[hip.Tensor(p, qt, r, c, bs) for _, p, r, c in mats] for _ in range(n_copies)]
    cols = mats[0][3]
    dx = torch.from_numpy(x).to("cuda:0")
    xq = torch.empty(hip.xprep_bytes(qt, bs, cols) + 256, dtype=torch.uint8, device="cuda:0")
    xq_addr = (xq.data_ptr() + 255) & ~255
    ys = [torch.empty(r, device="cuda:0") for _, _, r, _ in mats]

    def step(i, stream):
        ts = copies[i % n_copies]
        if split:
            hip.xprep(qt, bs, cols, dx, xq_addr, stream=stream)
            hip.matvec_group_prepared(ts, dx, xq_addr, ys, stream=stream)
        else:
            hip.matvec_group(ts, dx, ys, stream=stream)

    for i in range(warmup):
        step(i, torch.cuda.current_stream())
    torch.cuda.synchronize()
    ms = graph_ms(torch, step, steps)
    # the bare-read floor: one launch per step that only streams the same
    # tensors' device bytes, over the same rotation, timed the same way
    sink = torch.zeros(1, dtype=torch.int32, device="cuda:0")

    def read_step(i, stream):
        hip.stream_read(copies[i % n_copies], sink, stream=stream)

    for i in range(warmup):
        read_step(i, torch.cuda.current_stream())
    torch.cuda.synchronize()
    read_ms = graph_ms(torch, read_step, steps)
    for ts in copies:
        for t in ts:
            t.free()
    return {"ms_per_step": ms, "read_ms_per_step": read_ms, "n_copies": n_copies,
            "rotation_mib": n_copies * per_copy / (1 << 20)}


def cpu_baseline_dense(qt, bs, mats, x, budget_s=10.0):
    """QStream's own AVX2 kernel (oracle/_ref) on host cores, 1 thread; falls
    back to this build's scalar restatement (oracle) if _ref is absent."""
    from oracle.oracle import Oracle, ref_avx2
    ref = ref_avx2()
    kind, fn = ("reference", None)
    if ref is not None:
        def fn(p, r, c):
            return ref.matvec(qt, p, x, r, c, bs, isa="avx2")
        name = {9: "qsf_matvec_outlier_2bit_avx2", 3: "qsf_matvec_4bit_avx2"}[qt]
    else:
        kind = "port"
        o = Oracle()

        def fn(p, r, c):
            return o.matvec(qt, p, x, r, c, bs)
        name = "oracle scalar"
    # distinct host copies, rotated, >= HOST_ROTATE_BYTES in all: past the
    # host's last-level cache, so every step reads its weights from DRAM
    per_step = algo_bytes(mats)
    n_host = max(4, math.ceil(HOST_ROTATE_BYTES / per_step))
    hcopies = [[(np.array(p, copy=True), r, c) for _, p, r, c in mats] for _ in range(n_host)]
    times = []
    t_start = time.perf_counter()
    i = 0
    while time.perf_counter() - t_start < budget_s or len(times) < 3:
        t = time.perf_counter()
        for p, r, c in hcopies[i % n_host]:
            fn(p, r, c)
        times.append(time.perf_counter() - t)
        i += 1
        if len(times) >= 200:
            break
    med = float(np.median(times))
    return {"value": per_step / med / 1e9, "unit": "GB/s", "cores": 1, "kind": kind,
            "sample": f"{name}, {len(times)} steps ({len(mats)} matrices per step) over {n_host} host "
                      f"copies ({n_host * per_step / (1 << 20):.0f} MiB rotated), median "
                      f"{med * 1e3:.1f} ms/step, {time.perf_counter() - t_start:.1f} s"}


def _sha16(path: str):
    import hashlib
    try:
        with open(path, "rb") as f:
            return hashlib.sha256(f.read()).hexdigest()[:16]
    except OSError:
        return None


def measured_traffic(key: str):
    """HBM bytes per launch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE
    (scaled by the copy-kernel calibration), as recorded in
    profiles/traffic.json, or None when not measured or when the kernel
    source it was measured on (`kernel_src`, sha256 prefix
    `kernel_src_sha16`) has changed since."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f)[key]
    except (OSError, KeyError, ValueError):
        return None
    src, sha = rec.get("kernel_src"), rec.get("kernel_src_sha16")
    if not src or not sha or _sha16(os.path.join(ROOT, src)) != sha:
        return None
    return rec.get("traffic_bytes")


def run_profile(torch, hip, cfg, steps, warmup):
    """Eager launches only (no graph, no events): the command the rocprofv3
    counter passes run."""
    qt, bs, mats, x = cfg1_data() if cfg == 1 else cfg0_data()
    per_copy = sum(len(p) for _, p, _, _ in mats)
    n_copies = max(2, math.ceil(ROTATE_BYTES / per_copy))
    copies = [[hip.Tensor(p, qt, r, c, bs) for _, p, r, c in mats] for _ in range(n_copies)]
    dx = torch.from_numpy(x).to("cuda:0")
    ys = [torch.empty(r, device="cuda:0") for _, _, r, _ in mats]
    stream = torch.cuda.current_stream()
    for i in range(warmup + steps):
        hip.matvec_group(copies[i % n_copies], dx, ys, stream=stream)
    torch.cuda.synchronize()
    log(f"profile run: config {cfg}, {warmup} + {steps} launches done")


def table_slot_step_us(hip, qt, bs, mats, x, calls=200, lookahead=None):
    """PCIe-inclusive latency of the drop-in path: the qsf_matvec_fn table
    slot (host x and y, synchronous; x prepared from host-mapped memory by
    one small dispatch, the GEMV writing y into host-mapped memory, one
    stream synchronisation) called through ctypes with precomputed pointers,
    weights already resident in the device arena (one copy, so they may sit
    in the MALL).  Every step has its own x, as a decode loop does (the
    matrices of one step share it, as gate and up share a token's x), so
    each step pays one x preparation.  With the slots' look-ahead (the
    library default) the first call of a step, once learnt, runs the second
    matrix in its own launch and the second call is served its result;
    lookahead=0 times every call alone.  Microseconds per step."""
    from qstream_amd import qsf_format as F
    L = hip.load()
    old = L.qsf_hip_slot_lookahead(-1 if lookahead is None else lookahead)
    name = {F.Q2: "matvec_2bit", F.Q3: "matvec_3bit", F.Q4: "matvec_4bit",
            F.Q4SYM: "matvec_4bit_sym", F.Q2_OUTLIER: "matvec_outlier_2bit",
            F.Q4_OUTLIER: "matvec_outlier_4bit"}[qt]
    fn = getattr(L, f"qsf_{name}_hip")
    ws = [np.frombuffer(p, np.uint8) for _, p, _, _ in mats]
    xs = [np.ascontiguousarray(x * (1.0 + 2.0 ** -10 * i), np.float32) for i in range(4)]
    outs = [np.empty(r, np.float32) for _, _, r, _ in mats]
    steps = [[(w.ctypes.data, xh.ctypes.data, o.ctypes.data, r, c, bs)
              for w, o, (_, _, r, c) in zip(ws, outs, mats)] for xh in xs]
    for i in range(10):
        for a in steps[i % 4]:
            fn(*a)
    t0 = time.perf_counter()
    for i in range(calls):
        for a in steps[i % 4]:
            fn(*a)
    dt = time.perf_counter() - t0
    L.qsf_hip_slot_lookahead(old)
    for w in ws:
        hip.arena_forget(w)
    return dt / calls * 1e6


def bench_dense(torch, hip, cfg, steps, warmup, with_cpu=True, split=False, slot=True,
                cpu_budget=10.0):
    qt, bs, mats, x = cfg1_data() if cfg == 1 else cfg0_data()
    log(f"config {cfg}: data ready ({len(mats)} matrices)")
    res = run_dense(torch, hip, qt, bs, mats, x, steps, warmup, split)
    bytes_step = algo_bytes(mats)
    us_step = res["ms_per_step"] * 1e3
    value = bytes_step / (us_step * 1e-6) / 1e9
    out = {
        "value": value,
        "ms_per_step": res["ms_per_step"],
        "us_per_call": us_step / len(mats),
        "bytes_per_step": bytes_step,
        "rotation_mib": res["rotation_mib"],
    }
    if not split:
        # one GEMV launch per step: the graph-replayed timed region per
        # launch is the kernel's time (launch gaps included, so it errs low)
        out["roofline"] = {"bound": "hbm", "kernel": "decode GEMV (one launch per step)",
                           "timing": "graph replay of the steps",
                           "achieved": round(value, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                           "frac": round(value / HBM_PEAK_GBS, 4),
                           "traffic": measured_traffic(f"cfg{cfg}"),
                           "kernel_us": round(us_step, 3), "launches_timed": steps,
                           "bytes_per_launch": bytes_step}
    read_us = res["read_ms_per_step"] * 1e3
    out["read_floor"] = {"kernel": "stream_read_kernel (one launch per step, same rotated tensors)",
                         "us_per_step": round(read_us, 3),
                         "achieved": round(bytes_step / (read_us * 1e-6) / 1e9, 2), "unit": "GB/s",
                         "frac": round(bytes_step / (read_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                         "gemv_over_floor": round(us_step / read_us, 3)}
    if slot:
        out["table_slot_us_per_step"] = table_slot_step_us(hip, qt, bs, mats, x)
        out["table_slot_alone_us_per_step"] = table_slot_step_us(hip, qt, bs, mats, x, lookahead=0)
    if with_cpu:
        out["cpu_baseline"] = cpu_baseline_dense(qt, bs, mats, x, cpu_budget)
    return out


def cpu_baseline_prefill(payload, xb, m, n, k, bs, budget_s=10.0):
    """The reference's prefill: one qsf_matvec_4bit call per token
    (src/engine.c:1289-1295), QStream's AVX2 kernel (oracle/_ref), 1 thread,
    on as many of the M tokens as fit in the time budget."""
    from oracle.oracle import Oracle, ref_avx2
    from qstream_amd import qsf_format as F
    ref = ref_avx2()
    xf = (xb.astype(np.uint32) << 16).view(np.float32)
    # host copies of the weights in rotation, past the host LLC
    n_host = max(2, math.ceil(HOST_ROTATE_BYTES / len(payload)))
    hcopies = [np.array(np.frombuffer(payload, np.uint8), copy=True) for _ in range(n_host)]
    if ref is not None:
        kind, name = "reference", "qsf_matvec_4bit_avx2"

        def fn(w, x):
            return ref.matvec(F.Q4, w, x, n, k, bs, isa="avx2")
    else:
        kind, name, o = "port", "oracle scalar", Oracle()

        def fn(w, x):
            return o.matvec(F.Q4, w, x, n, k, bs)
    t0 = time.perf_counter()
    done = 0
    while done < m and (time.perf_counter() - t0 < budget_s or done < 2):
        fn(hcopies[done % n_host], xf[done])
        done += 1
    el = time.perf_counter() - t0
    return {"value": 2.0 * n * k * done / el / 1e12, "unit": "TFLOP/s", "cores": 1, "kind": kind,
            "sample": f"{name}, {done} of {m} tokens (one {n}x{k} matvec each) over {n_host} host "
                      f"weight copies ({n_host * len(payload) / (1 << 20):.0f} MiB rotated), {el:.1f} s"}


def profile_prefill(torch, hip, steps, warmup):
    """Eager config-4 launches only (for rocprofv3 passes)."""
    from qstream_amd import qsf_format as F
    payload, xb, m, n, k, bs = cfg4_data()
    n_copies = max(2, math.ceil(ROTATE_BYTES / len(payload)))
    copies = [hip.Tensor(payload, F.Q4, n, k, bs) for _ in range(n_copies)]
    dx = torch.from_numpy(xb.view(np.int16).copy()).to("cuda:0")
    y = torch.empty((m, n), device="cuda:0")
    for i in range(warmup + steps):
        copies[i % n_copies].prefill(dx, m, y, stream=torch.cuda.current_stream())
    torch.cuda.synchronize()
    log(f"profile run: config 4, {warmup} + {steps} launches done")


def bench_prefill(torch, hip, steps, warmup, with_cpu=True, cpu_budget=10.0):
    """Config 4: one MFMA prefill (x repack + GEMM launch) per step over a
    rotating weight copy.  The GEMM's own time: a graph of GEMM-only
    launches (the packed-x half of the prefill, qsf_hip_prefill_4bit_packed_dev)
    over the same rotation, x packed once before it, timed like the steps."""
    from qstream_amd import qsf_format as F
    payload, xb, m, n, k, bs = cfg4_data()
    log(f"config 4: data ready ({m}x{n}x{k}, block {bs})")
    n_copies = max(2, math.ceil(ROTATE_BYTES / len(payload)))
    copies = [hip.Tensor(payload, F.Q4, n, k, bs) for _ in range(n_copies)]
    dx = torch.from_numpy(xb.view(np.int16).copy()).to("cuda:0")
    y = torch.empty((m, n), device="cuda:0")

    def step(i, stream):
        copies[i % n_copies].prefill(dx, m, y, stream=stream)

    for i in range(warmup):
        step(i, torch.cuda.current_stream())
    torch.cuda.synchronize()
    ms = graph_ms(torch, step, steps)
    packed = torch.empty(hip.prefill_pack_bytes(m, k, bs) + 256, dtype=torch.uint8, device="cuda:0")
    paddr = (packed.data_ptr() + 255) & ~255
    hip.prefill_pack(dx, m, k, bs, paddr, stream=torch.cuda.current_stream())

    def gemm_step(i, stream):
        copies[i % n_copies].prefill_packed(paddr, m, y, stream=stream)

    for i in range(warmup):
        gemm_step(i, torch.cuda.current_stream())
    torch.cuda.synchronize()
    kus = graph_ms(torch, gemm_step, steps) * 1e3
    for t in copies:
        t.free()
    # the matrix-core ceiling on this box, beside the published peak: a graph
    # of launches of independent v_mfma_f32_16x16x32_bf16 chains, no memory
    sink = torch.zeros(4, dtype=torch.int32, device="cuda:0")
    probe_iters = 512
    probe_flop = hip.mfma_peak(probe_iters, sink)
    torch.cuda.synchronize()
    probe_us = graph_ms(torch, lambda i, st: hip.mfma_peak(probe_iters, sink, stream=st), 20) * 1e3
    probe = {"kernel": "mfma_peak_kernel (independent v_mfma_f32_16x16x32_bf16 chains on every SIMD, "
                       "no memory traffic)",
             "timing": "graph of 20 launches", "us_per_launch": round(probe_us, 3),
             "tflops": round(probe_flop / (probe_us * 1e-6) / 1e12, 1)}
    probe["frac_of_published_peak"] = round(probe["tflops"] / BF16_MFMA_PEAK_TFS, 4)
    flops = 2.0 * m * n * k
    out = {"value": flops / (ms * 1e-3) / 1e12, "ms_per_step": ms, "us_kernel": kus,
           "flops_per_step": flops, "weight_bytes": len(payload),
           "roofline": {"bound": "mfma", "kernel": "prefill_kernel (the GEMM half)",
                        "timing": "graph of GEMM-only launches over the rotation",
                        "achieved": round(flops / (kus * 1e-6) / 1e12, 2),
                        "peak": BF16_MFMA_PEAK_TFS, "unit": "TFLOP/s",
                        "frac": round(flops / (kus * 1e-6) / 1e12 / BF16_MFMA_PEAK_TFS, 4),
                        "traffic": measured_traffic("cfg4"), "kernel_us": round(kus, 3),
                        "launches_timed": steps},
           "rotation_mib": n_copies * len(payload) / (1 << 20), "m": m, "n": n, "k": k,
           "mfma_probe": probe}
    if with_cpu:
        out["cpu_baseline"] = cpu_baseline_prefill(payload, xb, m, n, k, bs, cpu_budget)
    return out


def profile_layers(torch, hip, steps, warmup):
    """Eager config-2 gate/up launches only (the dominant kernel), rotating
    over copies beyond the MALL, for rocprofv3 counter passes."""
    qt, bs, mats = cfg2_layer()
    gu = mats[4:6]
    per_copy = sum(len(p) for _, p, _, _ in gu)
    n_copies = max(2, math.ceil(ROTATE_BYTES / per_copy))
    copies = [[hip.Tensor(p, qt, r, c, bs) for _, p, r, c in gu] for _ in range(n_copies)]
    x = torch.from_numpy(np.random.default_rng(21).standard_normal(4096).astype(np.float32)).to("cuda:0")
    ys = [torch.empty(r, device="cuda:0") for _, _, r, _ in gu]
    stream = torch.cuda.current_stream()
    for i in range(warmup + steps):
        hip.matvec_group(copies[i % n_copies], x, ys, stream=stream)
    torch.cuda.synchronize()
    log(f"profile run: config 2 gate/up, {warmup} + {steps} launches done")


def profile_decode_layer(torch, hip, steps, warmup):
    """Eager launches of the layer step's dominant kernel only (the fused
    residual + norm + gate/up + act launch over 32 layers' pairs), for
    rocprofv3 counter passes."""
    qt, bs, mats = cfg2_layer()
    pairs = [hip.TensorPair(mats[4][1], mats[5][1], qt, mats[4][2], mats[4][3], bs) for _ in range(32)]
    g = torch.Generator(device="cuda:0").manual_seed(41)
    res, res2 = torch.randn(4096, device="cuda:0", generator=g), torch.empty(4096, device="cuda:0")
    x = torch.randn(4096, device="cuda:0", generator=g)
    w = torch.ones(4096, device="cuda:0")
    out = torch.empty(mats[4][2], device="cuda:0")
    stream = torch.cuda.current_stream()
    for i in range(warmup + steps):
        pairs[i % 32].residual_norm_gate_up_act(res, res2, x, w, 1e-5, out, 2, stream=stream)
    torch.cuda.synchronize()
    log(f"profile run: layer step gate/up, {warmup} + {steps} launches done")
    for pr in pairs:
        pr.free()


def upload_layer_tensors(hip, qt, bs, mats):
    """One layer's tensors, each on the decode engine that runs its launch
    fastest: o, a 4096 x 4096 matrix launched alone, on the dot-product
    kernels (4.8 against 5.8 us a launch on the matrix core, which needs
    more rows a launch to fill its workgroups), the others (q/k/v launched
    as a group, gate/up, down) on the library's default engine."""
    out = []
    for name, p, r, c in mats:
        prev = hip.gemv_engine(0) if name == "o" else None
        try:
            out.append(hip.Tensor(p, qt, r, c, bs))
        finally:
            if prev is not None:
                hip.gemv_engine(prev)
    return out


def bench_layers(torch, hip, steps, warmup, with_cpu=True, cpu_budget=10.0):
    """Config 2: 32 decoder layers at 3-bit back to back.  A step is the
    whole stack: per layer q/k/v in one grouped launch, o, gate/up grouped,
    down -- 128 launches, each on its own fresh x."""
    qt, bs, mats = cfg2_layer()
    log("config 2: layer quantised")
    layers = [upload_layer_tensors(hip, qt, bs, mats) for _ in range(32)]
    rng = np.random.default_rng(20)
    xs = [torch.from_numpy(rng.standard_normal((4, 11008)).astype(np.float32)).to("cuda:0")
          for _ in range(32)]
    ys = {n: torch.empty(r, device="cuda:0") for n, _, r, _ in mats}

    def step(i, stream):
        for li, ts in enumerate(layers):
            x = xs[li]
            hip.matvec_group(ts[0:3], x[0, :4096], [ys["q"], ys["k"], ys["v"]], stream=stream)
            hip.matvec_group(ts[3:4], x[1, :4096], [ys["o"]], stream=stream)
            hip.matvec_group(ts[4:6], x[2, :4096], [ys["gate"], ys["up"]], stream=stream)
            hip.matvec_group(ts[6:7], x[3], [ys["down"]], stream=stream)

    for i in range(warmup):
        step(i, torch.cuda.current_stream())
    torch.cuda.synchronize()
    ms = graph_ms(torch, step, steps)
    # Dominant kernel: the gate/up launch (45% of a layer's bytes).  Its
    # duration is the time per launch of a graph of 32 back-to-back gate/up
    # launches on the 32 layers' copies, HIP events around the replay on the
    # launch stream (kernel-edge event pairs on these eager launches read
    # well above the profiler's kernel durations).
    def gu_step(i, stream):
        hip.matvec_group(layers[i][4:6], xs[i][2, :4096], [ys["gate"], ys["up"]], stream=stream)

    gu_us = graph_ms(torch, gu_step, 32) * 1e3
    for ts in layers:
        for t in ts:
            t.free()
    per_layer = algo_bytes(mats)
    total = 32 * per_layer
    gu_bytes = algo_bytes(mats[4:6])
    out = {"value": total / (ms * 1e-3) / 1e9, "ms_per_step": ms, "bytes_per_step": total}
    out["roofline"] = {"bound": "hbm", "kernel": "decode GEMV, gate/up launch (2 x 11008x4096 3-bit)",
                       "timing": "graph of 32 gate/up launches (one a layer)",
                       "achieved": round(gu_bytes / (gu_us * 1e-6) / 1e9, 2),
                       "peak": HBM_PEAK_GBS, "unit": "GB/s",
                       "frac": round(gu_bytes / (gu_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                       "traffic": measured_traffic("cfg2"), "kernel_us": round(gu_us, 3),
                       "bytes_per_launch": gu_bytes}
    if with_cpu:
        out["cpu_baseline"] = cpu_baseline_layer(qt, bs, mats, cpu_budget)
    return out


def bench_decode_layer(torch, hip, steps, warmup, position=1023):
    """One device-resident 7B decoder layer step per step (LLaMA-7B shapes:
    hidden 4096, 32 heads of 128, intermediate 11008, 3-bit block 128
    weights): residual + NaN check + attention RMSNorm + q/k/v (one grouped
    launch: the previous layer's down output joins the residual, whose norm
    the q/k/v rows multiply), RoPE + int8 KV store + attention over
    `position` + 1 cached positions (two launches: rotation, store and the
    chunk pass in one, then the chunk combine), o, residual + FFN RMSNorm +
    gate/up with SiLU x up (one launch over the interleaved gate/up pair),
    down -- 6 launches, no host round trip.  The residual alternates
    between two buffers (a fused launch reads one while it writes the
    other).  Steps cycle over 32 layers' distinct weights and
    KV caches (2.9 GB), so neither stays in the MALL.  Bytes per step: the
    layer's weight payloads, the KV rows attention reads, activations."""
    qt, bs, mats = cfg2_layer()
    log("layer: weights quantised")
    hid, nh, hd, eid, max_seq, n_layers = 4096, 32, 128, 11008, position + 1, 32
    # q, k, v, o and down as tensors; gate and up as one interleaved pair
    layers = [upload_layer_tensors(hip, qt, bs, mats[:4] + mats[6:7]) for _ in range(n_layers)]
    pairs = [hip.TensorPair(mats[4][1], mats[5][1], qt, mats[4][2], mats[4][3], bs)
             for _ in range(n_layers)]
    g = torch.Generator(device="cuda:0").manual_seed(40)
    kcs = [torch.randint(-127, 128, (nh, max_seq, hd), dtype=torch.int8, device="cuda:0", generator=g)
           for _ in range(n_layers)]
    vcs = [torch.randint(-127, 128, (nh, max_seq, hd), dtype=torch.int8, device="cuda:0", generator=g)
           for _ in range(n_layers)]
    kss = [torch.rand((nh, max_seq), device="cuda:0", generator=g) * 0.02 for _ in range(n_layers)]
    vss = [torch.rand((nh, max_seq), device="cuda:0", generator=g) * 0.02 for _ in range(n_layers)]
    an_w = torch.ones(hid, device="cuda:0")
    fn_w = torch.ones(hid, device="cuda:0")
    rope = hip.Rope(hd, 10000.0)
    res = torch.randn(hid, device="cuda:0", generator=g)
    res2 = torch.empty(hid, device="cuda:0")
    ys = {n: torch.empty(r, device="cuda:0") for n, _, r, _ in mats}
    ys["down"].zero_()                        # the first layer's residual increment
    attn = torch.empty(nh * hd, device="cuda:0")
    bad = torch.zeros(1, dtype=torch.int32, device="cuda:0")

    def step(i, stream):
        li = i % n_layers
        ts = layers[li]
        hip.residual_norm_matvec_group(ts[0:3], res, res2, ys["down"], an_w, 1e-5,
                                       [ys["q"], ys["k"], ys["v"]], bad=bad, stream=stream)
        rope.apply_store_attend(ys["q"], ys["k"], ys["v"], nh, nh, position, kcs[li], vcs[li], kss[li],
                                vss[li], max_seq, attn, stream=stream)
        hip.matvec_group(ts[3:4], attn, [ys["o"]], stream=stream)
        pairs[li].residual_norm_gate_up_act(res2, res, ys["o"], fn_w, 1e-5, ys["gate"], 2, stream=stream)
        hip.matvec_group(ts[4:5], ys["gate"], [ys["down"]], stream=stream)

    for i in range(warmup):
        step(i, torch.cuda.current_stream())
    torch.cuda.synchronize()
    ms = graph_ms(torch, step, steps)
    # Dominant kernel: the fused residual + FFN norm + gate/up + SiLU x up
    # launch (45% of the layer's weight bytes), a graph of one such launch
    # per layer over the 32 layers' pairs, timed like the steps.
    def gu_step(i, stream):
        pairs[i % n_layers].residual_norm_gate_up_act(res2, res, ys["o"], fn_w, 1e-5, ys["gate"], 2,
                                                      stream=stream)

    gu_us = graph_ms(torch, gu_step, n_layers) * 1e3
    rope.free()
    for ts in layers:
        for t in ts:
            t.free()
    for pr in pairs:
        pr.free()
    kv_bytes = 2 * nh * max_seq * (hd + 4)
    total = algo_bytes(mats) + kv_bytes
    gu_bytes = algo_bytes(mats[4:6]) + 3 * 4 * hid     # + residual in/out and norm weights
    return {"value": total / (ms * 1e-3) / 1e9, "ms_per_step": ms, "bytes_per_step": total,
            "weight_bytes": algo_bytes(mats), "kv_bytes": kv_bytes, "position": position,
            "roofline": {"bound": "hbm",
                         "kernel": "residual + norm + gate/up + act launch (2 x 11008x4096 3-bit, interleaved)",
                         "timing": "graph of 32 such launches (one a layer)",
                         "achieved": round(gu_bytes / (gu_us * 1e-6) / 1e9, 2), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gu_bytes / (gu_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                         "traffic": measured_traffic("layer"), "kernel_us": round(gu_us, 3),
                         "bytes_per_launch": gu_bytes}}


def cpu_baseline_layer(qt, bs, mats, budget_s=10.0):
    """The reference's 3-bit matvec is scalar on every ISA
    (src/kernels.c:10): qsf_matvec_3bit_scalar from oracle/_ref (reference
    release flags), 1 thread, over one layer's matrices."""
    from oracle.oracle import Oracle, ref_avx2
    ref = ref_avx2()
    rng = np.random.default_rng(21)
    kind = "reference" if ref is not None else "port"
    o = None if ref is not None else Oracle()
    # host copies of the layer in rotation, past the host LLC
    n_host = max(2, math.ceil(HOST_ROTATE_BYTES / algo_bytes(mats)))
    hcopies = [[(np.array(np.frombuffer(p, np.uint8), copy=True), r, c) for _, p, r, c in mats]
               for _ in range(n_host)]
    xs = {c: rng.standard_normal(c).astype(np.float32) for _, _, _, c in mats}
    t0 = time.perf_counter()
    done = 0
    nbytes = 0
    while time.perf_counter() - t0 < budget_s or done == 0:
        for p, r, c in hcopies[done % n_host]:
            if ref is not None:
                ref.matvec(qt, p, xs[c], r, c, bs, isa="scalar")
            else:
                o.matvec(qt, p, xs[c], r, c, bs)
            nbytes += len(p) + 4 * c + 4 * r
        done += 1
    el = time.perf_counter() - t0
    return {"value": nbytes / el / 1e9, "unit": "GB/s", "cores": 1, "kind": kind,
            "sample": f"qsf_matvec_3bit_scalar over {done} layer(s) of 7 matrices, {n_host} host copies "
                      f"rotated ({n_host * algo_bytes(mats) / (1 << 20):.0f} MiB), {el:.1f} s"}


def profile_moe(torch, hip, steps, warmup, ntok):
    """Eager config-3 steps only (routing, gate/up, down, combine), for
    rocprofv3 counter passes."""
    from qstream_amd import qsf_format as F
    n_exp, dim, k = 32, 2880, 4
    # built in this process: worker processes started under a counter pass
    # each carry the profiler, and one of them has failed to exit
    ex = cfg3_experts(workers=1)
    tens = {n: [hip.Tensor(e[n], F.MXFP4, dim, dim, 32) for e in ex] for n in ("gate", "up", "down")}
    moe = hip.Moe(tens["gate"], tens["up"], tens["down"], dim, dim)
    rng = np.random.default_rng(30 + ntok)
    nset = 64
    logits = torch.from_numpy(rng.standard_normal((nset, ntok, n_exp)).astype(np.float32)).to("cuda:0")
    xs = torch.from_numpy(rng.standard_normal((nset, ntok, dim)).astype(np.float32)).to("cuda:0")
    out = torch.empty((ntok, dim), device="cuda:0")
    stream = torch.cuda.current_stream()
    for i in range(warmup + steps):
        moe.forward(k, 1, 2, ntok, xs[i % nset], logits[i % nset], out, stream=stream)
    torch.cuda.synchronize()
    log(f"profile run: config 3 batch {ntok}, {warmup} + {steps} steps done")
    moe.free()
    for ts in tens.values():
        for t in ts:
            t.free()


def bench_moe(torch, hip, steps, warmup, ntok, with_cpu=True, cpu_budget=10.0, ex=None):
    """Config 3: MXFP4 MoE FFN, 32 experts, hidden = expert dim = 2880,
    top-4 softmax routing, ntok tokens per step.  Each step draws new router
    logits (64 seeded sets in rotation), so the experts read change."""
    from qstream_amd import qsf_format as F
    n_exp, dim, k = 32, 2880, 4
    if ex is None:
        ex = cfg3_experts()
    log(f"config 3: experts ready (batch {ntok})")
    tens = {n: [hip.Tensor(e[n], F.MXFP4, dim, dim, 32) for e in ex] for n in ("gate", "up", "down")}
    moe = hip.Moe(tens["gate"], tens["up"], tens["down"], dim, dim)
    rng = np.random.default_rng(30 + ntok)
    nset = 64
    logits_h = rng.standard_normal((nset, ntok, n_exp)).astype(np.float32)
    xs = torch.from_numpy(rng.standard_normal((nset, ntok, dim)).astype(np.float32)).to("cuda:0")
    logits = torch.from_numpy(logits_h).to("cuda:0")
    out = torch.empty((ntok, dim), device="cuda:0")

    def step(i, stream):
        j = i % nset
        moe.forward(k, 1, 2, ntok, xs[j], logits[j], out, stream=stream)

    for i in range(warmup):
        step(i, torch.cuda.current_stream())
    torch.cuda.synchronize()
    ms = graph_ms(torch, step, steps)
    # algorithmic bytes per step: distinct experts x 3 matrices + activations
    per_mat = dim * (dim // 32) * 17
    distinct = []
    for i in range(steps):
        lg = logits_h[i % nset]
        sel = set()
        for t in range(ntok):
            sel.update(np.argsort(-lg[t], kind="stable")[:k].tolist())
        distinct.append(len(sel))
    bytes_step = float(np.mean(distinct)) * 3 * per_mat + ntok * dim * 4 * 2
    # Dominant kernel: the gate/up expert launch (two of the three matrices
    # of every distinct expert), timed like the steps, by graph replay of
    # steps that launch only it (qsf_hip_moe_stages: one token routes inside
    # it); with several tokens, a graph of routing + gate/up less one of the
    # routing launch alone.  Algorithmic bytes = its expert codes and scales
    # + x + h written.
    prev = hip.moe_stages(3)
    try:
        gu_ms = graph_ms(torch, step, steps)
        if ntok > 1:
            hip.moe_stages(1)
            gu_ms -= graph_ms(torch, step, steps)
    finally:
        hip.moe_stages(prev)
    gu_us = gu_ms * 1e3
    gu_bytes = np.asarray(distinct, np.float64) * 2 * per_mat + ntok * dim * 4 * 2
    roof = float(np.mean(gu_bytes)) / (gu_us * 1e-6) / 1e9
    moe.free()
    for ts in tens.values():
        for t in ts:
            t.free()
    res = {"value": bytes_step / (ms * 1e-3) / 1e9, "ms_per_step": ms, "bytes_per_step": bytes_step,
           "distinct_experts_mean": float(np.mean(distinct))}
    res["roofline"] = {"bound": "hbm", "kernel": "moe_gate_up_kernel",
                       "timing": ("graph of gate/up-only steps (routing inside the launch)" if ntok == 1 else
                                  "graph of routing + gate/up steps less a graph of routing-only steps"),
                       "achieved": round(roof, 2),
                       "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(roof / HBM_PEAK_GBS, 4),
                       "traffic": measured_traffic(f"cfg3_b{ntok}"),
                       "kernel_us": round(gu_us, 3),
                       "bytes_per_launch": round(float(np.mean(gu_bytes)))}
    if with_cpu:
        res["cpu_baseline"] = cpu_baseline_moe(ex, ntok, k, dim, logits_h, xs.cpu().numpy(),
                                               cpu_budget)
        # the reference's own GPT-OSS path, beside the port of the MXFP4 math
        # (per token, so batch 1 and batch 8 share one measurement)
        key = (k, dim)
        if key not in _MOE_REF4:
            _MOE_REF4[key] = cpu_baseline_moe_ref4(k, dim, min(3.0, cpu_budget))
        res["cpu_baseline"]["reference_4bit_path"] = _MOE_REF4[key]
    return res


def cpu_baseline_moe(ex, ntok, k, dim, logits_h, xs, budget_s=10.0):
    """No reference CPU kernel reads MXFP4 (the reference re-quantises GPT-OSS
    experts to its own formats: cpu_baseline_moe_ref4 times that path).  This
    times this build's scalar restatement of the same MoE token (oracle,
    strict fp32, 1 thread)."""
    from oracle.oracle import Oracle
    o = Oracle()
    t0 = time.perf_counter()
    toks = 0
    nbytes = 0.0
    per_mat = dim * (dim // 32) * 17
    while time.perf_counter() - t0 < budget_s or toks == 0:
        j = toks % len(logits_h)
        o.moe_token(ex, k, 1, 2, dim, dim, xs[j, 0], logits_h[j, 0])
        toks += 1
        nbytes += k * 3 * per_mat + 2 * dim * 4
    el = time.perf_counter() - t0
    return {"value": nbytes / el / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"oracle MoE token (scalar MXFP4), {toks} tokens, {el:.1f} s"}


_MOE_REF4 = {}


def cpu_baseline_moe_ref4(k, dim, budget_s=3.0):
    """The reference's own path for GPT-OSS experts: its converter re-quantises
    them to its 4-bit format (block 64), and each token then runs k experts'
    gate, up and down as qsf_matvec_4bit_avx2 calls (src/engine.c:1024-1107),
    1 thread.  Timed on synthetic 4-bit payloads of the experts' shape (codes
    random, every block's scale and zero a fixed normal fp16 pair: the AVX2
    kernel's time does not depend on the values), rotated over >= 768 MiB of
    distinct host matrices.  None without oracle/_ref."""
    from oracle.oracle import ref_avx2
    ref = ref_avx2()
    if ref is None:
        return None
    bs, bb = 64, 36
    nb = (dim + bs - 1) // bs
    per_mat = dim * nb * bb
    n_mats = max(3 * k, math.ceil(HOST_ROTATE_BYTES / per_mat))
    rng = np.random.default_rng(7)
    meta = np.frombuffer(np.array([0.003, -0.01], np.float16).tobytes(), np.uint8)
    mats = []
    for _ in range(n_mats):
        m = rng.integers(0, 256, (dim * nb, bb), dtype=np.uint8)
        m[:, :4] = meta
        mats.append(m.reshape(-1))
    x = rng.standard_normal(dim).astype(np.float32)
    times, i = [], 0
    t_start = time.perf_counter()
    while time.perf_counter() - t_start < budget_s or len(times) < 3:
        t = time.perf_counter()
        for _ in range(3 * k):
            ref.matvec(3, mats[i % n_mats], x, dim, dim, bs, isa="avx2")
            i += 1
        times.append(time.perf_counter() - t)
    med = float(np.median(times))
    return {"value": 3 * k * per_mat / med / 1e9, "unit": "GB/s", "us_per_token": round(med * 1e6, 1),
            "cores": 1, "kind": "reference",
            "sample": f"qsf_matvec_4bit_avx2 x {3 * k} a token (k = {k} experts' gate, up, down re-quantised "
                      f"to 4-bit block 64, {dim}x{dim}), {len(times)} tokens over {n_mats} host matrices "
                      f"({n_mats * per_mat / (1 << 20):.0f} MiB rotated), median {med * 1e3:.2f} ms/token"}


def copy_calibration(torch, steps, warmup, mib=512):
    """Plain device-to-device copy of a known size: the reference point for
    HBM counters (FETCH_SIZE / WRITE_SIZE per byte moved) and for what the
    memory system sustains on this box."""
    n = (mib << 20) // 4
    a = torch.randn(n, device="cuda:0")
    b = torch.empty_like(a)
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        b.copy_(a)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(steps):
        b.copy_(a)
    t1.record(stream)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    moved = 2 * n * 4
    return {"copy_mib": mib, "ms_per_copy": ms, "read_plus_write_GBs": moved / (ms * 1e-3) / 1e9}


DENSE_WORKLOAD = {1: "cfg1: 2-bit+outlier FFN gate+up, 2x 11008x4096, block 64, batch-1 decode",
                  0: "cfg0: 4-bit asym 4096x4096, block 64, batch-1 decode"}
DIGIT_DTYPE = "i4xi4->i32 digit dot, f32 accumulate"


def run_config(torch, hip, key: str, args, cpu_budget: float, cache: dict) -> dict:
    """One config's full JSON object (as printed when it runs alone)."""
    base = {"metric": METRIC, "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None}
    with_cpu = not args.no_cpu
    if key in ("0", "1"):
        cfg = int(key)
        r = bench_dense(torch, hip, cfg, args.steps, args.warmup, with_cpu=with_cpu,
                        split=args.split, slot=not args.no_slot, cpu_budget=cpu_budget)
        conf = {"workload": DENSE_WORKLOAD[cfg], "us_per_call": round(r["us_per_call"], 3),
                "us_per_step_graph": round(r["ms_per_step"] * 1e3, 3),
                "launch": "split x-prep + GEMV" if args.split else "one fused launch per step",
                "bytes_per_step": r["bytes_per_step"],
                "hbm_frac_of_8TBs": round(r["value"] / HBM_PEAK_GBS, 4),
                "rotation_mib": round(r["rotation_mib"], 1)}
        if "read_floor" in r:
            conf["read_floor"] = r["read_floor"]
        if "table_slot_us_per_step" in r:
            conf["table_slot_us_per_step_pcie"] = round(r["table_slot_us_per_step"], 3)
            conf["table_slot_lookahead_off_us_per_step_pcie"] = round(
                r["table_slot_alone_us_per_step"], 3)
            conf["table_slot_gbs_pcie"] = round(
                r["bytes_per_step"] / (r["table_slot_us_per_step"] * 1e-6) / 1e9, 2)
        line = dict(base, value=round(r["value"], 2), ms_per_step=round(r["ms_per_step"], 5),
                    dtype=DIGIT_DTYPE,
                    data="synthetic (seeded N(0,0.02)" + (" + Student-t outliers" if cfg == 1 else "")
                         + ", converter-semantics quantisation)",
                    config=conf)
    elif key == "2":
        r = bench_layers(torch, hip, args.steps, args.warmup, with_cpu=with_cpu, cpu_budget=cpu_budget)
        line = dict(base, value=round(r["value"], 2), ms_per_step=round(r["ms_per_step"], 5),
                    dtype=DIGIT_DTYPE, data="synthetic (seeded N(0,0.02), quantised to 3-bit block 128)",
                    config={"workload": "cfg2: 32 x 7B decoder layer at 3-bit block 128, batch-1 "
                                        "decode, back to back",
                            "launches_per_step": 128, "us_per_step_graph": round(r["ms_per_step"] * 1e3, 3),
                            "bytes_per_step": r["bytes_per_step"],
                            "hbm_frac_of_8TBs": round(r["value"] / HBM_PEAK_GBS, 4)})
    elif key in ("3", "3b1", "3b8"):
        ntok = args.moe_batch if key == "3" else int(key[2:])
        if "experts" not in cache:
            cache["experts"] = cfg3_experts(workers=args.data_workers)
        r = bench_moe(torch, hip, args.steps, args.warmup, ntok, with_cpu=with_cpu,
                      cpu_budget=cpu_budget, ex=cache["experts"])
        line = dict(base, value=round(r["value"], 2), ms_per_step=round(r["ms_per_step"], 5),
                    dtype="e2m1 x f32, f32 accumulate",
                    data="synthetic (seeded N(0,0.02) experts quantised to MXFP4; N(0,1) router logits "
                         "and activations)",
                    config={"workload": f"cfg3: MXFP4 MoE FFN, 32 experts 2880x2880, top-4, batch {ntok}",
                            "distinct_experts_mean": round(r["distinct_experts_mean"], 2),
                            "us_per_step_graph": round(r["ms_per_step"] * 1e3, 3),
                            "bytes_per_step": r["bytes_per_step"],
                            "hbm_frac_of_8TBs": round(r["value"] / HBM_PEAK_GBS, 4)})
    elif key == "layer":
        r = bench_decode_layer(torch, hip, args.steps, args.warmup)
        if with_cpu:
            qt, bs, mats = cfg2_layer()
            r["cpu_baseline"] = cpu_baseline_layer(qt, bs, mats, cpu_budget)
            r["cpu_baseline"]["sample"] += " (the layer's matvecs; the glue is under 1% of its bytes)"
        line = dict(base, value=round(r["value"], 2), ms_per_step=round(r["ms_per_step"], 5),
                    dtype=DIGIT_DTYPE + "; glue fp32",
                    data="synthetic (seeded N(0,0.02) weights quantised to 3-bit block 128; random "
                         "int8 KV cache)",
                    config={"workload": f"device-resident 7B decoder layer step (3-bit block 128), "
                                        f"attention over {r['position'] + 1} cached positions, "
                                        f"6 launches (residual + norm fused into q/k/v and into gate/up + "
                                        f"act*mul; RoPE + KV store fused into the attention chunk pass)",
                            "us_per_layer": round(r["ms_per_step"] * 1e3, 3),
                            "bytes_per_step": r["bytes_per_step"], "weight_bytes": r["weight_bytes"],
                            "kv_bytes": r["kv_bytes"],
                            "hbm_frac_of_8TBs": round(r["value"] / HBM_PEAK_GBS, 4)})
    elif key == "4":
        r = bench_prefill(torch, hip, args.steps, args.warmup, with_cpu=with_cpu, cpu_budget=cpu_budget)
        line = dict(base, metric="batched 4-bit prefill TFLOP/s (bf16 MFMA, % of 2.5 PFLOP/s dense peak)",
                    value=round(r["value"], 2), unit="TFLOP/s", ms_per_step=round(r["ms_per_step"], 5),
                    dtype="bf16 x bf16 -> f32 MFMA (4-bit codes as exact bf16 integers, fp32 "
                          "per-block scale and zero-point)",
                    data="synthetic (seeded N(0,0.02) weights, converter-semantics quantisation; "
                         "bf16 N(0,1) activations)",
                    config={"workload": f"cfg4: 4-bit asym prefill M={r['m']} x K={r['k']} x "
                                        f"N={r['n']}, block 64",
                            "us_kernel": round(r["us_kernel"], 3),
                            "us_per_step_graph": round(r["ms_per_step"] * 1e3, 3),
                            "mfma_util_of_peak": round(r["value"] / BF16_MFMA_PEAK_TFS, 4),
                            "flops_per_step": r["flops_per_step"],
                            "rotation_mib": round(r["rotation_mib"], 1),
                            "measured_mfma_ceiling": r["mfma_probe"],
                            "gemm_frac_of_measured_ceiling": round(
                                r["roofline"]["achieved"] / r["mfma_probe"]["tflops"], 4)})
    else:
        raise SystemExit(f"unknown --config {key}")
    if "roofline" in r:
        line["roofline"] = r["roofline"]
    if "cpu_baseline" in r:
        line["cpu_baseline"] = r["cpu_baseline"]
    return line


def nested(line: dict) -> dict:
    """A config's result as a nested field of the headline line."""
    keep = ("metric", "value", "unit", "ms_per_step", "dtype", "config", "roofline", "cpu_baseline")
    return {k: line[k] for k in keep if k in line}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="1",
                    help="1 (default: config 1 with every other config nested), headline (config 1 "
                         "alone), 0, 2, 3, 4, layer, or copy")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-slot", action="store_true", help="skip the table-slot (PCIe) timing")
    ap.add_argument("--data-workers", type=int, default=None,
                    help="processes that build config 3's experts (default: up to 16; 1 under a "
                         "profiler, whose worker processes have failed to exit)")
    ap.add_argument("--moe-batch", type=int, default=1, help="tokens per step for --config 3")
    ap.add_argument("--split", action="store_true",
                    help="stand-alone x-prep launch + GEMV on prepared digits")
    ap.add_argument("--copy-mib", type=int, default=512, help="size of --config copy")
    ap.add_argument("--profile", action="store_true",
                    help="eager launches only, no timing (for rocprofv3 counter passes)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the hot path runs "
              "on one GPU; across GPUs it would shard weight rows with no exchange)", file=sys.stderr)
        sys.exit(2)
    import torch
    from qstream_amd import qsf_hip
    qsf_hip.init(0)
    if args.config == "copy":
        print(json.dumps(copy_calibration(torch, args.steps, args.warmup, args.copy_mib)), flush=True)
        return
    if args.profile:
        if args.config == "layer":
            profile_decode_layer(torch, qsf_hip, args.steps, args.warmup)
            return
        cfg = int(args.config)
        if cfg == 2:
            profile_layers(torch, qsf_hip, args.steps, args.warmup)
        elif cfg == 3:
            profile_moe(torch, qsf_hip, args.steps, args.warmup, args.moe_batch)
        elif cfg == 4:
            profile_prefill(torch, qsf_hip, args.steps, args.warmup)
        else:
            run_profile(torch, qsf_hip, cfg, args.steps, args.warmup)
        return
    cache: dict = {}
    if args.config in ("1", "all"):
        # the headline (config 1) with every other config nested under "configs"
        t0 = time.perf_counter()
        line = run_config(torch, qsf_hip, "1", args, 10.0, cache)
        line["configs"] = {}
        for k in ("0", "2", "3b1", "3b8", "4", "layer"):
            line["configs"][k.replace("3b", "3_b")] = nested(run_config(torch, qsf_hip, k, args, 4.0, cache))
            log(f"config {k} done, {time.perf_counter() - t0:.0f} s in all")
        line["bench_wall_s"] = round(time.perf_counter() - t0, 1)
    elif args.config == "headline":
        line = run_config(torch, qsf_hip, "1", args, 10.0, cache)
    else:
        line = run_config(torch, qsf_hip, args.config, args, 10.0, cache)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
