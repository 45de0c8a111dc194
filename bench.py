"""Benchmark of the routed-expert decode path on one MI355X.

Default workload: Qwen3.6-35B-A3B-shape MoE
decode, one token through 40 layers' expert blocks, all resident in HBM:
hidden 2048, 256 routed experts (top-8, softmax renormalised), expert
intermediate 512, one always-on 4-bit shared expert with a sigmoid gate,
affine 4-bit g64 weights (codes uniform, scales bf16 |N(0,.02)|, biases
bf16 N(0,.01)), f32 router N(0,.02), residual stream N(0,1). Between
layers the next input is RMSNorm(residual) (unit bf16 weights). One step
= one token through the 40 layers: three kernels per layer (router +
shared gate/up; top-k + routed gate/up; down + combine) replayed from a
HIP graph (default) or one kernel per phase (--path kernels).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2]

--config c0/c3 run the other decode shapes, c1 the LM head, c4 the
512-token prefill layer and c5 the hidden-4096 decode shape (not a
BASELINE config), each with its own JSON line.

Prints one JSON line. value = µs per layer (lower is better); the
roofline object gives achieved HBM GB/s from the algorithmic bytes.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0

# The decode arithmetic: 4-/3-bit codes times x as 24-bit block floating
# point (one exponent per 32 inputs, three int8 limbs, exact int32 sums
# with v_dot4c_i32_i8), then the bf16 scale and bias and everything after
# (SwiGLU, the down matvec, the combine) in f32.
DECODE_DTYPE = "u4/u3 codes x 24-bit block-FP activations (int8 limbs, sdot4 int32 sums), f32 epilogue"

# Algorithmic bytes per unit (weights read once).
CONFIGS = {
    "c0": dict(name="OLMoE-1B-7B-shape MoE layer decode (1 token)", H=2048, I=1024, E=64, k=8, bits=4,
               normalize=False, shared=False, layers=16),
    "c2": dict(name="Qwen3.6-35B-A3B-shape MoE decode, 40 layers (1 token)", H=2048, I=512, E=256, k=8, bits=4,
               normalize=True, shared=True, layers=40),
    "c3": dict(name="Qwen3.6-35B-A3B-shape MoE decode, packed 3-bit routed, 40 layers (1 token)", H=2048, I=512,
               E=256, k=8, bits=3, normalize=True, shared=True, layers=40),
    "c1": dict(name="Qwen3-shape LM head: dense 4-bit qmv 151936x2048 + greedy argmax (1 token)", V=151936,
               H=2048, bits=4),
    "c4": dict(name="Qwen3.6-A3B-shape MoE layer prefill, 512 tokens (bf16 x, Zipf 1.1 routing)", H=2048, I=512,
               E=256, k=8, bits=4, tokens=512),
    # Not a BASELINE config: the reference's largest supported model shape
    # (Qwen3.5-397B-A17B), 16 of its 60 layers resident (58 GB).
    "c5": dict(name="Qwen3.5-397B-A17B-shape MoE decode, 16 layers (1 token)", H=4096, I=1024, E=512, k=10,
               bits=4, normalize=True, shared=True, layers=16),
}


# HBM bytes actually moved per unit of work, from rocprofv3 FETCH_SIZE and
# WRITE_SIZE passes scaled by a 256 MiB copy calibration (FETCH x 2.0,
# WRITE x 1.0): profiles/decode_c{0,2,3,5}_*.md (one layer = the three k_fa_*
# launches), profiles/lm_head_c1_qmv_argmax.md (k_qmv + argmax) and
# profiles/prefill_c4_a3b_4bit.md (the four prefill launches of one layer).
# None where no counter pass was taken (multi-token decode, per-phase path).
MEASURED_TRAFFIC = {"c0": 29_732_534, "c2": 18_897_532, "c3": 15_786_871, "c1": 175_922_937,
                    "c4": 558_463_070, "c5": 87_783_971}


def stream_read_peak(dev, gib=4):
    """Measured streaming-read bandwidth of this GPU: libsmoe's read kernel
    (128-bit non-temporal loads over the whole chip) over a `gib` GiB
    buffer, best of 5, GB/s."""
    import torch

    import streamoe_amd as sa

    kern = sa.Kernels(dev.index or 0)
    n = gib * (1 << 30)
    buf = torch.ones(n // 4, dtype=torch.float32, device=dev)
    sink = torch.empty(2048, dtype=torch.int32, device=dev)
    sa.check(kern.stream_read(buf, n, sink), "smoe_stream_read")
    torch.cuda.synchronize()
    best = 0.0
    for _ in range(5):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        sa.check(kern.stream_read(buf, n, sink), "smoe_stream_read")
        e1.record()
        torch.cuda.synchronize()
        best = max(best, n / (e0.elapsed_time(e1) * 1e-3) / 1e9)
    kern.close()
    del buf
    torch.cuda.empty_cache()
    return round(best, 1)


def layer_bytes(c, tokens=1, router_bits=32):
    """Algorithmic bytes of one layer for `tokens` tokens decoded together:
    the router and the shared expert once, each token's k routed experts
    (counted as distinct). An 8-bit router: its codes plus bf16 scales and
    biases per 64 inputs."""
    import streamoe_amd as sa

    routed = sa.ExpertLayout(c["H"], c["I"], c["bits"], 64).expert_size
    shared = sa.ExpertLayout(c["H"], c["I"], 4, 64).expert_size if c["shared"] else 0
    router = c["E"] * c["H"] * 4 if router_bits == 32 else c["E"] * c["H"] + c["E"] * (c["H"] // 64) * 4
    return tokens * c["k"] * routed + shared + router


def q8_rows(rows, hidden, seed):
    """A seeded 8-bit affine matrix [rows, hidden], group 64, with router-like
    weights (codes uniform, scales |N(0, 2e-4)|, biases N(0, 0.02), both bf16
    rounded): host (codes, scales, biases, 64) and its device QuantWeights
    ([codes | scales | biases], 256-byte aligned regions)."""
    import numpy as np
    import torch

    import streamoe_amd as sa

    rng = np.random.default_rng(seed)
    g = hidden // 64
    q = rng.integers(0, 256, (rows, hidden), dtype=np.uint8)

    def bf16(x):
        b = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
        return ((b + (((b >> 16) & 1) + 0x7FFF)) >> 16).astype(np.uint16)
    s = bf16(np.abs(rng.standard_normal((rows, g))) * 2e-4)
    b = bf16(rng.standard_normal((rows, g)) * 0.02)
    pad = lambda n: (n + 255) // 256 * 256  # noqa: E731
    so, bo = pad(q.size), pad(q.size) + pad(s.nbytes)
    buf = np.zeros(bo + pad(b.nbytes), np.uint8)
    buf[:q.size] = q.ravel()
    buf[so:so + s.nbytes] = s.ravel().view(np.uint8)
    buf[bo:bo + b.nbytes] = b.ravel().view(np.uint8)
    dev = torch.from_numpy(buf).cuda()
    return (q, s, b, 64), sa.QuantWeights(dev, 0, so, bo, 64, 8)


def router_logits(oracle, r, x):
    """Oracle router logits for an f32 router tensor or an 8-bit host tuple."""
    if isinstance(r, tuple):
        rc, y = oracle.dequant_matvec_8bit_gs(r[0], r[1], r[2], x.size, r[0].shape[0], r[3], x)
        assert rc == 0
        return y
    return oracle.f32_matvec(r.cpu().numpy(), x)


# LM head (config 1): decode tokens per timed graph replay.
LM_TOKENS = 20


# A GPU box grants one GPU's process a share of 16 host CPUs (the harness's
# worker-pool rule), whatever nproc reports; the baseline uses every CPU of
# that share that the process may run on.
BOX_CPU_SHARE = 16


def cpu_threads():
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    return max(1, min(n, BOX_CPU_SHARE))


def host_cpu():
    """What the CPU baseline ran on: CPU model, nproc, the CPUs this
    process may use, and the threads the baseline used."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        aff = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        aff = None
    return {"cpu_model": model, "nproc": os.cpu_count(), "affinity_cpus": aff, "threads_used": cpu_threads(),
            "box_cpu_share": BOX_CPU_SHARE}


def cpu_baseline_decode(c, arena_l0, router_l0, shared_l0, gate_l0, x, seconds):
    """The oracle (C restatement of the reference CPU path) on one resident
    layer, repeated for about `seconds`; µs per layer."""
    import numpy as np

    import oracle

    import streamoe_amd as sa

    lay = sa.ExpertLayout(c["H"], c["I"], c["bits"], 64)
    th = cpu_threads()
    h_mid = np.zeros(c["H"], np.float32)
    q8 = isinstance(router_l0, tuple)
    args = (arena_l0, lay.expert_size, c["H"], c["I"], c["E"], c["k"], 64, c["bits"], c["normalize"],
            None if q8 else router_l0)
    kw = dict(router_q8=router_l0 if q8 else None, gate_q8=gate_l0 if isinstance(gate_l0, tuple) else None)
    gate_w = None if isinstance(gate_l0, tuple) else gate_l0
    oracle.moe_decode_layer(*args, x, h_mid, shared_l0, gate_w, th, **kw)  # warm-up
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 5:
        t0 = time.perf_counter()
        oracle.moe_decode_layer(*args, x, h_mid, shared_l0, gate_w, th, **kw)
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return dict(value=med * 1e6, unit="us/layer", cores=th, kind="port",
                sample=f"{len(times)} runs of one {c['name'].split(',')[0]} layer (median), "
                       f"oracle/oracle.c with rows (router, gate/up, down) in parallel on {th} threads",
                host=host_cpu())


def decode_parity(kern, c, layers, arenas, routers, shareds, gates, norms, x0):
    """The timed computation checked against the oracle after the timing:
    one fresh token through all the layers (smoe_moe_decode_layers, the
    step the graph replays) against the oracle chain (router, the chosen
    experts' FFNs, combine, RMSNorm between layers; only the chosen experts'
    blobs are copied to the host), and layer 0 alone with the routing
    returned (idx in the reference's slot order, weights bit for bit)."""
    import numpy as np
    import torch

    import oracle

    H, I, k, bits = c["H"], c["I"], c["k"], c["bits"]
    stride = arenas[0].numel() // c["E"]
    resid = x0.clone()
    work = torch.empty_like(x0)
    sa_check = __import__("streamoe_amd").check
    sa_check(kern.moe_decode_layers(layers, norms, 1e-6, x0, resid, work), "smoe_moe_decode_layers")
    torch.cuda.synchronize()
    got = resid.cpu().numpy()
    r = x0.cpu().numpy().copy()
    x = r.copy()
    min_gap = 1.0
    for l in range(len(layers)):
        if l > 0:
            x = oracle.rms_norm_bf16(r, norms[l].cpu().numpy().view(np.uint16), 1e-6)
        logits = router_logits(oracle, routers[l], x)
        p = np.sort(oracle.softmax(logits))[::-1]
        min_gap = min(min_gap, float(p[k - 1] - p[k]))
        _, idx, w = oracle.router(logits, k, c["normalize"])
        outs = np.stack([oracle.expert_swiglu(arenas[l][int(e) * stride:(int(e) + 1) * stride].cpu().numpy(), bits,
                                              H, I, 64, x) for e in idx])
        sh = score = None
        if shareds[l] is not None:
            sh = oracle.expert_swiglu(shareds[l].cpu().numpy(), 4, H, I, 64, x)
            score = float(router_logits(oracle, gates[l] if isinstance(gates[l], tuple) else gates[l][None, :], x)[0])
        r = oracle.combine(outs, w, r, sh, float("nan") if score is None else score)
    chain_err = float(np.max(np.abs(got - r)) / np.max(np.abs(r)))
    # Layer 0 with idx / weights returned.
    zeros = torch.zeros(H, dtype=torch.float32, device=x0.device)
    out0 = torch.empty(H, dtype=torch.float32, device=x0.device)
    idx0 = torch.empty(k, dtype=torch.int32, device=x0.device)
    w0 = torch.empty(k, dtype=torch.float32, device=x0.device)
    sa_check(kern.moe_decode_layer(layers[0], x0, zeros, out0, idx0, w0), "smoe_moe_decode_layer")
    torch.cuda.synchronize()
    r8, g8 = isinstance(routers[0], tuple), isinstance(gates[0], tuple)
    want0, widx, ww, _ = oracle.moe_decode_layer(
        arenas[0].cpu().numpy(), stride, H, I, c["E"], k, 64, bits, c["normalize"],
        None if r8 else routers[0].cpu().numpy(), x0.cpu().numpy(), np.zeros(H, np.float32),
        None if shareds[0] is None else shareds[0].cpu().numpy(),
        None if gates[0] is None or g8 else gates[0].cpu().numpy(), router_q8=routers[0] if r8 else None,
        gate_q8=gates[0] if g8 else None)
    g0 = out0.cpu().numpy()
    return {"chain_rel_err": chain_err, "chain_layers": len(layers), "min_topk_prob_gap": min_gap,
            "layer0_rel_err": float(np.max(np.abs(g0 - want0)) / np.max(np.abs(want0))),
            "layer0_idx_equal": bool(np.array_equal(idx0.cpu().numpy(), widx)),
            # The logits come from the device's router matvec (another
            # summation order than the oracle's), so the weights agree to a
            # few ulps; with equal logits they are bit-identical
            # (tests/test_gpu_softmax.py).
            "layer0_weights_max_rel_diff": float(np.max(np.abs(w0.cpu().numpy() - ww) / np.abs(ww))),
            "tolerance": 1e-3}


def _sync_status(kern):
    import streamoe_amd as sa

    return sa._lib.smoe_sync(kern.h)


FA_TRACE_BLOCKS = 4096  # kFaTraceBlocks in streamoe_amd/csrc/kernels.h (8 points per block)


def trace_fused(kern, step, nl):
    """Per-block timestamps of the three-kernel decode from one graph replay,
    summarised over layers 1..nl-1 in microseconds. Points per block: 0
    start, 1 routing input landed (gate/up: logits; down: expert pointers),
    2 top-k set known, 3 weights landed, 4 arithmetic done, 5 stores
    acknowledged. Reported per kernel: span (first start to last
    acknowledged store), spread of block starts, mean durations between
    points, and the idle gap to the next kernel's first block."""
    import numpy as np
    import torch

    import streamoe_amd as sa
    from streamoe_amd import _abi

    P = 8
    per_layer = 3 * FA_TRACE_BLOCKS * P
    buf = torch.zeros(nl * per_layer, dtype=torch.int64, device="cuda")
    kern.set_option(_abi.SMOE_OPT_TRACE_BUFFER, buf.data_ptr())
    try:
        g = sa.capture_graph(kern, step)
        buf.zero_()
        g.replay()
        torch.cuda.synchronize()
    finally:
        kern.set_option(_abi.SMOE_OPT_TRACE_BUFFER, 0)
    t = buf.cpu().numpy().reshape(nl, 3, FA_TRACE_BLOCKS, P).astype(np.float64) * 0.01
    seg = {"route": [(0, 3, "to_weights"), (3, 4, "arith"), (4, 5, "store_ack")],
           "gateup": [(0, 1, "to_logits"), (1, 2, "topk"), (2, 3, "to_weights"), (3, 4, "arith"),
                      (4, 5, "store_ack")],
           "down": [(0, 1, "to_pointers"), (1, 3, "to_weights"), (3, 4, "arith"), (4, 5, "combine_store")]}
    out = {}
    for q, name in enumerate(["route", "gateup", "down"]):
        acc = {}
        for l in range(1, nl):
            b = t[l, q]
            b = b[b[:, 0] > 0]
            if not len(b):
                continue
            vals = {"span": b[:, 5].max() - b[:, 0].min(), "start_spread": b[:, 0].max() - b[:, 0].min()}
            for i, j, lab in seg[name]:
                ok = (b[:, i] > 0) & (b[:, j] > 0)
                if ok.any():
                    vals[lab] = (b[ok, j] - b[ok, i]).mean()
            nxt = t[l, q + 1] if q < 2 else (t[l + 1, 0] if l + 1 < nl else None)
            if nxt is not None:
                nb = nxt[nxt[:, 0] > 0]
                vals["gap_to_next"] = nb[:, 0].min() - b[:, 5].max()
            for kk, v in vals.items():
                acc.setdefault(kk, []).append(v)
        out[name] = {kk: round(float(np.mean(v)), 3) for kk, v in acc.items()}
    return out


def run_decode(args, c):
    import numpy as np
    import torch

    import streamoe_amd as sa

    dev = torch.device("cuda", 0)
    kern = sa.Kernels(0)
    H, I, E, k, nl = c["H"], c["I"], c["E"], c["k"], c["layers"]
    lay = sa.ExpertLayout(H, I, c["bits"], 64)
    slay = sa.ExpertLayout(H, I, 4, 64)
    stride = lay.expert_size
    arenas, routers, shareds, gates, norms, layers = [], [], [], [], [], []
    for l in range(nl):
        a = torch.empty(E * stride, dtype=torch.uint8, device=dev)
        sa.check(kern.synth_experts(a, E, stride, lay, 1000 + l), "synth")
        rq = gq = None  # 8-bit router / gate (device QuantWeights)
        if args.router_bits == 8:
            r, rq = q8_rows(E, H, 2000 + l)
        else:
            r = torch.empty((E, H), dtype=torch.float32, device=dev)
            sa.check(kern.synth_normal_f32(r, 2000 + l, 0.02), "synth")
        s = g = None
        if c["shared"]:
            s = torch.empty(slay.expert_size, dtype=torch.uint8, device=dev)
            sa.check(kern.synth_experts(s, 1, slay.expert_size, slay, 3000 + l), "synth")
            if args.router_bits == 8:
                g, gq = q8_rows(1, H, 4000 + l)
            else:
                g = torch.empty(H, dtype=torch.float32, device=dev)
                sa.check(kern.synth_normal_f32(g, 4000 + l, 0.02), "synth")
        nw = torch.full((H,), 0x3F80, dtype=torch.int16, device=dev)  # bf16 1.0
        arenas.append(a)
        routers.append(r)
        shareds.append(s)
        gates.append(g)
        norms.append(nw)
        if rq is not None:
            layers.append(kern.layer(lay, a, stride, E, k, c["normalize"], None, s, None, router_q=rq,
                                     shared_gate_q=gq))
            layers[-1]._keep_dev = (rq, gq)
        else:
            layers.append(kern.layer(lay, a, stride, E, k, c["normalize"], r, s, g))
    T = args.tokens
    x0 = torch.empty((T, H) if T > 1 else (H,), dtype=torch.float32, device=dev)
    sa.check(kern.synth_normal_f32(x0, 5000, 1.0), "synth")
    resid = x0.clone()
    work = torch.empty_like(x0)
    torch.cuda.synchronize()

    path = {"auto": 0, "kernels": 1, "fused": 3}[args.path]
    kern.set_decode_path(path)

    def step():
        if T > 1:
            sa.check(kern.moe_decode_tokens(layers, norms, 1e-6, T, x0, resid, work), "smoe_moe_decode_tokens")
        else:
            sa.check(kern.moe_decode_layers(layers, norms, 1e-6, x0, resid, work), "smoe_moe_decode_layers")

    stream = torch.cuda.current_stream(dev)
    graph = None
    if not args.eager:
        graph = sa.capture_graph(kern, step)

    run = graph.replay if graph is not None else step
    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        run()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1)
    ms_per_step = ms / args.steps
    us_layer = ms_per_step * 1e3 / nl
    sa.check(_sync_status(kern), "smoe_sync")
    assert torch.isfinite(resid).all(), "residual stream is not finite"
    phases = None
    if args.trace and T == 1:
        phases = trace_fused(kern, step, nl) if path in (0, 3) else None

    nbytes = layer_bytes(c, T, args.router_bits)
    achieved = nbytes / (us_layer * 1e-6) / 1e9
    out = {
        "metric": "4-bit MoE expert decode µs/layer + achieved HBM GB/s (% of peak), 1 GPU",
        "value": round(us_layer, 4),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DECODE_DTYPE,
        "data": "synthetic (seeded, generated on the device)",
        "seeds": {"experts": "1000 + layer", "router": "2000 + layer", "shared_expert": "3000 + layer",
                  "shared_gate": "4000 + layer", "x": 5000},
        "config": {"workload": c["name"], "hidden": H, "experts": E, "top_k": k, "inter": I, "bits": c["bits"],
                   "group": 64, "layers": nl, "shared_expert": c["shared"], "tokens": T,
                   "router": "f32" if args.router_bits == 32 else "8-bit affine, group 64",
                   "mode": "hipgraph" if graph is not None else "eager"},
        "gbps": round(achieved, 1),
        "pct_of_hbm_peak": round(100 * achieved / HBM_PEAK_GBS, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": MEASURED_TRAFFIC.get(c.get("key")) if path in (0, 3) and T == 1 and args.router_bits == 32 else None,
                     "unit_of_work": f"one layer, {T} token(s): {nbytes} algorithmic bytes",
                     "kernel": "decode layer: k_fa_route + k_fa_gateup + k_fa_down (one HIP graph)"
                               if path in (0, 3) else "decode layer (all launches)"},
        "wall_s": round(wall, 3),
    }
    if T > 1:
        out["us_per_layer_per_token"] = round(us_layer / T, 4)
        out["roofline"]["traffic"] = None
    if phases:
        out["phases_us"] = phases
    if T == 1 and not args.no_parity:
        out["parity"] = decode_parity(kern, c, layers, arenas, routers, shareds, gates, norms, x0)
    if not args.no_cpu and T == 1:
        a0 = arenas[0].cpu().numpy()
        r0 = routers[0] if isinstance(routers[0], tuple) else routers[0].cpu().numpy()
        s0 = None if shareds[0] is None else shareds[0].cpu().numpy()
        g0 = gates[0] if gates[0] is None or isinstance(gates[0], tuple) else gates[0].cpu().numpy()
        out["cpu_baseline"] = cpu_baseline_decode(c, a0, r0, s0, g0, x0.cpu().numpy(), args.cpu_seconds)
        out["cpu_baseline"]["gpu_speedup"] = round(out["cpu_baseline"]["value"] / us_layer, 1)
    kern.close()
    return out


def run_lm_head(args, c):
    """Config 1: y = W x (4-bit g64, 151936 x 2048) and argmax(y) per step
    (smoe_qmv_argmax), replayed from a HIP graph."""
    import numpy as np
    import torch

    import oracle
    import streamoe_amd as sa

    dev = torch.device("cuda", 0)
    kern = sa.Kernels(0)
    V, H, G = c["V"], c["H"], 64
    codes_b = V * H // 2
    sc_b = V * (H // G) * 2
    buf = torch.empty(codes_b + 2 * sc_b, dtype=torch.uint8, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(0xC1)
    buf[:codes_b].view(torch.int32).copy_(torch.randint(-2**31, 2**31 - 1, (codes_b // 4,), dtype=torch.int32,
                                                        device=dev, generator=g))
    scales = buf[codes_b:codes_b + sc_b].view(torch.int16)
    biases = buf[codes_b + sc_b:].view(torch.int16)
    sa.check(kern.synth_normal_bf16(scales, 0xC11, 0.02), "synth")
    scales.bitwise_and_(0x7FFF)  # |N(0, 0.02)|
    sa.check(kern.synth_normal_bf16(biases, 0xC12, 0.01), "synth")
    # One step = the LM head of LM_TOKENS decode tokens, each with its own
    # x, in one HIP graph (as in a decode loop, where the LM head sits in the
    # token's graph with the layers); value = µs per token. One graph per
    # token is timed too: it adds the graph launch (~7 µs) to every token.
    T = LM_TOKENS
    xs = torch.empty((T, H), dtype=torch.float32, device=dev)
    sa.check(kern.synth_normal_f32(xs, 0xC13, 1.0), "synth")
    ys = torch.empty((T, V), dtype=torch.float32, device=dev)
    ams = torch.empty(T, dtype=torch.int32, device=dev)
    x, y, am = xs[0], ys[0], ams[0:1]
    w = sa.QuantWeights(buf, 0, codes_b, codes_b + sc_b, G, 4)

    def step():
        for t in range(T):
            sa.check(kern.qmv_argmax(w, xs[t], ys[t], V, H, ams[t:t + 1]), "smoe_qmv_argmax")

    def step1():
        sa.check(kern.qmv_argmax(w, x, y, V, H, am), "smoe_qmv_argmax")

    stream = torch.cuda.current_stream(dev)

    def time_steps(fn, steps):
        graph = None if args.eager else sa.capture_graph(kern, fn)
        run = graph.replay if graph is not None else fn
        for _ in range(args.warmup):
            run()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            run()
        e1.record(stream)
        torch.cuda.synchronize()
        sa.check(_sync_status(kern), "smoe_sync")
        return e0.elapsed_time(e1) * 1e3 / steps, graph

    us_step, graph = time_steps(step, args.steps)
    us = us_step / T
    us_one, _ = time_steps(step1, args.steps * T)
    nbytes = codes_b + 2 * sc_b
    achieved = nbytes / (us * 1e-6) / 1e9
    out = {
        "metric": "4-bit MoE expert decode µs/layer + achieved HBM GB/s (% of peak), 1 GPU",
        "value": round(us, 3), "unit": "us/token (LM head qmv + argmax)", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(us_step / 1e3, 5), "higher_is_better": False, "scaling": "weak",
        "tokens_per_step": T, "us_per_token_one_graph_each": round(us_one, 3),
        "vs_baseline": None, "dtype": DECODE_DTYPE, "data": "synthetic (seeded, generated on the device)",
        "seeds": {"codes": "torch.Generator 0xC1", "scales": 0xC11, "biases": 0xC12, "x": 0xC13},
        "config": {"workload": c["name"], "vocab": V, "hidden": H, "bits": 4, "group": G, "tokens_per_graph": T,
                   "mode": "hipgraph" if graph is not None else "eager"},
        "gbps": round(achieved, 1), "pct_of_hbm_peak": round(100 * achieved / HBM_PEAK_GBS, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": MEASURED_TRAFFIC.get("c1"),
                     "unit_of_work": f"one token: {nbytes} algorithmic bytes (codes + bf16 scales/biases)",
                     "kernel": "k_qmv (with per-wave argmax partials) + k_argmax_final (smoe_qmv_argmax)"},
    }
    if not args.no_cpu:
        wh = buf.cpu().numpy()
        xh = x.cpu().numpy()
        packed = wh[:codes_b]
        sh = wh[codes_b:codes_b + sc_b].view(np.uint16)
        bh = wh[codes_b + sc_b:].view(np.uint16)
        t0 = time.perf_counter()
        want = oracle.lm_head(packed, sh, bh, H, V, G, xh)
        dt = time.perf_counter() - t0
        got = y.cpu().numpy()
        out["cpu_baseline"] = {"value": round(dt * 1e6, 1), "unit": "us/token", "cores": 1, "kind": "port",
                               "sample": "one full LM head matvec, oracle/oracle.c lm_head (single thread, as "
                                         "io/lm_head.rs:66-122)", "host": host_cpu(),
                               "gpu_speedup": round(dt * 1e6 / us, 1)}
        out["parity"] = {"rel_err": float(np.max(np.abs(got - want)) / np.max(np.abs(want))),
                         "argmax_gpu": int(am.cpu()[0]), "argmax_cpu": int(oracle.argmax(want))}
    kern.close()
    return out


def run_prefill(args, c):
    """Config 4: one MoE layer's routed experts over 512 tokens (bucket by
    expert, grouped gate/up GEMM, SwiGLU, down GEMM, weighted combine),
    replayed from a HIP graph. value = µs per layer."""
    import numpy as np
    import torch

    import oracle
    import streamoe_amd as sa

    dev = torch.device("cuda", 0)
    kern = sa.Kernels(0)
    H, I, E, k, n, bits = c["H"], c["I"], c["E"], c["k"], c["tokens"], c["bits"]
    lay = sa.ExpertLayout(H, I, bits, 64)
    stride = lay.expert_size
    arena = torch.empty(E * stride, dtype=torch.uint8, device=dev)
    sa.check(kern.synth_experts(arena, E, stride, lay, 0xC4), "synth")
    idx, w = sa.zipf_routing(n, E, k, 1.1, seed=0xC4)
    idx_d, w_d = torch.from_numpy(idx).to(dev), torch.from_numpy(w).to(dev)
    x = torch.empty((n, H), dtype=torch.int16, device=dev)
    sa.check(kern.synth_normal_bf16(x, 0xC41, 1.0), "synth")
    out = torch.empty((n, H), dtype=torch.float32, device=dev)
    ws = torch.empty(kern.moe_prefill_workspace_size(lay, n, E, k), dtype=torch.uint8, device=dev)
    # The whole MoE block variant: plus a 4-bit shared expert with its f32
    # gate (config 2's distributions) and the residual h_mid.
    slay = sa.ExpertLayout(H, I, 4, 64)
    shared = torch.empty(slay.expert_size, dtype=torch.uint8, device=dev)
    sa.check(kern.synth_experts(shared, 1, slay.expert_size, slay, 0xC45), "synth")
    gate = torch.empty(H, dtype=torch.float32, device=dev)
    sa.check(kern.synth_normal_f32(gate, 0xC46, 0.02), "synth")
    h_mid = torch.empty((n, H), dtype=torch.float32, device=dev)
    sa.check(kern.synth_normal_f32(h_mid, 0xC47, 1.0), "synth")
    hidden = torch.empty((n, H), dtype=torch.float32, device=dev)
    wsb = torch.empty(kern.moe_prefill_block_workspace_size(lay, n, E, k, True), dtype=torch.uint8, device=dev)

    def step():
        sa.check(kern.moe_prefill(lay, arena, stride, E, idx_d, w_d, x, True, n, k, out, ws), "smoe_moe_prefill")

    def step_block():
        sa.check(kern.moe_prefill_block(lay, arena, stride, E, idx_d, w_d, x, True, n, k, shared, gate, h_mid,
                                        hidden, wsb), "smoe_moe_prefill_block")

    stream = torch.cuda.current_stream(dev)

    def time_steps(fn):
        graph = None if args.eager else sa.capture_graph(kern, fn)
        run = graph.replay if graph is not None else fn
        for _ in range(args.warmup):
            run()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(args.steps):
            run()
        e1.record(stream)
        torch.cuda.synchronize()
        sa.check(_sync_status(kern), "smoe_sync")
        return e0.elapsed_time(e1) * 1e3 / args.steps, graph

    # The other tile choices on the same inputs (their own graphs), for
    # comparison; timed first, so that the reported value does not carry
    # the clock ramp of the first timed loop.
    main_opt = 1 if args.prefill_gemm == "16x16" else 0
    us_other = {}
    for opt, label in ((0, "32x32"), (1, "16x16"), (2, "32x32 gate/up, 16x16 down")):
        if opt != main_opt and not args.main_only:
            kern.set_prefill_gemm(opt)
            us_other[label] = round(time_steps(step)[0], 2)
    kern.set_prefill_gemm(main_opt)
    us, graph = time_steps(step)
    us_blk = None if args.main_only else time_steps(step_block)[0]
    hit = np.unique(idx)
    nbytes = len(hit) * stride + n * H * 2 + n * H * 4  # weights of hit experts + bf16 X + f32 Y
    flops = 2 * n * k * (2 * H * I + I * H)
    achieved = nbytes / (us * 1e-6) / 1e9
    tflops = flops / (us * 1e-6) / 1e12
    out_d = {
        "metric": "4-bit MoE expert decode µs/layer + achieved HBM GB/s (% of peak), 1 GPU",
        "value": round(us, 2), "unit": "us/layer (512-token prefill)", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(us / 1e3, 5), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4/u3 codes exact in bf16 (gate/up) and fp16 (down) MFMA, f32 accumulate, fp16 activations",
        "data": "synthetic (seeded, generated on the device)",
        "seeds": {"experts": 0xC4, "routing": "zipf s=1.1, seed 0xC4", "x": 0xC41},
        "config": {"workload": c["name"], "tokens": n, "hidden": H, "experts": E, "top_k": k, "inter": I,
                   "bits": bits, "group": 64, "experts_hit": int(len(hit)),
                   "mode": "hipgraph" if graph is not None else "eager"},
        "gbps": round(achieved, 1), "pct_of_hbm_peak": round(100 * achieved / HBM_PEAK_GBS, 2),
        "mfma_tflops": round(tflops, 2), "pct_of_bf16_mfma_peak": round(100 * tflops / 2500.0, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": MEASURED_TRAFFIC.get("c4"),
                     "unit_of_work": f"one layer: {nbytes} algorithmic bytes ({len(hit)} hit experts x {stride} "
                                     f"+ X + Y), {flops} flops",
                     "kernel": ("prefill layer: k_pf_route (+ per-token x preparation) + k_pf_gu64<false> (gate/up on "
                                "32x32 tiles, 16x16 for units of <= 16 rows, with the activation group sums) + "
                                "k_pf_gu64<true> (down, the same tiles) + k_pf_combine (one HIP graph)")
                               if args.prefill_gemm == "auto" else
                               ("prefill layer: k_pf_route (+ per-token x preparation) + k_pf_mm (gate/up on 16x16 "
                                "tiles, with the activation group sums) + k_pf_mm (down) + k_pf_combine (one HIP graph)")},
        "gemm_tiles": "32x32" if args.prefill_gemm == "auto" else "16x16",
        "other_tiles_us_per_layer": us_other,
    }
    blk_bytes = nbytes + slay.expert_size + 2 * n * H * 4  # + shared expert, h_mid read, gate
    blk_flops = flops + 2 * n * (2 * H * I + I * H)
    if args.main_only:
        kern.close()
        return out_d
    out_d["block_variant"] = {
        "what": "smoe_moe_prefill_block: the same routed experts plus a 4-bit shared expert over all tokens (extra "
                "work items of the same grouped GEMMs), its f32 sigmoid gate and the residual "
                "(h_mid + moe_sum) + sigmoid(g) * shared",
        "us_per_layer": round(us_blk, 2), "algorithmic_bytes": blk_bytes, "flops": blk_flops,
        "gbps": round(blk_bytes / (us_blk * 1e-6) / 1e9, 1),
        "frac_of_hbm_peak": round(blk_bytes / (us_blk * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "mfma_tflops": round(blk_flops / (us_blk * 1e-6) / 1e12, 2)}
    if not args.no_cpu:
        # The whole layer (a few seconds of CPU work), timed with all host
        # threads; doubles as a parity check of every token.
        ns = n
        xs = oracle.bf16_to_f32(x[:ns].cpu().numpy().view(np.uint16)).reshape(ns, H)
        ah = arena.cpu().numpy()
        buckets = oracle.build_expert_buckets(idx[:ns], w[:ns], ns, k, E)
        nt = cpu_threads()
        t0 = time.perf_counter()
        want = oracle.moe_permute_fuse(ah, stride, bits, H, I, 64, xs, buckets, ns, nthreads=nt)
        dt = time.perf_counter() - t0
        got = out[:ns].cpu().numpy()
        cpu_us = dt * 1e6
        out_d["cpu_baseline"] = {"value": round(cpu_us, 1), "unit": "us/layer (512 tokens)", "cores": nt,
                                 "kind": "port",
                                 "sample": f"all {ns} tokens through oracle moe_permute_fuse "
                                           f"(moe_cpu.rs:282-339 order), {dt:.2f} s", "host": host_cpu(),
                                 "gpu_speedup": round(cpu_us / us, 1)}
        out_d["parity"] = {"rel_err": float(np.max(np.abs(got - want)) / np.max(np.abs(want))),
                           "tokens_checked": ns, "tolerance": 1e-3}
        # The block: the routed sum above, the shared expert and gate per
        # token, the reference's combine.
        sh_h, g_h, hm = shared.cpu().numpy(), gate.cpu().numpy(), h_mid.cpu().numpy()
        so = np.stack([oracle.expert_swiglu(sh_h, 4, H, I, 64, xs[t], nt) for t in range(n)])
        sg = np.array([oracle.f32_matvec(g_h[None, :], xs[t])[0] for t in range(n)], np.float32)
        want_b = oracle.moe_combine_residual_n_tokens(hm, want, so, sg)
        got_b = hidden.cpu().numpy()
        out_d["block_variant"]["parity"] = {
            "rel_err": float(np.max(np.abs(got_b - want_b)) / np.max(np.abs(want_b))),
            "moe_part_rel_err": float(np.max(np.abs((got_b - hm) - (want_b - hm))) / np.max(np.abs(want_b - hm))),
            "tokens_checked": n, "tolerance": 1e-3}
    kern.close()
    return out_d


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--path", default="auto", choices=["auto", "kernels", "fused"],
                    help="decode path: auto (three-kernel where supported), kernels (one per phase), "
                         "fused (three-kernel only)")
    ap.add_argument("--prefill-gemm", default="auto", choices=["auto", "16x16"],
                    help="c4: the default GEMM tiles (32x32 where they apply) or the 16x16 ones "
                         "(SMOE_OPT_PREFILL_GEMM = 1); the other choices are timed beside it")
    ap.add_argument("--main-only", action="store_true",
                    help="c4: time the default tiles only (no other tiles, no block variant, no CPU leg): for "
                         "profiler runs whose per-kernel figures must come from the reported configuration")
    ap.add_argument("--eager", action="store_true", help="launch every step eagerly instead of replaying a HIP graph")
    ap.add_argument("--trace", action="store_true", help="report per-phase times from in-kernel timestamps")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-parity", action="store_true", help="skip the parity check of the timed work after timing")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-stream-peak", action="store_true", help="skip the measured streaming-read peak")
    ap.add_argument("--router-bits", type=int, default=32, choices=[32, 8],
                    help="decode configs: f32 router and shared gate (BASELINE's configs), or 8-bit affine "
                         "ones (group 64; the reference's A3B mlp.gate.weight / mlp.shared_expert_gate.weight)")
    ap.add_argument("--tokens", type=int, default=1, choices=[1, 2, 3, 4],
                    help="decode configs: tokens decoded together through the layers (value = us per layer "
                         "for all of them)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the multi-GPU "
              "sharding of this path is a design note, not a measured configuration.", file=sys.stderr)
        sys.exit(2)
    c = dict(CONFIGS[args.config], key=args.config)
    runner = {"c1": run_lm_head, "c4": run_prefill}.get(args.config, run_decode)
    out = runner(args, c)
    if not args.no_stream_peak:
        import torch

        peak = stream_read_peak(torch.device("cuda", 0))
        out["hbm_read_peak_measured_gbs"] = peak
        out["frac_of_measured_read_peak"] = round(out["gbps"] / peak, 4)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
