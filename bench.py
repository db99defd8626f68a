#!/usr/bin/env python3
"""MoE FFN forward benchmark on one MI355X (config c5 of the baseline).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Workload (one step = one MoE FFN forward of one synthetic batch, inputs and
weights resident in HBM): T=16384 tokens, hidden H=7168, ffn F=2048, E=64
experts, top-8 routing of N(0,1) logits plus a per-expert N(0, 1.5) skew;
bf16 activations ~ N(0,1), bf16 weights ~ N(0, 0.02).  Stages, all HIP
kernels of this repository on torch's current stream:
  top-k + mask + merge probs -> row-id map -> permuted-row source index ->
  fc1 + SwiGLU (grouped GEMM gathering its A rows from x, i.e. the permute
  fused into fc1) -> fc2 (grouped GEMM) -> merge unpermute.
The stand-alone permute kernel (x -> permuted rows) is timed separately on the
same map, after the timed steps, and reported under "standalone"; the four
grouped GEMMs of the layer's backward (dgrad and wgrad of fc1 and fc2, on the
same routing) and the reference grouped-GEMM cases (forward and backward) at
their own shapes are timed after that and reported under "backward", the
router front end and backward
(router GEMM, its top-k, the reference router cases) under "router" (none of
them is part of `value`).

Prints ONE JSON line: tokens/s of the whole step, per-stage device times
(HIP events on the launch stream, averaged over the timed steps) with their
achieved GB/s or TFLOP/s, the roofline of the dominant kernel (fc1) and the
CPU baseline (the oracle's eager-torch restatement of the same layer, timed on
this host's cores on a bounded token sample).
"""
from __future__ import annotations

import argparse
import importlib
import json
import os
import statistics
import sys
import time
from pathlib import Path

import torch

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 MFMA, TFLOP/s

METRIC = "MoE FFN fwd tokens/s; permute/unpermute GB/s; grouped-GEMM TFLOP/s vs peak"
CFG = dict(tokens=16384, hidden=7168, ffn=2048, experts=64, topk=8, skew=1.5)
SEED = 20261205


def stage_work(T, H, F, E, k):
    """Algorithmic bytes (each input read once, each output written once) or FLOPs per stage."""
    R = T * k
    return {
        # logits fp32 [T,E] in; values/indices [T,k], mask [T,E] u8, probs [T,E] fp32 out
        "topk": ("GB/s", 4 * T * E + 12 * T * k + T * E + 4 * T * E),
        # mask [T,E] u8 in; token-major int64 map [T,E] + offsets + source token per permuted row int32 [R] out
        "row_id_map": ("GB/s", T * E + 8 * T * E + 4 * (E + 1) + 4 * R),
        # x [T,H] bf16 + map [T,E] int64 in; permuted rows [R,H] bf16 out (stand-alone)
        "permute": ("GB/s", 2 * T * H + 8 * T * E + 2 * R * H),
        "fc1_swiglu": ("TFLOP/s", 2 * R * H * (2 * F)),
        "fc2": ("TFLOP/s", 2 * R * F * H),
        # z [R,H] bf16 + map int64 [T,E] + probs fp32 [T,E] in; out [T,H] bf16
        "unpermute_merge": ("GB/s", 2 * R * H + 8 * T * E + 4 * T * E + 2 * T * H),
    }


def cpu_baseline(pkg, x, logits, w1, w2, k, run_s=2.5):
    """Oracle CPU path on the first `n` tokens (full E/H/F weights); tokens/s, median of 3.

    n doubles from 64 until one run takes `run_s` seconds or covers the whole batch, which keeps
    the baseline to roughly 10-30 s of CPU work on any host.
    """
    from oracle import ref_torch

    threads = max(1, min(len(os.sched_getaffinity(0)), int(os.environ.get("OMP_NUM_THREADS", "1024"))))
    torch.set_num_threads(threads)
    w1c, w2c = w1.cpu(), w2.cpu()

    def run(n):
        xc, lc = x[:n].cpu(), logits[:n].cpu()
        t0 = time.perf_counter()
        ref_torch.moe_ffn_forward(xc, lc, w1c, w2c, k)
        return time.perf_counter() - t0

    n = 64
    t = run(n)  # warm-up + probe
    while n < x.shape[0] and t < run_s:
        n = min(2 * n, x.shape[0])
        t = run(n)
    times = [run(n) for _ in range(3)]
    med = statistics.median(times)
    return {"value": round(n / med, 1), "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"first {n} tokens of the c5 batch through oracle/ref_torch.moe_ffn_forward "
                      f"(eager torch on the CPU, full E=64/H=7168/F=2048 bf16 weights), median of 3 runs "
                      f"of {[round(v, 3) for v in times]} s"}


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or the platform's processor string."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


class _PowerClock:
    """Samples socket power (W) and shader clock (MHz) every 40 ms while active (amdsmi's GPU
    metrics table); the middle half of the samples is averaged.  Empty when amdsmi is absent."""

    def __init__(self):
        import threading
        self._threading = threading
        try:
            import amdsmi
            amdsmi.amdsmi_init()
            self._smi, self._h = amdsmi, amdsmi.amdsmi_get_processor_handles()[0]
        except Exception:  # no amdsmi on this host: report nothing
            self._smi = None

    def measure(self, fn, seconds=1.5):
        """Runs fn() back to back for `seconds`; returns (ms per call, power W or None, clock MHz or None)."""
        samples, stop = [], self._threading.Event()

        def loop():
            while not stop.is_set():
                try:
                    m = self._smi.amdsmi_get_gpu_metrics_info(self._h)
                    samples.append((m.get("current_socket_power"), m.get("current_gfxclk")))
                except Exception:
                    pass
                time.sleep(0.04)

        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        th = self._threading.Thread(target=loop) if self._smi is not None else None
        if th:
            th.start()
        times, t0 = [], time.perf_counter()
        while time.perf_counter() - t0 < seconds:
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(5)]
            ev[0].record()
            for i in range(4):
                fn()
                ev[i + 1].record()
            torch.cuda.synchronize()
            times += [ev[i].elapsed_time(ev[i + 1]) for i in range(4)]
        if th:
            stop.set()
            th.join()
        mid = samples[len(samples) // 4: 3 * len(samples) // 4] or samples
        pw = [a for a, _ in mid if isinstance(a, (int, float))]
        ck = [b for _, b in mid if isinstance(b, (int, float))]
        return (statistics.median(times), round(statistics.mean(pw), 1) if pw else None,
                round(statistics.mean(ck), 1) if ck else None)


def ceilings(pkg, dev):
    """Ceilings the roofline fractions are read against, measured on this GPU, plus the power and
    clock the c5 GEMMs (and hipBLASLt on the fc1 shape) run at.  One JSON line."""
    import ctypes

    lib = pkg._lib.probes()
    s = torch.cuda.current_stream().cuda_stream
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    pc = _PowerClock()
    out = {"metric": "ceilings", "device": torch.cuda.get_device_name(0), "cus": cus}

    waves, iters = cus * 8, 80000  # about 20 ms per call
    sink = torch.empty(waves * 64, dtype=torch.float32, device=dev)
    ms, pw, ck = pc.measure(lambda: lib.moe_probe_mfma(waves, iters, sink.data_ptr(), s), seconds=3.0)
    tf = waves * iters * 16 * 16384 / (ms * 1e-3) / 1e12
    out["mfma_bf16_register_loop"] = {"TFLOP/s": round(tf, 1), "frac_of_peak": round(tf / BF16_PEAK_TFLOPS, 4),
                                      "ms": round(ms, 3), "waves": waves, "power_W": pw, "clock_MHz": ck}

    nbytes = 2 << 30
    src = torch.empty(nbytes // 4, dtype=torch.int32, device=dev).fill_(7)
    dst = torch.empty(nbytes // 4, dtype=torch.int32, device=dev)
    nvec, blocks = nbytes // 16, cus * 16
    for mode, name, moved in ((0, "copy", 2 * nbytes), (1, "read_only", nbytes), (2, "write_only", nbytes),
                              (4, "copy_nt", 2 * nbytes), (5, "read_only_nt", nbytes), (6, "write_only_nt", nbytes)):
        ms, pw, ck = pc.measure(lambda: lib.moe_probe_stream(mode, src.data_ptr(), dst.data_ptr(), nvec, blocks, s),
                                seconds=1.0)
        gbs = moved / (ms * 1e-3) / 1e9
        out[name] = {"GB/s": round(gbs, 1), "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4), "ms": round(ms, 3),
                     "bytes": moved, "power_W": pw, "clock_MHz": ck}
    del src, dst

    # The c5 GEMMs of the timed step, and the library GEMM of the fc1 shape, under the same sampler.
    T, H, F, E, k = CFG["tokens"], CFG["hidden"], CFG["ffn"], CFG["experts"], CFG["topk"]
    inp, ops = pkg.inputs, pkg.ops
    x = inp.randn_bf16((T, H), seed=SEED, device=dev)
    logits = inp.router_logits(T, E, skew=CFG["skew"], seed=SEED, device=dev)
    w1 = inp.randn_bf16((E, 2 * F, H), std=0.02, seed=SEED + 10, device=dev)
    w2 = inp.randn_bf16((E, H, F), std=0.02, seed=SEED + 20, device=dev)
    _, _, mask = ops.topk(logits, k, with_mask=True)
    maps = ops.row_id_map(mask, expert_major=False, token_major=False, expert_offsets=True, src_rows=T * k)
    offs, src_tok = maps["expert_offsets"], maps["src_token"]
    h = torch.empty(T * k, F, dtype=torch.bfloat16, device=dev)
    z = torch.empty(T * k, H, dtype=torch.bfloat16, device=dev)
    for name, fn, flops in (
            ("fc1_swiglu", lambda: ops.grouped_gemm_gather(x, src_tok, w1, offs, swiglu=True, out=h), 2 * T * k * H * 2 * F),
            ("fc2", lambda: ops.grouped_gemm(h, w2, offs, out=z), 2 * T * k * F * H)):
        ms, pw, ck = pc.measure(fn, seconds=3.0)
        tf = flops / (ms * 1e-3) / 1e12
        out[name] = {"TFLOP/s": round(tf, 1), "frac_of_peak": round(tf / BF16_PEAK_TFLOPS, 4), "ms": round(ms, 4),
                     "power_W": pw, "clock_MHz": ck}
    del x, w1, w2, h, z
    m = T * k // E
    a = torch.randn(E, m, H, device=dev, dtype=torch.bfloat16)
    b = torch.randn(E, 2 * F, H, device=dev, dtype=torch.bfloat16).transpose(1, 2).contiguous()
    c = torch.empty(E, m, 2 * F, device=dev, dtype=torch.bfloat16)
    ms, pw, ck = pc.measure(lambda: torch.bmm(a, b, out=c), seconds=3.0)
    tf = 2 * E * m * H * 2 * F / (ms * 1e-3) / 1e12
    out["hipblaslt_bmm_fc1_shape"] = {"op": f"torch.bmm bf16 {E} x [{m}, {H}] @ [{H}, {2 * F}]", "TFLOP/s": round(tf, 1),
                                      "frac_of_peak": round(tf / BF16_PEAK_TFLOPS, 4), "ms": round(ms, 4),
                                      "power_W": pw, "clock_MHz": ck}
    return out


def library_reference(m, kdim, n, groups, dev, reps=5):
    """torch.bmm (hipBLASLt) on `groups` equal [m, kdim] @ [kdim, n] bf16 products; ms and TFLOP/s.

    The right operand is materialised K-major ([groups, kdim, n], contiguous), the layout the
    library's fastest kernel for this shape reads.
    """
    a = torch.randn(groups, m, kdim, device=dev, dtype=torch.bfloat16)
    b = torch.randn(groups, n, kdim, device=dev, dtype=torch.bfloat16).transpose(1, 2).contiguous()
    for _ in range(2):
        torch.bmm(a, b)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    ev[0].record()
    for _ in range(reps):
        torch.bmm(a, b)
    ev[1].record()
    torch.cuda.synchronize()
    ms = ev[0].elapsed_time(ev[1]) / reps
    flops = 2 * groups * m * kdim * n
    return {"op": f"torch.bmm bf16 {groups} x [{m}, {kdim}] @ [{kdim}, {n}]", "ms": round(ms, 4),
            "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 2)}


def _time_ms(fn, reps=5, warm=2):
    for _ in range(warm):
        fn()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    ev[0].record()
    for _ in range(reps):
        fn()
    ev[1].record()
    torch.cuda.synchronize()
    return ev[0].elapsed_time(ev[1]) / reps


def backward_gemms(pkg, x, row_map, offs, h, w1, w2, dev, library=False):
    """The grouped GEMMs of the layer's backward on this batch's routing (not part of the timed step).

    dz [R, H] and dy1 [R, 2F] are synthetic N(0,1) gradients; xp = the permuted x.  fc2 dgrad
    dh = dz @ W2[e]; fc2 wgrad dW2[e] = dz^T h; fc1 dgrad dxp = dy1 @ W1[e]; fc1 wgrad dW1[e] = dy1^T xp.
    Also the reference grouped-GEMM cases at their own shapes (uniform groups, T=4096): the backward ones,
    and the forward ones with hipBLASLt's single torch.mm beside the one-group cases.
    """
    ops, inp = pkg.ops, pkg.inputs
    R, H = h.shape[0], x.shape[1]
    F2 = w1.shape[1]
    dz = inp.randn_bf16((R, H), seed=SEED + 30, device=dev)
    dy1 = inp.randn_bf16((R, F2), seed=SEED + 40, device=dev)
    xp, _ = ops.permute(x, row_map, num_out=R, layout=ops.TOKEN_MAJOR, zero_tail=False)
    E = w1.shape[0]
    runs = {
        "fc2_dgrad": (lambda: ops.grouped_gemm_dgrad(dz, w2, offs), 2 * R * H * w2.shape[2]),
        "fc2_wgrad": (lambda: ops.grouped_gemm_wgrad(dz, h, offs), 2 * R * H * h.shape[1]),
        "fc1_dgrad": (lambda: ops.grouped_gemm_dgrad(dy1, w1, offs), 2 * R * F2 * H),
        "fc1_wgrad": (lambda: ops.grouped_gemm_wgrad(dy1, xp, offs), 2 * R * F2 * H),
    }
    out = {}
    for name, (fn, flops) in runs.items():
        ms = _time_ms(fn)
        out[name] = {"ms": round(ms, 4), "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 2),
                     "frac_of_peak": round(flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4), "flops": flops}
    if library:
        m = R // E
        a = torch.randn(E, m, H, device=dev, dtype=torch.bfloat16)
        b = torch.randn(E, H, w2.shape[2], device=dev, dtype=torch.bfloat16)
        out["library_fc2_dgrad_bmm_ms"] = round(_time_ms(lambda: torch.bmm(a, b)), 4)
        del a, b
    del dz, dy1, xp
    cases = {}
    for name, kind in [("case07_moe_grouped_gemm_fc1_dgrad", "dgrad"), ("case08_moe_grouped_gemm_fc2_dgrad", "dgrad"),
                       ("case13_grouped_gemm_single_group_fc1_dgrad", "dgrad"),
                       ("case19_grouped_gemm_single_group_fc2_dgrad", "dgrad"),
                       ("case05_moe_grouped_gemm_fc2_wgrad", "wgrad"), ("case09_moe_grouped_gemm_fc1_wgrad", "wgrad")]:
        case = getattr(pkg.cases, name)
        a, b = case.get_inputs(dev)
        model = case.Model()
        ms = _time_ms(lambda: model(a, b), reps=20, warm=5)  # sub-millisecond calls: more of them
        T, N, K, G = case.TOKENS, case.N, case.K, case.NUM_GROUPS
        flops = 2 * T * N * K
        hbm = 2 * (T * N + (G * N * K if kind == "dgrad" else T * K) + (T * K if kind == "dgrad" else G * N * K))
        cases[name.split("_")[0]] = {"ms": round(ms, 4), "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 2),
                                     "GB/s": round(hbm / (ms * 1e-3) / 1e9, 2), "bytes": hbm}
        del a, b
    # The forward reference cases at their own shapes (GB/s: x, w and out once each; with 40 groups of 102
    # rows every weight element serves 102 rows, so one pass over w bounds case03/04). Beside the one-group
    # cases, hipBLASLt's single torch.mm of the same product (x @ w[0].T), timed in alternation with ours
    # (three pairs, medians: the clock drifts between consecutive measurements).
    for name in ["case03_moe_grouped_gemm_fc1_fwd", "case04_moe_grouped_gemm_fc2_fwd",
                 "case10_grouped_gemm_single_group_fc1_fwd", "case14_grouped_gemm_single_group_fc2_fwd"]:
        case = getattr(pkg.cases, name)
        a, b = case.get_inputs(dev)
        model = case.Model()
        T, N, K, G = case.TOKENS, case.N, case.K, case.NUM_GROUPS
        flops, hbm = 2 * T * N * K, 2 * (T * K + G * N * K + T * N)
        if G == 1:
            bt = b[0].t()
            pairs = [(_time_ms(lambda: model(a, b)), _time_ms(lambda: torch.mm(a, bt))) for _ in range(3)]
            ms = statistics.median(p[0] for p in pairs)
            lib_ms = statistics.median(p[1] for p in pairs)
        else:
            ms = _time_ms(lambda: model(a, b))
        r = {"ms": round(ms, 4), "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 2),
             "frac_of_peak": round(flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
             "GB/s": round(hbm / (ms * 1e-3) / 1e9, 2), "bytes": hbm}
        if G == 1:
            r["library_mm_ms"] = round(lib_ms, 4)
        cases[name.split("_")[0]] = r
        del a, b
    case = pkg.cases.case37_ref_musa_asm_bf16_gemm_nn_256x384
    g, w = case.make_inputs(seed=0, device=dev)
    ms = _time_ms(lambda: case.kernel_function(g, w))
    cases["case37"] = {"ms": round(ms, 4), "TFLOP/s": round(2 * case.M * case.K * case.N / (ms * 1e-3) / 1e12, 2)}
    out["reference_cases"] = cases
    return out


def router_section(pkg, x, dev):
    """The router front end and its backward (not part of the timed step): the c5 router GEMM on this
    batch's x with a random [E, H] gate, alone and with the top-k, and the reference router cases at
    their own shapes (case38 logits, case39/case31 tf32 dgrad/wgrad, case11/case25 casts; 5 warm-up + 20 timed
    calls each, as these take well under a millisecond)."""
    ops, inp = pkg.ops, pkg.inputs
    T, H = x.shape
    E, k = CFG["experts"], CFG["topk"]
    wr = inp.randn_bf16((E, H), std=0.02, seed=SEED + 50, device=dev)
    out = {}
    ms = _time_ms(lambda: ops.router_logits(x, wr))
    out["c5_router_logits"] = {"ms": round(ms, 4), "TFLOP/s": round(2 * T * H * E / (ms * 1e-3) / 1e12, 2),
                               "GB/s": round(2 * (T * H + E * H) / (ms * 1e-3) / 1e9, 2)}
    ms = _time_ms(lambda: ops.router_topk(x, wr, k, with_logits=True, with_mask=True, with_probs=True))
    out["c5_router_topk"] = {"ms": round(ms, 4)}
    cases = {}
    c = pkg.cases.case38_ref_musa_asm_bf16_ssgemm_nt_320x256
    a, b = c.make_inputs(seed=0, device=dev)
    ms = _time_ms(lambda: c.kernel_function(a, b), reps=20, warm=5)
    cases["case38"] = {"ms": round(ms, 4), "TFLOP/s": round(2 * c.M * c.K * c.N / (ms * 1e-3) / 1e12, 2)}
    del a, b
    c = pkg.cases.case39_ref_musa_asm_tf32_ssgemm_nn_384x256
    a, b = c.make_inputs(seed=0, device=dev)
    ms = _time_ms(lambda: c.kernel_function(a, b), reps=20, warm=5)
    cases["case39"] = {"ms": round(ms, 4), "tf32 TFLOP/s": round(2 * c.M * c.K * c.N / (ms * 1e-3) / 1e12, 2)}
    del a, b
    c = pkg.cases.case31_ref_musa_asm_tf32_ssgemm_tn_128x256
    a, b = c.make_inputs(seed=0, device=dev)
    ms = _time_ms(lambda: c.kernel_function(a, b), reps=20, warm=5)
    cases["case31"] = {"ms": round(ms, 4), "tf32 TFLOP/s": round(2 * c.M * c.K * c.N / (ms * 1e-3) / 1e12, 2)}
    del a, b
    c = pkg.cases.case11_router_bwd_cast_bf16_to_fp32
    (a,) = c.get_inputs(dev)
    ms = _time_ms(lambda: c.kernel_function(a), reps=20, warm=5)
    cases["case11"] = {"ms": round(ms, 4), "GB/s": round(a.numel() * 6 / (ms * 1e-3) / 1e9, 2)}
    del a
    c = pkg.cases.case25_ref_unary_cast_fp32_to_bf16
    a = c.make_inputs(seed=0, device=dev)
    ms = _time_ms(lambda: c.kernel_function(a), reps=20, warm=5)
    cases["case25"] = {"ms": round(ms, 4), "GB/s": round(a.numel() * 6 / (ms * 1e-3) / 1e9, 2)}
    del a
    out["reference_cases"] = cases
    return out


def _progress(msg: str) -> None:
    """One line on stderr per finished section (stdout carries only the JSON result)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _median_ms(fn, flush, reps=50, warm=25):
    """Median device time of fn over `reps` calls after `warm` calls; 1 GiB is overwritten before each
    timed call so no input is served from the 256 MB Infinity Cache."""
    for _ in range(warm):
        fn()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    times = []
    for _ in range(reps):
        flush.zero_()
        ev[0].record()
        fn()
        ev[1].record()
        torch.cuda.synchronize()
        times.append(ev[0].elapsed_time(ev[1]))
    return statistics.median(times)


def _rate(ms, amount, unit):
    rate = amount / (ms * 1e-3) / (1e9 if unit == "GB/s" else 1e12)
    peak = HBM_PEAK_GBS if unit == "GB/s" else BF16_PEAK_TFLOPS
    return {"ms": round(ms, 4), unit: round(rate, 2), "frac_of_peak": round(rate / peak, 4),
            ("bytes" if unit == "GB/s" else "flops"): amount}


def config_lines(pkg, dev):
    """Per-kernel figures at the baseline configs C1-C5 and the reference-case shapes: median of 50
    timed calls after 25 warm-up calls, 1 GiB flushed before each call (one JSON line per config)."""
    ops, inp = pkg.ops, pkg.inputs
    flush = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    for name, cfg in inp.CONFIGS.items():
        T, H, E, k = cfg["tokens"], cfg["hidden"], cfg["experts"], cfg["topk"]
        seed = inp.SEED_CONFIG_BASE + int(name[1:])
        logits = inp.router_logits(T, E, skew=cfg["skew"], seed=seed, device=dev)
        x = inp.randn_bf16((T, H), seed=seed + 1, device=dev)
        _, _, mask, probs = ops.topk(logits, k, with_mask=True, with_probs=True)
        maps = ops.row_id_map(mask, expert_major=True, token_major=True, expert_major_i32=True, expert_offsets=True)
        R = int(maps["expert_offsets"][-1].item())
        tm = maps["token_major"]
        res = {"topk": _rate(_median_ms(lambda: ops.topk(logits, k, with_mask=True, with_probs=True), flush),
                             4 * T * E + 12 * T * k + T * E + 4 * T * E, "GB/s")}
        res["row_id_map_int64_both"] = _rate(_median_ms(lambda: ops.row_id_map(mask), flush), T * E + 16 * T * E, "GB/s")
        res["row_id_map_int32_em"] = _rate(_median_ms(
            lambda: ops.row_id_map(mask, expert_major=False, token_major=False, expert_major_i32=True), flush),
            T * E + 4 * T * E, "GB/s")
        xp = torch.empty(R, H, dtype=torch.bfloat16, device=dev)
        pp = torch.empty(R, dtype=torch.float32, device=dev)
        res["permute_with_probs"] = _rate(_median_ms(
            lambda: ops.permute(x, tm, probs, num_out=R, layout=ops.TOKEN_MAJOR, zero_tail=False, out=xp,
                                permuted_probs=pp), flush),
            2 * T * H + 8 * T * E + 4 * T * E + 2 * R * H + 4 * R, "GB/s")
        res["unpermute_merge"] = _rate(_median_ms(
            lambda: ops.unpermute(xp, tm, probs, layout=ops.TOKEN_MAJOR), flush),
            2 * R * H + 8 * T * E + 4 * T * E + 2 * T * H, "GB/s")
        if name == "c2":
            g = inp.randn_bf16((R, H), seed=seed + 2, device=dev)
            dpp = torch.randn(R, device=dev)
            em = maps["expert_major"]
            res["permute_bwd"] = _rate(_median_ms(lambda: ops.permute_bwd(g, dpp, em), flush),
                                       2 * R * H + 4 * R + 8 * T * E + 2 * T * H + 4 * T * E, "GB/s")
            del g
        del xp, pp
        yield ({"config": name, "tokens": T, "hidden": H, "experts": E, "topk": k, "routed_rows": R,
                      "kernels": res})
    for name, cfg in inp.GEMM_CONFIGS.items():
        seed = inp.SEED_CONFIG_BASE + int(name[1:])
        G, K, N = cfg["groups"], cfg["K"], cfg["N"]
        variants = {"zipf": inp.zipf_group_sizes(cfg["total"], G, seed=seed)}
        if name == "c4":
            variants["uniform_8192"] = [8192] * G
        res = {}
        for vname, sizes in variants.items():
            M = sum(sizes)
            a = inp.randn_bf16((M, K), seed=seed + 1, device=dev)
            w = inp.randn_bf16((G, N, K), std=0.02, seed=seed + 2, device=dev)
            offs = ops.group_offsets_from_splits(sizes, dev)
            out = torch.empty(M, N // 2 if cfg["swiglu"] else N, dtype=torch.bfloat16, device=dev)
            ms = _median_ms(lambda: ops.grouped_gemm(a, w, offs, swiglu=cfg["swiglu"], out=out), flush, reps=20, warm=5)
            res[("fc1_swiglu" if cfg["swiglu"] else "fc2") + "_" + vname] = dict(_rate(ms, 2 * M * K * N, "TFLOP/s"),
                                                                                group_rows=sizes)
            del a, w, out
        yield ({"config": name, "groups": G, "K": K, "N": N, "kernels": res})
    # Reference-case shapes (T=16384, E=320, H=8192): case12's mask, case17 permute, case15 unpermute.
    rm, sel = inp.reference_routing_mask()
    mask = rm.to(dev)
    T, E, H = mask.shape[0], mask.shape[1], 8192
    maps = ops.row_id_map(mask, expert_major=True, token_major=True)
    R = int(mask.sum().item())
    xr, probs = inp.case17_x_probs(sel)
    xr, probs = xr.to(dev), probs.to(dev)
    res = {"row_id_map_int64_both": _rate(_median_ms(lambda: ops.row_id_map(mask), flush), T * E + 16 * T * E, "GB/s")}
    tm, em = maps["token_major"], maps["expert_major"]
    xp = torch.empty(R, H, dtype=torch.bfloat16, device=dev)
    pp = torch.empty(R, dtype=torch.float32, device=dev)
    res["permute_with_probs (case17)"] = _rate(_median_ms(
        lambda: ops.permute(xr, tm, probs, num_out=R, layout=ops.TOKEN_MAJOR, zero_tail=False, out=xp,
                            permuted_probs=pp), flush), 2 * T * H + 8 * T * E + 4 * T * E + 2 * R * H + 4 * R, "GB/s")
    res["unpermute (case15)"] = _rate(_median_ms(lambda: ops.unpermute(xp, em, layout=ops.EXPERT_MAJOR), flush),
                                      2 * R * H + 8 * T * E + 2 * T * H, "GB/s")
    del xp, pp
    # The expert-major scatter of case21/22/30 (their own (t + k) mod E routing, R = 8T) with the output row
    # count known: the kernel alone, without the drop-ins' max/count read-back of the map.
    c21 = pkg.cases.case21_permute_with_mask_map_trans
    em21 = c21.make_row_id_map(device=dev)
    R21 = 8 * T
    x21 = inp.randn_bf16((T, H), seed=inp.SEED_CONFIG_BASE + 21, device=dev)
    p21 = torch.rand(T, E, device=dev) * (em21 >= 0).t()
    out21 = torch.empty(R21, H, dtype=torch.bfloat16, device=dev)
    pp21 = torch.empty(R21, dtype=torch.float32, device=dev)
    res["permute_expert_major (case21/30 map)"] = _rate(_median_ms(
        lambda: ops.permute(x21, em21, num_out=R21, layout=ops.EXPERT_MAJOR, zero_tail=False, out=out21), flush),
        2 * T * H + 8 * T * E + 2 * R21 * H, "GB/s")
    res["permute_expert_major_with_probs (case22 map)"] = _rate(_median_ms(
        lambda: ops.permute(x21, em21, p21, num_out=R21, layout=ops.EXPERT_MAJOR, zero_tail=False, out=out21,
                            permuted_probs=pp21), flush), 2 * T * H + 8 * T * E + 4 * T * E + 2 * R21 * H + 4 * R21, "GB/s")
    res["map_extent (case21 map: max and count)"] = _rate(_median_ms(lambda: ops.map_extent(em21), flush), 8 * T * E, "GB/s")
    del x21, p21, out21, pp21, em21
    yield ({"config": "reference_shapes", "tokens": T, "hidden": H, "experts": E, "routed_rows": R,
                  "kernels": res})
    del xr, probs, maps, mask
    yield (reference_case_line(pkg, dev, flush))


# The reference's published times for the dispatch cases, all on MTT S5000 (Moore Threads):
# "optimized" = its own kernel (kernel_results/README.md:14-17), "trace" = the production kernel's
# median/range in a profiler trace (the kernel_cases file cited).  None is on MI355X.
PUBLISHED_MTT_S5000_MS = {
    "case06": (2.0448, "optimized, kernel_results/README.md:14"),
    "case12": (0.4580, "optimized, kernel_results/README.md:15"),
    "case15": (1.3131, "optimized, kernel_results/README.md:16"),
    "case17": (2.5681, "optimized, kernel_results/README.md:17"),
    "case21": (3.313, "trace median, kernel_cases/case21_ref_permute_with_mask_map_trans.py:34-37"),
    "case22": (1.565, "trace 1.565-1.632, kernel_cases/case22_ref_moe_permute_mask_kernel_true.py:28-33"),
    "case23": (1.565, "trace median, kernel_cases/case23_ref_aten_topk.py:31-34"),
    "case24": (1.158, "trace 1.158-1.237, kernel_cases/case24_ref_moe_unpermute_mask_kernel_false.py:28-31"),
    "case30": (1.509, "trace 1.509-1.558, kernel_cases/case30_ref_moe_permute_mask_kernel.py:24-30"),
    "case32": (1.200, "trace 1.200-1.251, kernel_cases/case32_ref_moe_unpermute_mask_kernel.py:29-32"),
}


def reference_case_line(pkg, dev, flush):
    """Each dispatch case's drop-in `kernel_function` at the case's own default shape and inputs (the
    host-side checks and the max(row_id_map) read-back included where the reference does them), with
    algorithmic bytes and the reference's published MTT S5000 time beside it."""
    cases, inp = pkg.cases, pkg.inputs
    res = {}

    def add(name, fn, nbytes):
        r = _rate(_median_ms(fn, flush), nbytes, "GB/s")
        if name in PUBLISHED_MTT_S5000_MS:
            pub, src = PUBLISHED_MTT_S5000_MS[name]
            r.update(published_mtt_s5000_ms=pub, published_source=src, speedup_vs_published=round(pub / r["ms"], 2))
        res[name] = r

    c = cases.case06_cp_seq_chunk_index_select
    k_ag, v_ag, index = c.get_inputs(dev)
    add("case06", lambda: c.kernel_function(k_ag, v_ag, index), 2 * (k_ag.numel() + v_ag.numel()) * 2)
    del k_ag, v_ag, index

    c = cases.case12_moe_row_id_map_pass2
    (rmap,) = c.get_inputs(dev)
    T, E = rmap.shape
    add("case12", lambda: c.kernel_function(rmap), T * E + 16 * T * E)
    del rmap

    c = cases.case15_moe_unpermute_mask_fwd
    pin, em = c.get_inputs(dev)
    R, H = pin.shape
    E, T = em.shape
    add("case15", lambda: c.kernel_function(pin, em), 2 * R * H + 8 * T * E + 2 * T * H)
    del pin, em

    c = cases.case17_moe_permute_with_mask_map
    x, tm, probs = c.get_inputs(dev)
    T, H = x.shape
    E = probs.shape[1]
    R = c.get_init_inputs()[1]
    add("case17", lambda: c.kernel_function(x, tm, probs, num_out=R),
        2 * T * H + 8 * T * E + 4 * T * E + 2 * R * H + 4 * R)
    del x, tm, probs

    c = cases.case23_aten_topk
    logits = c.make_inputs(device=dev)
    T, E = logits.shape
    add("case23", lambda: c.kernel_function(logits, 8), 4 * T * E + 12 * T * 8)
    del logits

    # The deep_ep / TE scatter-gather cases share one (t + k) mod E routing of T=16384 tokens, top-8.
    c21, c22, c24, c30, c32 = (cases.case21_permute_with_mask_map_trans, cases.case22_moe_permute_mask_kernel_true,
                               cases.case24_moe_unpermute_mask_kernel_false, cases.case30_moe_permute_mask_kernel,
                               cases.case32_moe_unpermute_mask_kernel)
    T, H = c21.M, c21.HIDDEN
    em64 = c21.make_row_id_map(device=dev)
    em32 = c24.make_row_id_map(device=dev)
    E = em64.shape[0]
    R = T * c21.TOPK
    x = inp.randn_bf16((T, H), seed=21, device=dev)
    add("case21", lambda: c21.kernel_function(x, em64), 8 * E * T + 2 * T * H + 2 * R * H)
    add("case30", lambda: c30.kernel_function(x, em64), 8 * E * T + 2 * T * H + 2 * R * H)
    probs = c22.make_probs(em64, device=dev)
    add("case22", lambda: c22.kernel_function(x, em64, probs), 8 * E * T + 2 * T * H + 4 * T * E + 2 * R * H + 4 * R)
    del x, probs
    g = inp.randn_bf16((R, H), seed=24, device=dev)
    add("case24", lambda: c24.kernel_function(g, em32), 2 * R * H + 4 * E * T + 4 * T * H + 2 * T * H)
    pg = torch.randn(R, device=dev)
    add("case32", lambda: c32.kernel_function(g, em32, pg),
        2 * R * H + 4 * E * T + 4 * R + 4 * T * H + 2 * T * H + 4 * T * E)
    del g, pg, em64, em32
    return {"config": "reference_cases", "note": "each case's kernel_function at its own default shape",
            "kernels": res}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="after the timed steps, gather-copy this many MiB once (index_select_vec_kernel): "
                         "the known-size copy that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings")
    ap.add_argument("--library-reference", action="store_true",
                    help="also time torch.bmm (hipBLASLt) on the fc1 shape with equal groups "
                         "(E x [R/E, H] @ [H, 2F]): a library GEMM of the same size, reported beside the stages")
    ap.add_argument("--no-backward", action="store_true",
                    help="skip the backward grouped GEMMs (reported beside the forward, not in value)")
    ap.add_argument("--no-router", action="store_true",
                    help="skip the router front end / router backward timings (reported beside the forward)")
    ap.add_argument("--ceilings", action="store_true",
                    help="instead of the step benchmark, print one JSON line with the measured ceilings: a "
                         "register-only MFMA loop, copy / read-only / write-only streams, and the power and clock "
                         "under them, under the c5 GEMMs and under hipBLASLt on the fc1 shape")
    ap.add_argument("--configs", action="store_true",
                    help="instead of the step benchmark, print one JSON line per baseline config (C1-C5) and the "
                         "reference shapes with per-kernel medians (50 calls, 1 GiB flushed before each)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the MoE dispatch path here has no multi-GPU (expert-parallel) "
              "exchange; run it with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    pkg = importlib.import_module("1188b-reference-kernels_amd")
    dev = torch.device("cuda:0")
    if args.configs:
        for line in config_lines(pkg, dev):
            print(json.dumps(line), flush=True)
        return
    if args.ceilings:
        print(json.dumps(ceilings(pkg, dev)), flush=True)
        return
    T, H, F, E, k = CFG["tokens"], CFG["hidden"], CFG["ffn"], CFG["experts"], CFG["topk"]
    inp = pkg.inputs
    x = inp.randn_bf16((T, H), seed=SEED, device=dev)
    logits = inp.router_logits(T, E, skew=CFG["skew"], seed=SEED, device=dev)
    w1 = inp.randn_bf16((E, 2 * F, H), std=0.02, seed=SEED + 10, device=dev)
    w2 = inp.randn_bf16((E, H, F), std=0.02, seed=SEED + 20, device=dev)
    layer = pkg.moe_ffn.MoEFFN(w1, w2, k)
    ops = pkg.ops

    names = ["topk", "row_id_map", "fc1_swiglu", "fc2", "unpermute_merge"]
    out_buf = torch.empty(T, H, dtype=torch.bfloat16, device=dev)

    def step(ev=None):
        b = layer._buffers(T, dev)
        rec = (lambda i: ev[i].record()) if ev is not None else (lambda i: None)
        rec(0)
        _, _, mask, probs = ops.topk(logits, k, with_mask=True, with_probs=True)
        rec(1)
        maps = ops.row_id_map(mask, expert_major=False, token_major=True, expert_offsets=True, src_out=b["src"],
                              workspace=b["ws"])
        row_map, offs = maps["token_major"], maps["expert_offsets"]
        rec(2)
        ops.grouped_gemm_gather(x, b["src"], w1, offs, swiglu=True, out=b["h"], workspace=b["gemm_ws"])
        rec(3)
        ops.grouped_gemm(b["h"], w2, offs, out=b["z"], workspace=b["gemm_ws"])
        rec(4)
        ops.unpermute(b["z"], row_map, probs, layout=ops.TOKEN_MAJOR, out=out_buf)
        rec(5)
        return out_buf

    for _ in range(args.warmup):
        step()
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(len(names) + 1)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(args.steps):
        step(events[s])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / args.steps
    tokens_per_s = T / (elapsed / args.steps)
    _progress(f"{args.steps} timed steps: {ms_per_step:.3f} ms per step")

    work = stage_work(T, H, F, E, k)
    stages = {}
    for i, n in enumerate(names):
        ms = statistics.mean(ev[i].elapsed_time(ev[i + 1]) for ev in events)
        unit, amount = work[n]
        rate = amount / (ms * 1e-3) / (1e9 if unit == "GB/s" else 1e12)
        peak = HBM_PEAK_GBS if unit == "GB/s" else BF16_PEAK_TFLOPS
        stages[n] = {"ms": round(ms, 4), unit: round(rate, 2), "frac_of_peak": round(rate / peak, 4),
                     ("bytes" if unit == "GB/s" else "flops"): amount}

    # Stand-alone permute (the unfused path's first kernel) on this step's map.
    _, _, row_map, _ = layer.route(logits)
    xp = torch.empty(T * k, H, dtype=torch.bfloat16, device=dev)
    pev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    for _ in range(2):
        ops.permute(x, row_map, num_out=T * k, layout=ops.TOKEN_MAJOR, zero_tail=False, out=xp)
    pev[0].record()
    for _ in range(5):
        ops.permute(x, row_map, num_out=T * k, layout=ops.TOKEN_MAJOR, zero_tail=False, out=xp)
    pev[1].record()
    torch.cuda.synchronize()
    pms = pev[0].elapsed_time(pev[1]) / 5
    pbytes = work["permute"][1]
    standalone = {"permute": {"ms": round(pms, 4), "GB/s": round(pbytes / (pms * 1e-3) / 1e9, 2),
                              "frac_of_peak": round(pbytes / (pms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "bytes": pbytes}}
    del xp

    fc1 = stages["fc1_swiglu"]
    roofline = {"kernel": "grouped_gemm_pp_kernel<swiglu, gather, tails> (fc1 + SwiGLU)", "bound": "mfma",
                "achieved": fc1["TFLOP/s"], "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(fc1["TFLOP/s"] / BF16_PEAK_TFLOPS, 4), "traffic": None,
                "flops_per_launch": fc1["flops"], "avg_launch_ms": fc1["ms"]}
    # HBM bytes per fc1 launch come from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE runs
    # of this same workload (scaled by a known-size copy); counters cannot be read live here.
    traffic_file = REPO / "profiles" / "fc1_swiglu_c5_traffic.json"
    if traffic_file.exists():
        roofline["traffic"] = json.loads(traffic_file.read_text()).get("hbm_bytes_per_launch")
        roofline["traffic_source"] = "profiles/fc1_swiglu_c5_traffic.json"

    # Sanity: the layer's own forward gives the same output as the timed stage sequence.
    out_ref = step().clone()
    out = layer(x, logits)
    torch.cuda.synchronize()
    assert torch.equal(out, out_ref)

    if args.copy_probe_mib > 0:
        src = torch.empty(args.copy_probe_mib * 2 ** 20 // 2, dtype=torch.bfloat16, device=dev).view(1, -1)
        ops.index_select(src, torch.zeros(1, dtype=torch.int64, device=dev))
        torch.cuda.synchronize()
        del src

    backward = None
    if not args.no_backward:
        b = layer._buffers(T, dev)
        _, _, mask, _ = ops.topk(logits, k, with_mask=True, with_probs=True)
        maps = ops.row_id_map(mask, expert_major=False, token_major=True, expert_offsets=True, workspace=b["ws"])
        backward = backward_gemms(pkg, x, maps["token_major"], maps["expert_offsets"], b["h"], w1, w2, dev,
                                  library=args.library_reference)
        _progress("backward GEMMs and reference GEMM cases done")

    router = None if args.no_router else router_section(pkg, x, dev)
    if router is not None:
        _progress("router section done")

    library = None
    if args.library_reference:
        library = library_reference(T * k // E, H, 2 * F, E, dev)

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(pkg, x, logits, w1, w2, k)
        _progress("CPU baseline done")

    line = {
        "metric": METRIC, "value": round(tokens_per_s, 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations and logits + N(0,1.5) expert skew, N(0,0.02) weights)",
        "config": {"workload": "c5: MoE FFN forward, T=16384 H=7168 F=2048 E=64 top-8, one GPU",
                   "tokens": T, "hidden": H, "ffn": F, "experts": E, "topk": k, "routed_rows": T * k},
        "stages": stages,
        "standalone": standalone,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "device": torch.cuda.get_device_name(0),
    }
    if backward is not None:
        line["backward"] = backward
    if router is not None:
        line["router"] = router
    if library is not None:
        line["library_reference"] = library
    print(json.dumps(line))


if __name__ == "__main__":
    main()
