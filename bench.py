#!/usr/bin/env python3
"""Benchmark: the INT4-G32 quantized-linear path on one MI355X.

Step (the headline workload): one batch-1 decoder MLP pass, INT4 group-32 weights --
RMSNorm(4096, eps 1e-6) + fused gate||up GEMV K=4096 -> N=2x12288 with the SiLU*mul
epilogue (one kernel) -> down GEMV K=12288 -> N=4096.  ``value`` is algorithmic HBM bytes per step
(87,359,488 B: packed codes + bf16 scales + 4-bit zeros + activations in/out) divided by
the measured time per step, in GB/s.  Inputs are resident in HBM; the steps rotate over
``--copies`` distinct weight copies (>= 512 MiB in total) so the 256 MiB Infinity Cache
cannot serve them, and are replayed from one HIP graph.

The JSON line also carries:
  roofline      the dominant kernel (RMSNorm + fused gate||up GEMV) timed alone with HIP events on its
                launch stream: achieved GB/s on its algorithmic bytes vs the 8 TB/s HBM peak;
                ``traffic`` comes from the rocprofv3 FETCH_SIZE/WRITE_SIZE summary in
                profiles/ when present
  cpu_baseline  the oracle's torch-CPU dequant-then-matmul of the same MLP step on this host
  extra         the K=4096 N=12288 GEMV alone (GB/s, us/call, fraction of peak) beside a streaming
                read of the same bytes; the exact GEMV and the read over N = 12288 .. 98304; the
                decode step, the prompt pass, FP8, small-M, bf16-head and pointwise lines
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "moss-tts-optimized_amd"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "INT4-G32 GEMV HBM GB/s (% of peak) + 36-layer decode-step ms at bs=1"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
HIDDEN, INTER = 4096, 12288


def gemv_bytes(k: int, n: int, m: int = 1) -> int:
    """Algorithmic bytes of one INT4-G32 projection: codes + bf16 scales + 4-bit zeros +
    bf16 activations in and out."""
    return n * k // 2 + (k // 32) * n * 2 + (k // 32) * n // 2 + 2 * m * k + 2 * m * n


GATEUP_BYTES = gemv_bytes(HIDDEN, 2 * INTER) - 2 * 2 * INTER + 2 * INTER   # output is the SiLU*mul half
DOWN_BYTES = gemv_bytes(INTER, HIDDEN)
MLP_BYTES = GATEUP_BYTES + DOWN_BYTES                                      # 87,359,488
NORM_BYTES = 3 * 2 * HIDDEN                                                # x, weight, y
NORM_GATEUP_BYTES = GATEUP_BYTES + 2 * HIDDEN                              # + the RMSNorm weight


def _log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def _quantized(torch, w4g32, n, k, gen, dev):
    w = torch.randn((n, k), generator=gen, device=dev, dtype=torch.float32).mul_(0.02)
    pw = w4g32.quantize_minmax(w)
    del w
    return pw


def _time_graph(torch, graph, replays: int) -> float:
    """Seconds per replay, HIP events on the capture/replay stream."""
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(replays):
        graph.replay()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3 / replays


def _capture(torch, fn):
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        fn()
    torch.cuda.synchronize()
    return graph


def _traffic():
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    try:
        with open(path) as f:
            data = json.load(f)
        return data.get("norm_gateup_silu_k4096_n24576", {}).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(torch, budget_s: float, gateup, down, h, norm_w):
    """The oracle's torch-CPU dequant-then-matmul of one MLP step, dequantizing every call as the
    reference's contract does, on the same weights as the GPU run (``gateup``/``down``: AutoGPTQ
    ``(qweight, scales, qzeros)`` repacked from the GPU's first weight copy) and the same input:
    all threads of the affinity mask, then 4 threads (the reference's ``cpu_threads`` default)."""
    from oracle import pointwise as op
    from oracle import w4g32 as ow

    def step():
        x = op.rmsnorm(h, norm_w, 1e-6)
        t0 = time.perf_counter()
        w1 = ow.gptq_dequant_cpu(*gateup)
        t1 = time.perf_counter()
        y = torch.nn.functional.linear(x.float(), w1.t().float())
        t2 = time.perf_counter()
        a = ow.silu_mul_rounded(y[:, :INTER], y[:, INTER:])
        t3 = time.perf_counter()
        w2 = ow.gptq_dequant_cpu(*down)
        t4 = time.perf_counter()
        torch.nn.functional.linear(a.float(), w2.t().float()).bfloat16()
        t5 = time.perf_counter()
        return t5 - t0, (t1 - t0) + (t4 - t3), (t2 - t1) + (t5 - t4)

    def run(threads: int, budget: float):
        torch.set_num_threads(threads)
        first = step()[0]
        warm = 1 if first > budget / 6 else 3
        for _ in range(warm - 1):
            step()
        reps = max(3, min(10, int(budget / max(first, 1e-3))))
        rows = sorted((step() for _ in range(reps)), key=lambda r: r[0])
        med = rows[len(rows) // 2]
        return {"threads": threads, "ms_per_step": round(med[0] * 1e3, 3), "dequant_ms": round(med[1] * 1e3, 3),
                "matmul_ms": round(med[2] * 1e3, 3), "GB/s": round(MLP_BYTES / med[0] / 1e9, 3), "reps": reps,
                "warmup": warm}

    prev = torch.get_num_threads()
    threads = len(os.sched_getaffinity(0))
    full = run(threads, budget_s * 0.6)
    four = run(4, budget_s * 0.4)
    torch.set_num_threads(prev)
    return {"value": full["GB/s"], "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{full['reps']} full MLP steps (RMSNorm + gate||up K=4096 N=24576 + SiLU*mul + down "
                      f"K=12288 N=4096) on the GPU run's first weight copy, dequantizing every call; median "
                      f"after {full['warmup']} warm-up",
            "ms_per_step": full["ms_per_step"], "dequant_ms": full["dequant_ms"], "matmul_ms": full["matmul_ms"],
            "cpu_model": _cpu_model(), "threads_4": four}


# Launches per captured graph in the per-launch timings: the gap between two replays of a graph is
# spread over this many launches, so it stays a small part of each launch's time.
MIN_GRAPH_LAUNCHES = 64


def _per_launch(torch, fns, replays: int = 20) -> float:
    """Seconds per launch of ``fns`` (one launch each), the list repeated into one HIP graph of at
    least MIN_GRAPH_LAUNCHES launches."""
    reps = max(1, -(-MIN_GRAPH_LAUNCHES // len(fns)))
    graph = _capture(torch, lambda: [f() for _ in range(reps) for f in fns])
    return _time_graph(torch, graph, replays) / (len(fns) * reps)


def streaming_read_bench(torch, dev, nbytes: int):
    """The vendor library's own streaming read of ``nbytes`` (the K=4096 N=12288 GEMV's algorithmic
    bytes), per launch in a HIP graph over >= 512 MiB of distinct copies: torch's reductions of an
    int32 view along rows of 2 KiB (one output per row, no cross-workgroup step) and over the whole
    buffer.  The best of them is the per-launch read ceiling of a kernel that moves those bytes."""
    cols = 512
    rows = nbytes // (4 * cols)
    copies = [torch.randint(0, 2**31 - 1, (rows, cols), device=dev, dtype=torch.int32)
              for _ in range(max(2, -(-(512 << 20) // (rows * cols * 4))))]
    out = {}
    for name, fn in (("amax_rows", lambda b: torch.amax(b, dim=1)), ("sum_rows", lambda b: b.sum(dim=1)),
                     ("sum_all", lambda b: b.sum())):
        sec = _per_launch(torch, [lambda b=b: fn(b) for b in copies], replays=20)
        out[name] = round(sec * 1e6, 3)
    best = min(out, key=out.get)
    read_bytes = rows * cols * 4
    del copies
    torch.cuda.empty_cache()
    res = {"us_per_call": out[best], "kernel": f"torch.{best}", "bytes": read_bytes,
           "frac_of_peak": round(read_bytes / (out[best] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "all_us": out}
    _log(f"[bench] vendor streaming read of {read_bytes} B: {out} us per launch (best {best})")
    return res


def own_streaming_read_bench(torch, dev, nbytes: int):
    """The library's own streaming read (``moss_stream_read``: 16-byte loads, 1 KiB contiguous per
    wave instruction, nothing but the reads and an XOR) of ``nbytes``, per launch in a HIP graph
    over >= 512 MiB of distinct copies: the ceiling of one launch that only reads the GEMV's bytes."""
    from moss_tts._runtime import native

    n_copies = max(2, -(-(512 << 20) // nbytes))
    copies = [torch.empty(nbytes // 4, device=dev, dtype=torch.int32).random_() for _ in range(n_copies)]
    sink = torch.empty(int(native.lib().moss_stream_read_words(nbytes)), device=dev, dtype=torch.int32)

    def launch(b):
        native.call("moss_stream_read", native.ptr(b), nbytes, native.ptr(sink), native.stream_of(b))

    sec = min(_per_launch(torch, [lambda b=b: launch(b) for b in copies], replays=20) for _ in range(3))
    # the fixed cost of a launch in a graph: the same kernel on 16 bytes (one workgroup)
    tiny = copies[0][:4]
    floor = min(_per_launch(torch, [lambda: native.call("moss_stream_read", native.ptr(tiny), 16, native.ptr(sink),
                                                        native.stream_of(tiny))], replays=20) for _ in range(3))
    del copies, tiny
    torch.cuda.empty_cache()
    res = {"us_per_call": round(sec * 1e6, 3), "kernel": "moss_stream_read", "bytes": nbytes,
           "frac_of_peak": round(nbytes / sec / 1e9 / HBM_PEAK_GBS, 4),
           "launch_floor_us_16_bytes": round(floor * 1e6, 3)}
    _log(f"[bench] own streaming read of {nbytes} B: {res['us_per_call']} us per launch; of 16 B: "
         f"{res['launch_floor_us_16_bytes']} us")
    return res


def gemv_size_sweep(torch, dev, sizes=(12288, 24576, 49152, 98304)):
    """The exact INT4-G32 GEMV at K=4096 over N in ``sizes`` against the library's streaming read of
    the same bytes, each per launch in a HIP graph over >= 512 MiB of distinct copies: how the
    fraction of HBM peak that one launch reaches grows as its fixed costs (the dispatch and the
    first loads' latency) spread over more bytes."""
    from moss_tts._runtime import pointwise, w4g32

    gen = torch.Generator(device=dev)
    gen.manual_seed(11)
    x = pointwise.rmsnorm(torch.randn((1, HIDDEN), generator=gen, device=dev).bfloat16(),
                          torch.ones(HIDDEN, device=dev, dtype=torch.bfloat16), 1e-6)
    out = {}
    for n in sizes:
        nbytes = gemv_bytes(HIDDEN, n)
        copies = [_quantized(torch, w4g32, n, HIDDEN, gen, dev) for _ in range(max(2, -(-(512 << 20) // nbytes)))]
        sec = min(_per_launch(torch, [lambda w=w: w4g32.gemv(x, w) for w in copies], replays=20) for _ in range(3))
        del copies
        torch.cuda.empty_cache()
        rd = own_streaming_read_bench(torch, dev, nbytes)
        out[f"n{n}"] = {"bytes": nbytes, "gemv_us": round(sec * 1e6, 3),
                        "gemv_frac_of_peak": round(nbytes / sec / 1e9 / HBM_PEAK_GBS, 4),
                        "read_us": rd["us_per_call"], "read_frac_of_peak": rd["frac_of_peak"],
                        "gemv_time_over_read_time": round(sec * 1e6 / rd["us_per_call"], 4)}
        _log(f"[bench] GEMV K=4096 N={n}: {sec * 1e6:.2f} us ({out[f'n{n}']['gemv_frac_of_peak']:.1%}), "
             f"read of the same bytes {rd['us_per_call']} us ({rd['frac_of_peak']:.1%})")
    return out


def fp8_bench(torch, dev):
    """FP8 E4M3 weight-only linear, K=4096, N in {4096, 12288}, M in {1, 64}: weights N(0, 0.02)
    with per-output-channel fp32 scales s[n] = max|W[n, :]| / 448 and W8 = e4m3(W / s), activations
    bf16 N(0, 1); weights rotated over >= 600 MB of distinct copies so HBM, not the Infinity Cache,
    serves them.  Also the fused gate||up FP8 GEMV (N = 2 x 12288)."""
    from moss_tts._runtime import fp8

    out = {}
    gen = torch.Generator(device=dev).manual_seed(99)
    for n in (4096, 12288, 24576):
        k = HIDDEN
        copies = max(2, int(640e6 // (n * k)))
        ws, ss = [], []
        for _ in range(copies):
            w = torch.randn((n, k), generator=gen, device=dev, dtype=torch.float32).mul_(0.02)
            s = w.abs().amax(dim=1) / 448.0
            ws.append((w / s[:, None]).to(torch.float8_e4m3fn).view(torch.uint8))
            ss.append(s.contiguous())
            del w
        for m in ((1, 64) if n != 24576 else (1,)):
            x = torch.randn((m, k), generator=gen, device=dev).bfloat16()
            if n == 24576:
                sec = _per_launch(torch, [lambda i=i: fp8.fp8_silu_decode(x, ws[i], ss[i]) for i in range(copies)])
                key = "fp8_gateup_silu_k4096_n24576"
                nbytes = n * k + 4 * n + 2 * k + 2 * n // 2
            else:
                sec = _per_launch(torch, [lambda i=i: fp8.linear(x, ws[i], ss[i]) for i in range(copies)])
                key = f"fp8_linear_m{m}_k4096_n{n}"
                nbytes = n * k + 4 * n + 2 * m * k + 2 * m * n
            gbs = nbytes / sec / 1e9
            out[key] = {"us_per_call": round(sec * 1e6, 3), "GB/s": round(gbs, 1),
                        "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                        "TFLOP/s": round(2 * m * k * n / sec / 1e12, 2), "bytes": nbytes}
            _log(f"[bench] {key}: {sec * 1e6:.2f} us, {gbs:.0f} GB/s")
        del ws, ss
        torch.cuda.empty_cache()
    return out


def small_m_bench(torch, dev):
    """INT4-G32 linear at K = N = 4096 for M = 2..64 tokens (2 to 4: the multi-token GEMV; up to 32:
    the weight-streaming kernel; 64: the register tile) beside the M = 1 GEMV of the same shape;
    weights rotated over >= 600 MB of distinct copies.  GB/s counts the weight stream plus
    activations in and outputs out."""
    from moss_tts._runtime import w4g32

    out = {}
    gen = torch.Generator(device=dev).manual_seed(97)
    k = n = HIDDEN
    wbytes = n * k // 2 + n * (k // 32) * 2 + n * (k // 64)
    copies = [_quantized(torch, w4g32, n, k, gen, dev) for _ in range(max(2, int(600e6 // wbytes)))]
    gemv_us = None
    for m in (1, 2, 3, 4, 7, 15, 16, 32, 64):
        x = torch.randn((m, k), generator=gen, device=dev).bfloat16()
        if m == 1:
            fns = [lambda pw=pw: w4g32.gemv(x, pw) for pw in copies]
        else:
            fns = [lambda pw=pw: w4g32.gemm(x, pw) for pw in copies]
        sec = _per_launch(torch, fns, replays=10)
        nbytes = wbytes + 2 * m * k + 2 * m * n
        gbs = nbytes / sec / 1e9
        if m == 1:
            gemv_us = sec * 1e6
        out[f"int4_m{m}_k4096_n4096"] = {"us_per_call": round(sec * 1e6, 3), "GB/s": round(gbs, 1),
                                         "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                                         "vs_m1_gemv": round(sec * 1e6 / gemv_us, 3)}
        _log(f"[bench] INT4 M={m} K=N=4096: {sec * 1e6:.2f} us, {gbs:.0f} GB/s, {sec * 1e6 / gemv_us:.2f}x the M=1 GEMV")
    del copies
    torch.cuda.empty_cache()
    return out


def bf16_heads_bench(torch, dev):
    """The installed model's output heads: final add-RMSNorm + bf16-weight GEMV, K = 4096,
    N = 32 x 1024 + 2 (audio codebooks and the text head), weights rotated over >= 600 MB of copies.
    GB/s counts the bf16 weights, the norm weight and the activations in and out."""
    from moss_tts._runtime import bf16

    gen = torch.Generator(device=dev).manual_seed(96)
    k, n = HIDDEN, 32 * 1024 + 2
    copies = [(torch.randn((n, k), generator=gen, device=dev) * 0.02).bfloat16() for _ in range(3)]
    x = torch.randn((1, k), generator=gen, device=dev).bfloat16()
    res = torch.randn((1, k), generator=gen, device=dev).bfloat16()
    nw = (1 + 0.01 * torch.randn(k, generator=gen, device=dev)).bfloat16()
    fns = [lambda w=w: bf16.norm_gemv(x, nw, 1e-6, w, residual=res) for w in copies]
    sec = _per_launch(torch, fns, replays=10)
    nbytes = 2 * n * k + 2 * k + 3 * 2 * k + 2 * n
    gbs = nbytes / sec / 1e9
    _log(f"[bench] bf16 heads (add-RMSNorm + GEMV K={k} N={n}): {sec * 1e6:.2f} us, {gbs:.0f} GB/s")
    del copies
    torch.cuda.empty_cache()
    return {"us_per_call": round(sec * 1e6, 3), "GB/s": round(gbs, 1), "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
            "bytes": nbytes, "shape": f"K={k}, N={n}"}


def pointwise_bench(torch, dev):
    """The prompt pass's pointwise kernels at 512 tokens: add-RMSNorm (4096 wide), the q/k head
    RMSNorm + RoPE + KV-cache write, and SiLU*mul (24576 -> 12288).  Inputs are rotated over
    >= 300 MB of copies so they come from HBM; GB/s counts the bytes each kernel must read and
    write once."""
    from moss_tts._runtime import pointwise

    gen = torch.Generator(device=dev).manual_seed(97)
    n, out = 512, {}

    def copies_for(nbytes):
        return max(2, -(-300 * 2**20 // nbytes))

    # add-RMSNorm: x and residual in, summed and normalized out
    nb = 2 * n * HIDDEN * 2
    xs = [(torch.randn((n, HIDDEN), generator=gen, device=dev)).bfloat16() for _ in range(copies_for(nb))]
    res = torch.randn((n, HIDDEN), generator=gen, device=dev).bfloat16()
    nw = (1 + 0.01 * torch.randn(HIDDEN, generator=gen, device=dev)).bfloat16()
    cases = [("add_rmsnorm_512x4096", [lambda x=x: pointwise.add_rmsnorm(x, res, nw, 1e-6) for x in xs],
              4 * n * HIDDEN * 2 + 2 * HIDDEN)]
    # q/k norm + RoPE + KV write: qkv rows in; q, K and V rows out; one cos/sin row per token
    qkv_w = (pointwise.QH + 2 * pointwise.KH) * pointwise.HD
    nb = n * qkv_w * 2
    qkvs = [torch.randn((n, qkv_w), generator=gen, device=dev).bfloat16() for _ in range(copies_for(nb))]
    qn = (1 + 0.01 * torch.randn(pointwise.HD, generator=gen, device=dev)).bfloat16()
    kn = (1 + 0.01 * torch.randn(pointwise.HD, generator=gen, device=dev)).bfloat16()
    ang = torch.arange(n, device=dev, dtype=torch.float32)[:, None] * torch.rand(pointwise.HD, device=dev)
    cos, sin = ang.cos().bfloat16().contiguous(), ang.sin().bfloat16().contiguous()
    kc = torch.zeros((1, pointwise.KH, 2048, pointwise.HD), device=dev, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    pos = torch.arange(n, device=dev, dtype=torch.int64)
    cases.append(("qk_norm_rope_kv_512", [lambda q=q: pointwise.qk_rope(q, qn, kn, cos, sin, kc, vc, pos, 1e-6)
                                          for q in qkvs],
                  n * qkv_w * 2 + n * pointwise.QH * pointwise.HD * 2 + 2 * n * pointwise.KH * pointwise.HD * 2
                  + 2 * n * pointwise.HD * 2))
    # SiLU*mul: gate||up rows in, the product out
    nb = n * 2 * INTER * 2
    gus = [torch.randn((n, 2 * INTER), generator=gen, device=dev).bfloat16() for _ in range(copies_for(nb))]
    cases.append(("silu_mul_512x12288", [lambda g=g: pointwise.silu_mul(g) for g in gus], nb + n * INTER * 2))
    for name, fns, nbytes in cases:
        sec = _per_launch(torch, fns, replays=5)
        gbs = nbytes / sec / 1e9
        _log(f"[bench] {name}: {sec * 1e6:.2f} us, {gbs:.0f} GB/s")
        out[name] = {"us_per_call": round(sec * 1e6, 3), "GB/s": round(gbs, 1),
                     "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "bytes": nbytes, "copies": len(fns)}
    del xs, qkvs, gus
    torch.cuda.empty_cache()
    return out


def prefill_bench(torch, dev):
    """INT4-G32 prefill GEMMs at M=512 (QKV N=6144, O N=4096, gate||up N=24576, down K=12288):
    TFLOP/s against the 2.5 PFLOP/s dense bf16 MFMA peak."""
    from moss_tts._runtime import w4g32

    out = {}
    gen = torch.Generator(device=dev).manual_seed(98)
    x = torch.randn((512, INTER), generator=gen, device=dev).bfloat16()
    for name, k, n in (("qkv", HIDDEN, 6144), ("o", HIDDEN, HIDDEN), ("gate_up", HIDDEN, 2 * INTER),
                       ("down", INTER, HIDDEN)):
        pw = _quantized(torch, w4g32, n, k, gen, dev)
        xk = x[:, :k].contiguous()
        sec = _per_launch(torch, [lambda: w4g32.gemm(xk, pw)] * 8, replays=10)
        tf = 2 * 512 * k * n / sec / 1e12
        # for scale: the vendor library's plain bf16 GEMM (hipBLASLt through torch.matmul) on the
        # bit-exact dequantized weights, which does none of the dequantization work
        wb = w4g32.dequantize(pw)
        ref_sec = _per_launch(torch, [lambda: torch.matmul(xk, wb.t())] * 8, replays=10)
        out[f"gemm_m512_{name}_k{k}_n{n}"] = {
            "us_per_call": round(sec * 1e6, 2), "TFLOP/s": round(tf, 1),
            "frac_of_mfma_bf16_peak": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
            "hipblaslt_bf16_us_on_dequantized_weights": round(ref_sec * 1e6, 2)}
        _log(f"[bench] prefill GEMM M=512 {name}: {sec * 1e6:.1f} us, {tf:.0f} TFLOP/s "
             f"(hipBLASLt bf16 on the dequantized weights: {ref_sec * 1e6:.1f} us)")
        del pw, wb
    # the four projections of one layer, times the 36 layers (attention and norms not included)
    us = sum(v["us_per_call"] for v in out.values())
    ref_us = sum(v["hipblaslt_bf16_us_on_dequantized_weights"] for v in out.values())
    flop = 2 * 512 * (HIDDEN * 6144 + HIDDEN * HIDDEN + HIDDEN * 2 * INTER + INTER * HIDDEN)
    out["projections_36_layers"] = {"ms": round(36 * us / 1e3, 3), "TFLOP/s": round(flop / us / 1e6, 1),
                                    "frac_of_mfma_bf16_peak": round(flop / us / 1e6 / MFMA_BF16_PEAK_TFLOPS, 4),
                                    "hipblaslt_bf16_ms_on_dequantized_weights": round(36 * ref_us / 1e3, 3)}
    _log(f"[bench] prefill projections M=512, 36 layers: {36 * us / 1e3:.2f} ms, {flop / us / 1e6:.0f} TFLOP/s")
    return out


def prefill_pass_bench(torch, n_layers: int, dev, replays: int = 10, n: int = 512):
    """The n-token prompt pass alone (a bucket of 128, 160, 256 or 512 tokens, the whole 151936-row
    bf16 text head included, as the reference's prefill returns those logits): the bucket graph run
    once by ``prefill`` and then replayed ``replays`` times (13 executions in all, with the two eager
    warm-ups before capture, for a kernel trace)."""
    from moss_tts._runtime.decode import DecodeStepG32

    eng = DecodeStepG32.random(n_layers, max_length=2048, device=dev, seed=4242, text_head=True)
    eng.capture_prefill((n,))
    g = torch.Generator().manual_seed(5)
    ids = torch.cat([torch.randint(0, 151643, (n, 1), generator=g), torch.randint(0, 1024, (n, 32), generator=g)], 1)
    eng.prefill(ids)
    graph = eng.prefill_graphs[n][0]
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / replays
    _log(f"[bench] prefill of {n} tokens through {n_layers} layers: {ms:.3f} ms per replay ({replays} replays)")
    return ms


def decode_step_bench(torch, n_layers: int, steps: int, dev, w4a8: bool = False):
    """The full batch-1 decode step (embedding -> n_layers -> 32 INT4 heads, KV cache of 2048
    rows filled with N(0,1), current position 2047) captured as one graph; ms per step.
    ``w4a8``: the layer projections in the int8-activation arithmetic."""
    from moss_tts._runtime.decode import DecodeStepG32, FirstAudioGraph

    _log(f"[bench] building the {n_layers}-layer decode step (random INT4-G32 weights, KV 2048, w4a8={w4a8})")
    eng = DecodeStepG32.random(n_layers, max_length=2048, device=dev, seed=4242, w4a8=w4a8, text_head=not w4a8)
    eng.capture()
    ids = torch.tensor([[151643] + [i * 31 % 1025 for i in range(32)]], dtype=torch.int64)
    eng.step(ids, 2047)
    for _ in range(10):  # warm-up replays: clocks and caches settle before the timed ones
        eng.graph.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    runs = []
    for _ in range(3):  # median of three timed runs of `steps` replays each
        start.record()
        for _ in range(steps):
            eng.graph.replay()
        end.record()
        torch.cuda.synchronize()
        runs.append(start.elapsed_time(end) / steps)
    ms = sorted(runs)[1]
    # host time to enqueue one replay on an idle stream: when it approaches the step time the
    # step is bound by graph submission, not by the kernels
    host = []
    for _ in range(10):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        eng.graph.replay()
        host.append((time.perf_counter() - t0) * 1e3)
    torch.cuda.synchronize()
    host_ms = sorted(host)[len(host) // 2]
    # the 32 steps after the audio start as one graph (device-side advance between steps)
    burst = FirstAudioGraph(eng, 32)
    burst.warmup()
    first = torch.full((1, 1, 33), 1024, dtype=torch.int64, device=dev)
    first[0, 0, 0] = eng.audio_start_id
    burst.run(first, 2047 - 32)
    torch.cuda.synchronize()
    start.record()
    for _ in range(3):
        burst.run(first, 2047 - 32)
    end.record()
    torch.cuda.synchronize()
    burst_ms = start.elapsed_time(end) / (3 * 32)
    del burst
    prefill = full = None
    if not w4a8:
        # the text-phase step (FastLLM.full_step): the layers, the final norm and the whole text head
        # of 151936 bf16 rows (1.24 GB), captured as its own graph
        eng.capture_text()
        eng.full_step(ids, 2047)
        torch.cuda.synchronize()
        start.record()
        for _ in range(steps):
            eng.text_graph.replay()
        end.record()
        torch.cuda.synchronize()
        fms = start.elapsed_time(end) / steps
        fbytes = eng.step_bytes(2047) - eng.heads.packed.nbytes + eng.text_head.nbytes
        full = {"ms": round(fms, 4), "bytes": fbytes, "GB/s": round(fbytes / fms / 1e6, 1),
                "text_head_rows": eng.text_head.out_features}
        _log(f"[bench] text-phase step (layers + text head of {eng.text_head.out_features} rows): {fms:.3f} ms, "
             f"{fbytes / fms / 1e6:.0f} GB/s")
        eng.text_graph = None
        # the whole prompt pass of 512 tokens (36 layers of INT4 GEMMs, causal attention, norms,
        # SiLU*mul, the final norm and heads on the last token) as its bucket graph
        n = 512
        eng.capture_prefill((n,))
        g = torch.Generator().manual_seed(5)
        ids = torch.cat([torch.randint(0, 151643, (n, 1), generator=g), torch.randint(0, 1024, (n, 32), generator=g)], 1)
        eng.prefill(ids)
        graph = eng.prefill_graphs[n][0]
        torch.cuda.synchronize()
        start.record()
        for _ in range(5):
            graph.replay()
        end.record()
        torch.cuda.synchronize()
        pms = start.elapsed_time(end) / 5
        # the flop the pass performs: every layer's QKV for all n tokens; attention, O and the MLP for
        # all n tokens in the first n_layers - 1 layers and for the last token alone in the last one
        rest = HIDDEN * HIDDEN + HIDDEN * 2 * INTER + INTER * HIDDEN
        proj = 2 * HIDDEN * 6144 * n * n_layers + 2 * rest * (n * (n_layers - 1) + 1)
        attn = (n_layers - 1) * 32 * 2 * 2 * 128 * n * (n + 1) // 2 + 32 * 2 * 2 * 128 * n
        tf = (proj + attn) / pms / 1e9
        prefill = {"tokens": n, "layers": n_layers, "ms": round(pms, 3), "TFLOP/s": round(tf, 1),
                   "frac_of_mfma_bf16_peak": round(tf / MFMA_BF16_PEAK_TFLOPS, 4), "flop": proj + attn,
                   "parts": "embedding, per layer: norms, INT4 GEMMs, q/k-norm + RoPE + KV write, causal attention, "
                            "SiLU*mul (the last layer's attention, O and MLP for the last token only, whose logits "
                            "the pass returns); final norm + audio heads and the whole 151936-row bf16 text head "
                            "on the last token"}
        _log(f"[bench] prefill of {n} tokens through {n_layers} layers: {pms:.3f} ms, {tf:.0f} TFLOP/s")
        eng.prefill_graphs.clear()
    nbytes = eng.step_bytes(2047)
    _log(f"[bench] decode step ({n_layers} layers, w4a8={w4a8}): {ms:.3f} ms, {nbytes / ms / 1e6:.0f} GB/s; "
         f"host enqueue {host_ms:.3f} ms per replay; 32-step first-audio graph {burst_ms:.3f} ms per step")
    out = {"layers": n_layers, "ms_per_step": round(ms, 4), "bytes_per_step": nbytes,
           "GB/s": round(nbytes / ms / 1e6, 1), "frac_of_peak": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4),
           "kv_rows": 2048, "position": 2047, "target_ms": 4.0, "host_enqueue_ms": round(host_ms, 4),
           "first_audio_graph_ms_per_step": round(burst_ms, 4),
           "arithmetic": "w4a8 (int8 activations, integer dot)" if w4a8 else "w4a16 (exact bf16 dequant)"}
    if prefill is not None:
        out["prefill_512"] = prefill
    if full is not None:
        out["full_step_ms"] = full["ms"]
        out["full_step"] = full
    del eng
    torch.cuda.empty_cache()
    return out


def decode_budget(torch, n_layers: int, steps: int, dev, w4a8: bool = False) -> dict:
    """Per-kernel budget of the decode step (W4A16, or the W4A8 arithmetic) measured inside the step
    itself, untraced: for each kernel family, a graph of the step in which every launch of that
    family runs twice (the launches are idempotent: same inputs, same outputs) is timed against the
    plain step graph; the difference is what that family's launches cost in the step, dispatch gaps
    included.  The families' costs sum to about the step time, unlike traced kernel durations."""
    import contextlib

    from moss_tts._runtime import attention, sampling, w4g32
    from moss_tts._runtime import w4a8 as w8
    from moss_tts._runtime.decode import DecodeStepG32

    eng = DecodeStepG32.random(n_layers, max_length=2048, device=dev, seed=4242, w4a8=w4a8)
    ids = torch.tensor([[151643] + [i * 31 % 1025 for i in range(32)]], dtype=torch.int64)

    def time_step() -> float:
        eng.graph = None
        eng.capture()
        eng.step(ids, 2047)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            eng.graph.replay()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / steps * 1e3

    # The extra launch reads copies of the weights (and of the KV caches) made once, outside the
    # capture, during the eager warm-up: reading the same bytes the step's own launch reads right
    # after it would find part of them in the Infinity Cache and understate the family's cost.
    copies = {}

    def cold(obj):
        # keyed by storage: modules hand out a new PackedW4G32 view of the same tensors per access
        if isinstance(obj, w4g32.PackedW4G32):
            key = ("w", obj.qw.data_ptr(), obj.qw.numel())
        elif isinstance(obj, torch.Tensor):
            key = ("t", obj.data_ptr(), obj.numel())
        else:
            return obj
        if key not in copies:
            assert not torch.cuda.is_current_stream_capturing(), "copies are made during the eager warm-up"
            if isinstance(obj, w4g32.PackedW4G32):
                copies[key] = w4g32.PackedW4G32(obj.qw.clone(), obj.scales.clone(), obj.zeros.clone())
            else:
                copies[key] = obj.clone()
        return copies[key]

    @contextlib.contextmanager
    def doubled(module, name, pick, cold_args=()):
        orig = getattr(module, name)

        def twice(*a, **kw):
            if pick(*a, **kw):
                extra = [cold(v) if i in cold_args else v for i, v in enumerate(a)]
                orig(*extra, **kw)
            return orig(*a, **kw)

        setattr(module, name, twice)
        try:
            yield
        finally:
            setattr(module, name, orig)

    def width(a, kw):
        return a[3].N if len(a) > 3 else kw["w"].N

    if w4a8:
        def w8_k(a, kw):
            return (a[1] if len(a) > 1 else kw["w"]).K

        layer_families = [
            ("add-RMSNorm + int8 quantizer + q||k||v GEMV", w8, "norm_linear", lambda *a, **kw: not kw.get("paired"),
             n_layers, (3,)),
            ("q/k-norm + RoPE + KV write + attention split + merge with int8 output", attention,
             "decode_attention_qkv", lambda *a, **kw: True, n_layers, (5, 6)),
            ("O GEMV (K=4096, int8 input from the merge)", w8, "linear",
             lambda *a, **kw: w8_k(a, kw) == 4096 and not kw.get("paired"), n_layers, (1,)),
            ("add-RMSNorm + int8 quantizer + gate||up GEMV + SiLU*mul", w8, "norm_linear",
             lambda *a, **kw: bool(kw.get("paired")), n_layers, (3,)),
            ("down GEMV (K=12288) quantizing its bf16 input inside", w8, "linear", lambda *a, **kw: w8_k(a, kw) == 12288,
             n_layers, (1,)),
        ]
    else:
        layer_families = [
            ("add-RMSNorm + q||k||v GEMV", w4g32, "norm_gemv", lambda *a, **kw: width(a, kw) == 6144, n_layers,
             (3,)),
            ("q/k-norm + RoPE + KV write + attention split + merge", attention, "decode_attention_qkv",
             lambda *a, **kw: True, n_layers, (5, 6)),
            ("O GEMV (K=4096)", w4g32, "gemv", lambda *a, **kw: a[1].K == 4096, n_layers, (1,)),
            ("add-RMSNorm + gate||up GEMV + SiLU*mul", w4g32, "norm_gateup_silu", lambda *a, **kw: True,
             n_layers, (3,)),
            ("down GEMV (K=12288)", w4g32, "gemv", lambda *a, **kw: a[1].K == 12288, n_layers, (1,)),
        ]
    families = [("embedding sum", attention, "embedding_sum", lambda *a, **kw: True, 1, ())] + layer_families + [
        ("final add-RMSNorm + heads GEMV", w4g32, "norm_gemv", lambda *a, **kw: width(a, kw) > 6144, 1, (3,)),
        ("sampling (text and audio rows)", sampling, "sample_topk_pair", lambda *a, **kw: True, 1, ()),
        ("next-id composition", sampling, "compose_next_ids", lambda *a, **kw: True, 1, ()),
    ]
    base = [time_step() for _ in range(5)]
    base_us = sorted(base)[2]
    rows, total = [], 0.0
    for label, module, name, pick, count, cold_args in families:
        with doubled(module, name, pick, cold_args):
            t = sorted(time_step() for _ in range(5))[2]
        copies.clear()
        cost = t - base_us
        total += cost
        rows.append({"kernels": label, "launches_per_step": count, "us_per_step": round(cost, 1),
                     "us_per_launch": round(cost / count, 3)})
        _log(f"[bench] budget: {label}: {cost:.1f} us per step ({cost / count:.2f} us x {count})")
    _log(f"[bench] budget: step {base_us:.1f} us; sum of the families {total:.1f} us")
    return {"arithmetic": "w4a8" if w4a8 else "w4a16", "step_us": round(base_us, 1),
            "sum_of_families_us": round(total, 1), "families": rows,
            "method": "each family's launches doubled inside the captured step, the extra launch reading its "
                      "own copy of the weights and KV caches; cost = step time difference"}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=800)
    ap.add_argument("--warmup", type=int, default=80)
    ap.add_argument("--copies", type=int, default=8, help="distinct MLP weight copies rotated over")
    ap.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU-baseline work")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--decode-steps", type=int, default=30,
                    help="timed replays of the 36-layer decode step (0 skips it)")
    ap.add_argument("--decode-layers", type=int, default=36)
    ap.add_argument("--no-extras", action="store_true", help="skip the FP8 and prefill GEMM lines")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the 36-layer decode step (both arithmetics) and its lines, for a kernel trace")
    ap.add_argument("--decode-budget", action="store_true",
                    help="per-kernel budget of the 36-layer decode step (W4A16, then W4A8), measured inside the "
                         "untraced step")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the 36-layer prompt pass (10 graph replays), for a kernel trace")
    ap.add_argument("--prefill-tokens", type=int, choices=(128, 160, 256, 512), default=512,
                    help="prompt length (a bucket size) for --prefill-only")
    ap.add_argument("--pmc-pass", choices=("gemv", "gemm"), default=None,
                    help="eager launches only, for rocprofv3 --pmc: 'gemv' = a 512 MiB copy of known size, "
                         "then one fused gate||up GEMV and one K=4096 N=12288 GEMV per weight copy; "
                         "'gemm' = the four M=512 prefill GEMMs once each")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures the single-GPU path only: the INT4-G32 decode path runs on one "
              "MI355X (how it would shard is described, not run). Use --gpus 1.", file=sys.stderr)
        return 2
    if args.steps <= 0 or args.warmup < 0 or args.copies <= 0:
        print("steps must be positive, warmup non-negative", file=sys.stderr)
        return 2

    import torch

    from moss_tts._runtime import native, pointwise, w4a8, w4g32

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    arch = native.device_arch(0)
    if args.prefill_only:
        _log(f"[bench] device {torch.cuda.get_device_name(0)} ({arch}); {args.prefill_tokens}-token prompt pass only")
        prefill_pass_bench(torch, args.decode_layers, dev, n=args.prefill_tokens)
        return 0
    if args.decode_budget:
        _log(f"[bench] device {torch.cuda.get_device_name(0)} ({arch}); decode-step budget")
        for w4a8 in (False, True):
            print(json.dumps(decode_budget(torch, args.decode_layers, max(1, args.decode_steps), dev, w4a8=w4a8)),
                  flush=True)
        return 0
    if args.decode_only:
        _log(f"[bench] device {torch.cuda.get_device_name(0)} ({arch}); decode step only")
        for w8 in (False, True):
            decode_step_bench(torch, args.decode_layers, max(1, args.decode_steps), dev, w4a8=w8)
        return 0
    _log(f"[bench] device {torch.cuda.get_device_name(0)} ({arch}); building {args.copies} weight copies")

    gen = torch.Generator(device=dev).manual_seed(1234)
    copies = []
    for c in range(args.copies):
        copies.append((_quantized(torch, w4g32, 2 * INTER, HIDDEN, gen, dev),
                       _quantized(torch, w4g32, HIDDEN, INTER, gen, dev)))
    h = torch.randn((1, HIDDEN), generator=gen, device=dev).bfloat16()
    norm_w = (1 + 0.01 * torch.randn(HIDDEN, generator=gen, device=dev)).bfloat16()
    resident = sum(gu.nbytes + dn.nbytes for gu, dn in copies)
    _log(f"[bench] {resident / 2**20:.0f} MiB of packed MLP weights resident")

    if args.pmc_pass == "gemm":
        # the four M=512 prefill GEMMs plain, then in the fused forms the prompt pass runs (QKV with
        # the q/k-norm + RoPE + KV write, gate||up with SiLU*mul, O and down with the add-RMSNorm),
        # then the e4m3 M=64 linears (K=4096, N=4096 and 12288; split-K GEMM + reduction)
        from moss_tts._runtime import fp8

        del copies
        torch.cuda.empty_cache()
        x = torch.randn((512, INTER), generator=gen, device=dev).bfloat16()
        ws = {}
        for name, k, n in (("qkv", HIDDEN, 6144), ("o", HIDDEN, HIDDEN), ("gate_up", HIDDEN, 2 * INTER),
                           ("down", INTER, HIDDEN)):
            pw = _quantized(torch, w4g32, n, k, gen, dev)
            ws[name] = (pw, x[:, :k].contiguous())
            torch.cuda.synchronize()
            w4g32.gemm(ws[name][1], pw)
            torch.cuda.synchronize()
            _log(f"[bench] pmc pass: GEMM M=512 K={k} N={n} ({2 * 512 * k * n} flop)")
        hd = 128
        qn = (1 + 0.01 * torch.randn(hd, generator=gen, device=dev)).bfloat16()
        kn = (1 + 0.01 * torch.randn(hd, generator=gen, device=dev)).bfloat16()
        ang = torch.arange(1024, device=dev, dtype=torch.float32)[:, None] * torch.rand(hd, device=dev)
        cos, sin = ang.cos().bfloat16().contiguous(), ang.sin().bfloat16().contiguous()
        kc = torch.zeros((1, 8, 1024, hd), device=dev, dtype=torch.bfloat16)
        vc = torch.zeros_like(kc)
        pos = torch.arange(512, device=dev, dtype=torch.int64)
        res = torch.randn((512, HIDDEN), generator=gen, device=dev).bfloat16()
        torch.cuda.synchronize()
        w4g32.gemm_qk_rope(ws["qkv"][1], ws["qkv"][0], qn, kn, cos, sin, kc, vc, pos, 1e-6)
        torch.cuda.synchronize()
        w4g32.gemm_silu(ws["gate_up"][1], ws["gate_up"][0])
        torch.cuda.synchronize()
        w4g32.gemm_add_rmsnorm(ws["o"][1], ws["o"][0], res, norm_w, 1e-6)
        torch.cuda.synchronize()
        w4g32.gemm_add_rmsnorm(ws["down"][1], ws["down"][0], res, norm_w, 1e-6)
        torch.cuda.synchronize()
        _log("[bench] pmc pass: fused prefill forms M=512 (QKV + RoPE, gate||up + SiLU*mul, O / down + add-RMSNorm)")
        del ws
        torch.cuda.empty_cache()
        for n in (HIDDEN, 3 * HIDDEN):
            w = torch.randn((n, HIDDEN), generator=gen, device=dev).mul_(0.02)
            s8 = w.abs().amax(dim=1) / 448.0
            w8 = (w / s8[:, None]).to(torch.float8_e4m3fn).view(torch.uint8)
            x64 = torch.randn((64, HIDDEN), generator=gen, device=dev).bfloat16()
            torch.cuda.synchronize()
            fp8.linear(x64, w8, s8.contiguous())
            torch.cuda.synchronize()
            _log(f"[bench] pmc pass: e4m3 linear M=64 K={HIDDEN} N={n} ({n * HIDDEN + 4 * n + 2 * 64 * HIDDEN + 2 * 64 * n} B)")
        return 0
    if args.pmc_pass == "gemv":
        src = torch.empty(512 * 2**20 // 4, dtype=torch.int32, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        xs = pointwise.rmsnorm(h, norm_w, 1e-6)
        for gu, _ in copies:
            w4g32.norm_gateup_silu(h, norm_w, 1e-6, gu)
        torch.cuda.synchronize()
        for gu, _ in copies:
            w4g32.gemv(xs, gu.rows(0, INTER))
        torch.cuda.synchronize()
        _log(f"[bench] pmc pass done: copy {src.numel() * 4} B; {len(copies)} gate||up launches "
             f"({NORM_GATEUP_BYTES} algorithmic B each); {len(copies)} GEMV K=4096 N=12288 launches "
             f"({gemv_bytes(HIDDEN, INTER)} B each)")
        return 0

    def steps(count: int, offset: int = 0, dequant: int = w4g32.EXACT):
        def run():
            for i in range(count):
                gu, dn = copies[(offset + i) % len(copies)]
                a = w4g32.norm_gateup_silu(h, norm_w, 1e-6, gu, dequant=dequant)
                w4g32.gemv(a, dn, dequant=dequant)
        return run

    # one graph holds whole rotations over the copies and at least MIN_GRAPH_LAUNCHES launches
    cycle = len(copies) * max(1, -(-MIN_GRAPH_LAUNCHES // (2 * len(copies))))
    g_cycle = _capture(torch, steps(cycle))
    rem = args.steps % cycle
    g_rem = _capture(torch, steps(rem)) if rem else None

    for _ in range(max(1, -(-args.warmup // cycle))):
        g_cycle.replay()
    torch.cuda.synchronize()
    _log(f"[bench] warm-up done; timing {args.steps} steps")

    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    start.record(stream)
    for _ in range(args.steps // cycle):
        g_cycle.replay()
    if g_rem is not None:
        g_rem.replay()
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    sec = start.elapsed_time(end) / 1e3
    ms_per_step = sec / args.steps * 1e3
    value = MLP_BYTES / (sec / args.steps) / 1e9
    _log(f"[bench] {ms_per_step * 1e3:.2f} us/step ({value:.0f} GB/s), wall {wall:.3f}s")

    # the unrounded-dequant MLP step, reported beside the default (exact) one
    g_unr = _capture(torch, steps(cycle, dequant=w4g32.UNROUNDED))
    g_unr.replay()
    unr_s = _time_graph(torch, g_unr, max(1, args.steps // cycle)) / cycle

    # the same MLP step in the W4A8 arithmetic, as the decode step runs it: RMSNorm + int8
    # quantizer + gate||up with SiLU*mul in one kernel, then the quantizer + down in one kernel
    def steps_w4a8(count: int):
        def run():
            for i in range(count):
                gu, dn = copies[i % len(copies)]
                mid = w4a8.norm_linear(h, norm_w, 1e-6, gu, paired=True, rows_per_wave=2)
                w4a8.linear(mid, dn)
        return run

    g_w8 = _capture(torch, steps_w4a8(cycle))
    g_w8.replay()
    w8_s = _time_graph(torch, g_w8, max(1, args.steps // cycle)) / cycle
    _log(f"[bench] W4A8 MLP step: {w8_s * 1e6:.2f} us ({MLP_BYTES / w8_s / 1e9:.0f} GB/s)")

    # dominant kernel alone: fused gate||up GEMV over the rotating copies
    xs = pointwise.rmsnorm(h, norm_w, 1e-6)

    def per_launch(fn, launches):
        reps = max(1, -(-MIN_GRAPH_LAUNCHES // launches))
        graph = _capture(torch, lambda: [fn() for _ in range(reps)])
        return _time_graph(torch, graph, 50) / (launches * reps)

    gu_s = per_launch(lambda: [w4g32.norm_gateup_silu(h, norm_w, 1e-6, gu) for gu, _ in copies], len(copies))
    gu_gbs = NORM_GATEUP_BYTES / gu_s / 1e9
    gu_unr_s = per_launch(lambda: [w4g32.norm_gateup_silu(h, norm_w, 1e-6, gu, dequant=w4g32.UNROUNDED)
                                   for gu, _ in copies], len(copies))
    _log(f"[bench] gate||up GEMV: {gu_s * 1e6:.2f} us/launch, {gu_gbs:.0f} GB/s "
         f"(unrounded {gu_unr_s * 1e6:.2f} us)")

    # the K=4096, N=12288 GEMV alone, over >= 512 MiB of distinct weights
    gemv_copies = [gu.rows(0, INTER) for gu, _ in copies] + [gu.rows(INTER, 2 * INTER) for gu, _ in copies]
    ns_s = per_launch(lambda: [w4g32.gemv(xs, w) for w in gemv_copies], len(gemv_copies))
    ns_unr_s = per_launch(lambda: [w4g32.gemv(xs, w, dequant=w4g32.UNROUNDED) for w in gemv_copies],
                          len(gemv_copies))
    ns_bytes = gemv_bytes(HIDDEN, INTER)
    ns_gbs = ns_bytes / ns_s / 1e9
    a = w4g32.gateup_silu(xs, copies[0][0])
    dn_s = per_launch(lambda: [w4g32.gemv(a, dn) for _, dn in copies], len(copies))
    _log(f"[bench] GEMV K=4096 N=12288: {ns_s * 1e6:.2f} us, {ns_gbs:.0f} GB/s (unrounded {ns_unr_s * 1e6:.2f} us); "
         f"down K=12288 N=4096: {dn_s * 1e6:.2f} us, {DOWN_BYTES / dn_s / 1e9:.0f} GB/s")

    n_copies = len(copies)
    # the CPU baseline's weights: the GPU run's first copy, back in the AutoGPTQ layout
    cpu_weights = None
    if not args.no_cpu_baseline:
        from oracle import w4g32 as ow

        def to_gptq(pw):
            q, z = ow.rowunpack(pw.qw.cpu(), pw.zeros.cpu())
            return ow.pack_gptq(q, z, pw.scales.cpu())

        cpu_weights = (to_gptq(copies[0][0]), to_gptq(copies[0][1]), h.cpu(), norm_w.cpu())
    del copies, gemv_copies, g_cycle, g_unr, g_rem, g_w8
    torch.cuda.empty_cache()
    read = streaming_read_bench(torch, dev, ns_bytes)
    read["gemv_time_over_read_time"] = round(ns_s * 1e6 / read["us_per_call"], 4)
    own_read = own_streaming_read_bench(torch, dev, ns_bytes)
    own_read["gemv_time_over_read_time"] = round(ns_s * 1e6 / own_read["us_per_call"], 4)
    size_sweep = gemv_size_sweep(torch, dev) if not args.no_extras else None
    fp8_lines = fp8_bench(torch, dev) if not args.no_extras else None
    small_m = small_m_bench(torch, dev) if not args.no_extras else None
    heads_bf16 = bf16_heads_bench(torch, dev) if not args.no_extras else None
    pointwise_lines = pointwise_bench(torch, dev) if not args.no_extras else None
    prefill = prefill_bench(torch, dev) if not args.no_extras else None
    decode = decode_w4a8 = None
    if args.decode_steps > 0:
        decode = decode_step_bench(torch, args.decode_layers, args.decode_steps, dev)
        if not args.no_extras:
            decode_w4a8 = decode_step_bench(torch, args.decode_layers, args.decode_steps, dev, w4a8=True)

    cpu = None
    if not args.no_cpu_baseline:
        _log("[bench] CPU baseline (oracle, torch CPU) ...")
        cpu = cpu_baseline(torch, args.cpu_budget, *cpu_weights)
        _log(f"[bench] CPU baseline ({cpu['cpu_model']}): {cpu['ms_per_step']} ms/step on {cpu['cores']} threads "
             f"(dequant {cpu['dequant_ms']} ms, matmul {cpu['matmul_ms']} ms); {cpu['threads_4']['ms_per_step']} "
             f"ms/step on 4 threads")

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "decoder MLP, batch 1, INT4-G32 weights: RMSNorm(4096) + gate||up GEMV K=4096 "
                        "N=2x12288 with SiLU*mul epilogue + down GEMV K=12288 N=4096",
            "bytes_per_step": MLP_BYTES + NORM_BYTES,
            "algorithmic_bytes_counted": MLP_BYTES,
            "weight_copies": n_copies,
            "resident_weight_mib": round(resident / 2**20, 1),
            "weights": "N(0,0.02) fp32, min-max quantized per 32-input group on the GPU (seeded)",
            "activations": "bf16 N(0,1) through RMSNorm with weight 1+N(0,0.01)",
            "timing": f"HIP graphs of {cycle} steps rotating over the weight copies, HIP events on their stream",
            "parallelism": "single GPU",
        },
        "roofline": {
            "kernel": "w4g32_norm_gateup_silu_exact<2, 2, true> (RMSNorm + gate||up GEMV + SiLU*mul, one kernel)",
            "bound": "hbm",
            "achieved": round(gu_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
            "traffic": _traffic(),
            "algorithmic_bytes_per_launch": NORM_GATEUP_BYTES,
            "us_per_launch": round(gu_s * 1e6, 3),
        },
        "cpu_baseline": cpu,
        "extra": {
            "gemv_k4096_n12288": {"us_per_call": round(ns_s * 1e6, 3), "GB/s": round(ns_gbs, 1),
                                  "frac_of_peak": round(ns_gbs / HBM_PEAK_GBS, 4), "bytes": ns_bytes,
                                  "dequant": "exact", "vendor_streaming_read_same_bytes": read,
                                  "streaming_read_same_bytes": own_read},
            "gemv_k4096_size_sweep": size_sweep,
            "gemv_k4096_n12288_unrounded": {"us_per_call": round(ns_unr_s * 1e6, 3),
                                            "GB/s": round(ns_bytes / ns_unr_s / 1e9, 1),
                                            "frac_of_peak": round(ns_bytes / ns_unr_s / 1e9 / HBM_PEAK_GBS, 4)},
            "gateup_unrounded": {"us_per_call": round(gu_unr_s * 1e6, 3),
                                 "GB/s": round(NORM_GATEUP_BYTES / gu_unr_s / 1e9, 1)},
            "mlp_step_unrounded": {"us_per_step": round(unr_s * 1e6, 3), "GB/s": round(MLP_BYTES / unr_s / 1e9, 1)},
            "mlp_step_w4a8": {"us_per_step": round(w8_s * 1e6, 3), "GB/s": round(MLP_BYTES / w8_s / 1e9, 1),
                              "arithmetic": "int8 activations per 32-group, integer dot, fp32 group combine"},
            "gemv_down_k12288_n4096": {"us_per_call": round(dn_s * 1e6, 3),
                                       "GB/s": round(DOWN_BYTES / dn_s / 1e9, 1)},
            "wall_s_timed_region": round(wall, 4),
            "decode_step": decode,
            "decode_step_w4a8": decode_w4a8,
            "fp8": fp8_lines,
            "int4_small_m": small_m,
            "bf16_heads_k4096_n32770": heads_bf16,
            "pointwise_512_tokens": pointwise_lines,
            "prefill_gemm": prefill,
        },
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
