#!/usr/bin/env python3
"""Benchmark of the MI355X polynomial transcendental kernels (one GPU).

Headline workload ("B1 dense SiLU, FP16"): the
degree-3 polynomial SiLU forward on Llama-8B MLP gate activations
[8192 tokens, 14336] drawn N(0, 2^2), resident in HBM.  One step = one pass
of the kernel over the whole tensor.  `value` is Gelem/s over the K timed
steps.  Alongside it the JSON line carries

* `roofline`: algorithmic bytes (2 B read + 2 B written per element) per
  launch / average kernel time (HIP events on the launch stream) against the
  8 TB/s HBM peak, and the HBM traffic per launch measured by rocprofv3
  counters when a committed profile holds it;
* `cpu_baseline`: the CPU oracle (a C restatement of the same program, all
  host threads) timed on a bounded sample of the same tensor;
* `copy_ceiling`: the same one-pass driver copying the same tensor, the
  achievable ceiling of a 1-read/1-write stream of that size;
* `functions`: the per-function sweep, polynomial vs native vs copy, over
  2^16..2^28 elements (L2, MALL and HBM regimes; graph replay, median of 9
  rounds, implementations interleaved), every BASELINE configuration, and
  the sin/cos repeated-evaluation probes (the compute-bound regime, where
  Gevals/s is the issue rate of each program), and the fused attention
  forward at the reference's B2/B3/B5 component shape, polynomial score
  programs against hardware transcendentals (TFLOP/s vs the BF16 MFMA peak).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-sweep]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "fast-polynomial-transcendentals_amd", "python"))

HBM_PEAK_GBS = 8000.0
METRIC = "Gelem/s + % HBM roofline per function, poly vs native, L2 and HBM, 1 MI355X"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--no-sweep", action="store_true")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--sweep-reps", type=int, default=100)
    p.add_argument("--pmc-pass", action="store_true",
                   help="counter pass: 3 launches of the headline kernel and 3 plain "
                        "256 MiB copies (torch copy_) as the byte-count calibration")
    p.add_argument("--pmc-probes", action="store_true",
                   help="counter pass over the sin/cos repeated-evaluation probes: each "
                        "polynomial and native probe of the bench launched 4 times")
    p.add_argument("--pmc-attention", action="store_true",
                   help="counter pass over the attention forward: each score mode at the "
                        "component shape launched 3 times")
    p.add_argument("--attention-only", action="store_true",
                   help="time only the attention forward rows")
    p.add_argument("--open-weights", action="store_true",
                   help="model-level rows: prefill of randomly initialised Transformers models "
                        "(Llama-3-8B dims, GLM-4 MoE-lite dims, Gemma2 with head_dim 128; 2 layers) "
                        "unpatched and patched with each sfu_repro.open_weights family")
    p.add_argument("--pmc-sweep", action="store_true",
                   help="issue-rate counter pass: 3 eager launches of each polynomial, "
                        "native and copy kernel of the sweep at 2^20, 2^22 and 2^24 "
                        "elements (L2- and MALL-resident sizes)")
    return p.parse_args()


def _capi():
    import ctypes

    import torch  # noqa: F401  (HIP runtime first)

    lib = ctypes.CDLL(os.path.join(ROOT, "fast-polynomial-transcendentals_amd", "python",
                                   "libspline_hip.so"))
    return lib


def time_launches(launch, reps: int, warmup: int):
    """Average ms per launch over `reps` back-to-back launches, HIP events on
    the launch stream (torch's current stream)."""
    import torch

    for _ in range(warmup):
        launch()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        launch()
    stop.record()
    stop.synchronize()
    return start.elapsed_time(stop) / reps


def _graph(launch, reps: int):
    """`reps` launches captured in one HIP graph (replay removes the host
    launch cost that dominates small, L2-resident kernels)."""
    import torch

    launch()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            launch()
    g.replay()
    torch.cuda.synchronize()
    return g


def _replay_ms(g, reps: int):
    import torch

    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    g.replay()
    stop.record()
    stop.synchronize()
    return start.elapsed_time(stop) / reps


def time_graph(launch, reps: int, rounds: int = 9):
    """Average ms per launch of a captured graph of `reps` launches; median
    over `rounds` replays."""
    g = _graph(launch, reps)
    times = sorted(_replay_ms(g, reps) for _ in range(rounds))
    del g
    return times[len(times) // 2]


def time_graphs_alternating(launches, reps: int, rounds: int = 9):
    """Like time_graph for several launches at once, replaying them in
    alternating order within each round (the paper's protocol: median of 9
    rounds, implementations interleaved) so that clock or thermal drift
    does not favour one of them."""
    graphs = [_graph(fn, reps) for fn in launches]
    per = [[] for _ in launches]
    for r in range(rounds):
        order = range(len(graphs)) if r % 2 == 0 else reversed(range(len(graphs)))
        for i in order:
            per[i].append(_replay_ms(graphs[i], reps))
    del graphs
    return [sorted(t)[len(t) // 2] for t in per]


def make_unary(lib, name, out, x):
    import ctypes

    import torch

    fn = getattr(lib, name)
    fn.restype = ctypes.c_int
    args = (ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(x.data_ptr()),
            ctypes.c_int64(x.numel()))

    def launch():
        rc = fn(*args, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        if rc != 0:
            raise RuntimeError(f"{name} failed with {rc}")

    # the closure holds raw device pointers: keep the tensors alive with it
    # (graph capture empties torch's allocator cache, which unmaps freed memory)
    launch.tensors = (out, x)
    return launch


def read_traffic(kernel_tag: str):
    """HBM bytes per launch from the committed rocprofv3 counter summary."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(kernel_tag)
    except (OSError, ValueError):
        return None


def cpu_baseline(x_cpu_fp16, target_s: float = 10.0):
    """Oracle (C restatement, OpenMP) on a bounded sample of the workload."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc  # CPU baseline leg only

    sample = x_cpu_fp16.reshape(-1)[: 1 << 24].contiguous()
    bits = sample.view(__import__("torch").int16).numpy().view(np.uint16)
    orc.activation("swish", orc.FWD, 3, "f16", bits[:4096])  # load + warm
    done, t0 = 0, time.perf_counter()
    while True:
        orc.activation("swish", orc.FWD, 3, "f16", bits)
        done += bits.size
        el = time.perf_counter() - t0
        if el >= target_s:
            break
    return {
        "value": done / el / 1e9,
        "unit": "Gelem/s",
        "cores": orc.num_threads(),
        "kind": "port",
        "sample": (f"SiLU D3 FP16 oracle on the first 2^24 elements of the [8192,14336] N(0,2^2) "
                   f"tensor, {done // bits.size} passes in {el:.1f} s"),
    }


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_torch_native(x_cpu_fp16, target_s: float = 3.0):
    """Informational second CPU baseline: torch's FP32 SiLU on the host's
    threads over the same 2^24-element sample (not the program the GPU
    runs; the oracle above is)."""
    import torch

    xs = x_cpu_fp16.reshape(-1)[: 1 << 24].float()
    torch.nn.functional.silu(xs[:4096])
    done, t0 = 0, time.perf_counter()
    while True:
        torch.nn.functional.silu(xs).half()
        done += xs.numel()
        el = time.perf_counter() - t0
        if el >= target_s:
            break
    return {"value": done / el / 1e9, "unit": "Gelem/s", "threads": torch.get_num_threads(),
            "host": {"cpu_model": _cpu_model(), "nproc": os.cpu_count()},
            "sample": "torch.nn.functional.silu FP32 -> FP16 on the same 2^24-element sample"}


SWEEP_LOG2 = (16, 18, 20, 22, 24, 26, 28)


def _regime(n_log2: int) -> str:
    # aggregate L2 is 8 x 4 MB; the MALL is 256 MB
    return "l2" if n_log2 <= 21 else ("mall" if n_log2 <= 25 else "hbm")


def sweep(lib, reps: int):
    """Per-function polynomial vs native timing over 2^16..2^28 elements
    (L2-resident, MALL-resident, HBM), each size with the copy ceiling of the
    same driver, then the BASELINE configurations."""
    import torch

    out = []
    dev = torch.device("cuda:0")
    for n_log2 in SWEEP_LOG2:
        n = 1 << n_log2
        r = reps if n_log2 < 26 else max(5, reps // 5)
        g = torch.Generator(device=dev).manual_seed(n_log2)
        for dtype, sfx in ((torch.float16, ""), (torch.bfloat16, "_bf16")):
            x = (torch.randn(n, device=dev, generator=g) * 2.0).to(dtype)
            y = torch.empty_like(x)
            (copy_ms,) = time_graphs_alternating([make_unary(lib, "spline_hip_copy16", y, x)], r)
            for fam, deg in (("sigmoid", 3), ("tanh", 4), ("swish", 3)):
                row = {"function": f"{fam}_fwd", "dtype": "fp16" if not sfx else "bf16",
                       "degree": deg, "elements": n, "regime": _regime(n_log2)}
                poly_ms, nat_ms = time_graphs_alternating(
                    [make_unary(lib, f"launch_{fam}_fwd_d{deg}_kernel{sfx}", y, x),
                     make_unary(lib, f"launch_{fam}_fwd_native_kernel{sfx}", y, x)], r)
                for label, ms in (("poly", poly_ms), ("native", nat_ms), ("copy", copy_ms)):
                    row[f"{label}_us"] = round(ms * 1e3, 3)
                    row[f"{label}_gbs"] = round(4 * n / ms / 1e6, 1)
                row["poly_gelem_s"] = round(n / poly_ms / 1e6, 2)
                row["native_gelem_s"] = round(n / nat_ms / 1e6, 2)
                row["poly_frac_hbm_peak"] = round(row["poly_gbs"] / HBM_PEAK_GBS, 4)
                row["poly_frac_copy"] = round(copy_ms / poly_ms, 4)
                row["speedup"] = round(nat_ms / poly_ms, 3)
                out.append(row)
            del x, y
        torch.cuda.empty_cache()
    out.extend(config_rows(lib, reps))
    out.extend(probe_rows(lib, reps))
    out.extend(attention_rows(lib, reps))
    return out


MFMA_BF16_PEAK_TFLOPS = 2500.0
# B, Hq, Hkv, S, D: the reference's component shape, and its Llama 1B
# training model's attention (head_dim 64)
ATTN_SHAPES = ((1, 32, 8, 4096, 128), (1, 32, 8, 4096, 64))


def attention_rows(lib, reps: int, eager_launches: int = 0):
    rows = []
    for shape in ATTN_SHAPES:
        rows.extend(attention_rows_at(lib, reps, shape, eager_launches))
    return rows


def attention_rows_at(lib, reps: int, shape, eager_launches: int = 0):
    """The attention programs inside the fused forward and backward at the
    reference's component shape (causal GQA, B=1, S=4096, Hq=32, Hkv=8,
    D=128; and D=64, its Llama 1B training model's head size): B5 softmax with the D2 / D3 exp2 (every exponent, and the B5
    schedule: four of every 12 forward, 32 backward) against hardware exp2,
    B2 softcap 30 with the D4 tanh (analytical backward) against hardware
    tanh, B3 sigmoid attention with the direct D3 / D4 programs against
    hardware exp/rcp.  Causal FLOPs: forward 4 B Hq S^2 D / 2 (two products
    over the lower triangle), backward 2.5x that (five products, the usual
    FlashAttention count; the kernels recompute S and dP once more, so they
    issue 7/5 of it).  The bound is the dense BF16 MFMA peak.  With
    eager_launches > 0 each case is only launched that many times (a counter
    pass) and nothing is timed."""
    import ctypes
    import math

    import torch

    dev = torch.device("cuda:0")
    b, hq, hkv, s, d = shape
    g = torch.Generator(device=dev).manual_seed(30)
    q = torch.randn(b, hq, s, d, device=dev, generator=g).bfloat16()
    k = torch.randn(b, hkv, s, d, device=dev, generator=g).bfloat16()
    v = torch.randn(b, hkv, s, d, device=dev, generator=g).bfloat16()
    do = torch.randn(b, hq, s, d, device=dev, generator=g).bfloat16()
    # scores spread as after QK-norm with a learnt scale: s = q.k / sqrt(d) * 4
    qs = (q.float() * 4).bfloat16()
    o = torch.empty_like(q)
    scale = 1.0 / math.sqrt(d)
    flops = 4 * b * hq * s * s * d / 2
    sigmoid_bias = -math.log(s)

    def strides(*ts):
        vals = []
        for t in ts:  # [B, H, S, D]: (batch, head, sequence)
            vals += [t.stride(0), t.stride(1), t.stride(2)]
        return (ctypes.c_int64 * len(vals))(*vals)

    def fa(mode, qq, route=4, out=o, lse=None):
        lse_arg = lse if lse is not None else ctypes.c_void_p(0)
        return _launcher(lib, "launch_flash_attention_fwd_strided_bf16", out, lse_arg, qq, k, v, b, hq, hkv, s,
                         d, strides(qq, k, v, out), ctypes.c_int(mode), ctypes.c_int(route), ctypes.c_int(1),
                         ctypes.c_float(scale), ctypes.c_float(30.0), ctypes.c_float(sigmoid_bias))

    def fa_bwd(mode, grad, qq, route_fwd=4, route_bwd=0):
        # out and lse of the same forward, then the backward on them
        out = torch.empty_like(qq)
        lse = torch.zeros(b, hq, s, dtype=torch.float32, device=dev)
        fa(mode, qq, route_fwd, out, lse)()
        torch.cuda.synchronize()
        dq, dk, dv = torch.empty_like(qq), torch.empty_like(k), torch.empty_like(v)
        delta = torch.empty(b, hq, s, dtype=torch.float32, device=dev)
        ws = torch.empty(2, b, hq, s, d, dtype=torch.float32, device=dev)
        return _launcher(lib, "launch_flash_attention_bwd_strided_bf16", dq, dk, dv, delta, ws, qq, k, v, out, do,
                         lse, b, hq, hkv, s, d, strides(qq, k, v, out, do, dq, dk, dv), ctypes.c_int(mode),
                         ctypes.c_int(grad), ctypes.c_int(route_bwd), ctypes.c_int(1), ctypes.c_float(scale),
                         ctypes.c_float(30.0), ctypes.c_float(sigmoid_bias))

    groups = [("fwd", "B5 softmax exp2", flops,
               [("poly_d2", fa(1, q)), ("poly_d3", fa(2, q)), ("poly_d2_route12", fa(1, q, 12)),
                ("native", fa(0, q))]),
              ("fwd", "B2 softcap 30", flops, [("poly_d4", fa(4, qs)), ("native", fa(3, qs))]),
              ("fwd", "B3 sigmoid attention", flops, [("poly_b3", fa(6, q)), ("native", fa(5, q))]),
              ("bwd", "B5 softmax exp2", 2.5 * flops,
               [("poly_d2_route32", fa_bwd(1, 0, q, 12, 32)), ("native", fa_bwd(0, 0, q))]),
              ("bwd", "B2 softcap 30", 2.5 * flops,
               [("poly_d4_analytical", fa_bwd(4, 1, qs)), ("native", fa_bwd(3, 0, qs))]),
              ("bwd", "B3 sigmoid attention", 2.5 * flops,
               [("poly_b3_direct", fa_bwd(6, 5, q)), ("native", fa_bwd(5, 0, q))])]
    rows = []
    for direction, function, fl, launches in groups:
        if eager_launches:
            for _, fn in launches:
                for _ in range(eager_launches):
                    fn()
            torch.cuda.synchronize()
            continue
        times = time_graphs_alternating([fn for _, fn in launches], max(5, reps // 10))
        row = {"function": f"attention_{direction} {function}", "dtype": "bf16",
               "config": f"causal GQA B={b} S={s} Hq={hq} Hkv={hkv} D={d}", "flops": fl}
        for (label, _), ms in zip(launches, times):
            row[f"{label}_us"] = round(ms * 1e3, 2)
            row[f"{label}_tflops"] = round(fl / ms / 1e9, 1)
            row[f"{label}_frac_mfma_peak"] = round(fl / ms / 1e9 / MFMA_BF16_PEAK_TFLOPS, 4)
        for label, _ in launches[:-1]:
            row[f"{label}_speedup"] = round(row["native_us"] / row[f"{label}_us"], 3)
        rows.append(row)
    return rows


def open_weights_rows(seq_len: int = 2048, steps: int = 5):
    """Prefill (one forward of `seq_len` tokens, batch 1, BF16) of randomly
    initialised 2-layer models at the dims of the reference's open-weight
    models, unpatched ("native") and with each patch family of
    sfu_repro.open_weights (scripts/benchmark_open_weights.py's protocol:
    CUDA events around model(...), mean of `steps` after 2 warm-ups).
    Gemma2 "native" is the eager attention; the fused-attention variants
    replace it with the fused kernel, so they also change the attention
    algorithm (noted in the row)."""
    import torch

    from sfu_repro import open_weights as ow

    dev = torch.device("cuda:0")
    cases = [
        ("llama3-8b-2l", None, ["native", "spline_silu_d3_current", "fused_swiglu_d3_current"]),
        ("glm4-moe-lite-2l", "batched_mm",
         ["native", "fused_swiglu_d3_current", "spline_router_sigmoid_d3_current"]),
        ("gemma2-d128-2l", None, ["native", "gemma_tanh_current", "gemma_fa4_tanh_native",
                                  "gemma_fa4_tanh_d4_current"]),
    ]
    rows = []
    for preset, experts, variants in cases:
        model = ow.build_model(preset, dtype=torch.bfloat16, device=dev, experts_implementation=experts)
        slots = ow.collect_slots(model)
        tokens = ow.make_tokens(batch_size=1, seq_len=seq_len,
                                vocab_size=int(model.get_input_embeddings().num_embeddings), device=dev, seed=0)
        row = {"model": preset, "config": f"batch 1, {seq_len} tokens, BF16, random weights, 2 layers"}
        for variant in variants:
            res = ow.run_variant(model, slots, ow.parse_variant(variant), tokens, model_id=preset, mode="prefill",
                                 warmup=2, steps=steps, decode_steps=0, seed=0)
            row[f"{variant}_ms"] = round(res.prefill_ms, 3)
            row[f"{variant}_tokens_s"] = round(res.prefill_tokens_per_s, 1)
        ow.restore_gemma_attention()
        base = row["native_ms"]
        for variant in variants[1:]:
            row[f"{variant}_speedup"] = round(base / row[f"{variant}_ms"], 3)
        rows.append(row)
        del model, slots
        torch.cuda.empty_cache()
    return rows


PROBE_ITERS = 32


def probe_rows(lib, reps: int, eager_launches: int = 0):
    """Issue-rate comparison in the compute-bound regime: the reference's
    repeated-evaluation sin/cos probes (sincos_compute_*, rope_*_compute),
    polynomial vs hardware v_sin/v_cos, on 2^22 RoPE-sized angles (enough
    threads for every SIMD to hold 8 waves) with 32 evaluations each.  The
    loads and stores are negligible, so Gevals/s is the instruction issue
    rate of each program.  With eager_launches > 0 each probe is only
    launched that many times (a counter pass) and nothing is timed."""
    import torch

    dev = torch.device("cuda:0")
    n = 1 << 22
    g = torch.Generator(device=dev).manual_seed(20)
    a = torch.rand(n, device=dev, generator=g) * 200 - 100
    rows = []
    groups = [
        ("sincos_compute_f32", torch.float32,
         [("poly_d3_d4", "launch_sincos_d3_d4_compute_f32"), ("poly_d7_d6", "launch_sincos_d7_d6_compute_f32"),
          ("native", "launch_sincos_native_compute_f32")]),
        ("sincos_compute_fp16", torch.float16,
         [("poly_d3_d4", "launch_sincos_d3_d4_half_turn_fp16_compute"),
          ("poly_d5_d6", "launch_sincos_d5_d6_half_turn_fp16_compute"),
          ("native", "launch_sincos_native_fp16_compute")]),
        ("sincos_compute_bf16", torch.bfloat16,
         [("poly_d3_d4", "launch_sincos_d3_d4_half_turn_bf16_compute"),
          ("poly_d5_d6", "launch_sincos_d5_d6_half_turn_bf16_compute"),
          ("native", "launch_sincos_native_bf16_compute")]),
    ]
    for function, dt, impls in groups:
        out = torch.empty(2, n, dtype=dt, device=dev)
        launches = [(label, _launcher(lib, name, out, a, n, PROBE_ITERS)) for label, name in impls]
        if eager_launches:
            for _, fn in launches:
                for _ in range(eager_launches):
                    fn()
            torch.cuda.synchronize()
            continue
        times = time_graphs_alternating([fn for _, fn in launches], max(5, reps // 10))
        row = {"function": function, "config": f"2^22 angles U[-100,100], {PROBE_ITERS} evaluations each",
               "evaluations": n * PROBE_ITERS}
        for (label, _), ms in zip(launches, times):
            row[f"{label}_us"] = round(ms * 1e3, 2)
            row[f"{label}_gevals_s"] = round(n * PROBE_ITERS / ms / 1e6, 1)
        for label, _ in launches[:-1]:
            row[f"{label}_speedup"] = round(row["native_us"] / row[f"{label}_us"], 3)
        rows.append(row)
        del out
    # RoPE tables: positions 0..4095 x 64 frequencies, 16 positions summed per entry
    import math

    seq, d, it = 4096, 128, 16
    dims = torch.arange(0, d, 2, dtype=torch.float64)
    freq = 500000.0 ** (-dims / d)
    inc = torch.round(freq * (2.0 ** 32) / (2 * math.pi)).to(torch.int64).to(torch.int32).to(dev)
    fr = freq.float().to(dev)
    out = torch.empty(2, seq, d // 2, dtype=torch.float16, device=dev)
    launches = [("poly_half_d5_d6", _launcher(lib, "launch_rope_sincos_fixed_half_turn_d5_d6_fp16_compute",
                                              out, inc, seq, d // 2, it)),
                ("poly_quarter_d3_d4", _launcher(lib, "launch_rope_sincos_fixed_d3_d4_fp16_compute",
                                                 out, inc, seq, d // 2, it)),
                ("native", _launcher(lib, "launch_rope_sincos_native_fp16_compute", out, fr, seq, d // 2, it))]
    if eager_launches:
        for _, fn in launches:
            for _ in range(eager_launches):
                fn()
        torch.cuda.synchronize()
        return rows
    times = time_graphs_alternating([fn for _, fn in launches], max(5, reps // 10))
    ev = seq * (d // 2) * it
    row = {"function": "rope_sincos_compute_fp16", "config": f"S={seq}, F={d // 2}, theta=5e5, {it} positions each",
           "evaluations": ev}
    for (label, _), ms in zip(launches, times):
        row[f"{label}_us"] = round(ms * 1e3, 2)
        row[f"{label}_gevals_s"] = round(ev / ms / 1e6, 1)
    for label, _ in launches[:-1]:
        row[f"{label}_speedup"] = round(row["native_us"] / row[f"{label}_us"], 3)
    rows.append(row)
    return rows


PMC_SWEEP_LOG2 = (20, 22, 24)


def pmc_sweep(lib):
    """Counter pass for the cache-resident regimes: every kernel of the sweep
    launched 3 times, eagerly, after one warm launch of the same size (so
    the input sits in L2 / MALL as in back-to-back timing).  Prints the
    launch plan; rocprofv3 attributes counters by kernel name and grid
    size."""
    import torch

    dev = torch.device("cuda:0")
    plan = []
    for n_log2 in PMC_SWEEP_LOG2:
        n = 1 << n_log2
        g = torch.Generator(device=dev).manual_seed(n_log2)
        for dtype, sfx in ((torch.float16, ""), (torch.bfloat16, "_bf16")):
            x = (torch.randn(n, device=dev, generator=g) * 2.0).to(dtype)
            y = torch.empty_like(x)
            names = ["spline_hip_copy16"]
            for fam, deg in (("sigmoid", 3), ("tanh", 4), ("swish", 3)):
                names += [f"launch_{fam}_fwd_d{deg}_kernel{sfx}", f"launch_{fam}_fwd_native_kernel{sfx}"]
            for name in names:
                launch = make_unary(lib, name, y, x)
                launch()
                torch.cuda.synchronize()
                for _ in range(3):
                    launch()
                torch.cuda.synchronize()
                plan.append({"entry": name, "elements": n, "launches": 4})
            del x, y
    print(json.dumps({"pmc_sweep": plan}), flush=True)


def _vp(t):
    import ctypes

    return ctypes.c_void_p(t.data_ptr())


def _launcher(lib, name, *args):
    """Launch closure for a C-ABI entry point on torch's current stream."""
    import ctypes

    import torch

    fn = getattr(lib, name)
    fn.restype = ctypes.c_int
    conv = []
    for a in args:
        if isinstance(a, (ctypes._SimpleCData, ctypes.Array)):
            conv.append(a)
        elif isinstance(a, torch.Tensor):
            conv.append(_vp(a))
        elif isinstance(a, float):
            conv.append(ctypes.c_float(a))
        else:
            conv.append(ctypes.c_int64(a))

    def launch():
        rc = fn(*conv, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        if rc != 0:
            raise RuntimeError(f"{name} failed with {rc}")

    # the closure holds raw device pointers: keep the tensors alive with it
    # (graph capture empties torch's allocator cache, which unmaps freed memory)
    launch.tensors = tuple(a for a in args if isinstance(a, torch.Tensor))
    return launch


def _row(function, config, dtype, elements, alg_bytes, launches, reps):
    """Time each (label, launch) and report us, Gelem/s, GB/s, HBM fraction."""
    row = {"function": function, "config": config, "dtype": dtype, "elements": elements,
           "bytes_per_launch": alg_bytes}
    times = time_graphs_alternating([fn for _, fn in launches], reps)
    for (label, _), ms in zip(launches, times):
        row[f"{label}_us"] = round(ms * 1e3, 3)
        row[f"{label}_gelem_s"] = round(elements / ms / 1e6, 2)
        row[f"{label}_gbs"] = round(alg_bytes / ms / 1e6, 1)
    if "poly_gbs" in row:
        row["poly_frac_hbm_peak"] = round(row["poly_gbs"] / HBM_PEAK_GBS, 4)
    if "native_us" in row and "poly_us" in row:
        row["speedup"] = round(row["native_us"] / row["poly_us"], 3)
    return row


def config_rows(lib, reps: int):
    """The BASELINE.json configurations, polynomial vs native where a native
    baseline exists.  Synthetic inputs follow each config's recipe."""
    import math

    import numpy as np
    import torch

    dev = torch.device("cuda:0")
    rows = []
    big = max(5, reps // 5)

    # C0 / B3: 2^20 BF16 scores U[-16, 16], seed 0 -> y, dy.
    g = torch.Generator().manual_seed(0)
    s = (torch.rand(1 << 20, generator=g) * 32 - 16).to(torch.bfloat16).to(dev)
    y, dy = torch.empty_like(s), torch.empty_like(s)
    rows.append(_row("b3_direct_d3_d4", "C0 B3 2^20 U[-16,16]", "bf16", s.numel(), 6 * s.numel(),
                     [("poly", _launcher(lib, "launch_flash_sigmoid_direct_d3_d4_bf16", y, dy, s,
                                         s.numel()))], reps))
    rows.append(_row("b3_exp2_d2", "C0 B3-D2 2^20 U[-16,16]", "bf16", s.numel(), 6 * s.numel(),
                     [("poly", _launcher(lib, "launch_flash_sigmoid_exp2_d2_bf16", y, dy, s,
                                         s.numel()))], reps))
    del s, y, dy

    # C1 / B1 L2-resident variant [256, 4096] FP16 N(0, 2^2).
    x = (torch.randn(256, 4096, generator=g) * 2).half().to(dev)
    yy = torch.empty_like(x)
    rows.append(_row("swish_fwd_d3", "C1 B1 L2 [256,4096]", "fp16", x.numel(), 4 * x.numel(),
                     [("poly", _launcher(lib, "launch_swish_fwd_d3_kernel", yy, x, x.numel())),
                      ("native", _launcher(lib, "launch_swish_fwd_native_kernel", yy, x, x.numel()))],
                     reps))
    del x, yy

    # C3 / B2: softcap cap=30 on BF16 [4, 32, 2048, 2048], N(0, 15^2), 1 % +-200.
    gd = torch.Generator(device=dev).manual_seed(3)
    sc = torch.randn(4, 32, 2048, 2048, device=dev, generator=gd) * 15
    mask = torch.rand(sc.shape, device=dev, generator=gd) < 0.01
    sign = torch.where(torch.rand(sc.shape, device=dev, generator=gd) < 0.5, -200.0, 200.0)
    sc = torch.where(mask, sign, sc).to(torch.bfloat16)
    del mask, sign
    torch.cuda.empty_cache()
    out = torch.empty_like(sc)
    n = sc.numel()
    rows.append(_row("softcap_tanh_d4", "C3 B2 [4,32,2048,2048] cap=30", "bf16", n, 4 * n,
                     [("poly", _launcher(lib, "launch_softcap_tanh_d4_bf16", out, sc, n, 30.0)),
                      ("native", _launcher(lib, "launch_softcap_tanh_native_bf16", out, sc, n, 30.0))],
                     big))
    del sc, out
    torch.cuda.empty_cache()

    # C4 / B4: routed SwiGLU, 64 experts x 128 tokens (Zipf(1.1) ragged counts),
    # hidden 2048, N(0, 1).  The activation is elementwise over [sum(counts), H].
    p = np.arange(1, 65, dtype=np.float64) ** -1.1
    counts = np.random.default_rng(0).multinomial(64 * 128, p / p.sum())
    rows_total, h = int(counts.sum()), 2048
    gate = torch.randn(rows_total, h, device=dev, generator=gd).bfloat16()
    up = torch.randn(rows_total, h, device=dev, generator=gd).bfloat16()
    go = torch.randn(rows_total, h, device=dev, generator=gd).bfloat16()
    o, gg, gu = torch.empty_like(gate), torch.empty_like(gate), torch.empty_like(gate)
    n = gate.numel()
    cfg = f"C4 B4 experts=64 rows={rows_total} (max expert {int(counts.max())}) H=2048"
    rows.append(_row("swish_mul_fwd_d3", cfg, "bf16", n, 6 * n,
                     [("poly", _launcher(lib, "launch_swish_mul_fwd_d3_kernel_bf16", o, gate, up, n)),
                      ("native", _launcher(lib, "launch_swish_mul_fwd_native_kernel_bf16", o, gate, up, n))],
                     reps))
    rows.append(_row("swish_mul_bwd_d3", cfg, "bf16", n, 10 * n,
                     [("poly", _launcher(lib, "launch_swish_mul_bwd_d3_kernel_bf16", gg, gu, go, gate, up, n)),
                      ("native", _launcher(lib, "launch_swish_mul_bwd_native_kernel_bf16", gg, gu, go, gate, up, n))],
                     reps))
    packed = torch.cat((gate, up), -1)
    gp = torch.empty_like(packed)
    rows.append(_row("swish_mul_packed_fwd_d3", cfg + " packed [rows,4096]", "bf16", n, 6 * n,
                     [("poly", _launcher(lib, "launch_swish_mul_packed_fwd_d3_kernel_bf16", o, packed, rows_total, h)),
                      ("native", _launcher(lib, "launch_swish_mul_packed_fwd_native_kernel_bf16", o, packed, rows_total, h))],
                     reps))
    rows.append(_row("swish_mul_packed_bwd_d3", cfg + " packed [rows,4096]", "bf16", n, 10 * n,
                     [("poly", _launcher(lib, "launch_swish_mul_packed_bwd_d3_kernel_bf16", gp, go, packed, rows_total, h)),
                      ("native", _launcher(lib, "launch_swish_mul_packed_bwd_native_kernel_bf16", gp, go, packed, rows_total, h))],
                     reps))
    del gate, up, go, o, gg, gu, packed, gp
    torch.cuda.empty_cache()

    # C5 / B5: exp2 on FP32 logits [4, 32, 4096, 128] N(0, 4^2) minus row max -> BF16.
    lg = torch.randn(4, 32, 4096, 128, device=dev, generator=gd) * 4
    lg = lg - lg.amax(-1, keepdim=True)
    e = torch.empty(lg.shape, dtype=torch.bfloat16, device=dev)
    n = lg.numel()
    rows.append(_row("exp2_d2", "C5 B5 [4,32,4096,128] FP32->BF16", "f32->bf16", n, 6 * n,
                     [("poly", _launcher(lib, "launch_exp2_d2_f32_bf16", e, lg, n)),
                      ("poly_d3", _launcher(lib, "launch_exp2_d3_f32_bf16", e, lg, n)),
                      ("native", _launcher(lib, "launch_exp2_native_f32_bf16", e, lg, n))],
                     big))
    del lg, e
    torch.cuda.empty_cache()

    # C5 / RoPE: BF16 Q, K [4, 4096, 32, 128], theta 500000, positions 0..4095.
    b, sl, hh, d = 4, 4096, 32, 128
    q = torch.randn(b, sl, hh, d, device=dev, generator=gd).bfloat16()
    k = torch.randn(b, sl, hh, d, device=dev, generator=gd).bfloat16()
    qo = torch.empty(b, hh, sl, d, dtype=torch.bfloat16, device=dev)
    ko = torch.empty_like(qo)
    dims = torch.arange(0, d, 2, dtype=torch.float64)
    freq = 500000.0 ** (-dims / d)
    inc = torch.round(freq * (2.0 ** 32) / (2 * math.pi)).to(torch.int64).to(torch.int32).to(dev)
    fr = freq.float().to(dev)
    n = q.numel() + k.numel()
    rows.append(_row("rope_apply_d5_d6", "C5 RoPE Q,K [4,4096,32,128] theta=5e5", "bf16", n, 4 * n,
                     [("poly", _launcher(lib, "launch_rope_apply_fixed_half_turn_d5_d6_bf16", qo, ko, q, k, inc, b, sl, hh, hh, d)),
                      ("native", _launcher(lib, "launch_rope_apply_native_bf16", qo, ko, q, k, fr, b, sl, hh, hh, d))],
                     big))
    del q, k, qo, ko
    torch.cuda.empty_cache()
    return rows


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the elementwise path needs no cross-GPU exchange: each GPU would run the same "
              "kernel on its own contiguous shard).",
              file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    lib = _capi()
    dev = torch.device("cuda:0")
    if args.pmc_sweep:
        pmc_sweep(lib)
        return
    if args.pmc_probes:
        probe_rows(lib, 40, eager_launches=4)
        return
    if args.pmc_attention:
        attention_rows(lib, 40, eager_launches=3)
        return
    if args.attention_only:
        print(json.dumps({"functions": attention_rows(lib, args.sweep_reps)}), flush=True)
        return
    if args.open_weights:
        print(json.dumps({"models": open_weights_rows()}), flush=True)
        return

    # Synthetic B1 gate activations [8192, 14336] ~ N(0, 2^2), FP16, in HBM.
    rows, cols = 8192, 14336
    g = torch.Generator(device="cpu").manual_seed(0)
    x_cpu = (torch.randn(rows, cols, generator=g) * 2.0).to(torch.float16)
    x = x_cpu.to(dev)
    y = torch.empty_like(x)
    n = x.numel()
    launch = make_unary(lib, "launch_swish_fwd_d3_kernel", y, x)

    if args.pmc_pass:
        src = torch.empty(1 << 27, dtype=torch.float16, device=dev).normal_()
        dst = torch.empty_like(src)
        for _ in range(3):
            launch()
        torch.cuda.synchronize()
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"pmc_pass": True, "kernel_elements": n,
                          "copy_bytes_read": src.numel() * 2, "copy_bytes_written": dst.numel() * 2}))
        return

    for _ in range(args.warmup):
        launch()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        launch()
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = start.elapsed_time(stop) / args.steps
    value = n / (ms_per_step * 1e-3) / 1e9

    achieved_gbs = 4.0 * n / (ms_per_step * 1e-3) / 1e9
    traffic = read_traffic("swish_fwd_d3_f16_b1")
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "Gelem/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic N(0,2^2) gate activations, seed 0",
        "config": {"workload": "B1 dense SiLU D3 forward, FP16 [8192,14336] (BASELINE config 1)",
                   "elements": n, "kernel": "launch_swish_fwd_d3_kernel"},
        "roofline": {"bound": "hbm", "achieved": round(achieved_gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic},
        "wall_s_timed": round(wall, 3),
    }
    # Achievable ceiling: the same driver copying the same tensor.
    copy_ms = time_launches(make_unary(lib, "spline_hip_copy16", y, x), args.steps, args.warmup)
    copy_gbs = 4.0 * n / (copy_ms * 1e-3) / 1e9
    line["copy_ceiling"] = {"achieved": round(copy_gbs, 1), "unit": "GB/s",
                            "frac_hbm_peak": round(copy_gbs / HBM_PEAK_GBS, 4),
                            "kernel_frac_of_copy": round(copy_ms / ms_per_step, 4)}
    del y
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(x_cpu)
        line["cpu_torch_native"] = cpu_torch_native(x_cpu)
    if not args.no_sweep:
        line["functions"] = sweep(lib, args.sweep_reps)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
