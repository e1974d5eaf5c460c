"""Benchmark: tessery's prefill attention path on one MI355X.

Default workload qwen3_32x512 (the headline): B=32 rows, log-uniform valid lengths in [1,512]
(seed 4), execution width 16*ceil(max L/16) = 464, 16 query / 8 KV heads, head dim 128, fp16
operands with fp32 accumulation, per-head q/k RMSNorm + RoPE fused, 28 layers with independent
inputs resident in HBM. One step = the 28 layers: per layer the k norm+RoPE prologue and the
attention (q norm+RoPE inside), queued through the C ABI (HipRuntime -> mi_dispatch); the k planes
alternate between two buffers, so the runtime runs each layer's attention with the next layer's
k prologue in extra workgroups of the same launch (27 of 28 prologues), bit for bit the separate
launches.

It prints one JSON line: tokens/s (execution tokens B*S*layers per second), mask-exact TFLOP/s and
its fraction of the fp16 MFMA peak, the HBM roofline of the attention kernel from live per-launch
HIP-event timings, and the NumPy CPU oracle timed on the host on a bounded sample (float64 on all
cores, plus float32 and a one-thread float64 run). Layer 0 is checked against the float64 oracle
(max-abs <= 1e-4 with fp32 output; the exit status is 1 otherwise). A `secondary` object carries
kernel times and roofline fractions of the other configurations measured in the same run:
bge_32x512, qwen3_8x512 (fused and fp32 routes), qwen_qkv4_16x256 and the headline shape at full
length with fp16 output.

--workload selects one of the other measured configurations instead (one JSON line each):
  qwen3_8x512       B=8, S=512, lengths U{64..512} (seed 3), same fused path, 8 layers
  qwen3_32x512_full B=32, S=512, every length 512, the same fused path with fp16 output, 8 layers
  qwen3_8x512_f32   the same shape on the fp32 route (attention_tiled, D=128), 8 layers
  bge_32x512        BGE-small fp32 bidirectional attention, B=32, S=512, 12 heads x 32,
                    lengths U{2..512} (seed 2), 12 layers, route attention_tiled
  qwen_qkv4_16x256  uint4 QKV projection (x [4096,1024] fp16) -> k norm+RoPE -> fused attention,
                    lengths U{1..256} (seed 5), 8 layers
  qwen_tail_16x256  the rest of the Qwen3 layer on 4096 tokens, fp32 activations: o_proj ->
                    residual -> RMSNorm -> gate/up + SiLU -> down -> residual, 4 layers
  qwen_tail_1x128   the same tail on one 128-token sequence (fused gated4 route, split-K)
  bge_layer_32x512  whole BGE-small encoder layers (fp32) on 32x512 tokens, lengths U{2..512}
                    (seed 2): projections + bias, attention, LayerNorms, GELU MLP, 4 layers
  bge_plan_1x128    a 12-layer BGE-small stack on one 128-token sequence replayed as a prepared
                    plan, with plan replays as cached HIP graphs and launched one by one
"""

from __future__ import annotations

import argparse
import hashlib
import json
import os
import sys
import time
from pathlib import Path
from typing import Any, Callable

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from tessery_amd import HipRuntime, workloads  # noqa: E402

METRIC = "prefill attention tokens/s + TFLOP/s (% MFMA peak), Qwen3 GQA 32x512, 1 GPU"
PEAK_F16_TFLOPS = 2516.6
PEAK_F32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
LAYERS = 28
# max-abs parity bars of the fused route against the float64 oracle, layer 0
PARITY_F32_OUT = 1e-4
PARITY_F16_OUT = 2e-3
# rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of the attention kernel on this workload, with the
# copy-kernel calibration of each counter; valid for the kernel source it names
TRAFFIC_FILE = ROOT / "profiles" / "attention_f16_norm_rope_qwen3_32x512_traffic.txt"
KERNEL_SOURCE = ROOT / "tessery_amd" / "csrc" / "attention.hip"


def log(message: str) -> None:
    print(message, file=sys.stderr, flush=True)


def measured_traffic() -> int | None:
    """HBM bytes per attention launch from the committed counter summary, or None when it is
    missing or was measured on a different kernel source."""
    if not TRAFFIC_FILE.is_file():
        return None
    fields = {}
    for line in TRAFFIC_FILE.read_text().splitlines():
        key, sep, value = line.partition(":")
        if sep:
            fields[key.strip()] = value.strip()
    try:
        source = hashlib.sha256(KERNEL_SOURCE.read_bytes()).hexdigest()
        if fields.get("attention.hip sha256") != source:
            log("traffic summary was measured on another kernel source; traffic = null")
            return None
        fetch = float(fields["FETCH_SIZE KiB per dispatch"]) * float(fields["FETCH_SIZE factor"])
        write = float(fields["WRITE_SIZE KiB per dispatch"]) * float(fields["WRITE_SIZE factor"])
    except (KeyError, ValueError, OSError):
        return None
    return int(round((fetch + write) * 1024))


def blas_threads() -> int:
    try:
        from threadpoolctl import threadpool_info

        return max((i.get("num_threads", 0) for i in threadpool_info()), default=0)
    except Exception:  # threadpoolctl missing: report unknown
        return 0


def time_cpu(layer: Callable[[], Any], budget_s: float = 12.0) -> tuple[Any, float, int]:
    """Run `layer` once as warmup (its result is returned as the parity reference), then time up
    to 5 more runs within budget_s; returns (result, median seconds, runs timed)."""
    start = time.perf_counter()
    expected = layer()
    times = [time.perf_counter() - start]
    while sum(times) < budget_s and len(times) < 6:
        t0 = time.perf_counter()
        layer()
        times.append(time.perf_counter() - t0)
    return expected, float(np.median(times[1:] if len(times) > 1 else times)), max(1, len(times) - 1)


def run_timed(rt: HipRuntime, step: Callable[[], None], steps: int, warmup: int,
              launches_per_step: int, profile: bool = True) -> dict[str, Any]:
    """Warmup, then K steps launched back to back inside one command (synchronized before and
    after), then (profile) the same steps replayed with HIP events around every launch on the
    runtime stream (a command profiles at most 2048 launches). Returns wall seconds per step,
    event seconds per step and the per-kernel mean launch durations."""
    for _ in range(warmup):
        with rt.command():
            step()
    with rt.command():
        for _ in range(steps):
            step()
        launched = time.perf_counter()
    wall = time.perf_counter() - launched
    gpu = rt.last_gpu_seconds
    log(f"timed {steps} steps: wall {wall * 1e3:.3f} ms, events {gpu * 1e3:.3f} ms")
    if not profile:
        return {"step": wall / steps, "gpu_step": gpu / steps if gpu >= 0 else None, "kernel_s": {}}
    prof_steps = max(1, min(steps, 2048 // launches_per_step))
    with rt.profile_kernels() as records:
        with rt.command():
            for _ in range(prof_steps):
                step()
    kernels: dict[str, list[float]] = {}
    fused: dict[str, str] = {}
    fused_count: dict[str, int] = {}
    for r in records:
        # a launch the runtime ran inside the previous op's kernel has no time of its own
        if "fused_into" in r:
            fused[r["kernel"]] = r["fused_into"]
            fused_count[r["kernel"]] = fused_count.get(r["kernel"], 0) + 1
        else:
            kernels.setdefault(r["kernel"], []).append(r["gpu_seconds"])
    return {
        "step": wall / steps,
        "gpu_step": gpu / steps if gpu >= 0 else None,
        "kernel_s": {k: float(np.mean(v)) for k, v in kernels.items()},
        "kernel_step_s": {k: float(np.sum(v)) / prof_steps for k, v in kernels.items()},
        "fused": {k: v for k, v in fused.items() if k not in kernels},
        "fused_per_step": {k: v / prof_steps for k, v in fused_count.items()},
    }


def kernel_us(t: dict[str, Any]) -> dict[str, Any]:
    """Mean launch durations in microseconds; a route that only ran fused into another kernel is
    listed with the kernel that carried it instead of a time."""
    out: dict[str, Any] = {k: v * 1e6 for k, v in t["kernel_s"].items()}
    out.update({k: {"fused_into": v} for k, v in t.get("fused", {}).items()})
    return out


def upload_qwen_layers(rt: HipRuntime, shape: workloads.Shape, layers: int, seed: int,
                       out_bytes: int = 4):
    sets = []
    for layer in range(layers):
        t = workloads.qwen_layer(shape, layer, seed=seed)
        sets.append(
            {
                "q": rt.upload(t["q"]),
                "k": rt.upload(t["k"]),
                "v": rt.upload(t["v"]),
                "q_norm": rt.upload(t["q_norm"]),
                "k_norm": rt.upload(t["k_norm"]),
                "out": rt.buffer(t["q"].size * out_bytes),
            }
        )
        if layer == 0:
            host0 = t
    return sets, host0


def fused_attention(rt, shape, s, lengths_buf, k_work, out_dtype="f32"):
    rt._attention_norm_rope(
        [s["q"], s["k"], s["v"], lengths_buf, s["out"], s["q_norm"], s["k_norm"], k_work],
        tokens=shape.tokens,
        seq=shape.seq,
        heads=shape.heads,
        kv_heads=shape.kv_heads,
        dim=shape.dim,
        eps=workloads.EPS,
        theta=workloads.THETA,
        out_dtype=out_dtype,
    )


def qwen_cpu_layer(shape, lengths, host0, dtype=np.float64, rows=None):
    """NumPy oracle of one layer (float64: the reference formulation; float32: a timing variant):
    q/k norm + RoPE, then attention, over all batch rows or the first `rows`."""
    from oracle import attention, norm_rope

    qn = workloads.bf16_values(host0["q_norm"]).astype(np.float64)
    kn = workloads.bf16_values(host0["k_norm"]).astype(np.float64)
    rows = shape.batch if rows is None else rows
    q_in, k_in, v_in = (host0[name][:rows] for name in ("q", "k", "v"))

    def layer():
        q = norm_rope.norm_rope(q_in, qn, workloads.EPS, workloads.THETA, dtype)
        k = norm_rope.norm_rope(k_in, kn, workloads.EPS, workloads.THETA, dtype)
        return attention.attention(q, k, v_in, lengths[:rows], bidirectional=False, dtype=dtype)

    return layer


def qwen_cpu_baselines(shape, lengths, host0, layers: int) -> tuple[np.ndarray, dict]:
    """The CPU oracle timed on the host: float64 on every available core (the reported value, and
    the parity reference of layer 0), plus a float32 run on the same cores and a float64 run on
    one thread over a quarter of the batch rows, scaled to tokens/s of the whole layer."""
    from threadpoolctl import threadpool_limits

    expected, per_layer, runs = time_cpu(qwen_cpu_layer(shape, lengths, host0))
    line = cpu_baseline_line(shape, per_layer, runs, layers, " incl. q/k norm+RoPE")
    _, per32, runs32 = time_cpu(qwen_cpu_layer(shape, lengths, host0, np.float32), budget_s=6.0)
    rows = max(1, shape.batch // 4)
    with threadpool_limits(limits=1):
        _, per1, runs1 = time_cpu(qwen_cpu_layer(shape, lengths, host0, rows=rows), budget_s=8.0)
    # tokens/s of the sampled rows: per-row work differs, so the sample's own tokens count
    line["variants"] = [
        {"dtype": "f32", "threads": line["blas_threads"], "value": shape.tokens / per32,
         "unit": "tokens/s", "sample": f"1 layer, all rows, median of {runs32}"},
        {"dtype": "f64", "threads": 1, "value": rows * shape.seq / per1, "unit": "tokens/s",
         "sample": f"1 layer, batch rows 0..{rows - 1} of {shape.batch}, median of {runs1}"},
    ]
    return expected, line


def cpu_baseline_line(shape, per_layer: float, runs: int, layers: int, what: str) -> dict:
    return {
        "value": shape.tokens / per_layer,
        "unit": "tokens/s",
        "cores": len(os.sched_getaffinity(0)),
        "blas_threads": blas_threads(),
        "kind": "port",
        "sample": f"1 of {layers} layers (all {shape.batch} rows, S={shape.seq}), float64 NumPy "
        f"oracle{what}, median of {runs} runs; {per_layer * 1e3:.1f} ms/layer",
    }


def bench_qwen(args, name: str, shape, lengths, seed: int, layers: int, lengths_text: str,
               headline: bool, out_dtype: str = "f32") -> dict:
    out_bytes = 2 if out_dtype == "f16" else 4
    flop = workloads.attention_flop(shape, lengths)
    nbytes = workloads.attention_bytes(shape, lengths, 2, out_bytes)
    log(f"workload {name}: B={shape.batch} S={shape.seq} sumL={int(lengths.sum())} "
        f"layers={layers} out={out_dtype}; generating inputs")
    with HipRuntime() as rt:
        sets, host0 = upload_qwen_layers(rt, shape, layers, seed, out_bytes)
        lengths_buf = rt.upload(lengths)
        # k planes alternate between two buffers, so the attention of one layer and the k
        # prologue of the next touch different buffers (the runtime then runs them as one launch)
        k_work = [rt.buffer(2 * host0["k"].nbytes) for _ in range(2)]
        if args.calibrate_copy_mib:
            size = args.calibrate_copy_mib << 20
            src, dst = rt.buffer(size), rt.buffer(size)
            with rt.command():
                rt._dispatch("copy", [src, dst], threads=size, group_size=256)
            src.close()
            dst.close()
        log("inputs resident; warmup")

        def direct():
            for i, s in enumerate(sets):
                fused_attention(rt, shape, s, lengths_buf, k_work[i % 2], out_dtype)

        # a step is the layers' launches as one prepared plan, replayed as a cached HIP graph
        # (recorded by the first warmup step; profiled steps launch directly)
        bindings = [lengths_buf, *k_work] + [s[n] for s in sets for n in sorted(s)]

        def step():
            with rt._execution_plan((name, layers, out_dtype), bindings) as replayed:
                if not replayed:
                    direct()

        odt = np.float16 if out_bytes == 2 else np.float32
        with rt._workspace():
            t = run_timed(rt, step, args.steps, args.warmup, 2 * layers)
            # the parity check reads what a graph replay wrote: layer 0's output is poisoned with
            # NaN, one step is replayed, and the result must also equal the direct launches' bits
            rt.write(sets[0]["out"], np.full(host0["q"].shape, np.nan, odt))
            replays = rt.diagnostics()["graph_launches"]
            with rt.command():
                step()
            replayed = rt.diagnostics()["graph_launches"] > replays
            out_graph = rt.read(sets[0]["out"], host0["q"].shape, odt)
        t_direct = run_timed(rt, direct, args.steps, 1, 2 * layers, profile=False)
        out0 = rt.read(sets[0]["out"], host0["q"].shape, odt)
        graphs = rt.diagnostics()
        graph_bits_equal = bool(replayed and np.array_equal(out_graph, out0, equal_nan=False))

    step_s = t["step"]
    attn_avg = t["kernel_s"]["attention_f16_norm_rope"]
    # attention launches that also ran the next layer's k prologue in extra workgroups carry its
    # bytes too: the kernel's algorithmic traffic is its own plus the carried share
    carried = t["fused_per_step"].get("norm_rope_f16", 0.0) / layers
    pro_bytes = workloads.k_prologue_bytes(shape, lengths)
    kernel_bytes = nbytes + carried * pro_bytes
    achieved = kernel_bytes / attn_avg / 1e9
    tflops = flop * layers / step_s / 1e12
    result = {
        "metric": METRIC if headline else f"prefill attention tokens/s, Qwen3 GQA {name}, 1 GPU",
        "value": shape.tokens * layers / step_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_s * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": f"{name} causal GQA prefill, fused q/k RMSNorm+RoPE",
            "batch": shape.batch,
            "seq": shape.seq,
            "heads": shape.heads,
            "kv_heads": shape.kv_heads,
            "dim": shape.dim,
            "layers": layers,
            "valid_tokens": int(lengths.sum()),
            "lengths": lengths_text,
            "out_dtype": out_dtype,
        },
        "valid_tokens_per_s": int(lengths.sum()) * layers / step_s,
        "tflops": tflops,
        "mfma_frac": tflops / PEAK_F16_TFLOPS,
        "dense_convention_tflops": workloads.dense_flop(shape) * layers / step_s / 1e12,
        "gpu_event_ms_per_step": t["gpu_step"] * 1e3 if t["gpu_step"] is not None else None,
        "ms_per_step_direct_launches": t_direct["step"] * 1e3,
        "plan_graph": {"builds": graphs["graph_builds"], "launches": graphs["graph_launches"],
                       "replay_equals_direct_launches": graph_bits_equal},
        "kernel_us": kernel_us(t),
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": achieved / PEAK_HBM_GBS,
            "traffic": measured_traffic() if headline else None,
            "algorithmic_bytes": kernel_bytes,
            "attention_bytes": nbytes,
            "carried_k_prologue": {"share_of_launches": carried, "bytes": pro_bytes},
            "kernel": "attention_f16_norm_rope",
            # the whole step (k prologue + attention per layer) against the attention's own bytes
            "step_achieved": nbytes * layers / step_s / 1e9,
            "step_frac": nbytes * layers / step_s / 1e9 / PEAK_HBM_GBS,
            "mfma_tflops": flop / attn_avg / 1e12,
        },
    }
    if not args.no_cpu_baseline:
        log("cpu baseline")
        expected, result["cpu_baseline"] = qwen_cpu_baselines(shape, lengths, host0, layers)
        # layer 0 as a graph replay wrote it (bit-equal to the direct launches, checked above)
        err = float(np.max(np.abs(out_graph.astype(np.float64) - expected)))
        result["max_abs_err_layer0"] = err
        # the fused route carries q, k and P at ~22 bits: held to the fp32 bar with fp32 output
        bar = PARITY_F32_OUT if out_dtype == "f32" else PARITY_F16_OUT
        result["parity"] = {"max_abs": err, "bar": bar, "graph_replay": graph_bits_equal,
                            "ok": bool(err <= bar and graph_bits_equal)}
    else:
        result["cpu_baseline"] = None
    return result


def bench_bge(args, layers: int = 12) -> dict:
    """BGE-small fp32 bidirectional attention (route attention_tiled), 12 layers."""
    shape, lengths = workloads.bge_small_32x512()
    flop = workloads.attention_flop(shape, lengths)
    nbytes = workloads.attention_bytes(shape, lengths, 4, 4)
    log(f"workload bge_32x512: B={shape.batch} S={shape.seq} sumL={int(lengths.sum())}")
    with HipRuntime() as rt:
        host = [workloads.bge_layer(shape, layer) for layer in range(layers)]
        sets = [{k: rt.upload(v) for k, v in t.items()} for t in host]
        for s in sets:
            s["out"] = rt.buffer(shape.tokens * shape.heads * shape.dim * 4)
        lengths_buf = rt.upload(lengths)

        def step():
            for s in sets:
                rt._attention([s["q"], s["k"], s["v"], lengths_buf, s["out"]], tokens=shape.tokens,
                              seq=shape.seq, heads=shape.heads, kv_heads=shape.kv_heads,
                              dim=shape.dim, bidirectional=1)

        t = run_timed(rt, step, args.steps, args.warmup, layers)
        out0 = rt.read(sets[0]["out"], host[0]["q"].shape)
    step_s = t["step"]
    (kernel, avg), = t["kernel_s"].items()
    tflops_kernel = flop / avg / 1e12
    result = {
        "metric": "BGE-small encoder attention tokens/s + TFLOP/s (% fp32 MFMA peak), 32x512, 1 GPU",
        "value": shape.tokens * layers / step_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_s * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "bge_32x512 bidirectional attention, key-padding mask",
                   "batch": shape.batch, "seq": shape.seq, "heads": shape.heads,
                   "dim": shape.dim, "layers": layers, "valid_tokens": int(lengths.sum()),
                   "lengths": "uniform [2,512], seed 2"},
        "tflops": flop * layers / step_s / 1e12,
        "kernel_us": kernel_us(t),
        "roofline": {
            "bound": "mfma",
            "achieved": tflops_kernel,
            "peak": PEAK_F32_TFLOPS,
            "unit": "TFLOP/s",
            "frac": tflops_kernel / PEAK_F32_TFLOPS,
            "traffic": None,
            "algorithmic_flop": flop,
            "algorithmic_bytes": nbytes,
            "hbm_gbs": nbytes / avg / 1e9,
            "kernel": kernel,
        },
    }
    if not args.no_cpu_baseline:
        from oracle import attention

        def layer():
            return attention.attention(host[0]["q"], host[0]["k"], host[0]["v"], lengths,
                                       bidirectional=True)

        expected, per_layer, runs = time_cpu(layer)
        result["cpu_baseline"] = cpu_baseline_line(shape, per_layer, runs, layers, "")
        result["max_abs_err_layer0"] = float(np.max(np.abs(out0.astype(np.float64) - expected)))
    else:
        result["cpu_baseline"] = None
    return result


def bench_qwen_f32(args, layers: int = 8) -> dict:
    """The fp32 route at the Qwen3 8x512 shape (route attention_tiled, D = 128: the reference's own
    precision, used by the fp32 Qwen3 backend): q/k normalized and rotated on the host in
    float64 and rounded to fp32, v N(0,1), lengths U{64..512} (seed 3), 8 layers."""
    from oracle import norm_rope

    shape, lengths = workloads.qwen3_8x512()
    flop = workloads.attention_flop(shape, lengths)
    nbytes = workloads.attention_bytes(shape, lengths, 4, 4)
    log(f"workload qwen3_8x512_f32: B={shape.batch} S={shape.seq} sumL={int(lengths.sum())}")
    with HipRuntime() as rt:
        sets, host0 = [], None
        for layer in range(layers):
            t = workloads.qwen_layer(shape, layer, seed=3)
            qn = workloads.bf16_values(t["q_norm"]).astype(np.float64)
            kn = workloads.bf16_values(t["k_norm"]).astype(np.float64)
            host = {"q": norm_rope.norm_rope(t["q"], qn, workloads.EPS, workloads.THETA),
                    "k": norm_rope.norm_rope(t["k"], kn, workloads.EPS, workloads.THETA),
                    "v": t["v"]}
            host = {k: v.astype(np.float32) for k, v in host.items()}
            host0 = host0 or host
            s = {k: rt.upload(v) for k, v in host.items()}
            s["out"] = rt.buffer(host["q"].nbytes)
            sets.append(s)
        lengths_buf = rt.upload(lengths)

        def step():
            for s in sets:
                rt._attention([s["q"], s["k"], s["v"], lengths_buf, s["out"]], tokens=shape.tokens,
                              seq=shape.seq, heads=shape.heads, kv_heads=shape.kv_heads,
                              dim=shape.dim)

        t = run_timed(rt, step, args.steps, args.warmup, layers)
        out0 = rt.read(sets[0]["out"], host0["q"].shape)
    step_s = t["step"]
    (kernel, avg), = t["kernel_s"].items()
    tflops = flop / avg / 1e12
    result = {
        "metric": "prefill attention tokens/s, Qwen3 GQA 8x512, fp32 route, 1 GPU",
        "value": shape.tokens * layers / step_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_s * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "qwen3_8x512 causal GQA attention on the fp32 route (q/k normed)",
                   "batch": shape.batch, "seq": shape.seq, "heads": shape.heads,
                   "kv_heads": shape.kv_heads, "dim": shape.dim, "layers": layers,
                   "valid_tokens": int(lengths.sum()), "lengths": "uniform [64,512], seed 3"},
        "kernel_us": kernel_us(t),
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": PEAK_F32_TFLOPS,
                     "unit": "TFLOP/s", "frac": tflops / PEAK_F32_TFLOPS, "traffic": None,
                     "algorithmic_flop": flop, "algorithmic_bytes": nbytes,
                     "hbm_gbs": nbytes / avg / 1e9, "kernel": kernel},
        "cpu_baseline": None,
    }
    # layer 0 against the float64 oracle (the fp32 route's bar, max-abs 1e-4), also without the
    # CPU leg
    from oracle import attention

    expected = attention.attention(host0["q"], host0["k"], host0["v"], lengths, bidirectional=False)
    err = float(np.max(np.abs(out0.astype(np.float64) - expected)))
    result["max_abs_err_layer0"] = err
    result["parity"] = {"max_abs": err, "bar": PARITY_F32_OUT, "ok": err <= PARITY_F32_OUT}
    return result


def bench_qkv4_block(args, layers: int = 8) -> dict:
    """uint4 QKV projection -> k norm+RoPE -> fused attention, 8 independent layers."""
    shape, lengths, d = workloads.qwen_qkv4_16x256()
    m, k_in = d["x"].shape
    nq, nkv = shape.heads * shape.dim, shape.kv_heads * shape.dim
    n_total = nq + 2 * nkv
    gemm_flop = workloads.qkv4_flop(m, k_in, n_total)
    gemm_bytes = workloads.qkv4_bytes(m, k_in, n_total)
    attn_flop = workloads.attention_flop(shape, lengths)
    log(f"workload qwen_qkv4_16x256: M={m} K={k_in} N={n_total} sumL={int(lengths.sum())}")
    with HipRuntime() as rt:
        common = {name: rt.upload(d[name]) for name in ("w", "s", "b", "q_norm", "k_norm")}
        lengths_buf = rt.upload(lengths)
        k_work = rt.buffer(2 * m * nkv * 2)
        rng = np.random.default_rng((5, 1))
        sets = []
        for _ in range(layers):
            x = rt.upload(rng.standard_normal((m, k_in), dtype=np.float32).astype(np.float16))
            sets.append({"x": x, "yq": rt.buffer(m * nq * 2), "yk": rt.buffer(m * nkv * 2),
                         "yv": rt.buffer(m * nkv * 2), "out": rt.buffer(m * nq * 4)})

        def step():
            for s in sets:
                rt._qkv4([s["x"], common["w"], common["s"], common["b"], s["yq"], s["yk"],
                          s["yv"]], rows=m, k=k_in, q_cols=nq, kv_cols=nkv, scale_dtype="f16")
                rt._attention_norm_rope(
                    [s["yq"], s["yk"], s["yv"], lengths_buf, s["out"], common["q_norm"],
                     common["k_norm"], k_work], tokens=m, seq=shape.seq, heads=shape.heads,
                    kv_heads=shape.kv_heads, dim=shape.dim, eps=workloads.EPS,
                    theta=workloads.THETA)

        t = run_timed(rt, step, args.steps, args.warmup, 3 * layers)
    step_s = t["step"]
    ks = t["kernel_s"]
    gemm = ks["qkv4_f16"]
    return {
        "metric": "Qwen3 uint4 QKV projection + fused attention tokens/s, 16x256, 1 GPU",
        "value": m * layers / step_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_s * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "qwen_qkv4_16x256: qkv4 -> k norm+RoPE -> fused attention",
                   "rows": m, "k": k_in, "n": n_total, "layers": layers,
                   "valid_tokens": int(lengths.sum()), "lengths": "uniform [1,256], seed 5"},
        "kernel_us": kernel_us(t),
        "roofline": {
            "bound": "mfma",
            "achieved": gemm_flop / gemm / 1e12,
            "peak": PEAK_F16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": gemm_flop / gemm / 1e12 / PEAK_F16_TFLOPS,
            "traffic": None,
            "algorithmic_flop": gemm_flop,
            "algorithmic_bytes": gemm_bytes,
            "kernel": "qkv4_f16",
        },
        "attention_tflops": attn_flop / ks["attention_f16_norm_rope"] / 1e12,
        "cpu_baseline": None,
    }


def qwen_tail_launch(rt: HipRuntime, s: dict, tokens: int, hidden: int, width: int,
                     inter: int) -> None:
    """qwen3.py:246-280: h = x + o_proj(attended); out = h + down(gated4(rms_norm(h)))."""
    n = tokens * hidden
    rt._linear4([s["att"], *s["o"], s["proj"]], rows=tokens, cols=hidden, k=width)
    rt._dispatch("add", [s["x"], s["proj"], s["h"]], threads=n, n=n)
    rt._dispatch("rms_norm", [s["h"], s["post_norm"], s["norm"]], threads=tokens * 32,
                 group_size=32, cols=hidden, eps=workloads.EPS)
    rt._gated4([s["norm"], *s["gate"], *s["up"], s["g"], s["u"]], rows=tokens, cols=inter,
               k=hidden)
    rt._linear4([s["g"], *s["down"], s["proj"]], rows=tokens, cols=hidden, k=inter)
    rt._dispatch("add", [s["h"], s["proj"], s["out"]], threads=n, n=n)


def bench_qwen_tail(args, tokens: int = 16 * 256) -> dict:
    """Qwen3 layer tail on `tokens` tokens (fp32 activations, uint4 bf16-affine weights), 4
    independent layers: o_proj, residual, post-attention RMSNorm, gate/up + SiLU, down, residual."""
    layers, hidden, width, inter = 4, 1024, 2048, 3072
    wname = "qwen_tail_16x256" if tokens == 16 * 256 else f"qwen_tail_1x{tokens}"
    flop = workloads.tail_flop(tokens, hidden, width, inter)
    log(f"workload {wname}: T={tokens} hidden={hidden} attn={width} inter={inter}")
    with HipRuntime() as rt:
        host = [workloads.qwen_tail_16x256(layer) for layer in range(layers)]
        for d in host:  # the first `tokens` rows
            d["x"], d["attended"] = d["x"][:tokens].copy(), d["attended"][:tokens].copy()
        sets = []
        for d in host:
            s = {"x": rt.upload(d["x"]), "att": rt.upload(d["attended"]),
                 "post_norm": rt.upload(d["post_norm"])}
            for name in ("o", "gate", "up", "down"):
                s[name] = [rt.upload(a) for a in d[name]]
            for name, width_ in (("proj", hidden), ("h", hidden), ("norm", hidden), ("out", hidden),
                                 ("g", inter), ("u", inter)):
                s[name] = rt.buffer(tokens * width_ * 4)
            sets.append(s)

        def step():
            for s in sets:
                qwen_tail_launch(rt, s, tokens, hidden, width, inter)

        launches = 8 * layers
        t = run_timed(rt, step, args.steps, args.warmup, launches)
        out0 = rt.read(sets[0]["out"], (tokens, hidden))
    step_s = t["step"]
    ks = t["kernel_s"]
    # the four projections of a layer: every linear4 / gated4 launch of a step (the gated MLP's
    # gate + up + SiLU run as one launch from 1024 rows, carried by the gate's record)
    proj = sorted(k for k in t["kernel_step_s"] if k.startswith(("linear4", "gated4")))
    gemm_s = sum(t["kernel_step_s"][k] for k in proj) / layers
    kernel = " + ".join(proj)
    tflops = flop / gemm_s / 1e12
    # from 1024 rows linear4 runs on fp16 MFMA (row-scaled hi + lo halves of x, two MFMAs per
    # product): priced against the fp16 peak; below that on fp32 MFMA
    hilo = tokens >= 1024
    peak = PEAK_F16_TFLOPS if hilo else PEAK_F32_TFLOPS
    gemm_bytes = tokens * (width + hidden + hidden + 2 * inter + inter) * 4 + (
        (hidden * width + 2 * inter * hidden + hidden * inter) // 2)
    result = {
        "metric": f"Qwen3 layer tail (o_proj, RMSNorm, gated MLP) tokens/s, {wname[10:]}, 1 GPU",
        "value": tokens * layers / step_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_s * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"{wname}: o_proj -> residual -> RMSNorm -> gate/up+SiLU "
                               "-> down -> residual", "tokens": tokens, "hidden": hidden,
                   "attention_width": width, "intermediate": inter, "layers": layers},
        "tflops": flop * layers / step_s / 1e12,
        "kernel_us": kernel_us(t),
        "roofline": {
            "bound": "mfma",
            "achieved": tflops,
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": tflops / peak,
            "traffic": None,
            "algorithmic_flop": flop,
            "algorithmic_bytes": gemm_bytes,
            "kernel": kernel + (" (fp16 MFMA, hi + lo halves: 2x the algorithmic MFMA work)"
                                if hilo else " (fp32 MFMA)"),
        },
    }
    if not args.no_cpu_baseline:
        from oracle import qwen_block

        sample = min(512, tokens)
        d = host[0]

        def layer():
            return qwen_block.layer_tail(d["x"][:sample], d["attended"][:sample],
                                         {n: d[n] for n in ("o", "gate", "up", "down")},
                                         workloads.bf16_values(d["post_norm"]), eps=workloads.EPS)

        expected, per_sample, runs = time_cpu(layer)
        result["cpu_baseline"] = {
            "value": sample / per_sample,
            "unit": "tokens/s",
            "cores": len(os.sched_getaffinity(0)),
            "blas_threads": blas_threads(),
            "kind": "port",
            "sample": f"{sample} of {tokens} tokens of layer 0, float64 NumPy oracle, median of "
                      f"{runs} runs; {per_sample * 1e3:.1f} ms",
        }
        err = np.abs(out0[:sample].astype(np.float64) - expected)
        result["max_abs_err_layer0"] = float(err.max())
        result["max_rel_err_layer0"] = float(err.max() / np.abs(expected).max())
    else:
        result["cpu_baseline"] = None
    return result


def bge_layer_launch(rt: HipRuntime, s: dict, lengths_buf, tokens: int, seq: int) -> None:
    """bert.py:186-230: q/k/v projections with bias, bidirectional attention, output projection,
    residual + LayerNorm, intermediate projection + GELU, output projection, residual +
    LayerNorm (x updated in place, as the reference does)."""
    hidden, inter, heads = 384, 1536, 12

    def linear(src, dst, name, outputs, inputs):
        rt._matmul_bias_f32([s[src], s[name], s[dst], s[name + "_b"]], rows=tokens, cols=outputs,
                            k=inputs)

    def norm(name):
        rt._dispatch("layer_norm", [s["x"], s[name + "_w"], s[name + "_b"], s["x"]],
                     threads=tokens * 32, group_size=32, cols=hidden, eps=1e-12)

    for target, name in (("qb", "q"), ("kb", "k"), ("vb", "v")):
        linear("x", target, name, hidden, hidden)
    rt._attention([s["qb"], s["kb"], s["vb"], lengths_buf, s["att"]], tokens=tokens, seq=seq,
                  heads=heads, kv_heads=heads, dim=hidden // heads, bidirectional=1)
    linear("att", "proj", "o", hidden, hidden)
    rt._dispatch("add", [s["x"], s["proj"], s["x"]], threads=tokens * hidden, n=tokens * hidden)
    norm("ln1")
    linear("x", "act", "i", inter, hidden)
    rt._dispatch("gelu_f32", [s["act"]], threads=tokens * inter, n=tokens * inter)
    linear("act", "proj", "out", hidden, inter)
    rt._dispatch("add", [s["x"], s["proj"], s["x"]], threads=tokens * hidden, n=tokens * hidden)
    norm("ln2")


def bench_bge_layer(args) -> dict:
    """BGE-small encoder layers on 32x512 tokens (fp32), 4 independent layers: projections with
    bias, bidirectional attention, residual + LayerNorm, GELU MLP."""
    layers, batch, seq, hidden, inter = 4, 32, 512, 384, 1536
    tokens = batch * seq
    shape, lengths = workloads.bge_small_32x512()
    flop = workloads.bge_layer_gemm_flop(tokens)
    log(f"workload bge_layer_32x512: T={tokens} hidden={hidden} inter={inter}")
    with HipRuntime() as rt:
        host = [workloads.bge_encoder_layer(layer) for layer in range(layers)]
        lengths_buf = rt.upload(lengths)
        sets = []
        for d in host:
            s = {name: rt.upload(a) for name, a in d.items()}
            for name, width in (("qb", hidden), ("kb", hidden), ("vb", hidden), ("att", hidden),
                                ("proj", hidden), ("act", inter)):
                s[name] = rt.buffer(tokens * width * 4)
            sets.append(s)

        def step():
            for s in sets:
                bge_layer_launch(rt, s, lengths_buf, tokens, seq)

        # one layer first, from the pristine input, for the parity check
        with rt.command():
            bge_layer_launch(rt, sets[0], lengths_buf, tokens, seq)
        out0 = rt.read(sets[0]["x"], (tokens, hidden))
        t = run_timed(rt, step, args.steps, args.warmup, 12 * layers)
    step_s = t["step"]
    ks = t["kernel_s"]
    gemm_s = 6 * ks["matmul_bias_f32_chunk32"]  # the six projections of a layer
    tflops = flop / gemm_s / 1e12
    result = {
        "metric": "BGE-small encoder layer tokens/s, 32x512, 1 GPU",
        "value": tokens * layers / step_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_s * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "bge_layer_32x512: q/k/v projections -> bidirectional attention -> "
                               "o projection + LayerNorm -> GELU MLP + LayerNorm",
                   "batch": batch, "seq": seq, "hidden": hidden, "intermediate": inter,
                   "layers": layers, "lengths": "uniform [2,512], seed 2"},
        "tflops": flop * layers / step_s / 1e12,
        "kernel_us": kernel_us(t),
        "roofline": {
            "bound": "mfma",
            "achieved": tflops,
            "peak": PEAK_F32_TFLOPS,
            "unit": "TFLOP/s",
            "frac": tflops / PEAK_F32_TFLOPS,
            "traffic": None,
            "algorithmic_flop": flop,
            "kernel": "matmul_bias_f32_chunk32",
        },
    }
    if not args.no_cpu_baseline:
        from oracle import bert_block

        d = host[0]
        rows = 2  # a bounded sample: the first 2 batch rows of layer 0
        w = {k: v for k, v in d.items() if k != "x"}

        def layer():
            return bert_block.layer(d["x"][: rows * seq].reshape(rows, seq, hidden),
                                    lengths[:rows], w, heads=12, eps=1e-12)

        expected, per_sample, runs = time_cpu(layer)
        result["cpu_baseline"] = {
            "value": rows * seq / per_sample,
            "unit": "tokens/s",
            "cores": len(os.sched_getaffinity(0)),
            "blas_threads": blas_threads(),
            "kind": "port",
            "sample": f"{rows} of {batch} batch rows of layer 0, float64 NumPy oracle, median of "
                      f"{runs} runs; {per_sample * 1e3:.1f} ms",
        }
        got = out0[: rows * seq].reshape(rows, seq, hidden).astype(np.float64)
        result["max_abs_err_layer0"] = float(np.abs(got - expected).max())
    else:
        result["cpu_baseline"] = None
    return result


def bench_bge_plan(args) -> dict:
    """A 12-layer BGE-small encoder stack on one 128-token sequence, replayed as a prepared plan
    (the reference's _execution_plan path, bert.py:153-170): per-forward time with plan replays as
    cached HIP graphs and, in a second runtime, launched one by one (TESSERY_HIP_GRAPHS=0)."""
    layers, batch, seq, hidden, inter = 12, 1, 128, 384, 1536
    tokens = batch * seq
    lengths = np.array([seq], np.uint32)
    host = [workloads.bge_encoder_layer(layer, batch=batch, seq=seq) for layer in range(layers)]
    log(f"workload bge_plan_1x128: {layers} layers, T={tokens}")

    def measure(graphs: bool) -> tuple[float, dict]:
        previous = os.environ.get("TESSERY_HIP_GRAPHS")
        os.environ["TESSERY_HIP_GRAPHS"] = "1" if graphs else "0"
        try:
            rt = HipRuntime()
        finally:
            if previous is None:
                del os.environ["TESSERY_HIP_GRAPHS"]
            else:
                os.environ["TESSERY_HIP_GRAPHS"] = previous
        with rt:
            lengths_buf = rt.upload(lengths)
            sets = []
            for d in host:
                s = {name: rt.upload(a) for name, a in d.items()}
                for name, width in (("qb", hidden), ("kb", hidden), ("vb", hidden), ("att", hidden),
                                    ("proj", hidden), ("act", inter)):
                    s[name] = rt.buffer(tokens * width * 4)
                sets.append(s)
            bindings = [lengths_buf] + [s[n] for s in sets for n in sorted(s)]

            def forward():
                with rt.command():
                    with rt._execution_plan(("bge_plan", layers, seq), bindings) as replayed:
                        if not replayed:
                            for s in sets:
                                bge_layer_launch(rt, s, lengths_buf, tokens, seq)

            with rt._workspace():
                for _ in range(args.warmup + 2):
                    forward()
                start = time.perf_counter()
                reps = max(args.steps, 50)
                for _ in range(reps):
                    forward()
                per = (time.perf_counter() - start) / reps
            return per, rt.diagnostics()

    with_graphs, diag = measure(True)
    without, _ = measure(False)
    return {
        "metric": "BGE-small 12-layer encoder forward on one 128-token sequence, plan replay, 1 GPU",
        "value": tokens / with_graphs,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": max(args.steps, 50),
        "warmup": args.warmup,
        "ms_per_step": with_graphs * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "bge_plan_1x128: 12 encoder layers (144 launches) per forward, "
                               "replayed as one prepared plan", "batch": batch, "seq": seq,
                   "layers": layers},
        "ms_per_forward_graphs": with_graphs * 1e3,
        "ms_per_forward_launches": without * 1e3,
        "graph_builds": diag["graph_builds"],
        "graph_launches": diag["graph_launches"],
        "roofline": None,
        "cpu_baseline": None,
    }


def bench_model(args, arch: str) -> dict:
    """A whole embedding forward through the model backends: a synthetic weight pack of the real
    model shapes written to disk (config.json + model.safetensors, pinned by sha256), loaded by
    Qwen3Backend / BertBackend, and forward(ids, lengths) timed end to end (ids upload, every
    layer, pooling, result read; plan replayed as a HIP graph after the first call)."""
    import tempfile

    from tessery_amd.backends import BertBackend, Qwen3Backend

    batch, seq = 8, 512
    rng = np.random.default_rng(3)
    if arch == "qwen3":
        shape = workloads.QWEN3_0P6B
        config, tensors = workloads.qwen3_pack_tensors(21, **shape)
        lengths = workloads.lengths_uniform(3, batch, 64, seq)
        architecture, backend_cls, dims = "qwen3_uint4", Qwen3Backend, shape["hidden"]
        wname = "qwen3_model_8x512"
        what = "Qwen3-0.6B shapes (28 layers, hidden 1024, 16q/8kv x 128, MLP 3072, vocab 151669)"
    else:
        shape = workloads.BGE_SMALL
        config, tensors = workloads.bert_pack_tensors(22, **shape)
        lengths = workloads.lengths_uniform(2, batch, 2, seq)
        architecture, backend_cls, dims = "bert_f32", BertBackend, shape["hidden"]
        wname = "bge_model_8x512"
        what = "BGE-small shapes (12 layers, hidden 384, 12 heads x 32, MLP 1536, vocab 30522)"
    ids = rng.integers(0, shape["vocab"], (batch, seq)).astype(np.uint32)
    log(f"workload {wname}: {what}, lengths uniform, {int(lengths.sum())} valid tokens")
    with tempfile.TemporaryDirectory(dir="/tmp") as pack_dir:
        t0 = time.perf_counter()
        profile = workloads.write_pack(pack_dir, config, tensors, architecture=architecture,
                                       max_length=seq,
                                       min_dimensions=64 if arch == "qwen3" else dims)
        pack_bytes = profile.artifact("model.safetensors").size
        log(f"pack written: {pack_bytes / 2**20:.1f} MiB in {time.perf_counter() - t0:.1f} s")
        t0 = time.perf_counter()
        backend = backend_cls(pack_dir, profile, workspace_limit_bytes=1 << 30)
        load_s = time.perf_counter() - t0
        log(f"pack verified and uploaded in {load_s:.2f} s")
    try:
        rt = backend.runtime
        for _ in range(max(2, args.warmup)):
            out = backend.forward(ids, lengths, dimensions=dims)
        start = time.perf_counter()
        for _ in range(args.steps):
            out = backend.forward(ids, lengths, dimensions=dims)
        per = (time.perf_counter() - start) / args.steps
        log(f"timed {args.steps} forwards: {per * 1e3:.3f} ms each")
        diag = rt.diagnostics()
        rt._clear_plans()  # re-record once with events around every launch
        with rt.profile_kernels() as records:
            backend.forward(ids, lengths, dimensions=dims)
    finally:
        backend.close()
    kernel_s: dict[str, float] = {}
    proj_flop, proj_s = 0, 0.0
    for r in records:
        kernel_s[r["kernel"]] = kernel_s.get(r["kernel"], 0.0) + r["gpu_seconds"]
        # at 4096 rows every projection is a single launch over all rows
        if r["kernel"].startswith(("linear4", "gated4", "matmul")):
            mult = 2 if r["kernel"].startswith("gated4") else 1
            proj_flop += mult * 2 * r["rows"] * r["cols"] * r["k"]
            proj_s += r["gpu_seconds"]
    tokens = batch * seq
    proj_tflops = proj_flop / proj_s / 1e12
    # Qwen3's uint4 projections at 4096 rows run on fp16 MFMA (hi + lo halves of x); BGE's
    # dense projections on fp32 MFMA
    peak = PEAK_F16_TFLOPS if arch == "qwen3" else PEAK_F32_TFLOPS
    result = {
        "metric": f"{'Qwen3-0.6B' if arch == 'qwen3' else 'BGE-small'} embedding forward "
                  f"tokens/s (padded), {batch}x{seq}, 1 GPU",
        "value": tokens / per,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": max(2, args.warmup),
        "ms_per_step": per * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"{wname}: {what}, forward(ids, lengths) -> unit vectors",
                   "batch": batch, "seq": seq, "valid_tokens": int(lengths.sum()),
                   "dimensions": dims},
        "sequences_per_s": batch / per,
        "pack_mib": pack_bytes / 2**20,
        "load_s": load_s,
        "graph_builds": diag["graph_builds"],
        "graph_launches": diag["graph_launches"],
        "kernel_ms_per_forward": {k: v * 1e3 for k, v in sorted(kernel_s.items())},
        "roofline": {
            "bound": "mfma",
            "achieved": proj_tflops,
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": proj_tflops / peak,
            "traffic": None,
            "algorithmic_flop": proj_flop,
            "kernel": "all projection launches of one forward (summed FLOP / summed duration)",
        },
    }
    if not args.no_cpu_baseline:
        from oracle import models as oracle_models

        w = workloads.weights_of(tensors)
        sample = int(lengths[0])
        ids0, len0 = ids[:1, :sample], lengths[:1].copy()

        def forward_cpu():
            if arch == "qwen3":
                return oracle_models.qwen3_forward(
                    w, ids0, len0, layers=shape["layers"], heads=shape["heads"],
                    kv_heads=shape["kv_heads"], head_dim=shape["head_dim"],
                    eps=config["rms_norm_eps"], theta=config["rope_theta"], dimensions=dims)
            return oracle_models.bert_forward(w, ids0, len0, layers=shape["layers"],
                                              heads=shape["heads"], eps=config["layer_norm_eps"])

        expected, per_sample, runs = time_cpu(forward_cpu, budget_s=20.0)
        result["cpu_baseline"] = {
            "value": sample / per_sample,
            "unit": "tokens/s",
            "cores": len(os.sched_getaffinity(0)),
            "blas_threads": blas_threads(),
            "kind": "port",
            "sample": f"sequence 0 ({sample} tokens, all layers), float64 NumPy oracle, median of "
                      f"{runs}; {per_sample * 1e3:.0f} ms",
        }
        result["max_abs_err_seq0"] = float(np.abs(out[0] - expected[0]).max())
    else:
        result["cpu_baseline"] = None
    return result


def _kernel_summary(result: dict, peak_tflops: float) -> dict:
    roof = result["roofline"]
    summary = {
        "config": result["config"],
        "ms_per_step": result["ms_per_step"],
        "kernel_us": result["kernel_us"],
        "roofline": {key: roof[key] for key in ("kernel", "bound", "achieved", "peak", "unit",
                                                "frac")},
    }
    if "mfma_tflops" in roof:  # attention kernels on an HBM roof: their MFMA share as well
        summary["mfma_frac"] = roof["mfma_tflops"] / peak_tflops
    if "max_abs_err_layer0" in result:
        summary["max_abs_err_layer0"] = result["max_abs_err_layer0"]
    return summary


def secondary_measurements(args) -> dict:
    """Kernel times and roofline fractions of the other configurations, measured in the same run
    (2 warmup and 5 timed steps each, no CPU leg): BGE-small 32x512 fp32 attention (4 layers),
    Qwen3 8x512 fused attention (8 layers), the same shape on the fp32 route (4 layers), the
    uint4 QKV block 16x256 (8 layers), and the headline shape at full length (32 x 512, every
    length 512, fp16 output, 4 layers)."""
    sub = argparse.Namespace(steps=5, warmup=2, no_cpu_baseline=True, calibrate_copy_mib=0)
    out = {"bge_32x512": _kernel_summary(bench_bge(sub, layers=4), PEAK_F32_TFLOPS)}
    shape, lengths = workloads.qwen3_8x512()
    out["qwen3_8x512"] = _kernel_summary(
        bench_qwen(sub, "qwen3_8x512", shape, lengths, 3, 8, "uniform [64,512], seed 3",
                   headline=False), PEAK_F16_TFLOPS)
    out["qwen3_8x512_f32"] = _kernel_summary(bench_qwen_f32(sub, layers=4), PEAK_F32_TFLOPS)
    out["qwen_qkv4_16x256"] = _kernel_summary(bench_qkv4_block(sub, layers=8), PEAK_F16_TFLOPS)
    full, full_lengths = workloads.qwen3_32x512_full()
    out["qwen3_32x512_full_f16out"] = _kernel_summary(
        bench_qwen(sub, "qwen3_32x512_full", full, full_lengths, 4, 4, "all 512",
                   headline=False, out_dtype="f16"), PEAK_F16_TFLOPS)
    return out


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__,
                                     formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--layers", type=int, default=LAYERS, help="headline workload only")
    parser.add_argument("--workload", default="qwen3_32x512",
                        choices=["qwen3_32x512", "qwen3_8x512", "qwen3_32x512_full",
                                 "qwen3_8x512_f32", "bge_32x512",
                                 "qwen_qkv4_16x256",
                                 "qwen_tail_16x256", "qwen_tail_1x128", "bge_layer_32x512",
                                 "bge_plan_1x128", "qwen3_model_8x512", "bge_model_8x512"])
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-secondary", action="store_true",
                        help="headline only: skip the kernel figures of the other configurations")
    parser.add_argument("--calibrate-copy-mib", type=int, default=0,
                        help="also launch one copy of this many MiB (traffic-counter calibration)")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the attention path "
              "shards over batch rows with no exchange, see the multi-GPU design notes)",
              file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0 or not 1 <= args.layers <= LAYERS:
        parser.error("invalid steps / warmup / layers")

    if args.workload == "qwen3_32x512":
        shape, lengths = workloads.qwen3_32x512()
        result = bench_qwen(args, "qwen3_32x512", shape, lengths, 4, args.layers,
                            "log-uniform [1,512], seed 4", headline=True)
        if not args.no_secondary:
            log("secondary configurations")
            result["secondary"] = secondary_measurements(args)
    elif args.workload == "qwen3_8x512":
        shape, lengths = workloads.qwen3_8x512()
        result = bench_qwen(args, "qwen3_8x512", shape, lengths, 3, 8, "uniform [64,512], seed 3",
                            headline=False)
    elif args.workload == "qwen3_32x512_full":
        shape, lengths = workloads.qwen3_32x512_full()
        result = bench_qwen(args, "qwen3_32x512_full", shape, lengths, 4, 8, "all 512",
                            headline=False, out_dtype="f16")
    elif args.workload == "bge_32x512":
        result = bench_bge(args)
    elif args.workload == "qwen3_8x512_f32":
        result = bench_qwen_f32(args)
    elif args.workload == "qwen_tail_16x256":
        result = bench_qwen_tail(args)
    elif args.workload == "qwen_tail_1x128":
        result = bench_qwen_tail(args, tokens=128)
    elif args.workload == "bge_layer_32x512":
        result = bench_bge_layer(args)
    elif args.workload == "bge_plan_1x128":
        result = bench_bge_plan(args)
    elif args.workload == "qwen3_model_8x512":
        result = bench_model(args, "qwen3")
    elif args.workload == "bge_model_8x512":
        result = bench_model(args, "bge")
    else:
        result = bench_qkv4_block(args)
    print(json.dumps(result), flush=True)
    if "parity" in result and not result["parity"]["ok"]:
        log(f"parity failed: max abs {result['parity']['max_abs']:.3e} > {result['parity']['bar']}")
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
