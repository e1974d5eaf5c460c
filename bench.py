"""Benchmark: Qwen3-shaped causal GQA prefill attention at maximum batch on one MI355X.

Workload qwen3_32x512: B=32 rows, log-uniform valid lengths in [1,512] (seed 4), execution width
16*ceil(max L/16) = 464, 16 query / 8 KV heads, head dim 128, fp16 operands with fp32
accumulation, per-head q/k RMSNorm + RoPE fused, 28 layers with independent inputs resident in
HBM. One step = the 28 layers: per layer one k norm+RoPE launch and one attention launch (q
norm+RoPE inside), through the C ABI (HipRuntime -> mi_dispatch).

Prints one JSON line: tokens/s (execution tokens B*S*layers per second), mask-exact TFLOP/s and
its fraction of the fp16 MFMA peak, the HBM roofline of the attention kernel from live per-launch
HIP-event timings, and the float64 NumPy CPU oracle timed on the host on a bounded sample.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from tessery_amd import HipRuntime, workloads  # noqa: E402

METRIC = "prefill attention tokens/s + TFLOP/s (% MFMA peak), Qwen3 GQA 32x512, 1 GPU"
PEAK_F16_TFLOPS = 2516.6
PEAK_HBM_GBS = 8000.0
LAYERS = 28
# rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of the attention kernel on this workload, with the
# copy-kernel calibration of each counter; valid for the kernel source it names
TRAFFIC_FILE = ROOT / "profiles" / "attention_f16_norm_rope_qwen3_32x512_traffic.txt"
KERNEL_SOURCE = ROOT / "tessery_amd" / "csrc" / "attention.hip"


def log(message: str) -> None:
    print(message, file=sys.stderr, flush=True)


def upload_layers(rt: HipRuntime, shape: workloads.Shape, layers: int):
    sets = []
    for layer in range(layers):
        t = workloads.qwen_layer(shape, layer, seed=4)
        sets.append(
            {
                "q": rt.upload(t["q"]),
                "k": rt.upload(t["k"]),
                "v": rt.upload(t["v"]),
                "q_norm": rt.upload(t["q_norm"]),
                "k_norm": rt.upload(t["k_norm"]),
                "out": rt.buffer(t["q"].size * 4),
            }
        )
        if layer == 0:
            host0 = t
    return sets, host0


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


def encode_step(rt, shape, sets, lengths_buf, k_work):
    for s in sets:
        rt._attention_norm_rope(
            [s["q"], s["k"], s["v"], lengths_buf, s["out"], s["q_norm"], s["k_norm"], k_work],
            tokens=shape.tokens,
            seq=shape.seq,
            heads=shape.heads,
            kv_heads=shape.kv_heads,
            dim=shape.dim,
            eps=workloads.EPS,
            theta=workloads.THETA,
            out_dtype="f32",
        )


def cpu_baseline(shape, lengths, host0, budget_s: float = 12.0):
    """float64 NumPy oracle (norm+RoPE on q and k, attention) on layer 0, all 32 rows."""
    from oracle import attention, norm_rope

    try:
        from threadpoolctl import threadpool_info

        blas_threads = max((i.get("num_threads", 0) for i in threadpool_info()), default=0)
    except Exception:  # threadpoolctl missing: report unknown
        blas_threads = 0
    qn = workloads.bf16_values(host0["q_norm"]).astype(np.float64)
    kn = workloads.bf16_values(host0["k_norm"]).astype(np.float64)

    def layer():
        q = norm_rope.norm_rope(host0["q"], qn, workloads.EPS, workloads.THETA)
        k = norm_rope.norm_rope(host0["k"], kn, workloads.EPS, workloads.THETA)
        return attention.attention(q, k, host0["v"], lengths, bidirectional=False)

    start = time.perf_counter()
    expected = layer()  # warmup, also the parity reference
    times = [time.perf_counter() - start]
    while sum(times) < budget_s and len(times) < 6:
        t0 = time.perf_counter()
        layer()
        times.append(time.perf_counter() - t0)
    per_layer = float(np.median(times[1:] if len(times) > 1 else times))
    return expected, {
        "value": shape.tokens / per_layer,
        "unit": "tokens/s",
        "cores": len(os.sched_getaffinity(0)),
        "blas_threads": blas_threads,
        "kind": "port",
        "sample": f"1 of {LAYERS} layers (all {shape.batch} rows, S={shape.seq}), float64 NumPy "
        f"oracle incl. q/k norm+RoPE, median of {max(1, len(times) - 1)} runs; "
        f"{per_layer * 1e3:.1f} ms/layer",
    }


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--layers", type=int, default=LAYERS)
    parser.add_argument("--no-cpu-baseline", action="store_true")
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

    shape, lengths = workloads.qwen3_32x512()
    flop = workloads.attention_flop(shape, lengths)
    nbytes = workloads.attention_bytes(shape, lengths, 2, 4)
    log(f"workload qwen3_32x512: B={shape.batch} S={shape.seq} sumL={int(lengths.sum())} "
        f"layers={args.layers}; generating inputs")
    with HipRuntime() as rt:
        sets, host0 = upload_layers(rt, shape, args.layers)
        lengths_buf = rt.upload(lengths)
        k_work = rt.buffer(2 * host0["k"].nbytes)
        if args.calibrate_copy_mib:
            size = args.calibrate_copy_mib << 20
            src, dst = rt.buffer(size), rt.buffer(size)
            with rt.command():
                rt._dispatch("copy", [src, dst], threads=size, group_size=256)
            src.close()
            dst.close()
        log("inputs resident; warmup")
        for _ in range(args.warmup):
            with rt.command():
                encode_step(rt, shape, sets, lengths_buf, k_work)
        # timed region: K steps launched back to back; synchronized before and after
        with rt.command():
            for _ in range(args.steps):
                encode_step(rt, shape, sets, lengths_buf, k_work)
            launched = time.perf_counter()
        wall = time.perf_counter() - launched
        gpu = rt.last_gpu_seconds
        log(f"timed {args.steps} steps: wall {wall * 1e3:.3f} ms, events {gpu * 1e3:.3f} ms")
        # per-launch durations: HIP events recorded around every launch on the runtime stream,
        # over the same steps replayed once more (a command profiles at most 2048 launches)
        prof_steps = max(1, min(args.steps, 2048 // (2 * args.layers)))
        with rt.profile_kernels() as records:
            with rt.command():
                for _ in range(prof_steps):
                    encode_step(rt, shape, sets, lengths_buf, k_work)
        attn = [r["gpu_seconds"] for r in records if r["kernel"] == "attention_f16_norm_rope"]
        prologue = [r["gpu_seconds"] for r in records if r["kernel"] == "norm_rope_f16"]
        out0 = rt.read(sets[0]["out"], host0["q"].shape)

    step = wall / args.steps
    tokens = shape.tokens * args.layers
    attn_avg = float(np.mean(attn))
    achieved = nbytes / attn_avg / 1e9
    traffic = measured_traffic()
    tflops = flop * args.layers / step / 1e12
    result = {
        "metric": METRIC,
        "value": tokens / step,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": "qwen3_32x512 causal GQA prefill, fused q/k RMSNorm+RoPE",
            "batch": shape.batch,
            "seq": shape.seq,
            "heads": shape.heads,
            "kv_heads": shape.kv_heads,
            "dim": shape.dim,
            "layers": args.layers,
            "valid_tokens": int(lengths.sum()),
            "lengths": "log-uniform [1,512], seed 4",
            "out_dtype": "f32",
        },
        "valid_tokens_per_s": int(lengths.sum()) * args.layers / step,
        "tflops": tflops,
        "mfma_frac": tflops / PEAK_F16_TFLOPS,
        "dense_convention_tflops": workloads.dense_flop(shape) * args.layers / step / 1e12,
        "gpu_event_ms_per_step": gpu / args.steps * 1e3 if gpu >= 0 else None,
        "kernel_us": {"attention_f16_norm_rope": attn_avg * 1e6,
                      "norm_rope_f16": float(np.mean(prologue)) * 1e6},
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": achieved / PEAK_HBM_GBS,
            "traffic": traffic,
            "algorithmic_bytes": nbytes,
            "kernel": "attention_f16_norm_rope",
            "mfma_tflops": flop / attn_avg / 1e12,
        },
    }
    if not args.no_cpu_baseline:
        log("cpu baseline")
        expected, baseline = cpu_baseline(shape, lengths, host0)
        result["cpu_baseline"] = baseline
        result["max_abs_err_layer0"] = float(np.max(np.abs(out0.astype(np.float64) - expected)))
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
