"""The allocation-free entry point mi_attention_norm_rope_noalloc, through the C ABI, against the
attention_f16_norm_rope route (HipRuntime._attention_norm_rope -> mi_dispatch) on the same inputs.

Both run the same kernels on the same inputs; the no-alloc entry point keeps its RoPE tables and
k planes in the library's static scratch, built by the same kernels, so the outputs must be
bit-identical. Three calls in a row on one process share that scratch, each smaller than the one
before, so a stale value left by a larger call would show. Each output is also checked against
the float64 oracle at the route's own bars. The caller's device memory comes from hipMalloc of
the HIP runtime the library is linked against."""

import ctypes as ct

import numpy as np
import pytest

from oracle import attention as ref
from oracle import norm_rope
from tessery_amd import HipRuntime, runtime as rtmod, workloads

pytestmark = pytest.mark.gpu

H2D, D2H = 1, 2


class DeviceMemory:
    """hipMalloc'd buffers of the caller (the entry point allocates none of its own)."""

    def __init__(self):
        # loaded after libtessery_hip.so: the soname resolves to the HIP runtime it already uses
        self.hip = ct.CDLL("libamdhip64.so.7")
        self.hip.hipMalloc.argtypes = [ct.POINTER(ct.c_void_p), ct.c_size_t]
        self.hip.hipMemcpy.argtypes = [ct.c_void_p, ct.c_void_p, ct.c_size_t, ct.c_int]
        self.hip.hipFree.argtypes = [ct.c_void_p]
        self.pointers = []

    def upload(self, array):
        array = np.ascontiguousarray(array)
        ptr = self.alloc(array.nbytes)
        assert self.hip.hipMemcpy(ptr, array.ctypes.data, array.nbytes, H2D) == 0
        return ptr

    def alloc(self, nbytes):
        ptr = ct.c_void_p()
        assert self.hip.hipMalloc(ct.byref(ptr), nbytes) == 0
        self.pointers.append(ptr.value)
        return ptr.value

    def download(self, ptr, shape, dtype):
        result = np.empty(shape, dtype)
        assert self.hip.hipDeviceSynchronize() == 0
        assert self.hip.hipMemcpy(result.ctypes.data, ptr, result.nbytes, D2H) == 0
        return result

    def close(self):
        self.hip.hipDeviceSynchronize()
        for ptr in self.pointers:
            self.hip.hipFree(ptr)
        self.pointers.clear()


def route_output(rt, t, lengths, shape, out_dtype, bidirectional):
    """The existing entry point: the attention_f16_norm_rope route through mi_dispatch."""
    odt = np.float16 if out_dtype == "f16" else np.float32
    bufs = [rt.upload(a) for a in (t["q"], t["k"], t["v"], lengths)]
    bufs.append(rt.buffer(t["q"].size * np.dtype(odt).itemsize))
    bufs += [rt.upload(t["q_norm"]), rt.upload(t["k_norm"]), rt.buffer(2 * t["k"].nbytes)]
    try:
        with rt.command():
            rt._attention_norm_rope(bufs, tokens=shape.tokens, seq=shape.seq, heads=shape.heads,
                                    kv_heads=shape.kv_heads, dim=shape.dim, eps=workloads.EPS,
                                    theta=workloads.THETA, bidirectional=bidirectional,
                                    out_dtype=out_dtype)
        return rt.read(bufs[4], t["q"].shape, odt)
    finally:
        for b in bufs:
            b.close()


def noalloc_output(lib, mem, t, lengths, shape, out_dtype, bidirectional):
    odt = np.float16 if out_dtype == "f16" else np.float32
    q, k, v, lens, qn, kn = (mem.upload(a) for a in (t["q"], t["k"], t["v"], lengths,
                                                     t["q_norm"], t["k_norm"]))
    out = mem.alloc(t["q"].size * np.dtype(odt).itemsize)
    status = lib.mi_attention_norm_rope_noalloc(
        q, k, v, lens, out, qn, kn, shape.batch, shape.seq, shape.heads, shape.kv_heads,
        shape.dim, workloads.EPS, workloads.THETA, bidirectional, int(out_dtype == "f16"), None)
    assert status == 0
    return mem.download(out, t["q"].shape, odt)


def oracle_output(t, lengths, bidirectional):
    qn = workloads.bf16_values(t["q_norm"]).astype(np.float64)
    kn = workloads.bf16_values(t["k_norm"]).astype(np.float64)
    q = norm_rope.norm_rope(t["q"], qn, workloads.EPS, workloads.THETA)
    k = norm_rope.norm_rope(t["k"], kn, workloads.EPS, workloads.THETA)
    return ref.attention(q, k, t["v"], lengths, bidirectional=bool(bidirectional))


# (batch, seq, heads, kv_heads, dim, lengths, out dtype, bidirectional), largest first
CALLS = [
    (8, 512, 16, 8, 128, (512, 1, 300, 77, 512, 129, 64, 2), "f32", 0),
    (3, 200, 16, 8, 128, (200, 17, 1), "f16", 0),
    (2, 72, 8, 2, 64, (72, 40), "f32", 1),
]


def test_noalloc_matches_route_on_successive_calls():
    with HipRuntime() as rt:
        lib = rtmod._library()
        mem = DeviceMemory()
        try:
            for i, (b, s, h, kv, d, lens, out_dtype, bidi) in enumerate(CALLS):
                print(f"call {i}: B={b} S={s} H={h} KV={kv} D={d} out={out_dtype} bidi={bidi}",
                      flush=True)
                shape = workloads.Shape(b, s, h, kv, d, causal=not bidi)
                lengths = np.array(lens, np.uint32)
                t = workloads.qwen_layer(shape, 0, seed=40 + i)
                expected = route_output(rt, t, lengths, shape, out_dtype, bidi)
                got = noalloc_output(lib, mem, t, lengths, shape, out_dtype, bidi)
                mem.close()
                np.testing.assert_array_equal(got, expected)
                bar = 1e-4 if out_dtype == "f32" else 2e-3
                err = np.max(np.abs(got.astype(np.float64) - oracle_output(t, lengths, bidi)))
                assert err <= bar, err
        finally:
            mem.close()


def test_noalloc_rejects_shapes_beyond_its_scratch():
    """32 x 1024 tokens x 8 kv heads x 128 need 128 MiB of k planes: refused with status 2 before
    anything is launched (the pointers are never touched)."""
    with HipRuntime():
        lib = rtmod._library()
        fake = 256  # non-null stand-ins: the call returns before using any pointer
        args = [fake] * 7
        status = lib.mi_attention_norm_rope_noalloc(*args, 32, 1024, 16, 8, 128, 1e-6, 1e6, 0,
                                                    0, None)
        assert status == 2
        # invalid arguments are status 1: head dim outside {64, 128}
        status = lib.mi_attention_norm_rope_noalloc(*args, 1, 16, 16, 8, 96, 1e-6, 1e6, 0, 0,
                                                    None)
        assert status == 1


def test_noalloc_under_graph_capture():
    """The first call of the entry point in a fresh process made under hipStreamBeginCapture
    (global mode), the graph replayed three times with eager calls of another shape in between:
    every replay bit-equal to the route (tests/noalloc_capture_child.py)."""
    import json
    import subprocess
    import sys
    from pathlib import Path

    child = Path(__file__).resolve().parent / "noalloc_capture_child.py"
    print("child: graph capture of mi_attention_norm_rope_noalloc", flush=True)
    proc = subprocess.run([sys.executable, "-u", str(child)], capture_output=True, text=True,
                          timeout=110)
    lines = [line for line in proc.stdout.splitlines() if line.startswith("capture-result ")]
    assert lines, proc.stdout[-2000:] + proc.stderr[-2000:]
    result = json.loads(lines[-1][len("capture-result "):])
    assert result["status_under_capture"] == 0 and result["end_capture"] == 0, result
    assert result["replays_bit_equal"] == [True] * 6, result
    assert proc.returncode == 0, proc.stderr[-2000:]
