"""Child process of test_zz_no_alloc.py::test_noalloc_under_graph_capture (run on its own so that
the entry point's first call, which looks up its scratch array, happens under stream capture).

Captures one call of mi_attention_norm_rope_noalloc on a new stream in global capture mode,
instantiates the graph and replays it three times; before each replay the output is poisoned with
NaN, and between replays an eager call of another shape overwrites the shared scratch. Every
replay's output is compared bit for bit with the attention_f16_norm_rope route on the same
inputs. Prints one line `capture-result <json>`."""

import ctypes as ct
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

from tessery_amd import HipRuntime, runtime as rtmod, workloads  # noqa: E402
from test_zz_no_alloc import DeviceMemory, route_output  # noqa: E402

CAPTURE_GLOBAL = 0


def main() -> int:
    lib = rtmod._library()
    mem = DeviceMemory()
    hip = mem.hip
    for name in ("hipStreamCreate", "hipStreamBeginCapture", "hipStreamEndCapture",
                 "hipGraphInstantiate", "hipGraphLaunch", "hipStreamSynchronize",
                 "hipGraphExecDestroy", "hipGraphDestroy", "hipStreamDestroy"):
        getattr(hip, name).restype = ct.c_int
    hip.hipStreamBeginCapture.argtypes = [ct.c_void_p, ct.c_int]
    hip.hipStreamEndCapture.argtypes = [ct.c_void_p, ct.POINTER(ct.c_void_p)]
    hip.hipGraphInstantiate.argtypes = [ct.POINTER(ct.c_void_p), ct.c_void_p, ct.c_void_p,
                                        ct.c_void_p, ct.c_size_t]
    hip.hipGraphLaunch.argtypes = [ct.c_void_p, ct.c_void_p]
    hip.hipStreamSynchronize.argtypes = [ct.c_void_p]

    shape = workloads.Shape(4, 256, 16, 8, 128, causal=True)
    lengths = np.array([256, 3, 131, 64], np.uint32)
    t = workloads.qwen_layer(shape, 0, seed=61)
    other = workloads.Shape(2, 96, 8, 2, 64, causal=False)
    other_lengths = np.array([96, 50], np.uint32)
    t2 = workloads.qwen_layer(other, 0, seed=62)

    def args(tt, lens, sh, out):
        q, k, v, ln, qn, kn = (mem.upload(a) for a in (tt["q"], tt["k"], tt["v"], lens,
                                                       tt["q_norm"], tt["k_norm"]))
        return (q, k, v, ln, out, qn, kn, sh.batch, sh.seq, sh.heads, sh.kv_heads, sh.dim,
                workloads.EPS, workloads.THETA, int(not sh.causal), 0)

    out = mem.alloc(t["q"].size * 4)
    out2 = mem.alloc(t2["q"].size * 4)
    main_args = args(t, lengths, shape, out)
    other_args = args(t2, other_lengths, other, out2)

    stream = ct.c_void_p()
    assert hip.hipStreamCreate(ct.byref(stream)) == 0
    assert hip.hipStreamBeginCapture(stream, CAPTURE_GLOBAL) == 0
    status = lib.mi_attention_norm_rope_noalloc(*main_args, stream)
    graph = ct.c_void_p()
    ended = hip.hipStreamEndCapture(stream, ct.byref(graph))
    result = {"status_under_capture": status, "end_capture": ended}
    if status != 0 or ended != 0 or not graph.value:
        print("capture-result " + json.dumps(result), flush=True)
        return 1
    exec_ = ct.c_void_p()
    assert hip.hipGraphInstantiate(ct.byref(exec_), graph, None, None, 0) == 0

    with HipRuntime() as rt:
        expected = route_output(rt, t, lengths, shape, "f32", 0)
        expected_other = route_output(rt, t2, other_lengths, other, "f32", 1)
    poison = np.full(t["q"].shape, np.nan, np.float32)
    replays = []
    for r in range(3):
        assert hip.hipMemcpy(out, poison.ctypes.data, poison.nbytes, 1) == 0
        assert hip.hipGraphLaunch(exec_, stream) == 0
        assert hip.hipStreamSynchronize(stream) == 0
        got = mem.download(out, t["q"].shape, np.float32)
        replays.append(bool(np.array_equal(got, expected)))
        # an eager call of another shape between replays rewrites the shared scratch
        assert lib.mi_attention_norm_rope_noalloc(*other_args, None) == 0
        got2 = mem.download(out2, t2["q"].shape, np.float32)
        replays.append(bool(np.array_equal(got2, expected_other)))
    hip.hipGraphExecDestroy(exec_)
    hip.hipGraphDestroy(graph)
    hip.hipStreamDestroy(stream)
    mem.close()
    result["replays_bit_equal"] = replays
    print("capture-result " + json.dumps(result), flush=True)
    return 0 if all(replays) else 1


if __name__ == "__main__":
    sys.exit(main())
