"""Route selection without a GPU: HipRuntime methods called unbound on a recorder, the pattern of
tessery's tests/unit/test_runtime_loading.py:9-106."""

import json

import numpy as np
from types import SimpleNamespace

import pytest

from tessery_amd.runtime import HipRuntime
from tests.conftest import GOLDEN

ROUTES = json.loads((GOLDEN / "routes.json").read_text())


def recorder():
    calls = []
    return calls, SimpleNamespace(_dispatch=lambda *a, **kw: calls.append((a, kw)))


@pytest.mark.parametrize("case", ROUTES["attention"], ids=lambda c: f"s{c['seq']}d{c['dim']}")
def test_attention_route_table(case):
    calls, fake = recorder()
    seq, dim = case["seq"], case["dim"]
    HipRuntime._attention(fake, [], tokens=2 * seq, seq=seq, heads=4, kv_heads=2, dim=dim)
    (args, kwargs), = calls
    assert args[0] == case["name"]
    assert kwargs["group_size"] == case["group_size"]
    assert kwargs["threads"] == case["threads"]
    assert kwargs["scale"] == dim**-0.5


@pytest.mark.parametrize("dim,name,group", [(32, "attention_f16_scalar", 64), (64, "attention_f16", 256),
                                            (128, "attention_f16", 256), (8, "attention_f16_scalar", 64),
                                            (96, "attention_f16_scalar", 64)])
@pytest.mark.parametrize("out_dtype,flag", [(None, 0), ("f32", 0), ("f16", 1)])
def test_f16_route(dim, name, group, out_dtype, flag):
    calls, fake = recorder()
    HipRuntime._attention(fake, [], tokens=3 * 77, seq=77, heads=16, kv_heads=8, dim=dim,
                          precision="f16", out_dtype=out_dtype)
    (args, kwargs), = calls
    assert args[0] == name and kwargs["group_size"] == group and kwargs["threads"] == 231
    assert kwargs["out_f16"] == flag


def test_norm_rope_route_sequence():
    calls, fake = recorder()
    bufs = list("abcdefgh")
    HipRuntime._attention_norm_rope(fake, bufs, tokens=1024, seq=512, heads=16, kv_heads=8,
                                    dim=128, eps=1e-6, theta=1e6)
    assert [a[0] for a, _ in calls] == ["norm_rope_f16", "attention_f16_norm_rope"]
    assert calls[0][0][1] == ["b", "g", "d", "h"]
    assert calls[0][1]["heads"] == 8 and calls[0][1]["flags"] == 1  # hi + lo planes
    assert calls[1][0][1] == ["a", "h", "c", "d", "e", "f"]
    assert calls[1][1]["heads"] == 16 and calls[1][1]["kv_heads"] == 8 and calls[1][1]["out_f16"] == 0
    calls.clear()
    HipRuntime._attention_norm_rope(fake, bufs, tokens=1024, seq=512, heads=16, kv_heads=8,
                                    dim=128, out_dtype="f16")
    assert calls[1][1]["out_f16"] == 1


@pytest.mark.parametrize("rows,cols,k,selected", ROUTES["linear4"]["small3"])
def test_three_row_projection_guard(rows, cols, k, selected):
    calls, fake = recorder()
    HipRuntime._linear4(fake, [], rows=rows, cols=cols, k=k)
    assert any(a[0] == "linear4_small3" for a, _ in calls) == selected
    if selected:
        assert len(calls) == 1
        assert calls[0][1] == dict(threads=cols * 32, group_size=32, rows=3, cols=cols, k=k)


@pytest.mark.parametrize("rows,cols,k,selected", ROUTES["linear4"]["large"])
def test_large_tile_partition(rows, cols, k, selected):
    calls, fake = recorder()
    HipRuntime._linear4(fake, [], rows=rows, cols=cols, k=k)
    assert (calls[0][0][0] in ("linear4_16x32_k64", "linear4_32x32_k64")) == selected
    if selected and calls[0][0][0] == "linear4_16x32_k64":
        assert len(calls) == 1 + bool(rows % 16 >= 8) + bool(rows % 8)
        regions = [(0, rows // 16 * 16)]
        for args, kwargs in calls[1:]:
            start = kwargs["n"]
            end = start + 8 if args[0] == "linear4_tiled" else rows
            regions.append((start, end))
        assert regions[0][0] == 0 and regions[-1][1] == rows
        assert all(a[1] == b[0] for a, b in zip(regions[:-1], regions[1:]))


GATED_CASES = [(m, 3072, 1024) for m in (7, 16, 23, 24, 25, 48, 127, 128, 129, 159, 160, 161, 255,
                                         256, 257, 511, 512, 513, 4096)]
GATED_CASES += [(m, n, k) for m in (24, 128, 160) for n, k in ((1024, 1024), (3072, 2048), (3071, 1024))]


@pytest.mark.parametrize("rows,cols,k", GATED_CASES)
def test_gated_projection_guard_and_buffer_binding(rows, cols, k):
    """The fused gate/up selection and buffer binding of tessery's
    test_runtime_loading.py:167-218 (metal.py:501-530)."""
    calls = []
    fake = SimpleNamespace(
        _dispatch=lambda *a, **kw: calls.append(("dispatch", a, kw)),
        _linear4=lambda *a, **kw: calls.append(("linear", a, kw)),
    )
    buffers = [object() for _ in range(9)]
    HipRuntime._gated4(fake, buffers, rows=rows, cols=cols, k=k)
    if rows in (16, 24, 128, 160, 256, 512) and (cols, k) == (3072, 1024):
        assert len(calls) == (2 if rows == 24 else 1)
        assert calls[0][1] == ("gated4_16x32_k64", buffers[:8])
        assert calls[0][2] == dict(threads=rows // 16 * (cols // 32) * 256, group_size=256,
                                   rows=rows, cols=cols, k=k)
        if rows == 24:
            assert calls[1][1] == ("gated4_8x32", buffers[:8])
            assert calls[1][2] == dict(threads=(cols // 32) * 128, group_size=128, n=16,
                                       rows=rows, cols=cols, k=k)
    else:
        assert [c[0] for c in calls] == ["linear", "linear", "dispatch"]
        assert calls[0][1][0] == [*buffers[:4], buffers[7]]
        assert calls[1][1][0] == [buffers[0], *buffers[4:7], buffers[8]]
        assert calls[2][1] == ("silu_gate", buffers[7:])
        assert calls[2][2] == dict(threads=rows * cols, n=rows * cols)


BGE_SHAPES = ((384, 384), (1536, 384), (384, 1536))


@pytest.mark.parametrize("rows", [1, 7, 8, 9, 12, 15, 16, 129, 4096])
@pytest.mark.parametrize("cols,k", [(384, 384), (1536, 384), (384, 1536), (385, 384), (384, 1535),
                                    (384, 512), (384, 2048)])
def test_f32_verified_shapes_and_tail_dispatch(rows, cols, k):
    """_matmul_f32's partition (metal.py:664-700; test_runtime_loading.py:133-164)."""
    calls, fake = recorder()
    HipRuntime._matmul_f32(fake, [], rows=rows, cols=cols, k=k)
    if rows >= 8 and (cols, k) in BGE_SHAPES:
        assert calls[0][0][0] == "matmul_f32_chunk32"
        assert calls[0][1] == dict(threads=(rows // 8) * (cols // 32) * 128, group_size=128,
                                   rows=rows, cols=cols, k=k)
        assert len(calls) == 1 + bool(rows % 8)
        if rows % 8:
            assert calls[1][0][0] == "matmul_f32"
            assert calls[1][1] == dict(threads=((rows % 8 + 3) // 4) * cols * 32, group_size=32,
                                       n=rows // 8 * 8, rows=rows, cols=cols, k=k)
    else:
        tiled = rows >= 8 and rows % 8 == 0 and cols % 32 == 0 and k % 8 == 0 and k <= 512
        assert len(calls) == 1
        assert calls[0][0][0] == ("matmul_f32_tiled" if tiled else "matmul_f32")
        assert calls[0][1].get("n", 0) == 0


@pytest.mark.parametrize("rows", [1, 7, 8, 9, 15, 16, 129, 4096])
@pytest.mark.parametrize("cols,k", [(384, 384), (1536, 384), (384, 1536), (385, 384)])
def test_bge_affine_guarded_dispatch(rows, cols, k):
    """_matmul_bias_f32's partition and binding (metal.py:702-731;
    test_runtime_loading.py:219-262)."""
    calls = []
    fake = SimpleNamespace(
        _dispatch=lambda *a, **kw: calls.append((a, kw)),
        _matmul_f32=lambda *a, **kw: calls.append((("old_matmul", *a), kw)),
    )
    buffers = [object() for _ in range(4)]
    HipRuntime._matmul_bias_f32(fake, buffers, rows=rows, cols=cols, k=k)
    if cols == 385 or rows < 8:
        assert [c[0][0] for c in calls] == ["old_matmul", "add_bias"]
        assert calls[0][0][1] == buffers[:3]
        assert calls[1][0][1] == buffers[2:]
        assert calls[1][1] == dict(threads=rows * cols, n=rows * cols, cols=cols)
    else:
        expected = ["matmul_bias_f32_chunk32"] + (["matmul_bias_f32"] if rows % 8 else [])
        assert [c[0][0] for c in calls] == expected
        assert all(c[0][1] == buffers for c in calls)
        if rows % 8:
            assert calls[-1][1]["n"] == rows // 8 * 8


def launch_rows(launch, rows, cols):
    """Rows a launch covers, from its thread count (the row regions mi_dispatch derives,
    kernels.metal:32-51, 489-605, 655-684, 733-773, 306-322, 396-487)."""
    n = launch.fields.get("n", 0)
    if launch.name in ("linear4", "matmul_f32", "matmul_bias_f32"):
        return n, min(n + 4 * (launch.threads // (cols * 32)), rows)
    if launch.name in ("linear4_tiled", "matmul_f32_chunk32", "matmul_bias_f32_chunk32",
                       "matmul_f32_tiled"):
        return n, n + 8 * (launch.threads // ((cols // 32) * 128))
    if launch.name == "linear4_tail":
        return n, min(n + 8, rows)
    if launch.name in ("linear4_16x32_k64", "linear4_32x32_k64"):
        tile = 16 if "16x32" in launch.name else 32
        return 0, tile * (launch.threads // ((cols // 32) * 256))
    assert launch.name == "linear4_small3"
    return 0, 3


@pytest.mark.parametrize("cols,k", [(1024, 1024), (2048, 1024), (3072, 1024), (1024, 3072),
                                    (64, 128), (96, 64), (1025, 1024), (384, 384), (385, 384),
                                    (1536, 384), (384, 1536), (384, 2048)])
def test_planners_cover_every_row_once(cols, k):
    """linear4_plan and the dense planners cover rows [0, rows) exactly once at every height."""
    from tessery_amd.runtime import linear4_plan, matmul_bias_plan, matmul_plan

    for rows in range(1, 600):
        plans = [linear4_plan(rows=rows, cols=cols, k=k), matmul_plan(rows=rows, cols=cols, k=k)]
        bias = matmul_bias_plan(rows=rows, cols=cols, k=k)
        if bias is not None:
            plans.append(bias)
        for plan in plans:
            covered = np.zeros(rows, int)
            for launch in plan:
                start, end = launch_rows(launch, rows, cols)
                assert 0 <= start < end <= rows, (launch, rows)
                covered[start:end] += 1
            assert (covered == 1).all(), (rows, cols, k, plan)
