"""Runtime lifecycle on the GPU: resources, workspace leases, aborts, profiling limits and plan
replay (the behaviour tessery's test_kernels.py:41-52, 578-647 checks on its Metal runtime)."""

import numpy as np
import pytest

from oracle import attention as ref
from tessery_amd import InferenceError
from tests.test_gpu_attention import check_f32

pytestmark = pytest.mark.gpu


def test_add_and_resources(runtime):
    rng = np.random.default_rng(42)
    a = rng.normal(size=(7, 37)).astype(np.float32)
    b = rng.normal(size=a.shape).astype(np.float32)
    np.testing.assert_array_equal(runtime.add(a, b), a + b)
    assert runtime.active_bytes == 0
    assert runtime.peak_bytes == a.nbytes * 3
    with pytest.raises(InferenceError):
        runtime.add(a, b[:1])
    with pytest.raises(InferenceError):
        runtime.buffer(0)


def test_workspace_reuse_bound_abort_and_trim(runtime):
    runtime.workspace_limit_bytes = 1024
    with runtime._workspace() as allocate:
        a, b = allocate(512), allocate(512)
        assert a is not b
        with runtime.command():
            runtime._dispatch("add", [a, b, a], threads=128, n=128)
    assert runtime.active_bytes == runtime.cache_bytes == 1024
    allocations = runtime.diagnostics()["allocations"]
    with pytest.raises(InferenceError), runtime._workspace() as allocate:
        recovered = allocate(512)
        with runtime.command():
            runtime._dispatch("nonexistent_kernel", [recovered], threads=1)
    assert runtime.diagnostics()["allocations"] == allocations
    with pytest.raises(InferenceError):
        allocate(512)
    with runtime._workspace() as allocate:
        large = allocate(2048)
        assert large.pointer
    assert not large.pointer
    assert runtime.cache_bytes <= 1024
    runtime.trim_workspace()
    assert runtime.active_bytes == runtime.cache_bytes == 0


def test_invalid_shapes_are_rejected_before_launch(runtime):
    """A buffer smaller than the shape Params imply is refused at dispatch time."""
    q = np.zeros((1, 64, 4, 32), np.float32)
    small = np.zeros((1, 32, 2, 32), np.float32)
    bufs = [runtime.upload(q), runtime.upload(small), runtime.upload(small),
            runtime.upload(np.array([64], np.uint32)), runtime.buffer(q.nbytes)]
    try:
        with pytest.raises(InferenceError), runtime.command():
            runtime._attention(bufs, tokens=64, seq=64, heads=4, kv_heads=2, dim=32)
        with pytest.raises(InferenceError), runtime.command():  # heads not a multiple of kv
            runtime._attention(bufs[:1] * 3 + bufs[3:], tokens=64, seq=64, heads=4, kv_heads=3, dim=32)
    finally:
        for b in bufs:
            b.close()


@pytest.mark.parametrize("case", ["gated_rows", "gated_threads", "gated_small_out", "matmul_small_w",
                                  "tiled_cols", "layer_norm_group", "silu_small_up", "gelu_zero"])
def test_layer_routes_reject_bad_launches(runtime, case):
    """The projection, gated and elementwise routes refuse launches whose thread formula or
    buffer sizes do not match Params, at dispatch time (nothing is queued)."""
    f = lambda *shape: runtime.buffer(int(np.prod(shape)) * 4)  # noqa: E731
    w32 = runtime.buffer(64 * (64 // 8) * 4)
    sb = runtime.buffer(64 * (64 // 64) * 2)
    bufs = [w32, sb]
    try:
        if case.startswith("gated"):
            x, out = f(16, 64), f(16 if case != "gated_small_out" else 8, 64)
            bufs += [x, out]
            rows = 8 if case == "gated_rows" else 16
            threads = 2 * 256 if case != "gated_threads" else 2 * 256 + 1
            args = dict(threads=threads, group_size=256, rows=rows, cols=64, k=64)
            with pytest.raises(InferenceError), runtime.command():
                runtime._dispatch("gated4_16x32_k64", [x, w32, sb, sb, w32, sb, sb, out], **args)
        elif case == "matmul_small_w":
            x, w, out = f(8, 64), f(32, 64), f(8, 64)
            bufs += [x, w, out]
            with pytest.raises(InferenceError), runtime.command():
                runtime._dispatch("matmul_f32_tiled", [x, w, out], threads=2 * 128, group_size=128,
                                  rows=8, cols=64, k=64)
        elif case == "tiled_cols":
            x, w, out = f(8, 64), f(48, 64), f(8, 48)
            bufs += [x, w, out]
            with pytest.raises(InferenceError), runtime.command():
                runtime._dispatch("matmul_f32_chunk32", [x, w, out], threads=128, group_size=128,
                                  rows=8, cols=48, k=64)
        elif case == "layer_norm_group":
            x, v = f(4, 64), f(64)
            bufs += [x, v]
            with pytest.raises(InferenceError), runtime.command():
                runtime._dispatch("layer_norm", [x, v, v, x], threads=4 * 64, group_size=64, cols=64)
        elif case == "silu_small_up":
            g, u = f(100), f(99)
            bufs += [g, u]
            with pytest.raises(InferenceError), runtime.command():
                runtime._dispatch("silu_gate", [g, u], threads=100, n=100)
        else:
            x = f(10)
            bufs += [x]
            with pytest.raises(InferenceError), runtime.command():
                runtime._dispatch("gelu_f32", [x], threads=1, n=0)
    finally:
        for b in bufs:
            b.close()
    assert runtime.active_bytes == 0


def test_aborted_command_launches_nothing(runtime):
    x = np.arange(64, dtype=np.float32)
    a, out = runtime.upload(x), runtime.upload(np.full(64, -1.0, np.float32))
    try:
        with pytest.raises(InferenceError), runtime.command():
            runtime._dispatch("add", [a, a, out], threads=64, n=64)
            runtime._dispatch("absent", [a], threads=1)
        np.testing.assert_array_equal(runtime.read(out, (64,)), -1.0)
    finally:
        a.close()
        out.close()


def test_profile_timings_abort_and_recovery(runtime):
    a = np.arange(4096, dtype=np.float32)
    with runtime.profile_kernels() as records:
        np.testing.assert_array_equal(runtime.add(a, a), a + a)
        assert len(records) == 1 and records[0]["kernel"] == "add"
        assert np.isfinite(records[0]["gpu_seconds"]) and records[0]["gpu_seconds"] > 0
        with pytest.raises(InferenceError), runtime.profile_kernels():
            pass
        with pytest.raises(InferenceError), runtime.command():
            runtime._dispatch("absent", [], threads=1)
        assert len(records) == 1
        np.testing.assert_array_equal(runtime.add(a, a), a + a)
        assert len(records) == 2
    assert runtime.active_bytes == 0


def test_profile_capacity_aborts_without_partial_results(runtime):
    a = np.ones(1, dtype=np.float32)
    buffers = [runtime.upload(a) for _ in range(3)]
    try:
        with runtime.profile_kernels() as records:
            with pytest.raises(InferenceError), runtime.command():
                for _ in range(2049):
                    runtime._dispatch("add", buffers, threads=1, n=1)
            assert records == []
            np.testing.assert_array_equal(runtime.add(a, a), a + a)
            assert len(records) == 1
    finally:
        for b in buffers:
            b.close()


def test_plan_capture_and_replay(runtime):
    rng = np.random.default_rng(12)
    q = rng.normal(size=(2, 128, 4, 32)).astype(np.float32)
    k, v = [rng.normal(size=(2, 128, 2, 32)).astype(np.float32) for _ in range(2)]
    lengths = np.array([128, 50], np.uint32)
    expected = ref.attention(q, k, v, lengths, bidirectional=False)
    outs = []
    for _ in range(3):
        with runtime._workspace() as new:
            with runtime.command():
                bufs = [new(a.nbytes, a) for a in (q, k, v, lengths)] + [new(q.nbytes)]
                with runtime._execution_plan(("attn", 2, 128), bufs) as replayed:
                    if not replayed:
                        runtime._attention(bufs, tokens=256, seq=128, heads=4, kv_heads=2, dim=32)
            outs.append(runtime.read(bufs[-1], q.shape))  # still inside the lease
    for out in outs:
        check_f32(out, expected)
    diag = runtime.diagnostics()
    assert diag["plan_builds"] == 1 and diag["plan_hits"] == 2
    assert diag["dispatches"] == {"attention_tiled": 3}


def test_plan_evicted_while_its_replay_is_queued(runtime):
    """A replayed plan evicted from the cache by later captures in the same command (the cache
    holds 4 plans) still runs its queued launches."""
    rng = np.random.default_rng(15)
    q = rng.normal(size=(1, 64, 2, 32)).astype(np.float32)
    k, v = [rng.normal(size=(1, 64, 2, 32)).astype(np.float32) for _ in range(2)]
    lengths = np.array([40], np.uint32)
    expected = ref.attention(q, k, v, lengths, bidirectional=False)
    bufs = [runtime.upload(a) for a in (q, k, v, lengths)] + [runtime.buffer(q.nbytes)]
    outs = [runtime.buffer(q.nbytes) for _ in range(5)]
    try:
        with runtime._workspace():
            def plan(key, out):
                binding = bufs[:4] + [out]
                with runtime._execution_plan(key, binding) as replayed:
                    if not replayed:
                        runtime._attention(binding, tokens=64, seq=64, heads=2, kv_heads=2, dim=32)

            with runtime.command():
                plan(("a",), bufs[4])          # capture A
            with runtime.command():
                plan(("a",), bufs[4])          # replay A (queued) ...
                for i in range(4):             # ... then four captures evict it
                    plan(("b", i), outs[i])
            assert runtime.diagnostics()["plan_hits"] == 1
            for out in [bufs[4]] + outs[:4]:
                check_f32(runtime.read(out, q.shape), expected)
    finally:
        for b in bufs + outs:
            b.close()


@pytest.mark.parametrize("case", ["emb4_cols", "emb4_short_out", "emb4_short_ids", "emb4_scales",
                                  "embpos_positions", "embpos_types", "pool_dim", "pool_lengths",
                                  "pool_group", "pool_short_x"])
def test_model_end_routes_reject_bad_launches(runtime, case):
    """embedding4, embedding_position and pool_project refuse launches whose Params or thread
    counts do not fit their buffers (kernels.metal:21-30, 339-360), at dispatch time."""
    f = lambda *shape: runtime.buffer(int(np.prod(shape)) * 4)  # noqa: E731
    bufs = []
    try:
        if case.startswith("emb4"):
            cols, tokens, vocab = 64 if case != "emb4_cols" else 40, 4, 10
            ids = f(tokens if case != "emb4_short_ids" else tokens - 1)
            w = runtime.buffer(vocab * (64 // 8) * 4)
            s = runtime.buffer(vocab * 2 * (1 if case != "emb4_scales" else 0) or 2)
            out = f(tokens * cols - (8 if case == "emb4_short_out" else 0))
            bufs += [ids, w, s, out]
            with pytest.raises(InferenceError), runtime.command():
                runtime._dispatch("embedding4", [ids, w, s, s, out], threads=tokens * cols,
                                  n=tokens * cols, cols=cols)
        elif case.startswith("embpos"):
            cols, seq, tokens = 32, 8, 16
            ids, words = f(tokens), f(5, cols)
            positions = f(seq - 1 if case == "embpos_positions" else seq, cols)
            types = f(cols - 1 if case == "embpos_types" else cols)
            out = f(tokens, cols)
            bufs += [ids, words, positions, types, out]
            with pytest.raises(InferenceError), runtime.command():
                runtime._dispatch("embedding_position", [ids, words, positions, types, out],
                                  threads=tokens * cols, n=tokens * cols, cols=cols, seq=seq)
        else:
            batch, seq, cols = 3, 4, 64
            x = f(batch * seq * cols - (1 if case == "pool_short_x" else 0))
            lengths = runtime.buffer((batch - 1 if case == "pool_lengths" else batch) * 4)
            out = f(batch, cols)
            bufs += [x, lengths, out]
            with pytest.raises(InferenceError), runtime.command():
                runtime._dispatch("pool_project", [x, lengths, out], threads=batch * 32,
                                  group_size=64 if case == "pool_group" else 32, seq=seq,
                                  cols=cols, dim=cols + 1 if case == "pool_dim" else cols)
    finally:
        for b in bufs:
            b.close()


def test_buffers_closed_inside_a_command_live_until_it_finishes(runtime):
    """Closing a buffer while a command is open frees nothing yet: the queued launch still reads
    and writes it at finish, and the memory is released afterwards (runtime.mm keeps encoded
    buffers alive the same way)."""
    rng = np.random.default_rng(21)
    a = rng.normal(size=4096).astype(np.float32)
    b = rng.normal(size=4096).astype(np.float32)
    out = runtime.buffer(a.nbytes)
    try:
        with runtime.command():
            x, y = runtime.upload(a), runtime.upload(b)
            runtime._dispatch("add", [x, y, out], threads=a.size, n=a.size)
            x.close()
            y.close()
            # a new allocation made while the closed ones are pending must not reuse their memory
            z = runtime.upload(np.zeros_like(a))
            runtime._dispatch("add", [z, z, z], threads=a.size, n=a.size)
        np.testing.assert_array_equal(runtime.read(out, a.shape), a + b)
        np.testing.assert_array_equal(runtime.read(z, a.shape), 0.0)
        z.close()
    finally:
        out.close()
    assert runtime.active_bytes == 0


@pytest.mark.parametrize("case", ["qkv4_k", "norm_rope_heads", "rms_norm_rows"])
def test_launcher_limits_are_rejected_at_dispatch(runtime, case):
    """Shapes whose buffers fit but which a launcher cannot run (qkv4_f16 beyond K = 8192, the
    k prologue beyond 256 lanes per position, row kernels beyond 2^26 - 4 rows) are refused by
    mi_dispatch, before anything is queued, not at finish."""
    bufs = []
    try:
        if case == "qkv4_k":
            m, k, nq, nkv = 128, 16384, 128, 128
            n = nq + 2 * nkv
            bufs += [runtime.buffer(m * k * 2), runtime.buffer(n * (k // 8) * 4),
                     runtime.buffer(n * (k // 64) * 2), runtime.buffer(n * (k // 64) * 2),
                     runtime.buffer(m * nq * 2), runtime.buffer(m * nkv * 2),
                     runtime.buffer(m * nkv * 2)]
            with pytest.raises(InferenceError), runtime.command():
                runtime._qkv4(bufs, rows=m, k=k, q_cols=nq, kv_cols=nkv, scale_dtype="f16")
        elif case == "norm_rope_heads":
            b, s, heads, d = 1, 16, 33, 128
            bufs += [runtime.buffer(b * s * heads * d * 2), runtime.buffer(d * 2),
                     runtime.buffer(b * 4), runtime.buffer(2 * b * s * heads * d * 2)]
            with pytest.raises(InferenceError), runtime.command():
                runtime._dispatch("norm_rope_f16", bufs, threads=b * s, group_size=256,
                                  heads=heads, seq=s, dim=d, flags=1)
        else:
            rows = (1 << 26) - 3
            bufs += [runtime.buffer(rows * 4), runtime.buffer(2), runtime.buffer(rows * 4)]
            with pytest.raises(InferenceError), runtime.command():
                runtime._dispatch("rms_norm", bufs, threads=rows * 32, group_size=32, cols=1)
        assert runtime.diagnostics()["completed_commands"] == 0
    finally:
        for b in bufs:
            b.close()
