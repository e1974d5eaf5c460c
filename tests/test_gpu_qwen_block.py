"""Qwen3 attention block on fp16 activations, through the C ABI: uint4 QKV projection (one qkv4
launch) -> k norm + RoPE prologue -> fused q norm + RoPE attention. This is the op order of
qwen3.py:194-245 on the seeded 16x256 workload (x [4096, 1024], W_q 1024->2048, W_k / W_v
1024->1024, group-64 fp16 scale/bias, lengths U{1..256}).

Each stage is held to its own bar against float64:
  * projection: every output within fp16 rounding of the exact product (2^-11 |y| + 1e-4);
  * attention: max-abs <= 1e-4 (the fp32 bar) against the float64 oracle evaluated on the
    projection's fp16 outputs (the attention operands of this path are fp16 by definition; the
    fused route carries normalized q, k and P as hi + lo fp16 pairs and writes fp32).
The projection outputs reach |y| ~ 6, where one fp16 ulp is 2^-8, so the chain as a whole is
compared with an all-float64 chain only for the record (printed), not against a bar."""

import numpy as np
import pytest

from oracle import attention as ref_attention
from oracle import norm_rope as ref_norm_rope
from oracle import quant4 as ref_quant4
from tessery_amd import workloads

pytestmark = pytest.mark.gpu

FUSED_F32_MAX = 1e-4


def test_qkv4_norm_rope_attention_16x256(runtime):
    shape, lengths, d = workloads.qwen_qkv4_16x256()
    b, s, h, kv, dim = shape.batch, shape.seq, shape.heads, shape.kv_heads, shape.dim
    m, k_in = d["x"].shape
    nq, nkv = h * dim, kv * dim
    bufs = {name: runtime.upload(d[name]) for name in ("x", "w", "s", "b", "q_norm", "k_norm")}
    yq, yk, yv = (runtime.buffer(m * n * 2) for n in (nq, nkv, nkv))
    lens = runtime.upload(lengths)
    out = runtime.buffer(m * nq * 4)
    k_work = runtime.buffer(2 * m * nkv * 2)
    try:
        with runtime.command():
            runtime._qkv4([bufs["x"], bufs["w"], bufs["s"], bufs["b"], yq, yk, yv], rows=m,
                          k=k_in, q_cols=nq, kv_cols=nkv, scale_dtype="f16")
            runtime._attention_norm_rope(
                [yq, yk, yv, lens, out, bufs["q_norm"], bufs["k_norm"], k_work], tokens=m,
                seq=s, heads=h, kv_heads=kv, dim=dim, eps=workloads.EPS, theta=workloads.THETA)
        y = [runtime.read(buf, (m, n), np.float16) for buf, n in ((yq, nq), (yk, nkv), (yv, nkv))]
        got = runtime.read(out, (b, s, h, dim))
    finally:
        for buf in (*bufs.values(), yq, yk, yv, lens, out, k_work):
            buf.close()

    # projection stage
    rows = np.split(np.arange(nq + 2 * nkv), [nq, nq + nkv])
    exact = []
    for part, got_y in zip(rows, y):
        e = ref_quant4.linear4(d["x"], d["w"][part], d["s"][part], d["b"][part], "f16")
        err = np.abs(got_y.astype(np.float64) - e)
        assert np.all(err <= 2.0**-11 * np.abs(e) + 1e-4), float(err.max())
        exact.append(e)

    # attention stage, on the fp16 projection outputs
    gq = workloads.bf16_values(d["q_norm"]).astype(np.float64)
    gk = workloads.bf16_values(d["k_norm"]).astype(np.float64)

    def chain(q, k, v):
        qn = ref_norm_rope.norm_rope(q.reshape(b, s, h, dim), gq, workloads.EPS, workloads.THETA)
        kn = ref_norm_rope.norm_rope(k.reshape(b, s, kv, dim), gk, workloads.EPS, workloads.THETA)
        return ref_attention.attention(qn, kn, v.reshape(b, s, kv, dim), lengths,
                                       bidirectional=False)

    expected = chain(*(t.astype(np.float64) for t in y))
    err = float(np.max(np.abs(got.astype(np.float64) - expected)))
    assert err <= FUSED_F32_MAX, err
    end_to_end = float(np.max(np.abs(got.astype(np.float64) - chain(*exact))))
    print(f"attention stage max-abs {err:.3e}; against the all-float64 chain {end_to_end:.3e}")
