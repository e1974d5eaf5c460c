"""Pins the float64 attention oracle against independent references, so a plausible mistake
(wrong GQA mapping, causal off-by-one, padded rows treated as masked, missing scale) fails."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as ref


def _sdpa(q, k, v, lengths, bidirectional):
    """torch SDPA in float64 with masks built from tril() and key padding."""
    b, s, h, d = q.shape
    out = np.empty((b, s, h, d))
    for i in range(b):
        length = int(lengths[i])
        keys = torch.arange(s)[None, :] < length
        mask = keys.expand(s, s).clone()
        if not bidirectional:
            mask &= torch.ones(s, s, dtype=torch.bool).tril()
        # padded query rows p >= L attend every valid key
        tq = torch.from_numpy(q[i].astype(np.float64)).transpose(0, 1)[None]
        tk = torch.from_numpy(k[i].astype(np.float64)).transpose(0, 1)[None]
        tv = torch.from_numpy(v[i].astype(np.float64)).transpose(0, 1)[None]
        o = F.scaled_dot_product_attention(tq, tk, tv, attn_mask=mask[None, None], enable_gqa=True)
        out[i] = o[0].transpose(0, 1).numpy()
    return out


@pytest.mark.parametrize("bidirectional", [False, True])
@pytest.mark.parametrize(
    "b,s,h,kv,d,lengths",
    [
        (2, 5, 4, 2, 64, (5, 2)),  # tessery test_kernels.py:127-157 shape
        (2, 65, 4, 2, 32, (1, 65)),
        (3, 40, 6, 2, 16, (40, 17, 1)),
        (1, 33, 2, 2, 128, (33,)),
        (2, 9, 8, 1, 8, (3, 9)),
    ],
)
def test_oracle_matches_torch_sdpa(b, s, h, kv, d, lengths, bidirectional):
    rng = np.random.default_rng(11)
    q = rng.normal(size=(b, s, h, d))
    k = rng.normal(size=(b, s, kv, d))
    v = rng.normal(size=(b, s, kv, d))
    lengths = np.array(lengths, np.uint32)
    got = ref.attention(q, k, v, lengths, bidirectional=bidirectional)
    np.testing.assert_allclose(got, _sdpa(q, k, v, lengths, bidirectional), atol=1e-12, rtol=1e-12)


def test_gqa_mapping_is_consecutive_heads():
    """Heads 2j and 2j+1 share kv head j: swapping kv heads must change heads 0,1 only."""
    rng = np.random.default_rng(3)
    q = rng.normal(size=(1, 7, 4, 8))
    k = rng.normal(size=(1, 7, 2, 8))
    v = rng.normal(size=(1, 7, 2, 8))
    lengths = np.array([7], np.uint32)
    base = ref.attention(q, k, v, lengths, bidirectional=False)
    k2, v2 = k.copy(), v.copy()
    k2[:, :, 0] = rng.normal(size=(1, 7, 8))
    v2[:, :, 0] = rng.normal(size=(1, 7, 8))
    changed = ref.attention(q, k2, v2, lengths, bidirectional=False)
    assert not np.allclose(base[:, :, :2], changed[:, :, :2])
    np.testing.assert_array_equal(base[:, :, 2:], changed[:, :, 2:])


def test_online_loop_agrees():
    rng = np.random.default_rng(5)
    q = rng.normal(size=(2, 6, 4, 8))
    k = rng.normal(size=(2, 6, 2, 8))
    v = rng.normal(size=(2, 6, 2, 8))
    lengths = np.array([6, 3], np.uint32)
    for bidirectional in (False, True):
        a = ref.attention(q, k, v, lengths, bidirectional=bidirectional)
        b = ref.attention_online(q, k, v, lengths, bidirectional=bidirectional)
        np.testing.assert_allclose(a, b, atol=1e-12)


def test_padded_query_rows_attend_all_valid_keys():
    rng = np.random.default_rng(9)
    q = rng.normal(size=(1, 10, 1, 4))
    k = rng.normal(size=(1, 10, 1, 4))
    v = rng.normal(size=(1, 10, 1, 4))
    lengths = np.array([4], np.uint32)
    causal = ref.attention(q, k, v, lengths, bidirectional=False)
    bidi = ref.attention(q, k, v, lengths, bidirectional=True)
    # positions >= L see the same keys in both modes
    np.testing.assert_allclose(causal[0, 4:], bidi[0, 4:], atol=1e-14)
    # position 0 sees only key 0: output equals v[0]
    np.testing.assert_allclose(causal[0, 0, 0], v[0, 0, 0], atol=1e-14)


@pytest.mark.parametrize("bidirectional", [False, True])
@pytest.mark.parametrize("pattern", ["alternating", "later_maximum", "uniform"])
@pytest.mark.parametrize("seq", [65, 128, 129])
def test_extreme_logit_known_answers(bidirectional, pattern, seq):
    """Closed forms of tessery test_kernels.py:213-253: with logits near +-1131 the softmax is a
    uniform mean over the maximal keys."""
    rng = np.random.default_rng(718)
    heads, dim = 2, 128
    q = np.full((1, seq, heads, dim), 10, np.float32)
    k = q.copy()
    k[:, 1::2] *= -1
    if pattern == "later_maximum":
        k[:] = -10
        k[:, 32:64] = 10
    elif pattern == "uniform":
        k[:] = 0
    v = rng.normal(size=q.shape).astype(np.float32)
    length = 65 if pattern == "later_maximum" else 33
    v[:, length:] = 1e10
    got = ref.attention(q, k, v, np.array([length], np.uint32), bidirectional=bidirectional)
    for pos in range(seq):
        end = length if bidirectional else min(pos + 1, length)
        if pattern == "later_maximum":
            chosen = v[0, 32 : min(end, 64)] if end > 32 else v[0, :end]
        elif pattern == "alternating":
            chosen = v[0, :end:2]
        else:
            chosen = v[0, :end]
        np.testing.assert_allclose(got[0, pos], chosen.astype(np.float64).mean(axis=0), atol=1e-9)
