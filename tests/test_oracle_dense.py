"""The oracle's dense decode (orc_dense_attention), pinned on the CPU.

The reference's dense decode is SDPA over the visible cache
(src/refinekv/integrations/transformers.py:510-520):
softmax(q k^T / sqrt(D)) v.  Pins, each one independent of the oracle's C:
an fp64 brute force of that formula on the same bf16 inputs; two closed
forms (identical keys give the mean of the values, a dominant key gives its
own value row); and the reference's sparse path with every block expanded
(orc_sparse_attention, eps below every risk), which attends exactly the
prompt and suffix tokens in the same order and must agree bit for bit.
"""

import numpy as np
import pytest


def _bf16(oracle, x):
    return oracle.bf16_bits(np.asarray(x, np.float32))


def _value(oracle, bits):
    return oracle.bf16_value(bits).astype(np.float64)


def _brute(oracle, q, k, v):
    qb = _value(oracle, _bf16(oracle, q))
    s = np.einsum("hgd,htd->hgt", qb, _value(oracle, k)) / np.sqrt(q.shape[-1])
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    return np.einsum("hgt,htd->hgd", p, _value(oracle, v))


@pytest.mark.parametrize("H,G,D,L", [(1, 1, 16, 1), (2, 3, 64, 37), (1, 7, 128, 300),
                                     (3, 2, 160, 65), (1, 16, 32, 513)])
def test_dense_matches_fp64_brute_force(oracle_lib, H, G, D, L):
    rng = np.random.default_rng(H * 1000 + L)
    q = rng.standard_normal((H, G, D)).astype(np.float32)
    k = _bf16(oracle_lib, 2.0 * rng.standard_normal((H, L, D)))
    v = _bf16(oracle_lib, rng.standard_normal((H, L, D)))
    got = oracle_lib.dense_attention(q, k, v)
    want = _brute(oracle_lib, q, k, v)
    assert np.abs(got - want).max() <= 2e-6 * max(1.0, np.abs(want).max())


def test_identical_keys_give_the_mean_value(oracle_lib):
    rng = np.random.default_rng(7)
    H, G, D, L = 2, 4, 64, 200
    q = rng.standard_normal((H, G, D)).astype(np.float32)
    key = rng.standard_normal((H, 1, D))
    k = _bf16(oracle_lib, np.repeat(key, L, axis=1))
    v = _bf16(oracle_lib, rng.standard_normal((H, L, D)))
    got = oracle_lib.dense_attention(q, k, v)
    want = np.broadcast_to(_value(oracle_lib, v).mean(axis=1, keepdims=True), (H, G, D))
    assert np.abs(got - want).max() <= 1e-6


def test_dominant_key_gives_its_value_row(oracle_lib):
    rng = np.random.default_rng(3)
    H, G, D, L, hot = 1, 2, 32, 50, 17
    q = np.ones((H, G, D), np.float32)
    keys = 0.01 * rng.standard_normal((H, L, D))
    keys[:, hot] = 40.0  # logit 40 * 32 / sqrt(32) ~ 226 above the others
    k = _bf16(oracle_lib, keys)
    v = _bf16(oracle_lib, rng.standard_normal((H, L, D)))
    got = oracle_lib.dense_attention(q, k, v)
    want = _value(oracle_lib, v)[:, hot][:, None, :].astype(np.float32)
    assert np.array_equal(got, np.broadcast_to(want, got.shape))


@pytest.mark.parametrize("B,L,S", [(16, 100, 3), (32, 64, 0), (64, 300, 7)])
def test_dense_equals_sparse_with_every_block_expanded(oracle_lib, B, L, S):
    """reference.py:50-73 with no representative left is dense attention over
    the prompt followed by the suffix."""
    rng = np.random.default_rng(B + L + S)
    H, G, D = 2, 4, 64
    q = rng.standard_normal((H, G, D)).astype(np.float32)
    keys = rng.standard_normal((H, L + S, D)).astype(np.float32)
    values = rng.standard_normal((H, L + S, D)).astype(np.float32)
    summ = oracle_lib.summary(keys[:, :L], values[:, :L], B)
    N = -(-L // B)
    pad = np.zeros((H, N * B, D), np.float32)
    kp, vp = pad.copy(), pad.copy()
    kp[:, :L], vp[:, :L] = keys[:, :L], values[:, :L]
    k_bits, v_bits = _bf16(oracle_lib, keys), _bf16(oracle_lib, values)
    out, mask = oracle_lib.sparse_attention(
        q, summ, _bf16(oracle_lib, kp), _bf16(oracle_lib, vp), k_bits[:, L:], v_bits[:, L:],
        -1.0, "any")
    assert mask.all()
    dense = oracle_lib.dense_attention(q, k_bits, v_bits)
    assert np.array_equal(dense, out)
