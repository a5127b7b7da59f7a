"""Pin the oracle's elementary functions and the risk algebra.

exp/log are checked against fp64 libm (<= 1 and 2 ulp) with their special
values; the bf16 cast against torch's own cast; the direct (delta <= 10)
risk branch, which has no published known answer, against an fp64 closed
form of reference.py:10-34; selection special cases against the reference's
own CPU tests (tests/test_attention.py:74-128).
"""

import numpy as np
import pytest
import torch

from refinekv import testing


def _ulps(got, want):
    got = np.asarray(got, np.float64)
    want32 = np.asarray(want, np.float64).astype(np.float32)
    spacing = np.spacing(np.abs(want32)).astype(np.float64)
    return np.abs(got - want) / spacing


def test_expf_accuracy_and_special_values(oracle_lib):
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.uniform(-104, 89, 200000), rng.uniform(-1, 1, 100000),
                        np.linspace(-103.9, -87, 5000)]).astype(np.float32)
    y = oracle_lib.expf(x)
    want = np.exp(x.astype(np.float64))
    big = want >= 2.0 ** 128 * (1 - 2.0 ** -25)
    assert (y[big] == np.inf).all()
    normal = (want > 1.2e-38) & ~big
    assert _ulps(y[normal], want[normal]).max() <= 1.0
    sub = want <= 1.2e-38
    assert np.abs(y[sub] - want[sub]).max() <= 2.0 ** -149
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 88.72283, 88.7229, -104.5], np.float32)
    s = oracle_lib.expf(special)
    assert s[0] == 1.0 and s[1] == 1.0 and s[2] == np.inf and s[3] == 0.0
    assert np.isnan(s[4]) and np.isfinite(s[5]) and s[6] == np.inf and s[7] == 0.0


def test_logf_accuracy_and_special_values(oracle_lib):
    rng = np.random.default_rng(1)
    x = np.concatenate([np.exp(rng.uniform(-87, 88, 200000)), rng.uniform(0.5, 2, 100000),
                        np.arange(1, 129), np.array([1e-40, 1e-45, 3.4e38])]).astype(np.float32)
    y = oracle_lib.logf(x)
    want = np.log(x.astype(np.float64))
    assert _ulps(y, want).max() <= 2.0
    s = oracle_lib.logf(np.array([1.0, 0.0, -1.0, np.inf, np.nan], np.float32))
    assert s[0] == 0.0 and not np.signbit(s[0]) and s[1] == -np.inf
    assert np.isnan(s[2]) and s[3] == np.inf and np.isnan(s[4])


def test_bf16_rounding_matches_torch(oracle_lib):
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.standard_normal(100000) * np.exp(rng.uniform(-30, 30, 100000)),
                        [np.inf, -np.inf, 3.4e38, 1e-40, 0.0, -0.0]]).astype(np.float32)
    ties = (rng.integers(0, 2 ** 16, 1000).astype(np.uint32) << 16 | 0x8000).view(np.float32)
    x = np.concatenate([x, ties[np.isfinite(ties)]])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle_lib.bf16_bits(x), want)
    assert oracle_lib.bf16_bits(np.array([np.nan], np.float32))[0] == 0x7FC0


def _stats64(q, summ, D):
    """fp64 closed form of selection_statistics on tiny inputs."""
    qt = torch.from_numpy(q).to(torch.bfloat16).double()
    q2 = (qt.float() ** 2).to(torch.bfloat16).double()
    from oracle import bf16_value
    km = torch.from_numpy(bf16_value(summ["key_mean"])).double()
    el = torch.from_numpy(bf16_value(summ["ellipsoid"])).double()
    scale = D ** -0.5
    s = torch.einsum("hgd,hbd->hgb", qt, km) * scale
    delta = torch.einsum("hgd,hbd->hgb", q2, el).clamp_min(0).sqrt() * scale * (1 + 2 ** -8)
    z = s + torch.from_numpy(summ["counts"]).double().log()
    log_z = torch.logsumexp(z, -1, keepdim=True)
    log_c = torch.logsumexp(z + torch.log(torch.cosh(delta)), -1, keepdim=True)
    vmax = torch.from_numpy(summ["max_value_norm"]).double()[:, None, None]
    vn = torch.from_numpy(summ["value_norm"]).double()[:, None]
    risk = 2 * vmax * (z - log_c).exp() * (torch.cosh(delta) - 1) \
        + 2 * vn * (z - log_z).exp() * torch.tanh(delta / 2)
    return z, delta, risk, log_z[..., 0], log_c[..., 0]


@pytest.mark.parametrize("scale", [0.02, 0.1, 0.3])
def test_direct_branch_against_fp64_closed_form(oracle_lib, scale):
    q, k, v = testing.small_inputs(length=67, dim=64, dtype=torch.float32)
    q = q * scale  # small queries keep delta <= 10 (the direct branch)
    s = oracle_lib.summary(k.numpy(), v.numpy(), 16)
    qn = q[:, :, 0].numpy()
    st = oracle_lib.select_stats(qn, s)
    z, delta, risk, lz, lc = _stats64(qn, s, 64)
    assert (delta <= 10).all()
    np.testing.assert_allclose(st["delta"], delta.numpy(), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(st["log_z"], lz.numpy(), rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(st["log_c"], lc.numpy(), rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(st["risk"], risk.numpy(), rtol=3e-5, atol=1e-12)


def test_zero_query_has_zero_risk_and_selects_nothing(oracle_lib):
    """tests/test_transformers.py:121-141: a zero query has risk exactly 0."""
    _, k, v = testing.small_inputs(length=100, dim=64, dtype=torch.float32)
    s = oracle_lib.summary(k.numpy(), v.numpy(), 32)
    q = np.zeros((2, 4, 64), np.float32)
    mask, z, risk = oracle_lib.select(q, s, 0.0, "any")
    assert (risk == 0).all() and not mask.any()


def test_eps_zero_selects_all_and_huge_eps_none(oracle_lib):
    """tests/test_attention.py:74-103: eps=0 expands every block, eps=1e6 none."""
    q, k, v = testing.small_inputs(length=71, dim=64, dtype=torch.float32)
    s = oracle_lib.summary(k.numpy(), v.numpy(), 32)
    qn = q[:, :, 0].numpy()
    assert oracle_lib.select(qn, s, 0.0, "any")[0].all()
    assert not oracle_lib.select(qn, s, 1e6, "mean")[0].any()


def test_representative_multiplicity(oracle_lib):
    """tests/test_attention.py:93-103: values 1 (16 tokens) and 3 (3 tokens),
    nothing expanded -> output (16*1 + 3*3) / 19."""
    keys = np.zeros((1, 19, 64), np.float32)
    values = np.zeros_like(keys)
    values[:, :16] = 1
    values[:, 16:] = 3
    s = oracle_lib.summary(keys, values, 16)
    q = np.zeros((1, 2, 64), np.float32)
    empty = np.zeros((1, 0, 64), np.uint16)
    pages = oracle_lib.bf16_bits(np.concatenate([keys, np.zeros((1, 13, 64), np.float32)], 1))
    vpages = oracle_lib.bf16_bits(np.concatenate([values, np.zeros((1, 13, 64), np.float32)], 1))
    out, mask = oracle_lib.sparse_attention(q, s, pages, vpages, empty, empty, 1e6, "any")
    assert not mask.any()
    np.testing.assert_allclose(out, (16 + 9) / 19, rtol=1e-6)


def test_brute_force_mixed_attention(oracle_lib):
    """Tiny case: the mixed softmax equals the definition written out in fp64."""
    q, k, v = testing.small_inputs(length=40, dim=32, dtype=torch.float32, heads=1, group=2)
    s = oracle_lib.summary(k.numpy(), v.numpy(), 16)
    qn = q[:, :, 0].numpy()
    kb = torch.cat([k, k.new_zeros(1, 8, 32)], 1)
    vb = torch.cat([v, v.new_zeros(1, 8, 32)], 1)
    sk, sv = k[:, :3], v[:, :3]
    bits = lambda t: t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    out, mask = oracle_lib.sparse_attention(qn, s, bits(kb), bits(vb), bits(sk), bits(sv), 0.05,
                                            "any")
    mask_, z, risk = oracle_lib.select(qn, s, 0.05, "any")
    assert np.array_equal(mask, mask_)
    from oracle import bf16_value
    qt = q[:, :, 0].to(torch.bfloat16).double()[0]
    vm = torch.from_numpy(bf16_value(s["value_mean"])).double()[0]
    counts = s["counts"]
    for g in range(2):
        logits, vals = [], []
        for b in range(3):
            if not mask[0, b]:
                logits.append(float(z[0, g, b]))
                vals.append(vm[b])
        for b in range(3):
            if mask[0, b]:
                for t in range(counts[b]):
                    kt = k[0, b * 16 + t].to(torch.bfloat16).double()
                    logits.append(float(qt[g] @ kt) / np.sqrt(32))
                    vals.append(v[0, b * 16 + t].to(torch.bfloat16).double())
        for t in range(3):
            logits.append(float(qt[g] @ sk[0, t].to(torch.bfloat16).double()) / np.sqrt(32))
            vals.append(sv[0, t].to(torch.bfloat16).double())
        p = torch.softmax(torch.tensor(logits, dtype=torch.float64), 0)
        want = (p[:, None] * torch.stack(vals)).sum(0)
        np.testing.assert_allclose(out[0, g], want.numpy(), rtol=1e-5, atol=1e-6)
