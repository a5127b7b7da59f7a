"""HIP kernels vs the CPU oracle and the reference's golden vectors (GPU).

Bar: bit-exact summaries, selection dot products (z, delta) and
masks/counters against the oracle, which shares the kernels' fixed fp32
evaluation orders; log Z, log C and the risks, whose e^x and log x the
kernels take from the hardware's transcendental unit, within the error
those propagate (a few ulp, more where cosh(delta) - 1 and tanh(delta / 2)
cancel); attention outputs within the north-star tolerance (max-abs 2e-2,
mean-rel 1e-3) of the oracle's softmax, which is exact to fp64 over the same
bf16 inputs.
"""

import numpy as np
import pytest
import torch

import golden_cases as gc
from refinekv import (RefineKVConfig, build_summary, select_blocks, select_blocks_union,
                      sparse_attention, testing)

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
MAX_ABS, MEAN_REL = 2e-2, 1e-3


@pytest.fixture(scope="module")
def hip():
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    from refinekv import _hip

    _hip.lib()  # the HIP library must load: no fallback
    return _hip


@pytest.fixture(params=["step", "split"])
def decode_path(hip, request):
    """rkv_decode's two paths: the one-launch step (where the shape allows
    it) and the three kernels."""
    hip.set_decode_path(request.param)
    yield request.param
    hip.set_decode_path("step")


def assert_control_clean(hip, ws):
    """After every launch every workgroup's own launch counter holds the same
    launch count, no hand-off wait gave up (status word clear) and no head's
    poison word carries the last launch's tag (launch e tags its slots e + 1,
    so the last of n launches tags n).  Returns the launch count."""
    heads, group, dim, n = ws["hip_scratch_shape"]
    layout = hip.workspace_layout(heads, group, dim, n)
    tiles, ts = layout["step_workers"], layout["tile_stride"]
    words = ws["hip_scratch"][:layout["zf"]].view(torch.int64).cpu().numpy()
    lines = words[:(heads + 1) * 8].reshape(heads + 1, 8)
    assert lines[heads, 0] & 0xFFFFFFFF == 0, "a hand-off wait gave up"
    assert hip.workspace_status(ws) == 0
    launches = words[(heads + 1) * 8:(heads + 1) * 8 + heads * ts].reshape(heads, ts)[:, :tiles]
    assert np.all(launches == launches[0, 0]), launches
    assert launches[0, 0] == 0 or np.all(lines[:heads, 3] != launches[0, 0]), lines[:heads, 3]
    # start-order tickets: none, or one per workgroup of every launch
    assert lines[heads, 1] in (0, launches[0, 0] * tiles * heads), lines[heads, 1]
    return int(launches[0, 0])


def one_launch(hip, heads, group, dim, n_blocks, block):
    """Whether rkv_decode (default path) runs this shape as one launch, as the
    library itself decides on this device."""
    return hip.decode_plan(heads, group, dim, n_blocks, block) != "split"


def bits16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def bits32(t):
    a = t.detach().cpu().contiguous().numpy() if torch.is_tensor(t) else np.asarray(t)
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def oracle_summary_of(summary):
    return dict(counts=summary.counts.cpu().numpy(), key_mean=bits16(summary.key_mean),
                value_mean=bits16(summary.value_mean), ellipsoid=bits16(summary.ellipsoid),
                value_norm=summary.value_norm.cpu().numpy(),
                max_value_norm=summary.max_value_norm.cpu().numpy(),
                prompt_length=summary.prompt_length, block_size=summary.block_size)


def assert_summary_equal(summary, ref):
    assert np.array_equal(summary.counts.cpu().numpy(), ref["counts"])
    for name in ("key_mean", "value_mean", "ellipsoid"):
        got = bits16(getattr(summary, name))
        bad = int((got != ref[name]).sum())
        assert bad == 0, f"{name}: {bad} of {got.size} bf16 values differ"
    for name in ("value_norm", "max_value_norm"):
        got, want = bits32(getattr(summary, name)), bits32(ref[name])
        assert np.array_equal(got, want), f"{name}: {int((got != want).sum())} differ"


def assert_close_output(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    assert err.max() <= MAX_ABS, f"max-abs {err.max():.3e}"
    assert err.mean() <= MEAN_REL * np.abs(want).mean() + 1e-6, f"mean-abs {err.mean():.3e}"


# ---------------------------------------------------------------------------
# Device scalar math
# ---------------------------------------------------------------------------

def test_device_math_bitwise_equals_oracle(hip, oracle_lib):
    rng = np.random.default_rng(0)
    specials = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1.0, 88.72283, 88.7229, -103.97,
                         -104.5, 1e-40, 1e-45, 3.4e38, 88.8, 88.80001, 89.0, -104.0, -104.00001,
                         -1.0, -3.5, -1e-40, 1.17549435e-38, 1.1754942e-38, 1.41421356,
                         1.4142137, 0.70710677, -np.nan], np.float32)
    xe = np.concatenate([rng.uniform(-110, 90, 400000), rng.uniform(-1, 1, 200000),
                         specials]).astype(np.float32)
    xl = np.concatenate([np.exp(rng.uniform(-103, 88, 400000)), rng.uniform(0.5, 2, 200000),
                         np.arange(1, 129), specials]).astype(np.float32)
    for fn, x, want in (("exp", xe, oracle_lib.expf(xe)), ("log", xl, oracle_lib.logf(xl)),
                        ("bf16", xe, oracle_lib.bf16_value(oracle_lib.bf16_bits(xe))),
                        ("sqrt", np.abs(xl), np.sqrt(np.abs(xl)))):
        got = hip.math_probe(fn, torch.from_numpy(x).to(DEV)).cpu().numpy()
        g, w = got.view(np.uint32), np.asarray(want, np.float32).view(np.uint32)
        both_nan = np.isnan(got) & np.isnan(want)
        bad = (g != w) & ~both_nan
        assert not bad.any(), f"{fn}: {int(bad.sum())} differ, e.g. x={x[bad][:4]}"


def test_device_hardware_exp_log_error(hip):
    """exp_hw / log_hw (the selection kernels' e^x and log x) against fp64:
    e^x within 2^-23 (1 + |x|) relative where the result is normal (the
    hardware's ulp plus the rounding of x log2(e)), at most 2^-126 off below;
    log x within 2^-22 (1 + |log x|) absolute; special values exact."""
    rng = np.random.default_rng(1)
    xe = np.concatenate([rng.uniform(-110, 88.7, 400000), rng.uniform(-1, 1, 200000),
                         rng.uniform(-30, 0, 200000)]).astype(np.float32)
    got = hip.math_probe("exp_hw", torch.from_numpy(xe).to(DEV)).cpu().numpy().astype(np.float64)
    x64 = xe.astype(np.float64)
    want = np.exp(x64)
    normal = want >= 2.0 ** -126
    rel = np.abs(got[normal] - want[normal]) / want[normal]
    bound = 2.0 ** -23 * (1.0 + np.abs(x64[normal]))
    assert np.all(rel <= bound), f"exp_hw: worst {float(np.max(rel / bound)):.2f} x bound"
    assert np.all(np.abs(got[~normal] - want[~normal]) <= 2.0 ** -126)
    xl = np.concatenate([np.exp(rng.uniform(-87, 88, 400000)), rng.uniform(0.5, 2, 200000),
                         1.0 + rng.uniform(-1e-3, 1e-3, 100000)]).astype(np.float32)
    got = hip.math_probe("log_hw", torch.from_numpy(xl).to(DEV)).cpu().numpy().astype(np.float64)
    want = np.log(xl.astype(np.float64))
    err, bound = np.abs(got - want), 2.0 ** -22 * (1.0 + np.abs(want))
    assert np.all(err <= bound), f"log_hw: worst {float(np.max(err / bound)):.2f} x bound"
    sp = np.array([-np.inf, np.inf, np.nan, 0.0, -1.0], np.float32)
    e = hip.math_probe("exp_hw", torch.from_numpy(sp).to(DEV)).cpu().numpy()
    assert e[0] == 0.0 and e[1] == np.inf and np.isnan(e[2]) and e[3] == 1.0
    lg = hip.math_probe("log_hw", torch.from_numpy(sp).to(DEV)).cpu().numpy()
    assert np.isnan(lg[0]) and lg[1] == np.inf and np.isnan(lg[2]) and lg[3] == -np.inf
    assert np.isnan(lg[4])


# ---------------------------------------------------------------------------
# Summary
# ---------------------------------------------------------------------------

SUMMARY_CASES = [
    (torch.bfloat16, 128, 32, 4099), (torch.bfloat16, 128, 16, 1000), (torch.bfloat16, 128, 64, 4096),
    (torch.bfloat16, 32, 32, 517), (torch.bfloat16, 64, 16, 300), (torch.bfloat16, 96, 64, 1000),
    (torch.bfloat16, 160, 32, 333), (torch.bfloat16, 192, 16, 250), (torch.bfloat16, 224, 64, 130),
    (torch.bfloat16, 256, 32, 999), (torch.float16, 128, 32, 777), (torch.float16, 64, 64, 200),
    (torch.float32, 128, 32, 999), (torch.float32, 32, 16, 517), (torch.float32, 96, 64, 1000),
    (torch.float32, 256, 16, 400), (torch.bfloat16, 128, 32, 1), (torch.bfloat16, 64, 64, 63),
    # the streaming form (2-byte, staged, head_dim >= 192)
    (torch.bfloat16, 256, 16, 777), (torch.float16, 224, 16, 500),
    # the largest blocks (64 KiB and 128 KiB of K plus V)
    (torch.float32, 256, 64, 300), (torch.float32, 128, 64, 700),
    # blocks split over a workgroup's waves (16 tokens each), last block partial
    (torch.bfloat16, 128, 64, 1000), (torch.float16, 128, 64, 1999), (torch.bfloat16, 192, 32, 1001),
]


@pytest.mark.parametrize("dtype,dim,block,length", SUMMARY_CASES,
                         ids=lambda v: str(v).replace("torch.", ""))
def test_summary_bit_exact(hip, oracle_lib, dtype, dim, block, length):
    if dtype == torch.float32:
        _, k, v = testing.wide_inputs(length=length, dim=dim, heads=3)
    else:
        _, k, v = testing.small_inputs(length=length, dim=dim, heads=3, dtype=torch.float32)
        k, v = k * 3, v * 3
    k, v = k.to(dtype), v.to(dtype)
    ref = oracle_lib.summary(k.float().numpy(), v.float().numpy(), block)
    cfg = RefineKVConfig(backend="hip", block_size=block)
    summary = build_summary(k.to(DEV), v.to(DEV), cfg)
    torch.cuda.synchronize()
    assert_summary_equal(summary, ref)


def test_random_summaries_bit_exact(hip, oracle_lib):
    """30 seeded random (dtype, head_dim, block, length) summaries bit for bit
    against the oracle: every kernel form (split blocks, one wave per block,
    the stream for head_dim >= 192, the two-pass form) and partial last
    blocks."""
    rng = np.random.default_rng(77)
    for _ in range(30):
        dtype = [torch.bfloat16, torch.float16, torch.float32][int(rng.integers(0, 3))]
        dim = int(rng.choice([32, 64, 96, 128, 160, 192, 224, 256]))
        block = int(rng.choice([16, 32, 64]))
        length = int(rng.choice([rng.integers(1, 64), rng.integers(64, 5000)]))
        heads = int(rng.integers(1, 5))
        g = torch.Generator().manual_seed(int(rng.integers(0, 1 << 30)))
        k = (torch.randn(heads, length, dim, generator=g) * 2).to(dtype)
        v = torch.randn(heads, length, dim, generator=g).to(dtype)
        ref = oracle_lib.summary(k.float().numpy(), v.float().numpy(), block)
        summary = build_summary(k.to(DEV), v.to(DEV), RefineKVConfig(backend="hip", block_size=block))
        torch.cuda.synchronize()
        try:
            assert_summary_equal(summary, ref)
        except AssertionError as err:
            raise AssertionError(f"{dtype} d{dim} B{block} L{length} H{heads}: {err}") from None


def test_summary_of_strided_cache_view(hip, oracle_lib):
    """A prefix view of a larger (1, H, capacity, D) cache, as the hook passes it."""
    _, k, v = testing.small_inputs(length=3000, dim=128, heads=4)
    cache_k = torch.zeros(1, 4, 3100, 128, dtype=torch.bfloat16)
    cache_v = torch.zeros_like(cache_k)
    cache_k[0, :, :3000], cache_v[0, :, :3000] = k, v
    ref = oracle_lib.summary(k.float().numpy(), v.float().numpy(), 32)
    ck, cv = cache_k.to(DEV), cache_v.to(DEV)
    summary = build_summary(ck[0, :, :2990], cv[0, :, :2990], RefineKVConfig(backend="hip"))
    ref = oracle_lib.summary(k[:, :2990].float().numpy(), v[:, :2990].float().numpy(), 32)
    torch.cuda.synchronize()
    assert_summary_equal(summary, ref)
    # 2990 % 32 != 0: the pages are a padded copy; 2976 tokens: a view of the cache.
    s2 = build_summary(ck[0, :, :2976], cv[0, :, :2976], RefineKVConfig(backend="hip"))
    assert s2.keys.data_ptr() == ck.data_ptr()


def test_summary_of_rows_not_16_byte_aligned(hip, oracle_lib):
    """Rows 4-byte but not 16-byte aligned (a column slice of a wider buffer,
    token stride not a multiple of the row size)."""
    gen = torch.Generator(device=DEV).manual_seed(5)
    wide_k = torch.randn(3, 777, 98, generator=gen, device=DEV).to(torch.bfloat16)
    wide_v = torch.randn(3, 777, 98, generator=gen, device=DEV).to(torch.bfloat16)
    k, v = wide_k[:, :, 2:], wide_v[:, :, 2:]
    summary = build_summary(k, v, RefineKVConfig(backend="hip", block_size=32))
    ref = oracle_lib.summary(k.float().cpu().numpy(), v.float().cpu().numpy(), 32)
    torch.cuda.synchronize()
    assert_summary_equal(summary, ref)


@pytest.mark.parametrize("dtype,dim,block,length", [
    (torch.bfloat16, 128, 32, 4099), (torch.bfloat16, 64, 16, 300), (torch.float16, 128, 32, 777),
    (torch.float32, 96, 64, 1000), (torch.bfloat16, 256, 32, 999), (torch.float32, 256, 64, 300),
    (torch.bfloat16, 128, 64, 1000)])
def test_summary_written_with_the_cache(hip, oracle_lib, dtype, dim, block, length):
    """store_and_build_summary (one kernel: cache write + summary) equals the
    oracle's summary of the same keys/values bit for bit, and a cache copy
    followed by build_summary, and fills the cache."""
    from refinekv.summary import store_and_build_summary

    gen = torch.Generator(device=DEV).manual_seed(dim + length)
    # (H, L, D) sources with the projection's layout: token stride H * D
    keys = torch.randn(length, 3, dim, generator=gen, device=DEV).to(dtype).transpose(0, 1)
    values = torch.randn(length, 3, dim, generator=gen, device=DEV).to(dtype).transpose(0, 1)
    cache_k = torch.full((1, 3, length + 40, dim), float("nan"), device=DEV, dtype=dtype)
    cache_v = torch.full_like(cache_k, float("nan"))
    cfg = RefineKVConfig(backend="hip", block_size=block)
    fused = store_and_build_summary(keys, values, cache_k[0, :, :length], cache_v[0, :, :length],
                                    cfg)
    torch.cuda.synchronize()
    assert torch.equal(cache_k[0, :, :length], keys) and torch.equal(cache_v[0, :, :length], values)
    assert torch.isnan(cache_k[0, :, length:].float()).all()  # nothing written past the prompt
    assert_summary_equal(fused, oracle_lib.summary(keys.float().cpu().numpy(),
                                                   values.float().cpu().numpy(), block))
    ref = build_summary(keys.contiguous(), values.contiguous(), cfg)
    for name in ("counts", "key_mean", "value_mean", "ellipsoid", "value_norm", "max_value_norm"):
        a, b = getattr(fused, name), getattr(ref, name)
        assert torch.equal(a.view(torch.uint8) if a.is_floating_point() else a,
                           b.view(torch.uint8) if b.is_floating_point() else b), name
    assert torch.equal(fused.keys, ref.keys) and torch.equal(fused.values, ref.values)


# ---------------------------------------------------------------------------
# Selection statistics and masks
# ---------------------------------------------------------------------------

SELECT_CASES = [
    # heads, group, dim, block, prompt, reduction, eps, spikes
    (8, 4, 128, 32, 4096, "any", 0.01, 0.02),
    (4, 7, 128, 64, 3000, "max", 0.005, 0.05),
    (2, 16, 64, 16, 1000, "mean", 0.1, 0.05),
    (2, 1, 32, 32, 100, "any", 0.01, 0.1),
    (3, 5, 96, 16, 777, "mean", 0.02, 0.05),
    (2, 4, 256, 64, 999, "max", 0.01, 0.05),
    (2, 2, 160, 32, 2050, "any", 0.001, 0.01),
    (1, 4, 128, 32, 20000, "any", 0.01, 0.01),
    # 69 tiles: the rows' log Z / log C merged once (lse_merge_kernel) before
    # the decisions
    (1, 4, 128, 16, 70000, "any", 0.01, 0.01),
]


def _decode_case(heads, group, dim, block, prompt, spikes, suffix=16, seed=11):
    inp = testing.decode_inputs(heads=heads, group=group, dim=dim, prompt=prompt, suffix=suffix,
                                block=block, spike_fraction=spikes, anchors=4, seed=seed)
    return {k: (v.to(torch.bfloat16) if v.is_floating_point() else v) for k, v in inp.items()}


# Error of the kernels' e^x and log x (v_exp_f32 / v_log_f32 scaled by
# fp32 log2(e) and ln 2) against the oracle's, in units of 2^-24: about an
# ulp each plus |x| 2^-24 from rounding x log2(e).
HW_ULPS = 8


def ulp_distance(a, b):
    """|a - b| in units in the last place of fp32 (same-sign values)."""
    ia, ib = bits32(a).astype(np.int64), bits32(b).astype(np.int64)
    return np.abs(ia - ib)


def risk_tolerance(z, delta, log_z, log_c, risk):
    """Per-element bound on |risk_hip - risk_oracle| from the kernels' e^x
    and log x: risk = 2 vmax e^(z - log C) A + 2 |v| e^(z - log Z) th with
    A = cosh(delta) - 1 and th = tanh(delta / 2) from t = e^delta.  A
    relative error u in t gives coth(delta / 2) u in A and u / sinh(delta) in
    th; e^(z - log C) carries (|z - log C| + |log C|) u.  Summing every
    term's relative error bounds both parts of the risk."""
    u = HW_ULPS * 2.0 ** -24
    d = np.maximum(delta.astype(np.float64), 1e-30)
    small = d <= 10.0
    amp = np.where(small, 1.0 / np.tanh(d / 2) + 1.0 / np.sinh(np.minimum(d, 10.0)), 2.0)
    lz, lc = log_z[..., None].astype(np.float64), log_c[..., None].astype(np.float64)
    zz = z.astype(np.float64)
    rel = u * (4.0 + amp + np.abs(zz - lc) + np.abs(zz - lz) + np.abs(lc) + np.abs(lz))
    return rel * np.abs(risk.astype(np.float64)) + 1e-37


@pytest.mark.parametrize("reduction", ["any", "max", "mean"])
def test_masks_with_eps_next_to_a_risk(hip, oracle_lib, reduction):
    """eps placed at sampled blocks' reduced risks: ten times the hardware
    e^x / log x error bound above and below, every mask equals the oracle's;
    at the risk itself, a mask may differ from the oracle's only for a
    block whose reduced risk lies within that bound of eps."""
    heads, group, dim, block = 2, 4, 128, 32
    inp = _decode_case(heads, group, dim, block, 4096, 0.05)
    cfg0 = RefineKVConfig(backend="hip", block_size=block, eps=0.01, gqa_reduction=reduction)
    summary = build_summary(inp["prompt_keys"].to(DEV), inp["prompt_values"].to(DEV), cfg0)
    qn = inp["query"][:, :, 0].float().numpy()
    summ = oracle_summary_of(summary)
    st = oracle_lib.select_stats(qn, summ)
    tol = risk_tolerance(st["z"], st["delta"], st["log_z"], st["log_c"], st["risk"])
    risk = st["risk"].astype(np.float64)
    # the reduced risk of each (head, block) and its bound
    if reduction == "mean":
        red, bound = risk.mean(axis=1), tol.mean(axis=1)
    else:
        red, bound = risk.max(axis=1), tol.max(axis=1)
    rng = np.random.default_rng(5)
    picks = [tuple(x) for x in rng.choice(np.argwhere(np.isfinite(red) & (red > 1e-30)), 6)]
    for h, b in picks:
        r, tb = float(red[h, b]), float(bound[h, b])
        for eps, exact in ((r + 10 * tb, True), (r - 10 * tb, True), (r, False)):
            if eps <= 0.0:
                continue
            cfg = RefineKVConfig(backend="hip", block_size=block, eps=float(np.float32(eps)),
                                 gqa_reduction=reduction)
            got = hip.select(inp["query"].to(DEV), summary, cfg, {}).cpu().numpy().astype(np.uint8)
            want, _, _ = oracle_lib.select(qn, summ, cfg.eps, reduction)
            diff = got != want
            if exact:
                assert not diff.any(), (h, b, eps, int(diff.sum()))
            else:
                near = np.abs(red - cfg.eps) <= bound
                assert not (diff & ~near).any(), (h, b, eps, int((diff & ~near).sum()))


@pytest.mark.parametrize("heads,group,dim,block,prompt,reduction,eps,spikes", SELECT_CASES)
def test_selection_statistics(hip, oracle_lib, heads, group, dim, block, prompt, reduction, eps,
                              spikes):
    """z and delta bit for bit; log Z, log C within a few ulp and the risks
    within the error the kernels' hardware e^x and log x propagate; masks
    equal the oracle's."""
    inp = _decode_case(heads, group, dim, block, prompt, spikes)
    cfg = RefineKVConfig(backend="hip", block_size=block, eps=eps, gqa_reduction=reduction)
    summary = build_summary(inp["prompt_keys"].to(DEV), inp["prompt_values"].to(DEV), cfg)
    n = summary.num_blocks
    risk = torch.empty(heads, group, n, device=DEV)
    stats = torch.empty(heads, group, 2, device=DEV)
    ws = {}
    mask = hip.select(inp["query"].to(DEV), summary, cfg, ws, risk_out=risk, stats_out=stats)
    torch.cuda.synchronize()
    summ = oracle_summary_of(summary)
    qn = inp["query"][:, :, 0].float().numpy()
    st = oracle_lib.select_stats(qn, summ)
    layout = hip.workspace_layout(heads, group, dim, n)
    scratch = ws["hip_scratch"].cpu().numpy()
    rows, stride = heads * group, layout["z_stride"]  # blocks padded to whole tiles
    zf = scratch[layout["zf"]:layout["zf"] + rows * stride * 16].view(np.float32)
    zf = zf.reshape(rows, stride, 4)[:, :n]
    z, delta = np.ascontiguousarray(zf[..., 0]), np.ascontiguousarray(zf[..., 1])
    assert np.array_equal(bits32(z), bits32(st["z"].reshape(rows, n))), "z"
    assert np.array_equal(bits32(delta), bits32(st["delta"].reshape(rows, n))), "delta"
    sc = stats.cpu().numpy()
    assert ulp_distance(sc[..., 0], st["log_z"]).max() <= HW_ULPS, "log Z"
    assert ulp_distance(sc[..., 1], st["log_c"]).max() <= HW_ULPS, "log C"
    got_risk = risk.cpu().numpy()
    tol = risk_tolerance(st["z"], st["delta"], st["log_z"], st["log_c"], st["risk"])
    err = np.abs(got_risk.astype(np.float64) - st["risk"].astype(np.float64))
    assert np.all(np.isfinite(got_risk) == np.isfinite(st["risk"])), "risk finiteness"
    fin = np.isfinite(st["risk"])
    assert np.all(err[fin] <= tol[fin]), f"risk: worst {float(np.max(err[fin] / tol[fin])):.2f} x bound"
    want, _, _ = oracle_lib.select(qn, summ, eps, reduction)
    assert np.array_equal(mask.cpu().numpy().astype(np.uint8), want)
    # the public API returns the same mask
    api = select_blocks(inp["query"].to(DEV), summary, cfg, workspace={})
    assert torch.equal(api.cpu(), mask.cpu())


@pytest.mark.parametrize("heads,group,dim,block,prompt,reduction,eps,spikes", SELECT_CASES)
def test_anchor_union_matches_per_query_selection(hip, oracle_lib, heads, group, dim, block,
                                                  prompt, reduction, eps, spikes):
    """The batched anchor selection (one scoring launch over all queries)
    equals the OR of the oracle's per-query masks and of per-query HIP
    selections, for every reduction."""
    inp = _decode_case(heads, group, dim, block, prompt, spikes)
    cfg = RefineKVConfig(backend="hip", block_size=block, eps=eps, gqa_reduction=reduction)
    summary = build_summary(inp["prompt_keys"].to(DEV), inp["prompt_values"].to(DEV), cfg)
    count = 5
    gen = torch.Generator().manual_seed(7)
    # perturbed copies of the spike-aligned decode query
    queries = inp["query"].float() + 0.3 * torch.randn(heads, group, count, dim, generator=gen)
    queries[:, :, 0] = inp["query"][:, :, 0].float()
    queries = queries.to(torch.bfloat16)
    ws = {}
    got = select_blocks_union(queries.to(DEV), summary, cfg, workspace=ws).cpu().numpy()
    summ = oracle_summary_of(summary)
    want = np.zeros((heads, summary.num_blocks), np.uint8)
    hip_union = torch.zeros(heads, summary.num_blocks, dtype=torch.bool)
    for a in range(count):
        qa = queries[:, :, a]
        mask, _, _ = oracle_lib.select(qa.float().numpy(), summ, eps, reduction)
        want |= mask
        hip_union |= select_blocks(qa[:, :, None].to(DEV), summary, cfg, workspace={}).cpu()
    assert np.array_equal(got.astype(np.uint8), want)
    assert np.array_equal(got, hip_union.numpy())
    # a second call with the same workspace (its scratch reused) agrees
    again = select_blocks_union(queries.to(DEV), summary, cfg, workspace=ws).cpu().numpy()
    assert np.array_equal(again, got)


# ---------------------------------------------------------------------------
# Decode step
# ---------------------------------------------------------------------------

# (2, 4, 256, 64, 999, "max", ...) faulted the GPU with a since-removed
# persistent kernel (head_dim-256 build, 556 B/lane of register spills).
# head_dim above 160 now runs only the three kernels (score, attend, merge:
# no spills, LDS and index ranges checked on the CPU for this exact shape in
# tests/test_kernel_resources_cpu.py), and the case runs again.
DECODE_CASES = [
    c for c in SELECT_CASES + [
        (8, 4, 128, 32, 4096, "any", 0.0, 0.02),   # every block expanded (dense)
        (8, 4, 128, 32, 4096, "mean", 1e6, 0.02),  # none expanded
        (2, 2, 256, 32, 1500, "any", 0.01, 0.05),
        (2, 4, 224, 16, 700, "max", 0.01, 0.05),
        # few (row, column) units per merge slice: 1-2 query rows, short rows
        (2, 1, 64, 16, 9000, "any", 0.01, 0.05),
        (1, 2, 32, 16, 8200, "max", 0.01, 0.05),
        # more than 64 tiles per head (several tiles per lane in the step's
        # hand-offs), and more than the step takes (the three kernels run)
        (1, 4, 128, 16, 140000, "max", 0.01, 0.02),
        (1, 2, 64, 16, 310000, "any", 0.01, 0.01),
        # 176 tiles per head over 170 workgroups per head: the step's first
        # 6 workgroups score 2 tiles each, the rest one (the last one short)
        (3, 4, 128, 16, 180000, "any", 0.01, 0.02),
        # several tiles per workgroup, a 2-query group: 88 tiles per head
        # over 32 workgroups (3, 3, ..., 2 tiles each)
        (16, 2, 64, 16, 90000, "mean", 0.01, 0.02),
        # the same with every block expanded: a workgroup's share of the
        # head's expanded rows spans up to 178 blocks (64 ceil(T / W) + 2)
        (16, 2, 64, 16, 90000, "any", 0.0, 0.02),
    ]
]


def _pages_bits(t, block):
    return gc.bf16_bits(gc.padded_pages(t, block))


@pytest.mark.parametrize("heads,group,dim,block,prompt,reduction,eps,spikes", DECODE_CASES)
def test_decode_matches_oracle(hip, oracle_lib, decode_path, heads, group, dim, block, prompt,
                               reduction, eps, spikes):
    inp = _decode_case(heads, group, dim, block, prompt, spikes, suffix=16)
    cfg = RefineKVConfig(backend="hip", block_size=block, eps=eps, gqa_reduction=reduction)
    k, v = inp["prompt_keys"], inp["prompt_values"]
    summary = build_summary(k.to(DEV), v.to(DEV), cfg)
    summ = oracle_summary_of(summary)
    n = summary.num_blocks
    anchor = torch.zeros(heads, n, dtype=torch.bool)
    anchor[:, -1] = True
    anchor[0, 0] = True
    ws = {}
    qn = inp["query"][:, :, 0].float().numpy()
    kp, vp = _pages_bits(k, block), _pages_bits(v, block)
    for suffix in (0, 5, 16):
        for use_anchor in (False, True):
            a = anchor if use_anchor else None
            res = sparse_attention(inp["query"].to(DEV), summary,
                                   inp["suffix_keys"][:, :suffix].to(DEV),
                                   inp["suffix_values"][:, :suffix].to(DEV), cfg,
                                   anchor_mask=a.to(DEV) if a is not None else None,
                                   workspace=ws, return_selected=True)
            torch.cuda.synchronize()
            out, mask = oracle_lib.sparse_attention(
                qn, summ, kp, vp, gc.bf16_bits(inp["suffix_keys"][:, :suffix]),
                gc.bf16_bits(inp["suffix_values"][:, :suffix]), eps, reduction,
                None if a is None else a.numpy())
            assert np.array_equal(res.selected.cpu().numpy().astype(np.uint8), mask), \
                f"mask suffix={suffix} anchor={use_anchor}"
            got = res.output.float().cpu().numpy()[:, :, 0]
            assert_close_output(got, torch.from_numpy(out).to(torch.bfloat16).float().numpy())
    launches = assert_control_clean(hip, ws)
    assert launches == (6 if decode_path == "step" and one_launch(hip, heads, group, dim, n, block)
                        else 0)


def _random_decode_cases(n, seed):
    """Seeded random decode shapes across what the kernels take: head_dim
    32..256, groups 1..16, blocks 16/32/64, prompts from a few tokens to a
    few thousand, eps from 0 to 1e6, every reduction, suffixes 0..39 and
    optional anchors."""
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(n):
        cases.append(dict(
            dim=int(rng.choice([32, 64, 96, 128, 160, 256])),
            group=int(rng.choice([1, 2, 3, 4, 5, 7, 8, 12, 16])),
            heads=int(rng.integers(1, 9)),
            block=int(rng.choice([16, 32, 64])),
            prompt=int(rng.choice([rng.integers(1, 200), rng.integers(200, 3000),
                                   rng.integers(3000, 9000)])),
            eps=float(rng.choice([0.0, 1e-3, 1e-2, 0.05, 0.3, 1e6])),
            reduction=str(rng.choice(["mean", "max", "any"])),
            spikes=float(rng.choice([0.0, 0.02, 0.2])),
            suffix=int(rng.integers(0, 40)),
            anchor=bool(rng.integers(0, 2)),
            seed=int(rng.integers(0, 1 << 30))))
    return cases


def test_random_shapes_match_oracle(hip, oracle_lib, decode_path):
    """48 seeded random shapes per path: masks equal to the oracle's, outputs
    within tolerance, hand-off control words clean (two calls per workspace,
    the second after a launch on it)."""
    for c in _random_decode_cases(48, 2024):
        name = str(c)
        inp = testing.decode_inputs(heads=c["heads"], group=c["group"], dim=c["dim"],
                                    prompt=c["prompt"], suffix=max(c["suffix"], 1),
                                    block=c["block"], spike_fraction=c["spikes"], anchors=4,
                                    seed=c["seed"])
        inp = {k: (v.to(torch.bfloat16) if v.is_floating_point() else v) for k, v in inp.items()}
        cfg = RefineKVConfig(backend="hip", block_size=c["block"], eps=c["eps"],
                             gqa_reduction=c["reduction"])
        k, v = inp["prompt_keys"], inp["prompt_values"]
        summary = build_summary(k.to(DEV), v.to(DEV), cfg)
        n = summary.num_blocks
        anchor = None
        if c["anchor"]:
            g = torch.Generator().manual_seed(c["seed"])
            anchor = torch.rand(c["heads"], n, generator=g) < 0.1
        sl = c["suffix"]
        ws = {}
        for _ in range(2):
            res = sparse_attention(inp["query"].to(DEV), summary, inp["suffix_keys"][:, :sl].to(DEV),
                                   inp["suffix_values"][:, :sl].to(DEV), cfg,
                                   anchor_mask=anchor.to(DEV) if anchor is not None else None,
                                   workspace=ws, return_selected=True)
        torch.cuda.synchronize()
        out, mask = oracle_lib.sparse_attention(
            inp["query"][:, :, 0].float().numpy(), oracle_summary_of(summary),
            _pages_bits(k, c["block"]), _pages_bits(v, c["block"]),
            gc.bf16_bits(inp["suffix_keys"][:, :sl]), gc.bf16_bits(inp["suffix_values"][:, :sl]),
            c["eps"], c["reduction"], None if anchor is None else anchor.numpy())
        assert np.array_equal(res.selected.cpu().numpy().astype(np.uint8), mask), name
        got = res.output.float().cpu().numpy()[:, :, 0]
        try:
            assert_close_output(got, torch.from_numpy(out).to(torch.bfloat16).float().numpy())
        except AssertionError as err:
            raise AssertionError(f"{name}: {err}") from None
        if ws:
            assert_control_clean(hip, ws)


def test_device_suffix_length_matches_slicing(hip, decode_path):
    """tests/test_attention.py:186-204 for the HIP backend: bit-equal outputs."""
    q, keys, values = testing.small_inputs(length=71, dim=128)
    cfg = RefineKVConfig(backend="hip", gqa_reduction="mean")
    summary = build_summary(keys.to(DEV), values.to(DEV), cfg)
    sk, sv = [t.to(DEV) for t in testing.small_inputs(length=16, dim=128, seed=5)[1:]]
    visible = torch.zeros((), device=DEV, dtype=torch.int32)
    for count in (0, 1, 5, 16):
        visible.fill_(count)
        actual = sparse_attention(q.to(DEV), summary, sk, sv, cfg, suffix_length=visible,
                                  workspace={}).output.clone()
        expected = sparse_attention(q.to(DEV), summary, sk[:, :count], sv[:, :count], cfg,
                                    workspace={}).output.clone()
        assert torch.equal(actual, expected), count


def test_workspace_reuse_and_access_counter(hip, oracle_lib, decode_path):
    inp = _decode_case(4, 4, 128, 32, 5000, 0.05)
    cfg = RefineKVConfig(backend="hip", eps=0.01)
    summary = build_summary(inp["prompt_keys"].to(DEV), inp["prompt_values"].to(DEV), cfg)
    ws = {}
    counter = torch.zeros(1, dtype=torch.int64, device=DEV)
    outs = []
    for _ in range(3):
        out, mask = hip.decode(inp["query"].to(DEV), summary, inp["suffix_keys"].to(DEV),
                               inp["suffix_values"].to(DEV), cfg, None, ws, None, counter)
        outs.append(out.clone())
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[1], outs[2])
    want = oracle_lib.access_blocks(mask.cpu().numpy(), summary.counts.cpu().numpy())
    assert int(counter.item()) == 3 * want
    assert assert_control_clean(hip, ws) == (3 if decode_path == "step" else 0)


def test_graph_replays_match_eager(hip, decode_path):
    """A captured decode step replayed several times (suffix length advanced
    on the device between replays, eager work and syncs in between) gives the
    eager result every time."""
    inp = _decode_case(8, 4, 128, 32, 8192, 0.05, suffix=16, seed=3)
    cfg = RefineKVConfig(backend="hip", eps=0.01)
    summary = build_summary(inp["prompt_keys"].to(DEV), inp["prompt_values"].to(DEV), cfg)
    q, sk, sv = (inp[k].to(DEV) for k in ("query", "suffix_keys", "suffix_values"))
    length = torch.zeros((), dtype=torch.int32, device=DEV)
    ws = {}
    sparse_attention(q, summary, sk, sv, cfg, workspace=ws, suffix_length=length)  # warm
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        res = sparse_attention(q, summary, sk, sv, cfg, workspace=ws, suffix_length=length)
    for count in (3, 9, 16, 16):
        length.fill_(count)
        graph.replay()
        torch.cuda.synchronize()
        got = res.output.clone()
        want = sparse_attention(q, summary, sk[:, :count], sv[:, :count], cfg,
                                workspace={}).output
        torch.cuda.synchronize()
        assert torch.equal(got, want), count
    assert_control_clean(hip, ws)


@pytest.mark.parametrize("heads,group,dim,block,prompt", [
    (8, 4, 128, 32, 8192), (4, 7, 128, 64, 8192), (2, 8, 64, 16, 3000),
    (8, 4, 128, 32, 65536)])
def test_speculation_matches_the_normal_order_bit_for_bit(hip, heads, group, dim, block,
                                                          prompt):
    """After a launch that expanded every block of its tile, a step workgroup
    issues its tile's first page rows before the decision: when every block
    expands again the ring goes on from them and the result is the normal
    order's bit for bit, and when not (a sparse eps on the same workspace)
    the speculation is dropped and the normal order runs.  (At 65536 tokens
    a wave has 16 chunks of page rows, most of them after the decision.)"""
    inp = _decode_case(heads, group, dim, block, prompt, 0.05, suffix=16, seed=5)
    full = RefineKVConfig(backend="hip", block_size=block, eps=0.0, gqa_reduction="any")
    summary = build_summary(inp["prompt_keys"].to(DEV), inp["prompt_values"].to(DEV), full)
    q, sk, sv = (inp[k].to(DEV) for k in ("query", "suffix_keys", "suffix_values"))
    assert hip.decode_plan(heads, group, dim, summary.num_blocks, block) == "step"

    def run(cfg, ws):
        res = sparse_attention(q, summary, sk, sv, cfg, workspace=ws, return_selected=True)
        return res.output.clone(), res.selected.clone()

    hip.set_speculation("off")
    try:
        want_full = run(full, {})
        # the smallest of these eps that leaves some block unexpanded
        for eps in (0.01, 0.05, 0.2, 1.0, 5.0):
            sparse = RefineKVConfig(backend="hip", block_size=block, eps=eps,
                                    gqa_reduction="any")
            want_sparse = run(sparse, {})
            if not want_sparse[1].all():
                break
        hip.set_speculation("always")
        assert want_full[1].all() and not want_sparse[1].all()
        ws = {}
        got = [run(full, ws) for _ in range(3)]  # the first in the normal order, then speculating
        got.append(run(sparse, ws))              # speculates and misses
        got.append(run(full, ws))                # the previous launch did not expand every block
        got.append(run(full, ws))                # speculates again
        torch.cuda.synchronize()
    finally:
        hip.set_speculation("auto")
    for i, (out, mask) in enumerate(got):
        want = want_sparse if i == 3 else want_full
        assert torch.equal(mask, want[1]), i
        assert torch.equal(out, want[0]), i
    assert assert_control_clean(hip, ws) == len(got)


@pytest.mark.parametrize("path", [p for p in gc.fixture_paths() if "f32" not in p],
                         ids=lambda p: p.split("/")[-1][:-4])
def test_reference_golden_end_to_end(hip, path):
    """bf16 golden cases: HIP summary bit-exact to the reference, selection
    (with anchors) equal, outputs within tolerance of the reference's."""
    g, meta = gc.load(path)
    inp = gc.regenerate(meta)
    cfg = RefineKVConfig(backend="hip", **meta["config"])
    summary = build_summary(inp["keys"].to(DEV), inp["values"].to(DEV), cfg)
    ref = {k: g[k] for k in ("counts", "key_mean", "value_mean", "ellipsoid", "value_norm",
                             "max_value_norm")}
    torch.cuda.synchronize()
    assert_summary_equal(summary, ref)
    anchor = torch.from_numpy(g["anchor"]).bool().to(DEV) if "anchor" in g else None
    mask = select_blocks(inp["query"].to(DEV), summary, cfg, workspace={})
    assert np.array_equal(mask.cpu().numpy().astype(np.uint8), g["mask"])
    res = sparse_attention(inp["query"].to(DEV), summary, inp["suffix_keys"].to(DEV),
                           inp["suffix_values"].to(DEV), cfg, anchor_mask=anchor, workspace={},
                           return_selected=True)
    assert np.array_equal(res.selected.cpu().numpy().astype(np.uint8), g["selected"])
    assert_close_output(res.output.float().cpu().numpy(), g["output"])


def test_headline_shape_128k(hip, oracle_lib):
    """BASELINE config 3 shape (H_kv 8, G 4, d 128, 131072 prompt tokens, B 32):
    masks equal the oracle's at full size, outputs within tolerance (both
    decode paths), and the all-expanded step equals dense attention."""
    _headline_shape_128k(hip, oracle_lib)


def test_long_context_512k(hip, oracle_lib):
    """The sweep's longest context (H_kv 8, G 4, d 128, 524288 prompt tokens,
    B 32: 256 tiles per head, four times the workgroups the device holds for
    a head, so each of the step's 64 workgroups per head scores 4 tiles):
    masks equal the oracle's selection over this summary and outputs are
    within tolerance of the oracle's, for the one-launch step and for the
    three kernels.  (The summary kernel itself is pinned bit for bit at
    131072 tokens.)"""
    prompt, block, eps = 524288, 32, 0.01
    inp = _decode_case(8, 4, 128, block, prompt, 0.01, suffix=17, seed=5)
    cfg = RefineKVConfig(backend="hip", eps=eps, block_size=block)
    k, v = inp["prompt_keys"], inp["prompt_values"]
    summary = build_summary(k.to(DEV), v.to(DEV), cfg)
    summ = oracle_summary_of(summary)
    qn = inp["query"][:, :, 0].float().numpy()
    out, mask = oracle_lib.sparse_attention(qn, summ, _pages_bits(k, block),
                                            _pages_bits(v, block),
                                            gc.bf16_bits(inp["suffix_keys"]),
                                            gc.bf16_bits(inp["suffix_values"]), eps, "any")
    assert 0.005 < mask.mean() < 0.1
    assert hip.decode_plan(8, 4, 128, summary.num_blocks, block) == "step-tiles"
    for path in ("step", "split"):
        hip.set_decode_path(path)
        try:
            ws = {}
            res = sparse_attention(inp["query"].to(DEV), summary, inp["suffix_keys"].to(DEV),
                                   inp["suffix_values"].to(DEV), cfg, workspace=ws,
                                   return_selected=True)
            torch.cuda.synchronize()
            assert np.array_equal(res.selected.cpu().numpy().astype(np.uint8), mask), path
            assert_close_output(res.output.float().cpu().numpy()[:, :, 0],
                                torch.from_numpy(out).to(torch.bfloat16).float().numpy())
        finally:
            hip.set_decode_path("step")
        assert assert_control_clean(hip, ws) == (1 if path == "step" else 0)


def _headline_shape_128k(hip, oracle_lib):
    inp = _decode_case(8, 4, 128, 32, 131072, 0.02, suffix=65, seed=1)
    cfg = RefineKVConfig(backend="hip", eps=0.01)
    k, v = inp["prompt_keys"], inp["prompt_values"]
    kd, vd = k.to(DEV), v.to(DEV)
    summary = build_summary(kd, vd, cfg)
    summ = oracle_summary_of(summary)
    ref = oracle_lib.summary(k.float().numpy(), v.float().numpy(), 32)
    assert_summary_equal(summary, ref)
    qn = inp["query"][:, :, 0].float().numpy()
    out, mask = oracle_lib.sparse_attention(qn, summ, _pages_bits(k, 32), _pages_bits(v, 32),
                                            gc.bf16_bits(inp["suffix_keys"]),
                                            gc.bf16_bits(inp["suffix_values"]), 0.01, "any")
    assert 0.005 < mask.mean() < 0.1
    for path in ("step", "split"):
        hip.set_decode_path(path)
        ws = {}
        try:
            res = sparse_attention(inp["query"].to(DEV), summary, inp["suffix_keys"].to(DEV),
                                   inp["suffix_values"].to(DEV), cfg, workspace=ws,
                                   return_selected=True)
            torch.cuda.synchronize()
        finally:
            hip.set_decode_path("step")
        assert np.array_equal(res.selected.cpu().numpy().astype(np.uint8), mask), path
        assert_close_output(res.output.float().cpu().numpy()[:, :, 0],
                            torch.from_numpy(out).to(torch.bfloat16).float().numpy())
        assert assert_control_clean(hip, ws) == (1 if path == "step" else 0)
    dense = sparse_attention(inp["query"].to(DEV), summary, inp["suffix_keys"].to(DEV),
                             inp["suffix_values"].to(DEV), RefineKVConfig(backend="hip", eps=0),
                             workspace={}, return_selected=True)
    assert dense.selected.all()
    kk = torch.cat([kd, inp["suffix_keys"].to(DEV)], 1).float().repeat_interleave(4, 0)
    vv = torch.cat([vd, inp["suffix_values"].to(DEV)], 1).float().repeat_interleave(4, 0)
    want = torch.nn.functional.scaled_dot_product_attention(
        inp["query"].to(DEV).float().reshape(32, 1, 128), kk, vv)
    # The reference's output is in the query dtype: compare bf16 with bf16.
    assert_close_output(dense.output.float().reshape(32, 1, 128).cpu().numpy(),
                        want.to(torch.bfloat16).float().cpu().numpy())


# ---------------------------------------------------------------------------
# The BASELINE configs' attention ops at their full sizes
# ---------------------------------------------------------------------------

def _op_case(hip, oracle_lib, *, heads, group, block, prompt, reduction, eps, spikes, suffix,
             anchors, seed, paths=("step", "split"), repeats=1):
    """One decode step of the op at a config's full size, on each path:
    prompt-anchor union (when anchors > 0) equal to the OR of the oracle's
    per-query masks, decode masks equal to the oracle's, outputs within
    tolerance, control words consistent.  Returns the oracle mask."""
    inp = testing.decode_inputs(heads=heads, group=group, dim=128, prompt=prompt, suffix=suffix,
                                block=block, spike_fraction=spikes, anchors=max(anchors, 1),
                                seed=seed)
    inp = {k: (v.to(torch.bfloat16) if v.is_floating_point() else v) for k, v in inp.items()}
    cfg = RefineKVConfig(backend="hip", block_size=block, eps=eps, gqa_reduction=reduction)
    k, v = inp["prompt_keys"], inp["prompt_values"]
    summary = build_summary(k.to(DEV), v.to(DEV), cfg)
    summ = oracle_summary_of(summary)
    anchor = None
    if anchors:
        queries = inp["anchor_queries"]
        got = select_blocks_union(queries.to(DEV), summary, cfg, workspace={})
        want = np.zeros((heads, summary.num_blocks), np.uint8)
        for a in range(anchors):
            mask, _, _ = oracle_lib.select(queries[:, :, a].float().numpy(), summ, eps, reduction)
            want |= mask
        assert np.array_equal(got.cpu().numpy().astype(np.uint8), want), "anchor union"
        anchor = got
    qn = inp["query"][:, :, 0].float().numpy()
    out, mask = oracle_lib.sparse_attention(
        qn, summ, _pages_bits(k, block), _pages_bits(v, block), gc.bf16_bits(inp["suffix_keys"]),
        gc.bf16_bits(inp["suffix_values"]), eps, reduction,
        None if anchor is None else anchor.cpu().numpy())
    want_out = torch.from_numpy(out).to(torch.bfloat16).float().numpy()
    one = one_launch(hip, heads, group, 128, summary.num_blocks, block)
    for path in paths:
        hip.set_decode_path(path)
        ws = {}
        try:
            for _ in range(repeats):
                res = sparse_attention(inp["query"].to(DEV), summary, inp["suffix_keys"].to(DEV),
                                       inp["suffix_values"].to(DEV), cfg, anchor_mask=anchor,
                                       workspace=ws, return_selected=True)
                torch.cuda.synchronize()
                assert np.array_equal(res.selected.cpu().numpy().astype(np.uint8), mask), path
                assert_close_output(res.output.float().cpu().numpy()[:, :, 0], want_out)
        finally:
            hip.set_decode_path("step")
        assert assert_control_clean(hip, ws) == (repeats if path == "step" and one else 0)
    return mask


def test_config1_op_llama_32k(hip, oracle_lib):
    """BASELINE configs[1]'s attention op: 8 KV / 32 query heads, d 128,
    32768 prompt tokens, block 32, eps 0.01, "any", 32 prompt anchors,
    suffix 65 (the middle of a 128-token decode)."""
    mask = _op_case(hip, oracle_lib, heads=8, group=4, block=32, prompt=32768, reduction="any",
                    eps=0.01, spikes=0.02, suffix=65, anchors=32, seed=21)
    assert 0.005 < mask.mean() < 0.5


def test_config3_op_qwen_64k(hip, oracle_lib):
    """BASELINE configs[3]'s attention op: 4 KV / 28 query heads (group 7),
    d 128, 65536 prompt tokens, block 64, eps 0.005, "max", 64 prompt
    anchors."""
    _op_case(hip, oracle_lib, heads=4, group=7, block=64, prompt=65536, reduction="max",
             eps=0.005, spikes=0.02, suffix=65, anchors=64, seed=22)


def test_two_device_fulls_step_512k_block64(hip, oracle_lib):
    """8 KV heads of 6 query heads (eight-row passes, which score one tile
    per workgroup), 524288 prompt tokens, block 64: 128 tiles per head, 1024
    workgroups, twice what the device holds at once, so the one-launch step
    maps workgroups to (head, tile) by start-order tickets.  Two launches on
    one workspace (the tickets and tags of the second follow the first)."""
    n_blocks = 524288 // 64
    assert hip.decode_plan(8, 6, 128, n_blocks, 64) == "step-ticketed"
    _op_case(hip, oracle_lib, heads=8, group=6, block=64, prompt=524288, reduction="any",
             eps=0.01, spikes=0.02, suffix=17, anchors=0, seed=23, paths=("step",), repeats=2)


def test_sweep_512k_block16_three_kernels(hip, oracle_lib):
    """The op sweep's 524288-token point at block 16 (8 KV heads, G 4, d 128):
    32768 blocks, 512 tiles per head, more than the one-launch step holds,
    so rkv_decode runs the three kernels; masks equal the oracle's, outputs
    within tolerance."""
    n_blocks = 524288 // 16
    assert hip.decode_plan(8, 4, 128, n_blocks, 16) == "split"
    mask = _op_case(hip, oracle_lib, heads=8, group=4, block=16, prompt=524288,
                    reduction="any", eps=0.01, spikes=0.02, suffix=17, anchors=0, seed=25,
                    paths=("step",))
    assert 0.005 < mask.mean() < 0.1


@pytest.mark.parametrize("eps,spikes", [(0.01, 0.02), (0.0, 0.02)], ids=["eps0.01", "eps0"])
def test_sweep_512k_block64_several_tiles(hip, oracle_lib, eps, spikes):
    """The op sweep's 524288-token point at block 64 with G 4: 8192 blocks,
    128 tiles per head, so each of the one-launch step's 64 workgroups per
    head scores two tiles of 64-token blocks; at eps 0 every block of every
    head expands (each workgroup's share of the head's 524288 rows).  Both
    paths, two launches on one workspace."""
    n_blocks = 524288 // 64
    assert hip.decode_plan(8, 4, 128, n_blocks, 64) == "step-tiles"
    mask = _op_case(hip, oracle_lib, heads=8, group=4, block=64, prompt=524288,
                    reduction="any", eps=eps, spikes=spikes, suffix=33, anchors=0, seed=26,
                    repeats=2)
    if eps == 0.0:
        assert mask.all()
    else:
        assert 0.005 < mask.mean() < 0.1


def test_several_tiles_per_workgroup_128k_block16(hip, oracle_lib):
    """The headline shape at block 16: 128 tiles per head, twice the 64
    workgroups per head the device holds, so each workgroup of the one-launch
    step scores 2 tiles.  Both paths, two launches on one workspace, with
    prompt anchors."""
    n_blocks = 131072 // 16
    assert hip.decode_plan(8, 4, 128, n_blocks, 16) == "step-tiles"
    _op_case(hip, oracle_lib, heads=8, group=4, block=16, prompt=131072, reduction="any",
             eps=0.01, spikes=0.02, suffix=33, anchors=16, seed=24, repeats=2)


# ---------------------------------------------------------------------------
# A hand-off wait that gives up is reported, not silent
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("heads,group,block,prompt", [(8, 4, 32, 8192), (4, 7, 64, 16384)])
def test_handoff_give_up_is_reported_and_recoverable(hip, oracle_lib, heads, group, block, prompt):
    """With the test hook every wait of the one-launch step accepts no data
    and gives up after 64 polls: every kernel still ends, the status word is
    set and check_workspace raises, and the call's result says so in-band:
    every output row is NaN and every block is marked expanded (a plain call
    or a graph replay cannot return a plausible wrong answer).  After
    clearing the word, the same workspace decodes correctly again.  (Group
    7 runs the 8-row step, whose waves poll two rows' LSE slots at once.)"""
    inp = _decode_case(heads, group, 128, block, prompt, 0.02, suffix=9, seed=4)
    cfg = RefineKVConfig(backend="hip", eps=0.01, block_size=block)
    summary = build_summary(inp["prompt_keys"].to(DEV), inp["prompt_values"].to(DEV), cfg)
    assert one_launch(hip, heads, group, 128, summary.num_blocks, block)
    args = (inp["query"].to(DEV), summary, inp["suffix_keys"].to(DEV),
            inp["suffix_values"].to(DEV), cfg)
    ws = {}
    sparse_attention(*args, workspace=ws)
    torch.cuda.synchronize()
    assert hip.workspace_status(ws) == 0
    hip.set_handoff_test(64, 1)
    try:
        bad = sparse_attention(*args, workspace=ws, return_selected=True)
        torch.cuda.synchronize()
    finally:
        hip.set_handoff_test(0, 0)
    assert hip.workspace_status(ws) & 1
    assert torch.isnan(bad.output.float()).all()
    assert bad.selected.all()
    with pytest.raises(hip.HandoffError):
        hip.check_workspace(ws)
    hip.clear_workspace_status(ws)
    res = sparse_attention(*args, workspace=ws, return_selected=True)
    torch.cuda.synchronize()
    summ = oracle_summary_of(summary)
    out, mask = oracle_lib.sparse_attention(
        inp["query"][:, :, 0].float().numpy(), summ, _pages_bits(inp["prompt_keys"], block),
        _pages_bits(inp["prompt_values"], block), gc.bf16_bits(inp["suffix_keys"]),
        gc.bf16_bits(inp["suffix_values"]), 0.01, "any")
    assert np.array_equal(res.selected.cpu().numpy().astype(np.uint8), mask)
    assert_close_output(res.output.float().cpu().numpy()[:, :, 0],
                        torch.from_numpy(out).to(torch.bfloat16).float().numpy())
    assert assert_control_clean(hip, ws) == 3
