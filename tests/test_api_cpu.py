"""CPU behaviour of the public API.

The properties the reference's tests/test_attention.py:19-136 pin (summary
counts and layout, the ellipsoid bound, eps special cases, anchors, large
delta, config validation), on inputs of this suite's own, checked against
the C oracle and closed forms; the dispatch rules of the kernel backend; and
bit-for-bit agreement of the torch backend with the reference's golden
vectors (same torch operations in the same order).
"""

import numpy as np
import pytest
import torch

import golden_cases as gc
from refinekv import RefineKVConfig, build_summary, select_blocks, sparse_attention
from refinekv.attention import _backend


def _bits(t):
    return t.detach().contiguous().view(torch.int16).numpy().view(np.uint16)


def _oracle_summary(summary):
    return dict(counts=summary.counts.numpy(), key_mean=_bits(summary.key_mean),
                value_mean=_bits(summary.value_mean), ellipsoid=_bits(summary.ellipsoid),
                value_norm=summary.value_norm.numpy(),
                max_value_norm=summary.max_value_norm.numpy(),
                prompt_length=summary.prompt_length, block_size=summary.block_size)


def _cache(heads, length, dim, seed, dtype=torch.bfloat16, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    keys = (torch.randn(heads, length, dim, generator=g) * scale).to(dtype)
    values = torch.randn(heads, length, dim, generator=g).to(dtype)
    return keys, values


# -- summaries: counts, partial blocks, layout, no mutation ----------------
# (what the reference's tests/test_attention.py:19-56 pin, checked here
# against the C oracle's restatement of summary.py:46-113)

@pytest.mark.parametrize("block,extra", [(16, 1), (32, 5), (64, 63)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_partial_last_block_summary_matches_oracle(oracle_lib, block, extra, dtype):
    """A prompt of 2 whole blocks plus `extra` tokens: counts follow the
    closed form, every summary field of the short block (and the others)
    equals the oracle bit for bit, and the page view keeps (block, dim)
    rows with the padding zero."""
    length = 2 * block + extra
    keys, values = _cache(3, length, 96, seed=block + extra, dtype=dtype)
    summary = build_summary(keys, values, RefineKVConfig(block_size=block,
                                                         summary_chunk_blocks=2))
    assert summary.counts.tolist() == [block, block, extra]
    ref = oracle_lib.summary(keys.float().numpy(), values.float().numpy(), block)
    got = _oracle_summary(summary)
    for name in ("key_mean", "value_mean", "ellipsoid"):
        assert np.array_equal(got[name], ref[name]), name
    for name in ("value_norm", "max_value_norm"):
        assert np.array_equal(got[name].view(np.uint32), ref[name].view(np.uint32)), name
    assert summary.keys.shape == (3, 3, block, 96)
    assert summary.keys.stride()[2:] == (96, 1)
    assert not summary.keys[:, -1, extra:].any() and not summary.values[:, -1, extra:].any()


@pytest.mark.parametrize("length", [96, 90])
def test_summary_leaves_cache_untouched_and_views_it_when_aligned(length):
    """Pages alias a block-aligned prompt of a larger cache (no copy), are a
    padded copy otherwise, and the cache itself is never written."""
    cache_k, cache_v = _cache(2, 128, 32, seed=3, dtype=torch.float32)
    before_k, before_v = cache_k.clone(), cache_v.clone()
    summary = build_summary(cache_k[:, :length], cache_v[:, :length],
                            RefineKVConfig(backend="torch", block_size=32))
    assert torch.equal(cache_k, before_k) and torch.equal(cache_v, before_v)
    aligned = length % 32 == 0
    assert (summary.keys.data_ptr() == cache_k.data_ptr()) == aligned
    flat_k = summary.keys.reshape(2, -1, 32)
    flat_v = summary.values.reshape(2, -1, 32)
    assert torch.equal(flat_k[:, :length], before_k[:, :length])
    assert torch.equal(flat_v[:, :length], before_v[:, :length])


def test_ellipsoid_bounds_every_query_even_with_constant_axes(oracle_lib):
    """Five key axes held constant inside every block (zero width there) and
    random queries of very different scales: the ellipsoid stays finite,
    equals the oracle's bits, and sqrt(q^2 . W) bounds |q . (k - k_mean)|
    for every token (computed in fp64)."""
    keys, values = _cache(2, 150, 64, seed=9)
    keys[..., 10:15] = torch.tensor([7.0, -3.5, 0.0, 250.0, -0.125], dtype=torch.bfloat16)
    summary = build_summary(keys, values, RefineKVConfig(block_size=16, summary_chunk_blocks=3))
    assert torch.isfinite(summary.ellipsoid.float()).all()
    ref = oracle_lib.summary(keys.float().numpy(), values.float().numpy(), 16)
    assert np.array_equal(_bits(summary.ellipsoid), ref["ellipsoid"])
    g = torch.Generator().manual_seed(4)
    queries = torch.randn(2, 40, 64, generator=g, dtype=torch.float64)
    queries *= torch.logspace(-2, 2, 40, dtype=torch.float64)[None, :, None]
    pages = summary.keys.double()
    centered = pages - summary.key_mean.double()[:, :, None]
    valid = torch.arange(16)[None] < summary.counts[:, None]
    deviation = torch.einsum("hqd,hntd->hqnt", queries, centered).abs()
    deviation = deviation.masked_fill(~valid[None, None], 0).amax(-1)
    bound = torch.einsum("hqd,hnd->hqn", queries.square(), summary.ellipsoid.double()).sqrt()
    assert (deviation <= bound * (1 + 1e-9)).all()


# -- attention: special cases with closed forms -----------------------------
# (tests/test_attention.py:74-116 of the reference)

@pytest.mark.parametrize("suffix", [0, 7])
def test_eps_zero_expands_everything_and_equals_dense_softmax(oracle_lib, suffix):
    """eps = 0 selects every block (risk > 0 for a nonzero query); the output
    is then plain softmax attention over prompt + suffix, computed here in
    fp64 over the same bf16 values."""
    keys, values = _cache(2, 83 + suffix, 64, seed=21)
    q = torch.randn(2, 3, 1, 64, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    cfg = RefineKVConfig(backend="torch", eps=0.0, block_size=16)
    summary = build_summary(keys[:, :83], values[:, :83], cfg)
    result = sparse_attention(q, summary, keys[:, 83:], values[:, 83:], cfg,
                              return_selected=True)
    assert result.selected.all()
    logits = torch.einsum("hgd,htd->hgt", q[:, :, 0].double(), keys.double()) / 8.0
    want = torch.einsum("hgt,htd->hgd", logits.softmax(-1), values.double())
    got = result.output[:, :, 0].double()
    assert (got - want).abs().max() <= 8e-3  # bf16 output rounding
    out, mask = oracle_lib.sparse_attention(
        q[:, :, 0].float().numpy(), _oracle_summary(summary),
        _bits(gc.padded_pages(keys[:, :83], 16)), _bits(gc.padded_pages(values[:, :83], 16)),
        _bits(keys[:, 83:]), _bits(values[:, 83:]), 0.0, "any")
    assert mask.all()
    assert (got - torch.from_numpy(out).double()).abs().max() <= 8e-3


def test_unexpanded_short_block_weighs_by_its_true_count():
    """No block expands (eps huge) and every logit is equal (zero query and
    keys): the output is the count-weighted mean of the block value means,
    (32 * 2 + 5 * 7) / 37, with the short block counted 5 times, not 32."""
    cfg = RefineKVConfig(backend="torch", eps=1e9, block_size=32)
    keys = torch.zeros(1, 37, 32)
    values = torch.full((1, 37, 32), 2.0)
    values[:, 32:] = 7.0
    summary = build_summary(keys, values, cfg)
    result = sparse_attention(torch.zeros(1, 3, 1, 32), summary, keys[:, :0], values[:, :0], cfg,
                              return_selected=True)
    assert not result.selected.any()
    # (fp32 softmax weights e^{ln 32}, e^{ln 5}: a few ulp from the closed form)
    torch.testing.assert_close(result.output, torch.full_like(result.output, 99.0 / 37.0),
                               rtol=4e-7, atol=0)


def test_anchors_alone_decide_when_nothing_else_expands(oracle_lib):
    """At a threshold nothing reaches, the expanded set is exactly the anchor
    mask, and the output equals the oracle's for that selection."""
    keys, values = _cache(3, 200, 32, seed=13)
    q = torch.randn(3, 2, 1, 32, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16)
    cfg = RefineKVConfig(backend="torch", eps=1e9, block_size=16)
    summary = build_summary(keys, values, cfg)
    anchor = torch.zeros(3, summary.num_blocks, dtype=torch.bool)
    anchor[0, ::3] = True
    anchor[2, -1] = True
    result = sparse_attention(q, summary, keys[:, :0], values[:, :0], cfg, anchor_mask=anchor,
                              return_selected=True)
    assert torch.equal(result.selected, anchor)
    empty = np.zeros((3, 0, 32), np.uint16)
    out, mask = oracle_lib.sparse_attention(
        q[:, :, 0].float().numpy(), _oracle_summary(summary),
        _bits(gc.padded_pages(keys, 16)), _bits(gc.padded_pages(values, 16)), empty, empty,
        1e9, "any", anchor.numpy())
    assert np.array_equal(mask, anchor.numpy().astype(np.uint8))
    assert (result.output[:, :, 0].float() - torch.from_numpy(out)).abs().max() <= 8e-3


def test_huge_query_takes_the_large_delta_branch_and_stays_finite(oracle_lib):
    """A query scaled by 300 puts every block's delta far past 10 (the
    risk's large-delta forms): the mask equals the oracle's and every output
    is finite."""
    keys, values = _cache(2, 130, 64, seed=30)
    q = (torch.randn(2, 4, 1, 64, generator=torch.Generator().manual_seed(2)) * 300).to(
        torch.bfloat16)
    cfg = RefineKVConfig(backend="torch", block_size=32)
    summary = build_summary(keys, values, cfg)
    stats = oracle_lib.select_stats(q[:, :, 0].float().numpy(), _oracle_summary(summary))
    assert (stats["delta"] > 10).all()
    selected = select_blocks(q, summary, cfg)
    want, _, _ = oracle_lib.select(q[:, :, 0].float().numpy(), _oracle_summary(summary),
                                   cfg.eps, "any")
    assert np.array_equal(selected.numpy().astype(np.uint8), want)
    result = sparse_attention(q, summary, keys[:, :0], values[:, :0], cfg)
    assert torch.isfinite(result.output.float()).all()


@pytest.mark.parametrize("kwargs", [{"eps": float("inf")}, {"eps": -0.5}, {"block_size": 48},
                                    {"anchor_tokens": True}, {"anchor_tokens": 2.0},
                                    {"backend": "cuda"}, {"gqa_reduction": "min"},
                                    {"summary_chunk_blocks": -3},
                                    {"full_attention_layers": -1}])
def test_bad_config_values_raise_value_error(kwargs):
    with pytest.raises(ValueError):
        RefineKVConfig(**kwargs)


def test_triton_is_accepted_as_the_kernel_backend_name():
    """Configurations written for the reference (backend="triton") keep
    working: the name selects the gfx950 kernels, and off a ROCm device it
    fails as an explicit kernel request does."""
    assert RefineKVConfig(backend="triton").backend == "triton"
    q = torch.zeros(2, 4, 1, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="ROCm"):
        _backend(q, RefineKVConfig(backend="triton"))


def test_backend_dispatch_rules_on_cpu():
    q = torch.zeros(2, 4, 1, 64, dtype=torch.bfloat16)
    assert _backend(q, RefineKVConfig()) == "torch"
    assert _backend(q, RefineKVConfig(backend="torch")) == "torch"
    with pytest.raises(RuntimeError, match="ROCm"):
        _backend(q, RefineKVConfig(backend="hip"))


def test_device_suffix_length_requires_hip():
    keys, values = _cache(2, 71, 64, seed=42)
    q = torch.randn(2, 4, 1, 64, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    summary = build_summary(keys, values)
    with pytest.raises(ValueError, match="HIP"):
        sparse_attention(q, summary, keys[:, :4], values[:, :4], RefineKVConfig(),
                         suffix_length=torch.tensor(2, dtype=torch.int32))


def test_bf16_page_copy_is_made_once_per_cache_version():
    """An fp32 cache under the kernel backend: the bf16 copy of the pages is
    converted once and kept in the workspace; a write to the cache (a new
    tensor version) converts again, and no workspace means a fresh copy."""
    from refinekv.attention import _bf16_pages

    keys, values = _cache(2, 71, 64, seed=43, dtype=torch.float32)
    summary = build_summary(keys, values)
    ws = {}
    a = _bf16_pages(summary, ws)
    b = _bf16_pages(summary, ws)
    assert a.keys.dtype == a.values.dtype == torch.bfloat16
    assert a.keys is b.keys and a.values is b.values
    assert torch.equal(a.keys, summary.keys.to(torch.bfloat16))
    summary.keys[0, 1, 3] += 1.0  # the cache is written: the copy follows it
    c = _bf16_pages(summary, ws)
    assert c.keys is not a.keys and torch.equal(c.keys, summary.keys.to(torch.bfloat16))
    assert c.values is not a.values or summary.values._version == 0
    assert _bf16_pages(summary).keys is not c.keys
    bf = build_summary(keys.to(torch.bfloat16), values.to(torch.bfloat16))
    assert _bf16_pages(bf, ws) is bf


@pytest.fixture
def one_thread():
    # The fixtures were written single-threaded; MKL's matmul order depends on
    # the thread count.
    n = torch.get_num_threads()
    torch.set_num_threads(1)
    yield
    torch.set_num_threads(n)


@pytest.mark.parametrize("path", gc.fixture_paths(), ids=lambda p: p.split("/")[-1][:-4])
def test_torch_backend_reproduces_reference_bits(path, one_thread):
    g, meta = gc.load(path)
    inp = gc.regenerate(meta)
    cfg = RefineKVConfig(backend="torch", **meta["config"])
    summary = build_summary(inp["keys"], inp["values"], cfg)
    bits = lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16)
    for name in ("key_mean", "value_mean", "ellipsoid"):
        assert np.array_equal(bits(getattr(summary, name)), g[name]), name
    assert np.array_equal(summary.value_norm.numpy().view(np.uint32),
                          g["value_norm"].view(np.uint32))
    result = sparse_attention(inp["query"], summary, inp["suffix_keys"], inp["suffix_values"],
                              cfg, anchor_mask=None if "anchor" not in g else
                              torch.from_numpy(g["anchor"]).bool(), return_selected=True)
    assert np.array_equal(result.selected.numpy().astype(np.uint8), g["selected"])
    assert np.array_equal(result.output.float().numpy(), g["output"])
