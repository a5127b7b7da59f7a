"""CPU behaviour of the public API (the reference's CPU tests, restated).

Covers src/refinekv tests/test_attention.py:19-136 against this package's
torch backend, the config and dispatch rules of the hip backend, and
bit-for-bit agreement of the torch backend with the reference's golden
vectors (same torch operations in the same order).
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import golden_cases as gc
from refinekv import RefineKVConfig, build_summary, select_blocks, sparse_attention, testing
from refinekv.attention import _backend


def _inputs(length=71, dim=64):
    return testing.small_inputs(length=length, dim=dim)


@pytest.mark.parametrize("block", [16, 32, 64])
def test_partial_page_summaries_ignore_padding_and_preserve_layout(block):
    _, keys, values = _inputs(length=block + 3)
    keys = torch.cat([keys, torch.zeros_like(keys)], 1)[:, : block + 3]
    config = RefineKVConfig(block_size=block, summary_chunk_blocks=1)
    summary = build_summary(keys, values, config)
    assert summary.counts.tolist() == [block, 3]
    torch.testing.assert_close(summary.key_mean[:, -1],
                               keys[:, -3:].float().mean(1).to(torch.bfloat16))
    torch.testing.assert_close(summary.value_mean[:, -1],
                               values[:, -3:].float().mean(1).to(torch.bfloat16))
    assert summary.keys.stride(2) == keys.shape[-1]
    assert summary.keys.stride(3) == 1


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("length", [64, 67])
def test_summary_preserves_input_cache_and_exact_keys(dtype, length):
    g = torch.Generator().manual_seed(17)
    key_cache = torch.randn(2, 96, 64, generator=g).to(dtype)
    value_cache = torch.randn(2, 96, 64, generator=g).to(dtype)
    original_keys, original_values = key_cache.clone(), value_cache.clone()
    summary = build_summary(key_cache[:, :length], value_cache[:, :length],
                            RefineKVConfig(backend="torch", summary_chunk_blocks=1))
    assert torch.equal(key_cache, original_keys) and torch.equal(value_cache, original_values)
    assert torch.equal(summary.keys.reshape(2, -1, 64)[:, :length], original_keys[:, :length])
    assert torch.equal(summary.values.reshape(2, -1, 64)[:, :length],
                       original_values[:, :length])


def test_centered_ellipsoid_handles_constant_axes_and_bounds_sampled_queries():
    q, keys, values = _inputs(length=65, dim=128)
    keys[..., :3] = torch.tensor([96, 48, -80], dtype=torch.bfloat16)
    summary = build_summary(keys, values, RefineKVConfig(summary_chunk_blocks=1))
    assert torch.isfinite(summary.ellipsoid).all()
    centered = summary.keys.float() - summary.key_mean.float().unsqueeze(2)
    exact = torch.einsum("hgd,hbtd->hgbt", q[:, :, 0].float(), centered).abs()
    valid = torch.arange(summary.block_size)[None] < summary.counts[:, None]
    exact = exact.masked_fill(~valid[None, None], 0).amax(-1)
    bound = torch.einsum("hgd,hbd->hgb", q[:, :, 0].float().square(),
                         summary.ellipsoid.float()).sqrt()
    assert (exact <= bound + 1e-5).all()


@pytest.mark.parametrize("suffix_length", [0, 5])
def test_full_expansion_matches_dense_attention(suffix_length):
    q, keys, values = _inputs()
    config = RefineKVConfig(backend="torch", eps=0)
    summary = build_summary(keys, values, config)
    result = sparse_attention(q, summary, keys[:, :suffix_length], values[:, :suffix_length],
                              config, return_selected=True)
    assert result.selected.all()
    ek = torch.cat([keys, keys[:, :suffix_length]], 1).repeat_interleave(4, 0)
    ev = torch.cat([values, values[:, :suffix_length]], 1).repeat_interleave(4, 0)
    expected = F.scaled_dot_product_attention(q.reshape(8, 1, 64).float(), ek.float(), ev.float())
    torch.testing.assert_close(result.output.float().reshape(8, 1, 64), expected, atol=0.004,
                               rtol=0.02)


def test_representative_multiplicity_uses_actual_partial_page_count():
    config = RefineKVConfig(backend="torch", eps=1e6, block_size=16)
    keys = torch.zeros(1, 19, 64, dtype=torch.bfloat16)
    values = torch.zeros_like(keys)
    values[:, :16] = 1
    values[:, 16:] = 3
    summary = build_summary(keys, values, config)
    q = torch.zeros(1, 2, 1, 64)
    result = sparse_attention(q, summary, keys[:, :0], values[:, :0], config,
                              return_selected=True)
    assert not result.selected.any()
    torch.testing.assert_close(result.output, torch.full_like(result.output, (16 + 9) / 19))


def test_anchor_union_expands_only_requested_pages():
    q, keys, values = _inputs()
    config = RefineKVConfig(backend="torch", eps=1e6)
    summary = build_summary(keys, values, config)
    anchor = torch.zeros(2, summary.num_blocks, dtype=torch.bool)
    anchor[:, -1] = True
    result = sparse_attention(q, summary, keys[:, :0], values[:, :0], config,
                              anchor_mask=anchor, return_selected=True)
    assert torch.equal(result.selected, anchor)
    assert torch.isfinite(result.output).all()


def test_large_finite_delta_stays_finite():
    q, keys, values = _inputs()
    q = (q.float() * 200).to(torch.bfloat16)
    summary = build_summary(keys, values)
    selected = select_blocks(q, summary, RefineKVConfig(backend="torch"))
    result = sparse_attention(q, summary, keys[:, :0], values[:, :0],
                              RefineKVConfig(backend="torch"))
    assert selected.shape == (2, summary.num_blocks)
    assert torch.isfinite(result.output).all()


@pytest.mark.parametrize("kwargs", [{"eps": float("nan")}, {"eps": -1}, {"block_size": 10},
                                    {"anchor_tokens": -1}, {"backend": "triton"},
                                    {"gqa_reduction": "sum"}, {"summary_chunk_blocks": 0}])
def test_invalid_config_is_rejected(kwargs):
    with pytest.raises(ValueError):
        RefineKVConfig(**kwargs)


def test_backend_dispatch_rules_on_cpu():
    q = torch.zeros(2, 4, 1, 64, dtype=torch.bfloat16)
    assert _backend(q, RefineKVConfig()) == "torch"
    assert _backend(q, RefineKVConfig(backend="torch")) == "torch"
    with pytest.raises(RuntimeError, match="ROCm"):
        _backend(q, RefineKVConfig(backend="hip"))


def test_device_suffix_length_requires_hip():
    q, keys, values = _inputs()
    summary = build_summary(keys, values)
    with pytest.raises(ValueError, match="HIP"):
        sparse_attention(q, summary, keys[:, :4], values[:, :4], RefineKVConfig(),
                         suffix_length=torch.tensor(2, dtype=torch.int32))


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
