"""store_and_build_summary on the torch backend (CPU): the cache views get
the prompt and the summary equals build_summary of the written prompt."""

import torch

from refinekv import RefineKVConfig, build_summary
from refinekv.summary import store_and_build_summary


def test_store_and_build_summary_matches_copy_then_build():
    gen = torch.Generator().manual_seed(0)
    keys = torch.randn(70, 2, 32, generator=gen).transpose(0, 1)
    values = torch.randn(70, 2, 32, generator=gen).transpose(0, 1)
    cache = torch.zeros(2, 2, 100, 32)
    cfg = RefineKVConfig(backend="torch", block_size=16)
    got = store_and_build_summary(keys, values, cache[0, :, :70], cache[1, :, :70], cfg)
    assert torch.equal(cache[0, :, :70], keys) and torch.equal(cache[1, :, :70], values)
    assert not cache[:, :, 70:].any()
    want = build_summary(keys.contiguous(), values.contiguous(), cfg)
    for name in ("counts", "key_mean", "value_mean", "ellipsoid", "value_norm",
                 "max_value_norm", "keys", "values"):
        assert torch.equal(getattr(got, name), getattr(want, name)), name
    assert got.prompt_length == 70 and got.block_size == 16
