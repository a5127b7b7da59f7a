"""select_blocks_union on the torch backend (CPU): the OR of per-query
selections, checked against the CPU oracle's per-query masks."""

import numpy as np
import pytest
import torch

from refinekv import RefineKVConfig, build_summary, select_blocks_union, testing


@pytest.mark.parametrize("reduction", ["any", "max", "mean"])
def test_union_equals_or_of_oracle_masks(oracle_lib, reduction):
    inp = testing.decode_inputs(heads=2, group=4, dim=64, prompt=3000, suffix=4, block=32,
                                spike_fraction=0.1, anchors=4, seed=3)
    cfg = RefineKVConfig(backend="torch", block_size=32, eps=0.1, gqa_reduction=reduction)
    keys, values = (inp[k].to(torch.bfloat16) for k in ("prompt_keys", "prompt_values"))
    summary = build_summary(keys, values, cfg)
    gen = torch.Generator().manual_seed(1)
    # perturbed copies of the decode query: related but different selections
    queries = inp["query"].float() + 0.3 * torch.randn(2, 4, 3, 64, generator=gen)
    queries[:, :, 0] = inp["query"][:, :, 0].float()
    queries = queries.to(torch.bfloat16)
    got = select_blocks_union(queries, summary, cfg).numpy()
    summ = dict(counts=summary.counts.numpy(),
                key_mean=summary.key_mean.view(torch.int16).numpy().view(np.uint16),
                value_mean=summary.value_mean.view(torch.int16).numpy().view(np.uint16),
                ellipsoid=summary.ellipsoid.view(torch.int16).numpy().view(np.uint16),
                value_norm=summary.value_norm.numpy(),
                max_value_norm=summary.max_value_norm.numpy(),
                prompt_length=summary.prompt_length, block_size=summary.block_size)
    want = np.zeros(got.shape, np.uint8)
    for a in range(3):
        mask, _, _ = oracle_lib.select(queries[:, :, a].float().numpy(), summ, 0.1, reduction)
        want |= mask
    assert want.any() and not want.all()
    assert np.array_equal(got.astype(np.uint8), want)


def test_union_rejects_bad_shapes():
    inp = testing.decode_inputs(heads=1, group=2, dim=32, prompt=64, suffix=1, block=32, seed=0)
    cfg = RefineKVConfig(backend="torch", block_size=32)
    summary = build_summary(inp["prompt_keys"], inp["prompt_values"], cfg)
    with pytest.raises(ValueError):
        select_blocks_union(torch.zeros(1, 2, 32), summary, cfg)
