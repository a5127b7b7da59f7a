"""Seeded synthetic decode workloads (no datasets, no checkpoints).

One generator recipe serves the parity fixtures, the tests and the benchmark,
so every consumer sees the same tensors for the same seed.  Everything is
drawn on the CPU from ``torch.Generator('cpu')``, whose streams do not depend
on the machine, then cast and moved by the caller.

Recipe (per KV head h, prompt block b, head_dim D):
* query q ~ N(0, 1), shape (H, G, 1, D); prompt+suffix keys and values
  ~ N(0, 1), shape (H, P + S, D);
* every prompt token of block b gets the same key offset o[h, b] ~ N(0, s^2)
  (s = ``offset_std``), so block means differ;
* ``spike_fraction`` of the (h, b) pairs, chosen by ``randperm``, get
  ``spike_scale * mean_g q[h, g]`` added to every key of the block: these
  blocks carry most of the attention mass and must be expanded;
* anchor queries (H, G, A, D) = q + ``anchor_noise`` * N(0, 1), standing in
  for the tail prompt queries of a real model.
"""

import math

import torch


def decode_inputs(heads=8, group=4, dim=128, prompt=4096, suffix=16, block=32,
                  spike_fraction=0.02, anchors=32, offset_std=0.5, spike_scale=4.0,
                  anchor_noise=0.5, seed=0):
    g = torch.Generator("cpu").manual_seed(seed)
    query = torch.randn(heads, group, 1, dim, generator=g)
    keys = torch.randn(heads, prompt + suffix, dim, generator=g)
    values = torch.randn(heads, prompt + suffix, dim, generator=g)
    n_blocks = math.ceil(prompt / block)
    offset = torch.randn(heads, n_blocks, dim, generator=g) * offset_std
    keys[:, :prompt] += offset.repeat_interleave(block, dim=1)[:, :prompt]
    n_spikes = round(spike_fraction * heads * n_blocks)
    picks = torch.randperm(heads * n_blocks, generator=g)[:n_spikes]
    mean_query = query[:, :, 0].mean(1)
    for index in picks.tolist():
        h, b = divmod(index, n_blocks)
        keys[h, b * block:min((b + 1) * block, prompt)] += spike_scale * mean_query[h]
    anchor_queries = query + anchor_noise * torch.randn(heads, group, anchors, dim, generator=g)
    return dict(
        query=query,
        prompt_keys=keys[:, :prompt],
        prompt_values=values[:, :prompt],
        suffix_keys=keys[:, prompt:],
        suffix_values=values[:, prompt:],
        anchor_queries=anchor_queries,
        spikes=picks,
    )


def small_inputs(length=71, dim=64, seed=42, heads=2, group=4, dtype=torch.bfloat16):
    """The shape family of the reference's own unit tests
    (tests/test_attention.py:10-16): q (H, G, 1, D), K/V (H, L, D)."""
    g = torch.Generator("cpu").manual_seed(seed)

    def normal(shape):
        return torch.randn(shape, generator=g, dtype=dtype)

    return normal((heads, group, 1, dim)), normal((heads, length, dim)), normal((heads, length, dim))


def wide_inputs(length=1000, dim=96, seed=7, heads=2, group=4):
    """fp32 inputs with a wide dynamic range (|x| spans ~2^-12..2^12), where
    fp32 sums are inexact and so depend on the summation order."""
    g = torch.Generator("cpu").manual_seed(seed)

    def wide(shape):
        return torch.randn(shape, generator=g) * torch.exp(2.0 * torch.randn(shape, generator=g))

    return wide((heads, group, 1, dim)), wide((heads, length, dim)), wide((heads, length, dim))
