"""Prompt block summaries (mirror of src/refinekv/summary.py:10-113).

``build_summary`` runs the gfx950 summarizer for ROCm tensors (backend "auto"
or "hip") and a torch restatement otherwise.  Both produce the reference's
BlockSummary: bf16 count-weighted means, the centred diagonal ellipsoid
W^2 r^2 (1 + 2^-8) and fp32 per-block value norms, with the page views of the
cache as ``keys``/``values``.
"""

from dataclasses import dataclass

import torch

from .config import KERNEL_BACKENDS, RefineKVConfig


@dataclass
class BlockSummary:
    """Per-KV-head summaries of one immutable prompt prefix.

    ``keys``/``values`` are (kv_heads, blocks, block_size, head_dim) page views
    of the prompt K/V (sharing the cache allocation when the prompt length is a
    multiple of the block size); ``counts`` (blocks,) int64 holds the valid
    tokens per block; ``key_mean``, ``value_mean``, ``ellipsoid`` are
    (kv_heads, blocks, head_dim) bf16; ``value_norm`` (kv_heads, blocks) and
    ``max_value_norm`` (kv_heads,) are fp32.
    """

    keys: torch.Tensor
    values: torch.Tensor
    counts: torch.Tensor
    key_mean: torch.Tensor
    value_mean: torch.Tensor
    ellipsoid: torch.Tensor
    value_norm: torch.Tensor
    max_value_norm: torch.Tensor
    prompt_length: int
    block_size: int

    @property
    def num_blocks(self):
        return self.counts.numel()


def _pages(tensor, block_size):
    """(H, L, D) -> (H, N, B, D): a view when L % B == 0 and rows are dense,
    else a zero-padded copy (summary.py:35-43)."""
    heads, length, dim = tensor.shape
    padding = (-length) % block_size
    if padding:
        tensor = torch.cat([tensor, tensor.new_zeros(heads, padding, dim)], dim=1)
    pages = tensor.reshape(heads, -1, block_size, dim)
    if pages.stride(3) != 1 or pages.stride(2) != dim or pages.stride(1) != block_size * dim:
        pages = pages.contiguous()
    return pages


def _use_hip(keys, config):
    from . import _hip

    if not keys.is_cuda or config.backend == "torch":
        return False
    explicit = config.backend in KERNEL_BACKENDS
    if not _hip.is_rocm_device(keys):
        if explicit:
            raise RuntimeError("the HIP backend requires a ROCm device")
        return False
    supported = keys.dtype in _hip.DTYPE_CODES and keys.shape[-1] in _hip.SUPPORTED_DIMS
    if not supported:
        if explicit:
            raise ValueError("the HIP summarizer needs bf16/fp16/fp32 K/V with head_dim in "
                             "32..256 (multiple of 32)")
        return False
    _hip.lib()  # fail loudly when the kernels are not built
    return True


@torch.no_grad()
def build_summary(keys: torch.Tensor, values: torch.Tensor,
                  config: RefineKVConfig | None = None) -> BlockSummary:
    """Summaries of (kv_heads, tokens, head_dim) prompt keys/values."""
    config = config or RefineKVConfig()
    if keys.ndim != 3 or keys.shape != values.shape or min(keys.shape) <= 0:
        raise ValueError(
            "keys and values must have the same nonempty (kv_heads, tokens, dim) shape")
    if keys.device != values.device or keys.dtype != values.dtype:
        raise ValueError("keys and values must have the same device and dtype")
    if not keys.is_floating_point():
        raise TypeError("keys and values must be floating point")
    block = config.block_size
    length = keys.shape[1]
    keys, values = keys.detach(), values.detach()
    key_pages, value_pages = _pages(keys, block), _pages(values, block)
    if _use_hip(keys, config):
        from . import _hip

        fields = _hip.summary_fields(keys, values, block)
    else:
        from .reference import summary_fields

        fields = summary_fields(key_pages, value_pages, length, config)
    counts, key_mean, value_mean, ellipsoid, value_norm, max_value_norm = fields
    return BlockSummary(keys=key_pages, values=value_pages, counts=counts, key_mean=key_mean,
                        value_mean=value_mean, ellipsoid=ellipsoid, value_norm=value_norm,
                        max_value_norm=max_value_norm, prompt_length=length, block_size=block)


def store_and_build_summary(keys: torch.Tensor, values: torch.Tensor, cache_keys: torch.Tensor,
                            cache_values: torch.Tensor,
                            config: RefineKVConfig | None = None) -> BlockSummary:
    """Write (kv_heads, tokens, head_dim) prompt keys/values into the KV cache
    views cache_keys / cache_values and return build_summary of the written
    prompt, whose pages view the cache.  With the HIP backend one kernel does
    both from a single read of keys/values (the reference writes the cache,
    then build_summary reads it back, integrations/transformers.py:529-536);
    otherwise a copy, then build_summary."""
    config = config or RefineKVConfig()
    if keys.shape != cache_keys.shape or values.shape != cache_values.shape:
        raise ValueError("cache views must have the keys' and values' shape")
    if _use_hip(keys, config) and cache_keys.stride(-1) == 1 and cache_values.stride(-1) == 1:
        from . import _hip

        if keys.ndim != 3 or keys.shape != values.shape or min(keys.shape) <= 0:
            raise ValueError(
                "keys and values must have the same nonempty (kv_heads, tokens, dim) shape")
        block = config.block_size
        fields = _hip.summary_fields(keys.detach(), values.detach(), block, cache_keys,
                                     cache_values)
        counts, key_mean, value_mean, ellipsoid, value_norm, max_value_norm = fields
        return BlockSummary(keys=_pages(cache_keys, block), values=_pages(cache_values, block),
                            counts=counts, key_mean=key_mean, value_mean=value_mean,
                            ellipsoid=ellipsoid, value_norm=value_norm,
                            max_value_norm=max_value_norm, prompt_length=keys.shape[1],
                            block_size=block)
    cache_keys.copy_(keys)
    cache_values.copy_(values)
    return build_summary(cache_keys, cache_values, config)
