"""Single-token decode attention API (mirror of src/refinekv/attention.py:12-134).

``select_blocks`` and ``sparse_attention`` keep the reference's signatures,
validation and error types.  ``backend="hip"`` (or ``"triton"``, the
reference's name for its accelerated backend) runs the gfx950 kernels
through the C ABI; ``"auto"`` picks them for ROCm tensors whose shapes they
support (bf16 query, head_dim 32..256 in steps of 32, GQA group <= 16) and
the torch restatement otherwise.  The decode kernels read bf16 pages and
suffix rows: with another cache dtype "auto" takes the torch path and an
explicit kernel request converts them (the reference's Triton kernel
converts them as it loads, src/refinekv/kernels/attention.py:222-235).  On
a ROCm device "auto" never falls back silently when the library is missing:
it raises.
"""

import dataclasses
from typing import NamedTuple

import torch

from .config import KERNEL_BACKENDS, RefineKVConfig
from .summary import BlockSummary


class AttentionResult(NamedTuple):
    output: torch.Tensor
    selected: torch.Tensor | None


def _backend(query, config):
    """Mirror of attention.py:17-40 with the HIP backend in Triton's place."""
    from . import _hip

    if config.backend == "torch":
        return "torch"
    explicit = config.backend in KERNEL_BACKENDS
    on_rocm = _hip.is_rocm_device(query)
    if explicit and not on_rocm:
        raise RuntimeError("the HIP backend requires a ROCm GPU tensor")
    if not on_rocm:
        return "torch"
    if query.dtype != torch.bfloat16:
        if explicit:
            raise TypeError("the HIP backend requires BF16 queries")
        return "torch"
    dim, group = query.shape[-1], query.shape[1]
    if dim < 32 or dim > 256 or dim % 32 or group > _hip.MAX_GROUP:
        if explicit:
            raise ValueError("HIP requires head_dim in 32..256 (multiple of 32) and GQA group <= 16")
        return "torch"
    _hip.lib()  # raises when the kernels are not built: no silent fallback on a GPU
    return "hip"


def _validate(query, summary, config, anchor_mask=None):
    """Mirror of attention.py:43-59."""
    if query.ndim != 4 or query.shape[2] != 1 or min(query.shape) <= 0:
        raise ValueError("query must have shape (kv_heads, group_size, 1, head_dim)")
    if query.shape[0] != summary.keys.shape[0] or query.shape[-1] != summary.keys.shape[-1]:
        raise ValueError("query heads and dimension must match the summary")
    if query.device != summary.keys.device:
        raise ValueError("query and summary must be on the same device")
    if config.block_size != summary.block_size:
        raise ValueError("config.block_size must match the summary")
    if anchor_mask is not None:
        if anchor_mask.dtype != torch.bool or tuple(anchor_mask.shape) != (
            query.shape[0],
            summary.num_blocks,
        ):
            raise ValueError("anchor_mask must be boolean with shape (kv_heads, blocks)")
        if anchor_mask.device != query.device:
            raise ValueError("anchor_mask must be on the query device")


def _check_hip_summary(summary):
    if summary.key_mean.dtype != torch.bfloat16 or summary.ellipsoid.dtype != torch.bfloat16:
        raise TypeError("the HIP kernels need bf16 summaries (build_summary's format)")


def _page_identity(t):
    return (t.data_ptr(), t._version, t.dtype, tuple(t.shape), tuple(t.stride()))


def _bf16_pages(summary, workspace=None):
    """The summary with bf16 page views: the pages themselves, or a converted
    copy when the cache holds another dtype.  With a workspace the copy is
    made once and kept there, keyed by the page tensors' storage, version
    and layout (a write to the cache bumps the version and converts again),
    so a decode step does not move the whole prompt's K/V through a
    conversion (the reference converts only the pages it loads,
    kernels/attention.py:222-235)."""
    if summary.keys.dtype == torch.bfloat16 and summary.values.dtype == torch.bfloat16:
        return summary
    key = (_page_identity(summary.keys), _page_identity(summary.values))
    cached = workspace.get("hip_bf16_pages") if workspace is not None else None
    if cached is not None and cached[0] == key:
        keys, values = cached[1]
    else:
        keys, values = summary.keys.to(torch.bfloat16), summary.values.to(torch.bfloat16)
        if workspace is not None:
            workspace["hip_bf16_pages"] = (key, (keys, values))
    return dataclasses.replace(summary, keys=keys, values=values)


@torch.no_grad()
def select_blocks(query, summary, config=None, *, workspace=None):
    """Boolean (kv_heads, blocks) mask of expanded blocks for one query."""
    config = config or RefineKVConfig(block_size=summary.block_size)
    _validate(query, summary, config)
    if _backend(query, config) == "hip":
        from . import _hip

        _check_hip_summary(summary)
        return _hip.select(query, summary, config, workspace)
    from .reference import select_blocks as select_torch

    return select_torch(query, summary, config)[0]


@torch.no_grad()
def select_blocks_union(queries, summary, config=None, *, workspace=None):
    """Union of the (kv_heads, blocks) masks of several queries, (kv_heads,
    group_size, count, head_dim) -- the prompt-anchor mask.  The reference
    builds it with one select_blocks call per anchor query
    (integrations/transformers.py:539-552); the HIP backend scores all of them
    in one launch and ORs the decisions on the device."""
    config = config or RefineKVConfig(block_size=summary.block_size)
    if queries.ndim != 4 or min(queries.shape) <= 0:
        raise ValueError("queries must have shape (kv_heads, group_size, count, head_dim)")
    _validate(queries[:, :, :1], summary, config)
    if _backend(queries[:, :, :1], config) == "hip":
        from . import _hip

        _check_hip_summary(summary)
        return _hip.select_anchors(queries, summary, config, workspace)
    from .reference import select_blocks as select_torch

    union = None
    for position in range(queries.shape[2]):
        selected = select_torch(queries[:, :, position:position + 1], summary, config)[0]
        union = selected if union is None else union | selected
    return union


@torch.no_grad()
def sparse_attention(
    query: torch.Tensor,
    summary: BlockSummary,
    key_suffix: torch.Tensor,
    value_suffix: torch.Tensor,
    config: RefineKVConfig | None = None,
    *,
    anchor_mask: torch.Tensor | None = None,
    workspace: dict | None = None,
    return_selected: bool = False,
    suffix_length: torch.Tensor | None = None,
    access_counter: torch.Tensor | None = None,
) -> AttentionResult:
    """Attend to representatives, expanded prompt blocks and the exact suffix.

    ``query`` is (kv_heads, group_size, 1, head_dim); suffix K/V are
    (kv_heads, suffix_tokens, head_dim) and hold only visible tokens.
    ``suffix_length`` (a device int32 scalar) gives the valid prefix of a
    fixed-capacity suffix buffer, for HIP graph replay.  HIP outputs live in
    the workspace and are overwritten by the next call that reuses it; clone
    them to keep them longer.

    ``access_counter`` (no reference counterpart): an int64 scalar on the
    query device to which the call adds the block term of the access counter,
    the sum over (KV head, block) of the block's token count if it expanded
    and 1 otherwise (src/refinekv/integrations/transformers.py:590-594
    computes it from the mask); the HIP kernels add it in-kernel.
    """
    config = config or RefineKVConfig(block_size=summary.block_size)
    _validate(query, summary, config, anchor_mask)
    expected = (query.shape[0], query.shape[-1])
    if key_suffix.ndim != 3 or key_suffix.shape != value_suffix.shape:
        raise ValueError("suffix K/V must have matching (kv_heads, tokens, head_dim) shapes")
    if (key_suffix.shape[0], key_suffix.shape[-1]) != expected:
        raise ValueError("suffix heads and dimension must match the query")
    if key_suffix.device != query.device or value_suffix.device != query.device:
        raise ValueError("suffix K/V must be on the query device")
    backend = _backend(query, config)
    pages_bf16 = (summary.keys.dtype == torch.bfloat16 and summary.values.dtype == torch.bfloat16
                  and key_suffix.dtype == torch.bfloat16 and value_suffix.dtype == torch.bfloat16)
    if backend == "hip" and not pages_bf16 and config.backend not in KERNEL_BACKENDS:
        backend = "torch"  # "auto": the kernels read bf16 pages
    if access_counter is not None and (access_counter.shape != ()
                                       or access_counter.dtype != torch.int64
                                       or access_counter.device != query.device):
        raise ValueError("access_counter must be a scalar int64 tensor on the query device")
    if suffix_length is not None:
        if (suffix_length.shape != () or suffix_length.device != query.device
                or suffix_length.dtype != torch.int32):
            raise ValueError("suffix_length must be a scalar int32 tensor on the query device")
        if backend != "hip":
            raise ValueError("device-side suffix_length requires the HIP backend")
    if backend == "hip":
        from . import _hip

        _check_hip_summary(summary)
        output, mask = _hip.decode(query, _bf16_pages(summary, workspace),
                                   key_suffix.to(torch.bfloat16),
                                   value_suffix.to(torch.bfloat16), config, anchor_mask,
                                   workspace, suffix_length, access_counter)
        return AttentionResult(output, mask if return_selected else None)
    from .reference import sparse_attention as attention_torch

    output, selected = attention_torch(query, summary, key_suffix, value_suffix, config,
                                       anchor_mask)
    if access_counter is not None:
        access_counter += (selected * summary.counts).sum() + (~selected).sum()
    return AttentionResult(output, selected if return_selected else None)
