"""Validated RefineKV settings (mirror of src/refinekv/config.py:7-38).

The only change from the reference is the backend set: ``"hip"`` joins it,
and ``"triton"`` (the reference's accelerated backend) is accepted as another
name for it, so configurations written for the reference keep working.
``"auto"`` picks the HIP kernels for bf16 queries on a ROCm device and the
torch implementation for CPU tensors.
"""

from dataclasses import dataclass
import math

BACKENDS = ("auto", "torch", "hip", "triton")
KERNEL_BACKENDS = ("hip", "triton")  # explicit requests for the gfx950 kernels
REDUCTIONS = ("mean", "max", "any")


@dataclass(frozen=True)
class RefineKVConfig:
    """Diagonal-ellipsoid block selection and sparse decode settings.

    ``eps`` is the risk threshold (the paper's tau), not a token budget.
    ``gqa_reduction`` combines the per-query-head risks of one KV head:
    ``any`` expands a block when any head's risk exceeds ``eps``, ``max``
    compares the largest risk and ``mean`` the group mean.  ``anchor_tokens``
    unions the selections of the last N prompt queries into every decode step.
    """

    block_size: int = 32
    eps: float = 0.01
    gqa_reduction: str = "any"
    anchor_tokens: int = 0
    full_attention_layers: int = 0
    backend: str = "auto"
    summary_chunk_blocks: int = 512
    collect_stats: bool = False

    def __post_init__(self):
        if self.block_size not in (16, 32, 64):
            raise ValueError("block_size must be 16, 32, or 64")
        if not math.isfinite(self.eps) or self.eps < 0:
            raise ValueError("eps must be finite and nonnegative")
        if self.gqa_reduction not in REDUCTIONS:
            raise ValueError("gqa_reduction must be 'mean', 'max', or 'any'")
        if self.backend not in BACKENDS:
            raise ValueError("backend must be 'auto', 'torch', 'hip', or 'triton'")
        for name in ("anchor_tokens", "full_attention_layers"):
            value = getattr(self, name)
            if not isinstance(value, int) or isinstance(value, bool) or value < 0:
                raise ValueError(f"{name} must be a nonnegative integer")
        chunk = self.summary_chunk_blocks
        if not isinstance(chunk, int) or isinstance(chunk, bool) or chunk <= 0:
            raise ValueError("summary_chunk_blocks must be a positive integer")
