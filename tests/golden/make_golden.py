"""Write golden vectors from the reference's own torch path.

Runs only in the build container, where the reference is mounted read-only
at /root/reference.  It imports the reference package (pure Python + torch)
to record, for seeded inputs, the outputs of
  build_summary                 src/refinekv/summary.py:46-113
  selection_statistics          src/refinekv/reference.py:10-34
  select_blocks_reference       src/refinekv/reference.py:37-47
  sparse_attention_reference    src/refinekv/reference.py:50-73
and the access-counter term of src/refinekv/integrations/transformers.py:590-594.
Inputs are not stored: they are regenerated from the recorded recipe and seed
by refinekv.testing (CPU torch.Generator streams are machine independent); a
sha256 of the regenerated inputs is stored to prove it.  Output: one
compressed .npz per case next to this script.

Usage: python tests/golden/make_golden.py
"""

import hashlib
import importlib.util
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
REFERENCE_SRC = "/root/reference/src"


def _load_testing():
    # This build's recipe module, loaded by path: the package name `refinekv`
    # is taken by the reference inside this script.
    path = os.path.join(REPO, "refinekv-release_amd", "refinekv", "testing.py")
    spec = importlib.util.spec_from_file_location("rkv_testing_recipe", path)
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def digest(*tensors):
    h = hashlib.sha256()
    for t in tensors:
        h.update(t.detach().contiguous().float().numpy().tobytes())
    return h.hexdigest()


def record(ref, name, recipe, query, keys, values, suffix_k, suffix_v, cfg_kwargs,
           anchor_queries=None, anchor_last=False):
    config = ref.RefineKVConfig(backend="torch", **cfg_kwargs)
    summary = ref.build_summary(keys, values, config)
    z, risk, log_z, log_c = ref.reference.selection_statistics(query, summary)
    mask, _ = ref.reference.select_blocks_reference(query, summary, config)
    anchor = None
    if anchor_queries is not None:
        for a in range(anchor_queries.shape[2]):
            sel = ref.select_blocks(anchor_queries[:, :, a:a + 1], summary, config)
            anchor = sel if anchor is None else anchor | sel
    elif anchor_last:
        anchor = torch.zeros(keys.shape[0], summary.num_blocks, dtype=torch.bool)
        anchor[:, -1] = True
    result = ref.sparse_attention(query, summary, suffix_k, suffix_v, config,
                                  anchor_mask=anchor, return_selected=True)
    selected = result.selected
    groups = query.shape[1]
    accessed_blocks = int((selected * summary.counts).sum() + (~selected).sum())
    accessed = accessed_blocks * groups + query.shape[0] * groups * suffix_k.shape[1]
    out = dict(
        counts=summary.counts.numpy(),
        key_mean=_bits(summary.key_mean),
        value_mean=_bits(summary.value_mean),
        ellipsoid=_bits(summary.ellipsoid),
        value_norm=summary.value_norm.numpy(),
        max_value_norm=summary.max_value_norm.numpy(),
        z=z.numpy(),
        risk=risk.numpy(),
        log_z=log_z[..., 0].numpy(),
        log_c=log_c[..., 0].numpy(),
        mask=mask.numpy().astype(np.uint8),
        selected=selected.numpy().astype(np.uint8),
        output=result.output.float().numpy(),
        accessed_blocks=np.int64(accessed_blocks),
        accessed=np.int64(accessed),
    )
    if anchor is not None:
        out["anchor"] = anchor.numpy().astype(np.uint8)
    meta = dict(recipe=recipe, config=cfg_kwargs, torch=torch.__version__,
                input_sha256=digest(query, keys, values, suffix_k, suffix_v),
                cpu_capability=torch.backends.cpu.get_cpu_capability())
    out["meta"] = np.frombuffer(json.dumps(meta).encode(), dtype=np.uint8)
    path = os.path.join(HERE, f"{name}.npz")
    np.savez_compressed(path, **out)
    print(f"{name}: {os.path.getsize(path) / 1024:.0f} KiB, expanded "
          f"{selected.float().mean().item():.3f}, accessed {accessed}")


def main():
    sys.path.insert(0, REFERENCE_SRC)
    import refinekv as ref  # the reference package
    import refinekv.reference  # noqa: F401

    testing = _load_testing()
    torch.set_num_threads(1)

    # the CPU fp32 op, and the same tensors in bf16.
    recipe = dict(kind="decode_inputs", seed=0, heads=8, group=4, dim=128, prompt=4096,
                  suffix=16, block=32, spike_fraction=0.02, anchors=32)
    args = {k: v for k, v in recipe.items() if k != "kind"}
    inp = testing.decode_inputs(**args)
    cfg = dict(block_size=32, eps=0.01, gqa_reduction="any", anchor_tokens=32)
    for dtype, tag in ((torch.float32, "f32"), (torch.bfloat16, "bf16")):
        record(ref, f"config1_{tag}", dict(recipe, dtype=tag), inp["query"].to(dtype),
               inp["prompt_keys"].to(dtype), inp["prompt_values"].to(dtype),
               inp["suffix_keys"].to(dtype), inp["suffix_values"].to(dtype), cfg,
               anchor_queries=inp["anchor_queries"].to(dtype))

    # The reference's own Triton-parity shapes (tests/test_attention.py:139-183)
    # plus head_dim 32/96 and more partial blocks, each with an anchor on the
    # last block and a 5-token suffix.
    cases = [
        (16, "any", 0.0, 71, 64),
        (32, "mean", 0.1, 71, 128),
        (64, "max", 1e6, 71, 64),
        (16, "any", 0.2, 25001, 128),
        (32, "any", 0.01, 1000, 32),
        (64, "mean", 0.05, 3001, 96),
        (32, "max", 0.02, 4099, 128),
    ]
    for block, reduction, eps, length, dim in cases:
        q, k, v = testing.small_inputs(length=length, dim=dim)
        recipe = dict(kind="small_inputs", length=length, dim=dim, seed=42, dtype="bf16")
        name = f"small_b{block}_{reduction}_L{length}_d{dim}"
        record(ref, name, recipe, q, k, v, k[:, :5], v[:, :5],
               dict(block_size=block, eps=eps, gqa_reduction=reduction), anchor_last=True)

    # fp32 with a wide dynamic range: the summary's sums are inexact, so these
    # pin the summation orders for every head_dim / block family.
    for block, dim, length in ((16, 32, 517), (64, 96, 1000), (32, 128, 999), (32, 64, 640)):
        q, k, v = testing.wide_inputs(length=length, dim=dim)
        recipe = dict(kind="wide_inputs", length=length, dim=dim, seed=7, dtype="f32")
        record(ref, f"wide_f32_b{block}_L{length}_d{dim}", recipe, q, k, v, k[:, :3], v[:, :3],
               dict(block_size=block, eps=0.01, gqa_reduction="max"))

    # Large delta (tests/test_attention.py:119-128): q x 200.
    q, k, v = testing.small_inputs(length=71, dim=64)
    q = (q.float() * 200).to(torch.bfloat16)
    record(ref, "edge_large_delta", dict(kind="small_inputs", length=71, dim=64, seed=42,
                                         dtype="bf16", query_scale=200.0),
           q, k, v, k[:, :0], v[:, :0], dict(block_size=32, eps=0.01, gqa_reduction="any"))
    # Constant axes (tests/test_attention.py:59-71).
    q, k, v = testing.small_inputs(length=65, dim=128)
    k[..., :3] = torch.tensor([96, 48, -80], dtype=torch.bfloat16)
    record(ref, "edge_constant_axes", dict(kind="small_inputs", length=65, dim=128, seed=42,
                                           dtype="bf16", constant_axes=[96, 48, -80]),
           q, k, v, k[:, :2], v[:, :2], dict(block_size=32, eps=0.01, gqa_reduction="mean"))


if __name__ == "__main__":
    main()
