"""Regenerate the inputs of the golden fixtures in tests/golden/*.npz.

Each fixture records its recipe (refinekv.testing generators + seed); the
inputs are rebuilt here from CPU torch.Generator streams and checked against
the sha256 the fixture stores.
"""

import glob
import hashlib
import json
import os

import numpy as np
import torch

from refinekv import testing

GOLDEN_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def fixture_paths():
    return sorted(glob.glob(os.path.join(GOLDEN_DIR, "*.npz")))


def digest(*tensors):
    h = hashlib.sha256()
    for t in tensors:
        h.update(t.detach().contiguous().float().numpy().tobytes())
    return h.hexdigest()


def load(path):
    g = dict(np.load(path))
    meta = json.loads(bytes(g.pop("meta")).decode())
    return g, meta


def regenerate(meta):
    """Returns dict(query, keys, values, suffix_keys, suffix_values, anchor_queries)."""
    r = meta["recipe"]
    anchor_queries = None
    if r["kind"] == "decode_inputs":
        args = {k: v for k, v in r.items() if k not in ("kind", "dtype")}
        inp = testing.decode_inputs(**args)
        dt = torch.float32 if r["dtype"] == "f32" else torch.bfloat16
        q, k, v = inp["query"].to(dt), inp["prompt_keys"].to(dt), inp["prompt_values"].to(dt)
        sk, sv = inp["suffix_keys"].to(dt), inp["suffix_values"].to(dt)
        anchor_queries = inp["anchor_queries"].to(dt)
    elif r["kind"] == "wide_inputs":
        q, k, v = testing.wide_inputs(length=r["length"], dim=r["dim"], seed=r["seed"])
        sk, sv = k[:, :3], v[:, :3]
    else:
        q, k, v = testing.small_inputs(length=r["length"], dim=r["dim"], seed=r["seed"])
        if "query_scale" in r:
            q = (q.float() * r["query_scale"]).to(torch.bfloat16)
            sk, sv = k[:, :0], v[:, :0]
        elif "constant_axes" in r:
            k[..., :3] = torch.tensor(r["constant_axes"], dtype=torch.bfloat16)
            sk, sv = k[:, :2], v[:, :2]
        else:
            sk, sv = k[:, :5], v[:, :5]
    return dict(query=q, keys=k, values=v, suffix_keys=sk, suffix_values=sv,
                anchor_queries=anchor_queries)


def bf16_bits(t):
    return t.to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)


def padded_pages(t, block):
    """(H, L, D) -> (H, N*B, D) zero-padded, as summary.py's _pages does."""
    H, L, D = t.shape
    pad = (-L) % block
    if pad:
        t = torch.cat([t, t.new_zeros(H, pad, D)], 1)
    return t
