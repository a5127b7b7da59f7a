"""torch restatement of the reference's CPU path (``backend="torch"``).

Follows src/refinekv/summary.py:46-113 and src/refinekv/reference.py:10-73
operation by operation, so on the same torch build it returns the same bits
as the reference.  It serves CPU tensors and explicit ``backend="torch"``;
ROCm tensors use the HIP kernels.
"""

import math

import torch


def summary_fields(key_pages, value_pages, length, config):
    block = config.block_size
    n_blocks = key_pages.shape[1]
    counts = torch.full((n_blocks,), block, device=key_pages.device, dtype=torch.int64)
    last = length - (n_blocks - 1) * block
    counts[-1] = last
    sizes = counts.float()[None, :, None]
    key_mean = (key_pages.sum(2, dtype=torch.float32) / sizes).to(torch.bfloat16)
    value_mean = (value_pages.sum(2, dtype=torch.float32) / sizes).to(torch.bfloat16)
    hi, lo = key_pages.amax(2), key_pages.amin(2)
    if last < block:
        tail = key_pages[:, -1, :last]
        hi[:, -1], lo[:, -1] = tail.amax(1), tail.amin(1)
    mean32 = key_mean.float()
    width = torch.maximum(hi.float() - mean32, mean32 - lo.float())
    width2 = width.clamp_min(1e-6).square().to(torch.bfloat16)
    ellipsoid = torch.empty_like(width2)
    step = config.summary_chunk_blocks
    for start in range(0, n_blocks, step):
        end = min(start + step, n_blocks)
        # A copy: .float() of an fp32 cache would alias it.
        c = key_pages[:, start:end].to(dtype=torch.float32, copy=True)
        c.sub_(key_mean[:, start:end].float().unsqueeze(2))
        c.mul_(torch.rsqrt(width2[:, start:end].float()).unsqueeze(2))
        c.square_()
        dist = c.sum(-1)
        if end == n_blocks and last < block:
            dist[:, -1, last:] = -torch.inf
        r2 = dist.amax(-1).clamp_min(0).sqrt().square()
        ellipsoid[:, start:end] = (r2.unsqueeze(-1) * width2[:, start:end].float()
                                   * (1 + 2 ** -8)).to(torch.bfloat16)
    norms = torch.linalg.vector_norm(value_pages, dim=-1, dtype=torch.float32)
    if last < block:
        norms[:, -1, last:] = -torch.inf
    value_norm = norms.amax(-1)
    return counts, key_mean, value_mean, ellipsoid, value_norm, value_norm.amax(-1)


def selection_statistics(query, summary):
    """z, risk (H, G, N) and log Z, log C (H, G, 1) (reference.py:10-34)."""
    q = query[:, :, 0].to(torch.bfloat16).float()
    q2 = q.square().to(torch.bfloat16).float()
    scale = q.shape[-1] ** -0.5
    s = torch.einsum("hgd,hbd->hgb", q, summary.key_mean.float()) * scale
    proj = torch.einsum("hgd,hbd->hgb", q2, summary.ellipsoid.float())
    delta = proj.clamp_min(0).sqrt() * scale * (1 + 2 ** -8)
    z = s + summary.counts.float().log()[None, None, :]
    clipped = delta.clamp(max=10)
    small = delta <= 10
    log_cosh = torch.where(small, ((clipped.exp() + (-clipped).exp()) * 0.5).log(),
                           delta + ((1 + (-2 * delta).exp()) * 0.5).log())
    log_z = torch.logsumexp(z, -1, keepdim=True)
    log_c = torch.logsumexp(z + log_cosh, -1, keepdim=True)
    vmax2 = 2 * summary.max_value_norm[:, None, None]
    t = clipped.exp()
    direct = vmax2 * (z - log_c).exp()
    direct = direct * (0.5 * (t + t.reciprocal()) - 1)
    exp_neg = (-delta).exp()
    lcm1 = delta + 2 * (1 - exp_neg).clamp_min(1e-30).log() - math.log(2)
    large = vmax2 * (z - log_c + lcm1).exp()
    tanh_half = torch.where(small, (t - 1) / (t + 1), (1 - exp_neg) / (1 + exp_neg))
    value = 2 * summary.value_norm[:, None] * (z - log_z).exp() * tanh_half
    return z, torch.where(small, direct, large) + value, log_z, log_c


def select_blocks(query, summary, config):
    """(mask (H, N) bool, z) (reference.py:37-47)."""
    z, risk, log_z, log_c = selection_statistics(query, summary)
    if config.gqa_reduction == "mean":
        selected = risk.mean(1) > config.eps
    elif config.gqa_reduction == "max":
        selected = risk.amax(1) > config.eps
    else:
        selected = (risk > config.eps).any(1)
    bad_global = (~torch.isfinite(log_z) | ~torch.isfinite(log_c)).any(1)
    bad_local = (~torch.isfinite(risk)).any(1)
    return selected | bad_global | bad_local, z


@torch.no_grad()
def sparse_attention(query, summary, key_suffix, value_suffix, config, anchor_mask=None):
    """Mixed attention by explicit concatenation (reference.py:50-73)."""
    selected, z = select_blocks(query, summary, config)
    if anchor_mask is not None:
        selected = selected | anchor_mask
    q = query[:, :, 0].to(torch.bfloat16).float()
    scale = q.shape[-1] ** -0.5
    valid = torch.arange(summary.block_size, device=q.device)[None] < summary.counts[:, None]
    outputs = []
    for h in range(q.shape[0]):
        take = selected[h, :, None] & valid
        keys = torch.cat([summary.keys[h][take].to(torch.bfloat16).float(),
                          key_suffix[h].to(torch.bfloat16).float()])
        values = torch.cat([summary.values[h][take].to(torch.bfloat16).float(),
                            value_suffix[h].to(torch.bfloat16).float()])
        logits = torch.cat([z[h, :, ~selected[h]], q[h] @ keys.T * scale], -1)
        values = torch.cat([summary.value_mean[h, ~selected[h]].float(), values], 0)
        outputs.append(logits.softmax(-1) @ values)
    return torch.stack(outputs).unsqueeze(2).to(query.dtype), selected
