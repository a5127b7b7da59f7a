"""rkv_decode_static (no workspace, the library's own device scratch) against
rkv_decode on the same inputs: bit-identical outputs, masks and access
counts, for two calls in a row on one stream, the second with a smaller
shape (different layout of the shared scratch), and again in the reverse
order; a shape whose workspace exceeds the scratch is refused before any
launch; a static call whose hand-off waits give up (forced from the host,
every kernel still ends) reports it in its own status word, which the next
call does not clear, and in-band: NaN output rows, every block expanded."""

import numpy as np
import pytest
import torch

from refinekv import RefineKVConfig, build_summary, testing

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")

# (heads, group, dim, block, prompt, reduction, eps, suffix): the first takes
# the one-launch step, the second is smaller; the third takes the three kernels
SHAPES = [(8, 4, 128, 32, 16384, "any", 0.01, 9), (2, 7, 64, 64, 3000, "max", 0.005, 4),
          (1, 4, 128, 16, 140000, "mean", 0.02, 5)]


@pytest.fixture(scope="module")
def hip():
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    from refinekv import _hip

    _hip.lib()
    return _hip


def _case(shape, seed):
    heads, group, dim, block, prompt, reduction, eps, suffix = shape
    inp = testing.decode_inputs(heads=heads, group=group, dim=dim, prompt=prompt, suffix=suffix,
                                block=block, spike_fraction=0.03, anchors=1, seed=seed)
    inp = {k: (v.to(torch.bfloat16).to(DEV) if v.is_floating_point() else v)
           for k, v in inp.items()}
    cfg = RefineKVConfig(backend="hip", block_size=block, eps=eps, gqa_reduction=reduction)
    summary = build_summary(inp["prompt_keys"], inp["prompt_values"], cfg)
    anchor = torch.zeros(heads, summary.num_blocks, dtype=torch.bool, device=DEV)
    anchor[:, 0] = True
    return inp, cfg, summary, anchor


def _both(hip, shape, seed):
    inp, cfg, summary, anchor = _case(shape, seed)
    length = torch.tensor(inp["suffix_keys"].shape[1] - 1, dtype=torch.int32, device=DEV)
    args = (inp["query"], summary, inp["suffix_keys"], inp["suffix_values"], cfg)
    count_ref = torch.zeros(1, dtype=torch.int64, device=DEV)
    out_ref, mask_ref = hip.decode(*args, anchor, {}, length, count_ref)
    out_ref, mask_ref = out_ref.clone(), mask_ref.clone()
    out = torch.empty_like(out_ref)
    mask = torch.empty_like(mask_ref)
    count = torch.zeros(1, dtype=torch.int64, device=DEV)
    hip.decode_static(*args, out, mask, anchor, length, count)
    torch.cuda.synchronize()
    assert torch.equal(mask, mask_ref), shape
    assert torch.equal(out.view(torch.int16), out_ref.view(torch.int16)), shape
    assert int(count.item()) == int(count_ref.item()) > 0, shape
    return mask


@pytest.mark.parametrize("order", [(0, 1, 2), (2, 1, 0)])
def test_static_scratch_decode_equals_workspace_decode(hip, order):
    for i, index in enumerate(order):
        mask = _both(hip, SHAPES[index], seed=40 + i)
        assert 0 < mask.float().mean().item() < 1


def test_static_scratch_rejects_oversized_shapes(hip):
    heads, group, dim = 64, 16, 128
    n_blocks = 1 << 16
    assert hip.workspace_bytes(heads, group, dim, n_blocks) > 64 << 20
    q = torch.zeros(heads * group * dim, dtype=torch.bfloat16, device=DEV)
    rc = hip.lib().rkv_decode_static(
        q.data_ptr(), q.data_ptr(), q.data_ptr(), q.data_ptr(), q.data_ptr(), q.data_ptr(),
        q.data_ptr(), 0, q.data_ptr(), 0, None, 0, 0, None, 0, 0, 0, None, heads, group, dim,
        n_blocks, 32, n_blocks * 32, 0.01, 2, None, q.data_ptr(), q.data_ptr(), None,
        torch.cuda.current_stream().cuda_stream)
    assert rc == 4
    assert b"rkv_decode_static" in hip.lib().rkv_last_error()


def test_static_scratch_give_up_is_reported(hip):
    """rkv_set_handoff_test(64, 1): every wait of the static call's one-launch
    step accepts no data and gives up after 64 polls.  The static status
    word reports it (and keeps it across the next call, whose fill kernels
    clear only the shape's counters and slots), the output rows are NaN and
    the mask is all-expanded; after clearing, a call matches rkv_decode."""
    shape = SHAPES[0]
    assert hip.decode_plan(8, 4, 128, 16384 // 32, 32) == "step"
    inp, cfg, summary, anchor = _case(shape, seed=50)
    args = (inp["query"], summary, inp["suffix_keys"], inp["suffix_values"], cfg)
    hip.static_status(clear=True)
    assert hip.static_status() == 0
    out = torch.empty(8, 4, 1, 128, dtype=torch.bfloat16, device=DEV)
    mask = torch.empty(8, summary.num_blocks, dtype=torch.bool, device=DEV)
    hip.set_handoff_test(64, 1)
    try:
        hip.decode_static(*args, out, mask, anchor)
        torch.cuda.synchronize()
    finally:
        hip.set_handoff_test(0, 0)
    assert torch.isnan(out.float()).all()
    assert mask.all()
    assert hip.static_status() & 1
    # a clean call afterwards: correct again, and the word still reports the
    # earlier give-up until it is cleared
    _both(hip, shape, seed=51)
    assert hip.static_status(clear=True) & 1
    assert hip.static_status() == 0
    _both(hip, shape, seed=52)
    assert hip.static_status() == 0


def test_static_scratch_checks_caller_buffers(hip):
    inp, cfg, summary, anchor = _case(SHAPES[1], seed=53)
    args = (inp["query"], summary, inp["suffix_keys"], inp["suffix_values"], cfg)
    good_out = torch.empty(2, 7, 1, 64, dtype=torch.bfloat16, device=DEV)
    good_mask = torch.empty(2, summary.num_blocks, dtype=torch.bool, device=DEV)
    for out, mask in ((good_out[:1], good_mask), (good_out, good_mask[:, :-1]),
                      (good_out.float(), good_mask), (good_out, good_mask.to(torch.uint8)),
                      (torch.empty(2, 7, 1, 128, dtype=torch.bfloat16, device=DEV)[..., ::2],
                       good_mask)):
        with pytest.raises(ValueError, match="rkv_decode_static"):
            hip.decode_static(*args, out, mask, anchor)
