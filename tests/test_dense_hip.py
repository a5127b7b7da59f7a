"""rkv_dense_decode (the dense decode kernel) against the CPU oracle (GPU).

Bar: outputs within the attention tolerance used for the sparse path
(max-abs 2e-2, mean-rel 1e-3) of orc_dense_attention, which is exact to fp64
over the same bf16 inputs; repeated calls bit for bit; a graph replay with a
device length equal to eager calls at each length.  Shapes cover the
configs' head layouts (Llama 8 x 4, Qwen 4 x 7), groups up to 16, every
head_dim 32..160, ragged lengths, one token, and a strided cache view whose
capacity exceeds the attended length.
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
MAX_ABS, MEAN_REL = 2e-2, 1e-3


@pytest.fixture(scope="module")
def hip():
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    from refinekv import _hip

    _hip.lib()  # the HIP library must load: no fallback
    return _hip


def assert_close_output(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    assert err.max() <= MAX_ABS, f"max-abs {err.max():.3e}"
    assert err.mean() <= MEAN_REL * np.abs(want).mean() + 1e-6, f"mean-abs {err.mean():.3e}"


def _inputs(H, G, D, L, seed, cap=None, spikes=0.0):
    gen = torch.Generator().manual_seed(seed)
    cap = cap or L
    q = torch.randn(H, G, D, generator=gen).to(torch.bfloat16)
    k = torch.randn(1, H, cap, D, generator=gen)
    if spikes:
        # a few tokens aligned with the queries, so the softmax is peaked
        hot = torch.rand(H, cap, generator=gen) < spikes
        k[0][hot] += 3.0 * q.float().mean(1, keepdim=True).expand(H, cap, D)[hot]
    v = torch.randn(1, H, cap, D, generator=gen)
    return q, k.to(torch.bfloat16), v.to(torch.bfloat16)


def _oracle(oracle_lib, q, k, v, L):
    """The oracle's output in the query dtype (bf16), as SDPA returns it."""
    bits = lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    out = oracle_lib.dense_attention(q.float().numpy(), bits(k[0, :, :L]), bits(v[0, :, :L]))
    return torch.from_numpy(out).to(torch.bfloat16).float().numpy()


@pytest.mark.parametrize("H,G,D,L", [
    (8, 4, 128, 4096), (4, 7, 128, 3000), (2, 16, 64, 999), (1, 1, 32, 17), (3, 5, 160, 1000),
    (2, 8, 96, 64), (1, 3, 128, 1), (2, 12, 128, 2049)])
def test_dense_matches_oracle(hip, oracle_lib, H, G, D, L):
    q, k, v = _inputs(H, G, D, L, seed=H * 100 + L, spikes=0.01)
    out = hip.dense_decode(q.to(DEV), k[0].to(DEV), v[0].to(DEV))
    torch.cuda.synchronize()
    assert out.shape == (H, G, D) and out.dtype == torch.bfloat16
    assert_close_output(out.float().cpu().numpy(), _oracle(oracle_lib, q, k, v, L))


def test_dense_on_a_cache_view_longer_than_the_length(hip, oracle_lib):
    """A (1, H, capacity, D) cache of which the first L tokens are valid: the
    stale tail is never read into the result."""
    H, G, D, cap, L = 4, 4, 128, 5000, 3333
    q, k, v = _inputs(H, G, D, L, seed=5, cap=cap)
    k[0, :, L:] = 1e4  # would dominate if it were attended
    kd, vd = k.to(DEV), v.to(DEV)
    out = hip.dense_decode(q.to(DEV), kd[0], vd[0], length=L)
    torch.cuda.synchronize()
    assert_close_output(out.float().cpu().numpy(), _oracle(oracle_lib, q, k, v, L))


def test_dense_repeats_bit_for_bit(hip):
    q, k, v = _inputs(8, 4, 128, 8192, seed=11)
    qd, kd, vd = q.to(DEV), k[0].to(DEV), v[0].to(DEV)
    ws = {}
    outs = [hip.dense_decode(qd, kd, vd, workspace=ws).clone() for _ in range(3)]
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[1], outs[2])


def test_dense_graph_replay_with_a_device_length(hip, oracle_lib):
    """Captured once with a device length; each replay at a new length equals
    the eager call at that length and the oracle."""
    H, G, D, cap = 8, 4, 128, 2048
    q, k, v = _inputs(H, G, D, cap, seed=21, cap=cap)
    qd, kd, vd = q.to(DEV), k[0].to(DEV), v[0].to(DEV)
    length = torch.tensor(1000, dtype=torch.int32, device=DEV)
    ws = {}
    out = torch.empty(H, G, D, dtype=torch.bfloat16, device=DEV)
    hip.dense_decode(qd, kd, vd, length=length, workspace=ws, output=out)  # sizes the workspace
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        hip.dense_decode(qd, kd, vd, length=length, workspace=ws, output=out)
    for n in (1000, 1, 1777, 2048, 999):
        length.fill_(n)
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        eager = hip.dense_decode(qd, kd, vd, length=torch.tensor(n, dtype=torch.int32,
                                                                 device=DEV))
        torch.cuda.synchronize()
        assert torch.equal(got, eager), n
        assert_close_output(got.float().cpu().numpy(), _oracle(oracle_lib, q, k, v, n))


def test_dense_headline_shape_matches_oracle(hip, oracle_lib):
    """The headline decode's head layout at its full 131072-token context."""
    H, G, D, L = 8, 4, 128, 131072
    q, k, v = _inputs(H, G, D, L, seed=1, spikes=0.001)
    out = hip.dense_decode(q.to(DEV), k[0].to(DEV), v[0].to(DEV))
    torch.cuda.synchronize()
    assert_close_output(out.float().cpu().numpy(), _oracle(oracle_lib, q, k, v, L))


def test_dense_rejects_what_it_does_not_run(hip):
    q, k, v = _inputs(2, 4, 256, 64, seed=0)
    with pytest.raises(TypeError):
        hip.dense_decode(q.to(DEV), k[0].to(DEV), v[0].to(DEV))  # head_dim 256
    q, k, v = _inputs(2, 4, 64, 64, seed=0)
    with pytest.raises(TypeError):
        hip.dense_decode(q.half().to(DEV), k[0].half().to(DEV), v[0].half().to(DEV))
    with pytest.raises(ValueError):
        hip.dense_decode(q.to(DEV), k[0].to(DEV), v[0].to(DEV), length=65)
