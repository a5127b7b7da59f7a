"""The Transformers adapter (reference tests/test_transformers.py, restated).

CPU tests use tiny random-init Llama / Qwen2 models and the torch backend;
the GPU tests (marked gpu) run the same models in bf16 with backend="hip":
dynamic and static caches give the same tokens, and graph-replayed decode
gives the eager tokens.
"""

import pytest
import torch

transformers = pytest.importorskip("transformers")
from refinekv import RefineKV, RefineKVConfig, make_visible_static_cache  # noqa: E402


def tiny_model(family="llama", device="cpu"):
    torch.manual_seed(9)
    config_cls, model_cls = {
        "llama": (transformers.LlamaConfig, transformers.LlamaForCausalLM),
        "qwen2": (transformers.Qwen2Config, transformers.Qwen2ForCausalLM),
    }[family]
    config = config_cls(vocab_size=64, hidden_size=128, intermediate_size=256,
                        num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                        pad_token_id=0, eos_token_id=None)
    model = model_cls(config).eval().to(device)
    return model.to(torch.bfloat16) if device == "cuda" else model


def generate(model, length=39, static=False, **extra):
    ids = torch.arange(length, device=model.device)[None] % 61 + 3
    options = {"cache_implementation": "static"} if static else {}
    options.update(extra)
    return model.generate(input_ids=ids, attention_mask=torch.ones_like(ids), max_new_tokens=4,
                          do_sample=False, **options)


def assert_released(model, session, implementation, hooks):
    assert model.config._attn_implementation == implementation
    assert hooks == (len(model._forward_pre_hooks), len(model._forward_hooks))
    assert not session._layers
    assert not hasattr(model, "_refinekv_session")
    assert all(not hasattr(m.self_attn, "_refinekv_session") for m in model.model.layers)
    assert "generate" not in model.__dict__


@pytest.mark.parametrize("family", ["llama", "qwen2"])
@pytest.mark.parametrize("static", [False, True])
def test_generation_with_anchors_and_request_reset(family, static):
    model = tiny_model(family)
    implementation = model.config._attn_implementation
    hooks = len(model._forward_pre_hooks), len(model._forward_hooks)
    config = RefineKVConfig(backend="torch", anchor_tokens=3, eps=1e6, collect_stats=True)
    with RefineKV(model, config) as session:
        out = generate(model, static=static)
        assert out.shape == (1, 43)
        if static:
            assert type(session._cache.layers[0]).__name__ == "_VisibleStaticLayer"
        stats = session.stats
        assert 0 < stats["equivalent_access_ratio"] <= 1
        assert stats["decode_attention_calls"] == 6  # 3 decode forwards x 2 layers
        assert all(s.anchor_mask is not None for s in session._layers.values())
        # a new generation in the same context rebuilds every layer's prompt state
        shorter = generate(model, length=17, static=static)
        assert shorter.shape == (1, 21)
        assert session.stats["decode_attention_calls"] == 6
        assert all(s.prompt_length == 17 for s in session._layers.values())
    assert_released(model, session, implementation, hooks)


def test_access_counter_closed_form():
    """accessed = sum over decode calls of G * (sum_b sel_b * count_b + #unselected)
    + H_q * suffix; dense = H_q * visible (transformers.py:590-594)."""
    model = tiny_model()
    with RefineKV(model, RefineKVConfig(backend="torch", eps=1e6, collect_stats=True)) as s:
        generate(model, length=39)
        stats = s.stats
    # eps 1e6 expands nothing: per head 2 representatives (39 tokens, block 32)
    q_heads, groups, layers = 4, 2, 2
    accessed = dense = 0
    for step in range(1, 4):  # 3 decode forwards; suffix holds `step` tokens
        visible = 39 + step
        accessed += layers * (2 * 2 * groups + q_heads * step)
        dense += layers * q_heads * visible
    assert stats["accessed"] == accessed and stats["dense"] == dense


def test_generation_config_static_uses_visible_cache():
    model = tiny_model()
    model.generation_config.cache_implementation = "static"
    with RefineKV(model, RefineKVConfig(backend="torch")) as session:
        assert generate(model).shape == (1, 43)
        assert type(session._cache.layers[0]).__name__ == "_VisibleStaticLayer"


def test_visible_cache_exposes_written_prefix():
    model = tiny_model()
    cache = make_visible_static_cache(model, 8)
    layer = cache.layers[0]
    k = torch.randn(1, 2, 3, 32)
    keys, values = layer.update(k, k + 1)
    assert keys.shape[2] == 3 and layer.get_seq_length() == 3
    assert layer.get_mask_sizes(1) == (4, 0)
    keys, _ = layer.update(k[:, :, :1], k[:, :, :1])
    assert keys.shape[2] == 4 and torch.equal(keys[:, :, :3], k)
    with pytest.raises(ValueError, match="capacity"):
        layer.update(torch.randn(1, 2, 5, 32), torch.randn(1, 2, 5, 32))
    with pytest.raises(ValueError, match="positive"):
        make_visible_static_cache(model, 0)


def test_stock_static_cache_is_rejected():
    model = tiny_model()
    ids = torch.arange(39)[None] % 61 + 3
    cache = transformers.StaticCache(config=model.config, max_cache_len=43)
    with RefineKV(model):
        with pytest.raises(ValueError, match="stock StaticCache is unsupported"):
            model.generate(input_ids=ids, max_new_tokens=4, past_key_values=cache)


def test_dense_layers_match_native_generation_and_leave_other_models_alone():
    model, other = tiny_model(), tiny_model()
    with torch.inference_mode():
        expected = generate(model)
    other_implementation = other.config._attn_implementation
    with RefineKV(model, RefineKVConfig(full_attention_layers=2, collect_stats=True)) as s:
        actual = generate(model)
        assert other.config._attn_implementation == other_implementation
    assert torch.equal(actual, expected)
    assert s.stats["equivalent_access_ratio"] == 1


def test_errors_restore_the_model():
    model = tiny_model()
    implementation = model.config._attn_implementation
    with pytest.raises(ValueError, match="unpadded"):
        with RefineKV(model):
            with pytest.raises(RuntimeError, match="active"):
                with RefineKV(model):
                    pass
            model.generate(input_ids=torch.tensor([[0, 3, 4]]),
                           attention_mask=torch.tensor([[0, 1, 1]]), max_new_tokens=2)
    assert model.config._attn_implementation == implementation
    assert not hasattr(model, "_refinekv_session")
    with pytest.raises(ValueError, match="inference-only"):
        with RefineKV(model.train()):
            pass
    model.eval()
    with pytest.raises(RuntimeError, match="RefineKV context"):
        from refinekv.integrations.transformers import _refinekv_attention

        _refinekv_attention(model.model.layers[0].self_attn, None, None, None, None)


@pytest.mark.parametrize("family", ["llama", "qwen2"])
def test_anchor_queries_come_from_the_tail_projection(family, monkeypatch):
    """A projection of the whole prompt that rounds differently must not
    change the anchors (transformers.py:505-507)."""
    model = tiny_model(family)
    for layer in model.model.layers:
        proj = layer.self_attn.q_proj
        with torch.no_grad():
            proj.weight.zero_()
            if proj.bias is not None:
                proj.bias.zero_()
        original = proj.forward

        def perturbed(hidden, original=original):
            out = original(hidden)
            return out + 1 if hidden.shape[1] > 2 else out

        monkeypatch.setattr(proj, "forward", perturbed)
    with RefineKV(model, RefineKVConfig(backend="torch", eps=0, anchor_tokens=2)) as s:
        generate(model)
        assert all(not st.anchor_mask.any() for st in s._layers.values())


def test_visible_prefix_mask_decides_the_dense_kernel():
    """The dense decode kernel attends tokens [0, visible) and takes no mask,
    so the hook uses it only when the model's mask says exactly that; a
    masked (padded) prompt token, a visible token past the prefix or an
    additive bias sends the call to SDPA with the mask applied."""
    from refinekv.integrations.transformers import RefineKV as Hook, mask_is_visible_prefix

    L, visible = 12, 9
    lo = torch.finfo(torch.bfloat16).min
    prefix = torch.arange(L) < visible
    additive = torch.zeros(1, 1, 1, L, dtype=torch.bfloat16).masked_fill(~prefix, lo)
    assert mask_is_visible_prefix(None, visible, L)
    assert mask_is_visible_prefix(prefix.view(1, 1, 1, L), visible, L)
    assert mask_is_visible_prefix(additive, visible, L)
    assert mask_is_visible_prefix(additive.float().masked_fill(~prefix, float("-inf")), visible, L)
    padded = additive.clone()
    padded[..., 2] = lo
    assert not mask_is_visible_prefix(padded, visible, L)
    assert not mask_is_visible_prefix(prefix.view(1, 1, 1, L) & (torch.arange(L) != 0), visible, L)
    assert not mask_is_visible_prefix(additive.masked_fill(torch.arange(L) == visible, 0), visible,
                                      L)
    assert not mask_is_visible_prefix(additive.masked_fill(torch.arange(L) == 1, -0.5), visible,
                                      L)
    assert not mask_is_visible_prefix(additive[..., :L - 1], visible, L)

    # _dense_decode with a padded prompt token: the kernel is not asked, and
    # SDPA's output ignores the masked token
    model = tiny_model()
    attn = model.model.layers[0].self_attn
    calls = []

    class Self:
        def _hip_dense_decode(self, *args):
            calls.append(args)
            return None

    gen = torch.Generator().manual_seed(4)
    q = torch.randn(1, 4, 1, 32, generator=gen)
    k = torch.randn(1, 2, L, 32, generator=gen)
    v = torch.randn(1, 2, L, 32, generator=gen)
    out, _ = Hook._dense_decode(Self(), attn, q, k, v, padded.float(), 32 ** -0.5, {}, visible, {})
    assert not calls
    v2 = v.clone()
    v2[:, :, 2] += 100.0  # the masked token's value does not reach the output
    out2, _ = Hook._dense_decode(Self(), attn, q, k, v2, padded.float(), 32 ** -0.5, {}, visible,
                                 {})
    assert torch.equal(out, out2)
    Hook._dense_decode(Self(), attn, q, k, v, additive.float(), 32 ** -0.5, {}, visible, {})
    assert len(calls) == 1


def test_graph_mode_preconditions_on_cpu():
    model = tiny_model()
    ids = torch.tensor([[3, 4, 5]])
    with RefineKV(model, RefineKVConfig(backend="torch"), cuda_graph=True):
        with pytest.raises(ValueError, match="fixed output"):
            model.generate(input_ids=ids, max_new_tokens=4)
        with pytest.raises(ValueError, match="GPU BF16 model"):
            model.generate(input_ids=ids, max_new_tokens=4, min_new_tokens=4, eos_token_id=None)
        with pytest.raises(ValueError, match="does not support"):
            model.generate(input_ids=ids, max_new_tokens=4, min_new_tokens=4, eos_token_id=None,
                           top_k=3)


# ---------------------------------------------------------------------------
# GPU: backend="hip"
# ---------------------------------------------------------------------------

def _gpu_or_skip():
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    from refinekv import _hip

    _hip.lib()


@pytest.mark.gpu
@pytest.mark.parametrize("family", ["llama", "qwen2"])
def test_hip_generation_dynamic_equals_static(family):
    _gpu_or_skip()
    model = tiny_model(family, "cuda")
    config = RefineKVConfig(backend="hip", eps=1e6, anchor_tokens=2)
    with RefineKV(model, config):
        dynamic = generate(model)
    with RefineKV(model, config):
        static = generate(model, static=True)
    assert torch.equal(dynamic, static)


@pytest.mark.gpu
@pytest.mark.parametrize("family", ["llama", "qwen2"])
@pytest.mark.parametrize("reduction,anchors", [("mean", 0), ("any", 2)])
def test_hip_graph_decode_matches_eager(family, reduction, anchors):
    _gpu_or_skip()
    model = tiny_model(family, "cuda")
    if family == "qwen2":
        model.generation_config.repetition_penalty = 1.05
    config = RefineKVConfig(backend="hip", eps=0.01, gqa_reduction=reduction,
                            anchor_tokens=anchors)
    requests = []
    for length in (39, 17):
        ids = torch.arange(length, device="cuda")[None] % 61 + 3
        options = dict(input_ids=ids, attention_mask=torch.ones_like(ids), max_new_tokens=8,
                       min_new_tokens=8, eos_token_id=None, forced_eos_token_id=None,
                       do_sample=False)
        with RefineKV(model, config):
            eager = model.generate(**options)
        requests.append((options, eager))
    with RefineKV(model, config, cuda_graph=True):
        for options, eager in requests:
            assert torch.equal(model.generate(**options), eager)


@pytest.mark.gpu
def test_hip_stats_and_dense_layers():
    _gpu_or_skip()
    model = tiny_model("llama", "cuda")
    with RefineKV(model, RefineKVConfig(backend="hip", eps=1e6, collect_stats=True)) as s:
        generate(model)
        stats = s.stats
    assert stats["decode_attention_calls"] == 6 and 0 < stats["equivalent_access_ratio"] < 1
    with RefineKV(model, RefineKVConfig(backend="hip", full_attention_layers=2,
                                        collect_stats=True)) as s:
        generate(model)
        assert s.stats["equivalent_access_ratio"] == 1


@pytest.mark.gpu
def test_hip_dense_layers_run_the_dense_kernel_and_match_the_oracle(monkeypatch, oracle_lib):
    """Dense layers (full_attention_layers) decode through rkv_dense_decode
    over the visible prefix: every call's output against the oracle's dense
    attention of the same query, keys and values."""
    import numpy as np

    _gpu_or_skip()
    from refinekv import _hip

    calls = []
    real = _hip.dense_decode

    def record(query, keys, values, length=None, workspace=None, output=None):
        out = real(query, keys, values, length=length, workspace=workspace, output=output)
        calls.append((query.clone(), keys[:, :length].clone(), values[:, :length].clone(),
                      out.clone()))
        return out

    monkeypatch.setattr(_hip, "dense_decode", record)
    model = tiny_model("llama", "cuda")
    with RefineKV(model, RefineKVConfig(backend="hip", full_attention_layers=1,
                                        collect_stats=True)) as session:
        generate(model)
        assert session.stats["decode_attention_calls"] == 6
    assert len(calls) == 3  # layer 0, three decode steps

    def bits(t):
        return t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)

    for step, (q, k, v, out) in enumerate(calls):
        assert k.shape[1] == 40 + step  # the visible prefix: prompt + tokens so far
        want = oracle_lib.dense_attention(q.float().cpu().numpy(), bits(k), bits(v))
        want = torch.from_numpy(want).to(torch.bfloat16).float().numpy()
        err = np.abs(out.float().cpu().numpy() - want)
        assert err.max() <= 2e-2 and err.mean() <= 1e-3 * np.abs(want).mean() + 1e-6


# ---------------------------------------------------------------------------
# GPU: the hook's decode calls against the CPU oracle (eager and graph replay)
# ---------------------------------------------------------------------------

def _oracle_check(oracle_lib, call):
    """The oracle's sparse_attention on one recorded decode call: mask equal,
    output within the north-star tolerance.  Returns the expanded fraction."""
    import numpy as np

    def bits(t):
        return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)

    s = call["summary"]
    summ = dict(counts=s.counts.cpu().numpy(), key_mean=bits(s.key_mean),
                value_mean=bits(s.value_mean), ellipsoid=bits(s.ellipsoid),
                value_norm=s.value_norm.cpu().numpy(),
                max_value_norm=s.max_value_norm.cpu().numpy(), prompt_length=s.prompt_length,
                block_size=s.block_size)
    n = call["suffix"]
    anchor = call["anchor"]
    out, mask = oracle_lib.sparse_attention(
        call["query"][:, :, 0].float().cpu().numpy(), summ, bits(s.keys), bits(s.values),
        bits(call["key_suffix"][:, :n]), bits(call["value_suffix"][:, :n]), call["eps"],
        call["reduction"], None if anchor is None else anchor.cpu().numpy())
    got_mask = call["selected"].cpu().numpy().astype(np.uint8)
    assert np.array_equal(got_mask, mask), "hook mask differs from the oracle"
    want = torch.from_numpy(out).to(torch.bfloat16).float().numpy()
    got = call["output"][:, :, 0].float().cpu().numpy()
    err = np.abs(got - want)
    assert err.max() <= 2e-2 and err.mean() <= 1e-3 * np.abs(want).mean() + 1e-6, err.max()
    return float(mask.mean())


class _Recorder:
    """Wraps the hook's sparse_attention: eager calls are recorded with
    copies of their inputs and outputs; a call under graph capture records a
    device copy of the query into the graph (so every replay refreshes it)
    and keeps references to the persistent buffers the replays reuse."""

    def __init__(self, real):
        self.real = real
        self.eager, self.graph = [], []

    def __call__(self, query, summary, key_suffix, value_suffix, config, *, anchor_mask=None,
                 workspace=None, return_selected=False, suffix_length=None,
                 access_counter=None):
        from refinekv.attention import AttentionResult

        result = self.real(query, summary, key_suffix, value_suffix, config,
                           anchor_mask=anchor_mask, workspace=workspace, return_selected=True,
                           suffix_length=suffix_length, access_counter=access_counter)
        call = dict(summary=summary, anchor=anchor_mask, eps=config.eps,
                    reduction=config.gqa_reduction, key_suffix=key_suffix,
                    value_suffix=value_suffix)
        if torch.cuda.is_current_stream_capturing():
            call.update(query=query.clone(), output=result.output, selected=result.selected,
                        suffix_tensor=suffix_length)
            self.graph.append(call)
        else:
            n = key_suffix.shape[1] if suffix_length is None else int(suffix_length.item())
            call.update(query=query.clone(), output=result.output.clone(),
                        selected=result.selected.clone(), suffix=n,
                        key_suffix=key_suffix.clone(), value_suffix=value_suffix.clone())
            self.eager.append(call)
        return AttentionResult(result.output, result.selected if return_selected else None)


def small_model(family):
    torch.manual_seed(3)
    config_cls, model_cls = {
        "llama": (transformers.LlamaConfig, transformers.LlamaForCausalLM),
        "qwen2": (transformers.Qwen2Config, transformers.Qwen2ForCausalLM),
    }[family]
    config = config_cls(vocab_size=512, hidden_size=512, intermediate_size=1024,
                        num_hidden_layers=2, num_attention_heads=8, num_key_value_heads=2,
                        pad_token_id=0, eos_token_id=None)
    return model_cls(config).eval().to("cuda").to(torch.bfloat16)


@pytest.mark.gpu
@pytest.mark.parametrize("family,reduction,anchors", [("llama", "any", 4), ("qwen2", "max", 0)])
def test_hip_hook_decode_calls_match_oracle(family, reduction, anchors, monkeypatch, oracle_lib):
    """Every decode call the hook makes (eager generation: visible cache,
    suffix slices; then graph replays: device suffix length over the full
    buffer) has the oracle's mask and output for the query, summary, suffix
    and anchor mask it was given."""
    _gpu_or_skip()
    from refinekv.integrations import transformers as hook

    model = small_model(family)
    recorder = _Recorder(hook.sparse_attention)
    monkeypatch.setattr(hook, "sparse_attention", recorder)
    config = RefineKVConfig(backend="hip", eps=0.01, block_size=16, gqa_reduction=reduction,
                            anchor_tokens=anchors)
    gen = torch.Generator().manual_seed(11)
    ids = torch.randint(3, 500, (1, 700), generator=gen).cuda()
    options = dict(input_ids=ids, attention_mask=torch.ones_like(ids), max_new_tokens=6,
                   min_new_tokens=6, eos_token_id=None, forced_eos_token_id=None,
                   do_sample=False)
    with RefineKV(model, config):
        eager_tokens = model.generate(**options)
    assert len(recorder.eager) == 5 * 2  # 5 decode forwards x 2 layers
    fractions = [_oracle_check(oracle_lib, call) for call in recorder.eager]
    assert all(0 < f <= 1 for f in fractions)
    recorder.eager.clear()
    with RefineKV(model, config, cuda_graph=True):
        graph_tokens = model.generate(**options)
        # (the graph's replays have run: its last replay left its query copy,
        # mask and output in the recorded buffers)
        assert len(recorder.graph) == 2
        for call in recorder.graph:
            call["suffix"] = int(call["suffix_tensor"].item())
            assert call["suffix"] == 5
            _oracle_check(oracle_lib, call)
    assert torch.equal(graph_tokens, eager_tokens)
    assert recorder.eager, "the graph path's warm-up steps run eagerly"
    for call in recorder.eager:
        _oracle_check(oracle_lib, call)
