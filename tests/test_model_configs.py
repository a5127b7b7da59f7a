"""BASELINE.json model configs through the Transformers hook on the GPU.

configs[1] (Llama-3.1-8B shape, 32768-token prompt, block 32, eps 0.01,
"any", 32 prompt anchors), configs[2] (the same shape at 131072 prompt
tokens, no anchors) and configs[3] (Qwen2.5-7B shape, group 7, RoPE
theta 1e6 with static YaRN factor 4, 65536-token prompt, block 64, eps
0.005, "max", 64 anchors), random-init weights and uniform random prompt ids:
a few greedy decode steps with RefineKV(backend="hip", collect_stats=True).
Sampled (layer, step) decode calls are compared with the CPU oracle (mask
equal, output within tolerance), every call's mask is checked against the
in-kernel access counter's closed form (transformers.py:590-594), and the
hand-off status of every layer is clean.
"""

import numpy as np
import pytest
import torch

transformers = pytest.importorskip("transformers")
from refinekv import RefineKV, RefineKVConfig  # noqa: E402

pytestmark = pytest.mark.gpu

CONFIGS = {
    "llama32k": dict(family="llama", prompt=32768, block=32, eps=0.01, reduction="any",
                     anchors=32),
    "llama128k": dict(family="llama", prompt=131072, block=32, eps=0.01, reduction="any",
                      anchors=0),
    "qwen64k": dict(family="qwen2", prompt=65536, block=64, eps=0.005, reduction="max",
                    anchors=64),
}
DECODE_STEPS = 3
SAMPLES = ((0, 0), (7, 1), (13, 2), (-1, 2))  # (layer, decode step)


def _model(family, positions):
    if family == "llama":
        config = transformers.LlamaConfig(
            vocab_size=128256, hidden_size=4096, intermediate_size=14336, num_hidden_layers=32,
            num_attention_heads=32, num_key_value_heads=8, max_position_embeddings=positions,
            rms_norm_eps=1e-5, rope_parameters={"rope_type": "default", "rope_theta": 500000.0},
            bos_token_id=None, eos_token_id=None, pad_token_id=None)
        cls = transformers.LlamaForCausalLM
    else:
        config = transformers.Qwen2Config(
            vocab_size=152064, hidden_size=3584, intermediate_size=18944, num_hidden_layers=28,
            num_attention_heads=28, num_key_value_heads=4, max_position_embeddings=4 * 32768,
            rms_norm_eps=1e-6, rope_parameters={"rope_type": "yarn", "factor": 4.0,
                                                "original_max_position_embeddings": 32768,
                                                "rope_theta": 1000000.0},
            use_sliding_window=False, bos_token_id=None, eos_token_id=None, pad_token_id=None)
        cls = transformers.Qwen2ForCausalLM
    torch.manual_seed(0)
    saved = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device("cuda"):
            model = cls(config)
    finally:
        torch.set_default_dtype(saved)
    return model.eval(), config


@pytest.mark.parametrize("name", sorted(CONFIGS))
def test_model_config_decode_calls_match_oracle(name, monkeypatch, oracle_lib):
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    from refinekv.integrations import transformers as hook
    from test_transformers import _oracle_check, _Recorder

    spec = CONFIGS[name]
    model, mconfig = _model(spec["family"], spec["prompt"] + 16)
    recorder = _Recorder(hook.sparse_attention)
    monkeypatch.setattr(hook, "sparse_attention", recorder)
    config = RefineKVConfig(backend="hip", block_size=spec["block"], eps=spec["eps"],
                            gqa_reduction=spec["reduction"], anchor_tokens=spec["anchors"],
                            collect_stats=True)
    gen = torch.Generator().manual_seed(1)
    ids = torch.randint(0, mconfig.vocab_size, (1, spec["prompt"]), generator=gen).cuda()
    with RefineKV(model, config) as session:
        model.generate(input_ids=ids, attention_mask=torch.ones_like(ids),
                       max_new_tokens=DECODE_STEPS + 1, min_new_tokens=DECODE_STEPS + 1,
                       eos_token_id=None, do_sample=False)
        stats = session.stats  # also raises if any layer's hand-off status is set
        layers = mconfig.num_hidden_layers
        assert len(recorder.eager) == DECODE_STEPS * layers
        anchors = [recorder.eager[i]["anchor"] for i in range(layers)]
        if spec["anchors"]:
            assert all(a is not None and a.any() for a in anchors)
        else:
            assert all(a is None for a in anchors)
    group = mconfig.num_attention_heads // mconfig.num_key_value_heads
    # the in-kernel access counter equals the closed form over every call's mask
    blocks = sum(oracle_lib.access_blocks(c["selected"].cpu().numpy(),
                                          c["summary"].counts.cpu().numpy())
                 for c in recorder.eager)
    suffix = sum(mconfig.num_attention_heads * c["suffix"] for c in recorder.eager)
    assert stats["accessed"] == blocks * group + suffix
    assert stats["decode_attention_calls"] == DECODE_STEPS * layers
    for layer, step in SAMPLES:
        layer %= layers
        call = recorder.eager[step * layers + layer]
        assert call["suffix"] == step + 1
        fraction = _oracle_check(oracle_lib, call)
        assert 0 < fraction <= 1
