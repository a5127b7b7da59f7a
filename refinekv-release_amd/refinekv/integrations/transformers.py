"""RefineKV inside Hugging Face generation (the reference's adapter API,
src/refinekv/integrations/transformers.py).

``with RefineKV(model, config): model.generate(...)`` runs the prompt with
dense SDPA, builds each layer's block summary (and prompt-anchor mask) from
the prefill K/V, and answers every later single-token step with
``sparse_attention`` over the summary plus the exact generated suffix.  The
model's modules are not modified: a named attention function ("refinekv") is
registered with Transformers and selected for the duration of the context;
hooks that are removed on exit keep the per-request state.

Written against the transformers 5.x cache API (``StaticLayer``,
``Cache(layers=...)``, ``get_mask_sizes(query_length)``, no
``cache_position`` argument to the model).
"""

from dataclasses import dataclass, field
from functools import wraps
import math

import torch

try:
    from transformers import AttentionInterface, AttentionMaskInterface
    from transformers.cache_utils import Cache, StaticCache, StaticLayer
    from transformers.integrations.sdpa_attention import sdpa_attention_forward
except ImportError as error:  # the reference raises the same way (transformers.py:9-16)
    raise ImportError("the RefineKV Transformers adapter needs the 'transformers' package") from error

from ..attention import select_blocks_union, sparse_attention
from ..config import RefineKVConfig
from ..summary import BlockSummary, build_summary, store_and_build_summary

_NO_ATTRIBUTE = object()
SUPPORTED_MODEL_TYPES = ("llama", "qwen2")


def _query_length(arg):
    """get_mask_sizes receives the query length (transformers 5.x) or the
    cache positions (older releases)."""
    return arg if isinstance(arg, int) else int(arg.shape[0])


class _VisibleStaticLayer(StaticLayer):
    """Preallocated K/V exposing only the tokens written so far
    (transformers.py:25-63): attention sees real tokens only, so the prompt
    needs no padding mask and decode appends in place."""

    is_compileable = False

    def __init__(self, max_cache_len):
        super().__init__(max_cache_len)
        self.visible = 0
        # Set by the RefineKV session for its sparse layers: the prompt write
        # then also builds the layer's block summary (prefill_summary) from
        # the same read of the prompt's keys and values.
        self.summary_config = None
        self.prefill_summary = None

    def lazy_initialization(self, key_states, value_states):
        self.dtype, self.device = key_states.dtype, key_states.device
        batch, heads = key_states.shape[:2]
        self.batch_size = self.max_batch_size = batch
        self.num_heads = heads
        self.k_head_dim, self.v_head_dim = key_states.shape[-1], value_states.shape[-1]
        self.keys = torch.empty((batch, heads, self.max_cache_len, self.k_head_dim),
                                dtype=self.dtype, device=self.device)
        self.values = torch.empty((batch, heads, self.max_cache_len, self.v_head_dim),
                                  dtype=self.dtype, device=self.device)
        self.is_initialized = True

    def update(self, key_states, value_states, *args, **kwargs):
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        start = self.visible
        end = start + key_states.shape[-2]
        if end > self.max_cache_len:
            raise ValueError("visible KV cache capacity exceeded")
        if start == 0 and self.summary_config is not None and key_states.shape[0] == 1:
            self.prefill_summary = store_and_build_summary(
                key_states[0], value_states[0], self.keys[0, :, :end], self.values[0, :, :end],
                self.summary_config)
        else:
            self.keys[:, :, start:end].copy_(key_states)
            self.values[:, :, start:end].copy_(value_states)
        self.visible = end
        return self.keys[:, :, :end], self.values[:, :, :end]

    def get_mask_sizes(self, query_length):
        return self.visible + _query_length(query_length), 0

    def get_seq_length(self):
        return self.visible

    def get_max_length(self):
        return self.max_cache_len


def make_visible_static_cache(model, max_cache_len):
    """A preallocated cache with a mask-free visible prefix (transformers.py:66-73)."""
    if not isinstance(max_cache_len, int) or isinstance(max_cache_len, bool) or max_cache_len <= 0:
        raise ValueError("max_cache_len must be a positive integer")
    return Cache(layers=[_VisibleStaticLayer(max_cache_len) for _ in model.model.layers])


class _GraphStaticLayer(_VisibleStaticLayer):
    """Fixed K/V addresses for graph replay (transformers.py:75-105): the
    prompt is written once, then every decode token goes to the device
    position ``write_position`` (a shared int64 tensor the step advances), and
    attention sees the whole buffer; the device suffix length masks it."""

    def __init__(self, max_cache_len, write_position):
        super().__init__(max_cache_len)
        self.graph_decode = False
        self.write_position = write_position

    def update(self, key_states, value_states, *args, **kwargs):
        if not self.graph_decode:
            if self.visible:
                raise ValueError("graph cache requires one complete prompt prefill")
            return super().update(key_states, value_states)
        self.keys.index_copy_(2, self.write_position, key_states)
        self.values.index_copy_(2, self.write_position, value_states)
        return self.keys, self.values

    def get_mask_sizes(self, query_length):
        if self.graph_decode:
            return self.max_cache_len, 0
        return _query_length(query_length), 0


@dataclass
class _LayerState:
    """One attention layer's request state (transformers.py:108-114)."""

    prompt_length: int
    visible_length: int
    summary: BlockSummary | None = None
    anchor_mask: torch.Tensor | None = None
    workspace: dict = field(default_factory=dict)


def mask_is_visible_prefix(mask, visible, length):
    """Whether a decode query's attention mask (None, boolean with True =
    attend, or additive with 0 = attend and the dtype's minimum or -inf =
    masked; any broadcastable shape ending in the key length) lets every
    query head see exactly the tokens [0, visible) of a cache of `length`
    tokens: what the dense decode kernel attends.  A padded or otherwise
    masked token inside the prefix, a visible token past it, or any other
    additive bias gives False (the SDPA path then applies the mask, as
    transformers.py:510-520 does).  Reads the mask on the host."""
    if mask is None:
        return True
    if mask.shape[-1] != length:
        return False
    if mask.dtype == torch.bool:
        allowed = mask
    else:
        zero = mask == 0
        blocked = mask <= torch.finfo(mask.dtype).min / 2
        if not bool((zero | blocked).all()):
            return False
        allowed = zero
    want = torch.arange(length, device=mask.device) < visible
    return bool((allowed == want).all())


def _refinekv_attention(module, query, key, value, attention_mask, dropout=0.0, scaling=None,
                        **kwargs):
    """The registered "refinekv" attention function (transformers.py:117-123)."""
    session = getattr(module, "_refinekv_session", None)
    if session is None:
        raise RuntimeError("the RefineKV attention interface runs only inside a RefineKV context")
    return session._attention(module, query, key, value, attention_mask, scaling, kwargs)


def _register():
    # A named implementation next to Transformers' own; SDPA's mask builder.
    AttentionInterface.register("refinekv", _refinekv_attention)
    AttentionMaskInterface.register("refinekv", AttentionMaskInterface()["sdpa"])


def _rotary(model_type):
    if model_type == "qwen2":
        from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb
    else:
        from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
    return apply_rotary_pos_emb


class RefineKV:
    """Dense prefill, then RefineKV single-sequence cached decode.

    Example::

        with RefineKV(model, RefineKVConfig(anchor_tokens=32)):
            output = model.generate(**inputs, max_new_tokens=128, do_sample=False)

    Supported: Llama and Qwen2/Qwen2.5 in eval mode, batch 1, one unpadded
    prompt per generation starting from an empty cache, DynamicCache or the
    visible-prefix static cache (``cache_implementation="static"``).  The
    state lives in this object and is released on exit.  ``cuda_graph=True``
    runs fixed-length greedy decode as replays of one captured HIP graph over
    a private preallocated cache (bf16 model on the GPU, kernel backend).
    """

    def __init__(self, model, config: RefineKVConfig | None = None, *, cuda_graph=False):
        self.model = model
        self.config = config or RefineKVConfig()
        self.cuda_graph = cuda_graph
        self._graph_mode = False
        self._graph_suffix_length = None
        self._layers = {}
        self._anchor_queries = {}
        self._handles = []
        self._cache = None
        self._active = False
        self._totals = self._zero_totals()
        self._block_accesses = None  # device int64: the kernels' block term
        self._group = 1

    @staticmethod
    def _zero_totals():
        return dict(accessed=0, dense=0, decode_attention_calls=0)

    @property
    def stats(self):
        """Decode-only KV access counters (transformers.py:161-176): an
        unexpanded block counts as one representative token.  Reading this
        synchronizes the device when counters are tensors, and raises
        refinekv._hip.HandoffError if a HIP decode step of a live layer had a
        hand-off wait give up (its outputs were not to be trusted)."""
        self.check_handoffs()
        totals = {k: (v.item() if torch.is_tensor(v) else v) for k, v in self._totals.items()}
        blocks = self._block_accesses
        if blocks is not None:
            # the kernels' block term counts per KV head; each serves `group` query heads
            totals["accessed"] += int(blocks.item()) * self._group
        dense = totals["dense"]
        totals["equivalent_access_ratio"] = totals["accessed"] / dense if dense else None
        return totals

    def check_handoffs(self):
        """Raise HandoffError if any live layer's HIP decode workspace had a
        hand-off wait give up (a host synchronization per layer)."""
        from .. import _hip

        for state in self._layers.values():
            if "hip_scratch" in state.workspace:
                _hip.check_workspace(state.workspace)

    # -- context ---------------------------------------------------------
    def __enter__(self):
        model = self.model
        if self._active or hasattr(model, "_refinekv_session"):
            raise RuntimeError("this model already has an active RefineKV context")
        if model.training:
            raise ValueError("RefineKV is inference-only; call model.eval() first")
        if model.config.model_type not in SUPPORTED_MODEL_TYPES:
            raise ValueError("the Transformers adapter supports model_type='llama' or 'qwen2'")
        if getattr(model.config, "use_sliding_window", False):
            raise ValueError("sliding-window attention is not supported")
        if getattr(model.config, "output_attentions", False):
            raise ValueError("RefineKV does not return attention weights")
        self._modules = list(model.model.layers)
        if any(getattr(m.self_attn, "sliding_window", None) is not None for m in self._modules):
            raise ValueError("sliding-window attention is not supported")
        _register()
        self._saved_implementation = model.config._attn_implementation
        self._saved_layer_implementations = [
            m.self_attn.config._attn_implementation for m in self._modules
        ]
        self._inference = torch.inference_mode()
        self._inference.__enter__()
        try:
            self._install()
        except BaseException:
            self._restore()
            self._inference.__exit__(None, None, None)
            raise
        self._active = True
        return self

    def _install(self):
        model = self.model
        model.set_attn_implementation("refinekv")
        model._refinekv_session = self
        # layer identity -> index (no reliance on architecture-specific attributes)
        self._module_indices = {}
        for index, layer in enumerate(self._modules):
            layer.self_attn._refinekv_session = self
            self._module_indices[id(layer.self_attn)] = index
            if self.config.anchor_tokens and index >= self.config.full_attention_layers:
                self._handles.append(layer.self_attn.register_forward_pre_hook(
                    self._capture_anchor_queries, with_kwargs=True))
        self._saved_generate = model.__dict__.get("generate", _NO_ATTRIBUTE)
        original_generate = model.generate

        @wraps(original_generate)
        def generate(*args, **kwargs):
            return self._generate(original_generate, args, kwargs)

        model.generate = generate
        self._handles.append(model.register_forward_pre_hook(self._before_forward,
                                                             with_kwargs=True))
        self._handles.append(model.register_forward_hook(self._after_forward, with_kwargs=True))

    def _restore(self):
        for handle in self._handles:
            handle.remove()
        self._handles.clear()
        for layer, saved in zip(getattr(self, "_modules", []),
                                getattr(self, "_saved_layer_implementations", [])):
            if getattr(layer.self_attn, "_refinekv_session", None) is self:
                del layer.self_attn._refinekv_session
            layer.self_attn.config._attn_implementation = saved
        if getattr(self.model, "_refinekv_session", None) is self:
            del self.model._refinekv_session
        if hasattr(self, "_saved_generate"):
            if self._saved_generate is _NO_ATTRIBUTE:
                self.model.__dict__.pop("generate", None)
            else:
                self.model.generate = self._saved_generate
            del self._saved_generate
        if hasattr(self, "_saved_implementation"):
            self.model.config._attn_implementation = self._saved_implementation
        # request state is released; the counters stay readable after exit
        self._layers.clear()
        self._anchor_queries.clear()
        self._cache = None
        self._graph_mode = False
        self._graph_suffix_length = None
        self._active = False

    def __exit__(self, exc_type, exc_value, traceback):
        try:
            self._restore()
        finally:
            self._inference.__exit__(exc_type, exc_value, traceback)
        return False

    def _reset_request(self, cache):
        self._layers.clear()
        self._anchor_queries.clear()
        self._totals = self._zero_totals()
        self._block_accesses = None
        self._cache = cache
        # the visible caches build the sparse layers' summaries as they take
        # the prompt
        for index, layer in enumerate(getattr(cache, "layers", ())):
            if isinstance(layer, _VisibleStaticLayer):
                sparse = index >= self.config.full_attention_layers
                layer.summary_config = self.config if sparse else None
                layer.prefill_summary = None

    # -- generate --------------------------------------------------------
    def _generate(self, original_generate, args, kwargs):
        """transformers.py:226-264: fresh state per call, static-cache
        requests get the visible-prefix cache, graph mode on request."""
        self._reset_request(None)
        if self.cuda_graph:
            return self._generate_graph(args, kwargs)
        if isinstance(kwargs.get("past_key_values"), StaticCache):
            raise ValueError("stock StaticCache is unsupported; use cache_implementation='static' "
                             "or make_visible_static_cache")
        generation = kwargs.get("generation_config") or self.model.generation_config
        implementation = kwargs.get("cache_implementation", generation.cache_implementation)
        if implementation == "static":
            if kwargs.get("past_key_values") is not None:
                raise ValueError("pass either a static cache request or past_key_values")
            ids = kwargs.get("input_ids", args[0] if args else None)
            if not isinstance(ids, torch.Tensor) or ids.ndim != 2:
                raise ValueError("static cache generation requires input_ids of shape (1, tokens)")
            prompt = ids.shape[1]
            new_tokens = kwargs.get("max_new_tokens", generation.max_new_tokens)
            if new_tokens is not None:
                capacity = prompt + int(new_tokens)
            else:
                capacity = int(kwargs.get("max_length", generation.max_length) or 0)
            if capacity <= prompt:
                raise ValueError("static cache capacity must exceed prompt length")
            kwargs["past_key_values"] = make_visible_static_cache(self.model, capacity)
            kwargs["cache_implementation"] = None
        kwargs["disable_compile"] = True  # summaries are built inside the forward
        return original_generate(*args, **kwargs)

    def _generate_graph(self, args, kwargs):
        """Fixed-length greedy decode replaying one captured step
        (transformers.py:302-440)."""
        input_ids, new_tokens, penalty, mask = self._check_graph_request(args, kwargs)
        model, device = self.model, input_ids.device
        prompt = input_ids.shape[1]
        position = torch.tensor([prompt], device=device, dtype=torch.long)
        cache = Cache(layers=[_GraphStaticLayer(prompt + new_tokens, position)
                              for _ in model.model.layers])
        prefill = model(input_ids=input_ids, attention_mask=mask, past_key_values=cache,
                        use_cache=True, logits_to_keep=1)
        seen = None
        if penalty != 1.0:
            seen = torch.zeros_like(prefill.logits[:, -1], dtype=torch.bool)
            seen.scatter_(1, input_ids, True)

        def pick(scores):
            scores = scores.float()
            if seen is not None:
                penalized = torch.where(scores < 0, scores * penalty, scores / penalty)
                scores = torch.where(seen, penalized, scores)
            return scores.argmax(-1, keepdim=True)

        token = pick(prefill.logits[:, -1]).clone()
        produced = torch.empty(new_tokens, device=device, dtype=input_ids.dtype)
        produced[:1].copy_(token.reshape(1))
        del prefill
        for layer in cache.layers:
            layer.graph_decode = True
        slot = torch.ones(1, device=device, dtype=torch.long)
        self._graph_suffix_length = torch.zeros((), device=device, dtype=torch.int32)
        self._graph_mode = True

        def step():
            self._graph_suffix_length.add_(1)
            if seen is not None:
                seen.scatter_(1, token, True)
            out = model(input_ids=token, attention_mask=None, past_key_values=cache,
                        position_ids=position.unsqueeze(0), use_cache=True, logits_to_keep=1)
            following = pick(out.logits[:, -1])
            produced.index_copy_(0, slot, following.reshape(1))
            token.copy_(following)
            position.add_(1)
            slot.add_(1)

        try:
            warmup = min(2, new_tokens - 2)
            side = torch.cuda.Stream(device=device)
            side.wait_stream(torch.cuda.current_stream(device))
            with torch.cuda.stream(side):
                for _ in range(warmup):
                    step()
            torch.cuda.current_stream(device).wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                step()
            # capture only records; each replay produces one token
            for _ in range(new_tokens - 1 - warmup):
                graph.replay()
            torch.cuda.synchronize(device)
            return torch.cat((input_ids, produced.view(1, -1)), dim=1)
        finally:
            self._graph_mode = False
            self._graph_suffix_length = None

    _GRAPH_KWARGS = frozenset((
        "input_ids", "attention_mask", "max_new_tokens", "min_new_tokens", "do_sample",
        "num_beams", "use_cache", "eos_token_id", "forced_eos_token_id", "pad_token_id",
        "cache_implementation", "disable_compile", "repetition_penalty"))
    _GRAPH_INERT_PROCESSORS = {
        "encoder_repetition_penalty": (None, 1.0), "no_repeat_ngram_size": (None, 0),
        "bad_words_ids": (None, []), "suppress_tokens": (None, []),
        "begin_suppress_tokens": (None, []), "forced_bos_token_id": (None,),
        "sequence_bias": (None, {}), "force_words_ids": (None, []), "constraints": (None, []),
        "watermarking_config": (None,)}

    def _check_graph_request(self, args, kwargs):
        """The reference's graph-mode preconditions (transformers.py:304-388)."""
        extra = set(kwargs) - self._GRAPH_KWARGS
        if extra:
            raise ValueError(f"CUDA Graph generation does not support {sorted(extra)}")
        if args:
            if len(args) != 1 or "input_ids" in kwargs:
                raise ValueError("pass one input_ids tensor to CUDA Graph generation")
            input_ids = args[0]
        else:
            input_ids = kwargs.get("input_ids")
        if (not isinstance(input_ids, torch.Tensor) or input_ids.ndim != 2
                or input_ids.shape[0] != 1 or input_ids.dtype != torch.long):
            raise ValueError("CUDA Graph generation requires one input_ids sequence")
        new_tokens = kwargs.get("max_new_tokens")
        if not isinstance(new_tokens, int) or new_tokens < 4:
            raise ValueError("CUDA Graph generation requires max_new_tokens >= 4")
        if (kwargs.get("min_new_tokens") != new_tokens or "eos_token_id" not in kwargs
                or kwargs["eos_token_id"] is not None):
            raise ValueError("CUDA Graph generation requires fixed output: "
                             "min_new_tokens=max_new_tokens and eos_token_id=None")
        gen = self.model.generation_config
        if (kwargs.get("do_sample", gen.do_sample)
                or (kwargs.get("num_beams", gen.num_beams) or 1) != 1
                or kwargs.get("use_cache", gen.use_cache) not in (None, True)
                or kwargs.get("forced_eos_token_id", gen.forced_eos_token_id) is not None
                or kwargs.get("cache_implementation", gen.cache_implementation)
                not in (None, "static")
                or (gen.num_return_sequences or 1) != 1):
            raise ValueError("CUDA Graph generation supports greedy, single-beam, "
                             "static-cache decode only")
        penalty = kwargs.get("repetition_penalty", getattr(gen, "repetition_penalty", 1.0))
        penalty = 1.0 if penalty is None else float(penalty)
        if not math.isfinite(penalty) or penalty <= 0:
            raise ValueError("repetition_penalty must be finite and positive")
        active = [name for name, inert in self._GRAPH_INERT_PROCESSORS.items()
                  if getattr(gen, name, None) not in inert]
        if active:
            raise ValueError(f"CUDA Graph generation does not support logits processors {active}")
        if (not input_ids.is_cuda or input_ids.device != self.model.device
                or self.model.dtype != torch.bfloat16 or self.config.backend == "torch"
                or self.config.collect_stats or self.config.full_attention_layers):
            raise ValueError("CUDA Graph requires a GPU BF16 model, the kernel backend, no "
                             "stats, and no dense layers")
        mask = kwargs.get("attention_mask")
        if mask is not None and (not isinstance(mask, torch.Tensor)
                                 or mask.shape != input_ids.shape
                                 or mask.device != input_ids.device or not bool(mask.all())):
            raise ValueError("CUDA Graph generation requires an unpadded prompt")
        return input_ids, new_tokens, penalty, mask

    # -- hooks -----------------------------------------------------------
    def _before_forward(self, module, args, kwargs):
        """Per-forward checks and request reset (transformers.py:442-483)."""
        inputs = kwargs.get("input_ids")
        if inputs is None:
            inputs = kwargs.get("inputs_embeds")
        if inputs is None and args:
            inputs = args[0]
        if inputs is not None and inputs.shape[0] != 1:
            raise ValueError("RefineKV requires batch_size=1 and num_beams=1")
        if not kwargs.get("use_cache", self.model.config.use_cache):
            raise ValueError("RefineKV requires use_cache=True")
        if kwargs.get("output_attentions", False):
            raise ValueError("RefineKV does not return attention weights")
        cache = kwargs.get("past_key_values")
        if cache is not None and cache is self._cache:
            return
        if cache is not None and cache.get_seq_length() != 0:
            raise ValueError("start each RefineKV generation with an empty KV cache")
        if not self._prompt_unpadded(kwargs.get("attention_mask"), inputs):
            raise ValueError("RefineKV requires an unpadded prompt")
        self._reset_request(cache)

    @staticmethod
    def _prompt_unpadded(mask, inputs):
        if isinstance(mask, dict):
            mask = mask.get("full_attention")
        if mask is None:
            return True
        if mask.ndim == 2:
            return bool(mask.all())
        if mask.ndim == 4 and inputs is not None:
            # a prepared causal mask: its last prompt row must see every token
            last = mask[0, 0, -1, :inputs.shape[1]]
            return bool(last.all()) if mask.dtype == torch.bool else bool((last == 0).all())
        return False

    def _after_forward(self, module, args, kwargs, output):
        cache = getattr(output, "past_key_values", None)
        if cache is not None:
            self._cache = cache

    def _capture_anchor_queries(self, module, args, kwargs):
        """RoPE'd queries of the last anchor_tokens prompt positions, from a
        projection of the tail alone (transformers.py:485-508): a projection of
        the whole prompt can round differently in bf16 and move blocks across
        the threshold."""
        index = self._module_indices[id(module)]
        if index in self._layers:
            return  # decode step
        hidden = kwargs.get("hidden_states", args[0] if args else None)
        rope = kwargs.get("position_embeddings", args[1] if len(args) > 1 else None)
        if hidden is None or rope is None:
            raise RuntimeError("prompt anchors require hidden states and RoPE embeddings")
        count = min(self.config.anchor_tokens, hidden.shape[1])
        tail = hidden[:, -count:]
        query = module.q_proj(tail).view(*tail.shape[:-1], -1, module.head_dim).transpose(1, 2)
        cos, sin = rope
        query, _ = _rotary(self.model.config.model_type)(
            query, query, cos[..., -count:, :], sin[..., -count:, :])
        self._anchor_queries[index] = query[0].detach()  # (q_heads, count, d)

    # -- attention -------------------------------------------------------
    def _attention(self, module, query, key, value, mask, scaling, kwargs):
        """transformers.py:522-596: the first call of a layer is the prompt,
        every later call one decode token."""
        if query.shape[0] != 1:
            raise ValueError("RefineKV requires batch_size=1")
        index = self._module_indices[id(module)]
        state = self._layers.get(index)
        if state is None:
            return self._prefill(module, index, query, key, value, mask, scaling, kwargs)
        if query.shape[2] != 1:
            raise ValueError("RefineKV supports one full prefill followed by single-token decode")
        heads, dim = key.shape[1], query.shape[-1]
        groups = query.shape[1] // heads
        if self._graph_mode:
            if state.summary is None:
                raise ValueError("CUDA Graph does not support dense attention layers")
            result = sparse_attention(
                query[0].reshape(heads, groups, 1, dim), state.summary,
                key[0, :, state.prompt_length:], value[0, :, state.prompt_length:],
                self.config, anchor_mask=state.anchor_mask, workspace=state.workspace,
                suffix_length=self._graph_suffix_length)
            return self._to_model_layout(result.output, query), None
        state.visible_length += 1
        if key.shape[2] < state.visible_length:
            raise ValueError("the KV cache no longer contains the full visible prefix")
        if state.summary is None:
            if self.config.collect_stats:
                dense = query.shape[1] * state.visible_length
                self._record(dense, dense)
            return self._dense_decode(module, query, key, value, mask, scaling, kwargs,
                                      state.visible_length, state.workspace)
        counter = None
        if self.config.collect_stats:
            # expanded blocks count their tokens, the others one representative:
            # the call adds that block term (per KV head) to one device counter
            if self._block_accesses is None:
                self._block_accesses = torch.zeros((), dtype=torch.int64, device=query.device)
                self._group = groups
            counter = self._block_accesses
        result = sparse_attention(
            query[0].reshape(heads, groups, 1, dim), state.summary,
            key[0, :, state.prompt_length:state.visible_length],
            value[0, :, state.prompt_length:state.visible_length],
            self.config, anchor_mask=state.anchor_mask, workspace=state.workspace,
            access_counter=counter)
        if self.config.collect_stats:
            suffix = query.shape[1] * (state.visible_length - state.prompt_length)
            self._record(suffix, query.shape[1] * state.visible_length)
        return self._to_model_layout(result.output, query), None

    @staticmethod
    def _to_model_layout(output, query):
        # (kv_heads, group, 1, d) -> (1, 1, q_heads, d), the attention interface's layout
        q_heads, dim = query.shape[1], query.shape[-1]
        return output.reshape(q_heads, 1, dim).transpose(0, 1).unsqueeze(0)

    def _prefill(self, module, index, query, key, value, mask, scaling, kwargs):
        prompt = query.shape[2]
        output = sdpa_attention_forward(module, query, key, value, mask, dropout=0,
                                        scaling=scaling, **kwargs)
        state = _LayerState(prompt, prompt)
        if index >= self.config.full_attention_layers:
            state.summary = self._stored_summary(index, prompt)
            if state.summary is None:
                state.summary = build_summary(key[0, :, :prompt], value[0, :, :prompt],
                                              self.config)
            state.anchor_mask = self._anchor_mask(index, state, query, key, prompt)
        self._layers[index] = state
        return output

    def _stored_summary(self, index, prompt):
        """The summary the visible cache built while writing this layer's
        prompt, if it did."""
        layers = getattr(self._cache, "layers", None)
        if layers is None or index >= len(layers):
            return None
        layer = layers[index]
        summary = getattr(layer, "prefill_summary", None)
        if summary is None or summary.prompt_length != prompt:
            return None
        layer.prefill_summary = None
        return summary

    def _anchor_mask(self, index, state, query, key, prompt):
        """Union of the selections of the last anchor_tokens prompt queries
        (transformers.py:539-552)."""
        count = min(self.config.anchor_tokens, prompt)
        queries = self._anchor_queries.pop(index, None)
        if count and queries is None:
            raise RuntimeError(f"missing prompt anchor queries in layer {index}")
        if not count:
            return None
        heads, dim = key.shape[1], query.shape[-1]
        groups = query.shape[1] // heads
        # one batched selection over the anchor queries (the reference calls
        # select_blocks once per anchor query and ORs the masks)
        q = queries[:, :count].reshape(heads, groups, count, dim)
        return select_blocks_union(q, state.summary, self.config, workspace=state.workspace)

    def _dense_decode(self, module, query, key, value, mask, scaling, kwargs, visible,
                      workspace=None):
        """Dense layers and the dense baseline: SDPA with an explicit additive
        mask over the visible prefix (transformers.py:510-520; the mask-free
        GQA path can round differently in bf16).  With a kernel backend on a
        ROCm device, shapes the dense decode kernel runs go to it instead
        (the same tokens [0, visible), the same default scaling) when the
        model's mask lets the query see exactly those tokens."""
        out = None
        if mask_is_visible_prefix(mask, visible, key.shape[2]):
            out = self._hip_dense_decode(query, key, value, scaling, visible, workspace)
        if out is not None:
            return out, None
        if mask is None:
            mask = query.new_full((1, 1, 1, key.shape[2]), torch.finfo(query.dtype).min)
            mask[..., :visible] = 0
        elif mask.dtype == torch.bool:
            mask = query.new_zeros(mask.shape).masked_fill(~mask, torch.finfo(query.dtype).min)
        return sdpa_attention_forward(module, query, key, value, mask, dropout=0,
                                      scaling=scaling, **kwargs)

    def _hip_dense_decode(self, query, key, value, scaling, visible, workspace):
        """rkv_dense_decode over the visible prefix when the backend allows the
        kernels and the shape is one it runs (bf16, batch 1, head_dim 32..160
        in steps of 32, group <= 16, scaling 1/sqrt(head_dim)); else None."""
        from .. import _hip
        from ..config import KERNEL_BACKENDS

        if workspace is None or self.config.backend not in KERNEL_BACKENDS + ("auto",):
            return None
        if not _hip.is_rocm_device(query):
            return None
        heads, dim = key.shape[1], query.shape[-1]
        group = query.shape[1] // heads
        if (query.shape[0] != 1 or query.shape[2] != 1 or query.shape[1] != heads * group
                or not query.dtype == key.dtype == value.dtype == torch.bfloat16
                or dim % 32 or not 32 <= dim <= _hip.DENSE_MAX_DIM or group > _hip.MAX_GROUP):
            return None
        if scaling is not None and not math.isclose(scaling, dim ** -0.5, rel_tol=1e-6):
            return None
        out = _hip.dense_decode(query[0, :, 0].reshape(heads, group, dim), key[0], value[0],
                                length=visible, workspace=workspace)
        return self._to_model_layout(out.unsqueeze(2), query)

    def _record(self, accessed, dense):
        self._totals["accessed"] = self._totals["accessed"] + accessed
        self._totals["dense"] += dense
        self._totals["decode_attention_calls"] += 1
