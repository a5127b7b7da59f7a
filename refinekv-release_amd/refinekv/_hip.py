"""ctypes binding of librefinekv_hip.so, the gfx950 kernels behind ``backend="hip"``.

The library's C ABI (declared in include/refinekv_hip.h) takes raw device
pointers, element strides and the current HIP stream; it allocates nothing
and never synchronizes, so calls can be captured in a HIP graph.  This module
owns the per-call plumbing: argument checks the kernels rely on, the
caller-owned workspace, and mapping C error codes to Python exceptions.
There is no fallback: if the library is missing, calls raise.

Hand-off checking: the one-launch decode step's waits are bounded; a wait
that gives up sets a sticky status word in the workspace instead of
hanging.  ``check_workspace`` reads it and raises; with the environment
variable ``REFINEKV_HIP_CHECK=1`` every ``decode`` call checks it (a host
synchronization per call, so not under graph capture).
"""

import ctypes
import os

import torch

LIB_NAME = "librefinekv_hip.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
REDUCTION_CODES = {"mean": 0, "max": 1, "any": 2}  # src/refinekv/kernels/runtime.py:23
DTYPE_CODES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}
SUPPORTED_DIMS = tuple(range(32, 257, 32))
MAX_GROUP = 16

_lib = None
_load_error = None

CHECK_HANDOFFS = os.environ.get("REFINEKV_HIP_CHECK", "0") not in ("", "0")

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_int = ctypes.c_int
_size = ctypes.c_size_t
_u32 = ctypes.c_uint32


class HipUnavailable(RuntimeError):
    pass


def _bind(lib):
    lib.rkv_last_error.restype = ctypes.c_char_p
    lib.rkv_version.restype = _int
    lib.rkv_summary.argtypes = [_p, _i64, _i64, _p, _i64, _i64, _int, _i64, _i64, _i64, _i64, _p,
                                _p, _p, _p, _p, _p, _p]
    lib.rkv_summary.restype = _int
    lib.rkv_summary_store.argtypes = [_p, _i64, _i64, _p, _i64, _i64, _int, _i64, _i64, _i64,
                                      _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _p, _p, _p, _p,
                                      _p, _p]
    lib.rkv_summary_store.restype = _int
    lib.rkv_workspace_bytes.argtypes = [_i64, _i64, _i64, _i64]
    lib.rkv_workspace_bytes.restype = _size
    lib.rkv_workspace_layout.argtypes = [_i64, _i64, _i64, _i64, _p]
    lib.rkv_workspace_layout.restype = _int
    lib.rkv_select.argtypes = [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _int,
                               _p, _p, _p, _p, _p, _p, _size, _p]
    lib.rkv_select.restype = _int
    lib.rkv_select_anchors.argtypes = [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
                                       _f32, _int, _i64, _p, _p, _size, _p]
    lib.rkv_select_anchors.restype = _int
    lib.rkv_decode.argtypes = [_p, _p, _p, _p, _p, _p, _p, _i64, _p, _i64, _p, _i64, _i64, _p,
                               _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64, _f32,
                               _int, _p, _p, _p, _p, _p, _size, _p]
    lib.rkv_decode.restype = _int
    lib.rkv_math_probe.argtypes = [_int, _p, _p, _i64, _p]
    lib.rkv_math_probe.restype = _int
    lib.rkv_set_profile_events.argtypes = [_p]
    lib.rkv_set_profile_events.restype = _int
    lib.rkv_set_decode_path.argtypes = [_int]
    lib.rkv_set_decode_path.restype = _int
    lib.rkv_workspace_status.argtypes = [_p, _size, _i64, _i64, _i64, _i64, _p, _p]
    lib.rkv_workspace_status.restype = _int
    lib.rkv_workspace_clear_status.argtypes = [_p, _size, _i64, _i64, _i64, _i64, _p]
    lib.rkv_workspace_clear_status.restype = _int
    lib.rkv_decode_plan.argtypes = [_i64, _i64, _i64, _i64, _i64, _p]
    lib.rkv_decode_plan.restype = _int
    lib.rkv_set_handoff_test.argtypes = [_u32, _u32]
    lib.rkv_set_handoff_test.restype = _int
    lib.rkv_set_speculation.argtypes = [_int]
    lib.rkv_set_speculation.restype = _int
    lib.rkv_decode_static.argtypes = lib.rkv_decode.argtypes[:-3] + [_p]
    lib.rkv_decode_static.restype = _int
    lib.rkv_static_status.argtypes = [_p, _int, _p]
    lib.rkv_static_status.restype = _int
    lib.rkv_dense_decode.argtypes = [_p, _p, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64,
                                     _p, _p, _p, _size, _p]
    lib.rkv_dense_decode.restype = _int
    lib.rkv_dense_plan.argtypes = [_i64, _i64, _i64, _i64, _p, _p]
    lib.rkv_dense_plan.restype = _int
    return lib


def lib():
    """The loaded library; raises HipUnavailable if it is not built."""
    global _lib, _load_error
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise HipUnavailable(
                f"RefineKV HIP library not built ({LIB_PATH}); run __graft_entry__.build()")
        try:
            _lib = _bind(ctypes.CDLL(LIB_PATH))
        except OSError as error:  # pragma: no cover - depends on the image
            _load_error = error
            raise HipUnavailable(f"cannot load {LIB_PATH}: {error}") from error
    return _lib


def is_rocm_device(tensor):
    return tensor.is_cuda and torch.version.hip is not None


def _check(rc, name):
    if rc:
        message = lib().rkv_last_error().decode(errors="replace")
        if rc in (1, 4):
            raise ValueError(f"{name}: {message}")
        if rc == 2:
            raise TypeError(f"{name}: {message}")
        raise RuntimeError(f"{name}: {message}")


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


# ---------------------------------------------------------------------------
# Summary
# ---------------------------------------------------------------------------

def _row_aligned(t, nbytes):
    """t with dim stride 1, its data pointer and head/token strides multiples
    of ``nbytes`` (a copy only when the view is not)."""
    es = t.element_size()
    ok = (t.stride(-1) == 1 and t.data_ptr() % nbytes == 0
          and all((t.stride(i) * es) % nbytes == 0 for i in range(t.dim() - 1)))
    return t if ok else t.clone(memory_format=torch.contiguous_format)


def summary_fields(keys, values, block, cache_keys=None, cache_values=None):
    """Run the summary kernel on (H, L, D) keys/values; returns the tensors of
    BlockSummary other than the page views.  With cache_keys / cache_values
    ((H, L, D) views of the KV cache, head_dim dense) the same kernel also
    writes every token there (rkv_summary_store)."""
    heads, length, dim = keys.shape
    need = keys.element_size() * (2 if dim <= 128 else 4)
    keys, values = _row_aligned(keys, need), _row_aligned(values, need)
    n_blocks = -(-length // block)
    dev = keys.device
    counts = torch.empty(n_blocks, device=dev, dtype=torch.int64)
    key_mean = torch.empty(heads, n_blocks, dim, device=dev, dtype=torch.bfloat16)
    value_mean = torch.empty_like(key_mean)
    ellipsoid = torch.empty_like(key_mean)
    value_norm = torch.empty(heads, n_blocks, device=dev, dtype=torch.float32)
    max_value_norm = torch.empty(heads, device=dev, dtype=torch.float32)
    outputs = (_ptr(counts), _ptr(key_mean), _ptr(value_mean), _ptr(ellipsoid),
               _ptr(value_norm), _ptr(max_value_norm), _stream(dev))
    sources = (_ptr(keys), keys.stride(0), keys.stride(1), _ptr(values), values.stride(0),
               values.stride(1), DTYPE_CODES[keys.dtype], heads, length, dim, block)
    if cache_keys is None:
        _check(lib().rkv_summary(*sources, *outputs), "rkv_summary")
    else:
        for cache in (cache_keys, cache_values):
            if (cache.shape != keys.shape or cache.dtype != keys.dtype or cache.stride(-1) != 1
                    or cache.device != dev):
                raise ValueError("cache views must match keys/values with a dense head_dim")
        rc = lib().rkv_summary_store(
            *sources, _ptr(cache_keys), cache_keys.stride(0), cache_keys.stride(1),
            _ptr(cache_values), cache_values.stride(0), cache_values.stride(1), *outputs)
        _check(rc, "rkv_summary_store")
    return counts, key_mean, value_mean, ellipsoid, value_norm, max_value_norm


# ---------------------------------------------------------------------------
# Workspace
# ---------------------------------------------------------------------------

def workspace_bytes(heads, group, dim, n_blocks):
    return int(lib().rkv_workspace_bytes(heads, group, dim, n_blocks))


LAYOUT_NAMES = ("control", "zf", "lse", "lse_slots", "part_ml", "part_acc", "counts", "full",
                "total", "n_tiles", "z_stride", "tile_stride", "step_workers")
# rkv_set_decode_path codes: the one-launch step where it fits, or always the
# three kernels (score, attend, merge).
DECODE_PATHS = {"step": 0, "split": 1}


def workspace_layout(heads, group, dim, n_blocks):
    """Byte offsets of the workspace regions (rkv_workspace_layout)."""
    out = (ctypes.c_int64 * len(LAYOUT_NAMES))()
    _check(lib().rkv_workspace_layout(heads, group, dim, n_blocks, out), "rkv_workspace_layout")
    return dict(zip(LAYOUT_NAMES, list(out)))


def _buffer(workspace, name, shape, device, dtype, zero=False):
    """Reusable tensor keyed by name (the reference's workspace dict,
    src/refinekv/kernels/runtime.py:26-37); zero-filled when first made if
    `zero`."""
    tensor = workspace.get(name) if workspace is not None else None
    if (tensor is None or tuple(tensor.shape) != tuple(shape) or tensor.device != device
            or tensor.dtype != dtype):
        tensor = (torch.zeros if zero else torch.empty)(shape, device=device, dtype=dtype)
        if workspace is not None:
            workspace[name] = tensor
    return tensor


def _scratch(workspace, heads, group, dim, n_blocks, device):
    """The kernels' workspace, zero-filled when made for a shape: its first
    region holds the one-launch step's hand-off counters, which count that
    shape's tiles (a new shape gets a new buffer)."""
    shape = (heads, group, dim, n_blocks)
    nbytes = workspace_bytes(*shape)
    tensor = workspace.get("hip_scratch") if workspace is not None else None
    if (tensor is None or workspace.get("hip_scratch_shape") != shape
            or tensor.device != device or tensor.numel() != nbytes):
        tensor = torch.zeros(nbytes, device=device, dtype=torch.uint8)
        if workspace is not None:
            workspace["hip_scratch"] = tensor
            workspace["hip_scratch_shape"] = shape
    return tensor


# ---------------------------------------------------------------------------
# Selection and decode
# ---------------------------------------------------------------------------

def _summary_args(summary):
    return (_ptr(summary.key_mean), _ptr(summary.ellipsoid), _ptr(summary.value_norm),
            _ptr(summary.max_value_norm))


def select(query, summary, config, workspace=None, risk_out=None, stats_out=None,
           accessed=None, anchor_mask=None):
    """Expanded-block mask (H, N) for one query (H, G, 1, D); a fresh tensor."""
    heads, group, _, dim = query.shape
    q = query.reshape(heads * group, dim)
    if not q.is_contiguous():
        q = q.contiguous()
    n_blocks = summary.num_blocks
    scratch = _scratch(workspace, heads, group, dim, n_blocks, query.device)
    mask = torch.empty(heads, n_blocks, device=query.device, dtype=torch.bool)
    anchor = anchor_mask.contiguous() if anchor_mask is not None else None
    rc = lib().rkv_select(
        _ptr(q), *_summary_args(summary), heads, group, dim, n_blocks, summary.block_size,
        summary.prompt_length, float(config.eps), REDUCTION_CODES[config.gqa_reduction],
        _ptr(anchor), _ptr(mask), _ptr(risk_out), _ptr(stats_out), _ptr(accessed),
        _ptr(scratch), scratch.numel(), _stream(query.device))
    _check(rc, "rkv_select")
    return mask


def select_anchors(queries, summary, config, workspace=None):
    """Union of the expanded-block masks of queries (H, G, A, D): one launch
    scores every (query, head, tile), one ORs the decisions.  The scratch is
    its own workspace entry (sized for H * A heads), apart from the decode
    step's."""
    heads, group, count, dim = queries.shape
    q = queries.permute(2, 0, 1, 3).contiguous()  # (A, H, G, D)
    n_blocks = summary.num_blocks
    shape = (heads * count, group, dim, n_blocks)
    nbytes = workspace_bytes(*shape)
    scratch = workspace.get("hip_anchor_scratch") if workspace is not None else None
    if scratch is None or scratch.numel() < nbytes or scratch.device != queries.device:
        scratch = torch.empty(nbytes, device=queries.device, dtype=torch.uint8)
        if workspace is not None:
            workspace["hip_anchor_scratch"] = scratch
    mask = torch.empty(heads, n_blocks, device=queries.device, dtype=torch.bool)
    rc = lib().rkv_select_anchors(
        _ptr(q), *_summary_args(summary), heads, group, dim, n_blocks, summary.block_size,
        summary.prompt_length, float(config.eps), REDUCTION_CODES[config.gqa_reduction], count,
        _ptr(mask), _ptr(scratch), scratch.numel(), _stream(queries.device))
    _check(rc, "rkv_select_anchors")
    return mask


def decode(query, summary, key_suffix, value_suffix, config, anchor_mask=None, workspace=None,
           suffix_length=None, accessed=None):
    """One decode step: returns (output (H, G, 1, D), mask (H, N) bool).

    Both outputs live in ``workspace`` and are overwritten by the next call
    that reuses it (the reference's contract, src/refinekv/attention.py:96-98).
    """
    heads, group, _, dim = query.shape
    device = query.device
    q = query.reshape(heads * group, dim)
    if not q.is_contiguous():
        q = q.contiguous()
    n_blocks = summary.num_blocks
    scratch = _scratch(workspace, heads, group, dim, n_blocks, device)
    mask = _buffer(workspace, "hip_mask", (heads, n_blocks), device, torch.bool)
    output = _buffer(workspace, "hip_output", (heads, group, 1, dim), device, query.dtype)
    ch_bytes = dim // 16 * 2
    need = 16 if ch_bytes % 16 == 0 else (8 if ch_bytes % 8 == 0 else 4)
    key_suffix = _row_aligned(key_suffix, need)
    value_suffix = _row_aligned(value_suffix, need)
    anchor = None
    if anchor_mask is not None:
        anchor = anchor_mask if anchor_mask.is_contiguous() else anchor_mask.contiguous()
    kp, vp = summary.keys, summary.values
    capacity = key_suffix.shape[1]
    rc = lib().rkv_decode(
        _ptr(q), _ptr(summary.key_mean), _ptr(summary.ellipsoid), _ptr(summary.value_mean),
        _ptr(summary.value_norm), _ptr(summary.max_value_norm), _ptr(kp), kp.stride(0), _ptr(vp),
        vp.stride(0), _ptr(key_suffix) if capacity else None, key_suffix.stride(0),
        key_suffix.stride(1), _ptr(value_suffix) if capacity else None, value_suffix.stride(0),
        value_suffix.stride(1), capacity, _ptr(suffix_length), heads, group, dim, n_blocks,
        summary.block_size, summary.prompt_length, float(config.eps),
        REDUCTION_CODES[config.gqa_reduction], _ptr(anchor), _ptr(mask), _ptr(output),
        _ptr(accessed), _ptr(scratch), scratch.numel(), _stream(device))
    _check(rc, "rkv_decode")
    if CHECK_HANDOFFS and not torch.cuda.is_current_stream_capturing():
        check_workspace(workspace if workspace is not None else {"hip_scratch": scratch,
                                                                  "hip_scratch_shape": (
                                                                      heads, group, dim,
                                                                      n_blocks)})
    return output, mask


class HandoffError(RuntimeError):
    """A wait of the one-launch decode step gave up: the call's output and
    mask are not to be trusted."""


def workspace_status(workspace):
    """The sticky hand-off status word of a decode workspace (0 = clean); a
    host synchronization."""
    scratch = workspace.get("hip_scratch") if workspace else None
    if scratch is None:
        return 0
    heads, group, dim, n_blocks = workspace["hip_scratch_shape"]
    word = ctypes.c_uint32()
    _check(lib().rkv_workspace_status(_ptr(scratch), scratch.numel(), heads, group, dim, n_blocks,
                                      ctypes.byref(word), _stream(scratch.device)),
           "rkv_workspace_status")
    return int(word.value)


def clear_workspace_status(workspace):
    scratch = workspace.get("hip_scratch") if workspace else None
    if scratch is None:
        return
    heads, group, dim, n_blocks = workspace["hip_scratch_shape"]
    _check(lib().rkv_workspace_clear_status(_ptr(scratch), scratch.numel(), heads, group, dim,
                                            n_blocks, _stream(scratch.device)),
           "rkv_workspace_clear_status")


def check_workspace(workspace):
    """Raise HandoffError if a decode step on this workspace had a hand-off
    wait give up since the status was last cleared."""
    status = workspace_status(workspace)
    if status & 1:
        raise HandoffError(
            "rkv_decode: a hand-off wait of the one-launch step gave up (its workgroups were "
            "not all running at once); outputs computed with this workspace are invalid")


PLAN_NAMES = {0: "split", 1: "step", 2: "step-ticketed", 3: "step-tiles"}


def decode_plan(heads, group, dim, n_blocks, block):
    """The path rkv_decode takes for a shape on the current device: "split"
    (three kernels), "step" (one launch, grid resident), "step-ticketed"
    (one launch, workgroups mapped by start-order tickets) or "step-tiles"
    (one resident launch, each workgroup scoring several tiles)."""
    mode = ctypes.c_int()
    _check(lib().rkv_decode_plan(heads, group, dim, n_blocks, block, ctypes.byref(mode)),
           "rkv_decode_plan")
    return PLAN_NAMES[mode.value]


def set_handoff_test(spin_limit=0, skew=0):
    """Test hook: the step's poll limit per wait (0 = default) and a skew
    that makes every wait run out (0 = off), for later calls on this thread."""
    _check(lib().rkv_set_handoff_test(spin_limit, skew), "rkv_set_handoff_test")


SPECULATION_MODES = {"off": 0, "auto": 1, "always": 2}


def set_speculation(mode="auto"):
    """Test hook: the one-launch step's speculation (issuing the first page
    rows of a workgroup's tile before the decision when the previous launch
    on the workspace expanded every block of it) for later calls on this
    thread: "off", "auto" (the default) or "always"; True and False mean
    "auto" and "off".  Results are the same bit for bit either way."""
    if isinstance(mode, bool):
        mode = "auto" if mode else "off"
    if mode not in SPECULATION_MODES:
        raise ValueError(f"speculation mode {mode!r}: one of {sorted(SPECULATION_MODES)}")
    _check(lib().rkv_set_speculation(SPECULATION_MODES[mode]), "rkv_set_speculation")


def decode_static(query, summary, key_suffix, value_suffix, config, output, mask,
                  anchor_mask=None, suffix_length=None, accessed=None):
    """decode() through rkv_decode_static: the library's own device scratch,
    no workspace, nothing allocated by the call; output (H, G, 1, D) in the
    query's dtype and mask (H, N) bool are the caller's, contiguous and on
    the query's device (checked before the call: the kernels write them
    whole)."""
    heads, group, _, dim = query.shape
    expect = ((output, (heads, group, 1, dim), query.dtype, "output"),
              (mask, (heads, summary.num_blocks), torch.bool, "mask"))
    for t, shape, dtype, name in expect:
        if tuple(t.shape) != shape or t.dtype != dtype:
            raise ValueError(f"rkv_decode_static: {name} must be {shape} {dtype}, "
                             f"got {tuple(t.shape)} {t.dtype}")
        if t.device != query.device or not t.is_contiguous():
            raise ValueError(f"rkv_decode_static: {name} must be contiguous on {query.device}")
    if accessed is not None and (accessed.dtype != torch.int64 or accessed.numel() < 1 or
                                 accessed.device != query.device):
        raise ValueError("rkv_decode_static: accessed must be an int64 tensor on the query's "
                         "device")
    q = query.reshape(heads * group, dim)
    if not q.is_contiguous():
        q = q.contiguous()
    kp, vp = summary.keys, summary.values
    capacity = key_suffix.shape[1]
    rc = lib().rkv_decode_static(
        _ptr(q), _ptr(summary.key_mean), _ptr(summary.ellipsoid), _ptr(summary.value_mean),
        _ptr(summary.value_norm), _ptr(summary.max_value_norm), _ptr(kp), kp.stride(0), _ptr(vp),
        vp.stride(0), _ptr(key_suffix) if capacity else None, key_suffix.stride(0),
        key_suffix.stride(1), _ptr(value_suffix) if capacity else None, value_suffix.stride(0),
        value_suffix.stride(1), capacity, _ptr(suffix_length), heads, group, dim,
        summary.num_blocks, summary.block_size, summary.prompt_length, float(config.eps),
        REDUCTION_CODES[config.gqa_reduction], _ptr(anchor_mask), _ptr(mask), _ptr(output),
        _ptr(accessed), _stream(query.device))
    _check(rc, "rkv_decode_static")
    return output, mask


def static_status(clear=False):
    """The status word of rkv_decode_static's scratch on the current device
    (bit 0: a hand-off wait of a static call gave up since the last clear;
    that call wrote NaN output rows and an all-expanded mask); a host
    synchronization.  clear=True zeroes it after reading."""
    word = ctypes.c_uint32()
    device = torch.device("cuda", torch.cuda.current_device())
    _check(lib().rkv_static_status(ctypes.byref(word), 1 if clear else 0, _stream(device)),
           "rkv_static_status")
    return int(word.value)


# ---------------------------------------------------------------------------
# Dense decode
# ---------------------------------------------------------------------------

DENSE_MAX_DIM = 160


def dense_plan(heads, group, dim, length):
    """(splits, workspace bytes) of rkv_dense_decode for this shape on the
    current device."""
    splits, nbytes = ctypes.c_int64(), ctypes.c_size_t()
    _check(lib().rkv_dense_plan(heads, group, dim, length, ctypes.byref(splits),
                                ctypes.byref(nbytes)), "rkv_dense_plan")
    return int(splits.value), int(nbytes.value)


def dense_decode(query, keys, values, length=None, workspace=None, output=None):
    """Full attention of one query token per row over every cached token.

    query (H, G, D) or (H, G, 1, D) bf16; keys/values (H, T, D) bf16 views
    (head_dim dense, e.g. ``cache[0]`` of a (1, H, T, D) Transformers cache).
    ``length``: None attends all T tokens; an int attends the first `length`;
    a device int32 scalar attends the first min(max(length, 0), T) tokens as
    read when the kernel runs (graph replays).  Returns (H, G, D) bf16 (the
    ``output`` tensor when given), computed by rkv_dense_decode and
    merge of its per-split partials; the partials live in ``workspace``.
    """
    heads, group, dim = query.shape[0], query.shape[1], query.shape[-1]
    device = query.device
    if not query.dtype == keys.dtype == values.dtype == torch.bfloat16:
        raise TypeError("rkv_dense_decode: query, keys and values must be bfloat16")
    q = query.reshape(heads, group, dim)
    if not q.is_contiguous():
        q = q.contiguous()
    capacity = keys.shape[1]
    length_dev = None
    if isinstance(length, torch.Tensor):
        length_dev, cap = length, capacity
    else:
        cap = capacity if length is None else int(length)
        if not 0 < cap <= capacity:
            raise ValueError(f"length {length} outside 1..{capacity}")
    keys, values = _row_aligned(keys, 16), _row_aligned(values, 16)
    _, nbytes = dense_plan(heads, group, dim, cap)
    scratch = _buffer(workspace, "hip_dense_scratch", (nbytes,), device, torch.uint8)
    if output is None:
        output = torch.empty(heads, group, dim, device=device, dtype=query.dtype)
    rc = lib().rkv_dense_decode(
        _ptr(q), _ptr(keys), keys.stride(0), keys.stride(1), _ptr(values), values.stride(0),
        values.stride(1), heads, group, dim, cap, _ptr(length_dev), _ptr(output), _ptr(scratch),
        scratch.numel(), _stream(device))
    _check(rc, "rkv_dense_decode")
    return output


def set_decode_path(name):
    """Test hook: "step" (default) or "split" for later decode calls on this
    thread."""
    _check(lib().rkv_set_decode_path(DECODE_PATHS[name]), "rkv_set_decode_path")


def math_probe(fn, x):
    """Device scalar functions for tests: fn in {'exp', 'log', 'bf16', 'sqrt'}
    (the oracle's forms) and {'exp_hw', 'log_hw'} (the selection kernels')."""
    code = {"exp": 0, "log": 1, "bf16": 2, "sqrt": 3, "exp_hw": 4, "log_hw": 5}[fn]
    x = x.contiguous().float()
    y = torch.empty_like(x)
    _check(lib().rkv_math_probe(code, _ptr(x), _ptr(y), x.numel(), _stream(x.device)),
           "rkv_math_probe")
    return y
