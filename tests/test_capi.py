"""The C-ABI library loads and exports every entry point of include/refinekv_hip.h.

CPU only: no call here touches a GPU (rkv_workspace_bytes, rkv_workspace_layout,
rkv_version and rkv_last_error are host functions).
"""

import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "refinekv_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rkv_[a-z_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from refinekv import _hip

    if not os.path.exists(_hip.LIB_PATH):
        pytest.fail("librefinekv_hip.so is not built; run __graft_entry__.build()")
    return _hip.lib()


def test_header_is_valid_c():
    subprocess.run(["gcc", "-std=c99", "-fsyntax-only", "-Wall", "-Werror", "-x", "c", HEADER],
                   check=True)


def test_every_declared_symbol_is_exported(lib):
    names = declared_functions()
    assert {"rkv_summary", "rkv_select", "rkv_decode", "rkv_workspace_bytes",
            "rkv_last_error"} <= set(names)
    for name in names:
        assert hasattr(lib, name), name


def test_version_and_error_channel(lib):
    assert lib.rkv_version() == 2
    assert lib.rkv_workspace_layout(0, 0, 0, 0, None) == 1
    assert b"bad arguments" in lib.rkv_last_error()


def test_speculation_modes(lib):
    """rkv_set_speculation takes 0 (off), 1 (default) and 2 (every shape) and
    rejects anything else with RKV_INVALID_ARGUMENT (host-side only)."""
    from refinekv import _hip

    assert lib.rkv_set_speculation(3) == 1
    assert b"rkv_set_speculation: mode 3" in lib.rkv_last_error()
    assert lib.rkv_set_speculation(-1) == 1
    for mode in (0, 2, 1):
        assert lib.rkv_set_speculation(mode) == 0
    with pytest.raises(ValueError):
        _hip.set_speculation("sometimes")
    _hip.set_speculation(False)
    _hip.set_speculation("auto")


def rows_per_pass(group, dim):
    """Query rows one attention pass of the decode kernels carries: the next
    power of two >= group (at least 4), at most 64 // (dim // 16)."""
    want = 4
    while want < group and want < 16:
        want *= 2
    cap = 16
    while cap > 64 // (dim // 16):
        cap //= 2
    return min(want, cap)


def test_workspace_size_covers_layout(lib):
    from refinekv import _hip

    for heads, group, dim, n in ((8, 4, 128, 4096), (4, 7, 128, 1024), (2, 16, 64, 3),
                                 (1, 1, 256, 1), (8, 4, 128, 8192), (8, 4, 128, 16384),
                                 (3, 4, 128, 11250), (8, 8, 128, 16384), (8, 4, 160, 16384)):
        layout = _hip.workspace_layout(heads, group, dim, n)
        assert _hip.workspace_bytes(heads, group, dim, n) == layout["total"]
        assert layout["n_tiles"] == -(-n // 64)
        regions = [layout[k] for k in _hip.LAYOUT_NAMES[:9]]
        assert regions == sorted(regions) and all(r % 256 == 0 for r in regions)
        rows, tiles, ts = heads * group, layout["n_tiles"], layout["tile_stride"]
        # hand-off counters first: a 64-byte line per KV head, one more, and
        # a launch counter per tile
        assert layout["control"] == 0
        assert layout["zf"] >= (heads + 1) * 64 + heads * layout["tile_stride"] * 8
        # padded strides: zf rows cover whole tiles, per-tile rows 64 tiles
        assert layout["z_stride"] == tiles * 64 and ts % 64 == 0 and ts >= tiles
        assert layout["lse"] - layout["zf"] >= rows * layout["z_stride"] * 16
        assert layout["lse_slots"] - layout["lse"] >= rows * ts * 16
        assert layout["part_ml"] - layout["lse_slots"] >= rows * ts * 32
        assert layout["part_acc"] - layout["part_ml"] >= rows * ts * 8
        assert layout["counts"] - layout["part_acc"] >= rows * ts * dim * 4
        assert layout["full"] - layout["counts"] >= heads * ts * 4
        # the step's per-workgroup speculation flags (u64 each)
        assert layout["total"] - layout["full"] >= heads * ts * 8
        # the one-launch step's workgroups per head: every tile, topped up
        # with copies to min(S / heads, 256), each with a per-tile slot (S =
        # 256 for the 16-row kernels, which hold one workgroup per CU); with
        # more tiles than that, four-row passes up to head_dim 128 keep
        # min(S / heads, 256) workgroups scoring up to 4 tiles each
        want = min((256 if rows_per_pass(group, dim) == 16 else 512) // heads, 256)
        several = (tiles > want and rows_per_pass(group, dim) == 4 and dim <= 128
                   and -(-tiles // want) <= 4)
        assert layout["step_workers"] == (want if several else max(tiles, want))
        assert tiles <= ts and layout["step_workers"] <= ts
    assert _hip.workspace_bytes(0, 4, 128, 10) == 0
