"""Resources and index ranges of the built gfx950 kernels, checked on the CPU.

The kernel metadata (LDS bytes, scratch bytes per lane, VGPRs) is read from
the code objects inside this repository's own librefinekv_hip.so with the
ROCm LLVM tools; nothing is launched.  The index-range part restates, for
one shape, the address arithmetic of the kernels rkv_decode runs for it and
checks every access against its buffer's size: the head_dim-256 / block-64
decode shape (2 KV heads, group 4, 999 prompt tokens = 16 blocks) that
faulted the GPU with an earlier persistent kernel.
"""

import os
import re
import struct
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "refinekv-release_amd", "refinekv", "librefinekv_hip.so")
LLVM = "/opt/rocm/llvm/bin"
LDS_PER_WORKGROUP = 160 * 1024  # gfx950: a workgroup may take all of a CU's LDS

needs_tools = pytest.mark.skipif(
    not (os.path.exists(LIB) and os.path.exists(os.path.join(LLVM, "llvm-readelf"))),
    reason="needs the built library and the ROCm LLVM tools")


def _code_objects(tmp_path):
    """The gfx950 code objects of the library's .hip_fatbin section (one
    offload bundle per source file)."""
    fatbin = tmp_path / "fatbin.bin"
    subprocess.run([os.path.join(LLVM, "llvm-objcopy"), f"--dump-section=.hip_fatbin={fatbin}",
                    LIB, str(tmp_path / "stripped.so")], check=True)
    data = fatbin.read_bytes()
    magic = b"__CLANG_OFFLOAD_BUNDLE__"
    objects, pos = [], 0
    while (start := data.find(magic, pos)) >= 0:
        (entries,) = struct.unpack_from("<Q", data, start + len(magic))
        at = start + len(magic) + 8
        for _ in range(entries):
            offset, size, triple_len = struct.unpack_from("<QQQ", data, at)
            at += 24
            triple = data[at:at + triple_len].decode()
            at += triple_len
            if triple.endswith("gfx950"):
                path = tmp_path / f"co{len(objects)}.elf"
                path.write_bytes(data[start + offset:start + offset + size])
                objects.append(path)
        pos = start + 1
    return objects


@pytest.fixture(scope="module")
def kernels(tmp_path_factory):
    """{mangled kernel name: {lds, scratch, vgpr, spill}} for every kernel."""
    if not (os.path.exists(LIB) and os.path.exists(os.path.join(LLVM, "llvm-readelf"))):
        pytest.skip("needs the built library and the ROCm LLVM tools")
    table = {}
    for obj in _code_objects(tmp_path_factory.mktemp("co")):
        notes = subprocess.run([os.path.join(LLVM, "llvm-readelf"), "--notes", str(obj)],
                               check=True, capture_output=True, text=True).stdout
        for block in notes.split("  - .agpr_count")[1:]:
            def field(key):
                return int(re.search(r"\." + key + r":\s+(\d+)", block).group(1))
            name = re.search(r"\.name:\s+(\S+)", block).group(1)
            table[name] = dict(lds=field("group_segment_fixed_size"),
                               scratch=field("private_segment_fixed_size"),
                               vgpr=field("vgpr_count"), spill=field("vgpr_spill_count"),
                               obj=str(obj))
    assert table, "no kernels found in the library"
    return table


def _scratch_instructions(res, name):
    """Scratch accesses in a kernel's own disassembly (its frame may hold
    dead SGPR-spill slots the backend reserves after placing every spill in
    VGPR lanes: a private segment no instruction touches)."""
    text = subprocess.run([os.path.join(LLVM, "llvm-objdump"), "-d",
                           f"--disassemble-symbols={name}", res["obj"]],
                          check=True, capture_output=True, text=True).stdout
    assert name in text, name
    return [l for l in text.splitlines() if re.search(r"\bscratch_(load|store)", l)]


def _instances(kernels, family):
    """(template arguments, resources) of one kernel family; the arguments
    are the integers (and 0/1 bools) of its mangled name."""
    out = []
    for name, res in kernels.items():
        m = re.search(family + r"I((?:L[ib]\d+E)+)E", name)
        if m:
            out.append((tuple(int(x) for x in re.findall(r"L[ib](\d+)E", m.group(1))), res))
    return out


def _name_of(kernels, family, args):
    for name in kernels:
        m = re.search(family + r"I((?:L[ib]\d+E)+)E", name)
        if m and tuple(int(x) for x in re.findall(r"L[ib](\d+)E", m.group(1))) == args:
            return name
    raise KeyError((family, args))


@needs_tools
def test_step_kernel_exists_only_up_to_head_dim_128(kernels):
    dims = {args[0] for args, _ in _instances(kernels, "step_kernel")}
    assert dims == {32, 64, 96, 128}, dims


@needs_tools
def test_no_scratch_in_the_kernels_of_common_shapes(kernels):
    """Scratch (register spills or dynamically indexed arrays) is allowed
    only in the 16-row builds (GQA groups above 8) and the head_dim-160
    attend kernel (its two rings of five-operand chunks spill 9 registers);
    every other decode and summary kernel runs without it (the 8-row steps
    score one query row's slice of q at a time: holding four rows' across
    both passes spilled at head_dim 128)."""
    allowed = {("attend_kernel", (160, 4))}
    for family in ("step_kernel", "attend_kernel", "score_kernel", "summary_kernel"):
        for args, res in _instances(kernels, family):
            rows16 = family in ("step_kernel", "attend_kernel") and args[1] == 16
            if rows16 or (family, args) in allowed:
                continue
            assert res["spill"] == 0, (family, args, res)
            if res["scratch"]:
                assert not _scratch_instructions(res, _name_of(kernels, family, args)), (
                    family, args, res)
    for name, res in kernels.items():
        if any(k in name for k in ("merge_kernel", "decide_kernel", "anchor_decide_kernel")):
            assert res["scratch"] == 0, (name, res)


@needs_tools
def test_lds_of_every_kernel_fits_a_workgroup(kernels):
    for name, res in kernels.items():
        assert res["lds"] <= LDS_PER_WORKGROUP, (name, res)


# ---------------------------------------------------------------------------
# The head_dim-256, block-64 decode shape, restated on the CPU
# ---------------------------------------------------------------------------

H, G, D, B, L = 2, 4, 256, 64, 999
N = -(-L // B)                 # 16 blocks; the last holds 999 - 15 * 64 = 39 tokens
TILE, THREADS = 64, 256


def _score_smem(group, dim):
    """score_kernel's dynamic LDS (rkv_decode.hip score_smem)."""
    lanes = 8 if dim <= 128 else 16
    q_floats = 2 * group * (dim + lanes * 4)
    return 4 * (2 * group * TILE + q_floats)


@needs_tools
def test_head_dim_256_block_64_shape_takes_the_three_kernels_within_limits(kernels):
    """Its kernels: score_kernel<256> (dynamic LDS), attend_kernel<256, 4>,
    merge_kernel; none uses scratch, and each one's LDS fits."""
    (score,) = [r for a, r in _instances(kernels, "score_kernel") if a == (256,)]
    (attend,) = [r for a, r in _instances(kernels, "attend_kernel") if a == (256, 4)]
    assert score["scratch"] == attend["scratch"] == 0
    assert score["lds"] + _score_smem(G, D) <= LDS_PER_WORKGROUP
    assert attend["lds"] <= LDS_PER_WORKGROUP
    assert 256 not in {a[0] for a, _ in _instances(kernels, "step_kernel")}


def test_head_dim_256_block_64_index_ranges():
    """Every address the three kernels form for this shape, from their index
    arithmetic (rkv_decode.hip: score_dots, score_stats, decide_issue,
    attend_issue, attend_tile, merge_kernel), lies inside its buffer."""
    T = -(-N // TILE)                       # 1 tile
    tile_stride = 64                        # per-tile arrays: whole tiles of 64
    z_stride = T * TILE
    lanes, ch = 16, 16                      # Dots<256>: 16 lanes x 16 columns per block
    per_pass = THREADS // lanes
    passes = TILE // per_pass
    tid = np.arange(THREADS)
    for h in range(H):
        for tile in range(T):
            # score_dots: summary rows, clamped to the last block
            c, sub = tid % lanes, tid // lanes
            for ps in range(passes):
                b = np.minimum(tile * TILE + ps * per_pass + sub, N - 1)
                off = (h * N + b) * D + c * ch
                assert off.min() >= 0 and (off + ch).max() <= H * N * D
            # query words (two bf16 per word) of head h, staged into LDS
            words = np.arange(G * D // 2)
            assert (h * G * D) // 2 + words.max() < H * G * D // 2
            qw, qs = ch + 4, lanes * (ch + 4)
            g, e = 2 * words // D, 2 * words % D
            at = g * qs + (e // ch) * qw + e % ch
            assert at.max() + 1 < G * qs
            # score_stats: z row entries of valid blocks, one LSE partial per row
            lane = tid % 64
            b = tile * TILE + lane
            zrow = (h * G + np.arange(G))[:, None] * z_stride + b[None, b < N]
            assert zrow.max() < H * G * z_stride
            assert ((h * G + G - 1) * tile_stride + tile) * 4 + 3 < H * G * tile_stride * 4
            # attend: value means of the lane group's blocks (clamped)
            lg, cc = tid >> 4, tid & 15
            for i in range(TILE // 16):
                bb = np.minimum(tile * TILE + lg + 16 * i, N - 1)
                off = (h * N + bb) * D + cc * ch
                assert (off + ch).max() <= H * N * D
            # expanded rows of this tile's blocks: every block may expand
            list_ = np.arange(min(TILE, N - tile * TILE))
            rows = np.arange(len(list_) * B)
            block = tile * TILE + list_[rows >> 6]
            tok = rows & (B - 1)
            off = ((block << 6) + tok) * D + cc.max() * ch
            assert (off + ch).max() <= N * B * D           # the padded pages of one head
            last_live = (block != N - 1) | (tok < L - (N - 1) * B)
            assert last_live.sum() == L - tile * TILE * B  # masked rows: the padding only
            # combine buffer (CombineShared<256, 4>: 2 rows per chunk, slice 20)
            k_rows, slice_ = min(512 // D, G), D // 16 + 4
            idx = np.arange(0, k_rows * D, 2)
            d = idx % D
            at_d = (d // ch) * slice_ + d % ch
            assert at_d.max() + 1 < 16 * slice_
            # the tile's partials
            at = (h * G + G - 1) * tile_stride + tile
            assert (at + 1) * D <= H * G * tile_stride * D
    # merge_kernel: rows x 32-column slices over the T partials
    r = np.arange(H * G)[:, None]
    d = np.arange(0, D)[None, :]
    assert ((r * tile_stride + T - 1) * D + d).max() < H * G * tile_stride * D
    assert (r * D + d).max() < H * G * D


# Instructions that count in lgkmcnt (LDS, scalar memory, messages).
_LGKM = re.compile(r"^(ds_|s_load|s_buffer_load|s_memrealtime|s_memtime|s_sendmsg|s_dcache)")


def _vregs(operand):
    operand = operand.strip()
    m = re.match(r"v\[(\d+):(\d+)\]$", operand)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", operand)
    return {int(m.group(1))} if m else set()


def _unwaited_transposed_reads(lines):
    """Transposing LDS reads (ds_read_b64_tr_b16) whose destination registers
    are read or overwritten, or whose block is left, before an s_waitcnt
    lgkmcnt(k) that covers them (k at most the lgkmcnt operations issued
    after the read).  The fold issues these reads from inline asm, which the
    compiler does not see as loads: a copy it placed between a read and its
    wait would take the registers before the data lands."""
    ins = []
    for line in lines:
        m = re.match(r"\s+([a-z_0-9]+)\s*(.*?)\s*(//.*)?$", line)
        if m:
            ins.append((m.group(1), m.group(2)))
        elif line.strip().endswith(":"):
            ins.append(("<label>", ""))
    bad = []
    for i, (op, args) in enumerate(ins):
        if op != "ds_read_b64_tr_b16":
            continue
        dst, after = _vregs(args.split(",")[0]), 0
        for op2, args2 in ins[i + 1:]:
            if op2 in ("<label>", "s_branch", "s_setpc_b64") or op2.startswith("s_cbranch"):
                bad.append((i, op2))
                break
            if op2 == "s_waitcnt":
                m = re.search(r"lgkmcnt\((\d+)\)", args2)
                if m and int(m.group(1)) <= after:
                    break
            ops = args2.split(",")
            writes = not op2.startswith(("s_", "buffer_store", "global_store", "ds_write"))
            srcs = set().union(*(_vregs(o) for o in (ops[1:] if writes else ops)))
            if srcs & dst or (writes and _vregs(ops[0]) & dst):
                bad.append((i, f"{op2} {args2}"))
                break
            if _LGKM.match(op2):
                after += 1
    return bad


@needs_tools
def test_transposed_reads_are_waited_for_before_use(kernels):
    """Every asm-issued transposing LDS read of the step, attend and dense
    kernels is covered by its lgkmcnt wait before anything touches its
    registers (checked on this repository's own gfx950 disassembly)."""
    checked = 0
    for obj in sorted({res["obj"] for res in kernels.values()}):
        text = subprocess.run([os.path.join(LLVM, "llvm-objdump"), "-d", obj],
                              check=True, capture_output=True, text=True).stdout
        for block in re.split(r"\n(?=[0-9a-f]{16} <)", text):
            m = re.match(r"[0-9a-f]{16} <([^>]+)>:", block)
            if not m or "ds_read_b64_tr_b16" not in block:
                continue
            assert not _unwaited_transposed_reads(block.splitlines()[1:]), m.group(1)
            checked += block.count("ds_read_b64_tr_b16")
    assert checked > 0
