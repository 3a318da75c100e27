"""The C ABI library: loads, exports every symbol include/farope.h declares,
and rejects bad arguments on the host before launching anything.

No call here reaches a kernel launch (no GPU in the CPU tier): only the
host-only functions and argument-error paths are exercised.
"""
from __future__ import annotations

import ctypes
import os
import re

import pytest

from triton_fused_rope_flash_attn_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "farope.h")


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        from triton_fused_rope_flash_attn_amd import build

        build.build()
    return _lib.load()


def _header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(farope_[a-z_0-9]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert sorted(_lib.EXPORTS) == _header_functions()


def test_library_exports_every_header_symbol(lib):
    for name in _header_functions():
        assert hasattr(lib, name), name


def test_abi_version_matches_header(lib):
    m = re.search(r"#define FAROPE_ABI_VERSION (\d+)", open(HEADER).read())
    assert lib.farope_abi_version() == int(m.group(1))


def test_desc_struct_layout():
    assert ctypes.sizeof(_lib.AttnDesc) == 9 * 4


def test_strerror_covers_all_codes(lib):
    texts = {rc: _lib.strerror(rc) for rc in range(0, 10)}
    assert texts[0] == "success"
    assert len(set(texts.values())) == 10
    assert "unknown" in _lib.strerror(1234)


def test_rope_packed_elems(lib):
    assert lib.farope_rope_packed_elems(196, 32) == 197 * 32 * 2
    assert lib.farope_rope_packed_elems(1024, 64) == 1025 * 128


@pytest.mark.parametrize(
    "N,D,has_cls,fwd_var,fwd_items,bwd_var",
    [(197, 64, 1, 1, 1, 0), (208, 64, 0, 1, 1, 0), (192, 64, 1, 0, 1, 0), (256, 64, 0, 0, 1, 0),
     (257, 64, 1, 0, 1, 1), (1025, 128, 1, 0, 4, 3), (197, 128, 1, 0, 1, 3),
     (197, 256, 1, 0, 3, 1), (257, 256, 1, 0, 4, 1), (1100, 128, 1, 0, 5, 3),
     (3970, 128, 1, 0, 16, 2)],
)
def test_tile_table(lib, N, D, has_cls, fwd_var, fwd_items, bwd_var):
    """Forward variant 1 (one wave per plane) covers planes of 193 .. 208 tokens at D = 64."""
    desc = _lib.make_desc(8, 12, N, D, N - has_cls, has_cls, _lib.BF16, _lib.BF16, D ** -0.5)
    f = _lib.tile_config(desc, 0)
    b = _lib.tile_config(desc, 1)
    assert f[0] == fwd_var and f[2] == fwd_items and b[0] == bwd_var
    for t in (f, b):
        left = N - t[1] * t[2]               # rows for the tail kernels (at most 8)
        assert left <= 8 and t[2] >= 1
        assert left > 0 or (t[2] - 1) * t[1] < N   # otherwise: no empty block
    assert f[3] % 64 == 0 and b[3] % 64 == 0


def _ds_elems(B, H, N, D):
    """Workspace of the stored-dS backward (None where it does not apply: more
    than one key past the 128-key tiles, or a dS^T plane larger than 16 Q
    planes), in fp32 elements, each part from a
    64-float boundary: delta rows; with a lone last key one partial dK / dV
    row pair per 64-row tile; fp16 Q-hat rows; {|dO|, max |Q-hat|} per row;
    with a lone last key its dS per row; an int32 exponent per key tile; fp16
    K-hat rows of the key tiles; fp16 dS^T rows of the key tiles (pitch N
    rounded up to 64)."""
    r = N % 128
    t = r if N >= 128 and 0 < r <= 8 else 0
    if t > 1:
        return None
    n_kt = N // 128 if t else -(-N // 128)
    if n_kt * 128 * ((N + 63) // 64 * 64) > 16 * N * D:   # dS^T plane > 16 Q planes
        return None
    planes, rows = B * H, B * H * N
    kp, n_pt, nqp = n_kt * 128, -(-N // 64), (N + 63) // 64 * 64

    def al(x):
        return (x + 63) // 64 * 64

    xk = al(rows)
    hat = al(xk + (planes * n_pt * 2 * D if t else 0))
    stat = al(hat + rows * D // 2)
    dsl = al(stat + 2 * rows)
    kexp = al(dsl + (rows if t else 0))
    khat = al(kexp + planes * n_kt)
    dst = al(khat + planes * kp * D // 2)
    return dst + planes * kp * nqp // 2


@pytest.mark.parametrize(
    "B,H,N,D,io,ct,extra,hat",
    [
        (32, 12, 1025, 128, _lib.BF16, _lib.BF16, 4 * 2 * 128, True),   # HiRes: 4 dQ tiles per plane
        (2, 3, 257, 256, _lib.BF16, _lib.BF16, 4 * 2 * 256, True),      # 64-row dQ tiles
        (2, 3, 257, 128, _lib.F16, _lib.BF16, 1 * 2 * 128, True),       # fp16 I/O, bf16 compute
        (256, 12, 197, 64, _lib.BF16, _lib.BF16, None, False),          # one-pass backward: none
        (1800, 12, 197, 64, _lib.BF16, _lib.BF16, None, False),         # (> 4 Mi rows, still none)
        (4, 2, 2, 64, _lib.F16, _lib.F16, None, False),                 # N = 2, fp16: one-pass
        (2, 3, 257, 64, _lib.BF16, _lib.BF16, 0, False),                # no fp16 logits at D = 64
        (2, 3, 257, 128, _lib.F16, _lib.F16, 0, False),                 # fp16 compute
        (2, 3, 1100, 128, _lib.BF16, _lib.BF16, 0, True),               # 76 rows past the blocks
        (2, 3, 3970, 128, _lib.BF16, _lib.BF16, 0, True),               # dQ blocks leave 130 rows
     (1, 2, 4097, 128, _lib.BF16, _lib.BF16, 16 * 2 * 128, True),    # N = 4097: split path (dS^T > 16 Q planes)
        (1, 2, 3844, 128, _lib.BF16, _lib.BF16, 0, False),              # 4 tail rows: tail kernel
    ],
)
def test_bwd_workspace_elems(lib, B, H, N, D, io, ct, extra, hat):
    """No workspace for the one-pass backward (extra None: delta stays on chip).
    Otherwise delta rows; one partial dK / dV row pair per dQ tile when the
    plane's lone last key is summed by those tiles (fp16 logits, N = 1 + k * 256);
    then, from a 64-float boundary, the dQ pass's fp16 Q-hat rows for the dK/dV
    pass (fp16 logits, every row in a dQ tile); then, for the key-tile kernel
    with fp16 dS products (those shapes at head_dim 128), from a 64-float
    boundary, a {|dO|, max |Q-hat|} pair per row."""
    desc = _lib.make_desc(B, H, N, D, N - 1, True, io, ct, D ** -0.5)
    if extra is None:
        assert _lib.tile_config(desc, 1)[0] == 0
        assert _lib.bwd_workspace_elems(desc) == 0
        return
    n = B * H * N + B * H * extra
    if hat:
        n = (n + 63) // 64 * 64 + B * H * N * D // 2
    if hat and D == 128:
        n = (n + 63) // 64 * 64 + 2 * B * H * N
        ds = _ds_elems(B, H, N, D)
        if ds is not None:   # the stored-dS backward: the larger of the two layouts
            assert _lib.tile_config(desc, 1)[0] == 3
            n = max(n, ds)
        else:
            assert _lib.tile_config(desc, 1)[0] == 2
    assert _lib.bwd_workspace_elems(desc) == n
    bad = _lib.make_desc(B, H, N, 60, N - 1, True, io, ct, 0.125)
    assert _lib.bwd_workspace_elems(bad) == 0


def test_fp32_compute_takes_split_backward(lib):
    desc = _lib.make_desc(8, 12, 197, 64, 196, 1, _lib.F32, _lib.F32, 0.125)
    assert _lib.tile_config(desc, 1)[0] == 1


ROPE_ELEMS = 197 * 64   # farope_rope_packed_elems(196, 32): the table of the descriptors below


def _call_fwd(lib, desc, q=16, lse=16, rope=16, rope_elems=ROPE_ELEMS):
    s = _lib.Stride4(0, 0, 0, 1)
    return lib.farope_attn_fwd(
        ctypes.byref(desc) if desc is not None else None,
        q, s, 16, s, 16, s, rope, rope_elems, 16, s, None, lse, None,
    )


@pytest.mark.parametrize(
    "kwargs,expect",
    [
        (dict(D=66), _lib.ERR_HEAD_DIM),
        (dict(D=96), _lib.ERR_HEAD_DIM),
        (dict(D=512), _lib.ERR_HEAD_DIM),
        (dict(N=198), _lib.ERR_SEQ_LEN),
        (dict(io=7), _lib.ERR_DTYPE),
        (dict(ct=9), _lib.ERR_DTYPE),
        (dict(B=0), _lib.ERR_SHAPE),
    ],
)
def test_fwd_rejects_bad_descriptors(lib, kwargs, expect):
    a = dict(B=2, H=3, N=197, D=64, io=_lib.BF16, ct=_lib.BF16)
    a.update(kwargs)
    desc = _lib.make_desc(a["B"], a["H"], a["N"], a["D"], 196, True, a["io"], a["ct"], 0.125)
    assert _call_fwd(lib, desc) == expect


def test_fwd_rejects_null_and_misaligned(lib):
    assert _call_fwd(lib, None) == _lib.ERR_NULL
    desc = _lib.make_desc(2, 3, 197, 64, 196, True, _lib.BF16, _lib.BF16, 0.125)
    assert _call_fwd(lib, desc, q=None) == _lib.ERR_NULL
    assert _call_fwd(lib, desc, q=17) == _lib.ERR_ALIGN       # bf16 needs 2-byte alignment
    assert _call_fwd(lib, desc, rope=24) == _lib.ERR_ALIGN    # table needs 16-byte alignment


def test_fwd_rejects_a_table_of_another_geometry(lib):
    """rope_elems must be farope_rope_packed_elems(n_pos, head_dim / 2)."""
    desc = _lib.make_desc(2, 3, 197, 64, 196, True, _lib.BF16, _lib.BF16, 0.125)
    assert lib.farope_rope_packed_elems(196, 32) == ROPE_ELEMS
    for n in (0, ROPE_ELEMS - 2, ROPE_ELEMS + 64, 197 * 128, 196 * 64):
        assert _call_fwd(lib, desc, rope_elems=n) == _lib.ERR_TABLE
    assert _call_fwd(lib, desc, rope=None) == _lib.ERR_NULL


def _bwd(lib, desc, o_res=None, lse=16, rope=16, rope_elems=ROPE_ELEMS, dq=16, delta=16):
    """farope_attn_bwd with placeholder (never dereferenced) device pointers."""
    s = _lib.Stride4(0, 0, 0, 1)
    return lib.farope_attn_bwd(ctypes.byref(desc), 16, s, 16, s, 16, s, 16, s, o_res, 16, s, lse,
                               rope, rope_elems, dq, s, 16, s, 16, s, delta, None)


def _bwd_dq(lib, desc, delta=16, rope_elems=ROPE_ELEMS):
    s = _lib.Stride4(0, 0, 0, 1)
    return lib.farope_attn_bwd_dq(ctypes.byref(desc), 16, s, 16, s, 16, s, 16, s, 16, delta, 16,
                                  rope_elems, 16, s, None)


def _bwd_dk_dv(lib, desc, dv=16, rope_elems=ROPE_ELEMS):
    s = _lib.Stride4(0, 0, 0, 1)
    return lib.farope_attn_bwd_dk_dv(ctypes.byref(desc), 16, s, 16, s, 16, s, 16, s, 16, 16, 16,
                                     rope_elems, 16, s, dv, s, None)


def _bwd_noalloc(lib, desc, rope_elems):
    s = _lib.Stride4(0, 0, 0, 1)
    return lib.farope_attn_bwd_noalloc(ctypes.byref(desc), 16, s, 16, s, 16, s, 16, s, None, 16, s,
                                       16, 16, rope_elems, 16, s, 16, s, 16, s, None)


def test_bwd_entry_points_reject_bad_arguments(lib):
    s = _lib.Stride4(0, 0, 0, 1)
    bad = _lib.make_desc(2, 3, 197, 60, 196, True, _lib.BF16, _lib.BF16, 0.125)
    assert _bwd(lib, bad) == _lib.ERR_HEAD_DIM
    good = _lib.make_desc(2, 3, 197, 64, 196, True, _lib.BF16, _lib.BF16, 0.125)
    assert _bwd(lib, good, lse=None) == _lib.ERR_NULL
    assert _bwd(lib, good, dq=24 + 1) == _lib.ERR_ALIGN
    assert _bwd(lib, good, rope=24) == _lib.ERR_ALIGN
    assert _bwd(lib, good, rope_elems=ROPE_ELEMS + 2) == _lib.ERR_TABLE
    assert lib.farope_attn_bwd_preprocess(ctypes.byref(bad), 16, s, None, 16, s, 16, None) == _lib.ERR_HEAD_DIM
    assert _bwd_dq(lib, good, delta=3) == _lib.ERR_ALIGN
    assert _bwd_dq(lib, good, rope_elems=1) == _lib.ERR_TABLE
    assert _bwd_dk_dv(lib, good, dv=None) == _lib.ERR_NULL
    assert _bwd_dk_dv(lib, good, rope_elems=196 * 64) == _lib.ERR_TABLE
    assert lib.farope_rope_pack(16, 32, 1, 16, 32, 1, 196, 31, 16, None) == _lib.ERR_TABLE
    assert lib.farope_rope_pack(None, 32, 1, 16, 32, 1, 196, 32, 16, None) == _lib.ERR_NULL


def test_noalloc_bwd_rejects_oversize_before_any_launch(lib):
    """farope_attn_bwd_noalloc refuses calls whose B*H*N exceeds its static
    workspace (FAROPE_NOALLOC_MAX_ROWS) with FAROPE_ERR_SCRATCH, on the host."""
    m = re.search(r"#define FAROPE_NOALLOC_MAX_ROWS (\d+)", open(HEADER).read())
    assert int(m.group(1)) == _lib.NOALLOC_MAX_ROWS
    N = 1025   # split path; 4096 planes x 1025 rows > 4 Mi rows
    big = _lib.make_desc(64, 64, N, 128, N - 1, True, _lib.BF16, _lib.BF16, 128 ** -0.5)
    assert 64 * 64 * N > _lib.NOALLOC_MAX_ROWS
    assert _bwd_noalloc(lib, big, lib.farope_rope_packed_elems(N - 1, 64)) == _lib.ERR_SCRATCH
    bad = _lib.make_desc(2, 3, 197, 60, 196, True, _lib.BF16, _lib.BF16, 0.125)
    assert _bwd_noalloc(lib, bad, ROPE_ELEMS) == _lib.ERR_HEAD_DIM
    assert "static workspace" in _lib.strerror(_lib.ERR_SCRATCH)
