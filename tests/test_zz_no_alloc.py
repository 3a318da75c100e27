"""farope_attn_bwd_noalloc (static device workspace, no allocation) against
farope_attn_bwd (caller workspace), both called through the C ABI.

Workspace-path calls in a row (N = 257 at D = 128 through the stored-dS
backward, N = 257 at D = 64 through the split path, then a smaller D = 128
problem) and one one-pass call: the same kernels run with their workspace in
the library's static array instead of a caller buffer, so dQ, dK and dV must
be identical bit for bit.  The second call reuses the array the first one left behind.
The one-pass backward uses no workspace at all, so the no-alloc entry also
takes a one-pass call larger than the static array (4.26 Mi rows).
"""
from __future__ import annotations

import math
import sys

import pytest
import torch

from tests.cases import ROPE_BASE, make_inputs
from triton_fused_rope_flash_attn_amd import CosSinTable
from triton_fused_rope_flash_attn_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _one(B, H, side, has_cls, D, seed):
    N = side * side + int(has_cls)
    print(f"noalloc case B={B} H={H} N={N} D={D}", flush=True)
    sys.stdout.flush()
    cfg = dict(B=B, H=H, side=side, has_cls=has_cls, D=D, dtype=torch.bfloat16, scale=1.0, dout="randn")
    q, k, v, do = make_inputs(cfg, DEV, seed=seed)
    table = CosSinTable(ROPE_BASE, side, D, device=DEV)
    rope = table.packed()
    scale = 1.0 / math.sqrt(D)
    n_pos = side * side
    o, lse, res = torch.ops.farope.attn_fwd(q, k, v, rope, n_pos, has_cls, scale, _lib.BF16)
    desc = _lib.make_desc(B, H, N, D, n_pos, has_cls, _lib.BF16, _lib.BF16, scale)
    ref = [torch.empty_like(q) for _ in range(3)]
    ws = _lib.bwd_workspace_elems(desc)
    delta = torch.empty(ws, device=DEV, dtype=torch.float32) if ws else None
    _lib.attn_bwd(desc, q, k, v, o, do, lse, rope, *ref, delta, res)
    got = [torch.full_like(q, float("nan")) for _ in range(3)]
    _lib.attn_bwd_noalloc(desc, q, k, v, o, do, lse, rope, *got, res)
    torch.cuda.synchronize()
    for name, a, b in zip(("dQ", "dK", "dV"), got, ref):
        assert torch.isfinite(a).all(), name
        assert torch.equal(a, b), f"{name}: max diff {(a.float() - b.float()).abs().max().item():.3e}"
    return _lib.tile_config(desc, 1)[0]


def test_noalloc_one_pass_beyond_static_rows():
    """The one-pass backward keeps delta on chip and needs no workspace, so the
    no-alloc entry takes it at any size: here B*H*N = 4.26 Mi rows, more than
    the static array holds (FAROPE_NOALLOC_MAX_ROWS = 4 Mi).  Inputs are drawn on
    the GPU (any values serve: both entry points see the same ones)."""
    B, H, side, D = 1800, 12, 14, 64
    N = side * side + 1
    assert B * H * N > _lib.NOALLOC_MAX_ROWS
    print(f"noalloc one-pass case B={B} H={H} N={N} D={D}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(31)
    q, k, v, do = (torch.randn(B, H, N, D, device=DEV, generator=g).to(torch.bfloat16) for _ in range(4))
    table = CosSinTable(ROPE_BASE, side, D, device=DEV)
    rope = table.packed()
    scale = 1.0 / math.sqrt(D)
    o, lse, res = torch.ops.farope.attn_fwd(q, k, v, rope, N - 1, True, scale, _lib.BF16)
    desc = _lib.make_desc(B, H, N, D, N - 1, True, _lib.BF16, _lib.BF16, scale)
    assert _lib.tile_config(desc, 1)[0] == 0 and _lib.bwd_workspace_elems(desc) == 0
    ref = [torch.empty_like(q) for _ in range(3)]
    _lib.attn_bwd(desc, q, k, v, o, do, lse, rope, *ref, None, res)
    got = [torch.full_like(q, float("nan")) for _ in range(3)]
    _lib.attn_bwd_noalloc(desc, q, k, v, o, do, lse, rope, *got, res)
    torch.cuda.synchronize()
    for name, a, b in zip(("dQ", "dK", "dV"), got, ref):
        assert torch.isfinite(a).all(), name
        assert torch.equal(a, b), f"{name}: max diff {(a.float() - b.float()).abs().max().item():.3e}"


def test_noalloc_matches_workspace_entry_two_calls():
    # N = 257, D = 128: the stored-dS backward (variant 3: row pass, key tiles
    # that keep dS, dQ GEMM; the last key's partial dK / dV rows and dS, the
    # dS^T and K-hat planes all in the static array)
    assert _one(2, 3, 16, True, 128, seed=24) == 3
    assert _one(4, 6, 16, True, 64, seed=21) == 1    # split path, N = 257
    assert _one(2, 3, 7, True, 128, seed=22) == 3    # smaller, stored-dS path (one ragged key tile)
    assert _one(2, 4, 14, True, 64, seed=23) == 0    # one-pass path (no workspace used)
