"""GPU parity: the HIP kernels (through the C ABI) vs the fp32 PyTorch oracle.

Oracle: Python 2D RoPE + torch SDPA (math backend) in fp32 on the GPU,
from the same seeded inputs (cast to fp32) and the same CosSinTable.
Tolerance (north star): O/dQ/dK/dV max_abs_err <= 3e-2 and
mean_abs_err <= 1e-3 (TOL_MAX / TOL_MEAN in tests/cases.py).
"""
from __future__ import annotations

import math
import sys

import pytest
import torch

from oracle import torch_ref
from tests.cases import (CONFIGS, ROPE_BASE, TOL_MAX, TOL_MEAN, allowed, errors, make_inputs,
                         rounding_floor, seq_len)
from triton_fused_rope_flash_attn_amd import CosSinTable, TritonAttention, sdpa_triton_fa_rope
from triton_fused_rope_flash_attn_amd import _lib

from tests import _report

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()
    if "max_abs_err" in msg or msg.startswith("[fp16 range]"):
        _report.LINES.append(msg)


def _run_ours(q, k, v, do, table, has_cls, autocast_dtype=None, sum_loss=False):
    qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    if autocast_dtype is not None:
        with torch.autocast("cuda", dtype=autocast_dtype):
            o = sdpa_triton_fa_rope(qq, kk, vv, table, has_cls=has_cls)
    else:
        o = sdpa_triton_fa_rope(qq, kk, vv, table, has_cls=has_cls)
    if sum_loss:
        o.sum().backward()
    else:
        o.backward(do)
    torch.cuda.synchronize()
    return o.detach(), qq.grad, kk.grad, vv.grad


def _ref(q, k, v, do, table, has_cls):
    cosp, sinp = table.tables()
    return torch_ref.forward_backward(q.float(), k.float(), v.float(), do.float(), cosp, sinp, has_cls)


def _torch_bf16(q, k, v, do, table, has_cls):
    """torch-ROCm SDPA + Python RoPE in the input dtype (flash/efficient backends only)."""
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    qh = torch_ref.apply_rope(qq, table.COSP, table.SINP, has_cls)
    kh = torch_ref.apply_rope(kk, table.COSP, table.SINP, has_cls)
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        o = F.scaled_dot_product_attention(qh, kh, vv)
    o.backward(do)
    torch.cuda.synchronize()
    return o.detach(), qq.grad, kk.grad, vv.grad


def _paths_agree(tag, got, want, ref, mult_max=3.0, mult_mean=2.0):
    """Two backward paths on the same inputs: each gradient of `got` differs
    from `want` by at most `mult_max` / `mult_mean` x the bf16 storage floor of
    the fp32 oracle `ref` (max / mean), the scale at which two correct bf16
    results differ (each is itself held to about 2x that floor against the
    oracle, so their difference can reach the sum of both errors)."""
    fails = []
    for name, a, b, r in zip(("dQ", "dK", "dV"), got, want, ref):
        mx, mn = errors(a, b)
        fmx, fmn = rounding_floor(r, torch.bfloat16)
        _say(f"[{tag}] {name}: max_abs_err={mx:.3e} mean_abs_err={mn:.3e} between the paths "
             f"(bound {mult_max * fmx:.2e}/{mult_mean * fmn:.2e}, {mult_max:g}x / {mult_mean:g}x the storage floor)")
        if mx > mult_max * fmx or mn > mult_mean * fmn:
            fails.append(f"{name}: max {mx:.3e} mean {mn:.3e}")
    assert not fails, f"{tag}: " + "; ".join(fails)


def _compare(tag, ours, ref, tol_max=TOL_MAX, tol_mean=TOL_MEAN, out_dtype=None, other=None):
    """Check max/mean abs error of ours vs ref.

    With out_dtype set, the bound is max(tolerance, FLOOR_MULT x the error of
    storing ref in out_dtype), or the case's committed ceiling
    (tests/cases.py).  `other` (torch-ROCm bf16 SDPA + RoPE on the same
    inputs) is printed for comparison only.
    """
    names = ("O", "dQ", "dK", "dV")
    fails = []
    for i, (name, a, b) in enumerate(zip(names, ours, ref)):
        assert a.shape == b.shape, (name, a.shape, b.shape)
        assert torch.isfinite(a).all(), f"{tag} {name}: non-finite values"
        mx, mn = errors(a, b)
        lim_max, lim_mean = tol_max, tol_mean
        extra = ""
        omx = omn = 0.0
        if other is not None:
            omx, omn = errors(other[i], b)
        if out_dtype is not None and out_dtype != torch.float32:
            fmx, fmn = rounding_floor(b, out_dtype)
            lim_max, lim_mean = allowed(tag, name, fmx, fmn)
            lim_max, lim_mean = max(lim_max, tol_max), max(lim_mean, tol_mean)
            extra = f" | storage floor max {fmx:.3e} mean {fmn:.3e}"
        if other is not None:
            extra += f" | torch-bf16 max {omx:.3e} mean {omn:.3e}"
        _say(f"[{tag}] {name}: max_abs_err={mx:.3e} mean_abs_err={mn:.3e} (bound {lim_max:.2e}/{lim_mean:.2e}){extra}")
        if mx > lim_max or mn > lim_mean:
            fails.append(f"{name}: max {mx:.3e} (bound {lim_max:.2e}) mean {mn:.3e} (bound {lim_mean:.2e})")
    assert not fails, f"{tag}: " + "; ".join(fails)


@pytest.mark.parametrize("name", ["cpu", "vit_s", "vit_b", "vit_l", "hires"])
def test_parity_baseline_configs(name):
    cfg = CONFIGS[name]
    _say(f"case {name}: {cfg}")
    q, k, v, do = make_inputs(cfg, DEV)
    table = CosSinTable(ROPE_BASE, cfg["side"], cfg["D"], device=DEV)
    ours = _run_ours(q, k, v, do, table, cfg["has_cls"], sum_loss=cfg["dout"] == "ones")
    ref = _ref(q, k, v, do, table, cfg["has_cls"])
    other = None
    if cfg["dtype"] == torch.bfloat16:
        other = _torch_bf16(q, k, v, do, table, cfg["has_cls"])
    _compare(name, ours, ref, out_dtype=cfg["dtype"], other=other)


def test_lse_matches_logsumexp():
    cfg = dict(CONFIGS["vit_b"], B=4)
    q, k, v, _ = make_inputs(cfg, DEV)
    table = CosSinTable(ROPE_BASE, cfg["side"], cfg["D"], device=DEV)
    N, D = seq_len(cfg), cfg["D"]
    o, lse, _ = torch.ops.farope.attn_fwd(q, k, v, table.packed(), N - 1, True, 1 / math.sqrt(D), _lib.BF16)
    ref = torch_ref.logsumexp_rows(q.float(), k.float(), table.COSP, table.SINP, True)
    mx, _ = errors(lse, ref)
    _say(f"[lse] max_abs_err={mx:.3e}")
    assert mx < 2e-2


def test_autocast_fp32_leaves():
    """README example: fp32 leaves under bf16 autocast -> fp32 O and grads."""
    cfg = dict(CONFIGS["cpu"], dout="randn")
    q, k, v, do = make_inputs(cfg, DEV)
    table = CosSinTable(ROPE_BASE, 14, 64, device=DEV)
    ours = _run_ours(q, k, v, do, table, True, autocast_dtype=torch.bfloat16)
    assert ours[0].dtype == torch.float32 and ours[1].dtype == torch.float32
    ref = _ref(q, k, v, do, table, True)
    _compare("autocast-bf16", ours, ref)


@pytest.mark.parametrize("ac_dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_autocast_fp32_leaves_many_planes(ac_dtype):
    """fp32 leaves under bf16 / fp16 autocast (README:94-110, FA:65-73) with
    B*H = 1152 planes at N = 197, D = 64: the one-pass backward's persistent
    grid (one workgroup per CU, 256 CUs) gives every workgroup 4-5 planes, so
    each plane's K-hat tile in LDS is rewritten while the previous plane's last
    dQ products of the other waves may still read it.  The 32-bit-I/O variant
    reads K-hat^T from LDS in every dQ product; this is its regression test at
    the north-star tolerance (no storage floor: the outputs are fp32)."""
    cfg = dict(B=96, H=12, side=14, has_cls=True, D=64, dtype=torch.float32, scale=1.0, dout="randn")
    q, k, v, do = make_inputs(cfg, DEV, seed=11)
    table = CosSinTable(ROPE_BASE, 14, 64, device=DEV)
    ours = _run_ours(q, k, v, do, table, True, autocast_dtype=ac_dtype)
    for t in ours:
        assert t.dtype == torch.float32
    ref = _ref(q, k, v, do, table, True)
    _compare(f"autocast-{ac_dtype}-1152planes", ours, ref)


def test_fp16_io():
    cfg = dict(CONFIGS["vit_b"], B=8, dtype=torch.float16)
    q, k, v, do = make_inputs(cfg, DEV)
    table = CosSinTable(ROPE_BASE, 14, 64, device=DEV)
    ours = _run_ours(q, k, v, do, table, True)
    ref = _ref(q, k, v, do, table, True)
    _compare("fp16", ours, ref, out_dtype=torch.float16)


def test_fp32_compute_is_tight():
    """fp32 I/O without autocast computes in fp32 (bf16x3 split products)."""
    cfg = dict(CONFIGS["cpu"], dout="randn")
    q, k, v, do = make_inputs(cfg, DEV)
    table = CosSinTable(ROPE_BASE, 14, 64, device=DEV)
    ours = _run_ours(q, k, v, do, table, True)
    ref = _ref(q, k, v, do, table, True)
    _compare("fp32", ours, ref, tol_max=1e-4, tol_mean=1e-5)


@pytest.mark.parametrize(
    "side,has_cls,D",
    [(7, True, 64), (5, False, 64), (16, True, 64), (14, True, 128), (3, False, 128), (1, True, 64),
     (14, True, 32), (5, False, 32), (16, True, 32), (14, True, 256), (5, False, 256), (17, True, 256),
     (14, False, 64), (14, False, 32)],
)
def test_ragged_and_variant_shapes(side, has_cls, D):
    """Ragged N (N % 32 != 0), no-CLS, N > 256 (streamed fwd + split bwd), D=128, D=32,
    D=256 (the largest power of two the reference's kernels take, FA:146, FA:313), N=2,
    N = 196 / 197 (13 query subtiles of the forward's 256-row item) at D = 32, 64."""
    cfg = dict(B=3, H=5, side=side, has_cls=has_cls, D=D, dtype=torch.bfloat16, scale=1.0, dout="randn")
    q, k, v, do = make_inputs(cfg, DEV, seed=1)
    table = CosSinTable(ROPE_BASE, side, D, device=DEV)
    ours = _run_ours(q, k, v, do, table, has_cls)
    ref = _ref(q, k, v, do, table, has_cls)
    other = _torch_bf16(q, k, v, do, table, has_cls)
    _compare(f"side{side}-cls{int(has_cls)}-D{D}", ours, ref, out_dtype=torch.bfloat16, other=other)


@pytest.mark.parametrize("case", ["n256", "tile_scales"])
def test_stored_ds_backward(case):
    """The stored-dS backward (variant 3: head_dim 128, bf16 compute, 16-bit I/O):
    N = 256, no CLS (two full key tiles, no lone key, no ragged tile); and N = 257
    with V scaled by 2^-12 on the first 128 keys, so that the key tiles bound |dS|
    differently, store it at different powers of two (their exponents differ) and
    the dQ GEMM stages each tile's K-hat rows at its own scale."""
    B, H, D = 2, 3, 128
    side, has_cls = (16, False) if case == "n256" else (16, True)
    N = side * side + int(has_cls)
    desc = _lib.make_desc(B, H, N, D, N - int(has_cls), has_cls, _lib.BF16, _lib.BF16, 1 / math.sqrt(D))
    assert _lib.tile_config(desc, 1)[0] == 3
    cfg = dict(B=B, H=H, side=side, has_cls=has_cls, D=D, dtype=torch.bfloat16, scale=1.0, dout="randn")
    q, k, v, do = make_inputs(cfg, DEV, seed=7)
    if case == "tile_scales":
        v = v.clone()
        v[:, :, :128] *= 2.0 ** -12   # exact in bf16
    _say(f"case stored-ds {case}: N={N}")
    table = CosSinTable(ROPE_BASE, side, D, device=DEV)
    ours = _run_ours(q, k, v, do, table, has_cls)
    ref = _ref(q, k, v, do, table, has_cls)
    _compare(f"stored-ds-{case}-N{N}", ours, ref, out_dtype=torch.bfloat16)


@pytest.mark.parametrize(
    "side,has_cls,D,B,H,io",
    [(16, True, 128, 2, 3, "bf16"), (16, True, 32, 2, 3, "bf16"), (16, True, 256, 2, 3, "bf16"),
     (16, True, 128, 2, 3, "fp16"), (16, True, 128, 1, 2, "fp32"),
     (63, True, 128, 1, 2, "bf16"), (62, False, 128, 1, 2, "bf16")],
)
def test_tail_rows(side, has_cls, D, B, H, io):
    """Rows past the last full block (N % block_rows <= 8, e.g. N = 16^2 + 1, 63^2 + 1,
    62^2): computed by the tail kernels, or -- one row with fp16 logit operands (bf16,
    D 128 / 256) -- by one designated item per plane of the forward and dQ block kernels,
    not by a nearly empty block.  One tail row at every head dim and I/O type; two
    (N = 3970, dK/dV) and four (N = 3844, no CLS) rows."""
    dt = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[io]
    N = side * side + int(has_cls)
    code = _lib.DTYPE_CODE[dt]
    desc = _lib.make_desc(B, H, N, D, N - int(has_cls), has_cls, code, code, 1 / math.sqrt(D))
    rows = (_lib.tile_config(desc, 0)[1], _lib.tile_config(desc, 1)[1])   # forward, dK/dV block rows
    assert any(N >= r and 0 < N % r <= 8 for r in rows)
    cfg = dict(B=B, H=H, side=side, has_cls=has_cls, D=D, dtype=dt, scale=1.0, dout="randn")
    q, k, v, do = make_inputs(cfg, DEV, seed=5)
    table = CosSinTable(ROPE_BASE, side, D, device=DEV)
    ours = _run_ours(q, k, v, do, table, has_cls)
    ref = _ref(q, k, v, do, table, has_cls)
    if io == "fp32":
        _compare(f"tail-fp32-N{N}-D{D}", ours, ref, tol_max=1e-4, tol_mean=1e-5)
    else:
        _compare(f"tail-{io}-N{N}-D{D}", ours, ref, out_dtype=dt)


def test_tail_rows_generic_strides_and_split_entry_points():
    """Tail rows through the generic (d-strided) loads, and through the reference-style
    preprocess + dk_dv + dq entry points.  Those run other kernels than the one-call
    backward (the dK/dV kernel with split-bf16 dS, the fp32 tail-key kernel, rotating Q
    themselves), so they agree with it within a small multiple of the bf16 storage floor,
    not bit for bit."""
    B, H, side, D = 2, 2, 16, 128
    N = side * side + 1
    g = torch.Generator().manual_seed(6)
    base = [torch.randn(B, H, D, N, generator=g).to(torch.bfloat16).to(DEV) for _ in range(3)]
    q, k, v = (t.transpose(-1, -2) for t in base)
    assert q.stride(-1) != 1
    do = torch.randn(B, H, N, D, generator=g).to(torch.bfloat16).to(DEV)
    table = CosSinTable(ROPE_BASE, side, D, device=DEV)
    ours = _run_ours(q, k, v, do, table, True)
    ref = _ref(q, k, v, do, table, True)
    _compare("tail-d-strided", ours, ref, out_dtype=torch.bfloat16)

    q, k, v = (t.contiguous() for t in (q, k, v))
    rope = table.packed()
    scale = 1 / math.sqrt(D)
    o, lse, res = torch.ops.farope.attn_fwd(q, k, v, rope, N - 1, True, scale, _lib.BF16)
    dq, dk, dv = torch.ops.farope.attn_bwd(do, q, k, v, o, lse, rope, N - 1, True, scale, _lib.BF16, res)
    desc = _lib.make_desc(B, H, N, D, N - 1, True, _lib.BF16, _lib.BF16, scale)
    delta = torch.empty(B, H, N, device=DEV, dtype=torch.float32)
    dq2, dk2, dv2 = (torch.empty_like(q) for _ in range(3))
    _lib.attn_bwd_preprocess(desc, o, do, delta, res)
    _lib.attn_bwd_dk_dv(desc, q, k, v, do, lse, delta, rope, dk2, dv2)
    _lib.attn_bwd_dq(desc, q, k, v, do, lse, delta, rope, dq2)
    torch.cuda.synchronize()
    _compare("tail entry points", (o, dq2, dk2, dv2), ref, out_dtype=torch.bfloat16)
    _paths_agree("tail entry points vs one-call", (dq2, dk2, dv2), (dq, dk, dv), ref[1:])


def test_strided_qkv_views():
    """q/k/v as permuted views of one [B, N, 3, H, D] projection (ViT attention layout)."""
    B, H, side, D = 4, 12, 14, 64
    N = side * side + 1
    g = torch.Generator().manual_seed(3)
    qkv = torch.randn(B, N, 3, H, D, generator=g).to(torch.bfloat16).to(DEV)
    q, k, v = qkv.permute(2, 0, 3, 1, 4).unbind(0)
    assert not q.is_contiguous()
    do = torch.randn(B, H, N, D, generator=g).to(torch.bfloat16).to(DEV)
    table = CosSinTable(ROPE_BASE, side, D, device=DEV)
    ours = _run_ours(q, k, v, do, table, True)
    ref = _ref(q, k, v, do, table, True)
    _compare("qkv-views", ours, ref, out_dtype=torch.bfloat16)


def test_channel_strided_inputs_generic_path():
    """d-stride != 1 (generic gather path) gives the same answer."""
    B, H, side, D = 2, 3, 14, 64
    N = side * side + 1
    g = torch.Generator().manual_seed(4)
    base = [torch.randn(B, H, D, N, generator=g).to(torch.bfloat16).to(DEV) for _ in range(3)]
    q, k, v = (t.transpose(-1, -2) for t in base)
    assert q.stride(-1) != 1
    do = torch.randn(B, H, N, D, generator=g).to(torch.bfloat16).to(DEV)
    table = CosSinTable(ROPE_BASE, side, D, device=DEV)
    ours = _run_ours(q, k, v, do, table, True)
    ref = _ref(q, k, v, do, table, True)
    _compare("d-strided", ours, ref, out_dtype=torch.bfloat16)


@pytest.mark.parametrize(
    "side,has_cls,D,mode",
    [(14, True, 128, "d-strided"), (16, True, 64, "d-strided"), (14, True, 128, "autocast"),
     (16, True, 64, "autocast"), (14, True, 128, "fp16"), (16, True, 64, "fp32"),
     (14, True, 32, "d-strided"), (14, True, 32, "fp32"), (14, True, 32, "autocast"),
     (14, True, 256, "d-strided"), (14, True, 256, "fp32"), (14, True, 256, "autocast"),
     (7, True, 256, "fp16")],
)
def test_split_backward_io_variants(side, has_cls, D, mode):
    """The split backward (N > 256 or D = 128) with generic-stride inputs (element-wise
    staging), fp32 leaves under bf16 autocast (32-bit prefetch rows), fp16 I/O and fp32
    compute (the 4-wave tiles)."""
    N = side * side + int(has_cls)
    B, H = 2, 3
    g = torch.Generator().manual_seed(7)
    dtype = {"fp16": torch.float16, "fp32": torch.float32, "autocast": torch.float32}.get(mode, torch.bfloat16)
    if mode == "d-strided":
        q, k, v = (torch.randn(B, H, D, N, generator=g).to(dtype).to(DEV).transpose(-1, -2) for _ in range(3))
        assert q.stride(-1) != 1
    else:
        q, k, v = (torch.randn(B, H, N, D, generator=g).to(dtype).to(DEV) for _ in range(3))
    do = torch.randn(B, H, N, D, generator=g).to(dtype).to(DEV)
    table = CosSinTable(ROPE_BASE, side, D, device=DEV)
    ours = _run_ours(q, k, v, do, table, has_cls,
                     autocast_dtype=torch.bfloat16 if mode == "autocast" else None)
    ref = _ref(q, k, v, do, table, has_cls)
    tag = f"split-{mode}-N{N}-D{D}"
    if mode == "fp32":
        _compare(tag, ours, ref, tol_max=1e-4, tol_mean=1e-5)
    elif mode == "autocast":
        _compare(tag, ours, ref)
    else:
        _compare(tag, ours, ref, out_dtype=dtype)


def test_stride0_dout_from_sum():
    cfg = dict(CONFIGS["vit_b"], B=4)
    q, k, v, _ = make_inputs(cfg, DEV)
    table = CosSinTable(ROPE_BASE, 14, 64, device=DEV)
    ours = _run_ours(q, k, v, None, table, True, sum_loss=True)
    ones = torch.ones_like(q, dtype=torch.float32)
    ref = _ref(q, k, v, ones, table, True)
    other = _torch_bf16(q, k, v, ones.to(q.dtype), table, True)
    _compare("stride0-dO", ours, ref, out_dtype=torch.bfloat16, other=other)


def test_triton_attention_apply_signature():
    """TritonAttention.apply(Q, K, V, cos_sin, H_img, has_cls) as in the reference."""
    B, H, side, D = 2, 4, 16, 64
    cfg = dict(B=B, H=H, side=side, has_cls=False, D=D, dtype=torch.bfloat16, scale=1.0, dout="randn")
    q, k, v, do = make_inputs(cfg, DEV, seed=5)
    table = CosSinTable(ROPE_BASE, side, D, device=DEV)
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    o = TritonAttention.apply(qq, kk, vv, table, side, False)
    o.backward(do)
    ref = _ref(q, k, v, do, table, False)
    _compare("TritonAttention.apply", (o.detach(), qq.grad, kk.grad, vv.grad), ref, out_dtype=torch.bfloat16)


def test_split_entry_points_match_fused():
    """preprocess + dk_dv + dq entry points (reference launch structure) against the
    one-call backward (here the one-pass plane kernel): both within the north-star
    bound of the oracle, and within a small multiple of the bf16 storage floor of each other."""
    cfg = dict(CONFIGS["vit_b"], B=4)
    q, k, v, do = make_inputs(cfg, DEV)
    table = CosSinTable(ROPE_BASE, 14, 64, device=DEV)
    B, H, N, D = q.shape
    rope = table.packed()
    scale = 1 / math.sqrt(D)
    o, lse, res = torch.ops.farope.attn_fwd(q, k, v, rope, N - 1, True, scale, _lib.BF16)
    dq, dk, dv = torch.ops.farope.attn_bwd(do, q, k, v, o, lse, rope, N - 1, True, scale, _lib.BF16, res)
    desc = _lib.make_desc(B, H, N, D, N - 1, True, _lib.BF16, _lib.BF16, scale)
    delta = torch.empty(B, H, N, device=DEV, dtype=torch.float32)
    dq2, dk2, dv2 = (torch.empty_like(q) for _ in range(3))
    _lib.attn_bwd_preprocess(desc, o, do, delta)
    _lib.attn_bwd_dk_dv(desc, q, k, v, do, lse, delta, rope, dk2, dv2)
    _lib.attn_bwd_dq(desc, q, k, v, do, lse, delta, rope, dq2)
    torch.cuda.synchronize()
    ref_delta = (do.float() * o.float()).sum(-1)
    assert errors(delta, ref_delta)[0] < 1e-3
    ref = _ref(q, k, v, do, table, True)
    _compare("entry points", (o, dq2, dk2, dv2), ref, out_dtype=torch.bfloat16)
    _paths_agree("entry points vs one-pass", (dq2, dk2, dv2), (dq, dk, dv), ref[1:])


def test_deterministic():
    cfg = dict(CONFIGS["vit_b"], B=8)
    q, k, v, do = make_inputs(cfg, DEV)
    table = CosSinTable(ROPE_BASE, 14, 64, device=DEV)
    a = _run_ours(q, k, v, do, table, True)
    b = _run_ours(q, k, v, do, table, True)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_large_logits_finite():
    """Inputs x4 (logits std ~16): softmax must stay finite and accurate."""
    cfg = dict(CONFIGS["vit_b"], B=4, scale=4.0)
    q, k, v, do = make_inputs(cfg, DEV)
    table = CosSinTable(ROPE_BASE, 14, 64, device=DEV)
    ours = _run_ours(q, k, v, do, table, True)
    for t in ours:
        assert torch.isfinite(t).all()
    ref = _ref(q, k, v, do, table, True)
    other = _torch_bf16(q, k, v, do, table, True)
    # Logits with std ~16: bf16 operands cannot resolve near-ties, so the
    # bound here is "no worse than torch-ROCm bf16 SDPA + RoPE" (+25%).
    for i, name in enumerate(("O", "dQ", "dK", "dV")):
        mx, mn = errors(ours[i], ref[i])
        omx, omn = errors(other[i], ref[i])
        _say(f"[x4 inputs] {name}: ours max {mx:.3e} mean {mn:.3e} | torch-bf16 max {omx:.3e} mean {omn:.3e}")
        assert mn <= 1.25 * omn + 1e-4, name


@pytest.mark.parametrize("planes", [
    # (q scale, k scale, v scale) per (b, h) plane: 2^20 / 2^-20 push |Q-hat|
    # (with the logit scale) far past 2^12 and |K-hat| into fp16's subnormal
    # range, and the reverse makes K-hat overflow fp16; the logits themselves
    # stay those of unit inputs.  2^11 / 2^-11 stays below the rescale threshold.
    [(2.0 ** 20, 2.0 ** -20, 1.0), (1.0, 1.0, 1.0), (2.0 ** -20, 2.0 ** 20, 1.0), (2.0 ** 11, 2.0 ** -11, 1.0)],
    # V past fp16's range (2^20), deep in its subnormal range (2^-20), and
    # just past the 2^12 rescale threshold (2^11 x |N(0,1)| up to ~2^13)
    [(1.0, 1.0, 2.0 ** 20), (1.0, 1.0, 2.0 ** -20), (1.0, 1.0, 1.0), (1.0, 1.0, 2.0 ** 11)],
], ids=["qk", "v"])
def test_f16_logit_operand_range(planes):
    """bf16 compute at head_dim 128 takes the logits (and the forward's P V) from
    fp16 operands; a tile whose Q-hat or K-hat reaches 2^12, or whose V leaves
    [2^-10, 2^12), is computed again with its operands rescaled by powers of
    two.  With Q = a q0, K = k0 / a the logits are those of (q0, k0), O and dV
    are unchanged, dQ scales by 1/a and dK by a; with V = c v0, O, dQ and dK
    scale by c and dV is unchanged.  Each plane's outputs, divided by those
    factors, must meet the north-star tolerance against the fp32 oracle on the
    same (scaled, bf16) inputs."""
    B, H, side, D = 2, 2, 16, 128
    N = side * side + 1
    g = torch.Generator().manual_seed(3)
    q, k, v, do = (torch.randn(B, H, N, D, generator=g) for _ in range(4))
    fac = torch.ones(B, H, 4)
    for i, (a, c, w) in enumerate(planes):
        b, h = divmod(i, H)
        q[b, h] *= a
        k[b, h] *= c
        v[b, h] *= w
        fac[b, h] = torch.tensor([w, c * w, a * w, 1.0])   # O, dQ, dK, dV magnitude factors
    q, k, v, do = (t.to(torch.bfloat16).to(DEV) for t in (q, k, v, do))
    table = CosSinTable(ROPE_BASE, side, D, device=DEV)
    ours = _run_ours(q, k, v, do, table, True)
    ref = _ref(q, k, v, do, table, True)
    fails = []
    for i, name in enumerate(("O", "dQ", "dK", "dV")):
        assert torch.isfinite(ours[i]).all(), name
        for b in range(B):
            for h in range(H):
                f = fac[b, h, i].item()
                mx, mn = errors(ours[i][b, h].float() / f, ref[i][b, h].float() / f)
                _say(f"[fp16 range] plane ({b},{h}) scales {planes[b * H + h]} {name}/{f:g}: "
                     f"max {mx:.3e} mean {mn:.3e}")
                if mx > TOL_MAX or mn > TOL_MEAN:
                    fails.append(f"plane ({b},{h}) {name}: max {mx:.3e} mean {mn:.3e}")
    assert not fails, "; ".join(fails)


def test_torch_compile_fullgraph():
    """The ops trace as opaque nodes: torch.compile(fullgraph=True) of the public
    entry (RoPE table packing included) matches eager bit for bit, fwd and bwd."""
    import torch._dynamo

    cfg = dict(CONFIGS["vit_b"], B=2)
    q, k, v, do = make_inputs(cfg, DEV)
    table = CosSinTable(ROPE_BASE, 14, 64, device=DEV)

    def f(q, k, v):
        return sdpa_triton_fa_rope(q, k, v, table)

    torch._dynamo.reset()
    cf = torch.compile(f, fullgraph=True, backend="aot_eager")
    outs = []
    for fn in (f, cf):
        qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
        o = fn(qq, kk, vv)
        o.backward(do)
        torch.cuda.synchronize()
        outs.append((o.detach(), qq.grad, kk.grad, vv.grad))
    for name, a, b in zip(("O", "dQ", "dK", "dV"), *outs):
        _say(f"[compile] {name}: equal={torch.equal(a, b)}")
        assert torch.equal(a, b), name


def test_torch_compile_inductor_matches_oracle():
    """torch.compile(backend="inductor", fullgraph=True) of the public entry
    (the compiler of the reference README's comparison, README:165-195): O and
    the gradients match the fp32 oracle at the north-star tolerance."""
    import torch._dynamo

    cfg = dict(CONFIGS["vit_b"], B=4)
    q, k, v, do = make_inputs(cfg, DEV, seed=2)
    table = CosSinTable(ROPE_BASE, 14, 64, device=DEV)

    def f(q, k, v):
        return sdpa_triton_fa_rope(q, k, v, table)

    torch._dynamo.reset()
    cf = torch.compile(f, fullgraph=True, backend="inductor")
    qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    o = cf(qq, kk, vv)
    o.backward(do)
    torch.cuda.synchronize()
    ref = _ref(q, k, v, do, table, True)
    _compare("inductor", (o.detach(), qq.grad, kk.grad, vv.grad), ref, out_dtype=torch.bfloat16)
    torch._dynamo.reset()


@pytest.mark.parametrize("how", ["load_state_dict", "reassign"])
def test_checkpoint_reload_repacks_table(how):
    """A CosSinTable already used by the op takes new COSP/SINP, either from a
    checkpoint of a table with another base (state_dict keys of FA:1158-1159,
    loaded in place) or by reassigning the buffers.  The next call must use
    the new tables: it matches the oracle built from them, and differs from
    the output with the old tables."""
    cfg = dict(CONFIGS["vit_b"], B=2)
    q, k, v, do = make_inputs(cfg, DEV, seed=9)
    table = CosSinTable(ROPE_BASE, 14, 64, device=DEV)
    before = _run_ours(q, k, v, do, table, True)
    other = CosSinTable(10000.0, 14, 64, device=DEV)
    if how == "load_state_dict":
        ptr = table.COSP.data_ptr()
        table.load_state_dict(other.state_dict())
        assert table.COSP.data_ptr() == ptr   # loaded in place: same storage, new values
    else:
        table.COSP = other.COSP.clone()
        table.SINP = other.SINP.clone()
    assert torch.equal(table.COSP, other.COSP) and torch.equal(table.SINP, other.SINP)
    after = _run_ours(q, k, v, do, table, True)
    ref = _ref(q, k, v, do, other, True)
    _compare(f"reload-{how}", after, ref, out_dtype=torch.bfloat16)
    assert (after[0].float() - before[0].float()).abs().max().item() > 1e-1


def test_vit_attention_block_matches_reference_block():
    """RoPEAttention (qkv -> strided views -> fused op -> proj) vs the same block
    and weights with the oracle attention (Python RoPE + fp32 math SDPA) in
    its place: outputs and the gradients of x and both projections agree
    to the op's tolerance (the linear layers are identical bf16 GEMMs)."""
    from triton_fused_rope_flash_attn_amd import RoPEAttention

    torch.manual_seed(0)
    B, N, C, H = 8, 197, 384, 6

    def oracle_attn(q, k, v, table, H_img=None, has_cls=True):
        cosp, sinp = table.tables()
        return torch_ref.attention(q.float(), k.float(), v.float(), cosp, sinp, has_cls).to(q.dtype)

    ours = RoPEAttention(C, H, H_img=14, has_cls=True, device=DEV, dtype=torch.bfloat16)
    ref = RoPEAttention(C, H, H_img=14, has_cls=True, attn=oracle_attn, device=DEV, dtype=torch.bfloat16)
    ref.load_state_dict(ours.state_dict())
    x = torch.randn(B, N, C, device=DEV, dtype=torch.bfloat16)
    dy = torch.randn(B, N, C, device=DEV, dtype=torch.bfloat16)
    res = []
    for blk in (ours, ref):
        xx = x.clone().requires_grad_(True)
        y = blk(xx)
        y.backward(dy)
        torch.cuda.synchronize()
        res.append((y.detach().float(), xx.grad.float(), blk.qkv.weight.grad.float(),
                    blk.proj.weight.grad.float()))
    for name, a, b in zip(("y", "dx", "dWqkv", "dWproj"), *res):
        mx, mn = errors(a, b)
        scale = b.abs().mean().item()
        _say(f"[vit block] {name}: max {mx:.3e} mean {mn:.3e} (mean |ref| {scale:.3e})")
        assert torch.isfinite(a).all(), name
        assert mn <= 2e-2 * scale + 1e-3, name
