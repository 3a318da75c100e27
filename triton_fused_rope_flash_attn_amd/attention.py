"""Fused 2D-RoPE attention: PyTorch custom ops over the farope C ABI.

Public surface mirrors the reference ("fa_rope_full .py"):

* ``sdpa_triton_fa_rope(Q, K, V, cos_sin)``                 FA:1169-1170
* ``TritonAttention.apply(Q, K, V, cos_sin, H_img=14, has_cls=True)``
                                                             FA:1011-1138
* ``_sdpa_comp_dtype(x)``                                    FA:65-73

Q, K, V are ``[B, H, N, D]`` with any strides; O has Q's dtype; gradients
come back for Q, K and V.  The compute dtype is the autocast dtype when
autocast is enabled, else Q's dtype (FA:65-73); it is fixed at forward time
and reused by backward (FA:1061).

The work is done by two ``torch.library`` custom ops, ``farope::attn_fwd``
-> (O, LSE) and ``farope::attn_bwd`` -> (dQ, dK, dV), each a single call into
libfarope.so on the current HIP stream.  Both have fake (meta) kernels, so
the ops are opaque but traceable under ``torch.compile``.  There is no CPU
or eager-PyTorch fallback: CPU tensors raise.
"""
from __future__ import annotations

import math

import torch

from . import _lib
from .rope import CosSinTable, pack_rope_tables

__all__ = ["sdpa_triton_fa_rope", "TritonAttention", "_sdpa_comp_dtype", "rope_operand"]


def _sdpa_comp_dtype(x: torch.Tensor) -> torch.dtype:
    """Compute dtype: autocast dtype if autocast is on, else ``x.dtype`` (FA:65-73).

    Anything other than fp16/bf16/fp32 raises TypeError, as the reference's
    ``raise dtype`` does.
    """
    dtype = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled() else x.dtype
    if dtype in (torch.float16, torch.bfloat16, torch.float32):
        return dtype
    raise TypeError(f"farope: unsupported compute dtype {dtype} (float16, bfloat16, float32)")


def _check_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    if q.dim() != 4:
        raise ValueError(f"Q must be [B, H, N, D]; got shape {tuple(q.shape)}")
    if k.shape != q.shape or v.shape != q.shape:
        raise ValueError(
            f"Q, K, V must have the same shape; got {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}"
        )
    if q.dtype not in _lib.DTYPE_CODE:
        raise TypeError(f"farope: unsupported tensor dtype {q.dtype}")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError(f"farope: Q, K, V must share one dtype; got {q.dtype}, {k.dtype}, {v.dtype}")
    if not q.is_cuda:
        raise RuntimeError(
            f"farope runs on ROCm GPUs only (hand-written gfx950 kernels); got a {q.device} tensor"
        )
    if k.device != q.device or v.device != q.device:
        raise RuntimeError("farope: Q, K, V must be on the same device")


def _check_rope(rope: torch.Tensor, n_pos: int, d: int, device) -> None:
    want = (n_pos + 1) * (d // 2) * 2
    if rope.dtype != torch.float32 or rope.dim() != 1 or rope.numel() != want or not rope.is_contiguous():
        raise ValueError(
            f"farope: packed RoPE table must be contiguous fp32 of {want} elements "
            f"for n_pos={n_pos}, D={d}; got {rope.dtype} {tuple(rope.shape)}"
        )
    if rope.device != device:
        raise RuntimeError(f"farope: RoPE table on {rope.device}, tensors on {device}")


def _uses_residual(io_dtype: int, compute_dtype: int, head_dim: int) -> bool:
    """Whether the call keeps O's rounding residual for the backward's delta:
    bf16 tensors computed in bf16 at head_dim >= 128 (the rule of
    farope_attn_residual_elems, which the CPU tests check this against)."""
    return io_dtype == _lib.BF16 and compute_dtype == _lib.BF16 and head_dim >= 128


# ---------------------------------------------------------------------------
# custom ops
# ---------------------------------------------------------------------------
@torch.library.custom_op("farope::attn_fwd", mutates_args=())
def attn_fwd(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    rope: torch.Tensor,
    n_pos: int,
    has_cls: bool,
    softmax_scale: float,
    compute_dtype: int,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """-> (O, LSE, O_res).  O_res is O's rounding residual bf16(O - bf16(O))
    [B, H, N, D] where the call keeps one (see _uses_residual), else empty."""
    _check_qkv(q, k, v)
    B, H, N, D = q.shape
    _check_rope(rope, n_pos, D, q.device)
    o = torch.empty((B, H, N, D), dtype=q.dtype, device=q.device)
    lse = torch.empty((B, H, N), dtype=torch.float32, device=q.device)
    io = _lib.DTYPE_CODE[q.dtype]
    res = _uses_residual(io, compute_dtype, D)
    o_res = torch.empty((B, H, N, D) if res else (0,), dtype=q.dtype, device=q.device)
    desc = _lib.make_desc(B, H, N, D, n_pos, has_cls, io, compute_dtype, softmax_scale)
    with torch.cuda.device(q.device):
        _lib.attn_fwd(desc, q, k, v, rope, o, lse, o_res)
    return o, lse, o_res


@attn_fwd.register_fake
def _attn_fwd_fake(q, k, v, rope, n_pos, has_cls, softmax_scale, compute_dtype):
    B, H, N, D = q.shape
    res = _uses_residual(_lib.DTYPE_CODE.get(q.dtype, -1), compute_dtype, D)
    return (
        q.new_empty((B, H, N, D)),
        q.new_empty((B, H, N), dtype=torch.float32),
        q.new_empty((B, H, N, D) if res else (0,)),
    )


@torch.library.custom_op("farope::attn_bwd", mutates_args=())
def attn_bwd(
    do: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    o: torch.Tensor,
    lse: torch.Tensor,
    rope: torch.Tensor,
    n_pos: int,
    has_cls: bool,
    softmax_scale: float,
    compute_dtype: int,
    o_res: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """-> (dQ, dK, dV).  o_res: attn_fwd's third output (may be empty)."""
    _check_qkv(q, k, v)
    B, H, N, D = q.shape
    _check_rope(rope, n_pos, D, q.device)
    if do.shape != q.shape or o.shape != q.shape:
        raise ValueError("farope: dO and O must have Q's shape")
    if do.dtype != q.dtype:
        do = do.to(q.dtype)
    if lse.dtype != torch.float32 or lse.shape != (B, H, N) or not lse.is_contiguous():
        raise ValueError("farope: LSE must be contiguous fp32 [B, H, N]")
    dq = torch.empty((B, H, N, D), dtype=q.dtype, device=q.device)
    dk = torch.empty((B, H, N, D), dtype=k.dtype, device=q.device)
    dv = torch.empty((B, H, N, D), dtype=v.dtype, device=q.device)
    desc = _lib.make_desc(B, H, N, D, n_pos, has_cls, _lib.DTYPE_CODE[q.dtype], compute_dtype,
                          softmax_scale)
    # the backward's workspace (delta rows, and at head_dim 128 the rotated Q
    # rows, row statistics and stored dS^T of the key tiles); none for the
    # one-pass backward, which keeps delta on chip
    ws = _lib.bwd_workspace_elems(desc)
    delta = torch.empty(ws, dtype=torch.float32, device=q.device) if ws else None
    if o_res.numel() and (o_res.shape != q.shape or o_res.dtype != q.dtype or not o_res.is_contiguous()):
        raise ValueError("farope: O_res must be contiguous with Q's shape and dtype, or empty")
    with torch.cuda.device(q.device):
        _lib.attn_bwd(desc, q, k, v, o, do, lse, rope, dq, dk, dv, delta, o_res)
    return dq, dk, dv


@attn_bwd.register_fake
def _attn_bwd_fake(do, q, k, v, o, lse, rope, n_pos, has_cls, softmax_scale, compute_dtype, o_res):
    B, H, N, D = q.shape
    return q.new_empty((B, H, N, D)), k.new_empty((B, H, N, D)), v.new_empty((B, H, N, D))


def _fwd_setup_context(ctx, inputs, output):
    q, k, v, rope, n_pos, has_cls, softmax_scale, compute_dtype = inputs
    o, lse, o_res = output
    ctx.mark_non_differentiable(lse, o_res)
    # LSE's incoming gradient is never used: without this, autograd fills a
    # zero tensor for it on every backward (an extra kernel per step)
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(q, k, v, o, lse, rope, o_res)
    ctx.n_pos = n_pos
    ctx.has_cls = has_cls
    ctx.softmax_scale = softmax_scale
    ctx.compute_dtype = compute_dtype


def _fwd_backward(ctx, do, _dlse, _dres):
    if do is None:   # O received no gradient (grads are not materialised)
        return None, None, None, None, None, None, None, None
    q, k, v, o, lse, rope, o_res = ctx.saved_tensors
    dq, dk, dv = attn_bwd(do, q, k, v, o, lse, rope, ctx.n_pos, ctx.has_cls,
                          ctx.softmax_scale, ctx.compute_dtype, o_res)
    return dq, dk, dv, None, None, None, None, None


attn_fwd.register_autograd(_fwd_backward, setup_context=_fwd_setup_context)


# ---------------------------------------------------------------------------
# host-side argument handling shared by both public entry points
# ---------------------------------------------------------------------------
def rope_operand(cos_sin, n_pos: int, head_dim: int, device) -> torch.Tensor:
    """Packed kernel table for ``cos_sin`` (a CosSinTable or anything with ``tables()``).

    Unlike the reference, which never checks the table against the call,
    a table whose shape is not ``[n_pos, head_dim/2]`` raises ValueError.
    """
    cosp, sinp = cos_sin.tables()
    if tuple(cosp.shape) != (n_pos, head_dim // 2) or tuple(sinp.shape) != (n_pos, head_dim // 2):
        raise ValueError(
            f"RoPE table shape {tuple(cosp.shape)} does not match the call "
            f"(expected [{n_pos}, {head_dim // 2}] for H_img^2={n_pos}, D={head_dim})"
        )
    if cosp.device != device:
        raise RuntimeError(f"RoPE table is on {cosp.device}, Q/K/V on {device}")
    if isinstance(cos_sin, CosSinTable):
        return cos_sin.packed()
    return pack_rope_tables(cosp, sinp)


def _prepare(Q, K, V, cos_sin, H_img, has_cls):
    """Checks of TritonAttention.forward (FA:1014-1024) plus device/dtype checks."""
    BATCH_SIZE, NUM_HEADS, SEQ_LEN, HEAD_DIM = Q.size()
    assert (HEAD_DIM % 4) == 0, "HEAD_DIM must be divisible by 4 (2D RoPE requires pairs)."
    N_img = H_img ** 2
    if has_cls:
        assert SEQ_LEN == 1 + N_img, (
            f"SEQ_LEN must be 1 + H_img*W_img when has_cls=True (got {SEQ_LEN} vs {1 + N_img})."
        )
    else:
        assert SEQ_LEN == N_img, (
            f"SEQ_LEN must equal H_img*W_img when has_cls=False (got {SEQ_LEN} vs {N_img})."
        )
    _check_qkv(Q, K, V)
    comp = _sdpa_comp_dtype(Q)
    softmax_scale = 1.0 / (HEAD_DIM ** 0.5)
    rope = rope_operand(cos_sin, N_img, HEAD_DIM, Q.device)
    return rope, N_img, bool(has_cls), softmax_scale, _lib.DTYPE_CODE[comp]


class TritonAttention(torch.autograd.Function):
    """Autograd function with the reference's signature (FA:1011-1138).

    ``forward(ctx, Q, K, V, cos_sin, H_img=14, has_cls=True)`` -> O;
    ``backward`` returns gradients for Q, K, V only.  Saved for backward:
    Q, K, V, O, LSE, the packed table (the reference saves COSP/SINP) and
    O's rounding residual where the call keeps one.
    """

    @staticmethod
    def forward(ctx, Q, K, V, cos_sin, H_img=14, has_cls=True):
        rope, n_pos, has_cls, scale, comp = _prepare(Q, K, V, cos_sin, H_img, has_cls)
        O, M, R = attn_fwd(Q, K, V, rope, n_pos, has_cls, scale, comp)
        ctx.softmax_scale = scale
        ctx.comp = comp
        ctx.has_cls = has_cls
        ctx.n_pos = n_pos
        ctx.save_for_backward(Q, K, V, O, M, rope, R)
        return O

    @staticmethod
    def backward(ctx, dO):
        Q, K, V, O, M, rope, R = ctx.saved_tensors
        dQ, dK, dV = attn_bwd(dO, Q, K, V, O, M, rope, ctx.n_pos, ctx.has_cls,
                              ctx.softmax_scale, ctx.comp, R)
        return dQ, dK, dV, None, None, None


def sdpa_triton_fa_rope(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    cos_sin: CosSinTable,
    *,
    H_img: int | None = None,
    has_cls: bool = True,
) -> torch.Tensor:
    """Fused 2D-RoPE attention, fwd + bwd on MI355X (reference FA:1169-1170).

    With the defaults this behaves as the reference's
    ``TritonAttention.apply(Q, K, V, cos_sin)``: a CLS token at index 0 and
    ``SEQ_LEN = 1 + H_img**2``.  ``H_img`` defaults to the side of the
    (square) table in ``cos_sin``, which is 14 for the reference's default
    ``CosSinTable``; ``has_cls=False`` selects ``SEQ_LEN = H_img**2``.
    """
    if H_img is None:
        n_pos = cos_sin.tables()[0].shape[0]
        H_img = math.isqrt(n_pos)
        if H_img * H_img != n_pos:
            raise ValueError(f"RoPE table has {n_pos} rows, not a square H_img x H_img grid")
    rope, n_pos, has_cls, scale, comp = _prepare(Q, K, V, cos_sin, H_img, has_cls)
    O, _, _ = attn_fwd(Q, K, V, rope, n_pos, has_cls, scale, comp)
    return O
