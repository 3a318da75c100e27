"""PyTorch restatement: Python 2D RoPE + torch SDPA (the parity target).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Follows "fa_rope_full .py" (FA:n = line n):
  * ``axial_tables``   -- the pairwise tables of build_axial_rope_pairs
                          (FA:10-63), restated from the closed form.
  * ``apply_rope``     -- pair rotation (2p, 2p+1) with position
                          ``max(s - has_cls, 0)`` and the CLS row left
                          unrotated (FA:176-202, FA:248-272).
  * ``attention``      -- softmax(scale * q_hat k_hat^T) v via
                          ``F.scaled_dot_product_attention`` (math backend),
                          scale = 1/sqrt(D) (FA:1024); autograd gives
                          dQ/dK/dV (the contract of FA:1067-1138).
  * ``logsumexp_rows`` -- the per-row log-sum-exp the forward kernel stores
                          (FA:308-309, without the +1e-9).

Pinned by tests/test_oracle.py against the fp64 restatement in
``numpy_ref`` (independent formulation, closed-form gradients), finite
differences, ``torch.autograd.gradcheck``, special cases with known
answers, and the committed fixtures in tests/golden/.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel


def axial_tables(side: int, head_dim: int, base: float, dtype=torch.float64, device="cpu"):
    """(cos, sin) ``[side*side, head_dim//2]`` from the closed form (FA:10-63).

    Row l, pair p < P (P = head_dim//4): angle = (l // side) * base**(-p/P);
    pair p >= P: angle = (l % side) * base**(-(p-P)/P).
    """
    assert head_dim % 4 == 0
    P = head_dim // 4
    rows = torch.tensor([[l // side] for l in range(side * side)], dtype=torch.float64)
    cols = torch.tensor([[l % side] for l in range(side * side)], dtype=torch.float64)
    w = torch.tensor([base ** (-p / P) for p in range(P)], dtype=torch.float64)[None, :]
    ang = torch.cat([rows * w, cols * w], dim=1)
    return ang.cos().to(dtype=dtype, device=device), ang.sin().to(dtype=dtype, device=device)


def apply_rope(x: torch.Tensor, cosp: torch.Tensor, sinp: torch.Tensor, has_cls: bool) -> torch.Tensor:
    """Rotate channel pairs (2p, 2p+1) of ``x`` [..., N, D] by the table rows of each token.

    Token s uses row max(s - has_cls, 0); with has_cls the token at s = 0
    is returned unchanged (FA:177-179, FA:200-202).
    """
    N = x.shape[-2]
    pos = torch.clamp(torch.arange(N, device=x.device) - int(has_cls), min=0)
    c = cosp.to(device=x.device, dtype=x.dtype)[pos]  # [N, D/2]
    s = sinp.to(device=x.device, dtype=x.dtype)[pos]
    xe, xo = x[..., 0::2], x[..., 1::2]
    re = xe * c - xo * s
    ro = xo * c + xe * s
    out = torch.stack([re, ro], dim=-1).flatten(-2)
    if has_cls:
        out = torch.cat([x[..., :1, :], out[..., 1:, :]], dim=-2)
    return out


def attention(q, k, v, cosp, sinp, has_cls: bool, scale: float | None = None) -> torch.Tensor:
    """O = softmax(scale * R(q) R(k)^T) v with torch SDPA (math backend)."""
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    qh = apply_rope(q, cosp, sinp, has_cls)
    kh = apply_rope(k, cosp, sinp, has_cls)
    with sdpa_kernel([SDPBackend.MATH]):
        return F.scaled_dot_product_attention(qh, kh, v, scale=scale)


def logsumexp_rows(q, k, cosp, sinp, has_cls: bool, scale: float | None = None) -> torch.Tensor:
    """LSE[b, h, i] = logsumexp_j(scale * q_hat_i . k_hat_j), natural log."""
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    qh = apply_rope(q, cosp, sinp, has_cls)
    kh = apply_rope(k, cosp, sinp, has_cls)
    s = torch.matmul(qh, kh.transpose(-2, -1).contiguous()) * scale
    return torch.logsumexp(s, dim=-1)


def forward_backward(q, k, v, do, cosp, sinp, has_cls: bool, scale: float | None = None):
    """(O, dQ, dK, dV) of ``attention`` for upstream gradient ``do``, in q's dtype."""
    q = q.detach().requires_grad_(True)
    k = k.detach().requires_grad_(True)
    v = v.detach().requires_grad_(True)
    with torch.enable_grad():
        o = attention(q, k, v, cosp, sinp, has_cls, scale)
        dq, dk, dv = torch.autograd.grad(o, (q, k, v), grad_outputs=do)
    return o.detach(), dq, dk, dv
