"""fp64 numpy restatement with closed-form gradients (pins ``torch_ref``).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Formulated differently from ``torch_ref`` on purpose:
  * the rotation of token s is an explicit D x D block-diagonal matrix R_s
    (2x2 blocks [[c, -s], [s, c]] on channel pairs (2p, 2p+1);
    FA:200-202), the CLS token's R is the identity (FA:177-179);
  * softmax is written out with a running max (FA:280-309);
  * gradients use the closed forms the reference kernels implement:
      dV = P^T dO                                  (FA:623-627)
      delta_i = sum_d dO_id O_id                   (FA:352-354)
      dS = P * (dO V^T - delta)                    (FA:630-631)
      dK = R^T (scale * dS^T Q_hat)                (FA:634-662)
      dQ = R^T (scale * dS K_hat)                  (FA:968-993)
Tables come from ``axial_tables`` (closed form of FA:10-63) or are passed in.
"""
from __future__ import annotations

import math

import numpy as np


def axial_tables(side: int, head_dim: int, base: float):
    """(cos, sin) fp64 ``[side*side, head_dim//2]``: first D/4 pairs follow the
    row index l // side, last D/4 pairs the column index l % side."""
    assert head_dim % 4 == 0
    P = head_dim // 4
    cos = np.empty((side * side, head_dim // 2))
    sin = np.empty_like(cos)
    for l in range(side * side):
        r, c = divmod(l, side)
        for p in range(P):
            w = base ** (-p / P)
            cos[l, p], sin[l, p] = math.cos(r * w), math.sin(r * w)
            cos[l, P + p], sin[l, P + p] = math.cos(c * w), math.sin(c * w)
    return cos, sin


def rotation_matrices(n: int, cos: np.ndarray, sin: np.ndarray, has_cls: bool) -> np.ndarray:
    """R[s] (D x D) for tokens s < n."""
    d2 = cos.shape[1]
    D = 2 * d2
    R = np.zeros((n, D, D))
    for s in range(n):
        if has_cls and s == 0:
            R[s] = np.eye(D)
            continue
        l = max(s - int(has_cls), 0)
        for p in range(d2):
            c, sn = cos[l, p], sin[l, p]
            R[s, 2 * p, 2 * p] = c
            R[s, 2 * p, 2 * p + 1] = -sn
            R[s, 2 * p + 1, 2 * p] = sn
            R[s, 2 * p + 1, 2 * p + 1] = c
    return R


def _rotate(x: np.ndarray, R: np.ndarray) -> np.ndarray:
    # x [..., N, D], R [N, D, D]: out[..., s, :] = R[s] @ x[..., s, :]
    return np.einsum("sij,...sj->...si", R, x)


def forward(q, k, v, cos, sin, has_cls: bool, scale: float | None = None):
    """(O, LSE) in fp64 for q, k, v [B, H, N, D]."""
    q, k, v = (np.asarray(t, dtype=np.float64) for t in (q, k, v))
    N, D = q.shape[-2], q.shape[-1]
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    R = rotation_matrices(N, np.asarray(cos, np.float64), np.asarray(sin, np.float64), has_cls)
    qh, kh = _rotate(q, R), _rotate(k, R)
    S = scale * np.einsum("...id,...jd->...ij", qh, kh)
    m = S.max(axis=-1, keepdims=True)
    E = np.exp(S - m)
    l = E.sum(axis=-1, keepdims=True)
    P = E / l
    O = np.einsum("...ij,...jd->...id", P, v)
    lse = (m + np.log(l))[..., 0]
    return O, lse


def backward(q, k, v, do, cos, sin, has_cls: bool, scale: float | None = None):
    """(dQ, dK, dV) in fp64 from the closed-form gradient."""
    q, k, v, do = (np.asarray(t, dtype=np.float64) for t in (q, k, v, do))
    N, D = q.shape[-2], q.shape[-1]
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    R = rotation_matrices(N, np.asarray(cos, np.float64), np.asarray(sin, np.float64), has_cls)
    qh, kh = _rotate(q, R), _rotate(k, R)
    S = scale * np.einsum("...id,...jd->...ij", qh, kh)
    S = S - S.max(axis=-1, keepdims=True)
    P = np.exp(S)
    P = P / P.sum(axis=-1, keepdims=True)
    O = np.einsum("...ij,...jd->...id", P, v)
    dV = np.einsum("...ij,...id->...jd", P, do)
    dP = np.einsum("...id,...jd->...ij", do, v)
    delta = (do * O).sum(axis=-1, keepdims=True)
    dS = P * (dP - delta)
    dqh = scale * np.einsum("...ij,...jd->...id", dS, kh)
    dkh = scale * np.einsum("...ij,...id->...jd", dS, qh)
    Rt = np.transpose(R, (0, 2, 1))
    return _rotate(dqh, Rt), _rotate(dkh, Rt), dV
