"""Pin the oracle (oracle/torch_ref.py, oracle/numpy_ref.py).

The two restatements are formulated independently (torch: gather-based pair
rotation + torch SDPA + autograd; numpy: explicit rotation matrices +
closed-form gradients).  They are checked against each other, against
finite differences, gradcheck, known-answer special cases and invariants of
RoPE; planted mistakes (made in a copy of the oracle, on the CPU) must be
caught by these checks.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import numpy_ref, torch_ref


def _inputs(B, H, N, D, seed=0, scale=1.0):
    rng = np.random.default_rng(seed)
    return [rng.standard_normal((B, H, N, D)) * scale for _ in range(4)]


CASES = [(2, 2, 3, True, 16), (1, 3, 3, False, 16), (1, 1, 2, True, 8), (2, 1, 4, False, 32)]


@pytest.mark.parametrize("B,H,side,has_cls,D", CASES)
def test_torch_oracle_matches_fp64_closed_form(B, H, side, has_cls, D):
    N = side * side + int(has_cls)
    q, k, v, do = _inputs(B, H, N, D, seed=side + D)
    cos, sin = numpy_ref.axial_tables(side, D, 100.0)
    O, lse = numpy_ref.forward(q, k, v, cos, sin, has_cls)
    dq, dk, dv = numpy_ref.backward(q, k, v, do, cos, sin, has_cls)
    t = lambda a: torch.tensor(a, dtype=torch.float64)
    tc, ts = t(cos), t(sin)
    o2, dq2, dk2, dv2 = torch_ref.forward_backward(t(q), t(k), t(v), t(do), tc, ts, has_cls)
    lse2 = torch_ref.logsumexp_rows(t(q), t(k), tc, ts, has_cls)
    for a, b in ((O, o2), (lse, lse2), (dq, dq2), (dk, dk2), (dv, dv2)):
        assert np.abs(a - b.numpy()).max() < 1e-12


def test_closed_form_gradients_match_finite_differences():
    """numpy_ref.backward vs central differences of numpy_ref.forward (no torch)."""
    B, H, side, has_cls, D = 1, 1, 2, True, 8
    N = side * side + 1
    q, k, v, do = _inputs(B, H, N, D, seed=7)
    cos, sin = numpy_ref.axial_tables(side, D, 100.0)
    grads = numpy_ref.backward(q, k, v, do, cos, sin, has_cls)
    eps = 1e-6
    for which, g in enumerate(grads):
        args = [q.copy(), k.copy(), v.copy()]
        num = np.zeros_like(args[which])
        it = np.nditer(args[which], flags=["multi_index"])
        for _ in it:
            idx = it.multi_index
            a_p = [x.copy() for x in args]
            a_m = [x.copy() for x in args]
            a_p[which][idx] += eps
            a_m[which][idx] -= eps
            fp = (numpy_ref.forward(*a_p, cos, sin, has_cls)[0] * do).sum()
            fm = (numpy_ref.forward(*a_m, cos, sin, has_cls)[0] * do).sum()
            num[idx] = (fp - fm) / (2 * eps)
        assert np.abs(num - g).max() < 1e-7, which


def test_gradcheck_torch_oracle():
    side, D = 2, 8
    cos, sin = torch_ref.axial_tables(side, D, 100.0)
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(1, 2, 5, D, generator=g, dtype=torch.float64, requires_grad=True) for _ in range(3))
    assert torch.autograd.gradcheck(lambda a, b, c: torch_ref.attention(a, b, c, cos, sin, True), (q, k, v))


def test_sdpa_matches_brute_force_softmax():
    """torch SDPA (math) == explicit softmax(QK^T/sqrt(D))V when no rotation is applied."""
    g = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn(2, 3, 7, 16, generator=g, dtype=torch.float64) for _ in range(3))
    ident_c = torch.ones(7, 8, dtype=torch.float64)
    ident_s = torch.zeros(7, 8, dtype=torch.float64)
    o = torch_ref.attention(q, k, v, ident_c, ident_s, False)
    s = q @ k.transpose(-1, -2) / 4.0
    brute = torch.softmax(s, -1) @ v
    assert (o - brute).abs().max() < 1e-12


def test_special_cases():
    side, D = 3, 16
    cos, sin = numpy_ref.axial_tables(side, D, 100.0)
    N = side * side + 1
    q, k, v, _ = _inputs(1, 2, N, D, seed=3)
    # constant V rows -> O equals that row everywhere
    vc = np.broadcast_to(v[:, :, :1, :], v.shape).copy()
    O, _ = numpy_ref.forward(q, k, vc, cos, sin, True)
    assert np.abs(O - vc).max() < 1e-12
    # Q = 0 -> uniform attention -> O = mean_j V_j, LSE = log N
    O, lse = numpy_ref.forward(np.zeros_like(q), k, v, cos, sin, True)
    assert np.abs(O - v.mean(axis=2, keepdims=True)).max() < 1e-12
    assert np.abs(lse - math.log(N)).max() < 1e-12
    # N = 1 (side 1, no CLS) -> O = V
    c1, s1 = numpy_ref.axial_tables(1, D, 100.0)
    q1, k1, v1, _ = _inputs(2, 2, 1, D, seed=4)
    O, _ = numpy_ref.forward(q1, k1, v1, c1, s1, False)
    assert np.abs(O - v1).max() < 1e-12


def test_cls_token_is_not_rotated_and_rotation_is_orthogonal():
    side, D = 3, 16
    cos, sin = torch_ref.axial_tables(side, D, 100.0)
    x = torch.randn(2, 1, side * side + 1, D, dtype=torch.float64)
    xr = torch_ref.apply_rope(x, cos, sin, True)
    assert torch.equal(xr[..., 0, :], x[..., 0, :])
    # per-pair norms preserved
    pn = lambda t: t[..., 0::2] ** 2 + t[..., 1::2] ** 2
    assert (pn(xr) - pn(x)).abs().max() < 1e-12
    R = numpy_ref.rotation_matrices(side * side + 1, cos.numpy(), sin.numpy(), True)
    eye = np.eye(D)
    for s in range(side * side + 1):
        assert np.abs(R[s].T @ R[s] - eye).max() < 1e-12
    # with CLS, token s >= 1 uses table row s - 1: same as dropping the CLS token
    xr2 = torch_ref.apply_rope(x[..., 1:, :], cos, sin, False)
    assert torch.equal(xr2, xr[..., 1:, :])


def test_relative_position_property():
    """<R_m q, R_n k> depends only on the per-axis offset between grid cells m and n."""
    side, D = 6, 16
    cos, sin = numpy_ref.axial_tables(side, D, 100.0)
    R = numpy_ref.rotation_matrices(side * side, cos, sin, False)
    rng = np.random.default_rng(5)
    q, k = rng.standard_normal(D), rng.standard_normal(D)
    cell = lambda r, c: r * side + c
    ref = (R[cell(1, 2)] @ q) @ (R[cell(3, 1)] @ k)
    for dr, dc in ((1, 0), (2, 3), (0, 2)):
        m, n = cell(1 + dr, 2 + dc), cell(3 + dr, 1 + dc)
        assert abs((R[m] @ q) @ (R[n] @ k) - ref) < 1e-12
    # and it does depend on the offset
    other = (R[cell(1, 2)] @ q) @ (R[cell(3, 2)] @ k)
    assert abs(other - ref) > 1e-6


# ---------------------------------------------------------------------------
# Planted mistakes: each mutated restatement must be caught by the torch oracle
# comparison above (so that check really pins sign, axis order, position
# offset, scale and the transpose of the rotation).
# ---------------------------------------------------------------------------
def _mutant_forward(kind, q, k, v, cos, sin, has_cls):
    cos, sin = cos.copy(), sin.copy()
    N, D = q.shape[-2], q.shape[-1]
    P = D // 4
    scale = 1.0 / math.sqrt(D)
    if kind == "sin_sign":
        sin = -sin
    elif kind == "axis_swap":
        cos = np.concatenate([cos[:, P:], cos[:, :P]], 1)
        sin = np.concatenate([sin[:, P:], sin[:, :P]], 1)
    elif kind == "no_scale":
        scale = 1.0
    R = numpy_ref.rotation_matrices(N, cos, sin, has_cls)
    if kind == "pos_offset":
        R = numpy_ref.rotation_matrices(N, np.roll(cos, -1, 0), np.roll(sin, -1, 0), has_cls)
    if kind == "transposed_rotation":
        R = np.transpose(R, (0, 2, 1))
    qh = np.einsum("sij,...sj->...si", R, q)
    kh = np.einsum("sij,...sj->...si", R, k)
    S = scale * np.einsum("...id,...jd->...ij", qh, kh)
    P_ = np.exp(S - S.max(-1, keepdims=True))
    P_ /= P_.sum(-1, keepdims=True)
    return np.einsum("...ij,...jd->...id", P_, v)


@pytest.mark.parametrize("kind", ["sin_sign", "axis_swap", "no_scale", "pos_offset", "transposed_rotation"])
def test_planted_mistakes_are_detected(kind):
    side, D, has_cls = 3, 16, True
    N = side * side + 1
    q, k, v, _ = _inputs(1, 2, N, D, seed=11)
    cos, sin = numpy_ref.axial_tables(side, D, 100.0)
    bad = _mutant_forward(kind, q, k, v, cos, sin, has_cls)
    t = lambda a: torch.tensor(a, dtype=torch.float64)
    good = torch_ref.attention(t(q), t(k), t(v), t(cos), t(sin), has_cls).numpy()
    assert np.abs(bad - good).max() > 1e-3, kind
    # while the unmutated restatement agrees
    assert np.abs(numpy_ref.forward(q, k, v, cos, sin, has_cls)[0] - good).max() < 1e-12
