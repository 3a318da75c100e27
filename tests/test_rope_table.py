"""RoPE table builder and CosSinTable (reference FA:10-63, FA:1140-1166).

Pinned by the closed form of the angles, hand-computed known answers,
trigonometric identities and the orientation of the two axis halves.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import numpy_ref, torch_ref
from triton_fused_rope_flash_attn_amd import CosSinTable, build_axial_rope_pairs


@pytest.mark.parametrize("side,D,base", [(2, 8, 100.0), (14, 64, 100.0), (16, 64, 10000.0), (32, 128, 100.0), (3, 4, 7.0)])
def test_closed_form(side, D, base):
    cosp, sinp = build_axial_rope_pairs(side, D, torch.device("cpu"), base=base)
    assert cosp.shape == (side * side, D // 2) and sinp.shape == cosp.shape
    assert cosp.dtype == torch.float32 and cosp.is_contiguous() and sinp.is_contiguous()
    c64, s64 = numpy_ref.axial_tables(side, D, base)
    # fp32 angles (as the reference computes them) vs fp64 closed form:
    # |angle| <= side, fp32 relative error ~6e-8 -> ~3e-6 absolute at side 32.
    assert np.abs(cosp.numpy() - c64).max() < 5e-6
    assert np.abs(sinp.numpy() - s64).max() < 5e-6
    tc, ts = torch_ref.axial_tables(side, D, base)
    assert np.abs(tc.numpy() - c64).max() < 1e-12 and np.abs(ts.numpy() - s64).max() < 1e-12


def test_known_answers_side2_d8():
    """Hand-computed: side 2, D 8 -> P = 2 pairs per axis, w = (1, base^-1/2)."""
    base = 100.0
    cosp, sinp = build_axial_rope_pairs(2, 8, torch.device("cpu"), base=base)
    w1 = base ** -0.5  # 0.1
    # rows: l = 0 (r0,c0), 1 (r0,c1), 2 (r1,c0), 3 (r1,c1)
    exp_ang = np.array([
        [0, 0, 0, 0],
        [0, 0, 1, w1],
        [1, w1, 0, 0],
        [1, w1, 1, w1],
    ])
    assert np.allclose(cosp.numpy(), np.cos(exp_ang), atol=1e-7)
    assert np.allclose(sinp.numpy(), np.sin(exp_ang), atol=1e-7)


def test_row0_is_identity_and_unit_norm():
    cosp, sinp = build_axial_rope_pairs(14, 64, torch.device("cpu"), base=100.0)
    assert torch.equal(cosp[0], torch.ones(32)) and torch.equal(sinp[0], torch.zeros(32))
    assert torch.allclose(cosp ** 2 + sinp ** 2, torch.ones_like(cosp), atol=1e-6)


def test_orientation_first_half_follows_row_index():
    """Pairs p < D/4 depend only on l // side; pairs p >= D/4 only on l % side."""
    side, D = 5, 16
    cosp, _ = build_axial_rope_pairs(side, D, torch.device("cpu"), base=100.0)
    P = D // 4
    g = cosp.view(side, side, D // 2)  # [r, c, pair]
    # first half constant along c, second half constant along r
    assert torch.equal(g[:, :, :P], g[:, :1, :P].expand(side, side, P))
    assert torch.equal(g[:, :, P:], g[:1, :, P:].expand(side, side, P))
    # and the first half really varies with r (pair 0: angle = r)
    assert torch.allclose(g[:, 0, 0], torch.cos(torch.arange(side, dtype=torch.float32)))


def test_fp32_angles_match_reference_arithmetic():
    """Exactly the reference's fp32 expression base ** (-arange(P) / P) * pos."""
    side, D, base = 14, 64, 100.0
    P = D // 4
    inv = base ** (-torch.arange(0, P) / P)
    theta = torch.outer(torch.arange(side), inv)
    cosp, sinp = build_axial_rope_pairs(side, D, torch.device("cpu"), base=base)
    for l in (0, 1, 15, 100, 195):
        r, c = divmod(l, side)
        assert torch.equal(cosp[l, :P], torch.cos(theta[r]))
        assert torch.equal(cosp[l, P:], torch.cos(theta[c]))
        assert torch.equal(sinp[l, P:], torch.sin(theta[c]))


def test_head_dim_must_be_multiple_of_4():
    with pytest.raises(AssertionError, match="divisible by 4"):
        build_axial_rope_pairs(4, 6, torch.device("cpu"))


def test_cossin_table_buffers_and_state_dict():
    t = CosSinTable(100.0, H_img=14, D=64, device="cpu")
    cosp, sinp = t.tables()
    assert cosp is t.COSP and sinp is t.SINP
    assert list(t.state_dict().keys()) == ["COSP", "SINP"]
    assert t.H_img == 14
    ref_c, ref_s = build_axial_rope_pairs(14, 64, torch.device("cpu"), base=100.0)
    assert torch.equal(t.COSP, ref_c) and torch.equal(t.SINP, ref_s)
    # checkpoints produced with the reference's buffer names load unchanged
    t2 = CosSinTable(10000.0, H_img=14, D=64, device="cpu")
    t2.load_state_dict({"COSP": ref_c.clone(), "SINP": ref_s.clone()})
    assert torch.equal(t2.COSP, ref_c)


def test_default_base_argument():
    a = build_axial_rope_pairs(3, 8, torch.device("cpu"))
    b = build_axial_rope_pairs(3, 8, torch.device("cpu"), base=10000.0)
    assert torch.equal(a[0], b[0])
    assert math.isclose(a[0][4, 1].item(), math.cos(10000.0 ** -0.5), rel_tol=1e-6)
