"""Committed golden fixtures (tests/golden/, made by make_golden.py from the fp64 oracle).

CPU: both oracles and the package's table builder reproduce the fixtures.
GPU: the HIP path through the C ABI reproduces them (fp32 compute tightly,
bf16 compute within the north-star tolerance).
"""
from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch

from oracle import numpy_ref, torch_ref
from triton_fused_rope_flash_attn_amd import build_axial_rope_pairs

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    with np.load(os.path.join(HERE, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_tables_match_fixture():
    g = _load("rope_tables.npz")
    for side, D, base in ((2, 8, 100.0), (3, 16, 10000.0)):
        c, s = numpy_ref.axial_tables(side, D, base)
        assert np.array_equal(c, g[f"cos_s{side}_d{D}"]) and np.array_equal(s, g[f"sin_s{side}_d{D}"])
        cp, sp = build_axial_rope_pairs(side, D, torch.device("cpu"), base=base)
        assert np.abs(cp.numpy() - g[f"cos_s{side}_d{D}"]).max() < 5e-7
        assert np.abs(sp.numpy() - g[f"sin_s{side}_d{D}"]).max() < 5e-7


@pytest.mark.parametrize("has_cls", [True, False])
def test_oracles_match_fixture(has_cls):
    g = _load("attention.npz")
    t = f"cls{int(has_cls)}"
    args = [g[f"{t}_{n}"] for n in ("q", "k", "v")]
    O, lse = numpy_ref.forward(*args, g["cos"], g["sin"], has_cls)
    dq, dk, dv = numpy_ref.backward(*args, g[f"{t}_do"], g["cos"], g["sin"], has_cls)
    for name, arr in (("o", O), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert np.abs(arr - g[f"{t}_{name}"]).max() < 1e-12, name
    T = lambda a: torch.tensor(a, dtype=torch.float64)
    o2, dq2, dk2, dv2 = torch_ref.forward_backward(*(T(a) for a in args), T(g[f"{t}_do"]),
                                                    T(g["cos"]), T(g["sin"]), has_cls)
    for name, arr in (("o", o2), ("dq", dq2), ("dk", dk2), ("dv", dv2)):
        assert np.abs(arr.numpy() - g[f"{t}_{name}"]).max() < 1e-10, name


@pytest.mark.gpu
@pytest.mark.parametrize("has_cls", [True, False])
@pytest.mark.parametrize("dtype,tol", [(torch.float32, 2e-5), (torch.bfloat16, 3e-2)])
def test_gpu_path_matches_fixture(has_cls, dtype, tol):
    from triton_fused_rope_flash_attn_amd import CosSinTable, sdpa_triton_fa_rope

    g = _load("attention.npz")
    t = f"cls{int(has_cls)}"
    dev = "cuda"
    table = CosSinTable(100.0, H_img=2, D=64, device=dev)
    q, k, v = (torch.tensor(g[f"{t}_{n}"]).to(dtype).to(dev).requires_grad_(True) for n in ("q", "k", "v"))
    do = torch.tensor(g[f"{t}_do"]).to(dtype).to(dev)
    o = sdpa_triton_fa_rope(q, k, v, table, has_cls=has_cls)
    o.backward(do)
    torch.cuda.synchronize()
    for name, got in (("o", o), ("dq", q.grad), ("dk", k.grad), ("dv", v.grad)):
        want = g[f"{t}_{name}"]
        err = np.abs(got.detach().float().cpu().numpy() - want).max()
        print(f"[golden {t} {dtype}] {name}: max_abs_err={err:.3e}", flush=True)
        assert err < tol * max(1.0, float(np.abs(want).max())), name
    # LSE through the raw op
    o2, lse, _ = torch.ops.farope.attn_fwd(q.detach(), k.detach(), v.detach(), table.packed(), 4, has_cls,
                                         1 / math.sqrt(64), {torch.float32: 0, torch.bfloat16: 2}[dtype])
    assert np.abs(lse.cpu().numpy() - g[f"{t}_lse"]).max() < tol * 10
