"""Regenerate the committed golden fixtures from the fp64 numpy oracle.

    python tests/golden/make_golden.py

Writes, next to this file:
  rope_tables.npz  -- COSP/SINP (fp64 closed form) for (side 2, D 8, base 100)
                      and (side 3, D 16, base 10000)
  attention.npz    -- seeded q, k, v, dO (B=1, H=2, D=64) for side 2 with CLS
                      (N=5) and without (N=4), base 100, and the oracle's O,
                      LSE, dQ, dK, dV in fp64
The reference ships no fixtures of its own; these come from oracle/numpy_ref.py,
which tests/test_oracle.py pins independently.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import numpy_ref  # noqa: E402


def main():
    tabs = {}
    for side, D, base in ((2, 8, 100.0), (3, 16, 10000.0)):
        c, s = numpy_ref.axial_tables(side, D, base)
        tabs[f"cos_s{side}_d{D}"] = c
        tabs[f"sin_s{side}_d{D}"] = s
    np.savez_compressed(os.path.join(HERE, "rope_tables.npz"), **tabs)

    out = {}
    rng = np.random.default_rng(2024)
    side, D, base = 2, 64, 100.0
    cos, sin = numpy_ref.axial_tables(side, D, base)
    out["cos"], out["sin"] = cos, sin
    for has_cls in (True, False):
        N = side * side + int(has_cls)
        tag = f"cls{int(has_cls)}"
        # inputs are exactly representable in bf16 so every dtype path sees the same values
        q, k, v, do = (rng.standard_normal((1, 2, N, D)).astype(np.float32) for _ in range(4))
        q, k, v, do = (np.asarray(x.view(np.uint32) & 0xFFFF0000, dtype=np.uint32).view(np.float32) for x in (q, k, v, do))
        O, lse = numpy_ref.forward(q, k, v, cos, sin, has_cls)
        dq, dk, dv = numpy_ref.backward(q, k, v, do, cos, sin, has_cls)
        for name, arr in (("q", q), ("k", k), ("v", v), ("do", do), ("o", O), ("lse", lse),
                          ("dq", dq), ("dk", dk), ("dv", dv)):
            out[f"{tag}_{name}"] = arr
    np.savez_compressed(os.path.join(HERE, "attention.npz"), **out)
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
