"""Seeded inputs and tolerances shared by the parity tests, bench and smoke.

Input recipe (one per BASELINE config): q, k, v, dO drawn in that order
from ``torch.Generator().manual_seed(seed)`` on the CPU in fp32, scaled,
then cast to the config dtype and moved to the device, so every consumer
sees identical values.  RoPE base 100 everywhere.
"""
from __future__ import annotations

import torch

# north-star tolerance (bf16 vs the fp32 reference): max_abs_err, mean_abs_err
TOL_MAX = 3e-2
TOL_MEAN = 1e-3

CONFIGS = {
    # name: B, H, side (H_img), has_cls, D, dtype, input scale, dO kind
    "cpu": dict(B=2, H=8, side=14, has_cls=True, D=64, dtype=torch.float32, scale=1.0, dout="ones"),
    "vit_s": dict(B=512, H=6, side=14, has_cls=True, D=64, dtype=torch.bfloat16, scale=1.0, dout="randn"),
    "vit_b": dict(B=256, H=12, side=14, has_cls=True, D=64, dtype=torch.bfloat16, scale=1.0, dout="randn"),
    "vit_l": dict(B=128, H=16, side=16, has_cls=False, D=64, dtype=torch.bfloat16, scale=1.0, dout="randn"),
    "hires": dict(B=32, H=12, side=32, has_cls=True, D=128, dtype=torch.bfloat16, scale=2.0, dout="randn"),
}
ROPE_BASE = 100.0


def seq_len(cfg) -> int:
    return cfg["side"] ** 2 + int(cfg["has_cls"])


def make_inputs(cfg, device="cpu", seed=0, dtype=None):
    B, H, D = cfg["B"], cfg["H"], cfg["D"]
    N = seq_len(cfg)
    dtype = dtype or cfg["dtype"]
    g = torch.Generator().manual_seed(seed)
    shape = (B, H, N, D)
    q = torch.randn(shape, generator=g) * cfg["scale"]
    k = torch.randn(shape, generator=g) * cfg["scale"]
    v = torch.randn(shape, generator=g) * cfg["scale"]
    if cfg["dout"] == "ones":
        do = torch.ones(shape)
    else:
        do = torch.randn(shape, generator=g)
    return tuple(t.to(dtype).to(device) for t in (q, k, v, do))


def errors(got: torch.Tensor, ref: torch.Tensor):
    d = (got.float() - ref.float()).abs()
    return d.max().item(), d.mean().item()


def rounding_floor(ref: torch.Tensor, dtype):
    """(max, mean) of |round_to_dtype(ref) - ref|: the error of merely storing the exact answer."""
    d = (ref.to(dtype).float() - ref.float()).abs()
    return d.max().item(), d.mean().item()


# Where storing the exact answer in the output dtype already costs more than
# the fixed tolerance (large-magnitude outputs: HiRes, dO = ones, N = 2), the
# bound becomes FLOOR_MULT x that storage floor.
FLOOR_MULT = 2.0

# Committed per-case ceilings (max_abs_err, mean_abs_err) where the error of
# the standard algorithm itself exceeds FLOOR_MULT x the storage floor, each
# about 1.15x the error measured on MI355X, so a regression shows.
#   N = 2  (side 1 + CLS, D64): measured dQ 1.26e-2 / 1.13e-3, dK 1.44e-2 / 1.13e-3
#          against floors of 2.5e-4 / 3.0e-4 (two tokens: delta = rowsum(dO * O)
#          from the bf16-stored O dominates, FA:352-354 does the same; head_dim 64
#          keeps plain bf16 operands and no O residual)
# (HiRes, B32 H12 N1025 D128 with inputs x2, needs none: its largest ratio to the
# floor is dQ's mean, 2.15e-3 against 1.12e-3, 1.91x.)
CEILINGS = {
    "side1-cls1-D64": {"dQ": (3e-2, 1.3e-3), "dK": (3e-2, 1.3e-3)},
}


def allowed(tag: str, name: str, floor_max: float, floor_mean: float):
    """(max, mean) bound for tensor `name` of case `tag`: the north-star
    tolerance, or FLOOR_MULT x the storage floor where that is larger, or the
    committed ceiling of the case."""
    lim = (max(TOL_MAX, FLOOR_MULT * floor_max), max(TOL_MEAN, FLOOR_MULT * floor_mean))
    if name in CEILINGS.get(tag, {}):
        c = CEILINGS[tag][name]
        lim = (max(lim[0], c[0]), max(lim[1], c[1]))
    return lim
