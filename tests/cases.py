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
    # name: B, H, side (H_img), has_cls, D, dtype, input scale, dO kind[, seed]
    "cpu": dict(B=2, H=8, side=14, has_cls=True, D=64, dtype=torch.float32, scale=1.0, dout="ones"),
    # ViT-S has ViT-B's B*H and N: with the same seed its flat random stream,
    # and so every plane's inputs, would repeat ViT-B's exactly
    "vit_s": dict(B=512, H=6, side=14, has_cls=True, D=64, dtype=torch.bfloat16, scale=1.0, dout="randn",
                  seed=1),
    "vit_b": dict(B=256, H=12, side=14, has_cls=True, D=64, dtype=torch.bfloat16, scale=1.0, dout="randn"),
    "vit_l": dict(B=128, H=16, side=16, has_cls=False, D=64, dtype=torch.bfloat16, scale=1.0, dout="randn"),
    "hires": dict(B=32, H=12, side=32, has_cls=True, D=128, dtype=torch.bfloat16, scale=2.0, dout="randn"),
}
ROPE_BASE = 100.0


def seq_len(cfg) -> int:
    return cfg["side"] ** 2 + int(cfg["has_cls"])


def make_inputs(cfg, device="cpu", seed=None, dtype=None):
    """q, k, v, dO of config `cfg` from `seed` (default: the config's own, else 0)."""
    B, H, D = cfg["B"], cfg["H"], cfg["D"]
    N = seq_len(cfg)
    dtype = dtype or cfg["dtype"]
    g = torch.Generator().manual_seed(cfg.get("seed", 0) if seed is None else seed)
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

# Committed per-case ceilings (max_abs_err, mean_abs_err) for cases where
# the standard algorithm itself exceeds FLOOR_MULT x the storage floor, each
# about 1.15x the error measured on MI355X, so a regression shows.  None is
# needed: the two-token plane (side 1 + CLS, D 64), where delta from the
# bf16-stored O used to cost dQ / dK a mean error of 1.13e-3, now takes
# delta = sum_k P dP inside the one-pass backward (every plane of N <= 32),
# and measures 4.7e-4 / 4.2e-4.  (HiRes, B32 H12 N1025 D128 with inputs x2,
# needs none either: its largest ratio to the floor is dQ's mean, 2.15e-3
# against 1.12e-3, 1.91x.)
CEILINGS: dict = {}


def allowed(tag: str, name: str, floor_max: float, floor_mean: float):
    """(max, mean) bound for tensor `name` of case `tag`: the north-star
    tolerance, or FLOOR_MULT x the storage floor where that is larger, or the
    committed ceiling of the case."""
    lim = (max(TOL_MAX, FLOOR_MULT * floor_max), max(TOL_MEAN, FLOOR_MULT * floor_mean))
    if name in CEILINGS.get(tag, {}):
        c = CEILINGS[tag][name]
        lim = (max(lim[0], c[0]), max(lim[1], c[1]))
    return lim
