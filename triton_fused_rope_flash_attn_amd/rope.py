"""2D axial RoPE tables: ``build_axial_rope_pairs`` and ``CosSinTable``.

Same names, signatures, buffer names, shapes and values as the reference
("fa_rope_full .py", FA:10-63 and FA:1140-1166):

* ``COSP`` / ``SINP`` are fp32 ``[H_img**2, D/2]``.  For table row ``l`` the
  first D/4 pairs rotate by ``(l // H_img) * base**(-k/(D/4))`` and the last
  D/4 pairs by ``(l % H_img) * base**(-k/(D/4))`` (the reference calls these
  the "x" and "y" halves; FA:44-51 expand the 1-D table along the row index
  for the first half).
* ``COSP``/``SINP`` are persistent buffers, so ``state_dict`` keys match the
  reference's and checkpoints load unchanged.

The kernels consume a derived table (``CosSinTable.packed()``): fp32
``[(n_pos + 1), D/2, 2]`` with (cos, sin) interleaved per pair and an
identity row 0 for the CLS token.  It is built on the GPU by
``farope_rope_pack`` and cached per COSP/SINP tensor object, version and
storage, so an in-place update (e.g. ``load_state_dict``) or a reassigned
buffer rebuilds it; it is not part of ``state_dict``.
"""
from __future__ import annotations

import math
import weakref

import torch

__all__ = ["build_axial_rope_pairs", "CosSinTable", "pack_rope_tables"]


def build_axial_rope_pairs(
    side_len: int,
    head_dim: int,
    device: torch.device,
    base: float = 10000.0,
):
    """Pairwise 2-D axial RoPE tables for a ``side_len x side_len`` grid.

    Returns ``(cos_pairs, sin_pairs)``, each ``[side_len**2, head_dim // 2]``
    and contiguous.  Follows FA:10-63: frequencies ``base**(-k/P)`` for
    ``k < P = head_dim // 4`` (FA:35), angles ``pos * freq`` for
    ``pos < side_len`` (FA:38-39), row-index half first (FA:46-47, 57-58),
    column-index half second (FA:50-51, 59-60).
    """
    assert head_dim % 4 == 0, "need head_dim divisible by 4 for 2D axial RoPE"
    n_axis = head_dim // 4
    # Same fp32 arithmetic as the reference: int arange / int -> default float.
    freqs = base ** (-torch.arange(0, n_axis, device=device) / n_axis)
    angles = torch.outer(torch.arange(side_len, device=device), freqs)  # [side, n_axis]
    cos_1d, sin_1d = torch.cos(angles), torch.sin(angles)
    lin = torch.arange(side_len * side_len, device=device)
    r_idx, c_idx = lin // side_len, lin % side_len
    cos_pairs = torch.cat([cos_1d[r_idx], cos_1d[c_idx]], dim=1)
    sin_pairs = torch.cat([sin_1d[r_idx], sin_1d[c_idx]], dim=1)
    return cos_pairs.contiguous(), sin_pairs.contiguous()


def pack_rope_tables(cosp: torch.Tensor, sinp: torch.Tensor) -> torch.Tensor:
    """Kernel layout of (COSP, SINP): fp32 [(n_pos+1) * D/2 * 2] on their GPU."""

    if cosp.dim() != 2 or sinp.shape != cosp.shape:
        raise ValueError(
            f"COSP/SINP must both be [N_pos, D/2]; got {tuple(cosp.shape)} and {tuple(sinp.shape)}"
        )
    if cosp.dtype != torch.float32 or sinp.dtype != torch.float32:
        raise TypeError("COSP/SINP must be float32")
    if not cosp.is_cuda or sinp.device != cosp.device:
        raise RuntimeError(
            "farope runs on ROCm GPUs only: the RoPE tables must live on the GPU "
            f"(got {cosp.device} / {sinp.device})"
        )
    return torch.ops.farope.rope_pack(cosp, sinp)


@torch.library.custom_op("farope::rope_pack", mutates_args=())
def _rope_pack_op(cosp: torch.Tensor, sinp: torch.Tensor) -> torch.Tensor:
    """``farope_rope_pack`` as an opaque op, so the packing also traces under torch.compile."""
    from . import _lib

    n_pos, d2 = cosp.shape
    out = torch.empty((n_pos + 1) * d2 * 2, dtype=torch.float32, device=cosp.device)
    _lib.rope_pack(cosp, sinp, out)
    return out


@_rope_pack_op.register_fake
def _rope_pack_fake(cosp, sinp):
    n_pos, d2 = cosp.shape
    return cosp.new_empty(((n_pos + 1) * d2 * 2,))


class CosSinTable(torch.nn.Module):
    """Pairwise axial RoPE tables for an ``H_img x H_img`` grid (FA:1140-1166).

    ``COSP``/``SINP``: ``[H_img*H_img, D//2]`` fp32 persistent buffers.
    """

    def __init__(self, base: float, H_img: int = 14, D: int = 64, device: str = "cuda"):
        super().__init__()
        device = torch.device(device)
        cos_pairs, sin_pairs = build_axial_rope_pairs(
            side_len=H_img, head_dim=D, device=device, base=base
        )
        self.register_buffer("COSP", cos_pairs)
        self.register_buffer("SINP", sin_pairs)
        self._packed = None
        self._packed_key = None

    def tables(self):
        """``(COSP, SINP)``, each ``[N_pos, D2]`` fp32 (FA:1161-1166)."""
        return self.COSP, self.SINP

    def __getstate__(self):
        # The packed-table cache (weak references included) is derived state:
        # pickles and deep copies rebuild it on first use.
        state = self.__dict__.copy()
        state["_packed"] = None
        state["_packed_key"] = None
        return state

    @property
    def H_img(self) -> int:
        n_pos = self.COSP.shape[0]
        side = math.isqrt(n_pos)
        if side * side != n_pos:
            raise ValueError(f"RoPE table has {n_pos} rows, not a square grid")
        return side

    def packed(self) -> torch.Tensor:
        """Kernel-layout table, rebuilt whenever COSP/SINP may have changed.

        The cache holds weak references to the COSP/SINP tensor objects it was
        built from, with their version counters and storage pointers.  It is
        rebuilt when either buffer is a different object (``table.COSP = t``,
        ``.to()``, ``_apply``), was modified in place (``load_state_dict``,
        ``copy_``: the version counter moves) or points at other storage
        (``.data`` reassignment).  A new tensor that happens to reuse a freed
        address is still a different object, so it cannot hit a stale entry.

        Under ``torch.compile`` the table is packed inside the graph on every call
        (one small kernel): the cache key reads storage pointers, which traced
        tensors do not have.
        """
        c, s = self.COSP, self.SINP
        if torch.compiler.is_compiling():
            return pack_rope_tables(c, s)
        key = self._packed_key
        if (
            self._packed is None
            or key is None
            or key[0]() is not c
            or key[1]() is not s
            or key[2:] != (c._version, s._version, c.data_ptr(), s.data_ptr())
        ):
            self._packed = pack_rope_tables(c, s)
            self._packed_key = (weakref.ref(c), weakref.ref(s), c._version, s._version,
                                c.data_ptr(), s.data_ptr())
        return self._packed
