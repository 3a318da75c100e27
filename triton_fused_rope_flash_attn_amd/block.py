"""The ViT attention sub-layer around the fused op: the caller of the hot path.

``RoPEAttention`` is the attention half of a ViT block as the reference's
README benchmarks it (README:142-159, a ``vit_small_patch16_rope_224``-style
model): ``qkv`` Linear -> ``[B, N, 3, H, D]`` -> q, k, v as strided views of
that one buffer (no copies; the kernels take any strides, FA:1043) -> fused
2D-RoPE attention -> ``[B, N, C]`` -> ``proj`` Linear.  The RoPE tables are
a ``CosSinTable`` submodule, so ``state_dict`` carries ``rope.COSP`` /
``rope.SINP`` as the reference's buffers.
"""
from __future__ import annotations

from typing import Callable, Optional

import torch

from .attention import sdpa_triton_fa_rope
from .rope import CosSinTable

__all__ = ["RoPEAttention"]


class RoPEAttention(torch.nn.Module):
    """Multi-head self-attention with fused 2D axial RoPE for a ViT token grid.

    Args:
        dim: embedding width C (= num_heads * head_dim; head_dim % 4 == 0).
        num_heads: H.
        H_img: side of the square patch grid; N = H_img**2 (+1 with a CLS token).
        has_cls: token 0 is a CLS token that bypasses the rotation.
        rope_base: RoPE frequency base (the reference's ViT setting is 100).
        qkv_bias: bias on the fused qkv projection.
        attn: the attention function ``(q, k, v, table, H_img=, has_cls=) -> o``;
            ``sdpa_triton_fa_rope`` unless replaced (tests swap in a reference).
    """

    def __init__(self, dim: int, num_heads: int, H_img: int = 14, has_cls: bool = True,
                 rope_base: float = 100.0, qkv_bias: bool = True,
                 attn: Optional[Callable] = None, device=None, dtype=None):
        super().__init__()
        if dim % num_heads:
            raise ValueError(f"dim {dim} is not a multiple of num_heads {num_heads}")
        self.num_heads = num_heads
        self.head_dim = dim // num_heads
        self.H_img = H_img
        self.has_cls = bool(has_cls)
        self.qkv = torch.nn.Linear(dim, 3 * dim, bias=qkv_bias, device=device, dtype=dtype)
        self.proj = torch.nn.Linear(dim, dim, device=device, dtype=dtype)
        self.rope = CosSinTable(rope_base, H_img, self.head_dim, device=device if device is not None else "cuda")
        self.attn = attn if attn is not None else sdpa_triton_fa_rope

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        B, N, C = x.shape
        qkv = self.qkv(x).view(B, N, 3, self.num_heads, self.head_dim).permute(2, 0, 3, 1, 4)
        q, k, v = qkv.unbind(0)   # [B, H, N, D] views with strides (N*3C, D, 3C, 1)
        o = self.attn(q, k, v, self.rope, H_img=self.H_img, has_cls=self.has_cls)
        return self.proj(o.transpose(1, 2).reshape(B, N, C))
