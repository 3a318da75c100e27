"""MI355X-native fused 2D axial RoPE + FlashAttention-style SDPA (fwd + bwd).

Drop-in for the public API of v1kstrand/triton_fused_rope_flash_attn
("fa_rope_full .py"): ``CosSinTable``, ``build_axial_rope_pairs``,
``sdpa_triton_fa_rope`` and ``TritonAttention``, backed by hand-written
gfx950 HIP kernels in libfarope.so (C ABI: include/farope.h), and
``RoPEAttention``, the ViT attention sub-layer that calls it.
"""
from .rope import CosSinTable, build_axial_rope_pairs, pack_rope_tables
from .attention import TritonAttention, _sdpa_comp_dtype, sdpa_triton_fa_rope
from .block import RoPEAttention

__all__ = [
    "CosSinTable",
    "build_axial_rope_pairs",
    "pack_rope_tables",
    "sdpa_triton_fa_rope",
    "TritonAttention",
    "RoPEAttention",
]
