"""Host-side behaviour of the Python API (no GPU needed).

Covers the reference's argument checks and messages (FA:1016-1021), the
compute-dtype rule (FA:65-73), the no-fallback rule (CPU tensors raise),
RoPE-table validation, and the custom ops' fake (meta) kernels.
"""
from __future__ import annotations

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

from triton_fused_rope_flash_attn_amd import CosSinTable, TritonAttention, _sdpa_comp_dtype, sdpa_triton_fa_rope
from triton_fused_rope_flash_attn_amd import attention


def _qkv(B=2, H=3, N=197, D=64, dtype=torch.bfloat16):
    return [torch.randn(B, H, N, D).to(dtype) for _ in range(3)]


def test_comp_dtype_follows_input_without_autocast():
    for dt in (torch.float32, torch.float16, torch.bfloat16):
        assert _sdpa_comp_dtype(torch.zeros(1, dtype=dt)) == dt


def test_comp_dtype_follows_autocast(monkeypatch):
    monkeypatch.setattr(torch, "is_autocast_enabled", lambda *a: True)
    monkeypatch.setattr(torch, "get_autocast_dtype", lambda dev: torch.bfloat16)
    assert _sdpa_comp_dtype(torch.zeros(1, dtype=torch.float32)) == torch.bfloat16


def test_comp_dtype_rejects_other_dtypes():
    with pytest.raises(TypeError):
        _sdpa_comp_dtype(torch.zeros(1, dtype=torch.float64))


def test_head_dim_assert_message():
    q, k, v = _qkv(D=66)
    table = CosSinTable(100.0, 14, 64, device="cpu")
    with pytest.raises(AssertionError, match=r"HEAD_DIM must be divisible by 4 \(2D RoPE requires pairs\)\."):
        TritonAttention.apply(q, k, v, table)


def test_seq_len_assert_messages():
    table = CosSinTable(100.0, 14, 64, device="cpu")
    q, k, v = _qkv(N=196)
    with pytest.raises(AssertionError, match=r"SEQ_LEN must be 1 \+ H_img\*W_img when has_cls=True \(got 196 vs 197\)\."):
        TritonAttention.apply(q, k, v, table)
    q, k, v = _qkv(N=197)
    with pytest.raises(AssertionError, match=r"SEQ_LEN must equal H_img\*W_img when has_cls=False \(got 197 vs 196\)\."):
        TritonAttention.apply(q, k, v, table, 14, False)


def test_public_entry_defaults_match_reference():
    """sdpa_triton_fa_rope(Q, K, V, cos_sin) == TritonAttention.apply(Q, K, V, cos_sin): CLS, H_img 14."""
    table = CosSinTable(100.0, 14, 64, device="cpu")
    q, k, v = _qkv(N=196)
    with pytest.raises(AssertionError, match="got 196 vs 197"):
        sdpa_triton_fa_rope(q, k, v, table)


def test_cpu_tensors_fail_loudly_no_fallback():
    table = CosSinTable(100.0, 14, 64, device="cpu")
    q, k, v = _qkv()
    with pytest.raises(RuntimeError, match="ROCm GPUs only"):
        sdpa_triton_fa_rope(q, k, v, table)
    with pytest.raises(RuntimeError, match="ROCm GPUs only"):
        table.packed()


def test_mixed_dtypes_rejected():
    table = CosSinTable(100.0, 14, 64, device="cpu")
    q, k, v = _qkv()
    with pytest.raises(TypeError, match="share one dtype"):
        sdpa_triton_fa_rope(q, k.float(), v, table)


def test_table_shape_is_checked_against_the_call():
    table = CosSinTable(100.0, 14, 64, device="cpu")
    with pytest.raises(ValueError, match="does not match the call"):
        attention.rope_operand(table, 196, 128, torch.device("cpu"))
    with pytest.raises(ValueError, match="does not match the call"):
        attention.rope_operand(table, 256, 64, torch.device("cpu"))


def test_h_img_inferred_from_square_table_only():
    class Odd:
        def tables(self):
            return torch.zeros(10, 32), torch.zeros(10, 32)

    q, k, v = _qkv(N=11)
    with pytest.raises(ValueError, match="not a square"):
        sdpa_triton_fa_rope(q, k, v, Odd())


def test_fake_kernels_shapes_and_dtypes():
    with FakeTensorMode():
        q = torch.empty(2, 3, 197, 64, dtype=torch.bfloat16, device="cuda")
        rope = torch.empty(197 * 32 * 2, dtype=torch.float32, device="cuda")
        o, lse, res = torch.ops.farope.attn_fwd(q, q, q, rope, 196, True, 0.125, 2)
        assert o.shape == q.shape and o.dtype == q.dtype
        assert lse.shape == (2, 3, 197) and lse.dtype == torch.float32
        assert res.shape == (0,)   # head_dim 64: no residual
        q128 = torch.empty(2, 3, 197, 128, dtype=torch.bfloat16, device="cuda")
        rope128 = torch.empty(197 * 64 * 2, dtype=torch.float32, device="cuda")
        o2, _, res2 = torch.ops.farope.attn_fwd(q128, q128, q128, rope128, 196, True, 0.088, 2)
        assert res2.shape == q128.shape and res2.dtype == torch.bfloat16
        dq, dk, dv = torch.ops.farope.attn_bwd(q, q, q, q, o, lse, rope, 196, True, 0.125, 2, res)
        for t in (dq, dk, dv):
            assert t.shape == q.shape and t.dtype == q.dtype
        cosp = torch.empty(196, 32, dtype=torch.float32, device="cuda")
        packed = torch.ops.farope.rope_pack(cosp, cosp)
        assert packed.shape == (197 * 32 * 2,) and packed.dtype == torch.float32


def test_custom_ops_registered_with_autograd():
    assert hasattr(torch.ops.farope, "attn_fwd") and hasattr(torch.ops.farope, "attn_bwd")
    from torch._library.custom_ops import CustomOpDef

    assert isinstance(attention.attn_fwd, CustomOpDef)


def test_rope_attention_block_passes_strided_views():
    """The ViT block hands the op q/k/v as views of one qkv buffer (no copies)."""
    from triton_fused_rope_flash_attn_amd import RoPEAttention

    seen = {}

    def spy(q, k, v, table, H_img=None, has_cls=True):
        seen.update(shape=q.shape, strides=(q.stride(), k.stride(), v.stride()), H_img=H_img,
                    has_cls=has_cls, base=q.untyped_storage().data_ptr(),
                    offs=(q.storage_offset(), k.storage_offset(), v.storage_offset()),
                    table=table.tables()[0].shape)
        return q * 0

    B, N, C, H = 2, 197, 384, 6
    blk = RoPEAttention(C, H, H_img=14, has_cls=True, attn=spy, device="cpu")
    out = blk(torch.randn(B, N, C))
    D = C // H
    assert out.shape == (B, N, C)
    assert seen["shape"] == (B, H, N, D)
    assert seen["strides"] == ((N * 3 * C, D, 3 * C, 1),) * 3
    assert seen["offs"] == (0, C, 2 * C)
    assert seen["H_img"] == 14 and seen["has_cls"] is True
    assert seen["table"] == (196, D // 2)
    assert {"rope.COSP", "rope.SINP"} <= set(blk.state_dict())


def test_rope_attention_block_cpu_fails_loudly():
    from triton_fused_rope_flash_attn_amd import RoPEAttention

    blk = RoPEAttention(128, 2, H_img=4, has_cls=False, device="cpu")
    with pytest.raises(RuntimeError, match="ROCm GPUs only"):
        blk(torch.randn(1, 16, 128))


@pytest.mark.parametrize("has_cls", [True, False])
def test_bench_torch_rope_matches_oracle(has_cls):
    """bench.py's torch-ROCm comparison applies its own Python RoPE; it must be
    the oracle's rotation."""
    import importlib.util
    import pathlib

    from oracle import torch_ref
    from triton_fused_rope_flash_attn_amd import build_axial_rope_pairs

    spec = importlib.util.spec_from_file_location("bench", pathlib.Path(__file__).parents[1] / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    side, D = 4, 32
    N = side * side + int(has_cls)
    cosp, sinp = build_axial_rope_pairs(side, D, torch.device("cpu"), base=100.0)
    x = torch.randn(2, 3, N, D, generator=torch.Generator().manual_seed(1))
    torch.testing.assert_close(bench.torch_rope(x, cosp, sinp, has_cls),
                               torch_ref.apply_rope(x, cosp, sinp, has_cls), rtol=0, atol=0)


def test_packed_table_cache_invalidation(monkeypatch):
    """CosSinTable.packed() repacks after load_state_dict (in place), buffer
    reassignment, .data reassignment and in-place edits, and reuses the cache
    otherwise; pickles and deep copies drop the cache (it is derived state).
    The GPU packer is replaced by a counting stand-in."""
    import copy
    import pickle

    from triton_fused_rope_flash_attn_amd import rope as rope_mod

    calls = []

    def fake_pack(c, s):
        calls.append((c.clone(), s.clone()))
        return torch.cat([c.flatten(), s.flatten()])

    monkeypatch.setattr(rope_mod, "pack_rope_tables", fake_pack)
    t = CosSinTable(100.0, 4, 16, device="cpu")
    a = t.packed()
    assert len(calls) == 1 and t.packed() is a and len(calls) == 1
    other = CosSinTable(10000.0, 4, 16, device="cpu")
    t.load_state_dict(other.state_dict())
    b = t.packed()
    assert len(calls) == 2 and torch.equal(calls[-1][0], other.COSP)
    t.COSP = other.COSP.clone() * 0.5
    t.packed()
    assert len(calls) == 3 and torch.equal(calls[-1][0], other.COSP * 0.5)
    t.SINP.data = torch.zeros_like(t.SINP)
    t.packed()
    assert len(calls) == 4 and torch.equal(calls[-1][1], torch.zeros_like(t.SINP))
    t.COSP.mul_(2.0)
    t.packed()
    assert len(calls) == 5 and t.packed() is not b and len(calls) == 5
    assert len(pickle.dumps(t)) > 0   # the weak references are not pickled
    clone = copy.deepcopy(t)
    assert clone._packed is None and clone._packed_key is None
    assert torch.equal(clone.COSP, t.COSP)
    n = len(calls)
    clone.packed()
    assert len(calls) == n + 1


def test_residual_rule_matches_library():
    """attention._uses_residual (used for allocation and the fake kernels)
    agrees with the library's farope_attn_residual_elems for every dtype pair
    and head_dim."""
    from triton_fused_rope_flash_attn_amd import _lib

    for io in (_lib.F32, _lib.F16, _lib.BF16):
        for ct in (_lib.F32, _lib.F16, _lib.BF16):
            for D in (32, 64, 128, 256):
                desc = _lib.make_desc(2, 3, 197, D, 196, True, io, ct, D ** -0.5)
                n = _lib.residual_elems(desc)
                assert (n > 0) == attention._uses_residual(io, ct, D), (io, ct, D)
                assert n in (0, 2 * 3 * 197 * D)
