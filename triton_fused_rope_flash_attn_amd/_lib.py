"""ctypes binding of libfarope.so (the C ABI declared in include/farope.h).

Tensors cross the boundary as raw device pointers plus int64 element
strides; the HIP stream is torch's current stream on the tensors' device.
There is no fallback: if the library is missing or a call fails, a
RuntimeError says why.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libfarope.so")

F32, F16, BF16 = 0, 1, 2
DTYPE_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

# Status codes (farope_status).
OK = 0
(ERR_NULL, ERR_HEAD_DIM, ERR_SEQ_LEN, ERR_DTYPE, ERR_TABLE, ERR_SHAPE, ERR_LAUNCH, ERR_ALIGN,
 ERR_SCRATCH) = range(1, 10)
NOALLOC_MAX_ROWS = 4194304   # FAROPE_NOALLOC_MAX_ROWS

# Every function the header declares; tests check the library exports all of them.
EXPORTS = (
    "farope_abi_version",
    "farope_strerror",
    "farope_rope_packed_elems",
    "farope_rope_pack",
    "farope_attn_residual_elems",
    "farope_attn_bwd_workspace_elems",
    "farope_attn_fwd",
    "farope_attn_bwd_preprocess",
    "farope_attn_bwd_dk_dv",
    "farope_attn_bwd_dq",
    "farope_attn_bwd",
    "farope_attn_bwd_noalloc",
    "farope_tile_config",
)


class AttnDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("seq_len", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("n_pos", ctypes.c_int32),
        ("has_cls", ctypes.c_int32),
        ("io_dtype", ctypes.c_int32),
        ("compute_dtype", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float),
    ]


Stride4 = ctypes.c_int64 * 4
_P = ctypes.c_void_p
_S = ctypes.POINTER(ctypes.c_int64)
_D = ctypes.POINTER(AttnDesc)
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_Z = ctypes.c_size_t

_SIGNATURES = {
    "farope_abi_version": (ctypes.c_int, []),
    "farope_strerror": (ctypes.c_char_p, [ctypes.c_int]),
    "farope_rope_packed_elems": (ctypes.c_size_t, [_I32, _I32]),
    "farope_rope_pack": (ctypes.c_int, [_P, _I64, _I64, _P, _I64, _I64, _I32, _I32, _P, _P]),
    "farope_attn_residual_elems": (ctypes.c_size_t, [_D]),
    "farope_attn_bwd_workspace_elems": (ctypes.c_size_t, [_D]),
    "farope_attn_fwd": (ctypes.c_int, [_D, _P, _S, _P, _S, _P, _S, _P, _Z, _P, _S, _P, _P, _P]),
    "farope_attn_bwd_preprocess": (ctypes.c_int, [_D, _P, _S, _P, _P, _S, _P, _P]),
    "farope_attn_bwd_dk_dv": (
        ctypes.c_int,
        [_D, _P, _S, _P, _S, _P, _S, _P, _S, _P, _P, _P, _Z, _P, _S, _P, _S, _P],
    ),
    "farope_attn_bwd_dq": (ctypes.c_int, [_D, _P, _S, _P, _S, _P, _S, _P, _S, _P, _P, _P, _Z, _P, _S, _P]),
    "farope_attn_bwd": (
        ctypes.c_int,
        [_D, _P, _S, _P, _S, _P, _S, _P, _S, _P, _P, _S, _P, _P, _Z, _P, _S, _P, _S, _P, _S, _P, _P],
    ),
    "farope_attn_bwd_noalloc": (
        ctypes.c_int,
        [_D, _P, _S, _P, _S, _P, _S, _P, _S, _P, _P, _S, _P, _P, _Z, _P, _S, _P, _S, _P, _S, _P],
    ),
    "farope_tile_config": (ctypes.c_int, [_D, _I32, ctypes.POINTER(ctypes.c_int32)]),
}

_lib = None
_lock = threading.Lock()


def load() -> ctypes.CDLL:
    """Load libfarope.so once (after torch, so both share torch's HIP runtime)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"farope: HIP library not found at {LIB_PATH}; build it with "
                    "`python -m triton_fused_rope_flash_attn_amd.build` (or __graft_entry__.build())"
                )
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def strerror(rc: int) -> str:
    return load().farope_strerror(rc).decode()


def check(rc: int, what: str) -> None:
    if rc != OK:
        raise RuntimeError(f"{what}: {strerror(rc)} (status {rc})")


def strides(t: torch.Tensor) -> Stride4:
    return Stride4(*t.stride())


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def make_desc(B, H, N, D, n_pos, has_cls, io_dtype, compute_dtype, scale) -> AttnDesc:
    return AttnDesc(B, H, N, D, n_pos, int(bool(has_cls)), io_dtype, compute_dtype, float(scale))


def tile_config(desc: AttnDesc, which: int) -> tuple[int, int, int, int]:
    out = (ctypes.c_int32 * 4)()
    check(load().farope_tile_config(ctypes.byref(desc), which, out), "farope_tile_config")
    return tuple(out)


def rope_pack(cosp: torch.Tensor, sinp: torch.Tensor, out: torch.Tensor) -> None:
    n_pos, d2 = cosp.shape
    with torch.cuda.device(cosp.device):
        rc = load().farope_rope_pack(
            cosp.data_ptr(), cosp.stride(0), cosp.stride(1),
            sinp.data_ptr(), sinp.stride(0), sinp.stride(1),
            n_pos, d2, out.data_ptr(), stream_of(cosp),
        )
    check(rc, "farope_rope_pack")


def residual_elems(desc: AttnDesc) -> int:
    """Elements of the O-residual buffer the call uses (0: none); see farope_attn_residual_elems."""
    return int(load().farope_attn_residual_elems(ctypes.byref(desc)))


def bwd_workspace_elems(desc: AttnDesc) -> int:
    """fp32 elements of attn_bwd's delta workspace; see farope_attn_bwd_workspace_elems."""
    return int(load().farope_attn_bwd_workspace_elems(ctypes.byref(desc)))


def _ptr(t) -> int | None:
    """Device pointer of an optional buffer: None for a missing or empty tensor."""
    return t.data_ptr() if t is not None and t.numel() > 0 else None


def attn_fwd(desc: AttnDesc, q, k, v, rope, o, lse, o_res=None) -> None:
    rc = load().farope_attn_fwd(
        ctypes.byref(desc),
        q.data_ptr(), strides(q), k.data_ptr(), strides(k), v.data_ptr(), strides(v),
        rope.data_ptr(), rope.numel(), o.data_ptr(), strides(o), _ptr(o_res), lse.data_ptr(), stream_of(q),
    )
    check(rc, "farope_attn_fwd")


def attn_bwd(desc: AttnDesc, q, k, v, o, do, lse, rope, dq, dk, dv, delta, o_res=None) -> None:
    rc = load().farope_attn_bwd(
        ctypes.byref(desc),
        q.data_ptr(), strides(q), k.data_ptr(), strides(k), v.data_ptr(), strides(v),
        o.data_ptr(), strides(o), _ptr(o_res), do.data_ptr(), strides(do),
        lse.data_ptr(), rope.data_ptr(), rope.numel(),
        dq.data_ptr(), strides(dq), dk.data_ptr(), strides(dk), dv.data_ptr(), strides(dv),
        _ptr(delta), stream_of(q),
    )
    check(rc, "farope_attn_bwd")


def attn_bwd_noalloc(desc: AttnDesc, q, k, v, o, do, lse, rope, dq, dk, dv, o_res=None) -> None:
    """farope_attn_bwd_noalloc: the backward with the library's static delta workspace."""
    rc = load().farope_attn_bwd_noalloc(
        ctypes.byref(desc),
        q.data_ptr(), strides(q), k.data_ptr(), strides(k), v.data_ptr(), strides(v),
        o.data_ptr(), strides(o), _ptr(o_res), do.data_ptr(), strides(do),
        lse.data_ptr(), rope.data_ptr(), rope.numel(),
        dq.data_ptr(), strides(dq), dk.data_ptr(), strides(dk), dv.data_ptr(), strides(dv),
        stream_of(q),
    )
    check(rc, "farope_attn_bwd_noalloc")


def attn_bwd_preprocess(desc: AttnDesc, o, do, delta, o_res=None) -> None:
    rc = load().farope_attn_bwd_preprocess(
        ctypes.byref(desc), o.data_ptr(), strides(o), _ptr(o_res), do.data_ptr(), strides(do),
        delta.data_ptr(), stream_of(o),
    )
    check(rc, "farope_attn_bwd_preprocess")


def attn_bwd_dk_dv(desc: AttnDesc, q, k, v, do, lse, delta, rope, dk, dv) -> None:
    rc = load().farope_attn_bwd_dk_dv(
        ctypes.byref(desc),
        q.data_ptr(), strides(q), k.data_ptr(), strides(k), v.data_ptr(), strides(v),
        do.data_ptr(), strides(do), lse.data_ptr(), delta.data_ptr(), rope.data_ptr(), rope.numel(),
        dk.data_ptr(), strides(dk), dv.data_ptr(), strides(dv), stream_of(q),
    )
    check(rc, "farope_attn_bwd_dk_dv")


def attn_bwd_dq(desc: AttnDesc, q, k, v, do, lse, delta, rope, dq) -> None:
    rc = load().farope_attn_bwd_dq(
        ctypes.byref(desc),
        q.data_ptr(), strides(q), k.data_ptr(), strides(k), v.data_ptr(), strides(v),
        do.data_ptr(), strides(do), lse.data_ptr(), delta.data_ptr(), rope.data_ptr(), rope.numel(),
        dq.data_ptr(), strides(dq), stream_of(q),
    )
    check(rc, "farope_attn_bwd_dq")
