"""CPU: source-level rules of the HIP kernels.

Every 16-byte buffer store goes through ``buf_store16`` (csrc/common.h),
which puts a wait state behind the store: the compiler inserts it only when
the store's soffset is an inline constant, and a VALU write of the data
registers directly behind a store with an SGPR soffset made a kernel store
values that changed from call to call (tests/test_gpu_repeat.py).
"""
from __future__ import annotations

import os
import re

CSRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                    "triton_fused_rope_flash_attn_amd", "csrc")


def _sources():
    for name in sorted(os.listdir(CSRC)):
        if name.endswith((".hip", ".h")):
            with open(os.path.join(CSRC, name)) as fh:
                yield name, fh.read()


def test_16_byte_buffer_stores_use_the_guarded_helper():
    raw = re.compile(r"__builtin_amdgcn_raw_buffer_store_b(96|128)\s*\(")
    found = []
    for name, text in _sources():
        for m in raw.finditer(text):
            line = text.count("\n", 0, m.start()) + 1
            found.append((name, line))
    # the one allowed use: inside buf_store16 itself
    helper = [(n, l) for n, l in found if n == "common.h"]
    others = [(n, l) for n, l in found if n != "common.h"]
    assert not others, f"16-byte buffer stores outside buf_store16: {others}"
    assert len(helper) == 1, f"common.h should hold exactly the helper's store, found {helper}"
    common = dict(_sources())["common.h"]
    body = common[common.index("void buf_store16("):]
    body = body[:body.index("\n}\n")]
    assert 'asm volatile("s_nop 0"' in body, "buf_store16 lost its wait state"
