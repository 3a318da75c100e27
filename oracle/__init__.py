"""CPU/PyTorch restatement of the reference algorithm -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this package, and only as the checker (or as the timed CPU
baseline), never as a code path of the product.  The product
(``triton_fused_rope_flash_attn_amd``) never imports it and has no fallback
to it.

Contents
--------
``torch_ref``  -- the parity target named by the task: Python pairwise 2D
                  RoPE (with CLS bypass) followed by
                  ``torch.nn.functional.scaled_dot_product_attention``
                  (math backend), gradients by torch autograd.  Runs in fp32
                  on CPU, or on the GPU for full-size checks.
``numpy_ref``  -- an independent fp64 restatement: per-token 2x2 rotation
                  matrices, explicit softmax, and closed-form gradients.  It
                  pins ``torch_ref`` (and through it, torch's SDPA) on small
                  inputs.

How each function is pinned (beyond retyping the formula) is listed in the
module docstrings; every function has at least one check in ``tests/``
against a closed form, a library routine, brute force, an invariant, or the
committed golden fixtures in ``tests/golden/``.
"""
