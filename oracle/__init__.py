"""CPU oracle for the causal attention forward - TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
may import this package, and only as the checker.  The product path
(``custom_flash_attn`` -> ``libtfgfa.so``) never imports or calls it.

Contents (each restates the reference; file:line cited at each function):
  * bf16 rounding helpers (round-to-nearest-even, as torch's ``.to(torch.bfloat16)``);
  * ``attention_np``      - fp64 numpy restatement of model_inference.py:68-75, plus LSE;
  * ``attention_c``       - the same in C (attention_ref.c), OpenMP, row-sampled;
  * ``decode_np``         - one decode step over a KV cache: the last causal row of the
    same math over the first L cached keys (fp64 numpy);
  * ``manual_attention_torch`` - the reference's PyTorch CPU "manual" branch, fp32
    (the CPU baseline timed by bench.py);
  * ``CONFIGS`` / ``make_inputs`` - the seeded inputs of BASELINE.json's configs.

Pinning (tests/test_oracle.py): against torch's scaled_dot_product_attention in
fp64 (the library routine the reference's own tests use,
test/py/test_cuda_implementation.py:49-52), against a pure-Python brute force on
tiny inputs, and against closed forms (row 0, equal keys, constant V, causality,
permutation).  ``decode_np`` is pinned against ``attention_np``'s last causal row and
fp64 SDPA.  No golden vectors exist in the reference (it has no fixtures).
"""
from .oracle import (  # noqa: F401
    CONFIGS,
    attention_c,
    attention_np,
    bf16_bits_to_f32,
    decode_np,
    bf16_round,
    f32_to_bf16_bits,
    make_inputs,
    manual_attention_torch,
    sha256_bf16,
)
