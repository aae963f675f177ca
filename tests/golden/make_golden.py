"""Writes the committed golden fixtures for the attention forward.

The reference holds no golden vectors or fixtures (its tests draw unseeded torch.randn,
test/py/test_cuda_implementation.py:14-19, :78-80), so these are built here:

  * attn_<case>.npz - small seeded cases at the reference's test lengths
    (T in {10, 11, 15, 33, 63, 65}, test_cuda_implementation.py:93, and T = 128, :74)
    plus edge cases.  Each holds the bf16 bit patterns of Q, K, V (uint16), the
    scale and causal flag, and the expected O and LSE computed in fp64 by
    oracle.attention_np.  Before writing, the expected values are checked against
    torch.nn.functional.scaled_dot_product_attention evaluated in fp64 on the CPU
    (the library routine the reference's tests compare with, :49-52) and against the
    C oracle, so a fixture never records an unchecked number.
  * inputs_sha256.json - SHA-256 of the bf16 bytes of the seeded Q, K, V of
    BASELINE.json configs 1-4 (oracle.make_inputs), pinning the input generator.

Run from the repository root:  python tests/golden/make_golden.py
"""
import json
import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import (  # noqa: E402
    CONFIGS, attention_c, attention_np, bf16_round, f32_to_bf16_bits, make_inputs, sha256_bf16,
)

# name: (B, H, T, D, sigma_qk, causal, scale or None, seed)
CASES = {
    "T1": (1, 2, 1, 64, 1.0, True, None, 11),
    "T10": (1, 2, 10, 64, 1.0, True, None, 12),
    "T11": (1, 2, 11, 64, 1.0, True, None, 13),
    "T15": (1, 2, 15, 64, 1.0, True, None, 14),
    "T33": (1, 2, 33, 64, 1.0, True, None, 15),
    "T63": (1, 2, 63, 64, 1.0, True, None, 16),
    "T65": (1, 2, 65, 64, 1.0, True, None, 17),
    "T128": (2, 2, 128, 64, 1.0, True, None, 18),
    "T129_sigma3": (1, 2, 129, 64, 3.0, True, None, 19),
    "T96_noncausal": (1, 2, 96, 64, 1.0, False, None, 20),
    "T70_scale0.3": (1, 2, 70, 64, 1.0, True, 0.3, 21),
}


def make_case(B, H, T, D, sigma, causal, scale, seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    shape = (B, H, T, D)
    q = bf16_round(rng.standard_normal(shape, dtype=np.float32) * np.float32(sigma))
    k = bf16_round(rng.standard_normal(shape, dtype=np.float32) * np.float32(sigma))
    v = bf16_round(rng.standard_normal(shape, dtype=np.float32))
    s = 1.0 / math.sqrt(D) if scale is None else scale
    o, lse = attention_np(q, k, v, s, causal)

    # Cross-checks before anything is written.
    ref = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q).double(), torch.from_numpy(k).double(), torch.from_numpy(v).double(),
        is_causal=causal, scale=s,
    ).numpy()
    assert np.max(np.abs(ref - o)) < 1e-12, "oracle disagrees with torch SDPA (fp64)"
    oc, lc = attention_c(q, k, v, s, causal)
    assert np.max(np.abs(oc - o)) < 1e-12 and np.max(np.abs(lc - lse)) < 1e-12
    return dict(
        q_bits=f32_to_bf16_bits(q), k_bits=f32_to_bf16_bits(k), v_bits=f32_to_bf16_bits(v),
        scale=np.float64(s), causal=np.bool_(causal), o=o, lse=lse,
    )


def main():
    for name, spec in CASES.items():
        path = os.path.join(HERE, f"attn_{name}.npz")
        np.savez_compressed(path, **make_case(*spec))
        print("wrote", os.path.relpath(path, ROOT))
    hashes = {}
    for cname, cfg in CONFIGS.items():
        q, k, v = make_inputs(cfg)
        hashes[cname] = {"q": sha256_bf16(q), "k": sha256_bf16(k), "v": sha256_bf16(v),
                         "shape": [cfg.B, cfg.H, cfg.N, cfg.D], "seed": cfg.seed,
                         "sigma_qk": cfg.sigma_qk, "sigma_v": cfg.sigma_v}
    with open(os.path.join(HERE, "inputs_sha256.json"), "w") as f:
        json.dump(hashes, f, indent=1, sort_keys=True)
    print("wrote tests/golden/inputs_sha256.json")


if __name__ == "__main__":
    main()
