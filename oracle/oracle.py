"""CPU oracle for the causal attention forward - TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use this
module, as the checker; the product path never does.
"""
from __future__ import annotations

import ctypes
import hashlib
import math
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))

# --------------------------------------------------------------------------------------
# bf16 helpers.  The reference stores Q/K/V as torch.bfloat16 (the tests build them with
# dtype=torch.bfloat16, test/py/test_cuda_implementation.py:78-80); torch rounds fp32 to
# bf16 to nearest, ties to even.  These restate that rounding on the fp32 bit pattern.


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float32 values to bf16 (nearest, ties to even); return the uint16 bit patterns."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounding = np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))
    return ((b + rounding) >> np.uint32(16)).astype(np.uint16)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """Widen bf16 bit patterns (uint16) to float32 exactly."""
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(
        np.float32
    )


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bf16 value, returned as float32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def sha256_bf16(x: np.ndarray) -> str:
    """SHA-256 of the bf16 bytes of a bf16-representable float32 array."""
    return hashlib.sha256(f32_to_bf16_bits(x).tobytes()).hexdigest()


# --------------------------------------------------------------------------------------
# Reference semantics.


def attention_np(q, k, v, scale: float | None = None, causal: bool = True):
    """fp64 restatement of the reference's "manual" branch (src/py/model_inference.py:68-75).

    q: (..., N_q, D); k, v: (..., N_k, D) (N_k = N_q in the reference's model; the Triton
    wrapper allows N_k != N_q, src/py/triton_implementation.py:185-189).  Returns (o, lse) in
    float64 with o of q's shape and lse of shape (..., N_q): lse_i = log(sum_j exp(scale *
    q_i.k_j)) as src/py/triton_implementation.py:153-154 accumulates it.  The causal mask is
    triu(ones, diagonal=1) -> -inf (model_inference.py:55, :70-71), top-left aligned for
    N_q != N_k as in the Triton kernel (:127): key j is visible to query i iff j <= i.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    n, d = q.shape[-2], q.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(d)  # model_inference.py:72 divides by sqrt(head_dim)
    s = np.matmul(q, np.swapaxes(k, -1, -2)) * scale
    if causal:
        mask = np.triu(np.ones((n, k.shape[-2]), dtype=bool), k=1)
        s = np.where(mask, -np.inf, s)
    m = np.max(s, axis=-1, keepdims=True)
    p = np.exp(s - m)
    l = np.sum(p, axis=-1, keepdims=True)
    o = np.matmul(p / l, v)
    lse = (m + np.log(l))[..., 0]
    return o, lse


_LIB = None


def _lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"oracle library missing: build it with `make -C {_HERE}`")
        lib = ctypes.CDLL(path)
        lib.oracle_attn_fwd.restype = ctypes.c_int
        lib.oracle_attn_fwd.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_long, ctypes.c_long, ctypes.c_long, ctypes.c_double, ctypes.c_int,
            ctypes.c_void_p, ctypes.c_long,
        ]
        _LIB = lib
    return _LIB


def attention_c(q, k, v, scale: float | None = None, causal: bool = True, rows=None):
    """Same semantics as :func:`attention_np`, in C (attention_ref.c), for large shapes.

    q, k, v: float32 arrays (B, H, N, D) (bf16-rounded values).  ``rows`` optionally
    selects query rows (a 1-D int array); outputs then cover only those rows:
    o (B, H, len(rows), D) and lse (B, H, len(rows)), float64.
    """
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    *lead, n, d = q.shape
    bh = int(np.prod(lead)) if lead else 1
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    if rows is None:
        nrows, rows_arr = n, None
    else:
        rows_arr = np.ascontiguousarray(rows, dtype=np.int64)
        if rows_arr.size and (rows_arr.min() < 0 or rows_arr.max() >= n):
            raise ValueError("row index out of range")
        nrows = rows_arr.size
    o = np.empty((*lead, nrows, d), dtype=np.float64)
    lse = np.empty((*lead, nrows), dtype=np.float64)
    st = _lib().oracle_attn_fwd(
        q.ctypes.data, k.ctypes.data, v.ctypes.data, o.ctypes.data, lse.ctypes.data,
        bh, n, d, float(scale), 1 if causal else 0,
        None if rows_arr is None else rows_arr.ctypes.data, nrows,
    )
    if st != 0:
        raise RuntimeError(f"oracle_attn_fwd failed with status {st}")
    return o, lse


def decode_np(q, k_cache, v_cache, lens, scale: float | None = None):
    """One decode step over a KV cache, fp64: the last row of the causal forward.

    The reference has no KV cache; its generate() recomputes the causal forward over the
    prefix for every new token (src/py/model_inference.py:199-228) and keeps the last row,
    whose value under the "manual" branch (:68-75) is
        o = softmax_j(scale * q . k_j) v_j over j < L,   lse = log sum_j exp(scale * q . k_j).
    q: (B, H, D); k_cache, v_cache: (B, H, N_max, D); lens: B ints (keys attended per batch
    row, 0 <= L <= N_max).  Returns (o (B, H, D), lse (B, H)) in float64; L = 0 gives o = 0,
    lse = -inf.
    """
    q = np.asarray(q, dtype=np.float64)
    k_cache = np.asarray(k_cache, dtype=np.float64)
    v_cache = np.asarray(v_cache, dtype=np.float64)
    B, H, D = q.shape
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    o = np.zeros((B, H, D), dtype=np.float64)
    lse = np.full((B, H), -np.inf, dtype=np.float64)
    for b in range(B):
        L = int(lens[b])
        if L == 0:
            continue
        s = np.einsum("hjd,hd->hj", k_cache[b, :, :L], q[b]) * scale
        m = s.max(axis=-1, keepdims=True)
        p = np.exp(s - m)
        l = p.sum(axis=-1, keepdims=True)
        o[b] = np.einsum("hj,hjd->hd", p / l, v_cache[b, :, :L])
        lse[b] = (m + np.log(l))[:, 0]
    return o, lse


def manual_attention_torch(q, k, v):
    """The reference's PyTorch CPU attention path, fp32 (src/py/model_inference.py:68-75).

    q, k, v: CPU float32 tensors (B, H, N, D).  Computes the full N x N score matrix,
    masks with triu(diagonal=1), divides by sqrt(d) and applies softmax, then @ V -
    exactly the steps of the "manual" branch (dropout is the identity in eval mode).
    Returns (B, H, N, D) (the reference then transposes to (B, N, H, D), :75).
    """
    import torch

    n = q.shape[-2]
    attn = q @ k.transpose(-2, -1)
    mask_bool = torch.triu(torch.ones(n, n), diagonal=1).bool()
    attn.masked_fill_(mask_bool, -torch.inf)
    attn_weights = torch.softmax(attn / k.shape[-1] ** 0.5, dim=-1)
    return attn_weights @ v


# --------------------------------------------------------------------------------------
# BASELINE.json configs 1-4 (config 5, the GPT-2-medium forward, lives in the tests).


@dataclass(frozen=True)
class AttnConfig:
    name: str
    B: int
    H: int
    N: int
    D: int
    sigma_qk: float
    sigma_v: float
    seed: int

    @property
    def scale(self) -> float:
        return 1.0 / math.sqrt(self.D)

    @property
    def flops(self) -> float:
        """Algorithmic FLOPs, FlashAttention causal convention: 4*B*H*N^2*d / 2."""
        return 4.0 * self.B * self.H * self.N * self.N * self.D / 2.0

    @property
    def bytes(self) -> float:
        """Algorithmic HBM bytes: bf16 Q, K, V read + O written, fp32 LSE written."""
        return 2.0 * 4 * self.B * self.H * self.N * self.D + 4.0 * self.B * self.H * self.N


CONFIGS = {
    "config1": AttnConfig("config1", 1, 12, 256, 64, 1.0, 1.0, 1001),
    "config2": AttnConfig("config2", 8, 12, 1024, 64, 1.0, 1.0, 1002),
    "config3": AttnConfig("config3", 8, 25, 1024, 64, 3.0, 1.0, 1003),
    "config4": AttnConfig("config4", 1, 16, 8192, 64, 1.0, 1.0, 1004),
}


def make_inputs(cfg: AttnConfig):
    """Seeded Q, K, V for a config: iid normal from numpy PCG64(seed), drawn in the
    order Q, K, V as float32, times sigma, rounded to bf16 (returned as float32)."""
    rng = np.random.Generator(np.random.PCG64(cfg.seed))
    shape = (cfg.B, cfg.H, cfg.N, cfg.D)
    q = bf16_round(rng.standard_normal(shape, dtype=np.float32) * np.float32(cfg.sigma_qk))
    k = bf16_round(rng.standard_normal(shape, dtype=np.float32) * np.float32(cfg.sigma_qk))
    v = bf16_round(rng.standard_normal(shape, dtype=np.float32) * np.float32(cfg.sigma_v))
    return q, k, v
