"""The general forward (tfgfa_fwd): fp16 and bf16, head dims up to 128, N_q != N_k, strided
operands - the surface of the reference's Triton wrapper _flash_attn_forward
(src/py/triton_implementation.py:184-241).  GPU box only.

Against the CPU oracle (attention_c / attention_np, pinned in tests/test_oracle.py, including
N_q != N_k and other head dims) on the same dtype-rounded inputs: max|dO| <= 2e-2,
mean|dO| <= 2e-3, max|dLSE| <= 1e-3 (Q, K ~ N(0, 2^2), V ~ N(0, 1)).
"""
import math
import sys

import numpy as np
import pytest
import torch

from oracle import attention_c, attention_np

import custom_flash_attn

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TOL_MAX, TOL_MEAN, TOL_LSE = 2e-2, 2e-3, 1e-3
DTYPES = {"bf16": torch.bfloat16, "f16": torch.float16}


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _rand(shape, seed, dtype, sigma=1.0):
    """Returns (device tensor of `dtype`, its values as float32 numpy)."""
    g = np.random.Generator(np.random.PCG64(seed))
    x = torch.from_numpy(g.standard_normal(shape, dtype=np.float32) * np.float32(sigma)).to(dtype)
    return x.to(DEV), x.float().numpy()


def _cu_count():
    return custom_flash_attn.device_info()["cu_count"]


def _heads(grid, B, nq):
    """Heads per batch row that send a (B, H, nq) problem to one kernel: "split" (the split-key
    kernel, whose grid is chosen while B * H * ceil(nq / 128) is at most the CU count) or
    "regular" (fwd_kernel, one workgroup per 128-row query block)."""
    nqb = (nq + 127) // 128
    if grid == "split":
        assert B * 3 * nqb <= _cu_count()
        return 3
    return _cu_count() // (B * nqb) + 1


def _sample(x, B, H):
    """Heads (0, 0), (0, 1) and (B-1, H-1) of a (B, H, ...) array: the oracle checks these."""
    return np.stack([x[0, 0], x[0, 1], x[B - 1, H - 1]])[None]


def _check(o, lse, o_ref, lse_ref, label):
    o = o.float().cpu().numpy().astype(np.float64)
    lse = lse.cpu().numpy().astype(np.float64)
    d = np.abs(o - o_ref)
    dl = np.abs(lse - lse_ref)
    _say(f"{label}: max|dO|={d.max():.3e} mean|dO|={d.mean():.3e} max|dLSE|={dl.max():.3e}")
    assert np.isfinite(o).all() and np.isfinite(lse).all(), label
    assert d.max() <= TOL_MAX and d.mean() <= TOL_MEAN and dl.max() <= TOL_LSE, label


@pytest.mark.parametrize("grid", ["split", "regular"])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("D", [8, 16, 32, 40, 64, 72, 96, 120, 128])
@pytest.mark.parametrize("N,causal", [(65, True), (300, True), (300, False)])
def test_dtypes_and_head_dims(grid, dt, D, N, causal):
    dtype = DTYPES[dt]
    B = 2
    H = _heads(grid, B, N)
    q, qn = _rand((B, H, N, D), 7 * D + N, dtype, 2.0)
    k, kn = _rand((B, H, N, D), 7 * D + N + 1, dtype, 2.0)
    v, vn = _rand((B, H, N, D), 7 * D + N + 2, dtype)
    scale = 1.0 / math.sqrt(D)
    o, lse = custom_flash_attn.attention(q, k, v, causal=causal, return_lse=True)
    torch.cuda.synchronize()
    assert o.dtype == dtype
    o_ref, l_ref = attention_c(_sample(qn, B, H), _sample(kn, B, H), _sample(vn, B, H), scale, causal)
    o_s = torch.stack([o[0, 0], o[0, 1], o[B - 1, H - 1]])[None]
    l_s = torch.stack([lse[0, 0], lse[0, 1], lse[B - 1, H - 1]])[None]
    _check(o_s, l_s, o_ref, l_ref, f"{grid} grid (H={H}) {dt} D={D} N={N} causal={causal}")


@pytest.mark.parametrize("grid", ["split", "regular"])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("nq,nk", [(37, 300), (300, 37), (1, 129), (129, 1), (1000, 1500), (640, 64)])
@pytest.mark.parametrize("causal", [True, False])
def test_query_and_key_lengths_differ(grid, dt, nq, nk, causal):
    dtype = DTYPES[dt]
    D = 64 if nq % 2 else 128
    B = 2
    H = 2 if grid == "split" else _heads(grid, B, nq)
    q, qn = _rand((B, H, nq, D), nq + 3 * nk, dtype, 2.0)
    k, kn = _rand((B, H, nk, D), nq + 3 * nk + 1, dtype, 2.0)
    v, vn = _rand((B, H, nk, D), nq + 3 * nk + 2, dtype)
    o, lse = custom_flash_attn.attention(q, k, v, causal=causal, return_lse=True)
    torch.cuda.synchronize()
    o_ref, l_ref = attention_np(_sample(qn, B, H), _sample(kn, B, H), _sample(vn, B, H),
                                1.0 / math.sqrt(D), causal)
    o_s = torch.stack([o[0, 0], o[0, 1], o[B - 1, H - 1]])[None]
    l_s = torch.stack([lse[0, 0], lse[0, 1], lse[B - 1, H - 1]])[None]
    _check(o_s, l_s, o_ref, l_ref, f"{grid} grid (H={H}) {dt} N_q={nq} N_k={nk} D={D} causal={causal}")


@pytest.mark.parametrize("D", [96, 128])
def test_strided_projection_views_bitwise(D):
    """(B, N, H, D) projection views and an O buffer in that layout: bitwise equal to the
    contiguous call (same instance, the arithmetic does not depend on where rows live)."""
    B, H, N = 2, 3, 333
    x, _ = _rand((3, B, N, H * D), 900 + D, torch.float16, 2.0)
    q, k, v = (x[i].view(B, N, H, D).transpose(1, 2) for i in range(3))
    buf = torch.full((B, N, H, D + 8), 3.0, dtype=torch.float16, device=DEV)
    out, lse = custom_flash_attn.attention(q, k, v, out=buf[..., :D].transpose(1, 2), return_lse=True)
    ref, lse_ref = custom_flash_attn.attention(q.contiguous(), k.contiguous(), v.contiguous(), return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(out.contiguous().view(torch.int16), ref.view(torch.int16))
    assert torch.equal(lse, lse_ref)
    assert (buf[..., D:] == 3.0).all(), "padding after each row written"


def test_head_dim_not_a_multiple_of_8_is_padded():
    D = 36
    q, qn = _rand((1, 2, 200, D), 11, torch.bfloat16, 2.0)
    k, kn = _rand((1, 2, 200, D), 12, torch.bfloat16, 2.0)
    v, vn = _rand((1, 2, 200, D), 13, torch.bfloat16)
    o, lse = custom_flash_attn.attention(q, k, v, return_lse=True)
    torch.cuda.synchronize()
    assert o.shape == (1, 2, 200, D)
    o_ref, l_ref = attention_c(qn, kn, vn, 1.0 / 6.0, True)
    _check(o, lse, o_ref, l_ref, "D=36 padded")


def test_flash_attn_forward_mirror():
    """The Triton wrapper's call: causal, default scale 1/sqrt(d) (also for softmax_scale=0)."""
    q, qn = _rand((2, 4, 150, 80), 21, torch.float16, 2.0)
    k, kn = _rand((2, 4, 220, 80), 22, torch.float16, 2.0)
    v, vn = _rand((2, 4, 220, 80), 23, torch.float16)
    o = custom_flash_attn.flash_attn_forward(q, k, v)
    o0 = custom_flash_attn.flash_attn_forward(q, k, v, 0)
    o3 = custom_flash_attn.flash_attn_forward(q, k, v, 0.3)
    torch.cuda.synchronize()
    assert o.shape == q.shape and o.dtype == torch.float16
    assert torch.equal(o, o0)
    for out, sc in ((o, 1 / math.sqrt(80)), (o3, 0.3)):
        ref, _ = attention_np(qn, kn, vn, sc, True)
        d = np.abs(out.float().cpu().numpy() - ref)
        _say(f"flash_attn_forward scale={sc:.3f}: max|dO|={d.max():.3e}")
        assert d.max() <= TOL_MAX and d.mean() <= TOL_MEAN


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_head_dim_128_at_gpt2_xl_length(dt):
    """B=4, H=16, N=1024, D=128 (sampled rows of every head against the oracle)."""
    dtype = DTYPES[dt]
    B, H, N, D = 4, 16, 1024, 128
    q, qn = _rand((B, H, N, D), 31, dtype, 2.0)
    k, kn = _rand((B, H, N, D), 32, dtype, 2.0)
    v, vn = _rand((B, H, N, D), 33, dtype)
    o, lse = custom_flash_attn.attention(q, k, v, return_lse=True)
    torch.cuda.synchronize()
    rows = np.array([0, 1, 31, 32, 127, 128, 511, 777, 1022, 1023])
    o_ref, l_ref = attention_c(qn, kn, vn, 1.0 / math.sqrt(D), True, rows=rows)
    _check(o[:, :, rows], lse[:, :, rows], o_ref, l_ref, f"{dt} D=128 N=1024")


@pytest.mark.parametrize("grid", ["split", "regular"])
def test_bf16_d64_general_path_equals_forward(grid):
    H = _heads(grid, 2, 257)
    q, _ = _rand((2, H, 257, 64), 41, torch.bfloat16, 3.0)
    k, _ = _rand((2, H, 257, 64), 42, torch.bfloat16, 3.0)
    v, _ = _rand((2, H, 257, 64), 43, torch.bfloat16)
    a = custom_flash_attn.attention(q, k, v)
    b = custom_flash_attn.forward(q, k, v)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("grid", ["split", "regular"])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("D", [64, 128, 40])
@pytest.mark.parametrize("layout", ["contiguous", "projection views"])
@pytest.mark.parametrize("nq,nk,causal", [(1024, 1024, True), (300, 520, False), (97, 97, True)])
def test_o_only_call_equals_o_of_the_lse_call(grid, dt, D, layout, nq, nk, causal):
    """Without an LSE output the kernel does not keep the fp32 probability sum the LSE needs.
    O is normalised by the other sum (of the rounded probabilities) in both cases, so O is
    bitwise the same with and without the LSE, for every instance (dense GPT-2 layout,
    strided, head dims below the compiled ones)."""
    dtype = DTYPES[dt]
    B = 2
    H = _heads(grid, B, nq)
    if layout == "contiguous":
        q, qn = _rand((B, H, nq, D), 40 + D + nq, dtype, 3.0)
        k, kn = _rand((B, H, nk, D), 41 + D + nk, dtype, 3.0)
        v, vn = _rand((B, H, nk, D), 42 + D, dtype)
    else:
        x, _ = _rand((B, nq, 3, H, D), 43 + D + nq, dtype, 3.0)
        y, _ = _rand((B, nk, 2, H, D), 44 + D + nk, dtype, 2.0)
        q = x[:, :, 0].transpose(1, 2)
        k, v = y[:, :, 0].transpose(1, 2), y[:, :, 1].transpose(1, 2)
    o_only = custom_flash_attn.attention(q, k, v, causal=causal)
    o, lse = custom_flash_attn.attention(q, k, v, causal=causal, return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(o_only.view(torch.int16), o.view(torch.int16)), f"{grid} {dt} D={D} {layout}"
    if layout == "contiguous" and nq == 97:
        o_ref, l_ref = attention_c(_sample(qn, B, H), _sample(kn, B, H), _sample(vn, B, H),
                                   1.0 / math.sqrt(D), causal)
        o_s = torch.stack([o_only[0, 0], o_only[0, 1], o_only[B - 1, H - 1]])[None]
        l_s = torch.stack([lse[0, 0], lse[0, 1], lse[B - 1, H - 1]])[None]
        _check(o_s, l_s, o_ref, l_ref, f"O only, {grid} grid, {dt} D={D}")
