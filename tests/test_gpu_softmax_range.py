"""The forward's softmax over extreme score patterns (GPU box only).

The kernel keeps a per-row exp2 offset that moves only when a lane's running sum of its
probabilities, as rounded for the MFMA, would pass a bound (bf16: 2^64; fp16: the largest finite
float, passed exactly when a probability rounds to +inf, i.e. leaves fp16's range), or (a wave's
last half) when a score passes it by a margin (60 log2 units for bf16, 15 for fp16); a move
rescales O and both sums and recomputes the half's probabilities.  Random inputs at the configs'
scales move it about once per row, so these cases force the other paths: scores that climb by
far more than the margin every half (a move on every half, with rescale factors that underflow
to 0), scores that fall (no move after the first half), halves that alternate high and low,
scores of magnitude ~1e4 (one-hot rows), and probabilities at each element type's own bound.

Oracle: attention_np (fp64, tests/test_oracle.py) on the same bf16/fp16-rounded inputs.
Tolerances as everywhere: max|dO| <= 2e-2, mean|dO| <= 2e-3; LSE within 1e-3 plus the fp32
rounding of an LSE of that magnitude (4e-7 relative; it matters only for the ~1e4 case).
"""
import math
import sys

import numpy as np
import pytest
import torch

from oracle import attention_np

import custom_flash_attn

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
DTYPES = {"bf16": torch.bfloat16, "f16": torch.float16}


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _case(kind, N, D, seed, dtype):
    """q, k, v float32 arrays (1, 2, N, D) holding dtype-representable values."""
    g = np.random.Generator(np.random.PCG64(seed))
    q = g.standard_normal((1, 2, N, D), dtype=np.float32) * 0.1
    k = g.standard_normal((1, 2, N, D), dtype=np.float32) * 0.1
    v = g.standard_normal((1, 2, N, D), dtype=np.float32)
    j = np.arange(N, dtype=np.float32)
    # With q[..., 0] = 8, adding c to k[..., 0] adds 8 * c / sqrt(D) to the score (natural log
    # units); unit(A) is the c that adds A.
    unit = lambda a: a * math.sqrt(D) / 8.0
    if kind == "rising":      # +0.75 per key (~35 log2 units per 32-key half)
        q[..., 0] = 8.0
        k[..., 0] += unit(0.75) * j
    elif kind == "falling":   # the first keys dominate; later probabilities underflow
        q[..., 0] = 8.0
        k[..., 0] += unit(0.75) * (N - j)
    elif kind == "zigzag":    # 32-key halves alternately +40 and -40
        q[..., 0] = 8.0
        k[..., 0] += unit(40.0) * np.where((j // 32) % 2 == 0, 1.0, -1.0)
    elif kind == "huge":      # scores of order 1e3: one-hot rows
        q *= 3000.0
        k *= 30.0
    t = DTYPES[dtype]
    rnd = lambda x: torch.from_numpy(x).to(t).float().numpy()
    return rnd(q), rnd(k), rnd(v)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("kind", ["rising", "falling", "zigzag", "huge"])
@pytest.mark.parametrize("N,D", [(300, 64), (1024, 64), (700, 128)])
def test_extreme_score_patterns(kind, N, D, dtype):
    q, k, v = _case(kind, N, D, 17 * N + D, dtype)
    t = DTYPES[dtype]
    qd, kd, vd = (torch.from_numpy(x).to(t).to(DEV) for x in (q, k, v))
    scale = 1.0 / math.sqrt(D)
    o, lse = custom_flash_attn.attention(qd, kd, vd, return_lse=True)
    o_only = custom_flash_attn.attention(qd, kd, vd)  # the instance without the LSE's sum
    torch.cuda.synchronize()
    assert torch.equal(o_only.view(torch.int16), o.view(torch.int16)), "O-only call differs"
    o_ref, l_ref = attention_np(q, k, v, scale, True)
    o = o.float().cpu().numpy().astype(np.float64)
    lse = lse.cpu().numpy().astype(np.float64)
    d = np.abs(o - o_ref)
    dl = np.abs(lse - l_ref)
    span = np.abs(l_ref).max()
    _say(f"{kind} {dtype} N={N} D={D}: |LSE| up to {span:.1f}; max|dO|={d.max():.3e} "
         f"mean|dO|={d.mean():.3e} max|dLSE|={dl.max():.3e}")
    assert np.isfinite(o).all() and np.isfinite(lse).all(), "non-finite output"
    assert d.max() <= 2e-2 and d.mean() <= 2e-3
    assert (dl <= 1e-3 + 4e-7 * np.abs(l_ref)).all()


def _range_case(N, v_scale, positive):
    """Scores built so that the lane sums sit just under the kernel's 2^64 bound: q = (16, 0,
    ...), k_j = (0, ...) for j < 32 and (20.75, 0, ...) after, so every later key scores
    16 * 20.75 / 8 = 41.5 (59.87 log2 units) above the offset set by keys 0..31 and each
    probability is 2^59.87 (a lane's 16 of them sum to 2^63.87): the P.V of keys 32..63 runs
    with those probabilities, the next half's running sum passes 2^64 and moves the offset.
    V is v_scale times N(0, 1) clipped to +-7.99 (or |N(0, 1)| + 0.5 when ``positive``)."""
    g = np.random.Generator(np.random.PCG64(N + int(math.log2(v_scale))))
    q = np.zeros((1, 2, N, 64), dtype=np.float32)
    k = np.zeros((1, 2, N, 64), dtype=np.float32)
    q[..., 0] = 16.0
    k[:, :, 32:, 0] = 20.75
    z = g.standard_normal((1, 2, N, 64), dtype=np.float32)
    z = np.abs(z) + 0.5 if positive else np.clip(z, -7.99, 7.99)
    v = torch.from_numpy(z * np.float32(v_scale)).to(torch.bfloat16).float().numpy()
    return q, k, v


def test_bf16_range_inside_bound_matches_oracle():
    """Just inside the documented bound of the lazy offset (include/tfgfa.h: bf16 O stays finite
    while max|V| < 2^62): N = 1024, max|V| < 2^61, probabilities of 2^59.87 in the P.V of keys
    32..63.  O must be finite and match the fp64 oracle relative to V's scale (the absolute
    2e-2 / 2e-3 gates divided by 2^58); LSE as everywhere."""
    N, vs = 1024, 2.0 ** 58
    q, k, v = _range_case(N, vs, positive=False)
    assert np.abs(v).max() < 2.0 ** 62
    qd, kd, vd = (torch.from_numpy(x).to(torch.bfloat16).to(DEV) for x in (q, k, v))
    o, lse = custom_flash_attn.forward_lse(qd, kd, vd)
    o_only = custom_flash_attn.forward(qd, kd, vd)
    torch.cuda.synchronize()
    assert torch.equal(o_only.view(torch.int16), o.view(torch.int16)), "O-only call differs"
    o_ref, l_ref = attention_np(q, k, v, 0.125, True)
    o = o.float().cpu().numpy().astype(np.float64)
    lse = lse.cpu().numpy().astype(np.float64)
    d = np.abs(o - o_ref) / vs
    dl = np.abs(lse - l_ref)
    _say(f"range inside bound: max|V| = 2^{math.log2(np.abs(v).max()):.2f}; "
         f"max|dO|/2^58={d.max():.3e} mean={d.mean():.3e} max|dLSE|={dl.max():.3e}")
    assert np.isfinite(o).all() and np.isfinite(lse).all()
    assert d.max() <= 2e-2 and d.mean() <= 2e-3
    assert dl.max() <= 1e-3


def test_bf16_range_past_bound_overflows_as_documented():
    """Past the bound (all V near 2^66, N = 1024) the P.V of keys 32..63 at 2^59.87 leaves fp32
    for rows that see a few of them, and those rows come out non-finite, as include/tfgfa.h
    states (the exact-offset reference stays finite there).  Rows 0..31 and every LSE are
    unaffected."""
    N, vs = 1024, 2.0 ** 66
    q, k, v = _range_case(N, vs, positive=True)
    qd, kd, vd = (torch.from_numpy(x).to(torch.bfloat16).to(DEV) for x in (q, k, v))
    o, lse = custom_flash_attn.forward_lse(qd, kd, vd)
    torch.cuda.synchronize()
    o_ref, l_ref = attention_np(q, k, v, 0.125, True)
    o = o.float().cpu().numpy().astype(np.float64)
    lse = lse.cpu().numpy().astype(np.float64)
    assert np.isfinite(lse).all() and np.abs(lse - l_ref).max() <= 1e-3
    # Rows 0..31 attend only to keys of probability 1: finite, equal to the oracle.
    assert np.isfinite(o[:, :, :32]).all()
    assert (np.abs(o[:, :, :32] - o_ref[:, :, :32]) / vs).max() <= 2e-2
    # The last row's P.V of keys 32..63 is about 32 * 2^59.87 * 1.3 * 2^66 > 2^128.
    finite_rows = np.isfinite(o).all(axis=-1)
    _say(f"range past bound: non-finite rows {int((~finite_rows).sum())} of {finite_rows.size}")
    assert not finite_rows[:, :, -1].any()


@pytest.mark.parametrize("log2p", [15.9, 16.1])
def test_f16_probabilities_at_the_edge_of_fp16(log2p):
    """fp16 at its own bound: q = (16, 0, ...), k_j = 0 for j < 32 and (c, 0, ...) after, so every
    later key scores log2p log2 units above the offset set by keys 0..31.  At 15.9 each rounded
    probability (2^15.9 ~ 61147) is finite in fp16: no move, and the P.V of every later half runs
    with those probabilities.  At 16.1 (2^16.1 ~ 70240 > 65504) the conversion gives +inf, the
    rounded sum passes the bound and the offset moves.  Both must match the fp64 oracle with every
    output finite, O-only bitwise equal to O + LSE."""
    N, D = 1024, 64
    c = torch.tensor(log2p * 8.0 / (16.0 * math.log2(math.e)), dtype=torch.float16).item()
    q = np.zeros((1, 2, N, D), dtype=np.float32)
    k = np.zeros((1, 2, N, D), dtype=np.float32)
    q[..., 0] = 16.0
    k[:, :, 32:, 0] = c
    g = np.random.Generator(np.random.PCG64(int(log2p * 10)))
    v = torch.from_numpy(g.standard_normal((1, 2, N, D), dtype=np.float32)).half().float().numpy()
    qd, kd, vd = (torch.from_numpy(x).half().to(DEV) for x in (q, k, v))
    o, lse = custom_flash_attn.attention(qd, kd, vd, return_lse=True)
    o_only = custom_flash_attn.attention(qd, kd, vd)
    torch.cuda.synchronize()
    assert torch.equal(o_only.view(torch.int16), o.view(torch.int16)), "O-only call differs"
    o_ref, l_ref = attention_np(q, k, v, 1.0 / math.sqrt(D), True)
    o = o.float().cpu().numpy().astype(np.float64)
    lse = lse.cpu().numpy().astype(np.float64)
    d = np.abs(o - o_ref)
    dl = np.abs(lse - l_ref)
    _say(f"fp16 edge 2^{log2p}: c={c}; max|dO|={d.max():.3e} mean|dO|={d.mean():.3e} "
         f"max|dLSE|={dl.max():.3e}")
    assert np.isfinite(o).all() and np.isfinite(lse).all(), "non-finite output"
    assert d.max() <= 2e-2 and d.mean() <= 2e-3
    assert (dl <= 1e-3 + 4e-7 * np.abs(l_ref)).all()
