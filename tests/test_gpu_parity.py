"""Parity of the HIP kernel with the CPU oracle (GPU box only).

Tolerances: against the fp64/fp32 oracle on the same
bf16-rounded inputs, max|dO| <= 2e-2 and mean|dO| <= 2e-3; LSE (natural log) max
abs error <= 1e-3.  Shapes: BASELINE.json configs 1-4 (config 1 and 2 in full,
config 3 and 4 on sampled query rows of every head), the reference's boundary
lengths (test/py/test_cuda_implementation.py:93) and more edge cases.

Every call goes through the C ABI (via custom_flash_attn / _C).
"""
import json
import math
import os
import sys

import numpy as np
import pytest
import torch

from oracle import CONFIGS, attention_c, bf16_bits_to_f32, make_inputs, sha256_bf16

import custom_flash_attn
from custom_flash_attn import _C

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL_MAX, TOL_MEAN, TOL_LSE = 2e-2, 2e-3, 1e-3
DEV = "cuda:0"


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _to_dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(torch.bfloat16).to(DEV)


def _run(q, k, v, scale=None, causal=True):
    """numpy float32 (bf16-valued) inputs -> (O float32 numpy, LSE numpy)."""
    qd, kd, vd = _to_dev(q), _to_dev(k), _to_dev(v)
    o, lse = custom_flash_attn.forward_lse(qd, kd, vd, softmax_scale=scale, causal=causal)
    torch.cuda.synchronize()
    return o.float().cpu().numpy(), lse.cpu().numpy()


def _check(o, lse, o_ref, lse_ref, label):
    d = np.abs(o.astype(np.float64) - o_ref)
    dl = np.abs(lse.astype(np.float64) - lse_ref)
    _say(f"{label}: max|dO|={d.max():.3e} mean|dO|={d.mean():.3e} max|dLSE|={dl.max():.3e}")
    assert np.isfinite(o).all() and np.isfinite(lse).all(), f"{label}: non-finite output"
    assert d.max() <= TOL_MAX, f"{label}: max|dO| {d.max()}"
    assert d.mean() <= TOL_MEAN, f"{label}: mean|dO| {d.mean()}"
    assert dl.max() <= TOL_LSE, f"{label}: max|dLSE| {dl.max()}"


def _rand(shape, seed, sigma=1.0):
    g = np.random.Generator(np.random.PCG64(seed))
    return (g.standard_normal(shape, dtype=np.float32) * np.float32(sigma))


def _gen(seed):
    """A seeded device generator, so every random draw in these tests is the same on every run."""
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    return g


def _bf(x):
    return torch.from_numpy(x).to(torch.bfloat16).float().numpy()


# ------------------------------------------------------------------ fixtures


GOLDEN_FILES = sorted(f for f in os.listdir(GOLDEN) if f.endswith(".npz"))


@pytest.mark.parametrize("fname", GOLDEN_FILES)
def test_golden_fixtures(fname):
    z = np.load(os.path.join(GOLDEN, fname))
    q, k, v = (bf16_bits_to_f32(z[n]) for n in ("q_bits", "k_bits", "v_bits"))
    _say(f"golden {fname} shape={q.shape}")
    o, lse = _run(q, k, v, float(z["scale"]), bool(z["causal"]))
    _check(o, lse, z["o"], z["lse"], fname)


# ------------------------------------------------------------------ BASELINE configs


def _config_inputs(name):
    cfg = CONFIGS[name]
    q, k, v = make_inputs(cfg)
    with open(os.path.join(GOLDEN, "inputs_sha256.json")) as f:
        want = json.load(f)[name]
    assert (sha256_bf16(q), sha256_bf16(k), sha256_bf16(v)) == (want["q"], want["k"], want["v"])
    return cfg, q, k, v


@pytest.mark.parametrize("name", ["config1", "config2"])
def test_config_full(name):
    cfg, q, k, v = _config_inputs(name)
    _say(f"{name} B={cfg.B} H={cfg.H} N={cfg.N}")
    o, lse = _run(q, k, v, cfg.scale, True)
    o_ref, lse_ref = attention_c(q, k, v, cfg.scale, True)
    _check(o, lse, o_ref, lse_ref, name)


@pytest.mark.parametrize("name,nsample", [("config3", 96), ("config4", 40)])
def test_config_sampled_rows(name, nsample):
    cfg, q, k, v = _config_inputs(name)
    _say(f"{name} B={cfg.B} H={cfg.H} N={cfg.N} (sampled rows)")
    o, lse = _run(q, k, v, cfg.scale, True)
    g = np.random.Generator(np.random.PCG64(7))
    edges = [0, 1, 31, 32, 63, 64, 127, 128, 129, cfg.N // 2, cfg.N - 2, cfg.N - 1]
    rows = np.unique(np.concatenate([edges, g.integers(0, cfg.N, nsample - len(edges))]))
    o_ref, lse_ref = attention_c(q, k, v, cfg.scale, True, rows=rows)
    _check(o[:, :, rows], lse[:, :, rows], o_ref, lse_ref, name)
    # Whole-tensor properties at full size.
    assert np.isfinite(o).all() and np.isfinite(lse).all()
    np.testing.assert_array_equal(o[:, :, 0], v[:, :, 0])  # row 0 attends only to key 0
    assert np.all(np.abs(o) <= np.abs(v).max() + 1e-2)    # convex combination of V rows


@pytest.mark.parametrize("dtype,N,D", [(torch.bfloat16, 65536, 64), (torch.float16, 32768, 128)])
def test_long_sequences_sampled_rows(dtype, N, D):
    """Sequences far past the configs (32-bit offset arithmetic, 512-1024 key tiles per
    workgroup): sampled rows against the oracle, whole-tensor properties at full size."""
    B, H = 1, 2
    rnd = (lambda x: _bf(x)) if dtype == torch.bfloat16 else (lambda x: x.astype(np.float16).astype(np.float32))
    q, k, v = (rnd(_rand((B, H, N, D), 5000 + N + D + i, 2.0 if i < 2 else 1.0)) for i in range(3))
    _say(f"long sequence {dtype} N={N} D={D}")
    qd, kd, vd = (torch.from_numpy(x).to(dtype).to(DEV) for x in (q, k, v))
    o, lse = custom_flash_attn.attention(qd, kd, vd, return_lse=True)
    torch.cuda.synchronize()
    o, lse = o.float().cpu().numpy(), lse.cpu().numpy()
    g = np.random.Generator(np.random.PCG64(N))
    edges = [0, 1, 127, 128, N // 2 - 1, N // 2, N - 129, N - 128, N - 2, N - 1]
    rows = np.unique(np.concatenate([edges, g.integers(0, N, 22)]))
    o_ref, lse_ref = attention_c(q, k, v, 1.0 / math.sqrt(D), True, rows=rows)
    _check(o[:, :, rows], lse[:, :, rows], o_ref, lse_ref, f"N={N} D={D}")
    assert np.isfinite(o).all() and np.isfinite(lse).all()
    np.testing.assert_array_equal(o[:, :, 0], v[:, :, 0])  # row 0 attends only to key 0
    assert np.all(np.abs(o) <= np.abs(v).max() + 1e-2)


@pytest.mark.parametrize("name", ["config2", "config3", "config4"])
def test_config_full_tensor_vs_reference_cpu_path(name):
    """Every output element of configs 2-4 against the reference's own CPU attention path
    (the fp32 "manual" branch, src/py/model_inference.py:68-75), one (batch, head) at a time."""
    import torch as _t

    from oracle import manual_attention_torch

    cfg, q, k, v = _config_inputs(name)
    _say(f"{name} full tensor vs CPU fp32 manual path")
    o, lse = _run(q, k, v, cfg.scale, True)
    _t.set_num_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    worst, total, count = 0.0, 0.0, 0
    for b in range(cfg.B):
        for hh in range(cfg.H):
            ref = manual_attention_torch(_t.from_numpy(q[b:b + 1, hh:hh + 1]), _t.from_numpy(k[b:b + 1, hh:hh + 1]),
                                         _t.from_numpy(v[b:b + 1, hh:hh + 1]))[0, 0].numpy()
            d = np.abs(o[b, hh].astype(np.float64) - ref)
            worst = max(worst, float(d.max()))
            total += float(d.sum())
            count += d.size
    _say(f"{name} full: max|dO|={worst:.3e} mean|dO|={total / count:.3e}")
    assert worst <= TOL_MAX and total / count <= TOL_MEAN


@pytest.mark.parametrize("name", ["config2", "config3", "config4"])
def test_config_every_row_vs_fp64_oracle(name):
    """O and LSE of every row of configs 2-4 against the fp64 C oracle (attention_ref.c, the
    "manual" branch of src/py/model_inference.py:68-75 and the lse_i of
    src/py/triton_implementation.py:153-154), no sampling."""
    cfg, q, k, v = _config_inputs(name)
    _say(f"{name} every row vs fp64 oracle (O and LSE)")
    o, lse = _run(q, k, v, cfg.scale, True)
    o_ref, lse_ref = attention_c(q, k, v, cfg.scale, True)
    _check(o, lse, o_ref, lse_ref, f"{name} every row")


@pytest.mark.parametrize("B,H,N,nheads", [
    (32, 128, 256, 48),   # 4096 heads, 8192 workgroups: many dispatch rounds
    (3, 37, 1000, 24),    # 111 heads, not a multiple of the 8 XCDs; ragged last block
    (5, 13, 129, 0),      # 65 heads, a one-row last block (split-key kernel)
    (1, 3, 777, 0),       # 3 heads (split-key kernel), ragged
])
def test_grid_shapes_many_and_odd_head_counts(B, H, N, nheads):
    """Grids the configs do not cover: thousands of heads, head counts that do not divide
    over the XCDs (a head's blocks then land on different XCDs), one-row and ragged last
    blocks.  O and LSE of every row of nheads sampled heads (0: all heads) against the fp64
    oracle."""
    q, k, v = (_bf(_rand((B, H, N, 64), 7000 + B * H + N + i, 2.0 if i < 2 else 1.0)) for i in range(3))
    _say(f"grid B={B} H={H} N={N}")
    o, lse = _run(q, k, v)
    if nheads:
        g = np.random.Generator(np.random.PCG64(B * H + N))
        idx = np.unique(np.concatenate([[0, B * H - 1], g.choice(B * H, nheads, replace=False)]))
    else:
        idx = np.arange(B * H)
    pick = lambda x: np.ascontiguousarray(x.reshape(B * H, N, -1)[idx][None])
    o_ref, lse_ref = attention_c(pick(q), pick(k), pick(v), 0.125, True)
    _check(pick(o), lse.reshape(B * H, N)[idx][None], o_ref, lse_ref, f"B={B} H={H} N={N}")


# ------------------------------------------------------------------ reference test shapes


@pytest.mark.parametrize("T", [1, 2, 10, 11, 15, 33, 63, 64, 65, 127, 128, 129, 255, 257, 1000, 1024])
def test_boundary_lengths(T):
    """The reference's boundary lengths (test_cuda_implementation.py:93) and tile edges."""
    q, k, v = (_bf(_rand((2, 4, T, 64), 1000 + 3 * T + i)) for i in range(3))
    _say(f"boundary T={T}")
    o, lse = _run(q, k, v)
    o_ref, lse_ref = attention_c(q, k, v, 0.125, True)
    _check(o, lse, o_ref, lse_ref, f"T={T}")


@pytest.mark.parametrize("T", [1, 33, 64, 100, 128, 300, 1024])
def test_non_causal(T):
    q, k, v = (_bf(_rand((1, 3, T, 64), 2000 + T + i)) for i in range(3))
    _say(f"non-causal T={T}")
    o, lse = _run(q, k, v, 0.125, False)
    o_ref, lse_ref = attention_c(q, k, v, 0.125, False)
    _check(o, lse, o_ref, lse_ref, f"noncausal T={T}")


@pytest.mark.parametrize("scale", [0.05, 0.3, 1.0])
def test_explicit_scale(scale):
    q, k, v = (_bf(_rand((1, 2, 200, 64), 3000 + i)) for i in range(3))
    o, lse = _run(q, k, v, scale, True)
    o_ref, lse_ref = attention_c(q, k, v, scale, True)
    _check(o, lse, o_ref, lse_ref, f"scale={scale}")


def test_matches_reference_test_vs_sdpa_fp32():
    """test_flash_attention_vs_pytorch (test_cuda_implementation.py:72-91), against SDPA in fp32."""
    g = _gen(0)
    q, k, v = (torch.randn(2, 4, 128, 64, device=DEV, dtype=torch.bfloat16, generator=g) for _ in range(3))
    out = custom_flash_attn.forward(q, k, v)
    ref = torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float(), is_causal=True)
    torch.testing.assert_close(out.float(), ref, rtol=1e-2, atol=1e-2)
    assert out.shape == q.shape and out.dtype == torch.bfloat16 and out.device == q.device


# ------------------------------------------------------------------ invariants / sanitizing


def test_outputs_fully_written_and_guards_untouched():
    """NaN-poisoned outputs inside guard canaries: every element written, nothing outside."""
    B, H, N = 2, 3, 300
    g = _gen(11)
    q, k, v = (torch.randn(B, H, N, 64, device=DEV, dtype=torch.bfloat16, generator=g) for _ in range(3))
    guard = 4096
    o_buf = torch.full((guard + B * H * N * 64 + guard,), float("nan"), device=DEV, dtype=torch.bfloat16)
    l_buf = torch.full((guard + B * H * N + guard,), float("nan"), device=DEV, dtype=torch.float32)
    o_buf[:guard] = 7.0
    o_buf[-guard:] = 7.0
    l_buf[:guard] = 7.0
    l_buf[-guard:] = 7.0
    o = o_buf[guard:-guard]
    lse = l_buf[guard:-guard]
    _C.fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(), B, H, N, 64,
           0.125, True, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all() and torch.isfinite(lse).all()
    assert (o_buf[:guard] == 7.0).all() and (o_buf[-guard:] == 7.0).all()
    assert (l_buf[:guard] == 7.0).all() and (l_buf[-guard:] == 7.0).all()


def test_deterministic_bitwise():
    g = _gen(12)
    q, k, v = (torch.randn(4, 8, 777, 64, device=DEV, dtype=torch.bfloat16, generator=g) for _ in range(3))
    o1, l1 = custom_flash_attn.forward_lse(q, k, v)
    o2, l2 = custom_flash_attn.forward_lse(q, k, v)
    assert torch.equal(o1, o2) and torch.equal(l1, l2)


def test_causality_bitwise():
    g = _gen(13)
    q, k, v = (torch.randn(2, 4, 512, 64, device=DEV, dtype=torch.bfloat16, generator=g) for _ in range(3))
    o1 = custom_flash_attn.forward(q, k, v)
    i = 200
    k2, v2 = k.clone(), v.clone()
    tail = k2[:, :, i + 1:].shape
    k2[:, :, i + 1:] = torch.randn(tail, device=DEV, dtype=torch.bfloat16, generator=g)
    v2[:, :, i + 1:] = torch.randn(tail, device=DEV, dtype=torch.bfloat16, generator=g)
    o2 = custom_flash_attn.forward(q, k2, v2)
    assert torch.equal(o1[:, :, : i + 1], o2[:, :, : i + 1])
    assert not torch.equal(o1[:, :, i + 1:], o2[:, :, i + 1:])


def test_identical_keys_prefix_mean_and_constant_v():
    B, H, N = 1, 4, 300
    g = _gen(14)
    q = torch.randn(B, H, N, 64, device=DEV, dtype=torch.bfloat16, generator=g)
    k = torch.randn(B, H, 1, 64, device=DEV, dtype=torch.bfloat16, generator=g).expand(B, H, N, 64).contiguous()
    v = torch.randn(B, H, N, 64, device=DEV, dtype=torch.bfloat16, generator=g)
    o, lse = custom_flash_attn.forward_lse(q, k, v)
    mean = torch.cumsum(v.double(), dim=2) / torch.arange(1, N + 1, device=DEV, dtype=torch.float64)[None, None, :, None]
    assert (o.double() - mean).abs().max().item() <= TOL_MAX
    s = 0.125 * (q.double() * k.double()).sum(-1)
    ln = torch.log(torch.arange(1, N + 1, device=DEV, dtype=torch.float64))
    assert (lse.double() - (s + ln)).abs().max().item() <= TOL_LSE
    ones = torch.ones_like(v)
    k3 = torch.randn(q.shape, device=DEV, dtype=torch.bfloat16, generator=g)
    o1 = custom_flash_attn.forward(q * 3, k3 * 3, ones)
    assert (o1.float() - 1).abs().max().item() <= 1e-2


def test_empty_inputs():
    for shape in [(0, 2, 16, 64), (2, 0, 16, 64), (2, 2, 0, 64)]:
        q = torch.empty(shape, device=DEV, dtype=torch.bfloat16)
        o = custom_flash_attn.forward(q, q, q)
        assert o.shape == q.shape


def test_error_paths_on_device():
    g = _gen(15)
    q = torch.randn(1, 2, 16, 64, device=DEV, dtype=torch.bfloat16, generator=g)
    with pytest.raises(RuntimeError, match="^K_mat must be contiguous$"):
        custom_flash_attn.forward(q, q.transpose(2, 3).contiguous().transpose(2, 3), q)
    with pytest.raises(RuntimeError, match="Use bfloat16"):
        custom_flash_attn.forward(q.half(), q.half(), q.half())
    with pytest.raises(RuntimeError, match="head_dim must be 64"):
        x = torch.randn(1, 2, 16, 128, device=DEV, dtype=torch.bfloat16, generator=g)
        custom_flash_attn.forward(x, x, x)


def test_runs_on_side_stream():
    g = _gen(16)
    q, k, v = (torch.randn(2, 4, 300, 64, device=DEV, dtype=torch.bfloat16, generator=g) for _ in range(3))
    ref = custom_flash_attn.forward(q, k, v)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        out = custom_flash_attn.forward(q, k, v)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_device_info():
    info = custom_flash_attn.device_info()
    _say(f"device_info: {info}")
    assert info["cu_count"] > 0 and info["sclk_mhz"] > 0 and info["arch"].startswith("gfx")
