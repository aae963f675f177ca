"""Pins the CPU oracle (oracle/) before it is trusted as the checker of the HIP kernel.

Each check is chosen so that a plausible mistake in the oracle fails at least one of
them (see test_planted_mistakes_are_caught): the diagonal dropped from the causal mask,
the scale left out or applied twice, Q and K swapped, the softmax taken over the wrong
axis, the max-subtraction inconsistent with the LSE.

Sources of truth:
  * torch.nn.functional.scaled_dot_product_attention in fp64 on the CPU - the library
    routine the reference's tests compare against (test/py/test_cuda_implementation.py:49-52);
  * a pure-Python brute force on tiny inputs;
  * closed forms: row 0, identical keys, constant V, causality, permutation.
"""
import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import (
    CONFIGS, attention_c, attention_np, bf16_bits_to_f32, bf16_round, decode_np, f32_to_bf16_bits,
    make_inputs, manual_attention_torch, sha256_bf16,
)

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _rand(shape, seed, sigma=1.0):
    rng = np.random.Generator(np.random.PCG64(seed))
    return bf16_round(rng.standard_normal(shape, dtype=np.float32) * np.float32(sigma))


def _sdpa64(q, k, v, scale, causal):
    return torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(np.asarray(q, np.float64)), torch.from_numpy(np.asarray(k, np.float64)),
        torch.from_numpy(np.asarray(v, np.float64)), is_causal=causal, scale=scale,
    ).numpy()


def _lse_logsumexp64(q, k, scale, causal):
    s = torch.from_numpy(np.asarray(q, np.float64)) @ torch.from_numpy(np.asarray(k, np.float64)).transpose(-1, -2)
    s = s * scale
    if causal:
        n = s.shape[-1]
        s = s.masked_fill(torch.triu(torch.ones(n, n, dtype=torch.bool), 1), -math.inf)
    return torch.logsumexp(s, dim=-1).numpy()


def _brute(q, k, v, scale, causal):
    """Pure-Python triple loop, one (N, D) head."""
    n, d = len(q), len(q[0])
    o = [[0.0] * d for _ in range(n)]
    lse = [0.0] * n
    for i in range(n):
        js = range(i + 1) if causal else range(n)
        s = [scale * sum(q[i][t] * k[j][t] for t in range(d)) for j in js]
        z = sum(math.exp(x) for x in s)
        lse[i] = math.log(z)
        for jj, j in enumerate(js):
            w = math.exp(s[jj]) / z
            for t in range(d):
                o[i][t] += w * v[j][t]
    return o, lse


# ------------------------------------------------------------------ bf16 rounding


def test_bf16_rounding_matches_torch():
    rng = np.random.Generator(np.random.PCG64(5))
    x = np.concatenate([
        rng.standard_normal(100000, dtype=np.float32) * 7,
        np.array([0.0, -0.0, 1.0, -1.0, 1e-30, 3.0e38, 65504.0, 1.00390625, 1.01171875,
                  1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8], dtype=np.float32),  # ties both ways
    ])
    ours = f32_to_bf16_bits(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, ref)
    np.testing.assert_array_equal(bf16_bits_to_f32(ours), torch.from_numpy(x).to(torch.bfloat16).float().numpy())


# ------------------------------------------------------------------ library routine


@pytest.mark.parametrize("T", [1, 2, 10, 11, 15, 33, 63, 64, 65, 128, 200])
@pytest.mark.parametrize("causal", [True, False])
def test_oracle_matches_sdpa_fp64(T, causal):
    q, k, v = (_rand((2, 3, T, 64), 100 + T + i) for i in range(3))
    o, lse = attention_np(q, k, v, 0.125, causal)
    np.testing.assert_allclose(o, _sdpa64(q, k, v, 0.125, causal), rtol=0, atol=1e-12)
    np.testing.assert_allclose(lse, _lse_logsumexp64(q, k, 0.125, causal), rtol=0, atol=1e-12)
    oc, lc = attention_c(q, k, v, 0.125, causal)
    np.testing.assert_allclose(oc, o, rtol=0, atol=1e-12)
    np.testing.assert_allclose(lc, lse, rtol=0, atol=1e-12)


def test_oracle_custom_scale_and_wide_logits():
    q, k, v = _rand((1, 2, 97, 64), 1, 3.0), _rand((1, 2, 97, 64), 2, 3.0), _rand((1, 2, 97, 64), 3)
    for scale in (0.3, 0.125, 1.0):
        o, lse = attention_c(q, k, v, scale, True)
        np.testing.assert_allclose(o, _sdpa64(q, k, v, scale, True), rtol=0, atol=1e-11)
        np.testing.assert_allclose(lse, _lse_logsumexp64(q, k, scale, True), rtol=1e-13, atol=1e-11)


def test_oracle_row_subset_matches_full():
    q, k, v = (_rand((2, 2, 300, 64), 40 + i) for i in range(3))
    o, lse = attention_c(q, k, v)
    rows = np.array([0, 1, 63, 64, 127, 128, 299])
    os_, ls = attention_c(q, k, v, rows=rows)
    np.testing.assert_array_equal(os_, o[:, :, rows])
    np.testing.assert_array_equal(ls, lse[:, :, rows])
    with pytest.raises(ValueError):
        attention_c(q, k, v, rows=np.array([300]))


def test_manual_torch_path_matches_oracle():
    q, k, v = (_rand((2, 4, 128, 64), 60 + i) for i in range(3))
    out = manual_attention_torch(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v)).numpy()
    o, _ = attention_np(q, k, v)
    np.testing.assert_allclose(out, o, rtol=0, atol=2e-6)


# ------------------------------------------------------------------ brute force


@pytest.mark.parametrize("n,d,causal", [(1, 4, True), (5, 4, True), (7, 3, True), (6, 5, False)])
def test_oracle_matches_brute_force(n, d, causal):
    q, k, v = (_rand((1, 1, n, d), 7 * n + d + i) for i in range(3))
    scale = 0.7
    bo, bl = _brute(q[0, 0].tolist(), k[0, 0].tolist(), v[0, 0].tolist(), scale, causal)
    o, lse = attention_np(q, k, v, scale, causal)
    np.testing.assert_allclose(o[0, 0], np.array(bo), rtol=0, atol=1e-13)
    np.testing.assert_allclose(lse[0, 0], np.array(bl), rtol=0, atol=1e-13)
    oc, lc = attention_c(q, k, v, scale, causal)
    np.testing.assert_allclose(oc[0, 0], np.array(bo), rtol=0, atol=1e-13)
    np.testing.assert_allclose(lc[0, 0], np.array(bl), rtol=0, atol=1e-13)


# ------------------------------------------------------------------ closed forms


def test_row_zero_is_v_row_zero():
    q, k, v = (_rand((2, 3, 50, 64), 80 + i, 3.0) for i in range(3))
    o, lse = attention_c(q, k, v, 0.125, True)
    np.testing.assert_array_equal(o[:, :, 0], v[:, :, 0].astype(np.float64))
    s00 = 0.125 * np.einsum("bhd,bhd->bh", q[:, :, 0].astype(np.float64), k[:, :, 0].astype(np.float64))
    np.testing.assert_allclose(lse[:, :, 0], s00, rtol=0, atol=1e-12)


def test_identical_keys_give_prefix_mean():
    n = 40
    q = _rand((1, 2, n, 64), 90)
    k = np.broadcast_to(_rand((1, 2, 1, 64), 91), (1, 2, n, 64)).copy()
    v = _rand((1, 2, n, 64), 92)
    o, lse = attention_c(q, k, v, 0.125, True)
    prefix_mean = np.cumsum(v.astype(np.float64), axis=2) / np.arange(1, n + 1)[None, None, :, None]
    np.testing.assert_allclose(o, prefix_mean, rtol=0, atol=1e-12)
    s = 0.125 * np.einsum("bhnd,bhd->bhn", q.astype(np.float64), k[:, :, 0].astype(np.float64))
    np.testing.assert_allclose(lse, s + np.log(np.arange(1, n + 1)), rtol=0, atol=1e-12)


def test_constant_v_gives_constant_output():
    q, k = _rand((1, 2, 70, 64), 93, 3.0), _rand((1, 2, 70, 64), 94, 3.0)
    v = np.ones((1, 2, 70, 64), np.float32)
    o, _ = attention_c(q, k, v, 0.125, True)
    np.testing.assert_allclose(o, 1.0, rtol=0, atol=1e-13)


def test_causality_and_permutation():
    q, k, v = (_rand((2, 3, 64, 64), 95 + i) for i in range(3))
    o, lse = attention_c(q, k, v)
    i = 20
    k2, v2 = k.copy(), v.copy()
    k2[:, :, i + 1:] = _rand(k2[:, :, i + 1:].shape, 99)
    v2[:, :, i + 1:] = _rand(v2[:, :, i + 1:].shape, 98)
    o2, lse2 = attention_c(q, k2, v2)
    np.testing.assert_array_equal(o2[:, :, : i + 1], o[:, :, : i + 1])
    np.testing.assert_array_equal(lse2[:, :, : i + 1], lse[:, :, : i + 1])
    assert np.abs(o2[:, :, i + 1:] - o[:, :, i + 1:]).max() > 1e-3
    perm = np.array([2, 0, 1])
    o3, _ = attention_c(q[:, perm], k[:, perm], v[:, perm])
    np.testing.assert_array_equal(o3, o[:, perm])


# ------------------------------------------------------------------ planted mistakes


def _broken(kind):
    def f(q, k, v, scale, causal):
        q = np.asarray(q, np.float64)
        k = np.asarray(k, np.float64)
        v = np.asarray(v, np.float64)
        n = q.shape[-2]
        if kind == "swap_qk":
            q, k = k, q
        s = q @ np.swapaxes(k, -1, -2) * (1.0 if kind == "no_scale" else scale)
        if kind == "double_scale":
            s = s * scale
        if causal:
            diag = 0 if kind == "drop_diagonal" else 1
            s = np.where(np.triu(np.ones((n, n), bool), k=diag), -np.inf, s)
        ax = -2 if kind == "softmax_axis" else -1
        m = np.max(s, axis=ax, keepdims=True)
        p = np.exp(s - m)
        l = np.sum(p, axis=ax, keepdims=True)
        o = (p / l) @ v
        lse = np.log(l)[..., 0] if kind == "lse_without_max" else (m + np.log(l))[..., 0]
        if ax == -2:
            lse = np.zeros(o.shape[:-1])
        return o, lse
    return f


@pytest.mark.parametrize("kind", ["swap_qk", "no_scale", "double_scale", "drop_diagonal",
                                  "softmax_axis", "lse_without_max"])
def test_planted_mistakes_are_caught(kind):
    """A wrong oracle must fail the same comparisons the real one passes."""
    q, k, v = (_rand((1, 2, 33, 64), 120 + i, 2.0) for i in range(3))
    with np.errstate(all="ignore"):
        o, lse = _broken(kind)(q, k, v, 0.125, True)
    ref_o = _sdpa64(q, k, v, 0.125, True)
    ref_l = _lse_logsumexp64(q, k, 0.125, True)
    bad_o = not np.allclose(o, ref_o, rtol=0, atol=1e-6, equal_nan=False)
    bad_l = not np.allclose(lse, ref_l, rtol=0, atol=1e-6, equal_nan=False)
    assert bad_o or bad_l, f"planted mistake {kind!r} went unnoticed"


# ------------------------------------------------------------------ committed fixtures


GOLDEN_FILES = sorted(f for f in os.listdir(GOLDEN) if f.endswith(".npz"))


@pytest.mark.parametrize("fname", GOLDEN_FILES)
def test_golden_fixture_reproduces(fname):
    z = np.load(os.path.join(GOLDEN, fname))
    q, k, v = (bf16_bits_to_f32(z[n]) for n in ("q_bits", "k_bits", "v_bits"))
    o, lse = attention_c(q, k, v, float(z["scale"]), bool(z["causal"]))
    np.testing.assert_allclose(o, z["o"], rtol=0, atol=1e-12)
    np.testing.assert_allclose(lse, z["lse"], rtol=0, atol=1e-12)


def test_config_inputs_match_committed_hashes():
    with open(os.path.join(GOLDEN, "inputs_sha256.json")) as f:
        want = json.load(f)
    for name in ("config1", "config3"):  # config 2/4 hashes are checked by the GPU tests
        cfg = CONFIGS[name]
        q, k, v = make_inputs(cfg)
        assert [cfg.B, cfg.H, cfg.N, cfg.D] == want[name]["shape"]
        assert sha256_bf16(q) == want[name]["q"]
        assert sha256_bf16(k) == want[name]["k"]
        assert sha256_bf16(v) == want[name]["v"]
    # config 3 draws Q and K with sigma 3: their spread shows it.
    q, _, v = make_inputs(CONFIGS["config1"])
    assert 0.9 < q.std() < 1.1 and 0.9 < v.std() < 1.1


# ------------------------------------------------------------------ decode step


def test_decode_oracle_is_the_last_causal_row():
    """decode_np(q, cache, L) must equal row L-1 of the causal forward over the first L
    tokens, with q as that row's query (the value generate() keeps, model_inference.py:205)."""
    B, H, N_max, D = 3, 2, 90, 64
    kc, vc = _rand((B, H, N_max, D), 300, 3.0), _rand((B, H, N_max, D), 301)
    q = _rand((B, H, D), 302, 3.0)
    lens = [1, 57, 90]
    o, lse = decode_np(q, kc, vc, lens, 0.125)
    for b, L in enumerate(lens):
        qf = _rand((1, H, L, D), 303 + b, 3.0)
        qf[0, :, L - 1] = q[b]
        of, lf = attention_np(qf, kc[b:b + 1, :, :L], vc[b:b + 1, :, :L], 0.125, True)
        np.testing.assert_allclose(o[b], of[0, :, L - 1], rtol=0, atol=1e-12)
        np.testing.assert_allclose(lse[b], lf[0, :, L - 1], rtol=0, atol=1e-12)
        ref = torch.nn.functional.scaled_dot_product_attention(
            torch.from_numpy(q[b][:, None].astype(np.float64)),
            torch.from_numpy(kc[b, :, :L].astype(np.float64)),
            torch.from_numpy(vc[b, :, :L].astype(np.float64)), scale=0.125).numpy()[:, 0]
        np.testing.assert_allclose(o[b], ref, rtol=0, atol=1e-12)


def test_decode_oracle_empty_and_off_by_one():
    B, H, N_max, D = 2, 2, 40, 64
    kc, vc = _rand((B, H, N_max, D), 310, 2.0), _rand((B, H, N_max, D), 311)
    q = _rand((B, H, D), 312, 2.0)
    o, lse = decode_np(q, kc, vc, [0, 40])
    assert (o[0] == 0).all() and np.isneginf(lse[0]).all()
    # A length off by one either way must change the answer (the checks can see it).
    o_m, _ = decode_np(q, kc, vc, [0, 39])
    o_p, _ = decode_np(q, kc[:, :, :39], vc[:, :, :39], [0, 39])
    np.testing.assert_array_equal(o_m, o_p)
    assert np.abs(o_m[1] - o[1]).max() > 1e-3
    # One key: the output is that key's value row, lse = scale * q.k.
    o1, l1 = decode_np(q, kc, vc, [1, 1], 0.125)
    np.testing.assert_allclose(o1, vc[:, :, 0], rtol=0, atol=1e-15)
    np.testing.assert_allclose(l1, 0.125 * np.einsum("bhd,bhd->bh", q.astype(np.float64), kc[:, :, 0].astype(np.float64)), rtol=0, atol=1e-12)


# ------------------------------------------------------------------ general forward surface


@pytest.mark.parametrize("nq,nk", [(37, 61), (61, 37), (1, 20), (20, 1)])
@pytest.mark.parametrize("d", [8, 40, 128])
@pytest.mark.parametrize("causal", [True, False])
def test_oracle_nonsquare_and_head_dims_match_sdpa(nq, nk, d, causal):
    """N_q != N_k with the top-left causal mask of the Triton kernel
    (triton_implementation.py:127), which torch's SDPA also uses for is_causal with L != S."""
    q = _rand((2, 3, nq, d), 400 + nq + d, 2.0)
    k = _rand((2, 3, nk, d), 401 + nk + d, 2.0)
    v = _rand((2, 3, nk, d), 402 + nk + d)
    scale = 1.0 / math.sqrt(d)
    o, lse = attention_np(q, k, v, scale, causal)
    np.testing.assert_allclose(o, _sdpa64(q, k, v, scale, causal), rtol=0, atol=1e-12)
    s = np.einsum("bhid,bhjd->bhij", q.astype(np.float64), k.astype(np.float64)) * scale
    if causal:
        s = np.where(np.arange(nk)[None, :] > np.arange(nq)[:, None], -np.inf, s)
    np.testing.assert_allclose(lse, np.log(np.exp(s).sum(-1)), rtol=0, atol=1e-10)
