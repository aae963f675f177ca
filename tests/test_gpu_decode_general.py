"""Decode step widened to fp16 and head dims up to 128 (tfgfa_decode) against the CPU oracle
(GPU box only).

``decode_np`` (fp64, the last row of the causal forward over the first L cached tokens,
pinned in tests/test_oracle.py) is the checker, on inputs already rounded to the element type.
Tolerances as for the forward: max|dO| <= 2e-2, mean|dO| <= 2e-3, max|dLSE| <= 1e-3, with
Q, K ~ N(0, 3^2) and V ~ N(0, 1).

Covered per element type (bf16, fp16) and head dim (8, 40, 64, 96, 128): ragged lengths,
the fused append (cache row written, nothing else touched), the split-sequence path against
the one-workgroup path, strided caches (bitwise equal to contiguous ones), NaN rows for
invalid lengths, NaN / inf in cache rows past the length (no effect); and bf16 / D = 64
bitwise equal to the bf16 entry point.  At D = 96 and 128, both sides of the split threshold
(B*H at half the CUs splits, one head more does not).  The dense instances (contiguous operands
at D = 64 and 128, no strides read) bitwise equal to the strided ones, split and unsplit, with
and without the append.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import bf16_round, decode_np

import custom_flash_attn
from custom_flash_attn import _C

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TOL_MAX, TOL_MEAN, TOL_LSE = 2e-2, 2e-3, 1e-3
DTYPES = {"bf16": torch.bfloat16, "f16": torch.float16}
HEAD_DIMS = [8, 40, 64, 96, 128]


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _round(x, dt):
    return bf16_round(x) if dt == "bf16" else x.astype(np.float16).astype(np.float32)


def _rand(shape, seed, dt, sigma=1.0):
    g = np.random.Generator(np.random.PCG64(seed))
    return _round(g.standard_normal(shape, dtype=np.float32) * np.float32(sigma), dt)


def _dev(x, dt):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DTYPES[dt]).to(DEV)


def _check(o, lse, o_ref, lse_ref, label):
    o = o.float().cpu().numpy().astype(np.float64)
    lse = lse.cpu().numpy().astype(np.float64)
    d = np.abs(o - o_ref)
    fin = np.isfinite(lse_ref)
    dl = np.abs(lse[fin] - lse_ref[fin])
    _say(f"{label}: max|dO|={d.max():.3e} mean|dO|={d.mean():.3e} "
         f"max|dLSE|={dl.max() if dl.size else 0:.3e}")
    assert np.isfinite(o).all(), f"{label}: non-finite O"
    assert np.array_equal(np.isneginf(lse), ~fin), f"{label}: -inf LSE pattern differs"
    assert d.max() <= TOL_MAX and d.mean() <= TOL_MEAN, label
    assert dl.size == 0 or dl.max() <= TOL_LSE, label


def _case(B, H, N_max, D, seed, dt):
    kc = _rand((B, H, N_max, D), seed, dt, 3.0)
    vc = _rand((B, H, N_max, D), seed + 1, dt)
    q = _rand((B, H, D), seed + 2, dt, 3.0)
    return q, kc, vc


@pytest.mark.parametrize("D", HEAD_DIMS)
@pytest.mark.parametrize("dt", list(DTYPES))
def test_ragged_lengths_match_oracle(dt, D):
    B, H, N_max, lens = 3, 5, 700, [1, 345, 700]
    _say(f"decode {dt} D={D} B={B} H={H} N_max={N_max} lens={lens}")
    q, kc, vc = _case(B, H, N_max, D, 10 + D, dt)
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    o, lse = custom_flash_attn.decode(_dev(q, dt), _dev(kc, dt), _dev(vc, dt), sl, return_lse=True)
    torch.cuda.synchronize()
    assert o.dtype == DTYPES[dt] and o.shape == (B, H, D)
    o_ref, l_ref = decode_np(q, kc, vc, lens, D ** -0.5)
    _check(o, lse, o_ref, l_ref, f"{dt} D={D} ragged")


@pytest.mark.parametrize("D", HEAD_DIMS)
@pytest.mark.parametrize("dt", list(DTYPES))
def test_append_writes_row_and_attends_it(dt, D):
    B, H, N_max, lens = 2, 3, 300, [0, 299]
    _say(f"decode append {dt} D={D} lens={lens}")
    q, kc, vc = _case(B, H, N_max, D, 40 + D, dt)
    kn, vn = _rand((B, H, D), 50 + D, dt, 3.0), _rand((B, H, D), 60 + D, dt)
    kd, vd = _dev(kc, dt), _dev(vc, dt)
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    o, lse = custom_flash_attn.decode(_dev(q, dt), kd, vd, sl, _dev(kn, dt), _dev(vn, dt), return_lse=True)
    torch.cuda.synchronize()
    kw, vw = kc.copy(), vc.copy()
    for b, L in enumerate(lens):
        kw[b, :, L], vw[b, :, L] = kn[b], vn[b]
    assert np.array_equal(kd.float().cpu().numpy(), kw), "k cache: wrong row written or other rows touched"
    assert np.array_equal(vd.float().cpu().numpy(), vw), "v cache: wrong row written or other rows touched"
    o_ref, l_ref = decode_np(q, kw, vw, [L + 1 for L in lens], D ** -0.5)
    _check(o, lse, o_ref, l_ref, f"{dt} D={D} append")


@pytest.mark.parametrize("D", [40, 128])
@pytest.mark.parametrize("dt", list(DTYPES))
def test_split_and_single_workgroup_paths_agree(dt, D):
    """B*H = 4 splits each head; an empty workspace forces one workgroup per head."""
    B, H, N_max, L = 1, 4, 8192, 8000
    _say(f"decode split {dt} D={D} L={L}")
    q, kc, vc = _case(B, H, N_max, D, 70 + D, dt)
    qd, kd, vd = _dev(q, dt), _dev(kc, dt), _dev(vc, dt)
    sl = torch.tensor([L], dtype=torch.int32, device=DEV)
    ws = torch.empty(_C.decode_workspace_size(B, H, N_max, D), dtype=torch.uint8, device=DEV)
    split = custom_flash_attn.decode(qd, kd, vd, sl, return_lse=True, workspace=ws)
    single = custom_flash_attn.decode(qd, kd, vd, sl, return_lse=True,
                                      workspace=torch.empty(0, dtype=torch.uint8, device=DEV))
    torch.cuda.synchronize()
    o_ref, l_ref = decode_np(q, kc, vc, [L], D ** -0.5)
    _check(split[0], split[1], o_ref, l_ref, f"{dt} D={D} split")
    _check(single[0], single[1], o_ref, l_ref, f"{dt} D={D} single workgroup")


@pytest.mark.parametrize("D", [96, 128])
def test_split_threshold_at_half_the_cus(D):
    """Heads are split while B*H is at most half the CUs, and run one workgroup each above.
    The split path leaves its arrival words (64-bit, 128 bytes apart at the workspace start)
    at zero; the unsplit path never touches the workspace.  Both sides of the threshold
    against the oracle (fp16, ragged lengths)."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    N_max = 1024
    for B, H, splits in ((2, cus // 4, True), (1, cus // 2 + 1, False)):
        lens = [N_max - 1 - 37 * b for b in range(B)]
        _say(f"decode threshold D={D} B={B} H={H} lens={lens} split={splits}")
        q, kc, vc = _case(B, H, N_max, D, 300 + D + H, "f16")
        sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
        ws = torch.full((_C.decode_workspace_size(B, H, N_max, D),), 0x5A, dtype=torch.uint8,
                        device=DEV)
        o, lse = custom_flash_attn.decode(_dev(q, "f16"), _dev(kc, "f16"), _dev(vc, "f16"), sl,
                                          return_lse=True, workspace=ws)
        torch.cuda.synchronize()
        words = ws[: B * H * 128].view(torch.int64)[::16]
        expect = 0 if splits else int.from_bytes(b"\x5a" * 8, "little")
        assert torch.equal(words, torch.full_like(words, expect)), (B, H, words[:4])
        o_ref, l_ref = decode_np(q, kc, vc, lens, D ** -0.5)
        _check(o, lse, o_ref, l_ref, f"f16 D={D} B*H={B * H}")


@pytest.mark.parametrize("D", [40, 96])
@pytest.mark.parametrize("dt", list(DTYPES))
def test_strided_cache_is_bitwise_equal(dt, D):
    """(B, N_max, H, D) buffers viewed as (B, H, N_max, D): the GPT-2 projection layout."""
    B, H, N_max, lens = 2, 3, 400, [400, 77]
    _say(f"decode strided {dt} D={D}")
    q, kc, vc = _case(B, H, N_max, D, 90 + D, dt)
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    ref = custom_flash_attn.decode(_dev(q, dt), _dev(kc, dt), _dev(vc, dt), sl, return_lse=True)
    ks = _dev(kc, dt).transpose(1, 2).contiguous().transpose(1, 2)
    vs = _dev(vc, dt).transpose(1, 2).contiguous().transpose(1, 2)
    qbuf = torch.zeros(H, B, D + 8, dtype=DTYPES[dt], device=DEV)
    qv = qbuf[..., :D].transpose(0, 1)
    qv.copy_(_dev(q, dt))
    got = custom_flash_attn.decode(qv, ks, vs, sl, return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(got[0].view(torch.int16), ref[0].view(torch.int16))
    assert torch.equal(got[1], ref[1])


@pytest.mark.parametrize("append", [False, True])
@pytest.mark.parametrize("B,H,N_max,lens", [(1, 4, 4096, [3000]), (8, 25, 256, [255, 7, 128, 0, 200, 31, 254, 100])])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dt", list(DTYPES))
def test_dense_instances_equal_strided_ones(dt, D, B, H, N_max, lens, append):
    """Every operand contiguous at D = 64 or 128 (the KVCache layout) takes the dense instances,
    which compute offsets from the head index and read no strides; the same values in
    (B, N_max, H, D) caches, with q, k_new, v_new and o as views of wider rows, take the strided
    ones.  Results, and the appended cache row, must be bitwise equal: split heads (B*H = 4) and
    one workgroup per head (B*H = 200)."""
    _say(f"decode dense vs strided {dt} D={D} B={B} H={H} N_max={N_max} append={append}")
    q, kc, vc = _case(B, H, N_max, D, 300 + D + B, dt)
    kn, vn = _rand((B, H, D), 310 + D, dt, 3.0), _rand((B, H, D), 320 + D, dt)
    lens = lens if not append else [min(L, N_max - 1) for L in lens]
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    kd, vd = _dev(kc, dt), _dev(vc, dt)
    new = (_dev(kn, dt), _dev(vn, dt)) if append else (None, None)
    ref = custom_flash_attn.decode(_dev(q, dt), kd, vd, sl, *new, return_lse=True)
    ks = _dev(kc, dt).transpose(1, 2).contiguous().transpose(1, 2)
    vs = _dev(vc, dt).transpose(1, 2).contiguous().transpose(1, 2)

    def wide(x):  # (B, H, D) values as a view of (B, H, D + 8) rows
        buf = torch.zeros(B, H, D + 8, dtype=DTYPES[dt], device=DEV)
        buf[..., :D].copy_(x)
        return buf[..., :D]

    qv = wide(_dev(q, dt))
    newv = (wide(new[0]), wide(new[1])) if append else (None, None)
    ov = wide(torch.zeros(B, H, D, dtype=DTYPES[dt], device=DEV))
    got = custom_flash_attn.decode(qv, ks, vs, sl, *newv, out=ov, return_lse=True)
    torch.cuda.synchronize()
    assert not qv.is_contiguous() and not ks.is_contiguous()
    assert torch.equal(got[0].view(torch.int16), ref[0].view(torch.int16)), "O differs"
    assert torch.equal(got[1], ref[1]), "LSE differs"
    assert torch.equal(ks.view(torch.int16), kd.view(torch.int16)), "k caches differ"
    assert torch.equal(vs.view(torch.int16), vd.view(torch.int16)), "v caches differ"


@pytest.mark.parametrize("D", [8, 128])
@pytest.mark.parametrize("dt", list(DTYPES))
def test_invalid_lengths_give_nan_rows_only(dt, D):
    B, H, N_max = 3, 2, 64
    _say(f"decode invalid lengths {dt} D={D}")
    q, kc, vc = _case(B, H, N_max, D, 110 + D, dt)
    kd = _dev(kc, dt)
    k_before = kd.clone()
    sl = torch.tensor([-1, 30, 64], dtype=torch.int32, device=DEV)  # row 2: 64 + append > N_max
    kn, vn = _dev(_rand((B, H, D), 120, dt), dt), _dev(_rand((B, H, D), 121, dt), dt)
    o, lse = custom_flash_attn.decode(_dev(q, dt), kd, _dev(vc, dt), sl, kn, vn, return_lse=True)
    torch.cuda.synchronize()
    assert torch.isnan(o[0]).all() and torch.isnan(lse[0]).all()
    assert torch.isnan(o[2]).all() and torch.isnan(lse[2]).all()
    assert torch.isfinite(o[1]).all() and torch.isfinite(lse[1]).all()
    assert torch.equal(kd[0], k_before[0]) and torch.equal(kd[2], k_before[2]), "invalid rows appended"
    assert torch.equal(kd[1, :, 30], kn[1]), "valid row not appended"


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dt", list(DTYPES))
@pytest.mark.parametrize("append", [False, True])
def test_rows_past_the_length_never_reach_the_result(dt, D, append):
    """Cache rows at or past cache_seqlens (the first block of a chunk is loaded before the
    length is known) hold NaN / inf: the result is bitwise that of a cache holding zeros there."""
    B, H, N_max, lens = 4, 3, 600, [5, 33, 300, 0]
    _say(f"decode garbage past length {dt} D={D} append={append}")
    q, kc, vc = _case(B, H, N_max, D, 140 + D, dt)
    for b, L in enumerate(lens):
        kc[b, :, L:] = 0.0
        vc[b, :, L:] = 0.0
    kz, vz = _dev(kc, dt), _dev(vc, dt)
    kg, vg = kz.clone(), vz.clone()
    for b, L in enumerate(lens):
        kg[b, :, L:] = float("nan")
        vg[b, :, L:] = float("inf")
        vg[b, :, L + 1::2] = float("nan")
    qd = _dev(q, dt)
    kn = _dev(_rand((B, H, D), 150, dt, 3.0), dt) if append else None
    vn = _dev(_rand((B, H, D), 151, dt), dt) if append else None
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    ref = custom_flash_attn.decode(qd, kz, vz, sl, kn, vn, return_lse=True)
    got = custom_flash_attn.decode(qd, kg, vg, sl, kn, vn, return_lse=True)
    torch.cuda.synchronize()
    assert torch.isfinite(got[0][:3]).all()
    assert torch.equal(got[0].view(torch.int16), ref[0].view(torch.int16))
    assert torch.equal(got[1], ref[1])


def test_bf16_d64_is_bitwise_the_bf16_entry():
    B, H, N_max, lens = 4, 6, 1500, [1500, 1, 700, 1024]
    _say("decode general vs bf16 entry")
    q, kc, vc = _case(B, H, N_max, 64, 130, "bf16")
    qd, kd, vd = _dev(q, "bf16"), _dev(kc, "bf16"), _dev(vc, "bf16")
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    o_gen, l_gen = custom_flash_attn.decode(qd, kd, vd, sl, return_lse=True)
    o_old = torch.empty_like(o_gen)
    l_old = torch.empty_like(l_gen)
    ws = torch.empty(_C.decode_workspace_bytes(B, H, N_max), dtype=torch.uint8, device=DEV)
    z3 = (0, 0, 0)
    _C.decode(qd.data_ptr(), qd.stride(), kd.data_ptr(), kd.stride(), vd.data_ptr(), vd.stride(),
              0, z3, 0, z3, sl.data_ptr(), o_old.data_ptr(), o_old.stride(), l_old.data_ptr(),
              B, H, N_max, 64, 0.125, ws.data_ptr(), ws.numel(),
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(o_gen.view(torch.int16), o_old.view(torch.int16))
    assert torch.equal(l_gen, l_old)


def test_mixed_dtypes_and_bad_head_dims_raise():
    q = torch.zeros(1, 2, 64, dtype=torch.float16, device=DEV)
    kc = torch.zeros(1, 2, 16, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="q must have dtype"):
        custom_flash_attn.decode(q, kc, kc)
    with pytest.raises(RuntimeError, match="v_cache must have dtype"):
        custom_flash_attn.decode(q, kc.half(), kc)
    with pytest.raises(RuntimeError, match=r"multiple of 8 in \[8, 128\]"):
        k36 = torch.zeros(1, 2, 16, 36, dtype=torch.float16, device=DEV)
        custom_flash_attn.decode(q[..., :36], k36, k36)
    with pytest.raises(RuntimeError, match="Use bfloat16 or float16"):
        k32 = torch.zeros(1, 2, 16, 64, dtype=torch.float32, device=DEV)
        custom_flash_attn.decode(q.float(), k32, k32)
