"""The C ABI called directly through ctypes, as a non-Python FFI would bind it (GPU box only).

Each compute entry point of include/tfgfa.h is called with the argument lists a reference-side
ctypes binding would use (argtypes from the header's prototypes), on raw device pointers from
torch tensors.  Results are checked
against the fp64 oracle (``attention_np``, ``decode_np``, pinned in tests/test_oracle.py) to
the forward's tolerances (max|dO| <= 2e-2, mean|dO| <= 2e-3, max|dLSE| <= 1e-3) and bitwise
against the Python package, which reaches the same library through pybind11.
"""
import ctypes
import sys

import numpy as np
import pytest
import torch

from oracle import attention_np, decode_np

import custom_flash_attn

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TOL_MAX, TOL_MEAN, TOL_LSE = 2e-2, 2e-3, 1e-3
S3, S4 = ctypes.c_int64 * 3, ctypes.c_int64 * 4
P = ctypes.c_void_p


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def lib():
    L = ctypes.CDLL(custom_flash_attn.library_path())
    L.tfgfa_fwd_bf16.restype = ctypes.c_int
    L.tfgfa_fwd_bf16.argtypes = [P] * 5 + [ctypes.c_int] * 4 + [ctypes.c_float, ctypes.c_int, P]
    L.tfgfa_fwd_bf16_strided.restype = ctypes.c_int
    L.tfgfa_fwd_bf16_strided.argtypes = [P, ctypes.POINTER(ctypes.c_int64)] * 4 + [P] + [
        ctypes.c_int] * 4 + [ctypes.c_float, ctypes.c_int, P]
    L.tfgfa_fwd.restype = ctypes.c_int
    L.tfgfa_fwd.argtypes = [P, P] * 4 + [P] + [ctypes.c_int] * 6 + [ctypes.c_float, ctypes.c_int, P]
    L.tfgfa_decode_bf16.restype = ctypes.c_int
    L.tfgfa_decode_bf16.argtypes = [P, P] * 5 + [P] * 4 + [ctypes.c_int] * 4 + [
        ctypes.c_float, P, ctypes.c_size_t, P]
    L.tfgfa_decode.restype = ctypes.c_int
    L.tfgfa_decode.argtypes = [P, P] * 5 + [P] * 4 + [ctypes.c_int] * 5 + [
        ctypes.c_float, P, ctypes.c_size_t, P]
    L.tfgfa_decode_workspace_size.restype = ctypes.c_size_t
    L.tfgfa_decode_workspace_size.argtypes = [ctypes.c_int] * 4
    L.tfgfa_strerror.restype = ctypes.c_char_p
    return L


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _ok(lib, st):
    assert st == 0, lib.tfgfa_strerror(st).decode()


def _rand(shape, seed, sigma=1.0, dtype=torch.bfloat16):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(shape, device=DEV, generator=g) * sigma).to(dtype)


def _np(t):
    return t.float().cpu().numpy().astype(np.float64)


def _check(o, lse, o_ref, lse_ref, label):
    d = np.abs(_np(o) - o_ref)
    dl = np.abs(lse.cpu().numpy().astype(np.float64) - lse_ref)
    _say(f"{label}: max|dO|={d.max():.3e} mean|dO|={d.mean():.3e} max|dLSE|={dl.max():.3e}")
    assert d.max() <= TOL_MAX and d.mean() <= TOL_MEAN and dl.max() <= TOL_LSE, label


def test_fwd_bf16_matches_oracle_and_package(lib):
    B, H, N, D = 2, 3, 300, 64
    q, k, v = _rand((B, H, N, D), 1, 3.0), _rand((B, H, N, D), 2, 3.0), _rand((B, H, N, D), 3)
    o = torch.empty_like(q)
    lse = torch.empty(B, H, N, device=DEV)
    _ok(lib, lib.tfgfa_fwd_bf16(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                                B, H, N, D, D ** -0.5, 1, _stream()))
    o_pkg, lse_pkg = custom_flash_attn.forward_lse(q, k, v)
    torch.cuda.synchronize()
    o_ref, lse_ref = attention_np(_np(q), _np(k), _np(v))
    _check(o, lse, o_ref, lse_ref, "tfgfa_fwd_bf16")
    assert torch.equal(o.view(torch.int16), o_pkg.view(torch.int16)) and torch.equal(lse, lse_pkg)


def test_fwd_bf16_strided_reads_gpt2_views(lib):
    B, N, H, D = 2, 200, 5, 64
    x = _rand((B, N, 3, H, D), 4, 2.0)
    qv, kv, vv = (x[:, :, i].transpose(1, 2) for i in range(3))  # (B, H, N, D) views
    ctx = torch.empty(B, N, H, D, dtype=torch.bfloat16, device=DEV)
    ov = ctx.transpose(1, 2)
    args = []
    for t in (qv, kv, vv, ov):
        args += [t.data_ptr(), S4(*t.stride())]
    _ok(lib, lib.tfgfa_fwd_bf16_strided(*args, None, B, H, N, D, D ** -0.5, 1, _stream()))
    torch.cuda.synchronize()
    o_ref, _ = attention_np(_np(qv), _np(kv), _np(vv))
    d = np.abs(_np(ov) - o_ref)
    _say(f"tfgfa_fwd_bf16_strided: max|dO|={d.max():.3e} mean|dO|={d.mean():.3e}")
    assert d.max() <= TOL_MAX and d.mean() <= TOL_MEAN
    ref = custom_flash_attn.forward(qv.contiguous(), kv.contiguous(), vv.contiguous())
    assert torch.equal(ov.contiguous().view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("dtype,dcode,D,Nq,Nk,causal", [
    (torch.float16, 1, 128, 150, 220, 1),
    (torch.bfloat16, 0, 40, 97, 97, 0),
])
def test_fwd_general(lib, dtype, dcode, D, Nq, Nk, causal):
    B, H = 2, 2
    q = _rand((B, H, Nq, D), 5, 2.0, dtype)
    k, v = _rand((B, H, Nk, D), 6, 2.0, dtype), _rand((B, H, Nk, D), 7, 1.0, dtype)
    o = torch.empty_like(q)
    lse = torch.empty(B, H, Nq, device=DEV)
    _ok(lib, lib.tfgfa_fwd(q.data_ptr(), None, k.data_ptr(), None, v.data_ptr(), None, o.data_ptr(), None,
                           lse.data_ptr(), B, H, Nq, Nk, D, dcode, 0.1, causal, _stream()))
    torch.cuda.synchronize()
    o_ref, lse_ref = attention_np(_np(q), _np(k), _np(v), 0.1, bool(causal))
    _check(o, lse, o_ref, lse_ref, f"tfgfa_fwd {dtype} D={D}")


def _decode_case(B, H, N_max, D, dtype, seed):
    kc = _rand((B, H, N_max, D), seed, 3.0, dtype)
    vc = _rand((B, H, N_max, D), seed + 1, 1.0, dtype)
    q = _rand((B, H, D), seed + 2, 3.0, dtype)
    kn, vn = _rand((B, H, D), seed + 3, 3.0, dtype), _rand((B, H, D), seed + 4, 1.0, dtype)
    return q, kc, vc, kn, vn


@pytest.mark.parametrize("dtype,dcode,D", [(torch.bfloat16, 0, 64), (torch.float16, 1, 96)])
def test_decode_ctypes_stub_appends_and_attends(lib, dtype, dcode, D):
    """A ctypes decode loop as a reference-side caller would write it: append at cache_seqlens,
    attend, advance the lengths."""
    B, H, N_max, lens = 2, 4, 2048, [1500, 7]
    q, kc, vc, kn, vn = _decode_case(B, H, N_max, D, dtype, 20 + D)
    k_ref, v_ref = _np(kc), _np(vc)
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    out = torch.empty(B, H, D, dtype=dtype, device=DEV)
    lse = torch.empty(B, H, device=DEV)
    ws = torch.empty(lib.tfgfa_decode_workspace_size(B, H, N_max, D), dtype=torch.uint8, device=DEV)
    _ok(lib, lib.tfgfa_decode(q.data_ptr(), S3(*q.stride()), kc.data_ptr(), S4(*kc.stride()),
                              vc.data_ptr(), S4(*vc.stride()), kn.data_ptr(), S3(*kn.stride()),
                              vn.data_ptr(), S3(*vn.stride()), sl.data_ptr(), out.data_ptr(),
                              S3(*out.stride()), lse.data_ptr(), B, H, N_max, D, dcode, D ** -0.5,
                              ws.data_ptr(), ws.numel(), _stream()))
    sl.add_(1)
    torch.cuda.synchronize()
    for b, L in enumerate(lens):
        k_ref[b, :, L], v_ref[b, :, L] = _np(kn[b]), _np(vn[b])
    assert np.array_equal(_np(kc), k_ref) and np.array_equal(_np(vc), v_ref)
    assert sl.tolist() == [L + 1 for L in lens]
    o_ref, lse_ref = decode_np(_np(q), k_ref, v_ref, [L + 1 for L in lens], D ** -0.5)
    _check(out, lse, o_ref, lse_ref, f"tfgfa_decode {dtype} D={D}")


def test_decode_bf16_entry_equals_general_entry(lib):
    B, H, N_max, lens = 3, 5, 700, [700, 1, 333]
    q, kc, vc, _, _ = _decode_case(B, H, N_max, 64, torch.bfloat16, 40)
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    outs = []
    for general in (False, True):
        o = torch.empty(B, H, 64, dtype=torch.bfloat16, device=DEV)
        lse = torch.empty(B, H, device=DEV)
        args = [q.data_ptr(), S3(*q.stride()), kc.data_ptr(), S4(*kc.stride()), vc.data_ptr(),
                S4(*vc.stride()), None, None, None, None, sl.data_ptr(), o.data_ptr(), S3(*o.stride()),
                lse.data_ptr(), B, H, N_max, 64]
        tail = [0.125, None, 0, _stream()]
        st = lib.tfgfa_decode(*args, 0, *tail) if general else lib.tfgfa_decode_bf16(*args, *tail)
        _ok(lib, st)
        outs.append((o, lse))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0].view(torch.int16), outs[1][0].view(torch.int16))
    assert torch.equal(outs[0][1], outs[1][1])
    o_ref, lse_ref = decode_np(_np(q), _np(kc), _np(vc), lens, 0.125)
    _check(outs[0][0], outs[0][1], o_ref, lse_ref, "tfgfa_decode_bf16, one workgroup per head")


def test_errors_come_back_as_status_codes(lib):
    """Rejected before any launch: a head dim that is not a multiple of 8, a head dim other
    than 64 for the bf16 decode entry."""
    q = torch.zeros(1, 1, 8, 64, dtype=torch.bfloat16, device=DEV)
    st = lib.tfgfa_fwd_bf16(q.data_ptr(), q.data_ptr(), q.data_ptr(), q.data_ptr(), None, 1, 1, 8, 36,
                            0.125, 1, _stream())
    assert st > 0 and b"head dimension" in lib.tfgfa_strerror(st)
    z3, z4 = S3(0, 0, 1), S4(0, 0, 128, 1)
    st = lib.tfgfa_decode_bf16(q.data_ptr(), z3, q.data_ptr(), z4, q.data_ptr(), z4, None, None, None, None,
                               None, q.data_ptr(), z3, None, 1, 1, 4, 128, 0.125, None, 0, _stream())
    assert st > 0 and b"head dimension" in lib.tfgfa_strerror(st)


@pytest.mark.parametrize("nbytes", [1 << 20, 6553600, 33554432 + 48])
def test_stream_read_reads_every_word(lib, nbytes):
    """tfgfa_stream_read (the decode legs' plain-read floor): workgroup w folds 16-B words
    [w * per_wg, (w + 1) * per_wg) with xor into sink[w]; checked against the same fold on the
    CPU, so every byte of the buffer was read."""
    lib.tfgfa_stream_read.restype = ctypes.c_int
    lib.tfgfa_stream_read.argtypes = [P, ctypes.c_size_t, P, P]
    g = torch.Generator(device=DEV).manual_seed(nbytes & 0xFFFF)
    buf = torch.randint(-2**31, 2**31 - 1, (nbytes // 4,), device=DEV, dtype=torch.int32, generator=g)
    sink = torch.zeros(4096, device=DEV, dtype=torch.int32)
    _ok(lib, lib.tfgfa_stream_read(buf.data_ptr(), nbytes, sink.data_ptr(), _stream()))
    torch.cuda.synchronize()
    n16 = nbytes // 16
    wg = max(256, min(4096, n16 // 2048))
    per = -(-n16 // wg)
    words = buf.cpu().numpy().view(np.uint32).reshape(n16, 4)
    words = np.bitwise_xor.reduce(words, axis=1)
    exp = np.zeros(wg, dtype=np.uint32)
    for w in range(wg):
        chunk = words[w * per:(w + 1) * per]
        exp[w] = np.bitwise_xor.reduce(chunk) if chunk.size else 0
    got = sink.cpu().numpy().view(np.uint32)[:wg]
    assert np.array_equal(got, exp)
    _say(f"stream_read {nbytes} B: {wg} workgroups, every word folded")
    assert lib.tfgfa_stream_read(buf.data_ptr() + 4, 16, sink.data_ptr(), _stream()) != 0  # misaligned
