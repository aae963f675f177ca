"""CPU-side tests of the drop-in boundary: the C ABI library, the pybind11 module and the
Python shim's checks.  No kernel is launched: every call here returns before any HIP call
(argument validation happens first, include/tfgfa.h)."""
import ctypes
import os
import re
import types

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tfgfa.h")

import custom_flash_attn  # noqa: E402
from custom_flash_attn import _C  # noqa: E402


def _header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tfgfa_\w+)\s*\(", text)))


def _header_define(name):
    m = re.search(rf"#define\s+{name}\s+(-?\d+)", open(HEADER).read())
    return int(m.group(1))


@pytest.fixture(scope="module")
def lib():
    lib = ctypes.CDLL(custom_flash_attn.library_path())
    lib.tfgfa_fwd_bf16.restype = ctypes.c_int
    lib.tfgfa_fwd_bf16.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_void_p] + [ctypes.c_int] * 4 + [
        ctypes.c_float, ctypes.c_int, ctypes.c_void_p]
    lib.tfgfa_fwd_bf16_strided.restype = ctypes.c_int
    lib.tfgfa_fwd_bf16_strided.argtypes = [ctypes.c_void_p, ctypes.c_void_p] * 4 + [ctypes.c_void_p] + [
        ctypes.c_int] * 4 + [ctypes.c_float, ctypes.c_int, ctypes.c_void_p]
    lib.tfgfa_decode_bf16.restype = ctypes.c_int
    lib.tfgfa_decode_bf16.argtypes = [ctypes.c_void_p, ctypes.c_void_p] * 5 + [
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int] * 4 + [
        ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    lib.tfgfa_decode_workspace_bytes.restype = ctypes.c_size_t
    lib.tfgfa_decode_workspace_bytes.argtypes = [ctypes.c_int] * 3
    lib.tfgfa_decode.restype = ctypes.c_int
    lib.tfgfa_decode.argtypes = [ctypes.c_void_p, ctypes.c_void_p] * 5 + [
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int] * 5 + [
        ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    lib.tfgfa_decode_workspace_size.restype = ctypes.c_size_t
    lib.tfgfa_decode_workspace_size.argtypes = [ctypes.c_int] * 4
    lib.tfgfa_fwd.restype = ctypes.c_int
    lib.tfgfa_fwd.argtypes = [ctypes.c_void_p, ctypes.c_void_p] * 4 + [ctypes.c_void_p] + [
        ctypes.c_int] * 6 + [ctypes.c_float, ctypes.c_int, ctypes.c_void_p]
    lib.tfgfa_strerror.restype = ctypes.c_char_p
    lib.tfgfa_strerror.argtypes = [ctypes.c_int]
    lib.tfgfa_abi_version.restype = ctypes.c_int
    return lib


def test_library_exports_every_declared_symbol(lib):
    names = _header_functions()
    assert names == ["tfgfa_abi_version", "tfgfa_decode", "tfgfa_decode_bf16",
                     "tfgfa_decode_noalloc", "tfgfa_decode_scratch_bytes", "tfgfa_decode_splits",
                     "tfgfa_decode_workspace_bytes", "tfgfa_decode_workspace_size",
                     "tfgfa_device_info", "tfgfa_fwd", "tfgfa_fwd_bf16", "tfgfa_fwd_bf16_strided",
                     "tfgfa_stream_read", "tfgfa_strerror"]
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/tfgfa.h but not exported"


def _split_bytes(bh, D, S):
    """Workspace bytes of a split of S (include/tfgfa.h, tfgfa_decode_splits): arrival words
    (B*H*128 rounded up to 256), then B*H*S partials of D + 1 floats; none for S = 1."""
    return 0 if S <= 1 else -(-bh * 128 // 256) * 256 + bh * S * (D + 1) * 4


def test_decode_noalloc_scratch_holds_the_split_on_256_cus(lib):
    """tfgfa_decode_noalloc uses its static scratch as a workspace: on a 256-CU MI355X the split
    it then chooses is the full-workspace split for every shape (so its results are bitwise
    tfgfa_decode's), at most 280 KiB; with more CUs it splits only as far as the scratch holds."""
    lib.tfgfa_decode_splits.restype = ctypes.c_int
    lib.tfgfa_decode_splits.argtypes = [ctypes.c_int] * 5 + [ctypes.c_size_t]
    lib.tfgfa_decode_scratch_bytes.restype = ctypes.c_size_t
    lib.tfgfa_decode_workspace_size.restype = ctypes.c_size_t
    lib.tfgfa_decode_workspace_size.argtypes = [ctypes.c_int] * 4
    scratch = lib.tfgfa_decode_scratch_bytes()
    assert scratch == 320 * 1024
    worst = 0
    lengths = (1, 512, 1023, 1024, 1025, 2048, 4096, 8192, 16384, 32768, 1 << 20)
    for bh in list(range(1, 131)) + [200, 1000]:
        for D in range(8, 129, 8):
            for n in lengths:
                full = lib.tfgfa_decode_workspace_size(1, bh, n, D)
                S = lib.tfgfa_decode_splits(1, bh, n, D, 256, full)
                assert S >= 1 and (S == 1 or 2 * bh <= 256)
                assert lib.tfgfa_decode_splits(1, bh, n, D, 256, scratch) == S, (bh, D, n)
                worst = max(worst, _split_bytes(bh, D, S))
    assert worst <= 280 * 1024, worst
    # A part with more CUs: the full-workspace split may outgrow the scratch; the scratch's own
    # split always fits it.
    outgrown = 0
    for cu in (304, 512, 1024):
        for bh in (1, 8, 64, cu // 2):
            for D in (64, 128):
                full = lib.tfgfa_decode_workspace_size(1, bh, 1 << 16, D)
                s_full = lib.tfgfa_decode_splits(1, bh, 1 << 16, D, cu, full)
                s_scr = lib.tfgfa_decode_splits(1, bh, 1 << 16, D, cu, scratch)
                assert 1 <= s_scr <= s_full and _split_bytes(bh, D, s_scr) <= scratch
                outgrown += s_scr < s_full
    assert outgrown > 0
    # Out-of-range sizes.
    assert lib.tfgfa_decode_splits(0, 1, 16, 64, 256, 0) == 0
    assert lib.tfgfa_decode_splits(1, 1, 16, 36, 256, 0) == 0
    assert lib.tfgfa_decode_splits(1, 1, 16, 64, 0, 0) == 0
    assert lib.tfgfa_decode_splits(1, 4, 8192, 64, 256, 0) == 1  # no workspace: no split


def test_stream_read_validates_before_any_hip_call(lib):
    """tfgfa_stream_read (the measurement floor of the split decode legs) checks its arguments
    on the host: nothing to read is a no-op, a null pointer or a misaligned pointer or size is
    an error, all without touching a device."""
    lib.tfgfa_stream_read.restype = ctypes.c_int
    lib.tfgfa_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p]
    P, S = 0x10000, 0x20000  # never dereferenced: every call below returns before a launch
    assert lib.tfgfa_stream_read(P, 0, S, None) == _header_define("TFGFA_OK")
    assert lib.tfgfa_stream_read(None, 4096, S, None) == _header_define("TFGFA_ERR_NULL_POINTER")
    assert lib.tfgfa_stream_read(P, 4096, None, None) == _header_define("TFGFA_ERR_NULL_POINTER")
    assert lib.tfgfa_stream_read(P + 8, 4096, S, None) == _header_define("TFGFA_ERR_ALIGNMENT")
    assert lib.tfgfa_stream_read(P, 4100, S, None) == _header_define("TFGFA_ERR_ALIGNMENT")
    assert lib.tfgfa_stream_read(P, 4096, S + 2, None) == _header_define("TFGFA_ERR_ALIGNMENT")


def test_abi_version(lib):
    assert lib.tfgfa_abi_version() == _header_define("TFGFA_ABI_VERSION")
    assert _C.abi_version() == _header_define("TFGFA_ABI_VERSION")


def test_strerror_covers_every_status(lib):
    codes = [_header_define(n) for n in (
        "TFGFA_OK", "TFGFA_ERR_NULL_POINTER", "TFGFA_ERR_BAD_SHAPE", "TFGFA_ERR_HEAD_DIM",
        "TFGFA_ERR_SCALE", "TFGFA_ERR_CAUSAL_FLAG", "TFGFA_ERR_TOO_LARGE", "TFGFA_ERR_ALIGNMENT",
        "TFGFA_ERR_STRIDE", "TFGFA_ERR_CACHE", "TFGFA_ERR_DTYPE", "TFGFA_ERR_SCRATCH")]
    msgs = [lib.tfgfa_strerror(c).decode() for c in codes]
    assert len(set(msgs)) == len(msgs)
    assert lib.tfgfa_strerror(12345).decode() == "unknown tfgfa status"
    assert _C.strerror(3) == msgs[3]


# Fake, 16-byte-aligned device addresses: validation never dereferences them.
P = 0x10000


@pytest.mark.parametrize("args,code", [
    ((0, P, P, P, 0, 1, 1, 16, 64, 0.125, 1), "TFGFA_ERR_NULL_POINTER"),
    ((P, P, P, 0, 0, 1, 1, 16, 64, 0.125, 1), "TFGFA_ERR_NULL_POINTER"),
    ((P, P, P, P, 0, -1, 1, 16, 64, 0.125, 1), "TFGFA_ERR_BAD_SHAPE"),
    ((P, P, P, P, 0, 1, 1, -16, 64, 0.125, 1), "TFGFA_ERR_BAD_SHAPE"),
    ((P, P, P, P, 0, 1, 1, 16, 136, 0.125, 1), "TFGFA_ERR_HEAD_DIM"),   # > 128
    ((P, P, P, P, 0, 1, 1, 16, 36, 0.125, 1), "TFGFA_ERR_HEAD_DIM"),    # not a multiple of 8
    ((P, P, P, P, 0, 1, 1, 16, 0, 0.125, 1), "TFGFA_ERR_HEAD_DIM"),
    ((P, P, P, P, 0, 1, 1, 16, 64, 0.0, 1), "TFGFA_ERR_SCALE"),
    ((P, P, P, P, 0, 1, 1, 16, 64, -0.125, 1), "TFGFA_ERR_SCALE"),
    ((P, P, P, P, 0, 1, 1, 16, 64, float("nan"), 1), "TFGFA_ERR_SCALE"),
    ((P, P, P, P, 0, 1, 1, 16, 64, float("inf"), 1), "TFGFA_ERR_SCALE"),
    ((P, P, P, P, 0, 1, 1, 16, 64, 0.125, 2), "TFGFA_ERR_CAUSAL_FLAG"),
    ((P + 2, P, P, P, 0, 1, 1, 16, 64, 0.125, 1), "TFGFA_ERR_ALIGNMENT"),
    ((P, P, P, P + 8, 0, 1, 1, 16, 64, 0.125, 1), "TFGFA_ERR_ALIGNMENT"),
    ((P, P, P, P, P + 2, 1, 1, 16, 64, 0.125, 1), "TFGFA_ERR_ALIGNMENT"),
    ((P, P, P, P, 0, 65536, 65536, 16, 64, 0.125, 1), "TFGFA_ERR_TOO_LARGE"),
    ((P, P, P, P, 0, 1, 1, 1 << 30, 64, 0.125, 1), "TFGFA_ERR_TOO_LARGE"),
    ((P, P, P, P, 0, 0, 4, 16, 64, 0.125, 1), "TFGFA_OK"),   # empty problem: nothing launched
    ((P, P, P, P, 0, 2, 4, 0, 64, 0.125, 0), "TFGFA_OK"),
    ((0, 0, 0, 0, 0, 2, 4, 0, 64, 0.125, 1), "TFGFA_OK"),     # empty tensors have NULL data
    ((0, 0, 0, 0, 0, 2, 4, 0, 132, 0.125, 1), "TFGFA_ERR_HEAD_DIM"),  # sizes checked first
    ((0, P, P, P, 0, 1, 1, 16, 128, 0.125, 1), "TFGFA_ERR_NULL_POINTER"),  # d = 128 accepted
    ((0, P, P, P, 0, 1, 1, 16, 8, 0.125, 1), "TFGFA_ERR_NULL_POINTER"),    # d = 8 accepted
])
def test_c_abi_argument_validation(lib, args, code):
    assert lib.tfgfa_fwd_bf16(*args, None) == _header_define(code)


def _st(*vals):
    return (ctypes.c_int64 * 4)(*vals)


def _contig(B, H, N):
    return _st(H * N * 64, N * 64, 64, 1)


# Strided entry point.  Strides are checked before pointers, so a NULL-pointer status means the
# strides were accepted; no case here reaches a launch.
@pytest.mark.parametrize("B,H,N,qs,code", [
    (2, 3, 16, None, "TFGFA_ERR_NULL_POINTER"),                        # NULL strides: contiguous
    (2, 3, 16, (3 * 16 * 64, 16 * 64, 64, 1), "TFGFA_ERR_NULL_POINTER"),
    (2, 3, 16, (16 * 3 * 64, 64, 3 * 64, 1), "TFGFA_ERR_NULL_POINTER"),  # (B, N, H, D) view
    (2, 3, 16, (16 * 9 * 64, 64, 9 * 64, 1), "TFGFA_ERR_NULL_POINTER"),  # fused QKV rows
    (2, 3, 16, (3 * 16 * 72, 16 * 72, 72, 1), "TFGFA_ERR_NULL_POINTER"),  # padded rows
    (1, 1, 16, (7, 3, 64, 1), "TFGFA_ERR_NULL_POINTER"),                # size-1 dims ignored
    (2, 3, 1, (3 * 64, 64, 5, 1), "TFGFA_ERR_NULL_POINTER"),            # N = 1: row stride ignored
    (2, 3, 16, (3 * 16 * 64, 16 * 64, 64, 2), "TFGFA_ERR_STRIDE"),      # dim not dense
    (2, 3, 16, (3 * 16 * 64, 16 * 64, 32, 1), "TFGFA_ERR_STRIDE"),      # overlapping rows
    (2, 3, 16, (3 * 16 * 64, 16 * 64, 0, 1), "TFGFA_ERR_STRIDE"),
    (2, 3, 16, (3 * 16 * 64, 16 * 64, 68, 1), "TFGFA_ERR_STRIDE"),      # 136 B rows: misaligned
    (2, 3, 16, (3 * 16 * 64, 16 * 64 + 4, 64, 1), "TFGFA_ERR_STRIDE"),
    (2, 3, 16, (3 * 16 * 64 + 4, 16 * 64, 64, 1), "TFGFA_ERR_STRIDE"),
    (2, 3, 16, (-3 * 16 * 64, 16 * 64, 64, 1), "TFGFA_ERR_STRIDE"),
    (2, 3, 16, (3 * 16 * 64, -16 * 64, 64, 1), "TFGFA_ERR_STRIDE"),
    (2, 3, 16, (0, 0, 1 << 30, 1), "TFGFA_ERR_TOO_LARGE"),              # 32-bit buffer offsets
    (2, 3, 4096, (0, 0, (1 << 18), 1), "TFGFA_ERR_TOO_LARGE"),
    (0, 3, 16, (0, 0, 1, 5), "TFGFA_OK"),                               # empty: nothing checked
])
@pytest.mark.parametrize("which", [0, 1, 2, 3])
def test_c_abi_strided_validation(lib, B, H, N, qs, code, which):
    strides = [_contig(B, H, N) for _ in range(4)]
    strides[which] = None if qs is None else _st(*qs)
    args = []
    for s in strides:
        args += [None, s]
    assert lib.tfgfa_fwd_bf16_strided(*args, None, B, H, N, 64, 0.125, 1, None) == _header_define(code)


@pytest.mark.parametrize("os_,code", [
    ((0, 0, 64, 1), "TFGFA_ERR_STRIDE"),                    # every head onto one
    ((3 * 16 * 64, 0, 64, 1), "TFGFA_ERR_STRIDE"),
    ((3 * 16 * 64, 64, 64, 1), "TFGFA_ERR_STRIDE"),         # heads and rows collide
    ((3 * 16 * 64, 16 * 64 - 8, 64, 1), "TFGFA_ERR_STRIDE"),  # last row of a head hits the next
    ((16 * 3 * 64, 64, 3 * 64, 1), "TFGFA_ERR_NULL_POINTER"),  # (B, N, H, D) buffer
    ((64, 2 * 64, 6 * 64, 1), "TFGFA_ERR_NULL_POINTER"),     # batch innermost
    ((3 * 16 * 80, 16 * 80, 80, 1), "TFGFA_ERR_NULL_POINTER"),  # padded rows
])
def test_c_abi_strided_output_overlap(lib, os_, code):
    B, H, N = 2, 3, 16
    c = _contig(B, H, N)
    assert lib.tfgfa_fwd_bf16_strided(None, c, None, c, None, c, None, _st(*os_), None,
                                      B, H, N, 64, 0.125, 1, None) == _header_define(code)
    # Inputs may share elements (e.g. K broadcast over heads).
    assert lib.tfgfa_fwd_bf16_strided(None, _st(*os_), None, c, None, c, None, c, None,
                                      B, H, N, 64, 0.125, 1, None) == _header_define("TFGFA_ERR_NULL_POINTER")


def test_c_abi_strided_checks_sizes_before_strides(lib):
    bad = _st(0, 0, 1, 5)
    assert lib.tfgfa_fwd_bf16_strided(None, bad, None, bad, None, bad, None, bad, None,
                                      1, 1, 16, 132, 0.125, 1, None) == _header_define("TFGFA_ERR_HEAD_DIM")
    ok = _contig(1, 1, 16)
    assert lib.tfgfa_fwd_bf16_strided(P + 2, ok, P, ok, P, ok, P, ok, None,
                                      1, 1, 16, 64, 0.125, 1, None) == _header_define("TFGFA_ERR_ALIGNMENT")


def test_pybind_strided_raises_runtime_error_with_message():
    c = (64 * 16, 64 * 16, 64, 1)
    with pytest.raises(RuntimeError, match="unsupported strides"):
        _C.fwd_strided(P, (64 * 16, 64 * 16, 32, 1), P, c, P, c, P, c, 0, 1, 1, 16, 64, 0.125, True, 0)
    with pytest.raises(RuntimeError, match="tfgfa_fwd_bf16_strided failed"):
        _C.fwd_strided(0, c, P, c, P, c, P, c, 0, 1, 1, 16, 64, 0.125, True, 0)


# Decode entry point.  q, o, k_new, v_new: (B, H, 64) with strides [b, h, d]; caches
# (B, H, N_max, 64) with [b, h, n, d].  Every case stops before any HIP call.
def _s3(*v):
    return (ctypes.c_int64 * 3)(*v)


def _decode_args(B=2, H=3, N=100, q=None, kc=None, vc=None, kn=None, vn=None, seq=None, o=None,
                 lse=None, qs=None, ks=None, vs=None, kns=None, vns=None, os_=None, D=64,
                 scale=0.125, ws=None, ws_bytes=0):
    qs = qs or _s3(H * 64, 64, 1)
    ks = ks or _st(H * N * 64, N * 64, 64, 1)
    vs = vs or _st(H * N * 64, N * 64, 64, 1)
    kns = kns or _s3(H * 64, 64, 1)
    vns = vns or _s3(H * 64, 64, 1)
    os_ = os_ or _s3(H * 64, 64, 1)
    return (q, qs, kc, ks, vc, vs, kn, kns, vn, vns, seq, o, os_, lse, B, H, N, D, scale, ws,
            ws_bytes, None)


@pytest.mark.parametrize("kw,code", [
    (dict(B=-1), "TFGFA_ERR_BAD_SHAPE"),
    (dict(N=-5), "TFGFA_ERR_BAD_SHAPE"),
    (dict(D=128), "TFGFA_ERR_HEAD_DIM"),
    (dict(scale=0.0), "TFGFA_ERR_SCALE"),
    (dict(scale=float("nan")), "TFGFA_ERR_SCALE"),
    (dict(kn=P), "TFGFA_ERR_NULL_POINTER"),                     # k_new without v_new
    (dict(kn=P, vn=P), "TFGFA_ERR_CACHE"),                      # append needs cache_seqlens
    (dict(B=0), "TFGFA_OK"),                                    # empty: nothing launched
    (dict(H=0, kn=P, vn=P, seq=P), "TFGFA_OK"),
    (dict(), "TFGFA_ERR_NULL_POINTER"),                         # strides accepted, q NULL
    (dict(qs=_s3(192, 64, 2)), "TFGFA_ERR_STRIDE"),             # q dim not dense
    (dict(qs=_s3(192, 60, 1)), "TFGFA_ERR_STRIDE"),             # q head stride not a multiple of 8
    (dict(ks=_st(3 * 100 * 64, 100 * 64, 32, 1)), "TFGFA_ERR_STRIDE"),   # overlapping cache rows
    (dict(vs=_st(3 * 100 * 72, 100 * 72, 68, 1)), "TFGFA_ERR_STRIDE"),   # 136-byte rows
    (dict(ks=_st(3 * 100 * 64, 100 * 64, 64, 2)), "TFGFA_ERR_STRIDE"),
    (dict(os_=_s3(64, 64, 1)), "TFGFA_ERR_STRIDE"),             # O rows of two batches collide
    (dict(os_=_s3(0, 64, 1)), "TFGFA_ERR_STRIDE"),
    (dict(kn=P, vn=P, seq=P, kns=_s3(192, 64, 3)), "TFGFA_ERR_STRIDE"),
    (dict(q=P, kc=P, vc=P, o=P, B=1, H=1, qs=_s3(7, 5, 1), os_=_s3(3, 9, 1), ks=_st(1, 2, 64, 1),
          vs=_st(1, 2, 64, 1), lse=P + 2), "TFGFA_ERR_ALIGNMENT"),  # size-1 strides ignored
    (dict(N=1 << 24), "TFGFA_ERR_TOO_LARGE"),
    (dict(q=P + 8, kc=P, vc=P, o=P), "TFGFA_ERR_ALIGNMENT"),
    (dict(q=P, kc=P, vc=P, o=P, seq=P + 2), "TFGFA_ERR_ALIGNMENT"),
    (dict(q=P, kc=P, vc=P, o=P, ws=P + 8, ws_bytes=4096), "TFGFA_ERR_ALIGNMENT"),
    (dict(q=P, kc=None, vc=P, o=P), "TFGFA_ERR_NULL_POINTER"),
])
def test_c_abi_decode_validation(lib, kw, code):
    assert lib.tfgfa_decode_bf16(*_decode_args(**kw)) == _header_define(code)


def _general(args, dtype=0):
    """tfgfa_decode_bf16 arguments -> tfgfa_decode arguments (dtype after D)."""
    return args[:18] + (dtype,) + args[18:]


@pytest.mark.parametrize("kw,code", [
    (dict(), "TFGFA_ERR_NULL_POINTER"),                          # bf16 D = 64, q NULL
    (dict(B=-1), "TFGFA_ERR_BAD_SHAPE"),
    (dict(D=128, ks=_st(3 * 100 * 128, 100 * 128, 128, 1), vs=_st(3 * 100 * 128, 100 * 128, 128, 1),
          qs=_s3(384, 128, 1), os_=_s3(384, 128, 1)), "TFGFA_ERR_NULL_POINTER"),   # D = 128 accepted
    (dict(D=40), "TFGFA_ERR_NULL_POINTER"),                      # rows of 64 >= 40: accepted
    (dict(D=8), "TFGFA_ERR_NULL_POINTER"),
    (dict(D=36), "TFGFA_ERR_HEAD_DIM"),                          # not a multiple of 8
    (dict(D=0), "TFGFA_ERR_HEAD_DIM"),
    (dict(D=136), "TFGFA_ERR_HEAD_DIM"),                         # > 128
    (dict(D=128), "TFGFA_ERR_STRIDE"),                           # cache rows of 64 < D
    (dict(D=72, os_=_s3(72, 64, 1), qs=_s3(216, 72, 1),
          ks=_st(3 * 100 * 72, 100 * 72, 72, 1), vs=_st(3 * 100 * 72, 100 * 72, 72, 1)),
     "TFGFA_ERR_STRIDE"),                                        # O rows of 72 at stride 64 overlap
    (dict(scale=-1.0), "TFGFA_ERR_SCALE"),
    (dict(kn=P, vn=P), "TFGFA_ERR_CACHE"),
])
@pytest.mark.parametrize("dtype", [0, 1])
def test_c_abi_general_decode_validation(lib, kw, code, dtype):
    assert lib.tfgfa_decode(*_general(_decode_args(**kw), dtype)) == _header_define(code)


@pytest.mark.parametrize("dtype", [2, -1, 100])
def test_c_abi_general_decode_rejects_unknown_dtype(lib, dtype):
    assert lib.tfgfa_decode(*_general(_decode_args(), dtype)) == _header_define("TFGFA_ERR_DTYPE")


def test_general_decode_agrees_with_bf16_entry_on_d64_validation(lib):
    """Every argument case of the bf16 entry gets the same status from tfgfa_decode with
    dtype bf16, except head dims the general entry takes."""
    for kw in (dict(B=-1), dict(N=-5), dict(scale=0.0), dict(kn=P), dict(kn=P, vn=P), dict(B=0),
               dict(), dict(qs=_s3(192, 64, 2)), dict(ks=_st(3 * 100 * 64, 100 * 64, 32, 1)),
               dict(os_=_s3(64, 64, 1)), dict(N=1 << 24), dict(q=P + 8, kc=P, vc=P, o=P),
               dict(q=P, kc=P, vc=P, o=P, ws=P + 8, ws_bytes=4096)):
        args = _decode_args(**kw)
        assert lib.tfgfa_decode(*_general(args)) == lib.tfgfa_decode_bf16(*args), kw


def test_c_abi_noalloc_decode_validation(lib):
    """tfgfa_decode_noalloc takes tfgfa_decode's arguments less the workspace and reports every
    argument error the same way, before any HIP call (no compute call here)."""
    lib.tfgfa_decode_noalloc.restype = ctypes.c_int
    lib.tfgfa_decode_noalloc.argtypes = [ctypes.c_void_p, ctypes.c_void_p] * 5 + [
        ctypes.c_void_p] * 4 + [ctypes.c_int] * 5 + [ctypes.c_float, ctypes.c_void_p]
    for kw in (dict(), dict(B=-1), dict(N=-5), dict(D=36), dict(D=136), dict(scale=0.0),
               dict(kn=P), dict(kn=P, vn=P), dict(B=0), dict(qs=_s3(192, 64, 2)),
               dict(ks=_st(3 * 100 * 64, 100 * 64, 32, 1)), dict(os_=_s3(64, 64, 1)),
               dict(N=1 << 24), dict(q=P + 8, kc=P, vc=P, o=P), dict(q=P, kc=P, vc=P, o=P, seq=P + 2)):
        for dtype in (0, 1, 7):
            general = _general(_decode_args(**kw), dtype)
            noalloc = general[:20] + general[22:]
            assert lib.tfgfa_decode_noalloc(*noalloc) == lib.tfgfa_decode(*general), (kw, dtype)


def _decode_ws_bytes(B, H, N, D):
    """Decode workspace layout: one 64-bit arrival word per head, 128 bytes apart, rounded up to
    256 bytes; then one partial (D + 1 floats) per head per 128 cache rows."""
    return -(-B * H * 128 // 256) * 256 + B * H * (-(-N // 128)) * (D + 1) * 4


def test_decode_workspace_size(lib):
    assert lib.tfgfa_decode_workspace_size(8, 25, 1024, 64) == lib.tfgfa_decode_workspace_bytes(8, 25, 1024)
    assert lib.tfgfa_decode_workspace_size(1, 1, 1, 128) == 256 + 129 * 4
    assert lib.tfgfa_decode_workspace_size(2, 3, 300, 40) == 768 + 6 * 3 * 41 * 4
    for args in ((8, 25, 1024, 64), (1, 16, 8192, 128), (3, 5, 77, 8)):
        assert lib.tfgfa_decode_workspace_size(*args) == _decode_ws_bytes(*args)
    for bad in ((0, 1, 1, 64), (1, 0, 1, 64), (1, 1, 0, 64), (1, 1, 1, 0), (1, 1, 1, 12),
                (1, 1, 1, 136)):
        assert lib.tfgfa_decode_workspace_size(*bad) == 0
    assert _C.decode_workspace_size(2, 3, 300, 40) == lib.tfgfa_decode_workspace_size(2, 3, 300, 40)


def test_pybind_general_decode_raises_runtime_error_with_message():
    z3 = (0, 0, 0)
    with pytest.raises(RuntimeError, match="tfgfa_decode failed .*dtype"):
        _C.decode_general(P, z3, P, (0, 0, 0, 1), P, (0, 0, 0, 1), 0, z3, 0, z3, 0, P, z3, 0,
                          2, 3, 100, 64, 7, 0.125, 0, 0, 0)
    with pytest.raises(RuntimeError, match="unsupported head dimension"):
        _C.decode_general(P, z3, P, (0, 0, 0, 1), P, (0, 0, 0, 1), 0, z3, 0, z3, 0, P, z3, 0,
                          2, 3, 100, 20, 1, 0.125, 0, 0, 0)


def test_decode_workspace_bytes(lib):
    # arrival words, then one partial slot per 128 rows
    assert lib.tfgfa_decode_workspace_bytes(8, 25, 1024) == 25600 + 8 * 25 * 8 * 65 * 4
    assert lib.tfgfa_decode_workspace_bytes(1, 1, 1) == 256 + 65 * 4
    assert lib.tfgfa_decode_workspace_bytes(1, 16, 8193) == 2048 + 16 * 65 * 65 * 4
    for bad in ((0, 1, 1), (1, 0, 1), (1, 1, 0), (-1, 2, 3)):
        assert lib.tfgfa_decode_workspace_bytes(*bad) == 0
    assert _C.decode_workspace_bytes(8, 25, 1024) == lib.tfgfa_decode_workspace_bytes(8, 25, 1024)


def test_pybind_decode_raises_runtime_error_with_message():
    z3 = (0, 0, 0)
    with pytest.raises(RuntimeError, match="tfgfa_decode_bf16 failed .*cache_seqlens"):
        _C.decode(P, (192, 64, 1), P, (19200, 6400, 64, 1), P, (19200, 6400, 64, 1), P, (192, 64, 1),
                  P, (192, 64, 1), 0, P, (192, 64, 1), 0, 2, 3, 100, 64, 0.125, 0, 0, 0)
    with pytest.raises(RuntimeError, match="unsupported head dimension"):
        _C.decode(P, z3, P, (0, 0, 0, 1), P, (0, 0, 0, 1), 0, z3, 0, z3, 0, P, z3, 0,
                  2, 3, 100, 32, 0.125, 0, 0, 0)


def _fwd_args(q=None, k=None, v=None, o=None, lse=None, qs=None, ks=None, vs=None, os_=None, B=2,
              H=3, Nq=50, Nk=70, D=96, dtype=0, scale=0.125, causal=1):
    return (q, qs, k, ks, v, vs, o, os_, lse, B, H, Nq, Nk, D, dtype, scale, causal, None)


@pytest.mark.parametrize("kw,code", [
    (dict(), "TFGFA_ERR_NULL_POINTER"),                      # N_q != N_k, D = 96, NULL strides
    (dict(dtype=1, D=128), "TFGFA_ERR_NULL_POINTER"),        # fp16
    (dict(dtype=2), "TFGFA_ERR_DTYPE"),
    (dict(dtype=-1), "TFGFA_ERR_DTYPE"),
    (dict(D=100), "TFGFA_ERR_HEAD_DIM"),
    (dict(D=144), "TFGFA_ERR_HEAD_DIM"),
    (dict(Nk=0), "TFGFA_ERR_BAD_SHAPE"),                     # queries but no keys
    (dict(Nq=0, Nk=0), "TFGFA_OK"),                          # empty
    (dict(Nq=-1), "TFGFA_ERR_BAD_SHAPE"),
    (dict(ks=(70 * 3 * 96, 96, 3 * 96, 1)), "TFGFA_ERR_NULL_POINTER"),   # (B, N_k, H, D) view
    (dict(ks=(70 * 3 * 96, 96, 64, 1)), "TFGFA_ERR_STRIDE"),             # row stride < D
    (dict(qs=(50 * 3 * 104, 50 * 104, 104, 1)), "TFGFA_ERR_NULL_POINTER"),  # padded rows
    (dict(os_=(50 * 3 * 96, 96, 96, 1)), "TFGFA_ERR_STRIDE"),            # O heads and rows collide
    (dict(q=P, k=P, v=P, o=P + 8), "TFGFA_ERR_ALIGNMENT"),
])
def test_c_abi_general_forward_validation(lib, kw, code):
    args = list(_fwd_args(**{k_: v_ for k_, v_ in kw.items() if k_ not in ("qs", "ks", "vs", "os_")}))
    for key, idx in (("qs", 1), ("ks", 3), ("vs", 5), ("os_", 7)):
        if key in kw:
            args[idx] = _st(*kw[key])
    assert lib.tfgfa_fwd(*args) == _header_define(code)


def test_header_dtype_codes():
    assert _header_define("TFGFA_DTYPE_BF16") == _C.DTYPE_BF16 == 0
    assert _header_define("TFGFA_DTYPE_F16") == _C.DTYPE_F16 == 1


def test_pybind_raises_runtime_error_with_message():
    with pytest.raises(RuntimeError, match="unsupported head dimension"):
        _C.fwd(P, P, P, P, 0, 1, 1, 16, 136, 0.125, True, 0)
    with pytest.raises(RuntimeError, match="tfgfa_fwd failed .*dtype"):
        _C.fwd_general(P, (0, 0, 64, 1), P, (0, 0, 64, 1), P, (0, 0, 64, 1), P, (0, 0, 64, 1), 0,
                       1, 1, 16, 16, 64, 5, 0.125, True, 0)
    with pytest.raises(RuntimeError, match="null tensor pointer"):
        _C.fwd(0, P, P, P, 0, 1, 1, 16, 64, 0.125, True, 0)


# ------------------------------------------------------------------ shim checks


def test_forward_rejects_cpu_tensors_like_the_reference():
    q = torch.zeros(1, 1, 4, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="^Q must be a CUDA tensor$"):
        custom_flash_attn.forward(q, q, q)
    with pytest.raises(RuntimeError, match="^Q must be a CUDA tensor$"):
        custom_flash_attn.forward_lse(q, q, q)


class _FakeCuda:
    """Stands in for a device tensor so the shim's later checks can run on the CPU."""

    def __init__(self, shape=(1, 2, 8, 64), dtype=torch.bfloat16, contiguous=True, device="cuda:0",
                 last_stride=1):
        self.shape = torch.Size(shape)
        self.dtype = dtype
        self.is_cuda = True
        self._contig = contiguous
        self.device = torch.device(device)
        self._last_stride = last_stride

    def stride(self, dim=None):
        st = (0, 0, 0, self._last_stride)[-len(self.shape):]
        return st if dim is None else st[dim]

    def is_contiguous(self):
        return self._contig

    def dim(self):
        return len(self.shape)


@pytest.mark.parametrize("qkv,msg", [
    ((_FakeCuda(contiguous=False), _FakeCuda(), _FakeCuda()), "^Q must be contiguous$"),
    ((_FakeCuda(), _FakeCuda(contiguous=False), _FakeCuda()), "^K_mat must be contiguous$"),
    ((_FakeCuda(), _FakeCuda(), _FakeCuda(contiguous=False)), "^V must be contiguous$"),
    ((_FakeCuda(dtype=torch.float16),) * 3, r"^Unsupported tensor dtype. Use bfloat16.$"),
    ((_FakeCuda(dtype=torch.float32),) * 3, r"^Unsupported tensor dtype. Use bfloat16.$"),
    ((_FakeCuda(), _FakeCuda(dtype=torch.float16), _FakeCuda()), r"^Unsupported tensor dtype"),
    ((_FakeCuda(shape=(2, 8, 64)),) * 3, "must be 4-D"),
    ((_FakeCuda(), _FakeCuda(shape=(1, 2, 9, 64)), _FakeCuda()), "same shape"),
    ((_FakeCuda(), _FakeCuda(), _FakeCuda(device="cuda:1")), "same device"),
    ((_FakeCuda(shape=(1, 2, 8, 128)),) * 3, "head_dim must be 64"),
])
def test_shim_validation_messages(qkv, msg):
    with pytest.raises(RuntimeError, match=msg):
        custom_flash_attn._validate(*qkv)


@pytest.mark.parametrize("qkv,out,msg", [
    ((_FakeCuda(dtype=torch.float32), _FakeCuda(), _FakeCuda()), None, r"^Unsupported tensor dtype"),
    ((_FakeCuda(), _FakeCuda(dtype=torch.float16), _FakeCuda()), None, "k must have dtype"),
    ((_FakeCuda(shape=(2, 8, 64)),) * 3, None, "q must be 4-D"),
    ((_FakeCuda(), _FakeCuda(shape=(1, 3, 9, 64)), _FakeCuda()), None, "k must have shape"),
    ((_FakeCuda(), _FakeCuda(shape=(1, 2, 9, 64)), _FakeCuda()), None, "v must have shape"),
    ((_FakeCuda(), _FakeCuda(), _FakeCuda(device="cuda:1")), None, "v must be on"),
    ((_FakeCuda(shape=(1, 2, 8, 136)),) * 3, None, r"head_dim must be in \[1, 128\]"),
    ((_FakeCuda(), _FakeCuda(last_stride=2), _FakeCuda()), None, r"k must be dense in its last dimension"),
    ((_FakeCuda(),) * 3, _FakeCuda(shape=(1, 2, 8, 32)), "out must have shape"),
    ((_FakeCuda(),) * 3, _FakeCuda(dtype=torch.float32), r"^Unsupported tensor dtype"),
])
def test_attention_view_validation_messages(qkv, out, msg):
    # Non-contiguous views are accepted: only the last dimension must be dense.
    with pytest.raises(RuntimeError, match=msg):
        custom_flash_attn._check_view(qkv[0], "q", None)
        custom_flash_attn._check_view(qkv[1], "k", qkv[0])
        custom_flash_attn._check_view(qkv[2], "v", qkv[0], rows_from=qkv[1])
        if out is not None:
            custom_flash_attn._check_view(out, "out", qkv[0], rows_from=qkv[0])


def test_attention_rejects_cpu_tensors():
    q = torch.zeros(1, 1, 4, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="^q must be a CUDA tensor$"):
        custom_flash_attn.attention(q, q, q)


@pytest.mark.parametrize("shapes,dtypes,msg", [
    (((1, 2, 8, 160),) * 3, (torch.bfloat16,) * 3, "head dimensions up to 128"),
    (((1, 2, 8, 64),) * 3, (torch.bfloat16, torch.float16, torch.bfloat16), "same type"),
    (((1, 2, 8, 64),) * 3, (torch.float32,) * 3, "fp16 and bf16"),
    (((1, 2, 8, 64), (1, 2, 9, 64), (1, 2, 10, 64)), (torch.bfloat16,) * 3, None),
])
def test_flash_attn_forward_asserts_like_the_triton_wrapper(shapes, dtypes, msg):
    q, k, v = (torch.zeros(s, dtype=d) for s, d in zip(shapes, dtypes))
    with pytest.raises(AssertionError, match=msg):
        custom_flash_attn.flash_attn_forward(q, k, v)


def test_forward_is_positional_only():
    q = torch.zeros(1, 1, 4, 64, dtype=torch.bfloat16)
    with pytest.raises(TypeError):
        custom_flash_attn.forward(Q=q, K_mat=q, V=q)


# ------------------------------------------------------------------ GPT-2 caller (CPU)


def test_gpt2_manual_and_functional_agree_on_cpu():
    import model_inference as mi

    cfg = dict(mi.GPT_CONFIG_124M)
    cfg.update({"emb_dim": 128, "n_layers": 2, "n_heads": 2, "vocab_size": 97,
                "context_length": 64, "drop_rate": 0.0, "qkv_bias": True})
    outs = {}
    for impl in ("manual", "functional"):
        torch.manual_seed(0)
        model = mi.GPTModel(dict(cfg, impl_type=impl)).eval()
        mi.init_gpt2_weights(model, seed=7)
        idx = torch.randint(0, 97, (2, 40), generator=torch.Generator().manual_seed(3))
        with torch.no_grad():
            outs[impl] = model(idx)
    assert outs["manual"].shape == (2, 40, 97)
    torch.testing.assert_close(outs["manual"], outs["functional"], rtol=1e-4, atol=1e-5)


def test_gpt2_rejects_unknown_impl():
    import model_inference as mi

    with pytest.raises(ValueError, match="xla"):
        mi.MultiHeadAttention(8, 8, 4, 0.0, 2, "xla")


def test_gpt2_accepts_the_reference_impl_types():
    """The reference's four-way dispatch (src/py/model_inference.py:68-90) constructs with every
    impl_type it names; "hip" is this build's copy-free variant of "cuda"."""
    import model_inference as mi

    for impl in ("manual", "functional", "triton", "cuda", "hip"):
        att = mi.MultiHeadAttention(8, 8, 4, 0.0, 2, impl)
        assert att.impl_type == impl


def test_decode_workspace_not_cached_under_graph_capture(monkeypatch):
    """A decode() call made during graph capture gets its own workspace; eager calls share the
    cached per-(device, stream) buffer.  Runs on CPU tensors with the capture state forced."""
    import custom_flash_attn as cfa

    dev = torch.device("cpu")
    monkeypatch.setattr(cfa, "_WORKSPACES", {})
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    a = cfa._decode_workspace(dev, 256)
    b = cfa._decode_workspace(dev, 256)
    assert a.numel() >= 256 and b.numel() >= 256
    assert a is not b  # a fresh buffer per captured call
    assert cfa._WORKSPACES == {}  # and none of them cached

    class _S:
        cuda_stream = 1234

    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    monkeypatch.setattr(torch.cuda, "current_stream", lambda d=None: _S())
    c = cfa._decode_workspace(dev, 256)
    d = cfa._decode_workspace(dev, 128)
    assert c is d and c.numel() >= 256
    assert c is not a and c is not b  # eager calls never get a captured call's buffer
    assert list(cfa._WORKSPACES) == [(dev, 1234)]
