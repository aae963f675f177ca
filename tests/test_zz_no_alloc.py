"""tfgfa_decode_noalloc - the decode step with its split partials in the library's static
scratch instead of a caller's workspace - against tfgfa_decode with a full workspace, through
the C ABI (GPU box only).

Two calls in a row on the same GPU, the second smaller than the first, so the second runs on a
scratch still holding the first call's partials.  Named to be collected last: it passes alone in
a fresh process and after every other test.  Both shapes split their heads over several
workgroups (B * H well below the CU count), so the scratch is what carries the partials.
Results must be bitwise those of tfgfa_decode (the same split, the same merge) and within the
forward's tolerances of the fp64 oracle (decode_np).
"""
import ctypes
import sys

import numpy as np
import pytest
import torch

from oracle import decode_np

import custom_flash_attn

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
P = ctypes.c_void_p
S3, S4 = ctypes.c_int64 * 3, ctypes.c_int64 * 4
DT = {torch.bfloat16: 0, torch.float16: 1}


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def lib():
    L = ctypes.CDLL(custom_flash_attn.library_path())
    L.tfgfa_decode.restype = ctypes.c_int
    L.tfgfa_decode.argtypes = [P, P] * 5 + [P] * 4 + [ctypes.c_int] * 5 + [
        ctypes.c_float, P, ctypes.c_size_t, P]
    L.tfgfa_decode_noalloc.restype = ctypes.c_int
    L.tfgfa_decode_noalloc.argtypes = [P, P] * 5 + [P] * 4 + [ctypes.c_int] * 5 + [ctypes.c_float, P]
    L.tfgfa_decode_workspace_size.restype = ctypes.c_size_t
    L.tfgfa_decode_workspace_size.argtypes = [ctypes.c_int] * 4
    L.tfgfa_strerror.restype = ctypes.c_char_p
    return L


def _case(B, H, N, D, dtype, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = (torch.randn(B, H, D, device=DEV, generator=g) * 2).to(dtype)
    kc = (torch.randn(B, H, N, D, device=DEV, generator=g) * 2).to(dtype)
    vc = torch.randn(B, H, N, D, device=DEV, generator=g).to(dtype)
    lens = torch.tensor([N - 3 * b for b in range(B)], dtype=torch.int32, device=DEV)
    return q, kc, vc, lens


def _call(lib, fn, q, kc, vc, lens, ws=None):
    B, H, N, D = kc.shape
    o = torch.full((B, H, D), float("nan"), device=DEV, dtype=q.dtype)
    lse = torch.full((B, H), float("nan"), device=DEV, dtype=torch.float32)
    args = [q.data_ptr(), S3(*q.stride()), kc.data_ptr(), S4(*kc.stride()), vc.data_ptr(),
            S4(*vc.stride()), None, None, None, None, lens.data_ptr(), o.data_ptr(),
            S3(*o.stride()), lse.data_ptr(), B, H, N, D, DT[q.dtype], 1.0 / D ** 0.5]
    if fn == "tfgfa_decode":
        args += [ws.data_ptr(), ws.numel()]
    st = getattr(lib, fn)(*args, torch.cuda.current_stream().cuda_stream)
    assert st == 0, lib.tfgfa_strerror(st).decode()
    return o, lse


@pytest.mark.parametrize("first,second", [
    ((1, 16, 8192, 64, torch.bfloat16), (1, 8, 2048, 64, torch.bfloat16)),
    ((2, 8, 16384, 128, torch.float16), (1, 12, 4096, 96, torch.float16)),
])
def test_noalloc_matches_workspace_entry_point(lib, first, second):
    for n, (B, H, N, D, dtype) in enumerate((first, second)):
        _say(f"noalloc call {n + 1}: B={B} H={H} N={N} D={D} {dtype}")
        q, kc, vc, lens = _case(B, H, N, D, dtype, 100 * n + N + D)
        ws = torch.empty(lib.tfgfa_decode_workspace_size(B, H, N, D), dtype=torch.uint8, device=DEV)
        o_ws, l_ws = _call(lib, "tfgfa_decode", q, kc, vc, lens, ws)
        o_na, l_na = _call(lib, "tfgfa_decode_noalloc", q, kc, vc, lens)
        torch.cuda.synchronize()
        assert torch.equal(o_na.view(torch.int16), o_ws.view(torch.int16)), "O differs"
        assert torch.equal(l_na, l_ws), "LSE differs"
        o_ref, l_ref = decode_np(q.float().cpu().numpy(), kc.float().cpu().numpy(),
                                 vc.float().cpu().numpy(), lens.cpu().numpy(), 1.0 / D ** 0.5)
        d = np.abs(o_na.float().cpu().numpy() - o_ref)
        dl = np.abs(l_na.cpu().numpy() - l_ref)
        _say(f"  bitwise equal to tfgfa_decode; vs oracle max|dO|={d.max():.3e} "
             f"mean|dO|={d.mean():.3e} max|dLSE|={dl.max():.3e}")
        assert d.max() <= 2e-2 and d.mean() <= 2e-3 and dl.max() <= 1e-3


_CHILD = r"""
import ctypes, sys
sys.path[:0] = [sys.argv[1], sys.argv[2]]
import torch
import custom_flash_attn  # loads the library; no call into it before the capture below

P = ctypes.c_void_p
S3, S4 = ctypes.c_int64 * 3, ctypes.c_int64 * 4
L = ctypes.CDLL(custom_flash_attn.library_path())
L.tfgfa_decode.argtypes = [P, P] * 5 + [P] * 4 + [ctypes.c_int] * 5 + [ctypes.c_float, P, ctypes.c_size_t, P]
L.tfgfa_decode_noalloc.argtypes = [P, P] * 5 + [P] * 4 + [ctypes.c_int] * 5 + [ctypes.c_float, P]
L.tfgfa_decode_workspace_size.restype = ctypes.c_size_t
L.tfgfa_decode_workspace_size.argtypes = [ctypes.c_int] * 4
dev = "cuda:0"
B, H, N, D = 1, 8, 4096, 64
g = torch.Generator(device=dev).manual_seed(7)
q = (torch.randn(B, H, D, device=dev, generator=g) * 2).to(torch.bfloat16)
kc = (torch.randn(B, H, N, D, device=dev, generator=g) * 2).to(torch.bfloat16)
vc = torch.randn(B, H, N, D, device=dev, generator=g).to(torch.bfloat16)
lens = torch.full((B,), N - 5, dtype=torch.int32, device=dev)
ws = torch.empty(L.tfgfa_decode_workspace_size(B, H, N, D), dtype=torch.uint8, device=dev)
torch.cuda.synchronize()

def call(fn, o, lse, stream, ws=None):
    args = [q.data_ptr(), S3(*q.stride()), kc.data_ptr(), S4(*kc.stride()), vc.data_ptr(),
            S4(*vc.stride()), None, None, None, None, lens.data_ptr(), o.data_ptr(),
            S3(*o.stride()), lse.data_ptr(), B, H, N, D, 0, 1.0 / D ** 0.5]
    if ws is not None:
        args += [ws.data_ptr(), ws.numel()]
    st = fn(*args, stream)
    assert st == 0, f"status {st}"

o_g = torch.empty(B, H, D, device=dev, dtype=torch.bfloat16)
l_g = torch.empty(B, H, device=dev, dtype=torch.float32)
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):  # the library's first call of the process, during capture
    call(L.tfgfa_decode_noalloc, o_g, l_g, torch.cuda.current_stream().cuda_stream)
o_w, l_w = torch.empty_like(o_g), torch.empty_like(l_g)
o_e, l_e = torch.empty_like(o_g), torch.empty_like(l_g)
sh = torch.cuda.current_stream().cuda_stream
for rep in range(4):
    graph.replay()
    torch.cuda.synchronize()
    call(L.tfgfa_decode, o_w, l_w, sh, ws)
    torch.cuda.synchronize()
    assert torch.equal(o_g.view(torch.int16), o_w.view(torch.int16)), f"replay {rep}: O"
    assert torch.equal(l_g, l_w), f"replay {rep}: LSE"
    call(L.tfgfa_decode_noalloc, o_e, l_e, sh)  # eager noalloc between replays
    torch.cuda.synchronize()
    assert torch.equal(o_e.view(torch.int16), o_w.view(torch.int16)), f"eager {rep}: O"
print("__CHILD_OK__", flush=True)
"""


def test_first_noalloc_call_inside_graph_capture(tmp_path):
    """In a fresh process whose first call into the library is a tfgfa_decode_noalloc captured
    in a HIP graph (so the once-per-device device-property and scratch-symbol lookups run while
    the stream captures): four replays, with eager tfgfa_decode and noalloc calls in between,
    each bitwise equal to tfgfa_decode with a full workspace."""
    import os
    import subprocess

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    pkg = os.path.join(root, "tfg-flashattention_amd")
    _say("child process: first noalloc call during graph capture")
    r = subprocess.run([sys.executable, "-c", _CHILD, root, pkg], capture_output=True, text=True,
                       timeout=240)
    _say(r.stdout[-2000:] + r.stderr[-2000:])
    assert r.returncode == 0 and "__CHILD_OK__" in r.stdout
