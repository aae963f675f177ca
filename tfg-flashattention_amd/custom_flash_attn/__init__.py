"""custom_flash_attn - MI355X (gfx950) causal FlashAttention forward.

Drop-in for the reference's extension module of the same name
(src/cpp/torch_bind.cpp:21-49, built by src/py/setup.py:7-26), which the GPT-2
attention module calls as ``custom_flash_attn.forward(q, k, v)``
(src/py/model_inference.py:85-90).

The module layout differs from the reference on purpose: the compute lives in
``libtfgfa.so`` (hand-written HIP for gfx950 behind the C ABI of
``include/tfgfa.h``) and ``_C`` is a pybind11 binding over that ABI with no
libtorch in it.  This file does what torch_bind.cpp:13-31 does in C++: check
the tensors, allocate O with ``torch.empty_like`` and launch on the caller's
current stream.  There is no CPU or PyTorch fallback: if the native library is
missing, importing this package raises.
"""
from __future__ import annotations

import math
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))

try:
    from . import _C  # noqa: F401  (loads libtfgfa.so through its rpath)
except ImportError as exc:  # pragma: no cover - exercised only on a broken build
    raise ImportError(
        "custom_flash_attn: native extension not built "
        f"({exc}); run `make -C tfg-flashattention_amd/csrc` or __graft_entry__.build()"
    ) from exc

__all__ = ["forward", "forward_lse", "attention", "flash_attn_forward", "decode", "device_info",
           "HEAD_DIM", "MAX_HEAD_DIM", "library_path"]

HEAD_DIM = 64  # the head dimension of forward() (common_types.hpp:33 fixes K = 64 too)
MAX_HEAD_DIM = 128  # attention() / flash_attn_forward(): any head dim up to 128
_DTYPES = {torch.bfloat16: 0, torch.float16: 1}


def library_path() -> str:
    """Absolute path of the HIP shared library this package launches."""
    return os.path.join(_HERE, "libtfgfa.so")


def _check_input(x: torch.Tensor, name: str) -> None:
    # Same order and text as CHECK_CUDA / CHECK_CONTIGUOUS (torch_bind.cpp:13-19).
    if not x.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA tensor")
    if not x.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")


def _validate(Q: torch.Tensor, K_mat: torch.Tensor, V: torch.Tensor) -> None:
    _check_input(Q, "Q")
    _check_input(K_mat, "K_mat")
    _check_input(V, "V")
    if Q.dtype != torch.bfloat16:  # torch_bind.cpp:33-42 dispatches on Q's dtype only
        raise RuntimeError("Unsupported tensor dtype. Use bfloat16.")
    # Checks the reference leaves out (its kernel silently assumes them).
    if K_mat.dtype != torch.bfloat16 or V.dtype != torch.bfloat16:
        raise RuntimeError("Unsupported tensor dtype. Use bfloat16.")
    if Q.dim() != 4:
        raise RuntimeError(f"Q must be 4-D (batch, heads, seq_len, head_dim), got shape {tuple(Q.shape)}")
    if K_mat.shape != Q.shape or V.shape != Q.shape:
        raise RuntimeError(
            f"Q, K_mat and V must have the same shape, got {tuple(Q.shape)}, "
            f"{tuple(K_mat.shape)}, {tuple(V.shape)}"
        )
    if K_mat.device != Q.device or V.device != Q.device:
        raise RuntimeError("Q, K_mat and V must be on the same device")
    if Q.shape[3] != HEAD_DIM:
        raise RuntimeError(f"head_dim must be {HEAD_DIM}, got {Q.shape[3]}")


def _launch(Q, K_mat, V, O, lse, softmax_scale: float, causal: bool) -> None:
    B, H, N, D = Q.shape
    with torch.cuda.device(Q.device):
        stream = torch.cuda.current_stream(Q.device).cuda_stream
        _C.fwd(
            Q.data_ptr(), K_mat.data_ptr(), V.data_ptr(), O.data_ptr(),
            0 if lse is None else lse.data_ptr(),
            B, H, N, D, float(softmax_scale), bool(causal), stream,
        )


def forward(Q: torch.Tensor, K_mat: torch.Tensor, V: torch.Tensor, /) -> torch.Tensor:
    """Causal attention forward, ``softmax(Q K^T / sqrt(d)) V`` per (batch, head).

    Same call as the reference's ``custom_flash_attn.forward`` (torch_bind.cpp:21-45):
    positional Q, K_mat, V, each a contiguous bf16 CUDA(HIP) tensor of shape
    (B, H, N, 64); returns a new O of the same shape and dtype.  Errors raise
    RuntimeError with the reference's messages for device, contiguity and dtype.
    """
    _validate(Q, K_mat, V)
    O = torch.empty_like(Q)
    _launch(Q, K_mat, V, O, None, 1.0 / math.sqrt(Q.shape[3]), True)
    return O


def forward_lse(Q: torch.Tensor, K_mat: torch.Tensor, V: torch.Tensor, /,
                softmax_scale: float | None = None, causal: bool = True):
    """Like :func:`forward`, also returning the natural-log log-sum-exp.

    Returns ``(O, LSE)`` with LSE of shape (B, H, N), float32:
    ``LSE[b,h,i] = log(sum_{j<=i} exp(scale * q_i . k_j))`` - the ``lse_i`` of
    src/py/triton_implementation.py:153-154.  ``softmax_scale`` defaults to
    1/sqrt(head_dim) as in triton_implementation.py:197; ``causal=False`` drops the
    mask (all keys attend).
    """
    _validate(Q, K_mat, V)
    scale = (1.0 / math.sqrt(Q.shape[3])) if softmax_scale is None else float(softmax_scale)
    O = torch.empty_like(Q)
    lse = torch.empty(Q.shape[:3], dtype=torch.float32, device=Q.device)
    _launch(Q, K_mat, V, O, lse, scale, causal)
    return O, lse


def _check_view(x, name: str, ref, rows_from=None) -> None:
    """A (B, H, N, D) view: CUDA, fp16/bf16 like ``ref``, same B, H, D (and N as
    ``rows_from``, when given) and device, last dimension dense, D <= 128."""
    if not x.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA tensor")
    if x.dtype not in _DTYPES:
        raise RuntimeError("Unsupported tensor dtype. Use bfloat16 or float16.")
    if x.dim() != 4:
        raise RuntimeError(f"{name} must be 4-D (batch, heads, seq_len, head_dim), got shape {tuple(x.shape)}")
    if ref is not None:
        if x.dtype != ref.dtype:
            raise RuntimeError(f"{name} must have dtype {ref.dtype}, got {x.dtype}")
        want = (ref.shape[0], ref.shape[1], (rows_from if rows_from is not None else x).shape[2], ref.shape[3])
        if tuple(x.shape) != tuple(want):
            raise RuntimeError(f"{name} must have shape {tuple(want)}, got {tuple(x.shape)}")
        if x.device != ref.device:
            raise RuntimeError(f"{name} must be on {ref.device}, got {x.device}")
    if not 1 <= x.shape[3] <= MAX_HEAD_DIM:
        raise RuntimeError(f"head_dim must be in [1, {MAX_HEAD_DIM}], got {x.shape[3]}")
    if x.stride(3) != 1 and x.shape[3] > 1:
        raise RuntimeError(f"{name} must be dense in its last dimension (stride 1), got strides {x.stride()}")


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, out: torch.Tensor | None = None,
              softmax_scale: float | None = None, causal: bool = True, return_lse: bool = False):
    """Attention forward over strided (B, H, N, D) views, with no copies.

    ``q``: (B, H, N_q, D); ``k``, ``v``: (B, H, N_k, D); bf16 or fp16 (all alike); D up to 128;
    any strides whose last dimension is dense, e.g. the ``x.view(B, N, H, D).transpose(1, 2)``
    projections of a GPT-2 block (src/py/model_inference.py:64-66), which the reference's caller
    copies with ``.contiguous()`` first (:86-90).  ``out``, if given, is a (B, H, N_q, D) view of
    q's dtype the result is written into - pass ``buf.transpose(1, 2)`` of a (B, N, H, D) buffer
    and the (B, N, H*D) context needs no transposing copy (:92).  ``causal`` masks top-left
    aligned, as the reference's Triton kernel does (src/py/triton_implementation.py:127): query
    i sees keys j <= i.  Batch, head and row strides must be non-negative multiples of 8
    elements with row stride >= D and data 16-byte aligned; other layouts raise RuntimeError
    from the C ABI.  A head dim that is not a multiple of 8 is zero-padded to one (a copy of
    q, k, v), which leaves the scores unchanged.  Returns ``out`` (a new contiguous tensor
    when none is given), or ``(out, lse)`` with ``return_lse=True`` (lse contiguous
    (B, H, N_q) float32, natural log).
    """
    _check_view(q, "q", None)
    _check_view(k, "k", q)
    _check_view(v, "v", q, rows_from=k)
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    else:
        _check_view(out, "out", q, rows_from=q)
    B, H, Nq, D = q.shape
    Nk = k.shape[2]
    scale = (1.0 / math.sqrt(D)) if softmax_scale is None else float(softmax_scale)
    lse = torch.empty((B, H, Nq), dtype=torch.float32, device=q.device) if return_lse else None
    if D % 8:
        pad = 8 - D % 8
        qp, kp, vp = (torch.nn.functional.pad(t, (0, pad)) for t in (q, k, v))
        op = torch.empty(qp.shape, dtype=q.dtype, device=q.device)
        _launch_general(qp, kp, vp, op, lse, scale, causal)
        out.copy_(op[..., :D])
    else:
        _launch_general(q, k, v, out, lse, scale, causal)
    return (out, lse) if return_lse else out


def _launch_general(q, k, v, out, lse, scale, causal):
    B, H, Nq, D = q.shape
    with torch.cuda.device(q.device):
        stream = torch.cuda.current_stream(q.device).cuda_stream
        _C.fwd_general(
            q.data_ptr(), q.stride(), k.data_ptr(), k.stride(), v.data_ptr(), v.stride(),
            out.data_ptr(), out.stride(), 0 if lse is None else lse.data_ptr(),
            B, H, Nq, k.shape[2], D, _DTYPES[q.dtype], scale, bool(causal), stream,
        )


def flash_attn_forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, softmax_scale=None):
    """Drop-in for the reference's Triton wrapper ``_flash_attn_forward(q, k, v, softmax_scale)``
    (src/py/triton_implementation.py:184-241): causal attention of q (B, H, N_q, d) over k, v
    (B, H, N_k, d), d <= 128, fp16 or bf16, scale ``softmax_scale or 1/sqrt(d)``; returns a new
    O like q.  Argument errors are AssertionErrors with the wrapper's messages (:188-196).
    """
    batch, nheads, seqlen_q, d = q.shape
    _, _, seqlen_k, _ = k.shape
    assert k.shape == (batch, nheads, seqlen_k, d)
    assert v.shape == (batch, nheads, seqlen_k, d)
    assert d <= 128, "Flash Attention only supports head dimensions up to 128"
    assert q.dtype == k.dtype == v.dtype, "All tensors must have the same type"
    assert q.dtype in [torch.float16, torch.bfloat16], "Only supported types are fp16 and bf16"
    softmax_scale = softmax_scale or 1.0 / math.sqrt(d)
    o = torch.empty_like(q)
    return attention(q, k, v, out=o, softmax_scale=softmax_scale, causal=True)


def _check_vec(x, name: str, B: int, H: int, D: int, dtype, dev) -> None:
    if not x.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA tensor")
    if x.dtype != dtype:
        raise RuntimeError(f"{name} must have dtype {dtype}, got {x.dtype}")
    if tuple(x.shape) != (B, H, D):
        raise RuntimeError(f"{name} must have shape {(B, H, D)}, got {tuple(x.shape)}")
    if x.device != dev:
        raise RuntimeError(f"{name} must be on {dev}, got {x.device}")
    if x.stride(2) != 1:
        raise RuntimeError(f"{name} must be dense in its last dimension (stride 1), got strides {x.stride()}")


def decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
           cache_seqlens: torch.Tensor | None = None, k_new: torch.Tensor | None = None,
           v_new: torch.Tensor | None = None, *, out: torch.Tensor | None = None,
           softmax_scale: float | None = None, return_lse: bool = False,
           workspace: torch.Tensor | None = None):
    """One decode step: attention of one new query per (batch, head) over a KV cache.

    ``q``: (B, H, D).  ``k_cache``, ``v_cache``: (B, H, N_max, D) views (any strides with a
    dense last dimension, e.g. (B, N_max, H, D) buffers transposed).  bf16 or fp16, all
    operands alike; D a multiple of 8 up to 128 (GPT-2: bf16, D = 64).
    ``cache_seqlens``: int32 (B,) on the device, the number of valid cached rows per batch
    row (``None``: all N_max rows).  With ``k_new``/``v_new`` ((B, H, D)) the new token is
    written into cache row ``cache_seqlens[b]`` first and attended too; the caller advances
    ``cache_seqlens`` afterwards.  Returns ``out`` ((B, H, D), new if not given), or
    ``(out, lse)`` with ``return_lse=True`` (lse (B, H) float32, natural log).  The result
    equals the last row of the causal forward over the first L tokens - what the reference's
    generate() recomputes from scratch for every token (src/py/model_inference.py:199-228).
    A length that does not fit the cache yields NaN for that batch row (checked on the device).
    ``workspace``: optional uint8 device buffer for split-sequence work (per-head arrival words,
    then partials; no initialisation needed: each call installs its own random tag in the
    words and leaves them at zero; an empty buffer runs each head as one workgroup); when
    absent, a buffer of
    ``_C.decode_workspace_size(B, H, N_max, D)`` bytes is kept per device and stream and reused
    by eager calls.  A call made while the current stream is being captured into a graph gets
    a buffer of its own instead (allocated in the capture, never cached).
    """
    for t, n in ((k_cache, "k_cache"), (v_cache, "v_cache")):
        if not t.is_cuda:
            raise RuntimeError(f"{n} must be a CUDA tensor")
        if t.dtype not in _DTYPES:
            raise RuntimeError("Unsupported tensor dtype. Use bfloat16 or float16.")
        if t.dim() != 4:
            raise RuntimeError(f"{n} must be (B, H, N_max, D), got {tuple(t.shape)}")
        if t.stride(3) != 1:
            raise RuntimeError(f"{n} must be dense in its last dimension (stride 1), got strides {t.stride()}")
    B, H, N_max, D = k_cache.shape
    if not (8 <= D <= MAX_HEAD_DIM and D % 8 == 0):
        raise RuntimeError(f"head_dim must be a multiple of 8 in [8, {MAX_HEAD_DIM}], got {D}")
    if v_cache.dtype != k_cache.dtype:
        raise RuntimeError(f"v_cache must have dtype {k_cache.dtype}, got {v_cache.dtype}")
    if v_cache.shape != k_cache.shape:
        raise RuntimeError(f"v_cache must have shape {tuple(k_cache.shape)}, got {tuple(v_cache.shape)}")
    dev, dtype = k_cache.device, k_cache.dtype
    if v_cache.device != dev:
        raise RuntimeError(f"v_cache must be on {dev}, got {v_cache.device}")
    _check_vec(q, "q", B, H, D, dtype, dev)
    if (k_new is None) != (v_new is None):
        raise RuntimeError("k_new and v_new must be given together")
    if k_new is not None:
        _check_vec(k_new, "k_new", B, H, D, dtype, dev)
        _check_vec(v_new, "v_new", B, H, D, dtype, dev)
        if cache_seqlens is None:
            raise RuntimeError("appending k_new/v_new needs cache_seqlens")
    if cache_seqlens is not None:
        if cache_seqlens.dtype != torch.int32 or tuple(cache_seqlens.shape) != (B,):
            raise RuntimeError(f"cache_seqlens must be int32 of shape ({B},)")
        if cache_seqlens.device != dev or not cache_seqlens.is_contiguous():
            raise RuntimeError(f"cache_seqlens must be a contiguous tensor on {dev}")
    if out is None:
        out = torch.empty((B, H, D), dtype=dtype, device=dev)
    else:
        _check_vec(out, "out", B, H, D, dtype, dev)
    scale = (1.0 / math.sqrt(D)) if softmax_scale is None else float(softmax_scale)
    lse = torch.empty((B, H), dtype=torch.float32, device=dev) if return_lse else None
    if workspace is None:
        workspace = _decode_workspace(dev, _C.decode_workspace_size(B, H, N_max, D))
    elif not workspace.is_cuda or workspace.device != dev or not workspace.is_contiguous():
        raise RuntimeError(f"workspace must be a contiguous tensor on {dev}")
    zero3 = (0, 0, 0)
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        _C.decode_general(
            q.data_ptr(), q.stride(), k_cache.data_ptr(), k_cache.stride(),
            v_cache.data_ptr(), v_cache.stride(),
            0 if k_new is None else k_new.data_ptr(), zero3 if k_new is None else k_new.stride(),
            0 if v_new is None else v_new.data_ptr(), zero3 if v_new is None else v_new.stride(),
            0 if cache_seqlens is None else cache_seqlens.data_ptr(),
            out.data_ptr(), out.stride(), 0 if lse is None else lse.data_ptr(),
            B, H, N_max, D, _DTYPES[dtype], scale,
            workspace.data_ptr() if workspace.numel() else 0,
            workspace.numel() * workspace.element_size(), stream,
        )
    return (out, lse) if return_lse else out


_WORKSPACES: dict = {}


def _decode_workspace(dev, nbytes: int) -> torch.Tensor:
    """A decode workspace of at least ``nbytes`` for (device, current stream), reused across
    eager calls: it holds only the arrival words and partials of one call, and calls on one
    stream do not overlap.

    Under graph capture a fresh buffer is returned and not cached.  A cached one would be
    shared by the graph's replays and by later eager calls on the capture stream (a replay
    racing an eager call on another stream would mix their partials), and a graph would keep
    using the pool block of an entry that a later, larger request replaced.  The fresh buffer
    comes from the capture's memory pool and is released after the call like any temporary of
    a captured region: the replay uses it in stream order.  Later work of the same graph may
    reuse that memory; the next replay's call still needs no initialisation (its own tag
    replaces whatever the arrival words then hold)."""
    if torch.cuda.is_current_stream_capturing():
        return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    key = (dev, torch.cuda.current_stream(dev).cuda_stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
        _WORKSPACES[key] = ws
    return ws


def device_info() -> dict:
    """CU count, shader clock (MHz) and gfx arch of the current device (cached per device)."""
    return _C.device_info()
