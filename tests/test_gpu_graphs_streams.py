"""HIP graph capture and concurrent streams (GPU box only).

The entry points allocate nothing and clear no memory with memsets, so a caller may capture
them in a HIP graph.  Each graph below is replayed several times with eager work and
synchronisations in between, and every replay is checked bitwise against the eager result of
the same call (a replay that read stale or partial state would differ); the decode step is
replayed both as one kernel and as the split kernel plus its merge kernel.  Other tests run
different forward and decode problems on two streams at once.
"""
import sys

import pytest
import torch

import custom_flash_attn

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _randn(shape, seed, sigma=1.0, dtype=torch.bfloat16):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(shape, device=DEV, generator=g) * sigma).to(dtype)


def _same(a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_forward_and_strided_calls_replay_from_a_graph():
    B, H, N, D = 2, 4, 300, 64
    q, k, v = _randn((B, H, N, D), 1, 3.0), _randn((B, H, N, D), 2, 3.0), _randn((B, H, N, D), 3)
    x = _randn((B, N, 3, H, 96), 4, 2.0, torch.float16)
    qs, ks, vs = (x[:, :, i].transpose(1, 2) for i in range(3))
    ref_o, ref_lse = custom_flash_attn.forward_lse(q, k, v)
    ref_s = custom_flash_attn.attention(qs, ks, vs)
    out_o = torch.empty_like(ref_o)
    out_lse = torch.empty_like(ref_lse)
    out_s = torch.empty(ref_s.shape, dtype=ref_s.dtype, device=DEV)
    torch.cuda.synchronize()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            o, lse = custom_flash_attn.forward_lse(q, k, v)
            out_o.copy_(o)
            out_lse.copy_(lse)
            custom_flash_attn.attention(qs, ks, vs, out=out_s)
    torch.cuda.current_stream().wait_stream(side)
    for rep in range(4):
        out_o.fill_(0)
        out_lse.fill_(0)
        out_s.fill_(0)
        _ = (q.float() @ k.float().transpose(-1, -2).contiguous()).sum()  # eager work in between
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        _say(f"forward graph replay {rep}")
        assert _same(out_o, ref_o) and torch.equal(out_lse, ref_lse), f"replay {rep}: forward differs"
        assert torch.equal(out_s, ref_s), f"replay {rep}: strided fp16 differs"


def test_decode_steps_replay_from_a_graph():
    """A decode step captured once and replayed as the cache grows: the lengths live in device
    memory, so each replay appends at the current length and attends over it."""
    B, H, N_max, D = 2, 3, 256, 64
    kc, vc = torch.zeros(B, H, N_max, D, dtype=torch.bfloat16, device=DEV), torch.zeros(
        B, H, N_max, D, dtype=torch.bfloat16, device=DEV)
    kc_ref, vc_ref = kc.clone(), vc.clone()
    prefix = 100
    kc[:, :, :prefix] = _randn((B, H, prefix, D), 10, 3.0)
    vc[:, :, :prefix] = _randn((B, H, prefix, D), 11)
    kc_ref.copy_(kc)
    vc_ref.copy_(vc)
    seqlens = torch.full((B,), prefix, dtype=torch.int32, device=DEV)
    seqlens_ref = seqlens.clone()
    steps = 5
    qs = [_randn((B, H, D), 20 + t, 3.0) for t in range(steps)]
    kns = [_randn((B, H, D), 40 + t, 3.0) for t in range(steps)]
    vns = [_randn((B, H, D), 60 + t) for t in range(steps)]
    q_in, kn_in, vn_in = (torch.empty_like(qs[0]) for _ in range(3))
    out = torch.empty(B, H, D, dtype=torch.bfloat16, device=DEV)
    ws = torch.empty(custom_flash_attn._C.decode_workspace_bytes(B, H, N_max), dtype=torch.uint8, device=DEV)
    torch.cuda.synchronize()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            custom_flash_attn.decode(q_in, kc, vc, seqlens, kn_in, vn_in, out=out, workspace=ws)
            seqlens.add_(1)
    torch.cuda.current_stream().wait_stream(side)
    # Capturing does not run the work: the cache and lengths are untouched.
    torch.cuda.synchronize()
    assert torch.equal(seqlens, seqlens_ref) and torch.equal(kc, kc_ref)
    for t in range(steps):
        q_in.copy_(qs[t])
        kn_in.copy_(kns[t])
        vn_in.copy_(vns[t])
        torch.cuda.synchronize()
        graph.replay()
        ref = custom_flash_attn.decode(qs[t], kc_ref, vc_ref, seqlens_ref, kns[t], vns[t], workspace=ws.clone())
        seqlens_ref.add_(1)
        torch.cuda.synchronize()
        _say(f"decode graph replay {t}: length {prefix + t + 1}")
        assert torch.equal(seqlens, seqlens_ref)
        assert _same(kc, kc_ref) and _same(vc, vc_ref), f"step {t}: cache differs"
        assert _same(out, ref), f"step {t}: output differs"


def test_split_decode_steps_replay_from_a_graph():
    """Small B*H over a long cache: each step splits every head over several workgroups, the
    last to arrive merging them (arrival words in the workspace, reset to zero by each step).
    The step replays from one graph as the cache grows; every replay equals the eager step."""
    B, H, N_max, D = 1, 4, 4096, 64
    kc = torch.zeros(B, H, N_max, D, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    prefix = 3000
    kc[:, :, :prefix] = _randn((B, H, prefix, D), 90, 3.0)
    vc[:, :, :prefix] = _randn((B, H, prefix, D), 91)
    kc_ref, vc_ref = kc.clone(), vc.clone()
    seqlens = torch.full((B,), prefix, dtype=torch.int32, device=DEV)
    seqlens_ref = seqlens.clone()
    q_in, kn_in, vn_in = (torch.empty(B, H, D, dtype=torch.bfloat16, device=DEV) for _ in range(3))
    out = torch.empty(B, H, D, dtype=torch.bfloat16, device=DEV)
    lse = torch.empty(B, H, dtype=torch.float32, device=DEV)
    ws = torch.empty(custom_flash_attn._C.decode_workspace_bytes(B, H, N_max), dtype=torch.uint8, device=DEV)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            o, l = custom_flash_attn.decode(q_in, kc, vc, seqlens, kn_in, vn_in, out=out, workspace=ws,
                                            return_lse=True)
            lse.copy_(l)
            seqlens.add_(1)
    torch.cuda.current_stream().wait_stream(side)
    for t in range(4):
        q, kn, vn = _randn((B, H, D), 100 + t, 3.0), _randn((B, H, D), 110 + t, 3.0), _randn((B, H, D), 120 + t)
        q_in.copy_(q)
        kn_in.copy_(kn)
        vn_in.copy_(vn)
        _ = (q.float() * 2).sum()  # eager work in between
        torch.cuda.synchronize()
        graph.replay()
        ref, ref_lse = custom_flash_attn.decode(q, kc_ref, vc_ref, seqlens_ref, kn, vn, return_lse=True,
                                                workspace=torch.empty_like(ws))
        seqlens_ref.add_(1)
        torch.cuda.synchronize()
        _say(f"split decode graph replay {t}: length {prefix + t + 1}")
        assert torch.equal(seqlens, seqlens_ref)
        assert _same(kc, kc_ref) and _same(vc, vc_ref), f"step {t}: cache differs"
        assert _same(out, ref) and torch.equal(lse, ref_lse), f"step {t}: output differs"


def test_decode_on_two_streams_at_once():
    """Decode calls with their own workspaces on two streams at once (split and unsplit
    shapes) give the results of the same calls run one after the other."""
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    cases = []
    for i, (B, H, N, D, dt) in enumerate([(1, 8, 4096, 64, torch.bfloat16), (8, 25, 1024, 64, torch.bfloat16),
                                          (1, 16, 2048, 128, torch.float16)]):
        kc = _randn((B, H, N, D), 130 + i, 3.0, dt)
        vc = _randn((B, H, N, D), 140 + i, 1.0, dt)
        q = _randn((B, H, D), 150 + i, 3.0, dt)
        sl = torch.full((B,), N - 7, dtype=torch.int32, device=DEV)
        ws = torch.empty(custom_flash_attn._C.decode_workspace_size(B, H, N, D), dtype=torch.uint8, device=DEV)
        cases.append((q, kc, vc, sl, ws))
    refs = [custom_flash_attn.decode(q, kc, vc, sl, workspace=ws) for q, kc, vc, sl, ws in cases]
    torch.cuda.synchronize()
    ws2 = [torch.empty_like(c[4]) for c in cases]
    outs = []
    for rep in range(3):
        for i, (q, kc, vc, sl, ws) in enumerate(cases):
            with torch.cuda.stream(s1 if (i + rep) % 2 == 0 else s2):
                outs.append((i, custom_flash_attn.decode(q, kc, vc, sl, workspace=ws if rep % 2 == 0 else ws2[i])))
    torch.cuda.synchronize()
    for i, o in outs:
        assert torch.equal(o.view(torch.int16), refs[i].view(torch.int16)), f"case {i} differs"


def test_two_streams_at_once():
    B, H, N = 4, 8, 700
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    q1, k1, v1 = (_randn((B, H, N, 64), 70 + i, 3.0) for i in range(3))
    q2, k2, v2 = (_randn((B, H, N // 2, 128), 80 + i, 2.0, torch.float16) for i in range(3))
    ref1 = custom_flash_attn.forward(q1, k1, v1)
    ref2 = custom_flash_attn.attention(q2, k2, v2, causal=False)
    torch.cuda.synchronize()
    outs1, outs2 = [], []
    for _ in range(5):
        with torch.cuda.stream(s1):
            outs1.append(custom_flash_attn.forward(q1, k1, v1))
        with torch.cuda.stream(s2):
            outs2.append(custom_flash_attn.attention(q2, k2, v2, causal=False))
    torch.cuda.synchronize()
    for a, b in zip(outs1, outs2):
        assert _same(a, ref1)
        assert torch.equal(b, ref2)


def test_decode_captured_without_workspace_replays():
    """decode() captured with no workspace argument takes a fresh buffer from the capture's
    memory pool, released after the call; a later allocation in the same graph (here a
    temporary that a kernel fills with 1.0) may reuse that memory, so each replay's decode
    starts on arrival words that hold whatever the previous replay left there.  Every replay,
    with eager decode() calls on the same stream in between, is bitwise the eager result."""
    B, H, N, D = 1, 4, 4096, 64  # split heads (B*H far below the CU count)
    q = _randn((B, H, D), 1, 2.0)
    kc, vc = _randn((B, H, N, D), 2, 2.0), _randn((B, H, N, D), 3)
    lens = torch.full((B,), N, dtype=torch.int32, device=DEV)
    ref = custom_flash_attn.decode(q, kc, vc, lens, return_lse=True)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        o, lse = custom_flash_attn.decode(q, kc, vc, lens, return_lse=True)
        tmp = torch.empty(1 << 20, device=DEV, dtype=torch.float32)
        tmp.fill_(1.0)
    for rep in range(5):
        g.replay()
        eager_o, eager_l = custom_flash_attn.decode(q, kc, vc, lens, return_lse=True)
        torch.cuda.synchronize()
        assert _same(o, ref[0]) and torch.equal(lse, ref[1]), f"replay {rep}"
        assert _same(eager_o, ref[0]) and torch.equal(eager_l, ref[1]), f"eager after replay {rep}"
    _say("decode captured without a workspace: 5 replays bitwise equal to eager")
