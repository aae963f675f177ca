"""Cached GPT-2 decoding (prefill kernel + decode kernel with a KV cache) against the
reference's full-recompute path (GPU box only, except the argument checks).

The reference's generate() re-runs the whole prefix per token (src/py/model_inference.py:
199-228); the logits it samples from are those of the last position of a full forward.  Here
the same positions are computed from a KV cache: a prefill over the prompt, then one decode
step per token, teacher-forced along one fixed token sequence.  Gate: against the GPU full
forward ("hip" attention) relative L2 <= 1e-2 and argmax agreement >= 0.98; against the CPU
fp32 "manual" forward relative L2 <= 2e-2 (the bf16 autocast projections dominate both).
"""
import sys

import pytest
import torch

import model_inference as mi

SEED_W = 77


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _small_cfg(impl):
    cfg = dict(mi.GPT_CONFIG_124M)
    cfg.update({"emb_dim": 512, "n_layers": 4, "n_heads": 8, "vocab_size": 1000,
                "context_length": 256, "drop_rate": 0.0, "qkv_bias": True, "impl_type": impl})
    return cfg


def _rel(x, ref):
    x, ref = x.double(), ref.double()
    return ((x - ref).norm() / ref.norm()).item()


def test_generate_cached_rejects_overlong_requests():
    cfg = _small_cfg("manual")
    model = mi.GPTModel(cfg).eval()
    with pytest.raises(ValueError, match="exceeds context_size"):
        mi.generate_cached(model, torch.zeros(1, 250, dtype=torch.long), 10, 256)


def test_reference_generate_runs_on_cpu():
    cfg = _small_cfg("manual")
    cfg.update({"emb_dim": 128, "n_heads": 2, "n_layers": 2})
    torch.manual_seed(0)
    model = mi.GPTModel(cfg).eval()
    mi.init_gpt2_weights(model, 3)
    idx = torch.randint(0, 1000, (2, 7), generator=torch.Generator().manual_seed(1))
    out = mi.generate(model, idx, 5, 256, temperature=0.0)
    assert out.shape == (2, 12) and torch.equal(out[:, :7], idx)
    # Greedy tokens are the argmax of the full forward's last position at every step.
    with torch.no_grad():
        for t in range(7, 12):
            assert torch.equal(model(out[:, :t])[:, -1].argmax(-1), out[:, t])
    # eos_id (model_inference.py:224-225), B = 1: stop before the first sampled eos_id.
    one = out[:1]
    eos = one[0, 9].item()
    first = one[0, 7:].tolist().index(eos)
    assert torch.equal(mi.generate(model, idx[:1], 5, 256, temperature=0.0, eos_id=eos), one[:, :7 + first])


@pytest.mark.gpu
def test_cached_decode_logits_match_full_forward():
    torch.manual_seed(0)
    cfg = _small_cfg("manual")
    model = mi.GPTModel(cfg).eval()
    mi.init_gpt2_weights(model, SEED_W)
    B, P, T = 2, 40, 30                          # prompt 40 tokens, 30 decode steps
    seq = torch.randint(0, cfg["vocab_size"], (B, P + T), generator=torch.Generator().manual_seed(5))
    _say("cached GPT-2: CPU fp32 manual forward")
    with torch.no_grad():
        ref_cpu = model(seq)[:, P - 1:P + T - 1].float()
    gpu = model.to("cuda:0")
    for blk in gpu.trf_blocks:
        blk.att.impl_type = "hip"
    seq_d = seq.to("cuda:0")
    _say("cached GPT-2: full forward on the GPU")
    with torch.no_grad():
        full = gpu(seq_d)[:, P - 1:P + T - 1].float()
        cfg_c = {"n_heads": 8, "emb_dim": 512, "n_layers": 4}
        cache = mi.KVCache(cfg_c, B, P + T, "cuda:0")
        steps = [gpu(seq_d[:, :P], kv_cache=cache)[:, -1].float()]
        for t in range(P, P + T - 1):
            steps.append(gpu(seq_d[:, t:t + 1], kv_cache=cache)[:, -1].float())
    torch.cuda.synchronize()
    cached = torch.stack(steps, dim=1)
    assert cache.length == P + T - 1
    assert torch.equal(cache.seqlens.cpu(), torch.full((B,), P + T - 1, dtype=torch.int32))
    r_full = _rel(cached.cpu(), full.cpu())
    r_cpu = _rel(cached.cpu(), ref_cpu)
    r_full_cpu = _rel(full.cpu(), ref_cpu)
    agree = (cached.argmax(-1) == full.argmax(-1)).double().mean().item()
    _say(f"cached vs full GPU: rel_l2={r_full:.3e} argmax_agree={agree:.4f}; cached vs CPU fp32: "
         f"rel_l2={r_cpu:.3e} (full GPU vs CPU: {r_full_cpu:.3e})")
    assert r_full <= 1e-2 and agree >= 0.98
    assert r_cpu <= 2e-2
    # The cache holds the K/V the full forward computes (bf16 projections; the prefill and the
    # one-token steps may round differently in the GEMM, hence a tolerance).
    blk0 = gpu.trf_blocks[0]
    with torch.no_grad():
        x = blk0.norm1(gpu.tok_emb(seq_d[:, :P + T - 1]) + gpu.pos_emb(torch.arange(P + T - 1, device="cuda:0")))
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            k0 = blk0.att.W_key(x).view(B, P + T - 1, 8, 64).transpose(1, 2)
    torch.testing.assert_close(cache.k[0][:, :, :P + T - 1].float(), k0.float(), rtol=1e-2, atol=1e-2)


@pytest.mark.gpu
def test_generate_cached_samples_and_advances():
    torch.manual_seed(0)
    cfg = _small_cfg("hip")
    model = mi.GPTModel(cfg).eval().to("cuda:0")
    mi.init_gpt2_weights(model, SEED_W)
    idx = torch.randint(0, cfg["vocab_size"], (3, 12), device="cuda:0")
    torch.manual_seed(123)
    out = mi.generate_cached(model, idx, 20, 256, temperature=1.0, top_k=50)
    assert out.shape == (3, 32) and torch.equal(out[:, :12], idx)
    assert int(out.min()) >= 0 and int(out.max()) < cfg["vocab_size"]
    greedy = mi.generate_cached(model, idx, 8, 256, temperature=0.0)
    # Greedy cached tokens against the full forward's argmax along the same sequence; a step
    # whose top two full-forward logits are within 1e-2 may legitimately differ.
    with torch.no_grad():
        full = model(greedy[:, :-1])[:, 11:].float()
    top2 = full.topk(2, dim=-1).values
    decided = (top2[..., 0] - top2[..., 1]) > 1e-2
    same = full.argmax(-1) == greedy[:, 12:]
    assert bool(same[decided].all())


def test_top_k_filter_keeps_k_tokens_per_row():
    """Batch rows are filtered by their own k-th largest logit (the reference's (B,) threshold
    only broadcasts for B = 1)."""
    logits = torch.tensor([[0.0, 5.0, 1.0, 3.0], [4.0, -1.0, 2.0, 0.5]])
    torch.manual_seed(0)
    for _ in range(50):
        nxt = mi._next_token(logits, 1.0, 2)
        assert nxt[0, 0].item() in (1, 3) and nxt[1, 0].item() in (0, 2)
    assert mi._next_token(logits, 0.0, 2).flatten().tolist() == [1, 0]


@pytest.mark.gpu
def test_graphed_decode_steps_match_eager_cached_steps():
    """Decode steps replayed from a HIP graph give the eager cached steps' logits bitwise, step
    after step, with eager work on the stream between replays; greedy generation through the
    graph equals greedy generate_cached."""
    torch.manual_seed(0)
    cfg = _small_cfg("hip")
    model = mi.GPTModel(cfg).eval().to("cuda:0")
    mi.init_gpt2_weights(model, SEED_W)
    B, P, T = 2, 13, 9
    seq = torch.randint(0, cfg["vocab_size"], (B, P + T), generator=torch.Generator().manual_seed(8)).to("cuda:0")
    cfg_c = {"n_heads": 8, "emb_dim": 512, "n_layers": 4}
    eager_cache = mi.KVCache(cfg_c, B, P + T, "cuda:0")
    dec = mi.GraphedDecoder(model, B, P + T, "cuda:0")
    with torch.no_grad():
        le = model(seq[:, :P], kv_cache=eager_cache)[:, -1].float()
        lg = dec.prefill(seq[:, :P]).float()
        assert torch.equal(le, lg)
        for t in range(P, P + T):
            le = model(seq[:, t:t + 1], kv_cache=eager_cache)[:, -1].float()
            _ = (torch.randn(64, 64, device="cuda:0") @ torch.randn(64, 64, device="cuda:0")).sum()
            lg = dec.step(seq[:, t:t + 1]).float()
            torch.cuda.synchronize()
            _say(f"graphed decode step {t}: max|d logits| = {(le - lg).abs().max().item():.3e}")
            assert torch.equal(le, lg), f"step {t}: graph replay differs from the eager step"
    assert dec.cache.length == P + T and torch.equal(dec.cache.seqlens.cpu(), torch.full((B,), P + T, dtype=torch.int32))
    idx = seq[:, :P]
    a = mi.generate_cached(model, idx, 8, 256, temperature=0.0)
    b = mi.generate_graphed(model, idx, 8, 256, temperature=0.0, decoder=dec)
    c = mi.generate_graphed(model, idx, 8, 256, temperature=0.0)
    assert torch.equal(a, b) and torch.equal(a, c)


@pytest.mark.gpu
def test_eos_id_stops_cached_and_graphed_generators_at_the_same_token():
    """eos_id (model_inference.py:224-225): the loop stops before appending the first sampled
    token equal to eos_id.  Greedy, B = 1: the cached and graph-replayed generators stop where
    a run without eos_id first produces that token, and return the same prefix; an eos_id never
    produced leaves the full length."""
    torch.manual_seed(0)
    cfg = _small_cfg("hip")
    model = mi.GPTModel(cfg).eval().to("cuda:0")
    mi.init_gpt2_weights(model, SEED_W)
    P, T = 10, 12
    idx = torch.randint(0, cfg["vocab_size"], (1, P), generator=torch.Generator().manual_seed(21)).to("cuda:0")
    full = mi.generate_cached(model, idx, T, 256, temperature=0.0)
    assert full.shape == (1, P + T)
    new = full[0, P:].tolist()
    eos = new[T // 2]
    first = new.index(eos)
    _say(f"greedy tokens {new}; eos_id {eos} first sampled at step {first}")
    expect = full[:, :P + first]
    a = mi.generate_cached(model, idx, T, 256, temperature=0.0, eos_id=eos)
    b = mi.generate_graphed(model, idx, T, 256, temperature=0.0, eos_id=eos)
    assert torch.equal(a, expect) and torch.equal(b, expect)
    absent = next(t for t in range(cfg["vocab_size"]) if t not in new)
    c = mi.generate_graphed(model, idx, T, 256, temperature=0.0, eos_id=absent)
    assert torch.equal(c, full)
