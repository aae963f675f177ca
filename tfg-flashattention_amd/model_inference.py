"""GPT-2 model whose attention can run on the MI355X kernel - the caller of the hot path.

Mirrors the reference's model classes (src/py/model_inference.py:39-190) with the same
names, constructor arguments and config keys, so code written against the reference's
``GPTModel(cfg)`` runs unchanged, and its token loop ``generate`` (:199-228).  Added:
``KVCache`` and ``generate_cached``, the same loop with a KV cache (prefill once, then one
decode-kernel step per token).  The reference's data loader, training helpers, tokenizer and
pretrained-weight download (model_inference.py:23-37, :193-197, :229-376; gpt_download.py)
are not here.

``impl_type`` selects the attention implementation as at model_inference.py:68-90:
  * ``"manual"``     - the reference's explicit PyTorch path (:68-75);
  * ``"functional"`` - torch.nn.functional.scaled_dot_product_attention (:77-80);
  * ``"cuda"`` - custom_flash_attn.forward on ``.contiguous()`` copies of Q, K, V, as the
    reference's branch calls it (:85-90);
  * ``"hip"`` - the same gfx950 kernel through custom_flash_attn.attention, which reads the
    (B, H, N, d) views of the projections in place and writes O straight into a (B, N, H, d)
    buffer: no copies on either side of the kernel.
  * ``"triton"`` - the reference routes this to its Triton wrapper ``_flash_attn_forward``
    (:82-83); here it is custom_flash_attn.flash_attn_forward, the drop-in for that wrapper
    (same call, same asserts), running the same gfx950 kernel.  The Triton kernel itself is
    not rebuilt.
  There is no fallback for any of the three: if the extension is missing they raise.

Behaviour difference, on purpose: the reference's "cuda" branch reshapes the kernel's
(B, H, N, d) output straight to (B, N, H*d) without transposing (model_inference.py:92),
which scrambles heads and tokens.  Here the kernel output is transposed back to
(B, N, H, d) first, as the "manual" and "functional" branches do (:75, :80), so all
implementations compute the same function.
"""
from __future__ import annotations

import math
from typing import Callable, Dict

import torch
import torch.nn as nn
from torch.nn import functional as F

# --------------------------------------------------------------------------------------
# Attention implementations: (queries, keys, values, mask_bool, dropout) -> (B, N, H, d).
# queries/keys/values arrive as (B, H, N, d) views (model_inference.py:64-66).


def _attn_manual(q, k, v, mask_bool, dropout):
    # model_inference.py:68-75
    attn = q @ k.transpose(-2, -1)
    attn.masked_fill_(mask_bool, -torch.inf)
    attn_weights = torch.softmax(attn / k.shape[-1] ** 0.5, dim=-1)
    attn_weights = dropout(attn_weights)
    return (attn_weights @ v).transpose(1, 2)


def _attn_functional(q, k, v, mask_bool, dropout):
    # model_inference.py:77-80
    p = dropout.p if dropout.training else 0.0
    return F.scaled_dot_product_attention(q, k, v, is_causal=True, dropout_p=p).transpose(1, 2)


def _attn_cuda(q, k, v, mask_bool, dropout):
    # model_inference.py:85-90, plus the transpose back to (B, N, H, d).
    import custom_flash_attn  # raises if the native extension is not built

    out = custom_flash_attn.forward(q.contiguous(), k.contiguous(), v.contiguous())
    return out.transpose(1, 2)


def _attn_hip(q, k, v, mask_bool, dropout):
    # Same function as _attn_cuda with the copies fused away: q, k, v are read through their
    # strides and O lands in (B, N, H, d) order, ready for the .view(b, N, d_out) below.
    import custom_flash_attn  # raises if the native extension is not built

    b, h, n, d = q.shape
    out = torch.empty(b, n, h, d, dtype=q.dtype, device=q.device)
    custom_flash_attn.attention(q, k, v, out=out.transpose(1, 2))
    return out


def _attn_triton(q, k, v, mask_bool, dropout):
    # model_inference.py:82-83 (_flash_attn_forward on the (B, H, N, d) views), plus the
    # transpose back to (B, N, H, d) that the reference's branch leaves out (:92).
    import custom_flash_attn  # raises if the native extension is not built

    return custom_flash_attn.flash_attn_forward(q, k, v).transpose(1, 2)


ATTENTION_IMPLS: Dict[str, Callable] = {
    "manual": _attn_manual,
    "functional": _attn_functional,
    "triton": _attn_triton,
    "hip": _attn_hip,
    "cuda": _attn_cuda,
}


class MultiHeadAttention(nn.Module):
    """Causal multi-head self-attention (model_inference.py:39-94)."""

    def __init__(self, d_in, d_out, context_length, dropout, num_heads, impl_type, qkv_bias=False):
        super().__init__()
        assert d_out % num_heads == 0, "The output dimension must be a multiplicand of num_heads"
        if impl_type not in ATTENTION_IMPLS:
            raise ValueError(
                f"impl_type {impl_type!r} not available; choose one of {sorted(ATTENTION_IMPLS)}"
            )
        self.head_dim = d_out // num_heads
        self.num_heads = num_heads
        self.d_out = d_out
        self.impl_type = impl_type
        self.W_query = nn.Linear(d_in, d_out, bias=qkv_bias)
        self.W_key = nn.Linear(d_in, d_out, bias=qkv_bias)
        self.W_value = nn.Linear(d_in, d_out, bias=qkv_bias)
        self.out_proj = nn.Linear(d_out, d_out)
        self.dropout = nn.Dropout(dropout)
        self.register_buffer(
            "mask", torch.triu(torch.ones(context_length, context_length), diagonal=1)
        )

    def forward(self, x, kv_cache=None, layer: int = 0):
        if kv_cache is not None:
            return self._forward_cached(x, kv_cache, layer)
        b, num_tokens, _ = x.shape
        queries = self.W_query(x)
        keys = self.W_key(x)
        values = self.W_value(x)
        keys = keys.view(b, num_tokens, self.num_heads, self.head_dim).transpose(1, 2)
        queries = queries.view(b, num_tokens, self.num_heads, self.head_dim).transpose(1, 2)
        values = values.view(b, num_tokens, self.num_heads, self.head_dim).transpose(1, 2)
        mask_bool = self.mask.bool()[:num_tokens, :num_tokens]
        context_vec = ATTENTION_IMPLS[self.impl_type](queries, keys, values, mask_bool, self.dropout)
        context_vec = context_vec.contiguous().view(b, num_tokens, self.d_out)
        return self.out_proj(context_vec)


    def _forward_cached(self, x, cache, layer):
        """Attention against a KV cache (no counterpart in the reference, whose generate()
        re-runs the whole prefix, model_inference.py:199-228).

        Prefill (the cache is empty): the new tokens' K/V are copied into the cache and the
        causal forward kernel reads Q from the projection and K/V from the cache through their
        strides.  Decode (one new token): the decode kernel appends the token's K/V to the cache
        and attends over the cached prefix.  Both write the context straight into a
        (B, N, H*d) buffer.
        """
        import custom_flash_attn  # raises if the native extension is not built

        if self.impl_type not in ("hip", "cuda"):
            raise ValueError(f"cached attention runs on the HIP kernels; impl_type is {self.impl_type!r}")
        b, n, _ = x.shape
        H, hd = self.num_heads, self.head_dim
        q = self.W_query(x).view(b, n, H, hd)
        k = self.W_key(x).view(b, n, H, hd)
        v = self.W_value(x).view(b, n, H, hd)
        kc, vc = cache.k[layer], cache.v[layer]
        ctx = torch.empty(b, n, H, hd, dtype=q.dtype, device=q.device)
        if cache.length == 0:
            if n > kc.shape[2]:
                raise ValueError(f"{n} tokens do not fit a cache of {kc.shape[2]}")
            kc[:, :, :n].copy_(k.transpose(1, 2))
            vc[:, :, :n].copy_(v.transpose(1, 2))
            custom_flash_attn.attention(q.transpose(1, 2), kc[:, :, :n], vc[:, :, :n],
                                        out=ctx.transpose(1, 2))
        elif n == 1:
            custom_flash_attn.decode(q[:, 0], kc, vc, cache.seqlens, k[:, 0], v[:, 0],
                                     out=ctx[:, 0], workspace=cache.workspace)
        else:
            raise NotImplementedError("a cache that already holds tokens takes one new token per step")
        return self.out_proj(ctx.view(b, n, self.d_out))


class KVCache:
    """Per-layer K/V caches of a GPTModel for cached decoding.

    ``k[layer]``, ``v[layer]``: (B, H, max_len, head_dim) bf16 on ``device`` (each head's rows
    contiguous, which the decode kernel streams); ``seqlens``: int32 (B,) on the device, the
    cached rows per batch row; ``length``: the same count on the host.  ``workspace`` holds
    the decode kernel's split partials.
    """

    def __init__(self, cfg: dict, batch: int, max_len: int, device, dtype=torch.bfloat16):
        import custom_flash_attn

        H = cfg["n_heads"]
        hd = cfg["emb_dim"] // H
        self.max_len = max_len
        self.k = [torch.zeros(batch, H, max_len, hd, dtype=dtype, device=device) for _ in range(cfg["n_layers"])]
        self.v = [torch.zeros(batch, H, max_len, hd, dtype=dtype, device=device) for _ in range(cfg["n_layers"])]
        self.seqlens = torch.zeros(batch, dtype=torch.int32, device=device)
        self.length = 0
        nbytes = custom_flash_attn._C.decode_workspace_bytes(batch, H, max_len)
        self.workspace = torch.empty(nbytes, dtype=torch.uint8, device=device)

    def advance(self, n: int) -> None:
        self.length += n
        self.seqlens.add_(n)

    def reset(self) -> None:
        self.length = 0
        self.seqlens.zero_()


class GraphedDecoder:
    """One decode step of ``model`` (batch ``batch``, cache of ``max_len`` rows) captured in a
    HIP graph and replayed per token, so a step costs one graph launch instead of the ~20
    kernel launches (and their Python) per layer of an eager step.

    The step reads its token from ``self.tok`` and leaves the last position's logits in
    ``self.logits``.  Everything it depends on lives in device memory: the positions and the
    decode kernel's lengths come from ``cache.seqlens``, which the graph itself advances.
    Capture runs two eager warm-up steps on a side stream first (they write cache rows 0-1,
    which the prefill later overwrites), then resets the cache."""

    def __init__(self, model, batch: int, max_len: int, device):
        cfg = {"n_heads": model.trf_blocks[0].att.num_heads, "emb_dim": model.tok_emb.embedding_dim,
               "n_layers": len(model.trf_blocks)}
        self.model = model
        self.cache = KVCache(cfg, batch, max_len, device)
        self.tok = torch.zeros(batch, 1, dtype=torch.long, device=device)
        side = torch.cuda.Stream(device)
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.no_grad(), torch.cuda.stream(side):
            self.cache.length = 1
            self.cache.seqlens.fill_(1)
            for _ in range(2):
                model(self.tok, kv_cache=self.cache)
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph, stream=side):
                self.logits = model(self.tok, kv_cache=self.cache)[:, -1, :]
        torch.cuda.current_stream(device).wait_stream(side)
        self.cache.reset()

    def prefill(self, idx):
        """Eager prefill of the prompt; returns the last position's logits."""
        with torch.no_grad():
            return self.model(idx, kv_cache=self.cache)[:, -1, :]

    def step(self, tok):
        """Appends ``tok`` ((B, 1) token ids) and returns the next logits (a view of the
        graph's output buffer, overwritten by the next step)."""
        self.tok.copy_(tok)
        self.graph.replay()
        self.cache.length += 1  # the graph advanced cache.seqlens on the device
        return self.logits


class LayerNorm(nn.Module):
    """LayerNorm with eps 1e-5 and biased variance (model_inference.py:96-107)."""

    def __init__(self, config):
        super().__init__()
        self.eps = 1e-5
        self.scale = nn.Parameter(torch.ones(config["emb_dim"]))
        self.shift = nn.Parameter(torch.zeros(config["emb_dim"]))

    def forward(self, x):
        mean = torch.mean(x, dim=-1, keepdim=True)
        variance = torch.var(x, dim=-1, keepdim=True, unbiased=False)
        norm_x = (x - mean) / torch.sqrt(variance + self.eps)
        return norm_x * self.scale + self.shift


class GELU(nn.Module):
    """tanh-approximation GELU (model_inference.py:109-117)."""

    def forward(self, x):
        return 0.5 * x * (1 + torch.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * torch.pow(x, 3))))


class FeedForward(nn.Module):
    """Linear(d, 4d) -> GELU -> Linear(4d, d) (model_inference.py:119-128)."""

    def __init__(self, config):
        super().__init__()
        self.layers = nn.Sequential(
            nn.Linear(config["emb_dim"], 4 * config["emb_dim"]),
            GELU(),
            nn.Linear(4 * config["emb_dim"], config["emb_dim"]),
        )

    def forward(self, x):
        return self.layers(x)


class TransformerBlock(nn.Module):
    """Pre-LN block; attention runs under bf16 autocast on the GPU (model_inference.py:131-164)."""

    def __init__(self, cfg):
        super().__init__()
        self.att = MultiHeadAttention(
            d_in=cfg["emb_dim"], d_out=cfg["emb_dim"], context_length=cfg["context_length"],
            num_heads=cfg["n_heads"], dropout=cfg["drop_rate"], impl_type=cfg["impl_type"],
            qkv_bias=cfg["qkv_bias"],
        )
        self.ff = FeedForward(cfg)
        self.norm1 = LayerNorm(cfg)
        self.norm2 = LayerNorm(cfg)
        self.drop_shortcut = nn.Dropout(cfg["drop_rate"])

    def forward(self, x, kv_cache=None, layer: int = 0):
        shortcut = x
        x = self.norm1(x)
        # model_inference.py:153 - autocast only has an effect for CUDA(HIP) tensors, so it
        # is switched on only for them (same result, no warning on CPU-only hosts).
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16, enabled=x.is_cuda):
            x = self.att(x, kv_cache, layer)
        x = self.drop_shortcut(x)
        x = x + shortcut
        shortcut = x
        x = self.norm2(x)
        x = self.ff(x)
        x = self.drop_shortcut(x)
        return x + shortcut


class GPTModel(nn.Module):
    """Token + position embeddings, blocks, final LN, untied LM head (model_inference.py:166-190)."""

    def __init__(self, cfg):
        super().__init__()
        self.tok_emb = nn.Embedding(cfg["vocab_size"], cfg["emb_dim"])
        self.pos_emb = nn.Embedding(cfg["context_length"], cfg["emb_dim"])
        self.drop_emb = nn.Dropout(cfg["drop_rate"])
        self.trf_blocks = nn.Sequential(*[TransformerBlock(cfg) for _ in range(cfg["n_layers"])])
        self.final_norm = LayerNorm(cfg)
        self.out_head = nn.Linear(cfg["emb_dim"], cfg["vocab_size"], bias=False)

    def forward(self, in_idx, kv_cache=None):
        """Logits for ``in_idx``.  With ``kv_cache`` the tokens continue the cached sequence:
        positions start at the cached length, read from ``kv_cache.seqlens`` on the device (so a
        captured decode step stays correct on replay), and the cache advances by the token
        count."""
        _, seq_len = in_idx.shape
        tok_embeds = self.tok_emb(in_idx)
        pos = torch.arange(seq_len, device=in_idx.device)
        if kv_cache is not None:
            pos = kv_cache.seqlens[:, None].long() + pos  # (B, T)
        pos_embeds = self.pos_emb(pos)
        x = self.drop_emb(tok_embeds + pos_embeds)
        if kv_cache is None:
            x = self.trf_blocks(x)
        else:
            for layer, blk in enumerate(self.trf_blocks):
                x = blk(x, kv_cache, layer)
            kv_cache.advance(seq_len)
        x = self.final_norm(x)
        return self.out_head(x)


def _next_token(logits, temperature, top_k):
    # model_inference.py:207-222: optional top-k filter, then temperature sampling or argmax.
    # The reference takes min_val = top_logits[:, -1], shape (B,), which broadcasts against the
    # (B, vocab) logits only for B = 1; here it keeps a column, (B, 1), so batches work too.
    if top_k is not None:
        top_logits, _ = torch.topk(logits, top_k)
        min_val = top_logits[:, -1:]
        logits = torch.where(logits < min_val, torch.tensor(float("-inf"), device=logits.device), logits)
    if temperature > 0.0:
        logits = logits / temperature
        probs = torch.softmax(logits, dim=-1)
        return torch.multinomial(probs, num_samples=1)
    return torch.argmax(logits, dim=-1, keepdim=True)


def generate(model, idx, max_new_tokens, context_size, temperature=1.0, top_k=None, eos_id=None):
    """The reference's token loop (model_inference.py:199-228): every step re-runs the model
    over the last ``context_size`` tokens and samples from the last position's logits."""
    for _ in range(max_new_tokens):
        idx_cond = idx[:, -context_size:]
        with torch.no_grad():
            logits = model(idx_cond)[:, -1, :]
        idx_next = _next_token(logits, temperature, top_k)
        if idx_next == eos_id:
            break
        idx = torch.cat((idx, idx_next), dim=1)
    return idx


def generate_cached(model, idx, max_new_tokens, context_size, temperature=1.0, top_k=None,
                    eos_id=None):
    """:func:`generate` with a KV cache: one prefill over the prompt, then one decode step per
    new token (the decode kernel, which appends the token's K/V and attends over the cache).
    Same sampling.  The whole sequence must fit ``context_size`` (no sliding window: shifting
    positions would invalidate the cache)."""
    if idx.shape[1] + max_new_tokens > context_size:
        raise ValueError(f"prompt ({idx.shape[1]}) + max_new_tokens ({max_new_tokens}) exceeds "
                         f"context_size ({context_size})")
    cfg = {"n_heads": model.trf_blocks[0].att.num_heads, "emb_dim": model.tok_emb.embedding_dim,
           "n_layers": len(model.trf_blocks)}
    cache = KVCache(cfg, idx.shape[0], idx.shape[1] + max_new_tokens, idx.device)
    step_in = idx
    for _ in range(max_new_tokens):
        with torch.no_grad():
            logits = model(step_in, kv_cache=cache)[:, -1, :]
        idx_next = _next_token(logits, temperature, top_k)
        if idx_next == eos_id:
            break
        idx = torch.cat((idx, idx_next), dim=1)
        step_in = idx_next
    return idx


def generate_graphed(model, idx, max_new_tokens, context_size, temperature=1.0, top_k=None,
                     eos_id=None, decoder: GraphedDecoder | None = None):
    """:func:`generate_cached` with every decode step replayed from a :class:`GraphedDecoder`
    (built here unless one for this batch and length is passed in).  Same sampling."""
    if idx.shape[1] + max_new_tokens > context_size:
        raise ValueError(f"prompt ({idx.shape[1]}) + max_new_tokens ({max_new_tokens}) exceeds "
                         f"context_size ({context_size})")
    if decoder is None:
        decoder = GraphedDecoder(model, idx.shape[0], idx.shape[1] + max_new_tokens, idx.device)
    elif decoder.cache.max_len < idx.shape[1] + max_new_tokens:
        raise ValueError("the decoder's cache is shorter than prompt + max_new_tokens")
    decoder.cache.reset()
    logits = decoder.prefill(idx)
    for i in range(max_new_tokens):
        idx_next = _next_token(logits, temperature, top_k)
        if idx_next == eos_id:
            break
        idx = torch.cat((idx, idx_next), dim=1)
        if i + 1 < max_new_tokens:
            logits = decoder.step(idx_next)
    return idx


# Base config (model_inference.py:378-386) and the sizes of model_inference.py:393-397; the
# benchmark loop sets context_length 1024 and qkv_bias True (:415).
GPT_CONFIG_124M = {
    "vocab_size": 50257,
    "context_length": 256,
    "emb_dim": 768,
    "n_heads": 12,
    "n_layers": 12,
    "drop_rate": 0.1,
    "qkv_bias": False,
}

MODEL_CONFIGS = {
    "gpt2-small (124M)": {"emb_dim": 768, "n_layers": 12, "n_heads": 12},
    "gpt2-medium (355M)": {"emb_dim": 1024, "n_layers": 24, "n_heads": 16},
    "gpt2-large (774M)": {"emb_dim": 1280, "n_layers": 36, "n_heads": 20},
    "gpt2-xl (1558M)": {"emb_dim": 1600, "n_layers": 48, "n_heads": 25},
}


def gpt2_config(name: str, impl_type: str, drop_rate: float = 0.0) -> dict:
    """Config as the reference's benchmark builds it (model_inference.py:413-415)."""
    cfg = dict(GPT_CONFIG_124M)
    cfg.update(MODEL_CONFIGS[name])
    cfg.update({"context_length": 1024, "qkv_bias": True, "impl_type": impl_type, "drop_rate": drop_rate})
    return cfg


def init_gpt2_weights(model: nn.Module, seed: int) -> None:
    """Seeded random init in place of the pretrained download: every Linear/Embedding
    weight ~ N(0, 0.02^2), biases 0, LayerNorm scale 1 and shift 0."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    with torch.no_grad():
        for mod in model.modules():
            if isinstance(mod, (nn.Linear, nn.Embedding)):
                w = torch.empty(mod.weight.shape, dtype=torch.float32).normal_(0.0, 0.02, generator=g)
                mod.weight.copy_(w)
                if getattr(mod, "bias", None) is not None:
                    mod.bias.zero_()
            elif isinstance(mod, LayerNorm):
                mod.scale.fill_(1.0)
                mod.shift.zero_()
