"""Decoder-shaped stack around the MoE-MLP path.

openPangu-Embedded-1B-shaped and randomly initialised: 26 x (RMSNorm, causal
attention with 12 heads of 128 and a KV cache, RMSNorm, MoE-MLP), token embedding and
LM head over a 153,376-word vocabulary, bf16. Prefill a prompt, then greedy decode;
the MoE-MLP is ``IntegratedOpenPanguMoEMLP`` (eval path through the MI355X kernels,
the module tree of src/openpangu_moe.py:43-130), mirroring the reference's manual
decode benchmark (src/evaluation_triton.py:403-460). ``run`` reports the prefill time
(eager, events around each MoE-MLP call) and the decode step: one whole greedy step
(26 layers, LM head, argmax, next position) captured in a HIP graph with static shapes
-- the KV cache at its full length, the position a device tensor, a causal mask over
the cache -- replayed ``steps`` times, once with and once without the MoE-MLP, so the
MoE share is device time rather than host dispatch.

Attention is plain torch with contiguous right operands (the K cache is kept
transposed, so no transposed view enters a batched bf16 product); it is harness, not
part of the hot path.
"""
from __future__ import annotations

import math
import types
from typing import Dict, List

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops
from .model import IntegratedOpenPanguMoEMLP, physical_reorder_for_inference

VOCAB = 153376


class RMSNorm(nn.Module):
    def __init__(self, d: int, eps: float = 1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(d))
        self.eps = eps

    def forward(self, x):
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps) * self.weight.float()).to(x.dtype)


def rope(x: torch.Tensor, pos: torch.Tensor, base: float = 10000.0) -> torch.Tensor:
    """Rotary position embedding on [B, heads, L, hd] (half-split form)."""
    hd = x.shape[-1]
    inv = 1.0 / (base ** (torch.arange(0, hd, 2, device=x.device, dtype=torch.float32) / hd))
    ang = pos.float()[:, None] * inv[None, :]                       # [L, hd/2]
    cos, sin = ang.cos()[None, None], ang.sin()[None, None]
    x1, x2 = x.float()[..., : hd // 2], x.float()[..., hd // 2:]
    return torch.cat([x1 * cos - x2 * sin, x1 * sin + x2 * cos], -1).to(x.dtype)


class Attention(nn.Module):
    def __init__(self, d: int, heads: int, max_len: int):
        super().__init__()
        self.h, self.hd = heads, d // heads
        self.qkv = nn.Linear(d, 3 * d, bias=False)
        self.o = nn.Linear(d, d, bias=False)
        self.max_len = max_len
        self.kt_cache = None  # [B, h, hd, max_len]: K kept transposed
        self.v_cache = None   # [B, h, max_len, hd]
        self.len = 0

    def reset(self, B: int, device, dtype):
        self.kt_cache = torch.zeros(B, self.h, self.hd, self.max_len, device=device, dtype=dtype)
        self.v_cache = torch.zeros(B, self.h, self.max_len, self.hd, device=device, dtype=dtype)
        self.len = 0

    def forward(self, x):
        """Eager: L new tokens at host position ``self.len``."""
        B, L, D = x.shape
        q, k, v = self.qkv(x).view(B, L, 3, self.h, self.hd).permute(2, 0, 3, 1, 4)  # [B, h, L, hd] each
        pos = torch.arange(self.len, self.len + L, device=x.device)
        q, k = rope(q, pos), rope(k, pos)
        self.kt_cache[:, :, :, self.len:self.len + L] = k.transpose(-1, -2)
        self.v_cache[:, :, self.len:self.len + L] = v
        T = self.len + L
        kt = self.kt_cache[:, :, :, :T].contiguous()                    # [B, h, hd, T]
        s = torch.matmul(q.contiguous(), kt).float() / math.sqrt(self.hd)  # [B, h, L, T]
        if L > 1:
            causal = torch.ones(L, T, device=x.device, dtype=torch.bool).tril(T - L)
            s = s.masked_fill(~causal, float("-inf"))
        p = torch.softmax(s, -1).to(x.dtype)
        o = torch.matmul(p, self.v_cache[:, :, :T].contiguous())        # [B, h, L, hd]
        self.len = T
        return self.o(o.transpose(1, 2).reshape(B, L, D))

    def forward_static(self, x, pos_t, mask):
        """One token at device position ``pos_t`` ([1] int64), attending over the whole
        cache with ``mask`` ([max_len]: 0 up to pos_t, -inf after): static shapes, so a
        step can be captured in a graph."""
        B, L, D = x.shape
        q, k, v = self.qkv(x).view(B, L, 3, self.h, self.hd).permute(2, 0, 3, 1, 4)  # [B, h, 1, hd]
        q, k = rope(q, pos_t), rope(k, pos_t)
        self.kt_cache.index_copy_(3, pos_t, k.transpose(-1, -2).contiguous())
        self.v_cache.index_copy_(2, pos_t, v.contiguous())
        s = torch.matmul(q.contiguous(), self.kt_cache).float() / math.sqrt(self.hd)  # [B, h, 1, max_len]
        p = torch.softmax(s + mask, -1).to(x.dtype)
        o = torch.matmul(p, self.v_cache)                                  # [B, h, 1, hd]
        return self.o(o.transpose(1, 2).reshape(B, L, D))


class Block(nn.Module):
    def __init__(self, cfg, args, max_len: int):
        super().__init__()
        self.input_layernorm = RMSNorm(cfg.hidden_size)
        self.self_attn = Attention(cfg.hidden_size, cfg.num_attention_heads, max_len)
        self.post_attention_layernorm = RMSNorm(cfg.hidden_size)
        self.mlp = IntegratedOpenPanguMoEMLP(cfg, args)
        self.moe_events: List = []

    def forward(self, x):
        x = x + self.self_attn(self.input_layernorm(x))
        h = self.post_attention_layernorm(x)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        m = self.mlp(h)
        e1.record()
        self.moe_events.append((e0, e1))
        return x + m

    def forward_static(self, x, pos_t, mask, moe: bool = True):
        x = x + self.self_attn.forward_static(self.input_layernorm(x), pos_t, mask)
        h = self.post_attention_layernorm(x)
        # without the MoE-MLP the step keeps the norm and the residual add, so the
        # difference of the two step times is the MoE-MLP call alone
        return x + (self.mlp(h) if moe else h)


class DecoderStack(nn.Module):
    def __init__(self, layers: int = 26, hidden: int = 1536, heads: int = 12, experts: int = 16,
                 group: int = 384, tau: float = 0.70, vocab: int = VOCAB, max_len: int = 1152):
        super().__init__()
        self.cfg = types.SimpleNamespace(hidden_size=hidden, intermediate_size=experts * group,
                                         num_attention_heads=heads)
        self.args = types.SimpleNamespace(group_size=group, tau=tau)
        self.embed_tokens = nn.Embedding(vocab, hidden)
        self.layers = nn.ModuleList([Block(self.cfg, self.args, max_len) for _ in range(layers)])
        self.norm = RMSNorm(hidden)
        self.lm_head = nn.Linear(hidden, vocab, bias=False)

    @torch.no_grad()
    def init_random(self, seed: int = 0, std: float = 0.02):
        dev = self.embed_tokens.weight.device
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        for p in self.parameters():
            if p.dim() >= 2:
                p.copy_(torch.randn(p.shape, generator=g, device=p.device, dtype=torch.float32) * std)
        for blk in self.layers:
            mlp = blk.mlp
            E = mlp.moelayer.experts
            ids = torch.randperm(mlp.moelayer.dimension, generator=g, device=dev) % E
            mlp.moelayer.experts_masks.copy_(F.one_hot(ids, E).t().to(mlp.moelayer.experts_masks.dtype))

    def prepare_inference(self, tau: float):
        physical_reorder_for_inference(self.layers, tau)

    def forward(self, ids):
        x = self.embed_tokens(ids)
        for blk in self.layers:
            x = blk(x)
        return self.lm_head(self.norm(x[:, -1:]))

    def step_static(self, tok_t, pos_t, moe: bool = True, finite_t=None):
        """One greedy decode step on device state: token ``tok_t`` [1, 1] at position
        ``pos_t`` [1]; writes the next token into ``tok_t`` and advances ``pos_t``.
        ``finite_t`` ([1] bool, optional) is and-ed with "every logit is finite"."""
        ar = torch.arange(self.layers[0].self_attn.max_len, device=tok_t.device)
        mask = torch.where(ar <= pos_t, 0.0, float("-inf")).to(torch.float32)
        x = self.embed_tokens(tok_t)
        for blk in self.layers:
            x = blk.forward_static(x, pos_t, mask, moe)
        logits = self.lm_head(self.norm(x))
        if finite_t is not None:
            finite_t.logical_and_(torch.isfinite(logits).all().view(1))
        tok_t.copy_(logits.argmax(-1))
        pos_t.add_(1)


@torch.no_grad()
def build(prompt_len: int = 1024, steps: int = 128, layers: int = 26, tau: float = 0.70, seed: int = 0,
          device: str = "cuda:0"):
    """The random-init bf16 stack, reordered for inference (fp32 routers), with empty KV
    caches, and the random prompt ids [1, prompt_len]."""
    dev = torch.device(device)
    model = DecoderStack(layers=layers, max_len=prompt_len + steps).to(dev)
    model.init_random(seed)
    model = model.to(torch.bfloat16).eval()
    for blk in model.layers:  # the masked layer and projections feed the reorder; keep the router fp32
        blk.mlp.moelayer.float()
    model.prepare_inference(tau)
    for blk in model.layers:
        blk.self_attn.reset(1, dev, torch.bfloat16)
    g = torch.Generator(device="cpu")
    g.manual_seed(seed + 1)
    ids = torch.randint(0, VOCAB, (1, prompt_len), generator=g).to(dev)
    return model, ids


@torch.no_grad()
def run(prompt_len: int = 1024, steps: int = 128, layers: int = 26, tau: float = 0.70, seed: int = 0,
        device: str = "cuda:0", verify_steps: int = 3, moe_hook=None, moe_hook_steps: int = 0) -> Dict[str, float]:
    """Prefill ``prompt_len`` random token ids, then ``steps`` greedy decode steps at
    batch 1. Returns per-step and prefill times and the MoE-MLP share.

    Checks: the first ``verify_steps`` graph replays give the eager steps' tokens
    (``graph_replays_match_eager``) and every logit of those eager steps is finite
    (``logits_finite``). ``moe_hook(layer, mlp, hidden, out)``, when given, is called for
    every layer's MoE-MLP call of the first ``moe_hook_steps`` eager decode steps (e.g. to
    check each call against an oracle)."""
    dev = torch.device(device)
    model, ids = build(prompt_len, steps, layers, tau, seed, device)

    def moe_ms():
        torch.cuda.synchronize()
        t = sum(e0.elapsed_time(e1) for blk in model.layers for (e0, e1) in blk.moe_events)
        for blk in model.layers:
            blk.moe_events.clear()
        return t

    # warm-up on a short prompt (kernels, allocator), then reset the caches
    model(ids[:, :16])
    moe_ms()
    for blk in model.layers:
        blk.self_attn.reset(1, dev, torch.bfloat16)
    s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s0.record()
    logits = model(ids)
    s1.record()
    torch.cuda.synchronize()
    prefill_ms = s0.elapsed_time(s1)
    prefill_moe = moe_ms()
    nxt = logits.argmax(-1)

    checked = {}
    finite_t = torch.ones(1, dtype=torch.bool, device=dev)

    def decode_ms(moe: bool) -> float:
        """One captured greedy step replayed ``steps`` times from the prompt's end; the
        first replays are checked token for token against eager steps from the same state."""
        tok_t = nxt.clone().view(1, 1)
        pos_t = torch.tensor([prompt_len], device=dev, dtype=torch.int64)
        n_chk = min(verify_steps, steps)
        eager = []
        for i in range(n_chk):
            handles = []
            if moe and moe_hook is not None and i < moe_hook_steps:
                for li, blk in enumerate(model.layers):
                    handles.append(blk.mlp.register_forward_hook(
                        lambda mod, args, out, li=li: moe_hook(li, mod, args[0], out)))
            model.step_static(tok_t, pos_t, moe, finite_t)
            for h in handles:
                h.remove()
            eager.append(int(tok_t.item()))
        pos_t.fill_(prompt_len)
        tok_t.copy_(nxt.view(1, 1))
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):  # warm-up outside the graph (allocator, kernels)
            for _ in range(2):
                model.step_static(tok_t, pos_t, moe)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            model.step_static(tok_t, pos_t, moe)
        pos_t.fill_(prompt_len)
        tok_t.copy_(nxt.view(1, 1))
        replayed = []
        for _ in range(n_chk):
            graph.replay()
            replayed.append(int(tok_t.item()))
        checked[moe] = replayed == eager
        pos_t.fill_(prompt_len)
        tok_t.copy_(nxt.view(1, 1))
        s0.record()
        for _ in range(steps):
            graph.replay()
        s1.record()
        torch.cuda.synchronize()
        return s0.elapsed_time(s1) / steps

    decode_step = decode_ms(True)
    decode_step_no_moe = decode_ms(False)
    decode_moe = max(decode_step - decode_step_no_moe, 0.0)
    return {
        "layers": layers, "prompt": prompt_len, "steps": steps, "tau": tau,
        "prefill_ms": prefill_ms, "prefill_moe_ms": prefill_moe, "prefill_moe_share": prefill_moe / prefill_ms,
        "decode_ms_per_step": decode_step, "decode_ms_per_step_without_moe": decode_step_no_moe,
        "decode_moe_ms_per_step": decode_moe, "decode_moe_share": decode_moe / decode_step,
        "decode_moe_us_per_layer": decode_moe / layers * 1000.0,
        "graph_replays_match_eager": bool(checked.get(True)) and bool(checked.get(False)),
        "verified_steps": min(verify_steps, steps), "logits_finite": bool(finite_t.item()),
        "note": ("random-init bf16 weights, random prompt ids; prefill: events around each MoE-MLP call; "
                 "decode: one graph-captured greedy step (static-shape attention over the full cache) "
                 "replayed, MoE share = step time with minus without the MoE-MLP"),
    }
