"""A GPT-2 module tree with Hugging Face's module names (test infrastructure).

transformer.wte / wpe / h.{i}.ln_1 / attn.c_attn / attn.c_proj / ln_2 / mlp.c_fc / mlp.c_proj / ln_f
and a tied lm_head, with the projections as a `Conv1D` class that keeps its weight as
(in, out), as transformers does.  Attention scores and their softmax-weighted sums are computed
in fp32 with contiguous operands (no bf16 batched products on transposed views), whatever the
autocast state; the projections follow autocast.
"""
from __future__ import annotations

import math

import torch
from torch import nn
from torch.nn import functional as F


class Conv1D(nn.Module):
    def __init__(self, nf: int, nx: int):
        super().__init__()
        self.nf = nf
        self.weight = nn.Parameter(torch.empty(nx, nf))
        self.bias = nn.Parameter(torch.zeros(nf))
        nn.init.normal_(self.weight, std=0.02)

    def forward(self, x):
        out = torch.addmm(self.bias, x.reshape(-1, x.shape[-1]), self.weight)
        return out.reshape(*x.shape[:-1], self.nf)


class Attention(nn.Module):
    def __init__(self, d: int, heads: int):
        super().__init__()
        self.heads, self.d = heads, d
        self.c_attn = Conv1D(3 * d, d)
        self.c_proj = Conv1D(d, d)

    def forward(self, x):
        b, t, _ = x.shape
        q, k, v = self.c_attn(x).split(self.d, dim=2)
        hd = self.d // self.heads

        def heads(z):
            return z.reshape(b, t, self.heads, hd).permute(0, 2, 1, 3).float().contiguous()

        q, k, v = heads(q), heads(k), heads(v)
        with torch.autocast(device_type=x.device.type, enabled=False):
            scores = torch.matmul(q, k.transpose(-1, -2).contiguous()) / math.sqrt(hd)
            mask = torch.ones(t, t, dtype=torch.bool, device=x.device).tril()
            probs = torch.softmax(scores.masked_fill(~mask, float("-inf")), dim=-1)
            ctx = torch.matmul(probs, v)
        ctx = ctx.permute(0, 2, 1, 3).reshape(b, t, self.d).to(x.dtype)
        return self.c_proj(ctx)


class MLP(nn.Module):
    def __init__(self, d: int):
        super().__init__()
        self.c_fc = Conv1D(4 * d, d)
        self.c_proj = Conv1D(d, 4 * d)

    def forward(self, x):
        return self.c_proj(F.gelu(self.c_fc(x), approximate="tanh"))


class Block(nn.Module):
    def __init__(self, d: int, heads: int):
        super().__init__()
        self.ln_1, self.attn = nn.LayerNorm(d), Attention(d, heads)
        self.ln_2, self.mlp = nn.LayerNorm(d), MLP(d)

    def forward(self, x):
        x = x + self.attn(self.ln_1(x))
        return x + self.mlp(self.ln_2(x))


class Transformer(nn.Module):
    def __init__(self, vocab: int, positions: int, d: int, layers: int, heads: int):
        super().__init__()
        self.wte, self.wpe = nn.Embedding(vocab, d), nn.Embedding(positions, d)
        nn.init.normal_(self.wte.weight, std=0.02)
        nn.init.normal_(self.wpe.weight, std=0.01)
        self.h = nn.ModuleList(Block(d, heads) for _ in range(layers))
        self.ln_f = nn.LayerNorm(d)

    def forward(self, ids):
        pos = torch.arange(ids.shape[1], device=ids.device)
        x = self.wte(ids) + self.wpe(pos)[None]
        for block in self.h:
            x = block(x)
        return self.ln_f(x)


class GPT2LMHeadModel(nn.Module):
    def __init__(self, vocab=50257, positions=1024, d=1024, layers=24, heads=16):
        super().__init__()
        self.transformer = Transformer(vocab, positions, d, layers, heads)
        self.lm_head = nn.Linear(d, vocab, bias=False)
        self.lm_head.weight = self.transformer.wte.weight  # tied, as GPT-2

    def forward(self, ids):
        logits = self.lm_head(self.transformer(ids))
        return F.cross_entropy(logits[:, :-1].reshape(-1, logits.shape[-1]).float(), ids[:, 1:].reshape(-1))
