"""GPT-2 style pre-LN transformer block used as a test and benchmark model.

The same module the reference's tests build (tests/models/transformer.py:4-28):
ln1 -> c_attn -> per-head causal attention with a -inf upper-triangular mask
buffer -> c_proj + residual; ln2 -> fc -> GELU(tanh) -> proj + residual.
"""

import math

import torch
import torch.nn as nn
import torch.nn.functional as F


class Block(nn.Module):
    """GPT-2 style pre-LN transformer block (inference)."""

    def __init__(self, d=64, nh=4, T=16):
        super().__init__()
        self.nh = nh
        self.ln1 = nn.LayerNorm(d)
        self.ln2 = nn.LayerNorm(d)
        self.c_attn = nn.Linear(d, 3 * d)
        self.c_proj = nn.Linear(d, d)
        self.fc = nn.Linear(d, 4 * d)
        self.proj = nn.Linear(4 * d, d)
        self.register_buffer("mask", torch.full((T, T), float("-inf")).triu(1))

    def attn(self, x):
        T, C = x.shape
        q, k, v = self.c_attn(x).split(C, dim=1)
        hd = C // self.nh
        q = q.view(T, self.nh, hd).transpose(0, 1)
        k = k.view(T, self.nh, hd).transpose(0, 1)
        v = v.view(T, self.nh, hd).transpose(0, 1)
        att = (q @ k.transpose(-2, -1)) * (1.0 / math.sqrt(hd))
        att = att + self.mask[:T, :T]
        att = F.softmax(att, dim=-1)
        y = (att @ v).transpose(0, 1).contiguous().view(T, C)
        return self.c_proj(y)

    def forward(self, x):
        x = x + self.attn(self.ln1(x))
        x = x + self.proj(F.gelu(self.fc(self.ln2(x)), approximate="tanh"))
        return x


class Stack(nn.Module):
    """`layers` Blocks plus a final LayerNorm (GPT-2 small body without
    embeddings or LM head)."""

    def __init__(self, layers=12, d=768, nh=12, T=1024):
        super().__init__()
        self.blocks = nn.ModuleList(Block(d, nh, T) for _ in range(layers))
        self.ln_f = nn.LayerNorm(d)

    def forward(self, x):
        for b in self.blocks:
            x = b(x)
        return self.ln_f(x)


def gpt2_init_(module, std=0.02, seed=None):
    """Random init of the benchmark configs: Linear weights and biases
    ~N(0, std), LayerNorm gamma = 1, beta = 0."""
    gen = torch.Generator().manual_seed(seed) if seed is not None else None
    with torch.no_grad():
        for m in module.modules():
            if isinstance(m, nn.Linear):
                m.weight.copy_(torch.randn(m.weight.shape, generator=gen) * std)
                if m.bias is not None:
                    m.bias.copy_(torch.randn(m.bias.shape, generator=gen) * std)
            elif isinstance(m, nn.LayerNorm):
                m.weight.fill_(1.0)
                m.bias.fill_(0.0)
    return module
