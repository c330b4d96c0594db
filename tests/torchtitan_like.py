"""Small modules built like TorchTitan's llama3 / MoE ones (class names and
attributes of torchtitan/models/llama3/model/model.py and
torchtitan/models/moe/moe.py, which are not installed here), for testing the
converter of sfu_repro.torchtitan."""

import math

import torch
import torch.nn.functional as F
from torch import nn


class FeedForward(nn.Module):
    def __init__(self, dim, hidden):
        super().__init__()
        self.w1 = nn.Linear(dim, hidden, bias=False)
        self.w2 = nn.Linear(hidden, dim, bias=False)
        self.w3 = nn.Linear(dim, hidden, bias=False)

    def forward(self, x):
        return self.w2(F.silu(self.w1(x)) * self.w3(x))


class ScaledDotProductAttention(nn.Module):
    def forward(self, q, k, v, *, scale=None, enable_gqa=False):
        rep = q.shape[1] // k.shape[1]
        k = k.repeat_interleave(rep, dim=1)
        v = v.repeat_interleave(rep, dim=1)
        return F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=scale)


class Attention(nn.Module):
    def __init__(self, dim, n_heads, n_kv_heads):
        super().__init__()
        self.n_heads, self.n_kv_heads = n_heads, n_kv_heads
        self.head_dim = dim // n_heads
        self.wq = nn.Linear(dim, n_heads * self.head_dim, bias=False)
        self.wk = nn.Linear(dim, n_kv_heads * self.head_dim, bias=False)
        self.wv = nn.Linear(dim, n_kv_heads * self.head_dim, bias=False)
        self.wo = nn.Linear(n_heads * self.head_dim, dim, bias=False)
        self.inner_attention = ScaledDotProductAttention()
        self.attn_type = "sdpa"

    def init_weights(self, init_std):
        for lin in (self.wq, self.wk, self.wv, self.wo):
            nn.init.trunc_normal_(lin.weight, std=init_std)

    def forward(self, x):
        b, s, _ = x.shape
        q = self.wq(x).view(b, s, self.n_heads, self.head_dim).transpose(1, 2)
        k = self.wk(x).view(b, s, self.n_kv_heads, self.head_dim).transpose(1, 2)
        v = self.wv(x).view(b, s, self.n_kv_heads, self.head_dim).transpose(1, 2)
        out = self.inner_attention(q, k, v, scale=1.0 / math.sqrt(self.head_dim))
        return self.wo(out.transpose(1, 2).reshape(b, s, -1))


class Block(nn.Module):
    def __init__(self, dim, hidden, n_heads, n_kv_heads):
        super().__init__()
        self.attention = Attention(dim, n_heads, n_kv_heads)
        self.feed_forward = FeedForward(dim, hidden)
        self.attention_norm = nn.RMSNorm(dim)
        self.ffn_norm = nn.RMSNorm(dim)

    def forward(self, x):
        x = x + self.attention(self.attention_norm(x))
        return x + self.feed_forward(self.ffn_norm(x))


class Transformer(nn.Module):
    def __init__(self, dim=512, hidden=1024, n_layers=2, n_heads=4, n_kv_heads=2):
        super().__init__()
        self.n_layers = n_layers
        self.layers = nn.ModuleList(Block(dim, hidden, n_heads, n_kv_heads) for _ in range(n_layers))

    def forward(self, x):
        for layer in self.layers:
            x = layer(x)
        return x


class GroupedExperts(nn.Module):
    def __init__(self, dim, hidden, num_experts):
        super().__init__()
        self.w1 = nn.Parameter(torch.randn(num_experts, hidden, dim) * dim ** -0.5)
        self.w2 = nn.Parameter(torch.randn(num_experts, dim, hidden) * hidden ** -0.5)
        self.w3 = nn.Parameter(torch.randn(num_experts, hidden, dim) * dim ** -0.5)
        self.use_grouped_mm = True

    def forward(self, x, num_tokens_per_expert):
        outs, start = [], 0
        for e, n in enumerate(num_tokens_per_expert.tolist()):
            xe = x[start:start + n]
            outs.append((F.silu(xe @ self.w1[e].T) * (xe @ self.w3[e].T)) @ self.w2[e].T)
            start += n
        return torch.cat(outs)
