"""A model with MiniGPT's parameter structure, for the training-loop tests.

Restates the modules of src/minigpt/model.py:69-312 that own parameters --
token and position embeddings, pre-LN blocks with a fused QKV projection
(CausalSelfAttention.qkv_proj, model.py:92), an output projection and a 4x
MLP, a final LayerNorm and an lm_head tied to the token embedding
(model.py:297) -- with the same parameter names, shapes and the normal(0,
0.02) / zero-bias initialisation of model.py:301-312.  The forward pass
computes in fp32 whatever the parameter dtype (bf16 weights are widened), so
that bf16 parameters receive bf16 gradients without bf16 attention products;
attention is written out (the causal attention of model.py:132-139) so that a
rerun gives the same bits.
"""

from __future__ import annotations

import torch
from torch import nn
from torch.nn import functional as F


class _Linear(nn.Linear):
    def forward(self, x):
        return F.linear(x, self.weight.float(), None if self.bias is None else self.bias.float())


class _LayerNorm(nn.LayerNorm):
    def forward(self, x):
        return F.layer_norm(x, self.normalized_shape, self.weight.float(), self.bias.float(), self.eps)


class CausalSelfAttention(nn.Module):
    def __init__(self, n_embd: int, n_head: int):
        super().__init__()
        self.n_head = n_head
        self.qkv_proj = _Linear(n_embd, 3 * n_embd)
        self.out_proj = _Linear(n_embd, n_embd)

    def forward(self, x):
        B, T, C = x.shape
        q, k, v = self.qkv_proj(x).split(C, dim=-1)
        q, k, v = (t.view(B, T, self.n_head, C // self.n_head).transpose(1, 2).contiguous() for t in (q, k, v))
        # causal attention written out in fp32 (plain products on contiguous
        # operands, so the backward pass is deterministic)
        att = torch.matmul(q, k.transpose(-2, -1).contiguous()) * (1.0 / (C // self.n_head) ** 0.5)
        mask = torch.ones(T, T, dtype=torch.bool, device=x.device).tril()
        att = att.masked_fill(~mask, float("-inf")).softmax(dim=-1)
        y = torch.matmul(att, v)
        return self.out_proj(y.transpose(1, 2).contiguous().view(B, T, C))


class FeedForward(nn.Module):
    def __init__(self, n_embd: int):
        super().__init__()
        self.fc = _Linear(n_embd, 4 * n_embd)
        self.proj = _Linear(4 * n_embd, n_embd)

    def forward(self, x):
        return self.proj(F.gelu(self.fc(x), approximate="tanh"))


class TransformerBlock(nn.Module):
    def __init__(self, n_embd: int, n_head: int):
        super().__init__()
        self.ln_1 = _LayerNorm(n_embd)
        self.attn = CausalSelfAttention(n_embd, n_head)
        self.ln_2 = _LayerNorm(n_embd)
        self.mlp = FeedForward(n_embd)

    def forward(self, x):
        x = x + self.attn(self.ln_1(x))
        return x + self.mlp(self.ln_2(x))


class MiniGPT(nn.Module):
    def __init__(self, vocab_size=96, block_size=32, n_layer=2, n_head=4, n_embd=64, dtype=torch.float32,
                 unused_module: bool = False):
        super().__init__()
        self.token_embedding = nn.Embedding(vocab_size, n_embd)
        self.position_embedding = nn.Embedding(block_size, n_embd)
        self.blocks = nn.ModuleList(TransformerBlock(n_embd, n_head) for _ in range(n_layer))
        self.ln_f = _LayerNorm(n_embd)
        self.lm_head = _Linear(n_embd, vocab_size, bias=False)
        self.lm_head.weight = self.token_embedding.weight
        # a module whose parameters the forward pass never reads (its gradients
        # stay None in torch): exercises the optimizer's handling of them
        self.unused = _Linear(n_embd, n_embd) if unused_module else None
        self.apply(self._init_weights)
        self.to(dtype)

    @staticmethod
    def _init_weights(module):
        if isinstance(module, nn.Linear):
            nn.init.normal_(module.weight, mean=0.0, std=0.02)
            if module.bias is not None:
                nn.init.zeros_(module.bias)
        elif isinstance(module, nn.Embedding):
            nn.init.normal_(module.weight, mean=0.0, std=0.02)

    def forward(self, idx):
        pos = torch.arange(idx.shape[1], device=idx.device)
        x = self.token_embedding(idx).float() + self.position_embedding(pos).float()
        for b in self.blocks:
            x = b(x)
        return self.lm_head(self.ln_f(x))


def batches(n: int, vocab: int = 96, batch: int = 8, block: int = 32, seed: int = 1, device="cuda:0"):
    """n (input, target) pairs of token ids, the target the input shifted by one."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    out = []
    for _ in range(n):
        x = torch.randint(0, vocab, (batch, block + 1), generator=g)
        out.append((x[:, :-1].to(device), x[:, 1:].to(device)))
    return out
