"""Parameter sets of the workloads the optimizer step is measured and checked
on, as (name, shape) lists in named_parameters() order.

MiniGPT shapes follow src/minigpt/model.py:271-312 (token and position
embeddings, per block ln_1 / fused qkv_proj / out_proj / ln_2 / fc / proj with
biases, ln_f; lm_head tied to the token embedding, model.py:297, so it is not
a separate parameter).  Qwen3 shapes follow src/minigpt/qwen3_tp.py:756-800
(expected_qwen3_parameter_shapes) with a separate lm_head.
"""

from __future__ import annotations

import math
import random

Shape = tuple[int, ...]


def minigpt_shapes(vocab: int, block: int, n_layer: int, n_embd: int) -> list[tuple[str, Shape]]:
    c = n_embd
    out: list[tuple[str, Shape]] = [
        ("token_embedding.weight", (vocab, c)),
        ("position_embedding.weight", (block, c)),
    ]
    for i in range(n_layer):
        b = f"blocks.{i}"
        out += [
            (f"{b}.ln_1.weight", (c,)),
            (f"{b}.ln_1.bias", (c,)),
            (f"{b}.attn.qkv_proj.weight", (3 * c, c)),
            (f"{b}.attn.qkv_proj.bias", (3 * c,)),
            (f"{b}.attn.out_proj.weight", (c, c)),
            (f"{b}.attn.out_proj.bias", (c,)),
            (f"{b}.ln_2.weight", (c,)),
            (f"{b}.ln_2.bias", (c,)),
            (f"{b}.mlp.fc.weight", (4 * c, c)),
            (f"{b}.mlp.fc.bias", (4 * c,)),
            (f"{b}.mlp.proj.weight", (c, 4 * c)),
            (f"{b}.mlp.proj.bias", (c,)),
        ]
    out += [("ln_f.weight", (c,)), ("ln_f.bias", (c,))]
    return out


def qwen3_shapes(vocab: int = 151936, hidden: int = 4096, n_layer: int = 36, n_q: int = 32, n_kv: int = 8,
                 head_dim: int = 128, inter: int = 12288) -> list[tuple[str, Shape]]:
    qw, kvw = n_q * head_dim, n_kv * head_dim
    out: list[tuple[str, Shape]] = [("model.embed_tokens.weight", (vocab, hidden))]
    for i in range(n_layer):
        b = f"model.layers.{i}"
        out += [
            (f"{b}.self_attn.q_proj.weight", (qw, hidden)),
            (f"{b}.self_attn.k_proj.weight", (kvw, hidden)),
            (f"{b}.self_attn.v_proj.weight", (kvw, hidden)),
            (f"{b}.self_attn.o_proj.weight", (hidden, qw)),
            (f"{b}.self_attn.q_norm.weight", (head_dim,)),
            (f"{b}.self_attn.k_norm.weight", (head_dim,)),
            (f"{b}.mlp.gate_proj.weight", (inter, hidden)),
            (f"{b}.mlp.up_proj.weight", (inter, hidden)),
            (f"{b}.mlp.down_proj.weight", (hidden, inter)),
            (f"{b}.input_layernorm.weight", (hidden,)),
            (f"{b}.post_attention_layernorm.weight", (hidden,)),
        ]
    out += [("model.norm.weight", (hidden,)), ("lm_head.weight", (vocab, hidden))]
    return out


def ragged_shapes(n: int = 20000, max_elems: int = 4 * 1024 * 1024, total: int | None = 2_500_000_000,
                  seed: int = 5) -> list[tuple[str, Shape]]:
    """n tensors with log-uniform sizes over 1..max_elems (seeded), rescaled so
    the total is `total` elements when given.  Even indices are 2-D (decay
    group under the ndim >= 2 rule), odd indices 1-D (no-decay)."""
    rng = random.Random(seed)
    sizes = [max(1, int(round(math.exp(rng.uniform(0.0, math.log(max_elems)))))) for _ in range(n)]
    if total is not None:
        f = total / sum(sizes)
        sizes = [max(1, min(max_elems, int(round(s * f)))) for s in sizes]
    return [(f"t{i}", (1, s) if i % 2 == 0 else (s,)) for i, s in enumerate(sizes)]


#: the five workloads: name -> parameter set
WORKLOADS = {
    "minigpt_tiny_cpu": lambda: minigpt_shapes(vocab=96, block=128, n_layer=4, n_embd=128),
    "gpt2_small": lambda: minigpt_shapes(vocab=50304, block=1024, n_layer=12, n_embd=768),
    "gpt_1p3b": lambda: minigpt_shapes(vocab=50304, block=1024, n_layer=24, n_embd=2048),
    "qwen3_8b": lambda: qwen3_shapes(),
    "ragged_20k": lambda: ragged_shapes(),
}


def uniform_shapes(n: int, k: int) -> list[tuple[str, Shape]]:
    """k tensors of n // k elements each: a flat synthetic set for measuring
    how the step scales with its size and tensor count.  Even indices are 2-D
    (decay group), odd indices 1-D."""
    if k < 1 or n < k:
        raise ValueError(f"uniform set needs 1 <= k <= n, got n={n}, k={k}")
    m = n // k
    return [(f"u{i}", (1, m) if i % 2 == 0 else (m,)) for i in range(k)]


def shapes_of(name: str) -> list[tuple[str, Shape]]:
    """The parameter set of a named workload, or of 'uniform_<n>x<k>'
    (uniform_shapes(n, k))."""
    if name in WORKLOADS:
        return WORKLOADS[name]()
    parts = name.split("_", 1)
    if len(parts) == 2 and parts[0] == "uniform":
        n, _, k = parts[1].partition("x")
        if n.isdigit() and k.isdigit():
            return uniform_shapes(int(n), int(k))
    raise KeyError(f"unknown workload {name!r}: one of {sorted(WORKLOADS)} or uniform_<params>x<tensors>")


def numel(shape: Shape) -> int:
    n = 1
    for s in shape:
        n *= s
    return n


def count(shapes: list[tuple[str, Shape]]) -> tuple[int, int]:
    """(tensor count, parameter count)."""
    return len(shapes), sum(numel(s) for _, s in shapes)
