"""Parameter-set shapes of the benchmark and parity configurations.

The optimizer step sees a model only as the ordered list of its parameter
shapes. ``qwen3_param_shapes`` yields them in ``model.parameters()`` order of
torchure's Qwen3 (torchure/models/qwen3/qwen3.py:276-286; block layout
:243-250, attention :107-113, SwiGLU :223-225): token embedding (tied with
lm_head, so listed once), then per block q, k, v, o, q_norm, k_norm, norm1,
norm2, gate, up, down, then the final norm.
"""

from __future__ import annotations

import math

import numpy as np


def default_ffn_dim(emb_dim: int) -> int:
    """Qwen3TransformerBlock's default when ffn_dim is None (qwen3.py:247-249)."""
    return 256 * ((int(8 * emb_dim / 3) + 255) // 256)


def qwen3_param_shapes(num_layers, num_heads, num_kv_heads, emb_dim, head_dim, vocab_size,
                       ffn_dim=None) -> list[tuple[int, ...]]:
    if ffn_dim is None:
        ffn_dim = default_ffn_dim(emb_dim)
    q_out, kv_out = num_heads * head_dim, num_kv_heads * head_dim
    shapes = [(vocab_size, emb_dim)]
    for _ in range(num_layers):
        shapes += [
            (q_out, emb_dim), (kv_out, emb_dim), (kv_out, emb_dim), (emb_dim, q_out),
            (head_dim,), (head_dim,), (emb_dim,), (emb_dim,),
            (ffn_dim, emb_dim), (ffn_dim, emb_dim), (emb_dim, ffn_dim),
        ]
    shapes.append((emb_dim,))
    return shapes


# Benchmark and parity configurations (name -> Qwen3 kwargs).
CONFIGS = {
    "tiny": dict(num_layers=2, num_heads=4, num_kv_heads=2, emb_dim=256, head_dim=64,
                 vocab_size=4096, ffn_dim=768),
    "qwen3-0.6b": dict(num_layers=28, num_heads=16, num_kv_heads=8, emb_dim=1024, head_dim=128,
                       vocab_size=151936, ffn_dim=3072),
    "qwen3-0.6b-ref": dict(num_layers=28, num_heads=16, num_kv_heads=8, emb_dim=1024,
                           head_dim=128, vocab_size=151936, ffn_dim=None),
    "qwen3-4b": dict(num_layers=36, num_heads=32, num_kv_heads=8, emb_dim=2560, head_dim=128,
                     vocab_size=151936, ffn_dim=9728),
}


def shard_shapes(shapes, ranks: int, rank: int = 0) -> list[tuple[int, ...]]:
    """One rank's share of a parameter set sharded on dim 0 in ``ranks`` pieces, as
    ``torch.chunk`` splits it (FSDP2's ``Shard(0)``): pieces of ceil(d0 / ranks) rows,
    the last ones shorter or empty. Empty shares are left out."""
    if ranks < 1 or not 0 <= rank < ranks:
        raise ValueError(f"rank {rank} of {ranks}")
    out = []
    for shape in shapes:
        d0 = shape[0]
        step = -(-d0 // ranks)
        rows = max(0, min(d0, (rank + 1) * step) - rank * step)
        if rows:
            out.append((rows,) + tuple(shape[1:]))
    return out


def shapes_for(name: str) -> list[tuple[int, ...]]:
    """Shapes of a named configuration: a Qwen3 set from CONFIGS, "ragged" (the
    10,000-tensor stress list of ragged_shapes), or "<set>-shard<N>": rank 0's share of
    that set sharded on dim 0 over N ranks (one GPU's part of a sharded step)."""
    if name == "ragged":
        return ragged_shapes()
    base, sep, ranks = name.rpartition("-shard")
    if sep and ranks.isdigit():
        return shard_shapes(shapes_for(base), int(ranks))
    return qwen3_param_shapes(**CONFIGS[name])


def numel(shape) -> int:
    return int(math.prod(shape))


def ragged_shapes(n_tensors: int = 10000, max_log2: int = 24, seed: int = 5,
                  odd_frac: float = 0.3, one_d_frac: float = 0.4) -> list[tuple[int, ...]]:
    """The ragged stress list: sizes floor(exp(U(0, ln 2^max_log2))), about
    ``odd_frac`` of them forced to a length that is not a multiple of 8, and
    ``one_d_frac`` of them 1-D (no weight decay); the rest are 2-D [rows, 8k+r]
    shaped so that their numel is the drawn size."""
    rng = np.random.Generator(np.random.PCG64(seed))
    sizes = np.floor(np.exp(rng.uniform(0.0, max_log2 * math.log(2.0), n_tensors))).astype(np.int64)
    sizes = np.maximum(sizes, 1)
    odd = rng.uniform(size=n_tensors) < odd_frac
    up8 = (sizes + 7) // 8 * 8
    bump = sizes + 1 + rng.integers(0, 7, n_tensors)
    sizes = np.where(odd, np.where(sizes % 8 == 0, bump, sizes), up8)
    one_d = rng.uniform(size=n_tensors) < one_d_frac
    shapes = []
    for n, is1 in zip(sizes.tolist(), one_d.tolist()):
        shapes.append((n,) if is1 else (1, n))
    return shapes
