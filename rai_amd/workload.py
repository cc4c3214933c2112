"""Synthetic workloads: model shapes and prompts of the benchmarked configurations.

Prompts are token-id sequences (no tokenizer): uniform random ids, or a
"copy-heavy" sequence in which about half of the positions are copies of
earlier spans (span length uniform in [8, 32]) and the rest uniform random.
"""
from __future__ import annotations

import numpy as np

# Llama-family shapes of the benchmarked configurations.
TINYLLAMA = dict(hidden_size=2048, num_layers=22, num_heads=32, num_kv_heads=4, head_dim=64,
                 intermediate_size=5632, vocab_size=32000, rope_theta=10000.0, norm_eps=1e-5)
MISTRAL_7B = dict(hidden_size=4096, num_layers=32, num_heads=32, num_kv_heads=8, head_dim=128,
                  intermediate_size=14336, vocab_size=32000, rope_theta=10000.0, norm_eps=1e-5)
OLMOE = dict(hidden_size=2048, num_layers=16, num_heads=16, num_kv_heads=16, head_dim=128,
             intermediate_size=1024, vocab_size=50304, rope_theta=10000.0, norm_eps=1e-5,
             num_experts=64, experts_per_token=8, norm_topk_prob=False)

# W4A8 GEMV sweep shapes (rows x cols).
GEMV_SHAPES = [(4096, 4096), (14336, 4096), (4096, 14336), (32000, 4096)]
GEMV_TOKENS = [1, 5, 9, 17, 512]


def uniform_prompt(n: int, vocab: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return rng.integers(0, vocab, size=n, dtype=np.int64).astype(np.uint32)


def copy_heavy_prompt(n: int, vocab: int, seed: int, copy_frac: float = 0.5,
                      span_lo: int = 8, span_hi: int = 32) -> np.ndarray:
    """About `copy_frac` of the positions copy an earlier span (length U[lo, hi])."""
    rng = np.random.default_rng(seed)
    out = np.empty(n, np.uint32)
    i = 0
    while i < n:
        span = int(rng.integers(span_lo, span_hi + 1))
        if i >= span_hi and rng.random() < copy_frac:
            src = int(rng.integers(0, i - span + 1))
            take = min(span, n - i)
            out[i:i + take] = out[src:src + take]
        else:
            take = min(span, n - i)
            out[i:i + take] = rng.integers(0, vocab, size=take)
        i += take
    return out


def gemv_operands(rows: int, cols: int, m: int, gs: int, seed: int):
    """Random int4 weights (symmetric-RTN-like f16 params) and N(0,1) inputs."""
    rng = np.random.default_rng(seed)
    groups = -(-cols // gs)
    nib = rng.integers(0, 256, size=rows * cols // 2, dtype=np.uint8)
    scale = (np.abs(rng.normal(0.0, 0.02, size=(rows, groups))) / 7.0 + 1e-4).astype(np.float16)
    zero = (-8.0 * scale.astype(np.float64)).astype(np.float16)
    params = np.empty((rows, groups, 2), np.float16)
    params[:, :, 0] = scale
    params[:, :, 1] = zero
    x = rng.normal(0.0, 1.0, size=(m, cols)).astype(np.float32)
    return nib, params.view(np.uint8).reshape(-1), x
