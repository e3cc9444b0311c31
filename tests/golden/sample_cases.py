"""Inputs of the sample() golden vectors (sample_vectors.npz), regenerated from seeds with numpy's
PCG64 so that the large-vocabulary rows need not be stored; the fixture keeps a SHA-256 of each
input array to prove that the regeneration matches what the vectors were made from.

Rows are tie-free where it matters: the 64 largest logits of every row (and the 65th) are
distinct bf16 values, so the reference's torch.topk order is fully determined by value and the
comparison tests arithmetic, not tie order. A separate group of rows keeps bf16 ties on purpose
(recorded, not asserted, by the test: torch leaves the tie order unspecified)."""
import hashlib

import numpy as np

PARAMS = [  # (temperature, top_p, top_k)
    (1.0, 1.0, 64), (0.7, 0.9, 64), (1.3, 0.95, 40), (1.0, 0.5, 64), (0.6, 1.0, 8), (2.0, 0.8, 64),
    (1.0, 1.0, 1), (0.0, 1.0, 64),
]


def bf16_bits(a: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even."""
    b = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def tie_free_rows(rows: int, V: int, seed: int, sigma: float = 2.0) -> np.ndarray:
    """bf16 bits [rows, V]: N(0, sigma) background clipped to <= 3 sigma, plus 65 distinct bf16
    values drawn from (3 sigma, 6 sigma] at random positions (the top 65, no ties among them)."""
    rng = np.random.default_rng(seed)
    out = np.empty((rows, V), np.uint16)
    lo, hi = (int(bf16_bits(np.array([v], np.float32))[0]) for v in (3 * sigma, 6 * sigma))
    for r in range(rows):
        base = bf16_bits(np.minimum(rng.standard_normal(V).astype(np.float32) * sigma, 3 * sigma))
        top = rng.choice(np.arange(lo + 1, hi + 1, dtype=np.int64), size=65, replace=False)
        where = rng.choice(V, size=65, replace=False)
        base[where] = top.astype(np.uint16)
        out[r] = base
    return out


def tied_rows(rows: int, V: int, seed: int, sigma: float = 2.0) -> np.ndarray:
    """bf16 bits [rows, V] of plain N(0, sigma) logits: at these V the top 64 hold bf16 ties."""
    rng = np.random.default_rng(seed)
    return bf16_bits(rng.standard_normal((rows, V)).astype(np.float32) * sigma)


def uniforms(n: int, seed: int) -> np.ndarray:
    return np.random.default_rng(seed).random(n, dtype=np.float32)


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


# The case groups: (name, logits maker, rows, V, seed, draws per row and parameter set)
GROUPS = [
    ("full_vocab", tie_free_rows, 4, 248320, 11, 4),
    ("small_vocab", tie_free_rows, 64, 512, 12, 40),
    ("tied", tied_rows, 8, 248320, 13, 4),
]


def group_inputs(name: str):
    """(logits bits [rows, V], u [rows, len(PARAMS), draws]) of one group."""
    for g, maker, rows, V, seed, draws in GROUPS:
        if g == name:
            return maker(rows, V, seed), uniforms(rows * len(PARAMS) * draws, seed + 1000).reshape(rows, len(PARAMS),
                                                                                                   draws)
    raise KeyError(name)
