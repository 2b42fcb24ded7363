"""Seeded synthetic knowledge graphs and workloads for the five benchmark
configurations (C1..C5) of the FlashLog propagation hot path.

The reference ships no datasets or fixtures for this path, so parity tests and
the benchmark run on these generated graphs.  Generator: numpy
``Generator(PCG64(1234 + cfg))`` (1234 is the reference's default ``--seed``,
src/main.py:1028).  Degree and relation laws follow the configuration text:
uniform, or Zipf(s) -- p(k) proportional to rank(k)^-s over a seeded permutation.
Duplicate triples are kept (i.i.d. draws).
"""
from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class GraphConfig:
    name: str
    entities: int
    relations: int          # base relations R (inverses are implicit: n = 2R+1)
    triples: int
    rel_law: float          # 0 = uniform, else Zipf exponent over relations
    deg_law: float          # 0 = uniform, else Zipf exponent over entities
    batch: int              # queries per call (eval)
    channels: int = 3       # N (the model's L): BL = batch * channels
    hops: int = 3           # T
    c1: int = 1000
    c2: int = 400           # K = c2 // 2 edges per (source, query-channel, direction)
    use_topk: bool = True


CONFIGS = {
    1: GraphConfig("C1", 3_000, 12, 28_000, 0.0, 0.0, 32, use_topk=False),
    2: GraphConfig("C2", 41_000, 11, 87_000, 0.0, 1.1, 32),
    3: GraphConfig("C3", 14_500, 237, 272_000, 1.0, 1.1, 32),
    4: GraphConfig("C4", 123_000, 37, 1_080_000, 0.0, 1.2, 32),
    5: GraphConfig("C5", 4_600_000, 822, 20_000_000, 1.0, 1.3, 256),
}


def _zipf_probs(k, s, rng):
    ranks = np.arange(1, k + 1, dtype=np.float64)
    p = ranks ** (-s)
    p /= p.sum()
    return p[rng.permutation(k)]


def make_graph(cfg_id, scale=1.0, seed=None):
    """Returns (h, r, t) int64 arrays and the config.  ``scale`` < 1 shrinks
    entities and triples proportionally (for fast CPU tests)."""
    cfg = CONFIGS[cfg_id]
    rng = np.random.Generator(np.random.PCG64(1234 + cfg_id if seed is None else seed))
    E = max(8, int(round(cfg.entities * scale)))
    M = max(8, int(round(cfg.triples * scale)))
    R = cfg.relations
    if cfg.rel_law > 0:
        r = rng.choice(R, size=M, p=_zipf_probs(R, cfg.rel_law, rng))
    else:
        r = rng.integers(0, R, size=M)
    if cfg.deg_law > 0:
        pe = _zipf_probs(E, cfg.deg_law, rng)
        h = rng.choice(E, size=M, p=pe)
        t = rng.choice(E, size=M, p=pe)
    else:
        h = rng.integers(0, E, size=M)
        t = rng.integers(0, E, size=M)
    return h.astype(np.int64), r.astype(np.int64), t.astype(np.int64), E, R


def make_queries(h, r, t, R, B, rng, return_index=False):
    """B queries drawn from the triples; each is forward (h, r) or inverse
    (t, r + R) with probability 1/2 (the eval batches of src/main.py:717-720).
    return_index: also the triples' indices (the edge ids a training step
    hides, src/main.py:887-890); the draws are the same either way."""
    idx = rng.integers(0, h.shape[0], size=B)
    inv = rng.random(B) < 0.5
    src = np.where(inv, t[idx], h[idx])
    rel = np.where(inv, r[idx] + R, r[idx])
    tgt = np.where(inv, h[idx], t[idx])
    out = (src.astype(np.int64), rel.astype(np.int64), tgt.astype(np.int64))
    return out + (idx.astype(np.int64),) if return_index else out


def training_queries(h, r, t, R, idx):
    """The queries a training batch of triples idx propagates without
    wot_inv (src/dataloader.py:114-122): each triple forward (h, r -> t),
    then inverse (t, r + R -> h), interleaved."""
    src = np.stack([h[idx], t[idx]], 1).reshape(-1)
    rel = np.stack([r[idx], r[idx] + R], 1).reshape(-1)
    tgt = np.stack([t[idx], h[idx]], 1).reshape(-1)
    return src.astype(np.int64), rel.astype(np.int64), tgt.astype(np.int64)


def make_attention(B, L, n, hops, rng):
    """Per-hop attention w_t = softmax(N(0,1) logits) of shape [hops, B, L, n]
    (the DRUM model's softmax(w_all[:, t] / tau_1) with tau_1 = 1)."""
    logits = rng.standard_normal((hops, B, L, n)).astype(np.float32)
    logits -= logits.max(-1, keepdims=True)
    e = np.exp(logits)
    return (e / e.sum(-1, keepdims=True)).astype(np.float32)
