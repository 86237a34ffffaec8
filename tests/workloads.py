"""Seeded synthetic inputs for the five measured configurations (V = 248,320).

Shared by the parity tests and bench.py.  Every generator is a fixed numpy
PCG64 stream, so the same call gives the same bytes on every machine.  Uniforms
are j * 2^-23 with j uniform in [0, 2^23): the f32 values rand 0.9's
UniformFloat produces from 23 random bits.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

V = 248_320          # padded vocabulary of the Qwen 3.6 checkpoints (tokenizer.rs:319)
WORDS = V // 32      # allow-mask words per row


def uniforms(rng, n: int) -> np.ndarray:
    return (rng.integers(0, 1 << 23, n) * 2.0 ** -23).astype(np.float32)


@dataclass
class Workload:
    name: str
    logits: np.ndarray          # [rows, V] f32
    temperature: np.ndarray     # [rows] f64
    top_k: np.ndarray           # [rows] int
    top_p: np.ndarray           # [rows] f64
    u: np.ndarray               # [rows] f32
    mask: np.ndarray | None = None      # [rows, WORDS] u32
    drafts: np.ndarray | None = None    # [seqs, D] int32
    seqs: int = 0
    span: int = 0
    n_top: int = 0


def c1_single(seed: int = 101, greedy: bool = False, v: int = V) -> Workload:
    """C1: one row N(0, 3^2) with 16 spikes at +12; thinking defaults (or greedy)."""
    rng = np.random.default_rng(seed)
    x = rng.normal(0.0, 3.0, (1, v)).astype(np.float32)
    x[0, rng.choice(v, 16, replace=False)] = 12.0
    t = 0.0 if greedy else 1.0
    return Workload("C1" + ("-greedy" if greedy else ""), x, np.full(1, t), np.full(1, 20),
                    np.full(1, 0.95), uniforms(rng, 1))


def c2_batch(seed: int = 202, rows: int = 64, v: int = V) -> Workload:
    """C2: 64 rows N(0, 2.5^2), 8 spikes U(8, 14) each; instruct defaults."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, v), dtype=np.float32) * np.float32(2.5)
    for r in range(rows):
        x[r, rng.choice(v, 8, replace=False)] = rng.uniform(8.0, 14.0, 8).astype(np.float32)
    return Workload("C2", x, np.full(rows, 0.7), np.full(rows, 20), np.full(rows, 0.80),
                    uniforms(rng, rows))


def c3_masked(seed: int = 303, rows: int = 32, v: int = V) -> Workload:
    """C3: 32 rows N(0, 3^2) with allow-masks: a third ~1% dense in a few
    contiguous ranges, a third ~10% random, a third ~50% random; row 0 allows
    exactly one id."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, v), dtype=np.float32) * np.float32(3.0)
    allow = np.zeros((rows, v), bool)
    for r in range(rows):
        kind = r % 3
        if kind == 0:
            for _ in range(4):  # four ranges of ~0.25% each
                start = int(rng.integers(0, v - v // 400))
                allow[r, start:start + v // 400] = True
        elif kind == 1:
            allow[r] = rng.random(v) < 0.10
        else:
            allow[r] = rng.random(v) < 0.50
    allow[0] = False
    allow[0, int(rng.integers(0, v))] = True
    words = pack_mask(allow)
    return Workload("C3", x, np.full(rows, 1.0), np.full(rows, 20), np.full(rows, 0.95),
                    uniforms(rng, rows), mask=words)


def c4_verify(seed: int = 404, seqs: int = 16, depth: int = 15, v: int = V) -> Workload:
    """C4: 16 sequences x 16 positions N(0, 3^2) with 8 spikes at +12 per row; 15
    drafts per sequence, half the target argmax, half random."""
    rng = np.random.default_rng(seed)
    span = depth + 1
    rows = seqs * span
    x = rng.standard_normal((rows, v), dtype=np.float32) * np.float32(3.0)
    for r in range(rows):
        x[r, rng.choice(v, 8, replace=False)] = 12.0 + rng.uniform(0, 2, 8).astype(np.float32)
    drafts = np.zeros((seqs, depth), np.int32)
    for s in range(seqs):
        for i in range(depth):
            row = x[s * span + i]
            drafts[s, i] = int(np.argmax(row)) if rng.random() < 0.5 else int(rng.integers(0, v))
    return Workload("C4", x, np.full(rows, 1.0), np.full(rows, 20), np.full(rows, 0.95),
                    uniforms(rng, rows), drafts=drafts, seqs=seqs, span=span)


def c5_heterogeneous(seed: int = 505, rows: int = 256, v: int = V) -> Workload:
    """C5: 256 rows Student-t(3) x 2, per-row T in {0, .6, .7, 1, 1.3}, top_k in
    {1, 20, 50, 100}, top_p in {.8, .95, 1}; held_row statistics and top-20
    log-probs per row."""
    rng = np.random.default_rng(seed)
    # Student-t(3) = Z / sqrt(X/3) with X ~ chi^2(3), a sum of three squared normals
    z = rng.standard_normal((rows, v), dtype=np.float32)
    chi = np.zeros((rows, v), np.float32)
    for _ in range(3):
        n = rng.standard_normal((rows, v), dtype=np.float32)
        chi += n * n
    x = (z / np.sqrt(chi / np.float32(3.0)) * np.float32(2.0)).astype(np.float32)
    t = rng.choice([0.0, 0.6, 0.7, 1.0, 1.3], rows)
    k = rng.choice([1, 20, 50, 100], rows)
    p = rng.choice([0.8, 0.95, 1.0], rows)
    return Workload("C5", x, t, k, p, uniforms(rng, rows), n_top=20)


def pack_mask(allow: np.ndarray) -> np.ndarray:
    """[rows, n] bool -> [rows, ceil(n/32)] u32, bit t%32 of word t/32 (sampler.rs:87-93)."""
    rows, n = allow.shape
    nw = (n + 31) // 32
    a = np.zeros((rows, nw * 32), bool)
    a[:, :n] = allow
    sh = np.arange(32, dtype=np.uint64)
    w = (a.reshape(rows, nw, 32).astype(np.uint64) << sh).sum(axis=-1)
    return np.ascontiguousarray(w.astype(np.uint32))


def mask_bits(mask_row: np.ndarray, n: int) -> np.ndarray:
    """Unpack one packed allow-mask row to a bool vector of n ids (LSB-first words)."""
    w = mask_row.astype(np.uint32)
    bits = ((w[:, None] >> np.arange(32, dtype=np.uint32)[None, :]) & 1).astype(bool)
    return bits.reshape(-1)[:n]
