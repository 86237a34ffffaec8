"""Independent restatements used to cross-check the oracle (test code only).

These follow different algorithms from the oracle's so a shared mistake would
have to be made twice: llama.cpp's full-sort top-k/top-p (the reference's own
second oracle, src/sampler.rs:974-1006) and brute-force reductions.
"""
import numpy as np


def stable_desc_order(p: np.ndarray) -> np.ndarray:
    """Indices sorted by p descending, equal p in ascending id order."""
    p = np.asarray(p, np.float32)
    return np.lexsort((np.arange(p.size), -p.astype(np.float64)))


def llamacpp_filtered(probs: np.ndarray, k: int, top_p: float):
    """llama_sampler_top_k_impl + llama_sampler_top_p_apply on given probs
    (sampler.rs:974-1006): sort, cut to k, renormalise (serial f32), keep the
    shortest prefix reaching top_p.  Returns [(id, weight)] sorted by id."""
    order = stable_desc_order(probs)[: min(k, len(probs))]
    ranked = [(int(i), np.float32(probs[i])) for i in order]
    tp = np.float32(top_p)
    if tp < np.float32(1.0):
        s = np.float32(0.0)
        for _, w in ranked:
            s = np.float32(s + w)
        ranked = [(i, np.float32(w / s)) for i, w in ranked]
        cum = np.float32(0.0)
        keep = len(ranked)
        for j, (_, w) in enumerate(ranked):
            cum = np.float32(cum + w)
            if cum >= tp:
                keep = j + 1
                break
        ranked = ranked[:keep]
    return sorted(ranked)


def det_logits(n: int, seed: int, scale: float) -> np.ndarray:
    """The reference tests' LCG (sampler.rs:903-914), restated with Python ints."""
    out = np.zeros(n, np.float32)
    s = seed
    M = (1 << 64) - 1
    for i in range(n):
        s = (s * 6364136223846793005 + 1442695040888963407) & M
        u = np.float32(s >> 40) / np.float32(1 << 24)
        out[i] = np.float32(np.float32(np.float32(u - np.float32(0.5)) * np.float32(2.0)) * np.float32(scale))
    return out


def shaped(shape: str, n: int, k: int, seed: int, oracle) -> np.ndarray:
    """The Flat / Peaked / Ties rows of sampler.rs:1289-1316."""
    l = oracle.det_logits(n, seed, 0.5)
    if shape == "Peaked":
        for i in range(min(8, n)):
            l[(i * 977) % n] = np.float32(18.0 - 2.0 * i)
    elif shape == "Ties":
        step = n // (k + 2)
        if step == 0:
            l[:] = 6.0
        else:
            for i in range(k + 2):
                l[i * step] = 6.0
    return l
