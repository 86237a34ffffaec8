"""The claim behind the finalizer's check for controlled rows (order_settled,
draw_settled in xs_sampler.hip), tested by brute force on the CPU oracle.

The claim: when the decisions of a draw made with one softmax denominator S
clear the stated margins, every denominator D within the serial sum's error
bound of the exact sum draws the same token -- in particular the reference's
serial f32 sum (sampler.rs:301-305).  The margins below restate the kernel's
(the robust gap between consecutive e, the top-p cut and the draw against
(k + j + 4) and (k + keep + 4) 2^-23 of the values involved with 2 % to
spare, plus subnormal and negligible-entry slack); the test then draws each row with S and with
many D across the whole bound (the oracle's SUM_GIVEN), uniforms packed
around every cumulative-weight boundary, and requires: wherever the margins
pass, every D gives S's token.  It also requires that the margins fail near
every boundary (so the check is not vacuous) and that they pass for most
uniforms (so it is not a blanket refusal).
"""
import numpy as np
import pytest

from tests import workloads

NEG = 2.0 ** -65


def _f32(x):
    return np.float32(x)


def _chain(w):
    out, acc = [], np.float32(0.0)
    for t in w:
        acc = np.float32(acc + t)
        out.append(acc)
    return out


def _draw_model(e, S, k, top_p, u):
    """The finalizer's draw given the e of the top-k (p desc) and S, with the
    margins it checks; returns (index, settled, the cumulative weights below
    the total)."""
    p = (e / np.float32(S)).astype(np.float32)
    renorm = top_p < 1.0
    sumc = np.float32(1.0)
    w = p.copy()
    if renorm:
        acc = np.float32(-0.0)
        for t in w:
            acc = np.float32(acc + t)
        sumc = acc
        w = (w / sumc).astype(np.float32)
    c = _chain(w)
    keep, found = k, False
    if renorm:
        for j in range(k):
            if c[j] >= np.float32(top_p):
                keep, found = j + 1, True
                break
    tot = c[keep - 1]
    x = np.float32(np.float32(u) * tot)
    cum = [c[j] if j < keep - 1 else tot for j in range(k - 1)]
    idx = sum(1 for t in cum if t <= x)
    uu = 2.0 ** -23 * 1.02
    sl = (2.0 * k + 8.0) * 2.0 ** -148 * float(S) + 2.0 ** -50  # (the p's subnormal ulps, 1 / sum <= S)
    ok = True
    if renorm:
        j1 = keep - 1 if found else k - 1
        c1 = float(c[j1])
        m1 = uu * (k + j1 + 4) * c1 + sl
        ok &= (c1 - float(top_p) > m1) if found else (float(top_p) - c1 > m1)
        if found and keep >= 2:
            c0 = float(c[keep - 2])
            ok &= float(top_p) - c0 > uu * (k + keep + 2) * c0 + sl
    mt = uu * (k + keep + 4) * float(tot) + sl
    if idx >= 1:
        c0 = float(c[idx - 1])
        ok &= float(x) - c0 > uu * (k + idx + 3) * c0 + mt
    if idx < keep - 1:
        c1 = float(c[idx])
        ok &= c1 - float(x) > uu * (k + idx + 4) * c1 + mt
    return idx, ok, [float(t) / float(tot) for t in c[:keep - 1]]


def _order_model(e_sel, k, S, enc):
    """order_settled for a row whose selection (K' = k + 1, logit order) is e_sel."""
    thr = S * (1.01 + enc * 2.0 ** -24 * 1.02) * 2.0 ** -148

    def robust(a, b):
        if a == b:
            return True
        g = float(a) - float(b)
        return g > 2.0 ** -21 * float(a) and g > thr
    return all(robust(e_sel[i], e_sel[i + 1]) for i in range(len(e_sel) - 1) if e_sel[i] >= NEG)


@pytest.mark.parametrize("seed", range(4))
def test_settled_draws_are_denominator_free(oracle, seed):
    rng = np.random.default_rng(4400 + seed)
    v = 2048
    k = int(rng.choice([2, 5, 20, 40]))
    T = float(rng.choice([0.7, 1.0, 1.3]))
    top_p = float(rng.choice([0.5, 0.8, 0.95, 1.0]))
    x = (rng.normal(0, 3, v)).astype(np.float32)
    if seed % 2:
        x[rng.integers(0, v, 6)] = rng.uniform(8, 14, 6).astype(np.float32)
    allow = rng.random(v) < 0.5
    mask = workloads.pack_mask(allow[None, :])[0]
    ctl = oracle.Ctl(allowed=mask)
    # the row's selection, e and exact sum, from the oracle's own numbers
    o64 = oracle.sample_controlled(x, v, T, k, top_p, u=0.0, ctl=ctl, sum_mode=oracle.SUM_F64)
    oseq = oracle.sample_controlled(x, v, T, k, top_p, u=0.0, ctl=ctl, sum_mode=oracle.SUM_SEQ_F32)
    S = np.float32(o64.ssum)
    vals = np.where(allow, x, -np.inf).astype(np.float32)
    s = (vals * _f32(1.0 / T)).astype(np.float32) if T != 1.0 else vals
    ms = s.max()
    order = np.lexsort((np.arange(v), -s))[:k + 1]
    e_sel = np.array([oracle.exp(float(_f32(s[i] - ms))) for i in order], np.float32)
    assert _order_model(e_sel, k, float(S), v)  # continuous logits: no near-ties at this size
    e = e_sel[:k]
    # denominators across the serial sum's bound, the serial sum itself among them
    delta = v * 2.0 ** -24
    Ds = [np.float32(oseq.ssum)] + [np.float32(float(S) * (1.0 + f * delta)) for f in rng.uniform(-1, 1, 24)]
    # uniforms packed around every cumulative-weight boundary of the S draw, and random ones
    _, _, bounds = _draw_model(e, S, k, top_p, 0.0)
    us = list(rng.random(200).astype(np.float32))
    for base in bounds:
        # every ulp next to the boundary, then wider (the margins span about
        # (2k + 8) 2^-23 of the total)
        for d in list(range(-12, 13)) + list(range(-400, 401, 5)):
            us.append(np.float32(min(max(base + d * 2.0 ** -24, 0.0), 1 - 2.0 ** -24)))
    n_settled = n_unsettled = 0
    for u in us:
        idx, settled, _ = _draw_model(e, S, k, top_p, u)
        if not settled:
            n_unsettled += 1
            continue
        n_settled += 1
        tok = oracle.sample_controlled(x, v, T, k, top_p, u=float(u), ctl=ctl, sum_mode=oracle.SUM_GIVEN,
                                       s_given=float(S)).token
        for D in Ds:
            td = oracle.sample_controlled(x, v, T, k, top_p, u=float(u), ctl=ctl, sum_mode=oracle.SUM_GIVEN,
                                          s_given=float(D)).token
            assert td == tok, (seed, float(u), float(D), td, tok)
    assert n_unsettled > 0 and n_settled > 300, (n_settled, n_unsettled)
