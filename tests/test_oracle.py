"""The CPU oracle against the reference's known answers, closed forms and
independent restatements.  No GPU; runs in the default `-m "not gpu"` suite.

Each test names the reference test or the mathematical fact that pins it.
"""
import decimal
import math
import os
import subprocess

import numpy as np
import pytest

from tests import refimpl

STATUS = {"NAN": 1, "NO_FINITE": 2, "MASK_SHORT": 3, "FORCE_OOR": 4, "ZERO_WEIGHT": 5,
          "NARROW": 6}
UNIFORMS = [0.0, 0.25, 0.5, 0.75, 1.0 - 2.0 ** -23, 0.123456789]


def ctl_of(case, o):
    return o.Ctl(allowed=case.get("allowed"), banned=tuple(case.get("banned", ())),
                 bias=tuple(tuple(b) for b in case.get("bias", ())), pull=case.get("pull"),
                 force=case.get("force"))


# --- exp -------------------------------------------------------------------

def cr_exp_decimal(x: float) -> np.float32:
    """binary32 rounding of exp(x) evaluated at 60 digits (the closed form)."""
    decimal.getcontext().prec = 60
    v = decimal.Decimal(float(x)).exp()
    big = decimal.Decimal(2) ** 128  # inf rounds like the binary32 step past FLT_MAX
    if v >= big - decimal.Decimal(2) ** 103:
        return np.float32(np.inf)
    f = np.float32(min(float(v), 3.4028234663852886e38))
    cands = [np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))]
    cands = [c for c in cands if np.isfinite(c)]
    return min(cands, key=lambda c: abs(decimal.Decimal(float(c)) - v))


def test_exp_matches_60_digit_decimal_on_random_and_edge_inputs(oracle):
    rng = np.random.default_rng(7)
    xs = list(rng.uniform(-104, 89, 400).astype(np.float32))
    xs += list(rng.uniform(-1, 1, 100).astype(np.float32))
    xs += [0.0, -0.0, 1.0, -1.0, 88.72283, 88.7228394, -87.33655, -103.27893, -103.97207,
           -103.9721, 1e-30, -1e-30, np.float32(2.0 ** -149)]
    for x in xs:
        x = np.float32(x)
        got = oracle.exp(x)
        want = cr_exp_decimal(x)
        assert np.float32(got) == want, (float(x), got, float(want))


def test_exp_special_values(oracle):
    assert oracle.exp(0.0) == 1.0
    assert oracle.exp(float("-inf")) == 0.0
    assert oracle.exp(float("inf")) == float("inf")
    assert math.isnan(oracle.exp(float("nan")))
    assert oracle.exp(-104.5) == 0.0
    assert oracle.exp(89.5) == float("inf")
    # exp(x) for x just above ln(2^-150) rounds to the smallest subnormal
    assert oracle.exp(-103.9) == np.float32(2.0 ** -149)


def test_exp_strided_sweep_is_correctly_rounded(oracle):
    """A 1-in-4099 stride of every binary32 in [-104, 89] against x87 expl.
    (The exhaustive sweep, stride 1, also reports 0 mismatches and 0 inputs
    within 2^-58 of a rounding boundary.)"""
    exe = os.path.join(os.path.dirname(oracle.LIB_PATH), "exp_sweep")
    out = subprocess.run([exe, "4099", "4"], capture_output=True, text=True)
    first = out.stdout.splitlines()[0]
    assert "mismatch 0 hard 0" in first, out.stdout


# --- argmax ----------------------------------------------------------------

def test_argmax_first_maximal_index_brute_force(oracle):
    rng = np.random.default_rng(3)
    for _ in range(200):
        n = int(rng.integers(1, 300))
        v = rng.integers(-3, 4, n).astype(np.float32)  # many ties
        st, tok = oracle.argmax(v)
        assert st == 0 and tok == int(np.argmax(v))  # numpy: first occurrence


def test_argmax_errors(oracle):
    assert oracle.argmax([1.0, float("nan")])[0] == STATUS["NAN"]
    assert oracle.argmax([float("-inf")] * 3)[0] == STATUS["NO_FINITE"]
    assert oracle.argmax([-0.0, 0.0]) == (0, 0)
    assert oracle.argmax([float("-inf"), float("inf"), float("inf")]) == (0, 1)


# --- the reference's sample_controlled known answers ------------------------

def test_reference_sampler_cases(golden, oracle):
    for case in golden["sampler"]:
        enc = case["enc"]
        us = UNIFORMS if case.get("any_uniform") or "expect_in" in case else [0.5]
        for u in us:
            d = oracle.sample_controlled(case["logits"], enc, case["T"], case["k"], case["p"],
                                         u=u, ctl=ctl_of(case, oracle))
            if "expect_error" in case:
                assert d.status == STATUS[case["expect_error"]], (case["name"], d)
            elif "expect" in case:
                assert (d.status, d.token) == (0, case["expect"]), (case["name"], u, d)
            else:
                assert d.status == 0 and d.token in case["expect_in"], (case["name"], u, d)


def test_wide_nan_errors_on_both_paths(golden, oracle):
    c = golden["wide_nan"]
    v = np.full(c["n"], c["fill"], np.float32)
    for i, x in c["set"]:
        v[i] = x
    for T in (0.0, 1.0):
        assert oracle.sample_controlled(v, c["n"], T, 20, 1.0).status == STATUS["NAN"]


def test_top_k_desc_cases(golden, oracle):
    for case in golden["top_k_desc"]:
        if "probs" in case:
            p = case["probs"]
        elif "ascending" in case:
            p = np.arange(case["ascending"], dtype=np.float32)
        else:
            p = np.full(case["n"], case["fill"], np.float32)
            p[: case["head"][0]] = case["head"][1]
            p[case["nan_at"]] = np.nan
        st, got = oracle.top_k_desc(p, case["k"])
        if "expect_error" in case:
            assert st == STATUS[case["expect_error"]]
        else:
            assert st == 0
            assert [(np.float32(w), i) for w, i in got] == \
                [(np.float32(w), i) for w, i in case["expect"]], case["name"]


def test_top_k_boundary_ties_keep_the_lowest_ids(golden, oracle):
    c = golden["boundary_ties"]
    for k in c["ks"]:
        v = np.full(c["n"], c["low"], np.float32)
        v[: k + 1] = c["tie"]
        assert [i for _, i in oracle.top_k_desc(v, k)[1]] == list(range(k))
        v = np.full(c["n"], c["low"], np.float32)
        v[c["late_start"]: c["late_start"] + k + 1] = c["tie"]
        assert [i for _, i in oracle.top_k_desc(v, k)[1]] == \
            list(range(c["late_start"], c["late_start"] + k))


def test_top_k_desc_equals_brute_force_stable_sort(oracle):
    rng = np.random.default_rng(11)
    for _ in range(200):
        n = int(rng.integers(5, 400))
        k = int(rng.integers(1, n))
        p = (rng.integers(0, 6, n) / 8.0).astype(np.float32)  # heavy ties
        st, got = oracle.top_k_desc(p, k)
        order = refimpl.stable_desc_order(p)[:k]
        assert st == 0 and [i for _, i in got] == order.tolist()


# --- top-p and the candidate set --------------------------------------------

def test_top_p_measures_mass_renormalized(golden, oracle):
    for case in golden["top_p_renormalized"]:
        logits = np.log(np.asarray(case["weights"], np.float32))
        probs, _, _ = oracle.softmax_in_place(logits, 1.0)
        if "top3_mass" in case:
            top3 = np.float32(0)
            for x in probs[:3]:
                top3 = np.float32(top3 + x)
            assert abs(top3 - case["top3_mass"]) < 1e-5
        st, cands = oracle.candidate_set(probs, case["k"], case["p"])
        assert st == 0
        assert sorted(i for w, i in cands if w > 0) == case["expect_ids"], case["name"]


def test_top_p_of_zero_keeps_only_the_top_candidate(golden, oracle):
    c = golden["top_p_zero"]
    l = oracle.det_logits(*c["det_logits"])
    probs, _, _ = oracle.softmax_in_place(l, c["T"])
    want = refimpl.llamacpp_filtered(probs, c["k"], c["p"])
    assert len(want) == c["expect_len"]
    st, cands = oracle.candidate_set(probs, c["k"], c["p"])
    got = [(i, w) for w, i in cands if w > 0]
    assert st == 0 and len(got) == 1 and got[0][0] == want[0][0]
    assert abs(got[0][1] - want[0][1]) < 1e-6


def test_candidate_set_matches_llamacpp_filtering(golden, oracle):
    m = golden["llamacpp_matrix"]
    for n, scale in m["shapes"]:
        for seed in m["seeds"]:
            for k, p, T in m["params"]:
                l = oracle.det_logits(n, seed, scale)
                probs, _, _ = oracle.softmax_in_place(l, T)
                want = refimpl.llamacpp_filtered(probs, k, p)
                st, cands = oracle.candidate_set(probs, k, p)
                got = sorted((i, w) for w, i in cands if w > 0)
                assert st == 0 and [i for i, _ in want] == [i for i, _ in got], (n, seed, k, p)
                for (i, a), (_, b) in zip(want, got):
                    assert abs(a - b) <= m["rel_tol"] * abs(a)


@pytest.mark.parametrize("shape", ["Flat", "Peaked", "Ties"])
def test_candidate_sets_across_the_reference_matrix(shape, oracle):
    """sampler.rs:1359-1486: widths from a toy row to the padded vocabulary, k from
    greedy-collapse to wider than the row, p from biting to no-op."""
    for n in (64, 2048, 248_320):
        for k in (1, 20, 64):
            for p in (0.5, 0.95, 1.0):
                l = refimpl.shaped(shape, n, k, 90210, oracle)
                probs, _, _ = oracle.softmax_in_place(l, 1.0)
                st, cands = oracle.candidate_set(probs, k, p)
                ours = sorted(i for w, i in cands if w > 0)
                want = [i for i, _ in refimpl.llamacpp_filtered(probs, k, p)]
                assert st == 0 and ours == want, (shape, n, k, p)


def test_padded_mass_sums_to_one(golden, oracle):
    c = golden["padded_mass"]
    probs, _, _ = oracle.softmax_in_place(c["values"], 1.0)
    st, cands = oracle.candidate_set(probs, c["k"], c["p"])
    total = np.float32(0)
    for w, _ in cands:
        total = np.float32(total + w)
    assert st == 0 and abs(total - 1.0) < c["tol"]


def test_softmax_against_f64_closed_form(oracle):
    rng = np.random.default_rng(5)
    for T in (1.0, 0.7, 1.3):
        x = rng.normal(0, 3, 4096).astype(np.float32)
        s = x.astype(np.float32) * np.float32(1.0 / T) if T != 1.0 else x
        d = (s - s.max()).astype(np.float32)  # the reference subtracts in f32 (:303)
        ref = np.exp(d.astype(np.float64))
        ref /= ref.sum()
        got, mx, _ = oracle.softmax_in_place(x, T, oracle.SUM_F64)
        assert mx == s.max()
        np.testing.assert_allclose(got, ref, rtol=4e-7, atol=0)
        got_seq, _, _ = oracle.softmax_in_place(x, T, oracle.SUM_SEQ_F32)
        np.testing.assert_allclose(got_seq, ref, rtol=2e-4, atol=0)


def test_serial_sum_spread_on_the_workload_rows(oracle):
    """How far the reference's serial f32 denominator (controlled rows,
    sampler.rs:301-305) lies from the exact sum of the same f32 terms on rows
    shaped like C2, C3 and C5: ~1e-4 and more, far past the 1e-5 bar, so a
    device that used the exact sum on controlled rows at top_p >= 1 would miss
    the reference's weights; the serial sum has to be reproduced itself."""
    from tests import workloads
    spread = {}
    for name, wl in (("C2", workloads.c2_batch(rows=8)), ("C3", workloads.c3_masked(rows=9)),
                     ("C5", workloads.c5_heterogeneous(rows=8))):
        rows, V = wl.logits.shape
        T = np.where(wl.temperature > 0, wl.temperature, 1.0)  # every row stochastic here
        kw = dict(mask=wl.mask) if wl.mask is not None else {}
        seq = oracle.sample_rows(wl.logits, V, T, 20, 1.0, wl.u, sum_mode=oracle.SUM_SEQ_F32, **kw)
        ex = oracle.sample_rows(wl.logits, V, T, 20, 1.0, wl.u, sum_mode=oracle.SUM_F64, **kw)
        ok = (seq["status"] == 0) & (ex["status"] == 0)
        rel = np.abs(seq["ssum"][ok].astype(np.float64) / ex["ssum"][ok] - 1.0)
        spread[name] = (float(np.median(rel)), float(rel.max()))
    print("serial f32 sum vs exact (median, max):", spread)
    assert spread["C2"][0] > 1e-5 and spread["C3"][1] > 1e-5
    assert all(mx < 5e-3 for _, mx in spread.values())


def test_serial_f32_fold_stops_at_two_to_the_24(oracle):
    """SUM_SEQ_F32 is the reference's one-at-a-time f32 fold (sampler.rs:301-305):
    2^25 equal logits make 2^25 terms of exactly 1, and a serial f32 sum stops
    at 2^24 (2^24 + 1 rounds to even, back to 2^24); a pairwise or exact sum
    reaches 2^25, so either would fail here."""
    n = 1 << 25
    _, mx, ssum = oracle.softmax_in_place(np.zeros(n, np.float32), 1.0, oracle.SUM_SEQ_F32)
    assert mx == 0.0 and ssum == 2.0 ** 24
    _, _, exact = oracle.softmax_in_place(np.zeros(n, np.float32), 1.0, oracle.SUM_F64)
    assert exact == 2.0 ** 25


def test_serial_f32_fold_runs_in_id_order(oracle):
    """The fold adds the terms in id order from +0: a row whose max comes
    first absorbs every later term below half an ulp of 1 (exp(-20) < 2^-25),
    so its sum is exactly 1; the same terms with the max last accumulate first
    and end near 1 + n exp(-20).  A reversed fold swaps the two results.  The
    second value is checked against numpy's cumsum, a sequential f32 loop of
    its own."""
    n = 200_000
    first = np.concatenate([[0.0], np.full(n, -20.0)]).astype(np.float32)
    last = np.concatenate([np.full(n, -20.0), [0.0]]).astype(np.float32)
    _, _, s_first = oracle.softmax_in_place(first, 1.0, oracle.SUM_SEQ_F32)
    _, _, s_last = oracle.softmax_in_place(last, 1.0, oracle.SUM_SEQ_F32)
    t = np.float32(oracle.exp(-20.0))
    assert s_first == 1.0
    want = np.cumsum(np.concatenate([np.full(n, t, np.float32), [np.float32(1.0)]]),
                     dtype=np.float32)[-1]
    assert s_last == want and abs(s_last - (1.0 + n * float(t))) < 1e-3


def _lse_of(m: float, denom: float) -> float:
    return float(np.float64(m) + math.log(denom))


def test_held_row_fold_of_equal_terms_after_the_max(oracle):
    """held_row's f64 fold (generate.rs:1931-1932) in id order from the max:
    once the max's term 1.0 is in, each later term t lands on the 2^-52 grid
    of [1, 2), so n equal terms t >= 2^-53 after the max give exactly
    1 + n * rint(2^52 t) * 2^-52, and terms below 2^-53 are absorbed (the
    denominator stays exactly 1, where an exact sum would not).  An exact or
    pairwise sum differs from both closed forms."""
    n = 100_000
    for d in (-14.0, -20.0, -30.0, -36.0):   # t = exp(d) >= 2^-53, n t < 1
        row = np.concatenate([[5.0], np.full(n, 5.0 + d)]).astype(np.float32)
        dd = float(np.float32(np.float32(5.0 + d) - np.float32(5.0)))
        t = math.exp(dd)
        units = round(t * 2.0 ** 52)  # t * 2^52 is not a half-integer for these t
        denom = 1.0 + n * units * 2.0 ** -52
        assert denom < 2.0
        st, mx, lse = oracle.held_row(row, row.size)
        assert st == 0 and mx == 5.0
        assert lse == _lse_of(5.0, denom), (d, lse, _lse_of(5.0, denom))
        assert lse != _lse_of(5.0, math.fsum([1.0] + [t] * n)) or units * 2.0 ** -52 == t
    for d in (-37.0, -38.5, -40.0):          # t < 2^-53: absorbed
        row = np.concatenate([[5.0], np.full(n, 5.0 + d)]).astype(np.float32)
        st, mx, lse = oracle.held_row(row, row.size)
        assert st == 0 and lse == 5.0  # ln(1) = 0 exactly
        assert _lse_of(5.0, math.fsum([1.0] + [math.exp(d)] * n)) != 5.0


def test_held_row_fold_with_the_max_last(oracle):
    """The same terms with the max at the end: the fold sums them first (in f64,
    serially: a Python float loop is such a fold) and adds 1.0 last, so terms
    below 2^-53 now count.  Distinguishes the id-order fold from a reversed
    one, which would absorb them."""
    n = 50_000
    for d in (-40.0, -20.0):
        row = np.concatenate([np.full(n, 5.0 + d), [5.0]]).astype(np.float32)
        t = math.exp(float(np.float32(np.float32(5.0 + d) - np.float32(5.0))))
        acc = 0.0
        for _ in range(n):
            acc += t
        acc += 1.0
        st, mx, lse = oracle.held_row(row, row.size)
        assert st == 0 and mx == 5.0 and lse == _lse_of(5.0, acc)
        assert acc > 1.0


# --- the draw ----------------------------------------------------------------

def test_weighted_index_boundaries(oracle):
    # cum = [0.5]; x = u * 1.0.  partition_point(cum <= x): x == 0.5 -> index 1
    assert oracle.weighted_index([0.5, 0.5], 0.5) == (0, 1)
    assert oracle.weighted_index([0.5, 0.5], 0.5 - 2 ** -23) == (0, 0)
    # u = 0 picks the first positive weight; zero weights are unreachable
    assert oracle.weighted_index([0.0, 0.0, 0.3, 0.7], 0.0) == (0, 2)
    for u in UNIFORMS:
        assert oracle.weighted_index([0, 0, 1.0, 0, 0], u) == (0, 2)
    assert oracle.weighted_index([0.0, 0.0], 0.3)[0] == STATUS["ZERO_WEIGHT"]
    # three equal weights: x = u*3 against cum [1, 2]
    assert oracle.weighted_index([1, 1, 1], 1 / 3 + 2 ** -23)[1] == 1
    assert oracle.weighted_index([1, 1, 1], 2 / 3 + 2 ** -22)[1] == 2


def test_draw_frequencies_follow_llamacpp_semantics(golden, oracle):
    c = golden["draw_frequencies"]
    l = oracle.det_logits(*c["det_logits"])
    probs, _, _ = oracle.softmax_in_place(l, c["T"])
    want = refimpl.llamacpp_filtered(probs, c["k"], c["p"])
    assert len(want) < c["k"]
    mass = sum(float(w) for _, w in want)
    rng = np.random.default_rng(5150)
    us = (rng.integers(0, 1 << 23, c["draws"]) * 2.0 ** -23).astype(np.float32)
    rows = np.broadcast_to(l, (c["draws"], l.size))
    out = oracle.sample_rows(rows, l.size, c["T"], c["k"], c["p"], us, nthreads=4)
    assert (out["status"] == 0).all()
    hist = np.bincount(out["token"].astype(np.int64), minlength=l.size) / c["draws"]
    wanted = {i: float(w) / mass for i, w in want}
    for i in range(l.size):
        if i in wanted:
            assert abs(hist[i] - wanted[i]) < c["tol"], (i, hist[i], wanted[i])
        else:
            assert hist[i] == 0.0


# --- verify walk, drafter confidence, scoring --------------------------------

def test_accept_drafts_walks(golden, oracle):
    g = golden["accept_drafts"]
    for case in g["cases"]:
        samples = case["samples"]
        eog = [1 if s >= g["eog_at_or_above"] else 0 for s in samples]
        budget = case["budget"] if case["budget"] is not None else 1 << 62
        st, m, com, calls = oracle.accept_drafts(case["drafts"], budget, samples, eog)
        assert (st, m, com, calls) == (0, case["m"], case["committed"], case["calls"]), \
            case["name"]


def test_accept_drafts_errors_only_when_the_walk_reaches_the_row(oracle):
    drafts, samples = [10, 20, 30], [10, 99, 30, 40]
    # row 3 is corrupt, but the walk stops at the mismatch in row 1
    st, m, com, calls = oracle.accept_drafts(drafts, 99, samples, [0] * 4, [0, 0, 0, 1])
    assert (st, m, com, calls) == (0, 1, [10, 99], 2)
    st, *_ = oracle.accept_drafts(drafts, 99, samples, [0] * 4, [0, 1, 0, 0])
    assert st == 1


def test_draft_argmax_probs_matches_scalar(golden, oracle):
    c = golden["draft_argmax_probs"]
    i = np.arange(c["n"] * c["vocab"], dtype=np.float32)
    data = (np.sin(i * np.float32(c["step"])) * np.float32(c["amp"])).astype(np.float32)
    logits = data.reshape(c["n"], c["vocab"])
    ids, probs = oracle.draft_argmax_probs(logits)
    for r in range(c["n"]):
        row = logits[r]
        arg = int(np.argmax(row))
        want = 1.0 / np.exp((row - row[arg]).astype(np.float64)).sum()
        assert ids[r] == arg
        assert abs(probs[r] - want) < c["p_tol"]


def test_keep_confident(golden, oracle):
    c = golden["keep_confident"]
    for case in c["cases"]:
        assert oracle.keep_confident(c["ids"], case["probs"], case["p_min"]) == case["expect"]
    assert oracle.keep_confident([], [], c["empty"]["p_min"]) == c["empty"]["expect"]


def test_held_row_against_decimal(oracle):
    decimal.getcontext().prec = 50
    rng = np.random.default_rng(9)
    for _ in range(5):
        row = rng.normal(0, 4, 300).astype(np.float32)
        st, mx, lse = oracle.held_row(row, 280)
        vals = row[:280]
        m = max(vals)
        denom = sum(decimal.Decimal(float(np.float32(v - m))).exp() for v in vals)
        want = float(decimal.Decimal(float(m)) + denom.ln())
        assert st == 0 and mx == m and abs(lse - want) < 1e-12 * abs(want) + 1e-13
    assert oracle.held_row([1.0, float("nan")], 2)[0] == STATUS["NAN"]
    assert oracle.held_row([float("-inf")] * 4, 4)[0] == STATUS["NO_FINITE"]
    assert oracle.held_row([1.0, 2.0], 3)[0] == STATUS["NARROW"]


def test_last_logprobs_and_probs_against_decimal(oracle):
    """last_logprobs_for and last_probs (generate.rs:1871-1899) on small rows
    against 60-digit decimal from the same f32 values: each log-prob
    f64(v) - lse and each probability exp(f64(v) - lse) to 1e-13, the class
    sums of escape_mass (batch.rs:1638-1662) likewise, and an out-of-range id
    is the reference's error."""
    decimal.getcontext().prec = 60
    D = decimal.Decimal
    rng = np.random.default_rng(19)
    for trial in range(4):
        row = rng.normal(0, 4, 300).astype(np.float32)
        if trial % 2:
            row[17] = np.float32(row.max() + 30.0)  # a dominant id
        enc = 280
        vals = row[:enc]
        m = max(vals)
        denom = sum(D(float(np.float32(v - m))).exp() for v in vals)
        lse = D(float(m)) + denom.ln()
        ids = [0, 17, 279, int(np.argmax(vals)), 5]
        st, lp = oracle.last_logprobs_for(row, enc, ids)
        assert st == 0
        for i, got in zip(ids, lp):
            want = float(D(float(vals[i])) - lse)
            assert abs(got - want) <= 1e-13 * abs(want) + 1e-13, (trial, i, got, want)
        st, p = oracle.last_probs(row, enc)
        assert st == 0 and p.size == enc
        want_p = [float((D(float(v)) - lse).exp()) for v in vals]
        np.testing.assert_allclose(p, want_p, rtol=1e-13, atol=0)
        classes = np.zeros((2, (enc + 31) // 32), np.uint32)
        allow = rng.random((2, enc)) < 0.3
        for c in range(2):
            for t in np.nonzero(allow[c])[0]:
                classes[c, t >> 5] |= np.uint32(1 << (t & 31))
        got_c = oracle.class_masses(p, classes)
        for c in range(2):
            want_c = float(sum((D(float(vals[t])) - lse).exp() for t in np.nonzero(allow[c])[0]))
            assert abs(got_c[c] - want_c) <= 1e-13 * want_c, (trial, c)
    assert oracle.last_logprobs_for(row, 280, [280])[0] == oracle.ID_OOR
    assert oracle.last_logprobs_for(row, 280, [-1])[0] == oracle.ID_OOR
    assert oracle.last_probs([1.0, float("nan")], 2)[0] == STATUS["NAN"]


def test_last_probs_of_a_dominant_row_follow_the_fold(oracle):
    """A dominant id followed by n equal terms t >= 2^-53: the fold's
    denominator is exactly 1 + n rint(2^52 t) 2^-52 (held_row's serial f64
    sum), so the dominant id's probability is exactly exp(-ln(D)) and the row's
    probabilities sum to (1 + n t) / D -- not to 1, which an exactly summed
    denominator would give."""
    n = 50_000
    d = -25.0
    row = np.concatenate([[5.0], np.full(n, 5.0 + d)]).astype(np.float32)
    dd = float(np.float32(np.float32(5.0 + d) - np.float32(5.0)))
    t = math.exp(dd)
    denom = 1.0 + n * round(t * 2.0 ** 52) * 2.0 ** -52
    st, p = oracle.last_probs(row, row.size)
    assert st == 0
    lse = 5.0 + math.log(denom)
    assert p[0] == math.exp(5.0 - lse)
    assert abs(math.fsum(p) - (1.0 + n * t) / denom) < 1e-12
    assert abs(p[1] - t / denom) < 1e-18


def test_det_logits_matches_independent_lcg(oracle):
    for n, seed, scale in [(64, 1, 1.0), (100, 4242, 12.0), (33, 90210, 3.0)]:
        np.testing.assert_array_equal(oracle.det_logits(n, seed, scale),
                                      refimpl.det_logits(n, seed, scale))


def test_exp_table_constants_against_decimal():
    """The table the oracle and the kernel share: 2^(j/32) = hi + lo to 2^-104."""
    import re
    decimal.getcontext().prec = 60
    here = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    src = open(os.path.join(here, "oracle", "xs_oracle.c")).read()
    rows = re.findall(r"\{(0x[0-9a-fp.+-]+), (-?0x[0-9a-fp.+-]+)\},", src)
    assert len(rows) == 32
    ln2 = decimal.Decimal(2).ln()
    for j, (hi, lo) in enumerate(rows):
        exact = (ln2 * j / 32).exp()
        got = decimal.Decimal(float.fromhex(hi)) + decimal.Decimal(float.fromhex(lo))
        assert abs(got - exact) < exact * decimal.Decimal(2) ** -104
    kernel = open(os.path.join(here, "xwen_amd", "csrc", "xs_exp_table.h")).read()
    krows = re.findall(r"\{(0x[0-9a-fp.+-]+), (-?0x[0-9a-fp.+-]+)\}", kernel)
    assert [tuple(map(float.fromhex, r)) for r in krows] == \
        [tuple(map(float.fromhex, r)) for r in rows]


# --- select_option (batch.rs:1545-1588) ----------------------------------------

def test_select_option_known_answers(golden, oracle):
    c = golden["select_option"]
    sc = c["scores"]
    us = [j / 997 for j in range(997)]  # a grid over [0, 1) in place of the seeded draws
    for T, k, p in c["greedy"]:
        for u in us[:8]:
            assert oracle.select_option(sc, T, k, p, u) == (0, c["greedy_expect"])
    T, k, p = c["narrow"]
    assert all(oracle.select_option(sc, T, k, p, u)[1] < c["narrow_below"] for u in us)
    T, k, p = c["tight"]
    assert all(oracle.select_option(sc, T, k, p, u) == (0, c["tight_expect"]) for u in us)
    T, k, p = c["open"]
    assert any(oracle.select_option(sc, T, k, p, u)[1] >= c["open_reaches"] for u in us)


def test_truncate_nucleus_known_answers(golden, oracle):
    c = golden["truncate_nucleus"]
    for top_p, want in c["cases"]:
        assert oracle.truncate_nucleus(c["ranked"], top_p) == want


def test_select_option_draws_the_renormalized_mass(oracle):
    """With no cut, the share of a uniform grid that maps to option i is the
    softmax probability of its score at T (a closed form), to the grid step."""
    rng = np.random.default_rng(5)
    scores = rng.normal(0, 2, 7)
    T, N = 1.7, 20000
    got = np.bincount([oracle.select_option(scores, T, 50, 1.0, j / N)[1] for j in range(N)],
                      minlength=7) / N
    z = scores / T
    want = np.exp(z - z.max()) / np.exp(z - z.max()).sum()
    assert np.abs(got - want).max() <= 2.0 / N


def test_select_option_ties_and_errors(oracle):
    # equal scores rank by index: top_k = 2 never reaches the third
    assert all(oracle.select_option([1.0, 1.0, 1.0], 1.0, 2, 1.0, j / 64)[1] < 2 for j in range(64))
    # greedy ties go to the first listed option, NaN never wins
    assert oracle.select_option([float("nan"), 2.0, 2.0], 0.0, 20, 1.0) == (0, 1)
    # no mass: a NaN score makes every probability NaN (WeightedIndex refuses it)
    assert oracle.select_option([0.0, float("nan")], 1.0, 20, 0.9, 0.5)[0] == 5
    assert oracle.select_option([-np.inf, -np.inf], 1.0, 20, 0.9, 0.5)[0] == 5
