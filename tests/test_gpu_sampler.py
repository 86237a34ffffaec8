"""Parity of the HIP sampler (through the C ABI) with the CPU oracle.

The bar: greedy argmax, the top-k candidate set and the chosen ids bit-exact
with ties to the lower id; probabilities and log-probs within 1e-5 relative.

How each row is checked:
  * greedy rows: token and status equal the oracle's argmax (sampler.rs:268-286).
  * stochastic rows: the oracle is run with the device's softmax denominator
    (SUM_GIVEN); status, token, every candidate id and every post-top-p weight
    must then be bit-identical -- everything downstream of the denominator is
    the reference's f32 arithmetic in the reference's order.
  * the device denominator itself must lie within DENOM_RTOL of the exactly
    summed denominator (oracle SUM_F64), and its max equals the oracle's.
  * against the literal reference order (serial f32 sum, sampler.rs:301-305),
    tokens must agree on every row whose decision margins exceed MARGIN_EPS;
    rows below it are counted and reported, never re-seeded away.
  * controlled rows (an allow-mask or sparse controls), whose reference
    denominator is its serial f32 sum (oracle SUM_SEQ_F32): the token and the
    candidate ids equal the literal reference's on every row, with no margin
    rule.  At top_p >= 1, where the weights p = e / sum reach the caller
    unrenormalized, the device denominator is that serial sum bit for bit, so
    every weight is the reference's too; elsewhere the device divides by the
    exact sum (weights within PROB_RTOL of the reference's), unless the
    finalizer found the token unsettled by it and summed the row serially
    itself (then bit for bit again).
"""
import math
import os

import numpy as np
import pytest

from tests import refimpl, workloads

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DENOM_RTOL = 2e-6      # device softmax denominator vs the exact sum of the same f32 terms
PROB_RTOL = 1e-5       # probabilities and log-probs (north star)
MARGIN_EPS = 1e-5      # decision margin below which the serial-f32 order may flip a draw
V = workloads.V
WORST = {}  # largest deviations seen, printed at the end of the module
SERIAL_ROWS = [0]  # rows checked against the serial f32 denominator
SERIAL_SEEN = {"controlled": 0, "serial_sum": 0}  # controlled rows, and those the device summed serially


@pytest.fixture(scope="module", autouse=True)
def report_worst():
    yield
    print(f"\nworst deviations: {WORST}")


@pytest.fixture(scope="module")
def ctx():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from xwen_amd import sampler as xsm
    c = xsm.Context(max_rows=256, vocab=V)
    c.bind_current_stream()
    yield c
    c.close()


def dev(x):
    return torch.as_tensor(np.ascontiguousarray(x)).to("cuda")


def run_sample(ctx, logits, T, K, P, U, *, enc=None, width=None, mask=None, mask_words=None,
               cand_k=128, n_top=0, ctls=None, k_max=0, stats=True):
    """One xs_sample call; `ctls` is one SampleControl (sparse part) or None per row.
    cand_k=0 and stats=False make it a tokens-only call."""
    from xwen_amd import sampler as xsm
    rows = logits.shape[0]
    lg = dev(np.asarray(logits, np.float32))
    p = xsm.params_tensor(T, K, P, rows, "cuda")
    u = dev(np.broadcast_to(np.asarray(U, np.float32), (rows,)).copy())
    m = None if mask is None else dev(np.asarray(mask, np.uint32).view(np.int32))
    controls = None if ctls is None else xsm.controls_tensor(ctls, "cuda")
    out = xsm.sample_batch(ctx, lg, p, u, enc=enc, width=width, allowed=m,
                           allowed_words=mask_words, cand_k=cand_k, stats=stats, n_top=n_top,
                           controls=controls, k_max=k_max)
    torch.cuda.synchronize()
    return {k: (None if v is None else v.cpu().numpy()) for k, v in vars(out).items()}


def oracle_row(oracle, row, enc, T, k, p, u, mask_row=None, ctl=None, **kw):
    octl = None
    if mask_row is not None or ctl is not None:
        octl = oracle.Ctl(allowed=mask_row)
        if ctl is not None:
            octl.banned, octl.bias = tuple(ctl.banned), tuple(ctl.bias)
            octl.pull, octl.force = ctl.pull, ctl.force
    return oracle.sample_controlled(row, enc, float(T), int(k), float(p), u=float(u), ctl=octl,
                                    **kw)


def controlled_row(T, K, P, mask_row, ctl) -> bool:
    """A stochastic row on the reference's control path (sample_controlled's
    non-noop branch, sampler.rs:222-229), whose denominator is its serial f32
    sum (sampler.rs:301-305)."""
    controlled = mask_row is not None or (ctl is not None and not ctl.is_noop())
    return not (T <= 0.0 or K <= 1) and controlled


def serial_row(T, K, P, mask_row, ctl) -> bool:
    """A row whose denominator is the serial f32 sum on the device in a call
    that observes it (candidates or soft_sum): controlled and top_p >= 1."""
    return controlled_row(T, K, P, mask_row, ctl) and P >= 1.0


def check_controlled(oracle, row, enc, T, k, p, u, d, r, mrow, kw, tag):
    """A controlled stochastic row against the literal reference (the oracle
    with the serial f32 sum): status and token always; candidate ids, and the
    weights within PROB_RTOL (bit for bit when the device used that sum).
    Returns whether the device's denominator, when reported, is the serial sum."""
    oseq = oracle_row(oracle, row, enc, T, k, p, u, mrow, sum_mode=oracle.SUM_SEQ_F32, **kw)
    assert d["status"][r] == oseq.status, (tag, "status", d["status"][r], oseq.status)
    SERIAL_SEEN["controlled"] += 1
    if oseq.status != 0:
        return False
    assert d["token"][r] == oseq.token, (tag, "serial-f32 token", d["token"][r], oseq.token)
    serial_sum = False
    if d.get("soft_sum") is not None:
        serial_sum = np.float32(d["soft_sum"][r]).view(np.uint32) == np.float32(oseq.ssum).view(np.uint32)
        SERIAL_SEEN["serial_sum"] += int(serial_sum)
    if d.get("cand_id") is not None:
        ncmp = min(len(oseq.cand), d["cand_id"].shape[1])
        assert list(d["cand_id"][r, :ncmp]) == [i for _, i in oseq.cand][:ncmp], (tag, "serial-f32 ids")
        ws = np.array([w for w, _ in oseq.cand][:ncmp], np.float32)
        if serial_sum:
            np.testing.assert_array_equal(d["cand_w"][r, :ncmp].view(np.uint32), ws.view(np.uint32),
                                          err_msg=tag)
        else:
            np.testing.assert_allclose(d["cand_w"][r, :ncmp], ws, rtol=PROB_RTOL, atol=1e-30, err_msg=tag)
    return serial_sum


def check_rows(oracle, logits, T, K, P, U, d, *, enc=None, mask=None, rows=None, margins=True,
               label="", ctls=None):
    """Compare device outputs `d` with the oracle row by row; returns the count of
    rows whose serial-f32 decision margin fell below MARGIN_EPS."""
    n_rows, width = logits.shape
    enc = width if enc is None else enc
    T = np.broadcast_to(np.asarray(T, np.float64), (n_rows,))
    K = np.broadcast_to(np.asarray(K), (n_rows,))
    P = np.broadcast_to(np.asarray(P, np.float64), (n_rows,))
    U = np.broadcast_to(np.asarray(U, np.float32), (n_rows,))
    thin = 0
    for r in (range(n_rows) if rows is None else rows):
        mrow = None if mask is None else mask[r]
        kw = {} if ctls is None else {"ctl": ctls[r]}
        greedy = T[r] <= 0.0 or K[r] <= 1
        tag = f"{label} row {r} T={T[r]} k={K[r]} p={P[r]}"
        if greedy:
            o = oracle_row(oracle, logits[r], enc, T[r], K[r], P[r], U[r], mrow, **kw)
            assert (d["status"][r], d["token"][r] if o.status == 0 else -1) == \
                (o.status, o.token if o.status == 0 else -1), tag
            continue
        S = np.float32(d["soft_sum"][r])
        o = oracle_row(oracle, logits[r], enc, T[r], K[r], P[r], U[r], mrow,
                       sum_mode=oracle.SUM_GIVEN, s_given=S, **kw)
        assert d["status"][r] == o.status, (tag, d["status"][r], o.status)
        if o.status != 0:
            continue
        assert d["token"][r] == o.token, (tag, d["token"][r], o.token)
        if d.get("cand_id") is not None:  # a call without a candidate list checks the token only
            n = len(o.cand)
            assert d["n_cand"][r] == n, tag
            ncmp = min(n, d["cand_id"].shape[1])
            ids = [i for _, i in o.cand][:ncmp]
            ws = np.array([w for w, _ in o.cand][:ncmp], np.float32)
            assert list(d["cand_id"][r, :ncmp]) == ids, tag
            np.testing.assert_array_equal(d["cand_w"][r, :ncmp].view(np.uint32), ws.view(np.uint32),
                                          err_msg=tag)
        assert np.float32(d["soft_max"][r]) == np.float32(o.smax), tag
        # the denominator against the exact sum of the same correctly rounded terms
        o64 = oracle_row(oracle, logits[r], enc, T[r], K[r], P[r], U[r], mrow,
                         sum_mode=oracle.SUM_F64, **kw)
        rel = abs(float(S) - float(o64.ssum)) / float(o64.ssum)
        if controlled_row(T[r], K[r], P[r], mrow, kw.get("ctl")):
            # the literal reference (its serial f32 sum): token and ids always
            serial_sum = check_controlled(oracle, logits[r], enc, T[r], K[r], P[r], U[r], d, r, mrow, kw, tag)
            if serial_row(T[r], K[r], P[r], mrow, kw.get("ctl")):  # observed at top_p >= 1: bit for bit
                assert serial_sum, (tag, "serial sum", float(S))
            if serial_sum:
                WORST["serial_vs_exact"] = max(WORST.get("serial_vs_exact", 0.0), rel)
                SERIAL_ROWS[0] += 1
            else:
                WORST["denominator"] = max(WORST.get("denominator", 0.0), rel)
                assert rel <= DENOM_RTOL, (tag, float(S), o64.ssum, rel)
            continue
        WORST["denominator"] = max(WORST.get("denominator", 0.0), rel)
        assert rel <= DENOM_RTOL, (tag, float(S), o64.ssum, rel)
        if margins:
            oseq = oracle_row(oracle, logits[r], enc, T[r], K[r], P[r], U[r], mrow,
                              sum_mode=oracle.SUM_SEQ_F32, margins=True, **kw)
            margin = min(oseq.margin_order, oseq.margin_cut, oseq.margin_draw)
            if margin > MARGIN_EPS:
                assert oseq.token == d["token"][r], (tag, "serial-f32 order", margin)
            else:
                thin += 1
    return thin


def check_held_row(oracle, row, d, r, n_top, label=""):
    """held_row (generate.rs:1905-1933) outputs of row r against the reference's
    own fold: the oracle sums the f64 terms exp(f64(v - max)) one after another
    in id order, as the reference does.  row_max is bit-exact; row_lse and every
    top log-prob agree within 1e-5 relative, with a floor of four f64 ulps of
    lse (the log-prob is v - lse, so lse's last bits are all a log-prob of a
    dominant token carries)."""
    import math
    v = row.size
    st, mx, lse_serial = oracle.held_row(row, v)
    assert st == 0, label
    assert np.float32(d["row_max"][r]) == np.float32(mx), (label, r)
    floor = 4 * math.ulp(abs(lse_serial))
    assert abs(d["row_lse"][r] - lse_serial) <= PROB_RTOL * abs(lse_serial) + floor, \
        (label, r, d["row_lse"][r], lse_serial)
    order = refimpl.stable_desc_order(row)[:n_top]
    assert list(d["top_id"][r][:n_top]) == order.tolist(), (label, r)
    want = row[order].astype(np.float64) - lse_serial
    np.testing.assert_allclose(d["top_logprob"][r][:n_top].astype(np.float64), want,
                               rtol=PROB_RTOL, atol=floor, err_msg=f"{label} row {r}")


# --- the device exp ------------------------------------------------------------

def test_device_exp_is_correctly_rounded(oracle):
    from xwen_amd import _lib
    lib = _lib.load()
    neg = np.arange(0x80000000, 0xC2D00001, 4099, dtype=np.uint64).astype(np.uint32)
    pos = np.arange(0, 0x42B20001, 4099, dtype=np.uint64).astype(np.uint32)
    special = np.array([0x7FC00000, 0x7F800000, 0xFF800000, 0x80000000, 0x00000001, 0x80000001],
                       np.uint32)
    x = np.concatenate([neg, pos, special]).view(np.float32)
    x = np.concatenate([x, np.float32([-104.5, 89.5, -103.97, 88.72283, -87.33655])])
    xd = dev(x)
    yd = torch.empty_like(xd)
    assert lib.xs_test_exp(xd.data_ptr(), yd.data_ptr(), x.size, None) == 0
    torch.cuda.synchronize()
    want = oracle.exp_array(x)
    got = yd.cpu().numpy()
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all(), x[~same][:10]


# --- the five measured configurations --------------------------------------------

def test_c1_single_row_thinking_and_greedy(ctx, oracle):
    for greedy in (False, True):
        wl = workloads.c1_single(greedy=greedy)
        d = run_sample(ctx, wl.logits, wl.temperature, wl.top_k, wl.top_p, wl.u)
        assert d["status"][0] == 0
        check_rows(oracle, wl.logits, wl.temperature, wl.top_k, wl.top_p, wl.u, d, label=wl.name)
        if greedy:
            assert d["token"][0] == int(np.argmax(wl.logits[0]))


def test_c2_batch_of_64(ctx, oracle):
    wl = workloads.c2_batch()
    d = run_sample(ctx, wl.logits, wl.temperature, wl.top_k, wl.top_p, wl.u)
    assert (d["status"] == 0).all()
    thin = check_rows(oracle, wl.logits, wl.temperature, wl.top_k, wl.top_p, wl.u, d, label="C2")
    print(f"C2: {thin} of 64 rows below the decision margin {MARGIN_EPS}")
    assert thin <= 2


def test_c3_grammar_masked(ctx, oracle):
    wl = workloads.c3_masked()
    d = run_sample(ctx, wl.logits, wl.temperature, wl.top_k, wl.top_p, wl.u, mask=wl.mask)
    assert (d["status"] == 0).all()
    thin = check_rows(oracle, wl.logits, wl.temperature, wl.top_k, wl.top_p, wl.u, d,
                      mask=wl.mask, label="C3")
    # the one-hot mask forces its token
    only = int(np.nonzero(workloads.mask_bits(wl.mask[0], V))[0][0])
    assert d["token"][0] == only
    for r in range(wl.logits.shape[0]):
        assert workloads.mask_bits(wl.mask[r], V)[d["token"][r]]
    print(f"C3: {thin} rows below the decision margin")


def test_c4_speculative_verify(ctx, oracle):
    from xwen_amd import sampler as xsm
    wl = workloads.c4_verify()
    rows = wl.seqs * wl.span
    d = run_sample(ctx, wl.logits, wl.temperature, wl.top_k, wl.top_p, wl.u)
    check_rows(oracle, wl.logits, wl.temperature, wl.top_k, wl.top_p, wl.u, d, label="C4",
               margins=False)
    lg = dev(wl.logits)
    p = xsm.params_tensor(wl.temperature, wl.top_k, wl.top_p, rows, "cuda")
    u = dev(wl.u)
    eog = [248046, 248044]
    budgets = np.full(wl.seqs, 1 << 30, np.int32)
    budgets[3] = 2
    budgets[5] = 0
    for budget in (None, dev(budgets)):
        out = xsm.verify_batch(ctx, lg, wl.seqs, wl.span, p, u, dev(wl.drafts), budget=budget,
                               eog=eog)
        torch.cuda.synchronize()
        row_tok = out.row_token.cpu().numpy()
        np.testing.assert_array_equal(row_tok, d["token"])
        acc = out.accepted.cpu().numpy()
        com = out.committed.cpu().numpy()
        ncom = out.n_committed.cpu().numpy()
        sst = out.seq_status.cpu().numpy()
        bud = (np.full(wl.seqs, 1 << 62) if budget is None else budgets.astype(np.int64))
        for s in range(wl.seqs):
            toks = row_tok[s * wl.span:(s + 1) * wl.span]
            st, m, committed, _ = oracle.accept_drafts(
                list(wl.drafts[s]), int(bud[s]), list(toks), [t in eog for t in toks])
            assert (sst[s], acc[s], ncom[s]) == (st, m, len(committed)), s
            assert list(com[s, :ncom[s]]) == committed, s
            assert (com[s, ncom[s]:] == -1).all()
    # half the drafts are the argmax: some sequences must accept more than nothing
    assert acc.max() >= 1


def test_c5_heterogeneous_with_row_statistics(ctx, oracle):
    wl = workloads.c5_heterogeneous()
    d = run_sample(ctx, wl.logits, wl.temperature, wl.top_k, wl.top_p, wl.u, n_top=20)
    assert (d["status"] == 0).all()
    thin = check_rows(oracle, wl.logits, wl.temperature, wl.top_k, wl.top_p, wl.u, d, label="C5")
    print(f"C5: {thin} of 256 rows below the decision margin")
    for r in range(wl.logits.shape[0]):
        check_held_row(oracle, wl.logits[r], d, r, 20, label="C5")


def test_held_row_of_a_dominant_token_follows_the_serial_fold(ctx, oracle):
    """A token 20-35 above a 248,320-id bulk, at the first, a middle, the last
    and other ids.  The reference's serial f64 fold (generate.rs:1931-1932)
    absorbs every term after the max below 2^-53 and rounds the others to the
    2^-52 grid, which moves such a token's log-prob (about -1e-8 to -1e-14) by
    up to its whole size from the exactly summed value; the device must follow
    the fold at 1e-5.  Greedy and stochastic rows take the same statistics."""
    import math
    rng = np.random.default_rng(2718)
    positions = [0, V // 2, V - 1, 1234, 200_001, 77, 16_383, 16_384, 131_071]
    rows, worst_exact = [], 0.0
    for i, pos in enumerate(positions):
        x = rng.normal(0, [1.0, 3.0, 0.3][i % 3], V).astype(np.float32)
        x[pos] = x.max() + np.float32(20 + 15 * rng.random())
        rows.append(x)
        st, mx, lse_serial = oracle.held_row(x, V)
        terms = np.exp((x - np.float32(mx)).astype(np.float32).astype(np.float64))
        lse_exact = float(mx) + math.log(math.fsum(terms.tolist()))
        top = float(x[pos]) - lse_serial
        worst_exact = max(worst_exact, abs((float(x[pos]) - lse_exact) - top) / abs(top))
    x = np.stack(rows)
    T = np.where(np.arange(len(rows)) % 2 == 0, 0.0, 1.0)
    d = run_sample(ctx, x, T, 20, 0.95, 0.4, n_top=8)
    assert (d["status"] == 0).all()
    for r in range(len(rows)):
        check_held_row(oracle, x[r], d, r, 8, label="dominant")
    print(f"exact-sum log-prob off the serial fold by up to {worst_exact:.2e} on these rows")
    assert worst_exact > 1e-3  # the rows do exercise the fold


# --- the reference's own known answers -------------------------------------------

def _pad(values, ld=None):
    v = np.asarray(values, np.float32)
    ld = ld or max(4, (v.size + 3) // 4 * 4)
    out = np.full(ld, -np.inf, np.float32)
    out[: v.size] = v
    return out


UNIFORMS = [0.0, 0.25, 0.5, 0.75, 1.0 - 2.0 ** -23, 0.123456789]


def test_reference_cases(ctx, golden):
    """Every sampler known answer the reference's tests hold, controls included."""
    from xwen_amd import sampler as xsm
    names = {"NAN": 1, "NO_FINITE": 2, "MASK_SHORT": 3, "FORCE_OOR": 4, "ZERO_WEIGHT": 5,
             "NARROW": 6}
    ran = 0
    for case in golden["sampler"]:
        ctls = None
        if any(k in case for k in ("banned", "bias", "pull", "force")):
            ctls = [xsm.SampleControl(banned=case.get("banned", ()),
                                      bias=[tuple(b) for b in case.get("bias", ())],
                                      pull=tuple(case["pull"]) if "pull" in case else None,
                                      force=case.get("force"))]
        vals = case["logits"]
        width = len(vals)
        enc = case["enc"]
        row = _pad(vals, max(4, (max(width, enc) + 3) // 4 * 4))
        mask = None
        if "allowed" in case:
            mask = np.asarray([case["allowed"]], np.uint32)
        us = UNIFORMS if case.get("any_uniform") or "expect_in" in case else [0.5]
        for u in us:
            d = run_sample(ctx, row[None, :], case["T"], case["k"], case["p"], u, enc=enc,
                           width=width, mask=mask, mask_words=None if mask is None else mask.shape[1],
                           ctls=ctls)
            tag = (case["name"], u, int(d["status"][0]), int(d["token"][0]))
            if "expect_error" in case:
                assert d["status"][0] == names[case["expect_error"]], tag
            elif "expect" in case:
                assert (d["status"][0], d["token"][0]) == (0, case["expect"]), tag
            else:
                assert d["status"][0] == 0 and d["token"][0] in case["expect_in"], tag
        ran += 1
    assert ran >= 28


def test_wide_nan_errors_on_both_paths(ctx, golden):
    c = golden["wide_nan"]
    v = np.full(c["n"], c["fill"], np.float32)
    for i, x in c["set"]:
        v[i] = x
    for T in (0.0, 1.0):
        d = run_sample(ctx, v[None, :], T, 20, 1.0, 0.5)
        assert d["status"][0] == 1


def test_nan_in_a_full_width_row_and_masked_nan(ctx):
    rng = np.random.default_rng(4)
    x = rng.normal(0, 3, (4, V)).astype(np.float32)
    x[0, 123457] = np.nan
    x[1, V - 1] = np.nan
    d = run_sample(ctx, x, [1.0, 0.0, 1.0, 0.0], 20, 0.95, 0.5)
    assert list(d["status"]) == [1, 1, 0, 0]
    # a NaN at an id the allow-mask excludes is set to -inf first (apply_control)
    allow = np.ones((1, V), bool)
    allow[0, 123457] = False
    y = x[:1].copy()
    d = run_sample(ctx, y, 1.0, 20, 0.95, 0.5, mask=workloads.pack_mask(allow))
    assert d["status"][0] == 0


def test_infinities(ctx, oracle):
    x = np.zeros((4, 4096), np.float32)
    x[0, 7] = np.inf
    x[0, 9] = np.inf
    x[1, 7] = np.inf
    x[2, :] = -np.inf
    x[3, :] = -np.inf
    d = run_sample(ctx, x, [0.0, 1.0, 1.0, 0.0], 20, 0.95, 0.5)
    assert (d["status"][0], d["token"][0]) == (0, 7)     # greedy: first +inf
    assert d["status"][1] == 1                              # stochastic: inf - inf = NaN
    assert d["status"][2] == 1                              # no-op control, all -inf: NaN probs
    assert d["status"][3] == 2                              # greedy, nothing above -inf
    for r in range(4):
        o = oracle_row(oracle, x[r], 4096, [0.0, 1.0, 1.0, 0.0][r], 20, 0.95, 0.5)
        assert o.status == d["status"][r]
    # asking for the row statistics changes no draw: a +inf voids the
    # statistics (held_row needs a finite max) but not the greedy argmax
    s = run_sample(ctx, x, [0.0, 1.0, 1.0, 0.0], 20, 0.95, 0.5, n_top=4)
    assert list(s["status"]) == list(d["status"]) and s["token"][0] == 7
    assert np.isnan(s["row_lse"]).all()
    # with an allow-mask, a row left with no finite value is NO_FINITE
    allow = np.zeros((1, 4096), bool)
    allow[0, :16] = True
    y = np.full((1, 4096), -np.inf, np.float32)
    d = run_sample(ctx, y, 1.0, 20, 0.95, 0.5, mask=workloads.pack_mask(allow))
    assert d["status"][0] == 2


def test_tall_peaks_and_extreme_temperatures(ctx, oracle):
    """Rows shaped like a language model's logits: a few tokens 15-55 above a
    N(0, 3^2) bulk, at T from 1.0 down to 0.05.  The lanes holding the peaks
    start their softmax offsets far below them, where an f32 exponent of 60
    to 90 loses 3e-6 to rounding; the recount and the lane factor must still
    keep the denominator within DENOM_RTOL.  Also 1/T overflowing f32
    (T = 1e-45: every s is +-inf) and T = 1e6 (every s near 0)."""
    rng = np.random.default_rng(4242)
    rows, v = 16, 65536
    x = (rng.standard_normal((rows, v)) * 3.0).astype(np.float32)
    for r in range(rows):
        k = int(rng.integers(1, 6))
        ids = rng.choice(v, k, replace=False)
        x[r, ids] = (x[r].max() + rng.uniform(15, 55) - rng.uniform(0, 3, k)).astype(np.float32)
    T = [1.0, 0.7, 0.5, 0.1] * 3 + [1e-45, 1e6, 0.05, 2.0]
    K = [20, 50, 100, 20] * 3 + [20, 20, 40, 64]
    P = [0.95, 0.9, 1.0, 0.8] * 3 + [0.9, 0.95, 0.99, 0.9]
    U = rng.random(rows).astype(np.float32)
    d = run_sample(ctx, x, T, K, P, U)
    check_rows(oracle, x, T, K, P, U, d, label="tall peaks")


def test_huge_finite_logits_are_ordinary_values(ctx, oracle):
    """Finite logits of huge magnitude (-1e30 standing for a masked id, as
    some producers write it) are ordinary values to the reference: exp(s - max)
    is 0 below a moderate max, and 1 for every id equal to a huge max.  A
    lane whose softmax offset is that large must not turn its partial into
    inf (and then NaN once scaled by 0)."""
    rng = np.random.default_rng(4343)
    rows = 6
    x = (rng.standard_normal((rows, V)) * 3.0).astype(np.float32)
    x[0, rng.random(V) < 0.3] = -1e30             # scattered
    x[1, : V // 2] = -1e30                        # whole chunks and waves of them
    x[2, :] = -1e30                               # every id ties at a huge max
    x[3, :] = np.where(rng.random(V) < 0.5, -1e30, -2e30)
    x[4, rng.random(V) < 0.9] = -3.4e38           # near -FLT_MAX
    x[5, ::7] = 1e30                              # huge positive values tie at the max
    T = [1.0, 0.7, 1.0, 1.0, 0.5, 1.0]
    K = [20, 50, 20, 100, 20, 20]
    P = [0.95, 0.9, 0.95, 1.0, 0.9, 0.8]
    U = rng.random(rows).astype(np.float32)
    d = run_sample(ctx, x, T, K, P, U)
    assert (d["status"] == 0).all(), d["status"]
    check_rows(oracle, x, T, K, P, U, d, label="huge finite logits")


def test_narrow_row_short_mask_and_bad_k(ctx):
    x = np.zeros((2, 1024), np.float32)
    d = run_sample(ctx, x, 1.0, 20, 0.95, 0.5, enc=1024, width=1000)
    assert list(d["status"]) == [6, 6]
    mask = np.full((2, 32), 0xFFFFFFFF, np.uint32)
    d = run_sample(ctx, x, 1.0, 20, 0.95, 0.5, mask=mask, mask_words=31)
    assert list(d["status"]) == [3, 3]
    d = run_sample(ctx, x, 1.0, [20, 200], 0.95, 0.5)
    assert list(d["status"]) == [0, 7]


@pytest.mark.parametrize("shape", ["Flat", "Peaked", "Ties"])
def test_candidate_sets_across_the_reference_matrix(ctx, oracle, shape):
    """sampler.rs:1359-1486: toy row to the padded vocabulary, k from greedy to
    wider than the row, p from biting to no-op; candidate ids must equal the
    oracle's, ties included."""
    for n in (64, 2048, V):
        rows, params = [], []
        for k in (1, 20, 64):
            for p in (0.5, 0.95, 1.0):
                rows.append(refimpl.shaped(shape, n, k, 90210, oracle))
                params.append((1.0, k, p))
        x = np.stack(rows)
        T, K, P = (np.array(c) for c in zip(*params))
        U = np.linspace(0, 1 - 2 ** -23, len(rows)).astype(np.float32)
        d = run_sample(ctx, x, T, K, P, U)
        check_rows(oracle, x, T, K, P, U, d, label=f"{shape} n={n}", margins=False)


def test_candidate_set_matches_llamacpp_filtering(ctx, oracle, golden):
    m = golden["llamacpp_matrix"]
    for n, scale in m["shapes"]:
        rows, params = [], []
        for seed in m["seeds"]:
            for k, p, T in m["params"]:
                rows.append(oracle.det_logits(n, seed, scale))
                params.append((T, k, p))
        x = np.stack(rows)
        T, K, P = (np.array(c) for c in zip(*params))
        U = np.linspace(0.01, 0.99, len(rows)).astype(np.float32)
        d = run_sample(ctx, x, T, K, P, U)
        check_rows(oracle, x, T, K, P, U, d, label=f"llama.cpp n={n}", margins=False)
        for r in range(len(rows)):
            probs, _, _ = oracle.softmax_in_place(x[r], float(T[r]))
            want = refimpl.llamacpp_filtered(probs, int(K[r]), float(P[r]))
            nc = int(d["n_cand"][r])
            kept = sorted(int(i) for i, w in zip(d["cand_id"][r, :nc], d["cand_w"][r, :nc])
                          if w > 0)
            assert kept == [i for i, _ in want], (n, r)


def test_small_rows_and_sort_everything_branch(ctx, oracle):
    """top_k >= enc takes candidate_set's sort-everything branch; enc below the
    row width drops the padded ids (sampler.rs:1540-1571)."""
    rng = np.random.default_rng(12)
    for enc, width in ((5, 8), (13, 16), (100, 100), (127, 128)):
        x = rng.normal(0, 2, (6, width)).astype(np.float32)
        x[:, enc:] = 50.0  # padded ids carry the largest logits and must never win
        T = [1.0, 0.7, 1.3, 0.0, 1.0, 1.0]
        K = [enc, enc + 5, 3, 20, 2, 127]
        P = [1.0, 0.9, 0.5, 1.0, 0.0, 0.95]
        U = [0.3, 0.9, 0.5, 0.1, 0.7, 0.99]
        d = run_sample(ctx, x, T, K, P, U, enc=enc)
        assert (d["token"] < enc).all()
        check_rows(oracle, x, T, K, P, U, d, enc=enc, label=f"enc={enc}", margins=False)


def test_repeat_calls_are_identical(ctx):
    wl = workloads.c2_batch(rows=16)
    a = run_sample(ctx, wl.logits, wl.temperature, wl.top_k, wl.top_p, wl.u)
    for _ in range(3):
        b = run_sample(ctx, wl.logits, wl.temperature, wl.top_k, wl.top_p, wl.u)
        for key in ("token", "status", "n_cand", "soft_sum"):
            np.testing.assert_array_equal(a[key], b[key])
        for r in range(len(a["n_cand"])):  # entries past n_cand are not written
            n = min(int(a["n_cand"][r]), a["cand_id"].shape[1])
            for key in ("cand_id", "cand_w"):
                np.testing.assert_array_equal(a[key][r, :n], b[key][r, :n])


def test_draw_frequencies_follow_llamacpp_semantics(ctx, oracle, golden):
    """sampler.rs:1177-1223: 40,000 draws over one row land on the filtered
    candidates with llama.cpp's frequencies, within 0.01."""
    c = golden["draw_frequencies"]
    row = oracle.det_logits(*c["det_logits"])
    n = row.size
    draws = c["draws"]
    probs, _, _ = oracle.softmax_in_place(row, c["T"])
    want = refimpl.llamacpp_filtered(probs, c["k"], c["p"])
    mass = sum(float(w) for _, w in want)
    rng = np.random.default_rng(77)
    hist = np.zeros(n)
    batch = 250
    x = np.broadcast_to(row, (batch, n)).copy()
    for _ in range(draws // batch):
        U = (rng.integers(0, 1 << 23, batch) * 2.0 ** -23).astype(np.float32)
        d = run_sample(ctx, x, c["T"], c["k"], c["p"], U, cand_k=0)
        assert (d["status"] == 0).all()
        hist += np.bincount(d["token"], minlength=n)
    hist /= draws
    wanted = {i: float(w) / mass for i, w in want}
    for i in range(n):
        if i in wanted:
            assert abs(hist[i] - wanted[i]) < c["tol"], (i, hist[i], wanted[i])
        else:
            assert hist[i] == 0.0
