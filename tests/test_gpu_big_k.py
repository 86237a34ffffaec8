"""top_k past the streaming selection: 128 and up, and top_k >= the vocabulary
(candidate_set's whole-row branch, sampler.rs:322-338, xwen's only
top-p-only mode since top_k <= 1 is greedy).  The whole-row path computes
every probability, sorts the row by (p desc, id asc) and runs the serial f32
top-p and WeightedIndex chains; its tokens, candidate ids and weights must
equal the oracle's bit for bit given the device's softmax denominator, at full
width, with masks, sparse controls and in a verify block."""
import numpy as np
import pytest

from tests import workloads
from tests.test_gpu_sampler import check_rows, run_sample

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

V = workloads.V
KS = [128, 500, 1000, V, 10**6]


@pytest.fixture(scope="module")
def bigctx():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from xwen_amd import sampler as xsm
    c = xsm.Context(max_rows=12, vocab=V, k_max=2**31 - 1)
    c.bind_current_stream()
    yield c
    c.close()


def _rows(seed, n):
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 3, (n, V)).astype(np.float32)
    for r in range(n):
        x[r, rng.integers(0, V, 8)] = rng.uniform(8, 14, 8).astype(np.float32)
    return x, rng


def test_large_top_k_at_full_width(bigctx, oracle):
    x, rng = _rows(8128, 10)
    K = np.array([k for k in KS for _ in (0, 1)])
    P = np.array([0.8, 1.0] * len(KS))
    T = np.array([1.0, 0.7, 1.3, 1.0, 0.7, 1.0, 1.0, 0.6, 1.0, 1.0])
    U = workloads.uniforms(rng, 10)
    d = run_sample(bigctx, x, T, K, P, U, cand_k=V)
    assert (d["status"] == 0).all(), d["status"]
    assert list(d["n_cand"]) == [min(k, V) for k in K]
    thin = check_rows(oracle, x, T, K, P, U, d, label="big-k")
    print(f"big-k: {thin} of 10 rows below the decision margin")


def test_top_p_only_under_masks_and_controls(bigctx, oracle):
    """Grammar-masked rows with top_k >= V (the masked ids carry p = 0 and sit
    at the end of the candidate list in id order), a one-id mask, and bans,
    biases and a pull on a whole-row draw."""
    from xwen_amd import sampler as xsm
    x, rng = _rows(9128, 6)
    allow = np.zeros((6, V), bool)
    allow[0, 1000:3500] = True                    # ~1 %, one range
    allow[1] = rng.random(V) < 0.10
    allow[2] = rng.random(V) < 0.50
    allow[3, 77_777] = True                       # exactly one id: forced
    allow[4] = rng.random(V) < 0.30
    allow[5] = True
    mask = workloads.pack_mask(allow)
    K = np.array([10**6, V, 10**6, 10**6, 700, 10**6])
    P = np.array([0.95, 1.0, 0.8, 0.95, 0.9, 1.0])
    T = np.array([1.0, 1.0, 0.7, 1.0, 1.0, 1.3])
    U = workloads.uniforms(rng, 6)
    d = run_sample(bigctx, x, T, K, P, U, mask=mask, cand_k=V)
    assert (d["status"] == 0).all(), d["status"]
    assert d["token"][3] == 77_777
    check_rows(oracle, x, T, K, P, U, d, mask=mask, label="big-k masked")
    ctls = [None] * 6
    ctls[0] = xsm.SampleControl(banned=tuple(int(i) for i in np.argsort(-x[0])[:5]))
    ctls[2] = xsm.SampleControl(bias=((11, 6.0), (12, -3.0), (11, 1.5)))
    ctls[5] = xsm.SampleControl(pull=(4242, 0.7), banned=(5, 6, 7))
    d = run_sample(bigctx, x, T, K, P, U, cand_k=V, ctls=ctls)
    assert (d["status"] == 0).all(), d["status"]
    check_rows(oracle, x, T, K, P, U, d, ctls=ctls, label="big-k controlled")


def test_large_top_k_in_a_verify_block(bigctx, oracle):
    """xs_verify rows with top_k 500 and top_k >= V walk as accept_drafts."""
    from xwen_amd import sampler as xsm
    seqs, span = 3, 4
    x, rng = _rows(10128, seqs * span)
    K = np.array([500, 10**6, 300] * span).reshape(span, seqs).T.reshape(-1)
    T = np.full(seqs * span, 1.0)
    P = np.full(seqs * span, 0.95)
    U = workloads.uniforms(rng, seqs * span)
    # the draws row by row through the oracle, then the drafts: two matches
    # then a mismatch in sequence 0, all matches in 1, a mismatch at once in 2
    tok = []
    for r in range(seqs * span):
        d = run_sample(bigctx, x[r:r + 1], T[r], K[r], P[r], U[r:r + 1], cand_k=0)
        tok.append(int(d["token"][0]))
    tok = np.array(tok).reshape(seqs, span)
    drafts = tok[:, :span - 1].copy()
    drafts[0, 2] = (drafts[0, 2] + 1) % V
    drafts[2, 0] = (drafts[2, 0] + 1) % V
    lg = torch.as_tensor(x).cuda()
    p = xsm.params_tensor(T, K, P, seqs * span, "cuda")
    u = torch.as_tensor(U).cuda()
    out = xsm.verify_batch(bigctx, lg, seqs, span, p, u,
                           torch.as_tensor(drafts.astype(np.int32)).cuda())
    torch.cuda.synchronize()
    assert (out.row_token.cpu().numpy().reshape(seqs, span) == tok).all()
    assert out.accepted.cpu().tolist() == [2, 3, 0]
    assert out.n_committed.cpu().tolist() == [3, 4, 1]
    for r in range(seqs * span):
        o = oracle.sample_controlled(x[r], V, float(T[r]), int(K[r]), float(P[r]), u=float(U[r]),
                                     sum_mode=oracle.SUM_SEQ_F32, margins=True)
        if min(o.margin_order, o.margin_cut, o.margin_draw) > 1e-5:
            assert o.token == tok.reshape(-1)[r], r


def test_head_selection_tie_groups(bigctx, oracle):
    """top_k <= 1,024 takes a radix select on the values; the boundary's p can
    be shared by several adjacent values (T = 0.7 and 1.3 map neighbouring
    floats to one p), by a run of equal logits that fits the selection list or
    overflows it (the group's lowest ids are taken in id order), or be 0 (a
    mask leaves fewer ids than top_k: the rest of the row ties at p = 0).
    top_k 129, 1,024 and 1,025 sit on the path's edges."""
    x, rng = _rows(11128, 10)
    T = np.array([0.7, 1.3, 1.0, 1.0, 1.0, 1.3, 1.0, 1.0, 1.0, 0.7])
    K = np.array([1000, 1000, 1000, 1000, 500, 1000, 129, 1024, 1025, 1024])
    P = np.array([0.95, 1.0, 1.0, 0.9, 1.0, 1.0, 0.95, 1.0, 0.95, 1.0])
    # rows 2, 3: 600 ids above 6; a run of equal logits at 5 (500 ids: fits
    # the list; 3,000 ids: overflows it)
    for r, run in ((2, 500), (3, 3000)):
        x[r] = np.minimum(x[r], 4.0)
        ids = rng.permutation(V)
        x[r, ids[:600]] = rng.uniform(6.0, 9.0, 600).astype(np.float32)
        x[r, ids[600:600 + run]] = 5.0
    # row 5: the boundary inside a block of consecutive floats below 5
    base = np.float32(5.0)
    x[5] = np.minimum(x[5], 4.0)
    ids = rng.permutation(V)
    x[5, ids[:900]] = rng.uniform(6.0, 9.0, 900).astype(np.float32)
    steps = np.arange(1, 401, dtype=np.int64) // 4
    x[5, ids[900:1300]] = (base.view(np.int32) - steps).astype(np.int32).view(np.float32)
    # row 9: equal logits at the very top (the whole head one group)
    x[9, :] = np.minimum(x[9], 4.0)
    x[9, rng.integers(0, V, 1500)] = 7.5
    allow = np.ones((10, V), bool)
    allow[4] = False
    allow[4, rng.integers(0, V, 100)] = True   # ~100 ids < top_k 500: p = 0 ties
    mask = workloads.pack_mask(allow)
    U = workloads.uniforms(rng, 10)
    d = run_sample(bigctx, x, T, K, P, U, mask=mask, cand_k=1100)
    assert (d["status"] == 0).all(), d["status"]
    assert list(d["n_cand"]) == list(K)
    check_rows(oracle, x, T, K, P, U, d, mask=mask, label="head ties")


def test_a_call_bounds_its_own_top_k(bigctx, oracle):
    """xs_sample_args.k_max (no counterpart in the reference) bounds one call
    below the context's k_max: rows above it report XS_ROW_BAD_PARAM, rows
    within it draw exactly as without the bound, and a bound of 127 or less
    leaves the whole-row kernels out of the call."""
    x, rng = _rows(12128, 6)
    K = np.array([20, 100, 127, 2, 500, 128])
    T, P = 1.0, 0.9
    U = workloads.uniforms(rng, 6)
    full = run_sample(bigctx, x, T, K, P, U, cand_k=600)
    assert (full["status"] == 0).all(), full["status"]
    check_rows(oracle, x, T, K, P, U, full, label="unbounded call")
    for bound, ok in ((127, [True, True, True, True, False, False]), (600, [True] * 6), (500, [True] * 6)):
        d = run_sample(bigctx, x, T, K, P, U, cand_k=600, k_max=bound)
        for r in range(6):
            if ok[r]:
                assert d["status"][r] == 0 and d["token"][r] == full["token"][r], (bound, r)
                n = int(d["n_cand"][r])
                assert n == full["n_cand"][r], (bound, r)
                assert (d["cand_id"][r, :n] == full["cand_id"][r, :n]).all(), (bound, r)
                assert (d["cand_w"][r, :n] == full["cand_w"][r, :n]).all(), (bound, r)
            else:
                assert d["status"][r] == 7 and d["token"][r] == -1, (bound, r)  # XS_ROW_BAD_PARAM


def test_flat_rows_walk_the_whole_chain(bigctx, oracle):
    """Flat rows (N(0, 1) at T = 1, and equal logits) keep every weight above
    the sum's half-ulp, so the serial chains walk the whole sorted row: blocks
    crossed in one step from their grid units, carries into the next binade
    inside blocks, half-way terms, and cuts and draws far down the row (top_p
    0.5 and 0.95); quantised logits make many equal p (ties in id order)."""
    rng = np.random.default_rng(13128)
    rows = 8
    x = rng.normal(0, 1.0, (rows, V)).astype(np.float32)
    x[2] = np.round(x[2] * 4) / 4            # a few hundred distinct values
    x[3] = 0.0                               # every p equal
    x[4] = rng.uniform(-0.01, 0.01, V).astype(np.float32)
    x[5] = np.round(rng.normal(0, 3.0, V)).astype(np.float32)
    K = np.array([V, V, V, V, 10**6, V, 200_000, 50_000])
    P = np.array([0.95, 0.5, 0.95, 0.3, 1.0, 0.99, 0.95, 1.0])
    T = np.array([1.0, 1.0, 1.0, 1.0, 1.0, 0.8, 1.3, 1.0])
    U = workloads.uniforms(rng, rows)
    d = run_sample(bigctx, x, T, K, P, U, cand_k=4096)
    assert (d["status"] == 0).all(), d["status"]
    check_rows(oracle, x, T, K, P, U, d, label="flat whole rows")


def test_small_vocabularies_on_the_whole_row_path(oracle):
    """Whole rows of 129 to 9,000 ids (one partial block of chain terms, or
    none past the first 128), with masks and controls, top_k from 128 up."""
    from xwen_amd import sampler as xsm
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    rng = np.random.default_rng(14128)
    for enc in (129, 300, 4224, 4225, 9000):
        rows = 4
        ld = (enc + 3) // 4 * 4
        c = xsm.Context(max_rows=rows, vocab=ld, k_max=2**31 - 1)
        c.bind_current_stream()
        try:
            x = rng.normal(0, 1.5, (rows, ld)).astype(np.float32)
            allow = rng.random((rows, enc)) < np.array([[1.0], [0.7], [1.0], [0.9]])
            allow[:, 0] = True
            mask = workloads.pack_mask(allow)
            ctls = [None, None, xsm.SampleControl(banned=[1, 2, 3], bias=[(5, 2.0)]), None]
            K = [enc, 10**6, 128, max(128, enc - 1)]
            P = [0.9, 1.0, 0.95, 0.8]
            U = workloads.uniforms(rng, rows)
            d = run_sample(c, x, 1.0, K, P, U, enc=enc, mask=mask, ctls=ctls, cand_k=enc)
            assert (d["status"] == 0).all(), (enc, d["status"])
            check_rows(oracle, x, 1.0, K, P, U, d, enc=enc, mask=mask, ctls=ctls, label=f"enc {enc}")
        finally:
            c.close()


def test_tokens_only_rows_sort_what_the_sums_see(bigctx, oracle):
    """A call that returns tokens only, at top_k >= V, leaves p < 2^-26 out of
    the sort and the chains: each such term is added to a serial sum above
    0.5 and rounds back to it.  The same rows drawn with the full candidate
    list (every id sorted) and tokens only must give the same tokens, and the
    oracle's: rows with a few tall tokens (most terms left out), flat rows
    (none), masked rows (the masked ids at p = 0), top_p 0.8, 0.95 and 1, and
    uniforms from 0 to 1 - 2^-24."""
    rng = np.random.default_rng(8133)
    rows = 12
    x = np.empty((rows, V), np.float32)
    for r in range(rows):
        kind = r % 3
        if kind == 0:    # a few tall tokens over the bulk
            x[r] = rng.normal(0, 2.5, V).astype(np.float32)
            x[r, rng.integers(0, V, 8)] = rng.uniform(8, 14, 8).astype(np.float32)
        elif kind == 1:  # flat
            x[r] = rng.normal(0, 1, V).astype(np.float32)
        else:            # one dominant token
            x[r] = rng.normal(0, 3, V).astype(np.float32)
            x[r, rng.integers(0, V)] = np.float32(30.0)
    allow = rng.random((rows, V)) < 0.3
    allow[np.arange(rows), np.argmax(x, axis=1)] = True
    mask = workloads.pack_mask(allow)
    K = np.array([V, 10**6] * 6)
    T = np.array([1.0, 0.7, 1.3, 1.0] * 3)
    P = np.array([0.8, 0.95, 1.0] * 4)
    # (masked rows of top_k >= 128 take the serial denominator on every call
    # shape, so both calls draw them as the literal reference does)
    for m in (None, mask):
        for U in (workloads.uniforms(rng, rows),
                  np.array([0.0, 2.0**-24, 0.5, 1 - 2.0**-24] * 3, np.float32),
                  np.full(rows, 1 - 2.0**-24, np.float32)):
            Pm = P
            full = run_sample(bigctx, x, T, K, Pm, U, mask=m, cand_k=V)
            toks = run_sample(bigctx, x, T, K, Pm, U, mask=m, cand_k=0, stats=False)
            assert (full["status"] == 0).all() and (toks["status"] == 0).all()
            np.testing.assert_array_equal(toks["token"], full["token"])
            check_rows(oracle, x, T, K, Pm, U, full, mask=m, label="tokens only vs full sort")
