"""Controlled rows draw the literal reference's token on every call shape.

A controlled row (an allow-mask or sparse controls) is softmaxed by the
reference with a serial f32 sum (sampler.rs:301-305).  The device divides by
the exact sum unless the call observes the denominator at top_p >= 1, and its
finalizer checks that the serial sum could not change the token
(draw_settled); a row it cannot settle is summed serially by the finalizing
workgroup itself and drawn again.  So on every call shape -- tokens only, with
candidates, top_p < 1 or >= 1, verify blocks -- every controlled row's token
must equal the oracle's with SUM_SEQ_F32, with no margin rule.  The rows sent
to the fallback are counted (xs_test_serial_fallback) and printed.
"""
import numpy as np
import pytest

from tests import workloads
from tests.test_gpu_sampler import check_controlled, controlled_row, oracle_row, run_sample

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

V = workloads.V


@pytest.fixture(scope="module")
def ctx():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from xwen_amd import sampler as xsm
    c = xsm.Context(max_rows=64, vocab=V)
    c.bind_current_stream()
    yield c
    c.close()


def fallbacks(ctx, force=0):
    """Rows the finalizers summed serially on this context so far (synchronizes);
    force != 0 sends every checked row of later calls there."""
    import ctypes
    n = ctypes.c_uint32(0)
    assert ctx.lib.xs_test_serial_fallback(ctx.h, force, ctypes.byref(n)) == 0
    return int(n.value)


def check_all(oracle, x, T, K, P, U, d, *, mask=None, ctls=None, label=""):
    """Every row: controlled stochastic rows against the serial-f32 reference
    (token, ids, weights); greedy rows against the argmax; others by status and
    token against the exactly summed oracle where its margins are clear."""
    rows, v = x.shape
    T = np.broadcast_to(np.asarray(T, np.float64), (rows,))
    K = np.broadcast_to(np.asarray(K), (rows,))
    P = np.broadcast_to(np.asarray(P, np.float64), (rows,))
    U = np.broadcast_to(np.asarray(U, np.float32), (rows,))
    n_ctl = 0
    for r in range(rows):
        mrow = None if mask is None else mask[r]
        kw = {} if ctls is None else {"ctl": ctls[r]}
        tag = f"{label} row {r} T={T[r]} k={K[r]} p={P[r]}"
        if controlled_row(T[r], K[r], P[r], mrow, kw.get("ctl")):
            check_controlled(oracle, x[r], v, T[r], K[r], P[r], U[r], d, r, mrow, kw, tag)
            n_ctl += 1
            continue
        o = oracle_row(oracle, x[r], v, T[r], K[r], P[r], U[r], mrow, sum_mode=oracle.SUM_F64,
                       margins=True, **kw)
        assert d["status"][r] == o.status, (tag, d["status"][r], o.status)
        greedy = T[r] <= 0.0 or K[r] <= 1
        if o.status == 0 and (greedy or min(o.margin_order, o.margin_cut, o.margin_draw) > 1e-5):
            assert d["token"][r] == o.token, (tag, d["token"][r], o.token)
    return n_ctl


@pytest.mark.parametrize("top_p", [1.0, 0.95])
@pytest.mark.parametrize("shape", ["tokens", "candidates"])
def test_c3_rows_draw_the_serial_sum_token(ctx, oracle, top_p, shape):
    wl = workloads.c3_masked()
    rows = wl.logits.shape[0]
    before = fallbacks(ctx)
    d = run_sample(ctx, wl.logits, 1.0, 20, top_p, wl.u, mask=wl.mask,
                   cand_k=20 if shape == "candidates" else 0, stats=shape == "candidates")
    n = check_all(oracle, wl.logits, 1.0, 20, top_p, wl.u, d, mask=wl.mask, label=f"C3 p={top_p} {shape}")
    assert n == rows
    print(f"\nC3 top_p={top_p} {shape}: {n} controlled rows, {fallbacks(ctx) - before} summed serially by "
          f"their finalizer")


def _control_batch(b, v):
    from xwen_amd import sampler as xsm
    rng = np.random.default_rng(60_000 + b)
    rows = 24
    x = (rng.standard_t(3, (rows, v)) * 2 if b % 2 else rng.normal(0, 3, (rows, v))).astype(np.float32)
    if b % 3 == 2:
        x = (np.round(x * 2) / 2).astype(np.float32)  # exact ties
    T = rng.choice([0.0, 0.3, 0.7, 1.0, 1.5], rows)
    K = rng.choice([1, 5, 20, 64, 100], rows)
    P = rng.choice([0.5, 0.9, 0.95, 1.0], rows)
    U = rng.random(rows).astype(np.float32)
    ctls = []
    for r in range(rows):
        if rng.random() < 0.25:
            ctls.append(None)
            continue
        c = xsm.SampleControl()
        c.banned = [int(i) for i in rng.integers(0, v, int(rng.integers(0, 40)))]
        c.bias = [(int(i), float(rng.normal(0, 4))) for i in rng.integers(0, v, int(rng.integers(0, 40)))]
        if rng.random() < 0.2:
            c.pull = (int(rng.integers(0, v)), float(rng.choice([0.25, 0.5, 1.0])))
        if rng.random() < 0.05:
            c.force = int(rng.integers(0, v))
        ctls.append(c)
    mask = None
    if b % 2 == 1:
        allow = rng.random((rows, v)) < rng.choice([0.01, 0.1, 0.5])
        allow[np.arange(rows), rng.integers(0, v, rows)] = True
        mask = workloads.pack_mask(allow)
    return x, T, K, P, U, ctls, mask


@pytest.mark.parametrize("b", range(6))
@pytest.mark.parametrize("shape", ["tokens", "candidates"])
def test_random_controls_draw_the_serial_sum_token(ctx, oracle, b, shape):
    v = [4096, 65536, V][b % 3]
    x, T, K, P, U, ctls, mask = _control_batch(b, v)
    before = fallbacks(ctx)
    d = run_sample(ctx, x, T, K, P, U, ctls=ctls, mask=mask, cand_k=128 if shape == "candidates" else 0,
                   stats=shape == "candidates")
    n = check_all(oracle, x, T, K, P, U, d, mask=mask, ctls=ctls, label=f"controls {b} {shape} v {v}")
    print(f"\ncontrols batch {b} {shape}: {n} controlled rows, {fallbacks(ctx) - before} summed serially")


def _boundary_uniforms(oracle, x, T, K, P, mask, rng):
    """Per row, a uniform whose draw lands on a cumulative-weight boundary of the
    serial-f32 reference: the exact sum cannot settle such a token."""
    rows, v = x.shape
    U = np.zeros(rows, np.float32)
    for r in range(rows):
        o = oracle_row(oracle, x[r], v, T, K, P, 0.0, mask[r], sum_mode=oracle.SUM_SEQ_F32)
        w = np.array([c for c, _ in o.cand], np.float32)  # the weights after truncate_top_p
        cum, acc = [], np.float32(0.0)
        for t in w:
            acc = np.float32(acc + t)
            cum.append(acc)
        npos = int(np.count_nonzero(w))
        if npos < 2:  # one candidate with weight: no boundary below the total
            U[r] = np.float32(0.5)
            continue
        j = int(rng.integers(0, npos - 1))  # a boundary below the total: u < 1
        U[r] = np.float32(min(np.float64(cum[j]) / np.float64(cum[-1]), 1.0 - 2.0 ** -24))
    return U


@pytest.mark.parametrize("top_p", [1.0, 0.95])
def test_rows_on_a_draw_boundary_take_the_serial_sum(ctx, oracle, top_p):
    wl = workloads.c3_masked(seed=313, rows=16)
    rng = np.random.default_rng(77)
    U = _boundary_uniforms(oracle, wl.logits, 1.0, 20, top_p, wl.mask, rng)
    before = fallbacks(ctx)
    d = run_sample(ctx, wl.logits, 1.0, 20, top_p, U, mask=wl.mask, cand_k=0, stats=False)
    check_all(oracle, wl.logits, 1.0, 20, top_p, U, d, mask=wl.mask, label=f"boundary p={top_p}")
    sent = fallbacks(ctx) - before
    print(f"\nboundary uniforms top_p={top_p}: {sent} of 16 rows summed serially")
    assert sent >= 8  # (row 0 allows one id; the others sit on a boundary by construction)


@pytest.mark.parametrize("top_p", [1.0, 0.95, 0.5])
@pytest.mark.parametrize("shape", ["tokens", "candidates"])
def test_forced_fallback_matches_the_serial_reference(ctx, oracle, top_p, shape):
    """Every checked row sent to the finalizer's own serial sum: tokens, ids and
    (with candidates) weights equal the serial-f32 reference bit for bit."""
    wl = workloads.c3_masked(seed=323, rows=12)
    rows = wl.logits.shape[0]
    before = fallbacks(ctx, force=1)
    try:
        d = run_sample(ctx, wl.logits, 1.0, 20, top_p, wl.u, mask=wl.mask,
                       cand_k=20 if shape == "candidates" else 0, stats=shape == "candidates")
        sent = fallbacks(ctx, force=0) - before
    finally:
        fallbacks(ctx, force=0)
    check_all(oracle, wl.logits, 1.0, 20, top_p, wl.u, d, mask=wl.mask, label=f"forced p={top_p} {shape}")
    if shape == "candidates":
        for r in range(1, rows):  # row 0 allows one id: every sum is its single term
            oseq = oracle_row(oracle, wl.logits[r], V, 1.0, 20, top_p, wl.u[r], wl.mask[r],
                              sum_mode=oracle.SUM_SEQ_F32)
            ws = np.array([w for w, _ in oseq.cand], np.float32)
            np.testing.assert_array_equal(d["cand_w"][r, :len(ws)].view(np.uint32), ws.view(np.uint32))
            assert np.float32(d["soft_sum"][r]).view(np.uint32) == np.float32(oseq.ssum).view(np.uint32)
    # tokens only at top_p >= 1 and every call at top_p < 1 are checked; with
    # candidates at top_p >= 1 serial_kernel finalizes the rows instead; row 0
    # allows one id, whose draw needs no check
    expect = 0 if (shape == "candidates" and top_p >= 1.0) else rows - 1
    assert sent == expect, (sent, expect)


def test_verify_block_with_masks_walks_the_serial_sum_tokens(ctx, oracle):
    """A masked verify block (tokens only) against accept_drafts over the
    serial-f32 reference's tokens (generate.rs:4020-4046)."""
    from xwen_amd import sampler as xsm
    rng = np.random.default_rng(515)
    seqs, span = 4, 6
    rows = seqs * span
    x = (rng.normal(0, 3, (rows, V))).astype(np.float32)
    allow = rng.random((rows, V)) < 0.1
    mask = workloads.pack_mask(allow)
    U = workloads.uniforms(rng, rows)
    want = []
    for r in range(rows):
        o = oracle_row(oracle, x[r], V, 1.0, 20, 0.95, U[r], mask[r], sum_mode=oracle.SUM_SEQ_F32)
        assert o.status == 0
        want.append(o.token)
    drafts = np.array([[want[s * span + i] if (s + i) % 3 else int(rng.integers(0, V))
                        for i in range(span - 1)] for s in range(seqs)], np.int32)
    lg = torch.as_tensor(x).cuda()
    p = xsm.params_tensor(np.full(rows, 1.0), np.full(rows, 20), np.full(rows, 0.95), rows, "cuda")
    u = torch.as_tensor(U).cuda()
    m = torch.as_tensor(mask.view(np.int32)).cuda()
    vd = xsm.verify_batch(ctx, lg, seqs, span, p, u, torch.as_tensor(drafts).cuda(), allowed=m)
    torch.cuda.synchronize()
    for s in range(seqs):
        m_ok, committed = 0, []
        for i in range(span):
            t = want[s * span + i]
            committed.append(t)
            if i < span - 1 and t == drafts[s, i]:
                m_ok += 1
                continue
            break
        assert int(vd.accepted[s]) == m_ok, (s, int(vd.accepted[s]), m_ok)
        got = [int(t) for t in vd.committed[s].cpu().numpy()[:len(committed)]]
        assert got == committed, (s, got, committed)
