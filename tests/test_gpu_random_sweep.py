"""Seeded random parity sweep: batches of varied logit distributions (normal at
several scales, Student-t, tall peaks over a bulk, values quantized so that
exact ties are common, all-negative ties, Gumbel), random T / top_k / top_p
per row (greedy rows, K' across the fast and general finalizers), some with
random allow-masks, at three row widths; every row held to the oracle by the
same bar as the configured cases.  Batches of 24 rows spread each row over
the XCDs; batches of 72 (8 rows per XCD and more, a padded last group) take
the XCD-local hand-off."""
import numpy as np
import pytest

from tests import workloads
from tests.test_gpu_sampler import check_rows, run_sample

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from xwen_amd import sampler as xsm
    c = xsm.Context(max_rows=64, vocab=workloads.V)
    c.bind_current_stream()
    yield c
    c.close()


@pytest.fixture(scope="module")
def ctx_wide():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from xwen_amd import sampler as xsm
    c = xsm.Context(max_rows=128, vocab=workloads.V)
    c.bind_current_stream()
    yield c
    c.close()


def _batch(b, rows=24):
    rng = np.random.default_rng(90_000 + b)
    v = int(rng.choice([4096, 65536, 248320]))
    kind = b % 6
    if kind == 0:
        x = rng.normal(0, rng.choice([0.5, 1, 3, 8]), (rows, v))
    elif kind == 1:
        x = rng.standard_t(3, (rows, v)) * 2
    elif kind == 2:
        x = rng.normal(0, 3, (rows, v))
        for r in range(rows):
            ids = rng.choice(v, int(rng.integers(1, 6)), replace=False)
            x[r, ids] = x[r].max() + rng.uniform(5, 50, len(ids))
    elif kind == 3:
        x = np.round(rng.normal(0, 2, (rows, v)) * 4) / 4
    elif kind == 4:
        x = np.round(rng.normal(0, 1, (rows, v)), 1) - 30.0
    else:
        x = rng.gumbel(0, 1.5, (rows, v))
    x = x.astype(np.float32)
    T = rng.choice([0.0, 0.05, 0.3, 0.7, 1.0, 1.5, 2.0], rows)
    K = rng.choice([1, 2, 5, 20, 50, 64, 65, 100, 127], rows)
    P = rng.choice([0.3, 0.8, 0.95, 0.999, 1.0], rows)
    U = rng.random(rows).astype(np.float32)
    mask = None
    if b % 4 == 3:
        allow = rng.random((rows, v)) < rng.choice([0.01, 0.1, 0.5])
        allow[np.arange(rows), rng.integers(0, v, rows)] = True
        mask = workloads.pack_mask(allow)
    return x, T, K, P, U, mask, f"sweep batch {b} kind {kind} v {v}"


@pytest.mark.parametrize("b", range(18))
def test_random_batch(ctx, oracle, b):
    x, T, K, P, U, mask, label = _batch(b)
    d = run_sample(ctx, x, T, K, P, U, mask=mask)
    check_rows(oracle, x, T, K, P, U, d, mask=mask, label=label)


@pytest.mark.parametrize("b", range(6))
def test_random_batch_xcd_local(ctx_wide, oracle, b):
    x, T, K, P, U, mask, label = _batch(200 + b, rows=72)
    d = run_sample(ctx_wide, x, T, K, P, U, mask=mask)
    check_rows(oracle, x, T, K, P, U, d, mask=mask, label=label + " (72 rows)")


def _control_batch(b, rows=24):
    from xwen_amd import sampler as xsm
    rng = np.random.default_rng(70_000 + b)
    v = int(rng.choice([4096, 65536, 248320]))
    x = rng.standard_t(3, (rows, v)) * 2 if b % 2 else rng.normal(0, 3, (rows, v))
    if b % 3 == 2:
        x = np.round(x * 2) / 2
    x = x.astype(np.float32)
    T = rng.choice([0.0, 0.3, 0.7, 1.0, 1.5], rows)
    K = rng.choice([1, 5, 20, 64, 100], rows)
    P = rng.choice([0.5, 0.9, 1.0], rows)
    U = rng.random(rows).astype(np.float32)
    ctls = []
    for r in range(rows):
        if rng.integers(0, 6) == 0:
            ctls.append(None)
            continue
        banned = [int(i) for i in rng.choice(v + 50, int(rng.integers(0, 40)))]  # some past the vocabulary
        if rng.random() < 0.5:
            banned.append(int(np.argmax(x[r])))
        bias = [(int(i), float(rng.normal(0, 4))) for i in rng.choice(v, int(rng.integers(0, 30)))]
        pull = (int(rng.integers(0, v)), float(rng.choice([0.25, 0.5, 1.0, 1.5]))) if rng.random() < 0.4 else None
        force = int(rng.integers(0, v + 3)) if rng.random() < 0.15 else None
        ctls.append(xsm.SampleControl(banned=banned, bias=bias, pull=pull, force=force))
    mask = None
    if b % 4 == 3:
        allow = rng.random((rows, v)) < rng.choice([0.02, 0.3])
        allow[np.arange(rows), rng.integers(0, v, rows)] = True
        mask = workloads.pack_mask(allow)
    return x, T, K, P, U, ctls, mask, f"control sweep batch {b} v {v}"


@pytest.mark.parametrize("b", range(6))
def test_random_controls_batch(ctx, oracle, b):
    """Random sparse controls per row: bans (some past the vocabulary, some of
    the argmax), biases, pulls up to alpha 1.5 and forces (some out of range),
    with and without an allow-mask."""
    x, T, K, P, U, ctls, mask, label = _control_batch(b)
    d = run_sample(ctx, x, T, K, P, U, ctls=ctls, mask=mask)
    check_rows(oracle, x, T, K, P, U, d, ctls=ctls, mask=mask, label=label)


@pytest.mark.parametrize("b", range(3))
def test_random_controls_batch_xcd_local(ctx_wide, oracle, b):
    """The same random controls over 72 rows (the XCD-local hand-off)."""
    x, T, K, P, U, ctls, mask, label = _control_batch(100 + b, rows=72)
    d = run_sample(ctx_wide, x, T, K, P, U, ctls=ctls, mask=mask)
    check_rows(oracle, x, T, K, P, U, d, ctls=ctls, mask=mask, label=label + " (72 rows)")


@pytest.mark.parametrize("b", range(8))
def test_random_verify_block(ctx, oracle, b):
    """xs_verify over a random block: 1-8 sequences of span 1-8, drafts that are
    the row's argmax, its sampled token or a random id, random budgets (0
    included) and EOG ids taken from the sampled tokens; the walk must equal
    accept_drafts (src/generate.rs:4020-4046) over the same row tokens."""
    rng = np.random.default_rng(50_000 + b)
    _verify_block(ctx, oracle, rng, int(rng.integers(1, 9)), int(rng.integers(1, 9)), b)


@pytest.mark.parametrize("b", range(4))
def test_random_verify_block_xcd_local(ctx_wide, oracle, b):
    """The same over blocks of 64-128 rows (spans 4-16), whose rows hand off
    XCD-locally and whose sequences are walked by the last row's finalizer."""
    rng = np.random.default_rng(51_000 + b)
    span = int(rng.integers(4, 17))
    seqs = int(rng.integers(-(-64 // span), 128 // span + 1))
    _verify_block(ctx_wide, oracle, rng, seqs, span, b)


def _verify_block(ctx, oracle, rng, seqs, span, b):
    from xwen_amd import sampler as xsm
    rows, v = seqs * span, int(rng.choice([4096, 65536, 248320]))
    x = (rng.normal(0, 3, (rows, v)) if b % 2 else rng.standard_t(3, (rows, v)) * 2).astype(np.float32)
    T = rng.choice([0.0, 0.7, 1.0], rows)
    K = rng.choice([1, 20, 50], rows)
    P = rng.choice([0.9, 1.0], rows)
    U = rng.random(rows).astype(np.float32)
    d = run_sample(ctx, x, T, K, P, U)
    check_rows(oracle, x, T, K, P, U, d, label=f"verify sweep {b}", margins=False)
    tok = d["token"].reshape(seqs, span)
    arg = np.argmax(x, axis=1).reshape(seqs, span)
    pick = rng.integers(0, 3, (seqs, span))
    drafts = np.where(pick == 0, arg, np.where(pick == 1, tok, rng.integers(0, v, (seqs, span))))
    drafts = np.ascontiguousarray(drafts[:, :max(span - 1, 1)].astype(np.int32))
    eog = [int(t) for t in rng.choice(tok.ravel(), min(2, rows), replace=False)]
    budgets = rng.integers(0, span + 2, seqs).astype(np.int32)
    lg = torch.as_tensor(x).cuda()
    p = xsm.params_tensor(T, K, P, rows, "cuda")
    u = torch.as_tensor(U).cuda()
    out = xsm.verify_batch(ctx, lg, seqs, span, p, u, torch.as_tensor(drafts).cuda(),
                           budget=torch.as_tensor(budgets).cuda(), eog=eog)
    torch.cuda.synchronize()
    row_tok = out.row_token.cpu().numpy()
    np.testing.assert_array_equal(row_tok, d["token"])
    acc, com = out.accepted.cpu().numpy(), out.committed.cpu().numpy()
    ncom, sst = out.n_committed.cpu().numpy(), out.seq_status.cpu().numpy()
    for s in range(seqs):
        toks = list(row_tok[s * span:(s + 1) * span])
        st, m, committed, _ = oracle.accept_drafts(list(drafts[s][:span - 1]), int(budgets[s]), toks,
                                                   [t in eog for t in toks])
        assert (sst[s], acc[s], ncom[s]) == (st, m, len(committed)), (b, s)
        assert list(com[s, :ncom[s]]) == committed, (b, s)


@pytest.mark.parametrize("b", range(6))
def test_random_held_row_statistics(ctx, oracle, b):
    """held_row (src/generate.rs:1871-1933) on the sweep's distributions (no
    mask: held_row takes none), checked as check_held_row states; the draws
    held to the oracle as every row."""
    from tests.test_gpu_sampler import check_held_row
    x, T, K, P, U, _, label = _batch(b)
    n_top = int(np.random.default_rng(b).choice([1, 8, 20, 64]))
    d = run_sample(ctx, x, T, K, P, U, n_top=n_top)
    check_rows(oracle, x, T, K, P, U, d, label=label + " held_row")
    for r in range(x.shape[0]):
        check_held_row(oracle, x[r], d, r, n_top, label=label)


@pytest.fixture(scope="module")
def bigctx():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from xwen_amd import sampler as xsm
    c = xsm.Context(max_rows=16, vocab=workloads.V, k_max=2**31 - 1)
    c.bind_current_stream()
    yield c
    c.close()


@pytest.mark.parametrize("b", range(8))
def test_random_whole_row_batch(bigctx, oracle, b):
    """The whole-row path (top_k of 128 up to past the vocabulary) over the
    sweep's distributions, with masks and sparse controls on some batches."""
    from xwen_amd import sampler as xsm
    x, T, _, P, U, mask, label = _batch(200 + b)
    rows = 12
    x, T, P, U = x[:rows], T[:rows], P[:rows], U[:rows]
    mask = None if mask is None else mask[:rows]
    v = x.shape[1]
    rng = np.random.default_rng(60_000 + b)
    T = np.where(T == 0.0, 1.0, T)  # (greedy rows never reach the path)
    K = rng.choice([128, 129, 500, 1000, 5000, 2**31 - 1], rows)
    ctls = None
    if b % 3 == 1:
        ctls = [None if r % 3 == 0 else
                xsm.SampleControl(banned=[int(i) for i in rng.choice(v, 20)],
                                  bias=[(int(i), float(rng.normal(0, 3))) for i in rng.choice(v, 10)])
                for r in range(rows)]
    d = run_sample(bigctx, x, T, K, P, U, mask=mask, ctls=ctls, cand_k=5000)
    check_rows(oracle, x, T, K, P, U, d, mask=mask, ctls=ctls, label="whole-row " + label)
