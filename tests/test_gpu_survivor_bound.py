"""The row's survivor bound and the finalizer's survivor sort across row shapes
that stress them, against the CPU oracle: allow-masks of a few contiguous
ranges (few sub-records hold a finite value, so the bound comes from each
chunk's top group maxima rather than one key per sub-record), masks with
fewer finite ids than K', and dense rows at K' = 64 and 65, whose survivors can
outnumber one wave's lanes."""
import numpy as np
import pytest

from tests import workloads
from tests.test_gpu_sampler import check_rows, run_sample

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


def _uniforms(rng, n):
    return rng.integers(0, 1 << 23, n).astype(np.float32) * np.float32(2.0 ** -23)


def test_range_masks(ctx, oracle):
    rng = np.random.default_rng(81)
    rows = 24
    x = rng.standard_normal((rows, V), dtype=np.float32) * np.float32(3.0)
    allow = np.zeros((rows, V), bool)
    for r in range(rows):
        n_ranges, width = [(1, 40), (2, 300), (4, V // 400), (8, 2000)][r % 4]
        for _ in range(n_ranges):
            s = int(rng.integers(0, V - width))
            allow[r, s:s + width] = True
    mask = workloads.pack_mask(allow)
    K = np.array([20, 50, 63, 1, 40, 64] * 4)
    T = np.array([1.0, 0.7, 1.3, 1.0] * 6)
    P = np.array([0.95, 1.0, 0.9, 0.5, 1.0, 0.8] * 4)
    U = _uniforms(rng, rows)
    d = run_sample(ctx, x, T, K, P, U, mask=mask, cand_k=128)
    assert (d["status"] == 0).all(), d["status"]
    check_rows(oracle, x, T, K, P, U, d, mask=mask, margins=False, label="range masks")
    for r in range(rows):
        assert allow[r, d["token"][r]]


def test_fewer_finite_ids_than_k(ctx, oracle):
    """10 to 60 allowed ids scattered over the whole row, K' up to 64."""
    rng = np.random.default_rng(82)
    rows = 12
    x = rng.standard_normal((rows, V), dtype=np.float32) * np.float32(3.0)
    allow = np.zeros((rows, V), bool)
    for r in range(rows):
        allow[r, rng.choice(V, 10 + 5 * r, replace=False)] = True
    mask = workloads.pack_mask(allow)
    K = np.array([63, 20, 40, 64] * 3)
    T = np.array([1.0] * 6 + [0.6] * 6)
    P = np.array([1.0, 0.95, 0.9] * 4)
    U = _uniforms(rng, rows)
    d = run_sample(ctx, x, T, K, P, U, mask=mask, cand_k=128)
    assert (d["status"] == 0).all(), d["status"]
    check_rows(oracle, x, T, K, P, U, d, mask=mask, margins=False, label="sparse ids")


def test_dense_rows_at_k64(ctx, oracle):
    """K' = 64 (top_k 63) and 65 over N(0, s^2) rows of several spreads, and rows whose top
    hundreds of logits sit in a narrow band: many survivors per row."""
    rng = np.random.default_rng(83)
    rows = 32
    x = np.empty((rows, V), np.float32)
    for r in range(rows):
        x[r] = rng.standard_normal(V, dtype=np.float32) * np.float32([0.5, 1.0, 3.0, 8.0][r % 4])
        if r % 8 == 7:  # a plateau: 300 ids within 1e-3 of each other at the top
            ids = rng.choice(V, 300, replace=False)
            x[r, ids] = np.float32(40.0) + rng.uniform(0, 1e-3, 300).astype(np.float32)
    K = np.array([63, 63, 63, 64] * 8)
    T = np.array([1.0, 0.8, 1.5, 1.0] * 8)
    P = np.array([1.0, 0.99, 0.9, 1.0] * 8)
    U = _uniforms(rng, rows)
    d = run_sample(ctx, x, T, K, P, U, cand_k=128)
    assert (d["status"] == 0).all(), d["status"]
    check_rows(oracle, x, T, K, P, U, d, margins=False, label="dense k64")


def test_subnormal_boundary_ties(ctx, oracle):
    """Rows whose k-th probability is subnormal: neighbouring logits round to
    the same p, so the candidate set keeps the lowest ids of a p-tie that
    reaches past the selection.  Heavy-tailed rows (Student-t(3) x 2, as C5),
    and rows whose tied band sits mostly in one chunk, more than K' deep, so
    that chunk's entries stop inside the band and its logits are read."""
    rng = np.random.default_rng(84)
    rows = 12
    x = np.empty((rows, V), np.float32)
    for r in range(8):
        z = rng.standard_normal(V, dtype=np.float32)
        chi = sum(rng.standard_normal(V, dtype=np.float32) ** 2 for _ in range(3))
        x[r] = z / np.sqrt(chi / np.float32(3.0)) * np.float32(2.0)
    for r in range(8, rows):
        x[r] = rng.normal(-200.0, 1.0, V).astype(np.float32)
        x[r, 5 + 1000 * r] = np.float32(0.0)
        deep = 2 * 16384 + rng.choice(16384, 40, replace=False)      # chunk 2: 40 band values
        light = 9 * 16384 + rng.choice(16384, 10, replace=False)     # chunk 9: 10 more
        x[r, deep] = rng.uniform(-100.03, -100.0, 40).astype(np.float32)
        x[r, light] = rng.uniform(-100.03, -100.0, 10).astype(np.float32)
    T = np.array([1.0, 0.7, 1.3, 1.0, 1.0, 0.6, 1.0, 1.0, 1.0, 1.0, 1.0, 1.0])
    K = np.array([20, 20, 50, 100, 5, 20, 63, 2, 20, 21, 10, 50])
    P = np.array([0.95, 1.0, 0.95, 1.0, 1.0, 0.8, 1.0, 1.0, 1.0, 1.0, 0.999, 1.0])
    U = _uniforms(rng, rows)
    d = run_sample(ctx, x, T, K, P, U, cand_k=128)
    assert (d["status"] == 0).all(), d["status"]
    check_rows(oracle, x, T, K, P, U, d, margins=False, label="subnormal ties")


def test_draws_inside_runs_of_equal_probability(ctx, oracle):
    """K' > 64 (the general finalizer) on rows whose top 140 logits are
    consecutive floats below 0.25 on scattered ids: neighbouring logits round
    to the same p, so the (p desc, id asc) order differs from the logit order
    inside runs that carry real weight.  With no candidate list requested the
    finalizer leaves that order to the draw; with one it sorts.  Many
    uniforms per row land draws inside the runs; tokens against the oracle."""
    rng = np.random.default_rng(85)
    base = rng.normal(-20.0, 1.0, V).astype(np.float32)
    vals = [np.float32(0.25)]
    for _ in range(139):
        vals.append(np.nextafter(vals[-1], np.float32(-1.0)))
    ids = rng.choice(V, 140, replace=False)
    row = base.copy()
    row[ids] = np.array(vals, np.float32)
    rows = 32
    x = np.repeat(row[None, :], rows, axis=0)
    T = np.where(np.arange(rows) % 4 == 3, 0.9, 1.0)
    K = np.where(np.arange(rows) % 2 == 0, 100, 127)
    P = np.where(np.arange(rows) % 3 == 0, 0.9, 1.0)
    U = ((np.arange(rows) + 0.5) / rows).astype(np.float32)
    U = (np.floor(U * (1 << 23)) * 2.0 ** -23).astype(np.float32)
    for cand_k in (0, 128):
        d = run_sample(ctx, x, T, K, P, U, cand_k=cand_k)
        assert (d["status"] == 0).all(), d["status"]
        check_rows(oracle, x, T, K, P, U, d, margins=False, label=f"equal-p runs cand_k={cand_k}")


@pytest.mark.parametrize("background", ["flat", "normal"])
def test_thousands_of_subnormal_ties(ctx, oracle, background):
    """One dominant logit and thousands of logits whose p rounds to the
    smallest subnormal, packed into two chunks (their filter floors lie inside
    the tied band, so both chunks' logits are read): the tie list fills and
    keeps its lowest ids, and the read stops once the ties below the next
    chunk's first id are enough.  On a flat background every wave overflows
    (its entries are then incomplete, so every chunk's logits are read); on a
    normal one the other chunks' entries are complete."""
    rng = np.random.default_rng(86)
    rows = 4
    if background == "flat":
        x = np.full((rows, V), np.float32(-200.0))
    else:
        x = rng.normal(-200.0, 1.0, (rows, V)).astype(np.float32)
    for r in range(rows):
        x[r, 5 + r] = np.float32(0.0)
        c1 = 16384 + rng.choice(16384, 500, replace=False)
        c3 = 3 * 16384 + rng.choice(16384, 3000, replace=False)
        x[r, c1] = rng.uniform(-103.7, -103.3, 500).astype(np.float32)
        x[r, c3] = rng.uniform(-103.7, -103.3, 3000).astype(np.float32)
    T = np.ones(rows)
    K = np.array([127, 100, 64, 127])
    P = np.ones(rows)
    U = np.array([0.0, 0.5, 0.999, 0.25], np.float32)
    for cand_k in (128, 0):
        d = run_sample(ctx, x, T, K, P, U, cand_k=cand_k)
        assert (d["status"] == 0).all(), d["status"]
        check_rows(oracle, x, T, K, P, U, d, margins=False, label=f"subnormal ties {background} cand_k={cand_k}")


def test_kth_largest_over_few_finite_keys(ctx, oracle):
    """The K'-th largest key taken from compacted finite keys, at its edges.
    In the chunk bound (fewer than K' = 21 finite group maxima in a chunk):
    80 finite lane maxima in 20 four-lane groups, 20 (fewer than K'), 21
    (exactly K'), and one id.  In the finalizer's four-key bound (fewer than
    2K' sub-records with a finite first key): whole chunks allowed, 8 of them
    (128 finite keys, the most the compaction takes), 9 and 10 (144 and 160:
    the bitwise search), 11 (44 first keys: the one-key bound); and K' = 64
    and 41, where the chunk bound comes from lane maxima."""
    rng = np.random.default_rng(87)
    rows = 10
    x = rng.standard_normal((rows, V), dtype=np.float32) * np.float32(3.0)
    allow = np.zeros((rows, V), bool)
    chunk = 16 * 1024
    base = 5 * chunk + 3 * 1024  # slot 3 of chunk 5
    for g in range(20):          # group g covers ids 16g .. 16g + 15 of the slot (lanes 4g .. 4g + 3)
        allow[0, base + 16 * g: base + 16 * g + 16] = True
    for g in range(5):
        allow[1, base + 16 * g: base + 16 * g + 16] = True
        allow[2, base + 16 * g: base + 16 * g + 16] = True
    allow[2, base + 16 * 7: base + 16 * 7 + 4] = True  # one more lane, in a sixth group
    allow[3, base + 77] = True
    picks = [1, 3, 5, 7, 9, 11, 13, 14, 2, 6, 10]
    for r, c in zip(range(4, 10), [8, 9, 10, 11, 8, 10]):
        for ch in picks[:c]:
            allow[r, ch * chunk:(ch + 1) * chunk] = True
    mask = workloads.pack_mask(allow)
    K = np.array([20, 20, 20, 20, 20, 20, 20, 20, 63, 40])
    T = np.array([1.0, 0.7] * 5)
    P = np.array([0.9, 0.9, 1.0, 0.9, 0.9, 1.0, 0.9, 0.9, 0.95, 0.9])
    U = _uniforms(rng, rows)
    d = run_sample(ctx, x, T, K, P, U, mask=mask, cand_k=128)
    assert (d["status"] == 0).all(), d["status"]
    check_rows(oracle, x, T, K, P, U, d, mask=mask, margins=False, label="few finite keys")
    for r in range(rows):
        assert allow[r, d["token"][r]]
