"""Drafter confidence on the device: xs_argmax_probs (argmax_probs_device /
draft_argmax_probs, generate.rs:4059-4087) through the C ABI.

The bar: ids bit-exact (first maximal id, ties to the lower id); the
probability of the argmax within 1e-5 of 1 / sum exp(l - max) summed in f64,
the reference's own scalar check (draft_argmax_probs_matches_scalar,
generate.rs:5520-5552), and within PROB_RTOL relative at full width.
"""
import numpy as np
import pytest

from tests import workloads

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

PROB_RTOL = 1e-5
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


def _want(rows):
    """First maximal id and 1 / sum exp(f64(l - max)), as the reference's test
    computes them (generate.rs:5533-5544)."""
    ids, probs = [], []
    for row in rows:
        arg = int(np.argmax(row))  # numpy returns the first maximal index
        s = np.exp((row - row[arg]).astype(np.float64)).sum()
        ids.append(arg)
        probs.append(np.float32(1.0 / s))
    return np.array(ids), np.array(probs, np.float32)


def _run(ctx, x, width=None):
    from xwen_amd import sampler as xsm
    x = np.ascontiguousarray(x, np.float32)
    ids, probs = xsm.draft_argmax_probs(ctx, torch.as_tensor(x).to("cuda"), width=width)
    return ids, probs


def test_reference_known_answer(ctx, golden):
    c = golden["draft_argmax_probs"]
    i = np.arange(c["n"] * c["vocab"], dtype=np.float32)
    data = (np.sin(i * np.float32(c["step"])) * np.float32(c["amp"])).astype(np.float32)
    rows = data.reshape(c["n"], c["vocab"])
    ld = (c["vocab"] + 3) // 4 * 4
    x = np.full((c["n"], ld), np.nan, np.float32)  # padding past `width` is never read
    x[:, : c["vocab"]] = rows
    ids, probs = _run(ctx, x, width=c["vocab"])
    want_ids, want_p = _want(rows)
    assert (ids == want_ids).all()
    assert np.abs(probs - want_p).max() < c["p_tol"]


def test_full_width_batch_of_drafter_rows(ctx):
    # 15 drafter rows (the reference's draft depth) at V, peaked and flat
    rng = np.random.default_rng(11)
    x = rng.normal(0, 3, (15, V)).astype(np.float32)
    for r in range(0, 15, 2):
        x[r, rng.integers(0, V)] = np.float32(rng.uniform(8, 20))
    x[3] *= np.float32(0.01)  # nearly flat: p ~ 1/V
    ids, probs = _run(ctx, x)
    want_ids, want_p = _want(x)
    assert (ids == want_ids).all()
    np.testing.assert_allclose(probs, want_p, rtol=PROB_RTOL, atol=0)


def test_ties_take_the_lower_id_and_special_rows(ctx):
    rng = np.random.default_rng(12)
    x = rng.normal(0, 1, (6, V)).astype(np.float32)
    x[0, [70000, 5, 248000]] = np.float32(9.0)          # tie: id 5 wins, p ~ 1/3
    x[1, 123456] = np.nan                                # NaN: id -1, p NaN
    x[2, [40, 41]] = np.inf                              # +inf: first inf id, p NaN
    x[3, :] = -np.inf                                    # nothing above -inf: id -1, p NaN
    x[4, :] = np.float32(0.5)                            # constant row: id 0, p = 1/V
    x[5, V - 1] = np.float32(30.0)                       # last id, p ~ 1
    ids, probs = _run(ctx, x)
    assert ids[0] == 5 and ids[1] == -1 and ids[2] == 40 and ids[3] == -1
    assert ids[4] == 0 and ids[5] == V - 1
    assert np.isnan(probs[1]) and np.isnan(probs[2]) and np.isnan(probs[3])
    want_ids, want_p = _want(x[[0, 4, 5]])
    np.testing.assert_allclose(probs[[0, 4, 5]], want_p, rtol=PROB_RTOL, atol=0)
    assert abs(probs[4] * V - 1.0) < 1e-5


def test_keep_confident_over_device_probabilities(ctx):
    # the drafter walk: draft ids whose probabilities clear the floor, in order
    from xwen_amd import sampler as xsm
    rng = np.random.default_rng(13)
    x = rng.normal(0, 1, (4, V)).astype(np.float32)
    for r, spike in enumerate((30.0, 30.0, 2.0, 30.0)):
        x[r, 1000 + r] = np.float32(spike)
    ids, probs = _run(ctx, x)
    kept = xsm.keep_confident(list(ids), probs, 0.5)
    assert kept == [1000, 1001]


@pytest.mark.parametrize("b", range(6))
def test_random_drafter_blocks(ctx, b):
    """Seeded random blocks: 1-15 rows of width 17-V, normal, Student-t and
    quantized (exact ties at the top) logits, some rows with a tall peak."""
    rng = np.random.default_rng(3_000 + b)
    n, width = int(rng.integers(1, 16)), int(rng.integers(17, V + 1))
    ld = (width + 3) // 4 * 4
    kind = b % 3
    if kind == 0:
        rows = rng.normal(0, rng.choice([0.3, 3.0]), (n, width))
    elif kind == 1:
        rows = rng.standard_t(3, (n, width)) * 2
    else:
        rows = np.round(rng.normal(0, 2, (n, width)) * 2) / 2
    rows = rows.astype(np.float32)
    for r in range(n):
        if rng.random() < 0.4:
            rows[r, rng.integers(0, width)] = rows[r].max() + np.float32(rng.uniform(1, 30))
    x = np.full((n, ld), np.nan, np.float32)  # padding past `width` is never read
    x[:, :width] = rows
    ids, probs = _run(ctx, x, width=width)
    want_ids, want_p = _want(rows)
    assert (ids == want_ids).all()
    np.testing.assert_allclose(probs, want_p, rtol=PROB_RTOL, atol=0)
