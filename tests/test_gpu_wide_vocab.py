"""Rows wider than 262,144 ids (more than 64 sub-records per row, so every row
takes the general finalizer over several sub-record groups), up to the
context limit of 1,048,576, against the CPU oracle."""
import numpy as np
import pytest

from tests.test_gpu_sampler import check_rows, run_sample

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

VMAX = 1_048_576


@pytest.fixture(scope="module")
def ctx():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from xwen_amd import sampler as xsm
    c = xsm.Context(max_rows=8, vocab=VMAX)
    c.bind_current_stream()
    yield c
    c.close()


def _rows(enc, seed, n=6):
    rng = np.random.default_rng(seed)
    ld = (enc + 3) // 4 * 4
    x = np.full((n, ld), np.float32(40.0), np.float32)  # padded ids past enc must never win
    x[:, :enc] = rng.normal(0, 3, (n, enc)).astype(np.float32)
    for r in range(n):
        x[r, rng.integers(0, enc, 10)] = rng.uniform(9, 14, 10).astype(np.float32)
    return x, rng


@pytest.mark.parametrize("enc", [262_145, 600_000, VMAX])
def test_wide_rows_sample_like_the_oracle(ctx, oracle, enc):
    x, rng = _rows(enc, enc)
    T = [1.0, 0.7, 0.0, 1.0, 1.3, 1.0]
    K = [20, 100, 1, 64, 127, 5]
    P = [0.95, 0.9, 1.0, 1.0, 0.8, 0.5]
    U = rng.integers(0, 1 << 23, 6).astype(np.float32) * np.float32(2.0 ** -23)
    d = run_sample(ctx, x, T, K, P, U, enc=enc, cand_k=127)
    assert (d["status"] == 0).all(), d["status"]
    assert (d["token"] < enc).all()
    check_rows(oracle, x, T, K, P, U, d, enc=enc, margins=False, label=f"enc={enc}")


def test_wide_rows_with_statistics_and_ties(ctx, oracle):
    """held_row statistics at V = 600,000, and a row whose top logits tie over
    many ids across many sub-records (survivors past one wave's sort)."""
    from tests import refimpl
    enc = 600_000
    x, rng = _rows(enc, 7, n=4)
    x[3, rng.choice(enc, 400, replace=False)] = np.float32(15.0)  # 400-way tie at the top
    T = [1.0, 0.0, 0.7, 1.0]
    K = [20, 1, 50, 30]
    P = [0.95, 1.0, 0.9, 1.0]
    U = [0.25, 0.0, 0.75, 0.5]
    d = run_sample(ctx, x, T, K, P, U, enc=enc, cand_k=64, n_top=20)
    assert (d["status"] == 0).all(), d["status"]
    check_rows(oracle, x, T, K, P, U, d, enc=enc, margins=False, label="wide stats")
    for r in range(4):
        st, mx, lse = oracle.held_row(x[r], enc)
        assert st == 0
        assert np.float32(d["row_max"][r]) == np.float32(mx)
        assert abs(d["row_lse"][r] - lse) <= 1e-5 * abs(lse)
        order = refimpl.stable_desc_order(x[r][:enc])[:20]
        assert list(d["top_id"][r]) == order.tolist(), r
