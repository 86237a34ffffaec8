"""held_row outputs beside a masked or controlled draw.

held_row (src/generate.rs:1905-1933) reads the raw logit row; the allow-mask
and SampleControl (src/sampler.rs:85-121) shape only the draw.  A call that
asks for both gets the masked draw and the raw row's statistics: bit for bit
what the same call without the held outputs draws, and the row_max and
top ids a call without mask or controls reports.  The f64 log-sums (row_lse,
the log-probs) agree with that call's to the held_row bar: held_row's serial
fold is emulated by partial sums whose grouping follows the finalizer a row's
draw takes, so their last bits may differ between the two calls (both stay
within the bar of the reference's fold).  Everything is also held to the
oracle.  Row counts of 24 (each row spread over the XCDs) and 72 (the
XCD-local hand-off) are covered."""
import numpy as np
import pytest

from tests import workloads
from tests.test_gpu_random_sweep import _batch, _control_batch
from tests.test_gpu_sampler import PROB_RTOL, check_held_row, check_rows, dev

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

SCORES = ("score_logprob", "class_mass", "probs")


@pytest.fixture(scope="module")
def ctx():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from xwen_amd import sampler as xsm
    c = xsm.Context(max_rows=128, vocab=workloads.V)
    c.bind_current_stream()
    yield c
    c.close()


def call(ctx, x, T, K, P, U, *, mask=None, ctls=None, noalloc=False, **kw):
    from xwen_amd import sampler as xsm
    rows = x.shape[0]
    p = xsm.params_tensor(T, K, P, rows, "cuda")
    m = None if mask is None else dev(np.asarray(mask, np.uint32).view(np.int32))
    c = None if ctls is None else xsm.controls_tensor(ctls, "cuda")
    if noalloc:
        out = xsm.sample_batch_noalloc(dev(x), p, dev(U), allowed=m, controls=c, **kw)
    else:
        out = xsm.sample_batch(ctx, dev(x), p, dev(U), allowed=m, controls=c, **kw)
    torch.cuda.synchronize()
    return {k: v.cpu().numpy() for k, v in vars(out).items() if v is not None}


def same_bits(a, b, keys, tag):
    for k in keys:
        x, y = a[k], b[k]
        if x.dtype.kind == "f":
            x = x.view(np.uint32 if x.itemsize == 4 else np.uint64)
            y = y.view(np.uint32 if y.itemsize == 4 else np.uint64)
        np.testing.assert_array_equal(x, y, err_msg=f"{tag}: {k}")


def close_held(a, b, tag, extra=()):
    """row_max and the top ids bit for bit; the f64 log-sums and what they
    normalize (log-probs, scores, class masses, probabilities) within the
    held_row bar: 1e-5 relative with a floor of eight f64 ulps of lse."""
    same_bits(a, b, ("row_max", "top_id"), tag)
    lse = b["row_lse"].astype(np.float64)
    floor = 8 * np.spacing(np.abs(lse))
    for k in ("row_lse", "top_logprob", "top_logprob64") + tuple(extra):
        x, y = a[k].astype(np.float64), b[k].astype(np.float64)
        fl = floor.reshape((-1,) + (1,) * (x.ndim - 1))
        bad = ~((np.abs(x - y) <= PROB_RTOL * np.abs(y) + fl) | (np.isnan(x) & np.isnan(y)))
        assert not bad.any(), (tag, k, np.argwhere(bad)[:5].tolist())


def _cases():
    out = []
    for b, rows in ((3, 24), (7, 72)):
        x, T, K, P, U, mask, label = _batch(b, rows=rows)
        out.append((f"{label}, {rows} masked rows", x, T, K, P, U, mask, None))
    for b, rows in ((1, 24), (3, 72), (4, 72)):
        x, T, K, P, U, ctls, mask, label = _control_batch(b, rows=rows)
        out.append((f"{label}, {rows} controlled rows", x, T, K, P, U, mask, ctls))
    return out


@pytest.mark.parametrize("case", range(5))
def test_held_row_beside_a_masked_draw(ctx, oracle, case):
    tag, x, T, K, P, U, mask, ctls = _cases()[case]
    n_top = 20
    both = call(ctx, x, T, K, P, U, mask=mask, ctls=ctls, n_top=n_top, cand_k=20, stats=True)
    draw = call(ctx, x, T, K, P, U, mask=mask, ctls=ctls, cand_k=20, stats=True)
    raw = call(ctx, x, T, K, P, U, n_top=n_top)
    same_bits(both, draw, [k for k in draw], tag + " (the draw)")
    close_held(both, raw, tag + " (held_row over the raw row)")
    check_rows(oracle, x, T, K, P, U, both, mask=mask, ctls=ctls, label=tag)
    for r in range(x.shape[0]):
        check_held_row(oracle, x[r], both, r, n_top, label=tag)
    print(f"{tag}: draw and held_row outputs as in the separate calls; "
          f"statuses {np.unique(both['status']).tolist()}")


def test_scoring_reads_beside_a_masked_draw(ctx):
    """last_logprobs_for, escape_mass's class sums and last_probs
    (generate.rs:1871-1899, batch.rs:1628-1669) of masked rows read the raw
    row; an id out of range still fails the caller's row (token -1)."""
    from xwen_amd import _lib
    x, T, K, P, U, mask, tag = _batch(7, rows=72)
    rows, v = x.shape
    rng = np.random.default_rng(5)
    ids = rng.integers(0, v, (rows, 6)).astype(np.int32)
    ids[5, 2] = v  # one past the encodable ids
    classes = rng.integers(-2**31, 2**31, (rows, 2, v // 32), dtype=np.int64).astype(np.int32)
    kw = dict(score_ids=dev(ids), class_masks=dev(classes), probs=True)
    both = call(ctx, x, T, K, P, U, mask=mask, n_top=8, cand_k=20, **kw)
    draw = call(ctx, x, T, K, P, U, mask=mask, cand_k=20)
    raw = call(ctx, x, T, K, P, U, n_top=8, **kw)
    assert both["status"][5] == _lib.ROW_ID_OOR and both["token"][5] == -1
    keep = np.arange(rows) != 5
    for k in draw:
        np.testing.assert_array_equal(both[k][keep], draw[k][keep], err_msg=k)
    close_held(both, raw, tag + " scoring reads", extra=SCORES)
    assert np.isnan(both["score_logprob"][5, 2])


def test_noalloc_held_row_beside_a_masked_draw(ctx):
    """xs_sample_noalloc takes the same two passes in its static workspace."""
    x, T, K, P, U, ctls, mask, tag = _control_batch(3, rows=24)
    kw = dict(mask=mask, ctls=ctls, n_top=20, cand_k=20, stats=True)
    a = call(ctx, x, T, K, P, U, **kw)
    b = call(ctx, x, T, K, P, U, noalloc=True, **kw)
    same_bits(a, b, list(a), tag + " noalloc")
