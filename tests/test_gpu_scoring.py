"""The scoring reads of held rows against the oracle at full width.

The reference's scored batch path reads its held logit row three ways
(batch.rs:1504-1521, :1628-1669): last_logprobs_for(ids) -> f64(v[id]) - lse,
an out-of-range id being an error (generate.rs:1871-1883); last_probs ->
exp(f64(v) - lse) for every encodable id (:1893-1899), which escape_mass sums
over token-text classes; and held_row's lse itself (:1905-1933, the serial f64
fold).  The device returns each without reading the row back: f64 log-probs of
caller ids, f64 top-n log-probs, per-class masses over caller bitmasks, and
the whole f64 distribution.  Held to the oracle at 1e-5 relative, with a floor
of four f64 ulps of lse on log-probs (a log-prob is v - lse, so lse's last bits
are all a dominant id's log-prob carries) -- on dominant rows too, where the
serial fold and an exact sum of the same terms differ by up to the whole
log-prob.
"""
import math

import numpy as np
import pytest

from tests import workloads

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

V = workloads.V
RTOL = 1e-5


@pytest.fixture(scope="module")
def ctx():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from xwen_amd import sampler as xsm
    c = xsm.Context(max_rows=16, vocab=V)
    c.bind_current_stream()
    yield c
    c.close()


def _rows(rng, n):
    x = rng.normal(0, 3, (n, V)).astype(np.float32)
    for r in range(n):
        kind = r % 4
        if kind == 1:    # a dominant token: the serial fold decides its log-prob
            x[r, [0, V // 2, V - 1, int(rng.integers(0, V))][r % 4]] = np.float32(x[r].max() + rng.uniform(20, 35))
        elif kind == 2:  # heavy tails
            x[r] = (rng.standard_t(3, V) * 2).astype(np.float32)
        elif kind == 3:  # a few tall tokens and -inf entries
            x[r, rng.integers(0, V, 6)] = rng.uniform(8, 14, 6).astype(np.float32)
            x[r, rng.integers(0, V, 1000)] = -np.inf
    return x


def _class_masks(rng, rows, n_class, enc):
    allow = rng.random((rows, n_class, enc)) < rng.uniform(0.05, 0.6, (rows, n_class, 1))
    words = (enc + 31) // 32
    out = np.zeros((rows, n_class, words), np.uint32)
    for r in range(rows):
        out[r] = workloads.pack_mask(allow[r])
    return out


def test_scoring_reads_match_the_oracle(ctx, oracle):
    from xwen_amd import sampler as xsm
    rng = np.random.default_rng(1871)
    rows, n_class, n_score = 8, 3, 24
    x = _rows(rng, rows)
    ids = rng.integers(0, V, (rows, n_score)).astype(np.int32)
    ids[:, 0] = np.argmax(x, axis=1)           # the argmax (a dominant row's tiny log-prob)
    ids[:, 1] = 0
    ids[:, 2] = V - 1
    masks = _class_masks(rng, rows, n_class, V)
    lg = torch.as_tensor(x).cuda()
    p = xsm.params_tensor(0.0, 1, 1.0, rows, "cuda")
    u = torch.zeros(rows, dtype=torch.float32, device="cuda")
    out = xsm.sample_batch(ctx, lg, p, u, n_top=20, score_ids=torch.as_tensor(ids).cuda(),
                           class_masks=torch.as_tensor(masks.view(np.int32)).cuda(), probs=True)
    torch.cuda.synchronize()
    st = out.status.cpu().numpy()
    lse = out.row_lse.cpu().numpy()
    slp = out.score_logprob.cpu().numpy()
    cm = out.class_mass.cpu().numpy()
    pr = out.probs.cpu().numpy()
    top64 = out.top_logprob64.cpu().numpy()
    top_id = out.top_id.cpu().numpy()
    for r in range(rows):
        tag = f"row {r}"
        s, mx, lse_o = oracle.held_row(x[r], V)
        assert st[r] == 0 and s == 0, tag
        floor = 4 * math.ulp(abs(lse_o))
        assert abs(lse[r] - lse_o) <= RTOL * abs(lse_o) + floor, (tag, lse[r], lse_o)
        s, want = oracle.last_logprobs_for(x[r], V, ids[r].astype(np.int64))
        assert s == 0
        np.testing.assert_allclose(slp[r], want, rtol=RTOL, atol=floor, err_msg=tag)
        s, po = oracle.last_probs(x[r], V)
        assert s == 0
        np.testing.assert_allclose(pr[r], po, rtol=RTOL, atol=1e-300, err_msg=tag)
        np.testing.assert_allclose(cm[r], oracle.class_masses(po, masks[r]), rtol=RTOL, atol=1e-300,
                                   err_msg=tag)
        np.testing.assert_allclose(top64[r], x[r][top_id[r]].astype(np.float64) - lse_o, rtol=RTOL,
                                   atol=floor, err_msg=tag)
        assert (pr[r][np.isneginf(x[r])] == 0.0).all(), tag


def test_an_out_of_range_id_fails_its_row(ctx, oracle):
    """last_logprobs_for's error (generate.rs:1874-1879): a row with an id at or
    past enc (or negative) reports XS_ROW_ID_OOR, token -1, and NaN at that id;
    its other ids and the other rows are scored as usual; a NaN row keeps its
    own error."""
    from xwen_amd import _lib, sampler as xsm
    rng = np.random.default_rng(1879)
    rows, enc = 4, V - 250
    x = rng.normal(0, 3, (rows, V)).astype(np.float32)
    x[3, 77] = np.nan
    ids = np.array([[1, 2, 3], [5, enc, 7], [-1, 9, 10], [1, 2, 3]], np.int32)
    lg = torch.as_tensor(x).cuda()
    p = xsm.params_tensor(0.0, 1, 1.0, rows, "cuda")
    u = torch.zeros(rows, dtype=torch.float32, device="cuda")
    out = xsm.sample_batch(ctx, lg, p, u, enc=enc, score_ids=torch.as_tensor(ids).cuda())
    torch.cuda.synchronize()
    st, tok = out.status.cpu().numpy(), out.token.cpu().numpy()
    slp = out.score_logprob.cpu().numpy()
    assert list(st) == [0, _lib.ROW_ID_OOR, _lib.ROW_ID_OOR, _lib.ROW_NAN]
    assert tok[1] == -1 and tok[2] == -1
    assert np.isnan(slp[1, 1]) and np.isnan(slp[2, 0]) and np.isnan(slp[3]).all()
    for r, i in ((0, 0), (0, 2), (1, 0), (1, 2), (2, 1), (2, 2)):
        s, want = oracle.last_logprobs_for(x[r], enc, [int(ids[r, i])])
        assert s == 0
        assert abs(slp[r, i] - want[0]) <= RTOL * abs(want[0]) + 4 * math.ulp(30.0), (r, i)
    assert oracle.last_logprobs_for(x[1], enc, [enc])[0] == oracle.ID_OOR


def test_held_row_mirror_and_escape_mass(ctx, oracle):
    """The host mirror (HeldRow) over the same reads, and escape_mass's ratio
    (batch.rs:1664-1669) from two class masses against the oracle's: a field's
    'inside' class (ids whose text opens an option) and 'outside' class (every
    other id with content), formatting ids in neither."""
    from xwen_amd import sampler as xsm
    rng = np.random.default_rng(1628)
    rows = 3
    x = _rows(rng, rows)
    lg = torch.as_tensor(x).cuda()
    h = xsm.HeldRow(ctx, lg)
    ids = [0, 1234, V - 1]
    lp = h.last_logprobs_for(ids)
    kind = rng.integers(0, 3, V)  # 0 inside, 1 outside, 2 formatting
    masks = np.stack([workloads.pack_mask((kind == c)[None, :])[0] for c in (0, 1)])
    cm = h.class_masses(masks)
    probs = h.last_probs().cpu().numpy()
    for r in range(rows):
        s, want = oracle.last_logprobs_for(x[r], V, ids)
        _, _, lse_o = oracle.held_row(x[r], V)
        np.testing.assert_allclose(lp[r], want, rtol=RTOL, atol=4 * math.ulp(abs(lse_o)))
        _, po = oracle.last_probs(x[r], V)
        inside, outside = oracle.class_masses(po, masks)
        assert abs(xsm.escape_mass(cm[r, 0], cm[r, 1]) - xsm.escape_mass(inside, outside)) <= 1e-5
        np.testing.assert_allclose(probs[r], po, rtol=RTOL, atol=1e-300)
    with pytest.raises(xsm.SampleError):
        h.last_logprobs_for([V])
    assert xsm.escape_mass(0.0, 0.0) == 0.0
