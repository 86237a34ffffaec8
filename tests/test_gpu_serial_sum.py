"""The reference's own denominator on controlled rows at top_p >= 1.

On a row with an allow-mask or sparse controls the reference sums the softmax
terms one at a time in f32, in id order (softmax_in_place, sampler.rs:301-305,
reached from sample_controlled's non-noop branch, :222-229), and at top_p >= 1
the candidate weights are p = e / that sum, unrenormalized.  serial_kernel
reproduces that sum; here the device sum must equal the oracle's SUM_SEQ_F32
sum bit for bit, and with it the token and every candidate weight
(check_rows).  The serial sum sits ~1e-4 from the exact one on such rows
(reported as serial_vs_exact), so a device that kept the exact sum fails
these tests on the weights.

Cases: the C3 workload at top_p = 1; spiked rows whose runner-up terms lie
half-way between grid points of the running sum (round half to even); bans,
biases and pulls; rows whose prefix climbs through ~150 binades (more
segments to resolve term by term than the side buffer keeps, so the walk
recounts terms from the logits, controls included); rows of 1,048,576 ids
(several staging windows); the whole-row path (top_k >= V); and a verify
block."""
import numpy as np
import pytest

from tests import workloads
from tests.test_gpu_sampler import SERIAL_ROWS, check_rows, run_sample

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


def _checked(oracle, x, T, K, P, U, d, **kw):
    before = SERIAL_ROWS[0]
    check_rows(oracle, x, T, K, P, U, d, **kw)
    return SERIAL_ROWS[0] - before


def test_c3_masks_at_top_p_1(ctx, oracle):
    wl = workloads.c3_masked()
    rows = wl.logits.shape[0]
    for cand_k in (20, 128):
        d = run_sample(ctx, wl.logits, wl.temperature, wl.top_k, 1.0, wl.u, mask=wl.mask, cand_k=cand_k)
        assert (d["status"] == 0).all(), d["status"]
        n = _checked(oracle, wl.logits, wl.temperature, wl.top_k, 1.0, wl.u, d, mask=wl.mask,
                     label=f"C3 top_p=1 cand_k={cand_k}")
        assert n == rows


def test_spiked_rows_with_controls_at_top_p_1(ctx, oracle):
    """C2-shaped rows (a few tokens far above the bulk), where the running
    sum's grid is coarse against the runner-up terms; bans of the top token,
    biases and pulls."""
    from xwen_amd import sampler as xsm
    rng = np.random.default_rng(7301)
    rows = 24
    x = rng.normal(0, 2.5, (rows, V)).astype(np.float32)
    ctls = []
    for r in range(rows):
        spikes = rng.integers(0, V, 8)
        x[r, spikes] = rng.uniform(8, 14, 8).astype(np.float32)
        top = int(np.argmax(x[r]))
        kind = r % 4
        if kind == 0:
            ctls.append(xsm.SampleControl(banned=[top]))
        elif kind == 1:
            ctls.append(xsm.SampleControl(bias=[(int(spikes[1]), 2.5), (int(rng.integers(0, V)), -3.0)]))
        elif kind == 2:
            ctls.append(xsm.SampleControl(pull=(int(spikes[2]), 0.5), banned=[int(i) for i in rng.integers(0, V, 50)]))
        else:
            ctls.append(xsm.SampleControl(banned=[V + 5]))  # past the vocabulary: still a controlled row
    T = rng.choice([0.7, 1.0, 1.3], rows)
    K = rng.choice([20, 50, 100], rows)
    U = workloads.uniforms(rng, rows)
    d = run_sample(ctx, x, T, K, 1.0, U, ctls=ctls, cand_k=100)
    assert (d["status"] == 0).all(), d["status"]
    assert _checked(oracle, x, T, K, 1.0, U, d, ctls=ctls, label="spiked controlled") == rows


def test_rows_whose_prefix_climbs_many_binades(ctx, oracle):
    """Logits rising (or falling) linearly across the row over ~100 nats: the
    terms run from ~2^-150 to 1, so the serial sum changes binade ~150 times,
    each a segment added term by term -- more than the side buffer keeps, so
    the walk recounts terms from the logits, bans and biases included."""
    from xwen_amd import sampler as xsm
    rng = np.random.default_rng(7302)
    rows = 6
    ramp = np.linspace(-100.0, 0.0, V, dtype=np.float64)
    x = np.empty((rows, V), np.float32)
    x[0] = ramp
    x[1] = ramp[::-1]
    x[2] = ramp + rng.normal(0, 0.3, V)
    x[3] = np.where(rng.random(V) < 0.5, ramp, -1e30)
    x[4] = ramp
    x[5] = ramp[::-1] + rng.normal(0, 0.3, V)
    ctls = [None, None, None, None,
            xsm.SampleControl(banned=[int(i) for i in rng.integers(0, V, 300)],
                              bias=[(int(i), float(rng.normal(0, 2))) for i in rng.integers(0, V, 200)]),
            xsm.SampleControl(bias=[(V - 10, 1.0)], pull=(1000, 0.3))]
    allow = rng.random((rows, V)) < 0.9
    allow[np.arange(rows), np.argmax(x, axis=1)] = True
    mask = workloads.pack_mask(allow)
    U = workloads.uniforms(rng, rows)
    d = run_sample(ctx, x, 1.0, 20, 1.0, U, mask=mask, ctls=ctls, cand_k=20)
    assert (d["status"] == 0).all(), d["status"]
    assert _checked(oracle, x, 1.0, 20, 1.0, U, d, mask=mask, ctls=ctls, label="binade ramp") == rows


def test_short_rows_and_single_allowed_ids(ctx, oracle):
    """Narrow vocabularies (one segment, a partial slot) and masks that allow
    one id (the sum is exactly 1) or two."""
    rng = np.random.default_rng(7303)
    for enc in (1, 3, 200, 1024, 5000):
        rows = 4
        ld = (enc + 3) // 4 * 4
        x = rng.normal(0, 3, (rows, ld)).astype(np.float32)
        allow = np.zeros((rows, enc), bool)
        allow[0, rng.integers(0, enc)] = True
        allow[1, rng.integers(0, enc, 2)] = True
        allow[2] = True
        allow[3] = rng.random(enc) < 0.5
        allow[3, 0] = True
        mask = workloads.pack_mask(allow)
        U = workloads.uniforms(rng, rows)
        d = run_sample(ctx, x, 0.8, 20, 1.0, U, enc=enc, mask=mask, cand_k=20)
        assert (d["status"] == 0).all(), (enc, d["status"])
        assert _checked(oracle, x, 0.8, 20, 1.0, U, d, enc=enc, mask=mask, label=f"enc {enc}") == rows
        assert d["soft_sum"][0] == 1.0


def test_a_million_ids_over_several_windows(oracle):
    """1,048,576 ids: 4,096 segments, staged by the walk in several windows."""
    from xwen_amd import sampler as xsm
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    n_ids = 1_048_576
    c = xsm.Context(max_rows=3, vocab=n_ids)
    c.bind_current_stream()
    try:
        rng = np.random.default_rng(7304)
        x = rng.normal(0, 3, (3, n_ids)).astype(np.float32)
        allow = rng.random((3, n_ids)) < np.array([[0.05], [0.5], [1.0]])
        allow[:, 12345] = True
        mask = workloads.pack_mask(allow)
        U = workloads.uniforms(rng, 3)
        d = run_sample(c, x, 1.0, 50, 1.0, U, mask=mask, cand_k=50)
        assert (d["status"] == 0).all(), d["status"]
        assert _checked(oracle, x, 1.0, 50, 1.0, U, d, mask=mask, label="1M ids") == 3
    finally:
        c.close()


def test_whole_row_path_under_a_mask(oracle):
    """top_k >= V (the whole-row path) on masked rows at top_p = 1: every id's
    weight is e / (the serial sum)."""
    from xwen_amd import sampler as xsm
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    c = xsm.Context(max_rows=4, vocab=V, k_max=2**31 - 1)
    c.bind_current_stream()
    try:
        rng = np.random.default_rng(7305)
        x = rng.normal(0, 3, (4, V)).astype(np.float32)
        allow = rng.random((4, V)) < 0.3
        mask = workloads.pack_mask(allow)
        K = [V, 10**6, 300, 128]
        U = workloads.uniforms(rng, 4)
        d = run_sample(c, x, 1.0, K, 1.0, U, mask=mask, cand_k=V)
        assert (d["status"] == 0).all(), d["status"]
        assert _checked(oracle, x, 1.0, K, 1.0, U, d, mask=mask, label="whole row, masked") == 4
    finally:
        c.close()


def test_verify_block_at_top_p_1(ctx, oracle):
    """xs_verify rows under masks at top_p = 1 take the serial sum too: the
    block's row tokens equal xs_sample's, which equal the literal reference's."""
    from xwen_amd import sampler as xsm
    rng = np.random.default_rng(7306)
    seqs, span = 4, 6
    rows = seqs * span
    x = rng.normal(0, 3, (rows, V)).astype(np.float32)
    allow = rng.random((rows, V)) < 0.2
    drafts = np.zeros((seqs, span - 1), np.int32)
    for s in range(seqs):
        for i in range(span - 1):
            r = s * span + i
            ids = np.nonzero(allow[r])[0]
            drafts[s, i] = int(ids[np.argmax(x[r, ids])])
    mask = workloads.pack_mask(allow)
    U = workloads.uniforms(rng, rows)
    lg = torch.as_tensor(x).cuda()
    p = xsm.params_tensor(1.0, 20, 1.0, rows, "cuda")
    u = torch.as_tensor(U).cuda()
    m_dev = torch.as_tensor(mask.view(np.int32)).cuda()
    out = xsm.verify_batch(ctx, lg, seqs, span, p, u, torch.as_tensor(drafts).cuda(), allowed=m_dev)
    d = xsm.sample_batch(ctx, lg, p, u, allowed=m_dev, cand_k=20, stats=True)
    torch.cuda.synchronize()
    d = {k: (None if v is None else v.cpu().numpy()) for k, v in vars(d).items()}
    assert (d["status"] == 0).all()
    assert (out.row_token.cpu().numpy() == d["token"]).all()
    assert _checked(oracle, x, 1.0, 20, 1.0, U, d, mask=mask, label="verify top_p=1") == rows
    acc = out.accepted.cpu().numpy()
    for s in range(seqs):
        want = 0
        for i in range(span - 1):
            if d["token"][s * span + i] != drafts[s, i]:
                break
            want += 1
        assert acc[s] == want, (s, acc[s], want)
