"""xs_sample's row_order scheduling hint: any permutation gives the same
outputs as the natural order, row for row; a non-permutation is an argument
error."""
import numpy as np
import pytest

from tests import workloads
from xwen_amd import sampler as xsm

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

V = workloads.V


@pytest.fixture(scope="module")
def ctx():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    c = xsm.Context(max_rows=64, vocab=V)
    c.bind_current_stream()
    yield c
    c.close()


def _same(got, want):
    """Every output equal byte for byte; the candidate lists up to each row's
    n_cand (the entries past it are not written)."""
    for k, w in want.items():
        g = got[k]
        if k in ("cand_id", "cand_w"):
            for r in range(w.shape[0]):
                n = min(int(want["n_cand"][r]), w.shape[1])
                assert (g[r, :n].view(np.uint8) == w[r, :n].view(np.uint8)).all(), (k, r)
        else:
            assert (g.view(np.uint8) == w.view(np.uint8)).all(), k


def _outputs(ctx, wl, order, **kw):
    rows = wl.logits.shape[0]
    lg = torch.as_tensor(wl.logits).cuda()
    p = xsm.params_tensor(wl.temperature, wl.top_k, wl.top_p, rows, "cuda")
    u = torch.as_tensor(wl.u).cuda()
    out = xsm.sample_batch(ctx, lg, p, u, order=order, **kw)
    torch.cuda.synchronize()
    return {k: v.cpu().numpy() for k, v in vars(out).items() if v is not None}


def test_any_order_gives_the_same_draws(ctx):
    wl = workloads.c5_heterogeneous(rows=64)
    base = _outputs(ctx, wl, None, cand_k=100, n_top=20)
    rng = np.random.default_rng(91)
    orders = [xsm.cost_order(wl.temperature, wl.top_k), rng.permutation(64), np.arange(64)[::-1]]
    for order in orders:
        _same(_outputs(ctx, wl, order, cand_k=100, n_top=20), base)
    assert (base["status"] == 0).all()


def test_order_with_masks_and_controls(ctx):
    wl = workloads.c3_masked()
    rows = wl.logits.shape[0]
    mask = torch.as_tensor(wl.mask.view(np.int32)).cuda()
    S = xsm.SampleControl
    ctls = [S(banned=[int(np.argmax(wl.logits[r]))]) if r % 3 == 1 else None for r in range(rows)]
    controls = xsm.controls_tensor(ctls, "cuda")
    base = _outputs(ctx, wl, None, cand_k=20, allowed=mask, controls=controls)
    order = xsm.cost_order(wl.temperature, wl.top_k, controlled=[c is not None for c in ctls])
    _same(_outputs(ctx, wl, order, cand_k=20, allowed=mask, controls=controls), base)


def test_bad_orders_are_argument_errors(ctx):
    from xwen_amd import _lib
    wl = workloads.c2_batch(rows=8)
    lg = torch.as_tensor(wl.logits).cuda()
    p = xsm.params_tensor(wl.temperature, wl.top_k, wl.top_p, 8, "cuda")
    u = torch.as_tensor(wl.u).cuda()
    for order in ([0, 1, 2, 3, 4, 5, 6, 6], [0, 1, 2, 3, 4, 5, 6, 8], [-1, 1, 2, 3, 4, 5, 6, 7]):
        with pytest.raises(_lib.XsError):
            xsm.sample_batch(ctx, lg, p, u, order=order)
    # the host mirror checks the length (the library reads `rows` entries)
    for order in ([0, 1, 2], list(range(9))):
        with pytest.raises(ValueError):
            xsm.sample_batch(ctx, lg, p, u, order=order)
    # more rows than a launch's order table holds
    n = _lib.ORDER_MAX + 1
    big = xsm.Context(max_rows=n, vocab=1024)
    big.bind_current_stream()
    x = torch.zeros((n, 1024), dtype=torch.float32, device="cuda")
    pb = xsm.params_tensor(1.0, 20, 0.9, n, "cuda")
    ub = torch.zeros(n, dtype=torch.float32, device="cuda")
    # past ORDER_MAX rows an order is checked, then not applied: the natural
    # order's draws, and a non-permutation is still an error
    want = xsm.sample_batch(big, x, pb, ub, cand_k=20)
    got = xsm.sample_batch(big, x, pb, ub, cand_k=20, order=np.arange(n)[::-1].copy())
    torch.cuda.synchronize()
    assert torch.equal(got.token, want.token) and torch.equal(got.cand_id, want.cand_id)
    bad = np.arange(n)
    bad[5] = 4
    with pytest.raises(_lib.XsError):
        xsm.sample_batch(big, x, pb, ub, order=bad)
    torch.cuda.synchronize()
    big.close()


def test_ordered_call_in_a_graph():
    """An ordered call captured in a HIP graph keeps its order (the table is
    copied into the kernel's arguments at capture): every replay, with
    unordered eager calls in between, equals the eager ordered call."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    wl = workloads.c5_heterogeneous(rows=64)
    rows = 64
    c = xsm.Context(max_rows=rows, vocab=V)
    lg = torch.as_tensor(wl.logits).cuda()
    p = xsm.params_tensor(wl.temperature, wl.top_k, wl.top_p, rows, "cuda")
    u = torch.as_tensor(wl.u).cuda()
    order = xsm.cost_order(wl.temperature, wl.top_k)
    out = xsm.Draws(token=torch.empty(rows, dtype=torch.int32, device="cuda"),
                    status=torch.empty(rows, dtype=torch.int32, device="cuda"),
                    soft_sum=torch.empty(rows, dtype=torch.float32, device="cuda"),
                    soft_max=torch.empty(rows, dtype=torch.float32, device="cuda"))
    c.bind_current_stream()
    xsm.sample_batch(c, lg, p, u, stats=True, out=out, order=order)
    torch.cuda.synchronize()
    want_tok = out.token.cpu().numpy().copy()
    want_sum = out.soft_sum.cpu().numpy().copy()
    assert (out.status.cpu().numpy() == 0).all()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        c.bind_current_stream()
        with torch.cuda.graph(g, stream=side):
            c.bind_current_stream()
            xsm.sample_batch(c, lg, p, u, stats=True, out=out, order=order)
    c.bind_current_stream()
    torch.cuda.synchronize()
    for rep in range(4):
        out.token.fill_(-7)
        out.soft_sum.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert (out.token.cpu().numpy() == want_tok).all(), rep
        assert (out.soft_sum.cpu().numpy().view(np.uint32) == want_sum.view(np.uint32)).all(), rep
        # an unordered eager call on the same context in between
        d = xsm.sample_batch(c, lg, p, u)
        torch.cuda.synchronize()
        assert (d.token.cpu().numpy() == want_tok).all(), rep
    c.close()


def test_order_at_its_row_limit():
    """ORDER_MAX rows (the whole argument table) of 4,096 ids: reversed and
    shuffled orders give the natural order's draws row for row."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from xwen_amd import _lib
    n, v = _lib.ORDER_MAX, 4096
    rng = np.random.default_rng(1024)
    x = torch.as_tensor(rng.normal(0.0, 3.0, (n, v)).astype(np.float32)).cuda()
    T = rng.choice([0.0, 0.7, 1.0], n)
    K = rng.choice([1, 20, 100], n)
    p = xsm.params_tensor(T, K, 0.95, n, "cuda")
    u = torch.as_tensor(rng.random(n).astype(np.float32)).cuda()
    c = xsm.Context(max_rows=n, vocab=v)
    c.bind_current_stream()
    base = xsm.sample_batch(c, x, p, u, cand_k=100)
    torch.cuda.synchronize()
    want = {k: t.cpu().numpy() for k, t in vars(base).items() if t is not None}
    assert (want["status"] == 0).all()
    for order in (np.arange(n)[::-1], rng.permutation(n), xsm.cost_order(T, K)):
        got = xsm.sample_batch(c, x, p, u, cand_k=100, order=order)
        torch.cuda.synchronize()
        _same({k: t.cpu().numpy() for k, t in vars(got).items() if t is not None}, want)
    c.close()
