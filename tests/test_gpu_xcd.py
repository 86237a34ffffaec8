"""The XCD-local hand-off: every workgroup of a row runs on one XCD.

In a call of at least 8 rows per XCD, sample_kernel's grid puts a row's
chunks n workgroups apart (n the device's XCD count; the hardware deals
workgroup b to XCD b mod n), so the chunk
workgroups hand their sub-records to the row's finalizer through that XCD's
L2 (sc0 stores and loads) instead of through memory.  The row's arrival ticket
proves the placement: it sums the workgroups' XCDs and their squares, and a
row whose sums do not match the finalizer's XCD is failed (XS_ROW_INTERNAL),
never read.

Checked here, through the hook xs_test_xcd:
- the context confirmed the placement when it was created (its XCD count is
  printed);
- the split launch, where the hand-off crosses a launch boundary instead,
  gives bit-identical outputs on every workload shape, with row counts that
  are and are not multiples of the XCD count;
- a placement failure forced from the host (the odd chunks of each row
  report another XCD) fails every row of several chunks loudly, token -1,
  and a verify block's sequences with it; the next call is normal again;
- a call of fewer than 8 rows per XCD spreads each row over the XCDs and
  hands off through memory (one XCD would stream a lone row at its share of
  the bandwidth), so the forced failure leaves it untouched.
"""
import ctypes

import numpy as np
import pytest

from tests import workloads

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

V = workloads.V


@pytest.fixture(scope="module")
def ctx():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from xwen_amd import sampler as xsm
    c = xsm.Context(max_rows=256, vocab=V)
    c.bind_current_stream()
    yield c
    set_mode(c, 0)
    c.close()


def set_mode(ctx, mode):
    """xs_test_xcd: 0 normal, 1 split launch, 2 forced placement failure;
    returns the context's XCD count."""
    n = ctypes.c_int32(-1)
    assert ctx.lib.xs_test_xcd(ctx.h, mode, ctypes.byref(n)) == 0
    return int(n.value)


def dev(a):
    return torch.as_tensor(np.ascontiguousarray(a)).cuda()


def draw(ctx, wl, rows=None, **kw):
    from xwen_amd import sampler as xsm
    n = wl.logits.shape[0] if rows is None else rows
    p = xsm.params_tensor(wl.temperature[:n], wl.top_k[:n], wl.top_p[:n], n, "cuda")
    out = xsm.sample_batch(ctx, dev(wl.logits[:n]), p, dev(wl.u[:n]), **kw)
    torch.cuda.synchronize()
    return {k: v.cpu().numpy() for k, v in vars(out).items() if v is not None}


def same_bits(a, b, tag):
    assert a.keys() == b.keys(), tag
    for k in a:
        x, y = a[k], b[k]
        if x.dtype.kind == "f":
            x = x.view(np.uint32 if x.itemsize == 4 else np.uint64)
            y = y.view(np.uint32 if y.itemsize == 4 else np.uint64)
        np.testing.assert_array_equal(x, y, err_msg=f"{tag}: {k}")


def test_the_context_confirms_the_placement(ctx):
    n = set_mode(ctx, 0)
    print(f"XCDs confirmed by the context's placement probe: {n}")
    assert n >= 1


def _cases():
    """Row counts of 64 and more hand off XCD-locally (71, 72 and 100 pad the
    last group of 8); fewer spread each row over the XCDs."""
    c2, c5 = workloads.c2_batch(rows=80), workloads.c5_heterogeneous()
    c3, c3w = workloads.c3_masked(), workloads.c3_masked(seed=313, rows=72)
    return [
        ("C2 64 rows with candidates", c2, 64, dict(cand_k=20, stats=True)),
        ("C2 71 rows tokens only", c2, 71, {}),
        ("C2 13 rows tokens only", c2, 13, {}),
        ("C2 1 row", c2, 1, dict(cand_k=20)),
        ("C3 32 masked rows", c3, None, dict(allowed=dev(c3.mask.view(np.int32)), cand_k=20, stats=True)),
        ("C3 72 masked rows", c3w, None, dict(allowed=dev(c3w.mask.view(np.int32)), cand_k=20, stats=True)),
        ("C3 70 masked rows tokens only", c3w, 70, dict(allowed=dev(c3w.mask[:70].view(np.int32)))),
        ("C5 256 rows with held_row statistics", c5, None, dict(n_top=20, stats=True)),
        ("C5 100 rows with held_row statistics", c5, 100, dict(n_top=20)),
        ("C5 37 rows with held_row statistics", c5, 37, dict(n_top=20)),
    ]


def test_split_launch_gives_identical_outputs(ctx):
    for tag, wl, rows, kw in _cases():
        set_mode(ctx, 0)
        a = draw(ctx, wl, rows, **kw)
        set_mode(ctx, 1)
        b = draw(ctx, wl, rows, **kw)
        set_mode(ctx, 0)
        print(f"{tag}: identical in both launches; statuses {np.unique(a['status']).tolist()}")
        same_bits(a, b, tag)
        assert (a["status"] != 8).all(), tag
    # controlled rows at top_p 1 with candidates: serial_kernel sums and
    # finalizes them after sample_kernel's XCD-local launch
    c3w = workloads.c3_masked(seed=323, rows=72)
    c3w.top_p = np.full(72, 1.0)
    kw = dict(allowed=dev(c3w.mask.view(np.int32)), cand_k=20, stats=True)
    set_mode(ctx, 0)
    a = draw(ctx, c3w, None, **kw)
    set_mode(ctx, 1)
    b = draw(ctx, c3w, None, **kw)
    set_mode(ctx, 0)
    same_bits(a, b, "C3 72 masked rows at top_p 1 (serial denominator)")
    # a verify block small enough for one launch (64 rows)
    c4 = workloads.c4_verify(seqs=4)
    got = []
    for mode in (0, 1):
        set_mode(ctx, mode)
        got.append(verify(ctx, c4))
        set_mode(ctx, 0)
    same_bits(got[0], got[1], "C4 4 x 16 verify block")


def test_whole_row_rows_in_an_xcd_local_call():
    """64 rows at top_k 500 (the whole-row kernels draw them after the
    finalizers defer them) give the same outputs handed off XCD-locally and
    in the split launch."""
    from xwen_amd import sampler as xsm
    c = xsm.Context(max_rows=64, vocab=V, k_max=2**31 - 1)
    c.bind_current_stream()
    try:
        wl = workloads.c2_batch(seed=212)
        wl.top_k = np.full(64, 500)
        got = []
        for mode in (0, 1):
            set_mode(c, mode)
            got.append(draw(c, wl, None, cand_k=20, stats=True))
        set_mode(c, 0)
        same_bits(got[0], got[1], "64 rows at top_k 500")
        assert (got[0]["status"] == 0).all()
        assert (got[0]["n_cand"] == 500).all()
    finally:
        c.close()


def verify(ctx, c4):
    from xwen_amd import sampler as xsm
    rows = c4.seqs * c4.span
    p = xsm.params_tensor(c4.temperature, c4.top_k, c4.top_p, rows, "cuda")
    out = xsm.verify_batch(ctx, dev(c4.logits), c4.seqs, c4.span, p, dev(c4.u), dev(c4.drafts),
                           eog=[248046, 248044])
    torch.cuda.synchronize()
    return {k: v.cpu().numpy() for k, v in vars(out).items() if hasattr(v, "cpu")}


def test_a_forced_placement_failure_fails_rows_loudly(ctx):
    from xwen_amd import _lib
    n = set_mode(ctx, 0)
    if n < 2:
        pytest.skip("one XCD: no placement to fail")
    wl = workloads.c2_batch()
    good = draw(ctx, wl, cand_k=20)
    set_mode(ctx, 2)
    bad = draw(ctx, wl, cand_k=20)
    set_mode(ctx, 0)
    assert (bad["status"] == _lib.ROW_INTERNAL).all()
    assert (bad["token"] == -1).all()
    assert (bad["n_cand"] == 0).all()
    again = draw(ctx, wl, cand_k=20)
    same_bits(good, again, "after the forced failure")
    # fewer than 8 rows per XCD: each row spreads over the XCDs and hands off
    # through memory, with no placement to check
    for rows in (5, 40):
        small = draw(ctx, wl, rows, cand_k=20)
        set_mode(ctx, 2)
        small2 = draw(ctx, wl, rows, cand_k=20)
        set_mode(ctx, 0)
        same_bits(small, small2, f"{rows} rows, spread over the XCDs")
        assert (small["status"] == 0).all()
    # a verify block in one launch: every sequence stops at its first row,
    # with that row's status
    c4 = workloads.c4_verify(seqs=4)
    set_mode(ctx, 2)
    out = verify(ctx, c4)
    set_mode(ctx, 0)
    assert (out["seq_status"] == _lib.ROW_INTERNAL).all()
    assert (out["n_committed"] == 0).all()
