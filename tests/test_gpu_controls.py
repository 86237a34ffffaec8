"""SampleControl's bans, biases, pull and force on the device (apply_control,
sampler.rs:433-490) through the C ABI, at full width, against the CPU oracle.

Each row carries its own control set; rows are checked as every sampler row is
(token, status, candidate ids and weights bit-exact given the device
denominator, the denominator within DENOM_RTOL of the exact sum).  The small
known answers the reference's own tests hold run in test_gpu_sampler.py
(test_reference_cases).
"""
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


def _rows(n, seed):
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 3, (n, V)).astype(np.float32)
    spikes = rng.integers(0, V, (n, 6))
    for r in range(n):
        x[r, spikes[r]] = rng.uniform(9, 14, 6).astype(np.float32)
    return x, spikes, rng


def _controls(x, spikes, rng):
    """A control set per row covering every control and their interplay."""
    from xwen_amd import sampler as xsm
    S = xsm.SampleControl
    n = x.shape[0]
    out = []
    for r in range(n):
        top = int(np.argmax(x[r]))
        sp = [int(i) for i in spikes[r]]
        other = int(rng.integers(0, V))
        kind = r % 12
        if kind == 0:    # ban the argmax and the other spikes
            c = S(banned=[top] + sp[:3])
        elif kind == 1:  # bans past the vocabulary are skipped
            c = S(banned=[top, V + 5, 2 ** 32 - 1])
        elif kind == 2:  # a bias that makes a low id the winner, duplicates add in order
            c = S(bias=[(other, 20.0), (other, -1.25), (top, -30.0)])
        elif kind == 3:  # a bias on a banned id stays -inf; ids past the vocabulary skipped
            c = S(banned=[top], bias=[(top, 50.0), (V + 1, 3.0), (other, 0.5)])
        elif kind == 4:  # pull half way to the max
            c = S(pull=(other, 0.5))
        elif kind == 5:  # pull to the max: ties go to the lower id
            c = S(pull=(other, 1.0))
        elif kind == 6:  # pull past the max, after a bias lowered the max
            c = S(bias=[(top, -8.0)], pull=(other, 1.5))
        elif kind == 7:  # pull of a banned target is skipped; out-of-range target too
            c = S(banned=[other], pull=(other, 1.0)) if r % 24 == 7 else S(pull=(V + 3, 1.0))
        elif kind == 8:  # force beats a ban on the same id
            c = S(banned=[other, top], force=other)
        elif kind == 9:  # force after bias and pull: the target keeps its final value
            c = S(bias=[(other, 2.0)], pull=(other, 0.25), force=other)
        elif kind == 10:  # many bans (the whole top of the row), near the list limit
            order = np.argsort(-x[r], kind="stable")[:2000]
            c = S(banned=[int(i) for i in order])
        else:            # no control on this row
            c = None
        out.append(c)
    return out


@pytest.mark.parametrize("greedy", [False, True])
def test_controls_full_width(ctx, oracle, greedy):
    x, spikes, rng = _rows(24, 31 + greedy)
    ctls = _controls(x, spikes, rng)
    T = 0.0 if greedy else np.where(np.arange(24) % 2 == 0, 1.0, 0.7)
    K, P = 20, np.where(np.arange(24) % 3 == 0, 1.0, 0.9)
    U = rng.integers(0, 1 << 23, 24).astype(np.float32) * np.float32(2.0 ** -23)
    d = run_sample(ctx, x, T, K, P, U, ctls=ctls, cand_k=20)
    assert (d["status"] == 0).all(), d["status"]
    check_rows(oracle, x, T, K, P, U, d, ctls=ctls, label=f"controls greedy={greedy}")
    # the controls did what they say
    for r, c in enumerate(ctls):
        if c is not None and c.force is not None:
            assert d["token"][r] == c.force
        if c is not None and c.banned:
            assert d["token"][r] not in set(c.banned) or (c.force == d["token"][r])


def test_controls_with_an_allow_mask(ctx, oracle):
    wl = workloads.c3_masked()
    rows = wl.logits.shape[0]
    rng = np.random.default_rng(41)
    from xwen_amd import sampler as xsm
    ctls = []
    for r in range(rows):
        allowed = np.nonzero(workloads.mask_bits(wl.mask[r], V))[0]
        a = int(allowed[rng.integers(0, allowed.size)])
        top = int(allowed[np.argmax(wl.logits[r][allowed])])
        if r == 0:  # the one-hot row: banning its only token leaves nothing
            ctls.append(xsm.SampleControl(banned=[a]))
        elif r % 4 == 1:
            ctls.append(xsm.SampleControl(banned=[top], bias=[(a, 3.0)]))
        elif r % 4 == 2:
            ctls.append(xsm.SampleControl(pull=(a, 0.75)))
        elif r % 4 == 3:  # force a masked-out id: force beats the mask too
            out_id = int(np.nonzero(~workloads.mask_bits(wl.mask[r], V))[0][0])
            ctls.append(xsm.SampleControl(force=out_id))
        else:
            ctls.append(None)
    d = run_sample(ctx, wl.logits, wl.temperature, wl.top_k, wl.top_p, wl.u, mask=wl.mask,
                   ctls=ctls, cand_k=20)
    assert d["status"][0] == 2  # XS_ROW_NO_FINITE
    assert (d["status"][1:] == 0).all(), d["status"]
    check_rows(oracle, wl.logits, wl.temperature, wl.top_k, wl.top_p, wl.u, d, mask=wl.mask,
               ctls=ctls, label="C3+controls")


def test_control_errors_and_nan_rows(ctx):
    from xwen_amd import sampler as xsm
    S = xsm.SampleControl
    rng = np.random.default_rng(43)
    x = rng.normal(0, 1, (6, V)).astype(np.float32)
    x[2, 100] = np.nan            # NaN elsewhere: a force wipes it
    x[3, 7] = np.nan              # NaN at the forced target: it becomes 0
    x[4, 9] = np.nan              # NaN left in place: the draw fails
    ctls = [S(force=V),                                  # out of range
            S(banned=list(range(2049))),                 # past XS_CTL_MAX entries
            S(force=5), S(force=7), S(banned=[1]), None]
    d = run_sample(ctx, x, 1.0, 20, 0.95, 0.5, ctls=ctls, cand_k=20)
    assert list(d["status"]) == [4, 7, 0, 0, 1, 0]
    assert d["token"][2] == 5 and d["token"][3] == 7
    assert d["soft_max"][3] == 0.0 and d["soft_sum"][3] == 1.0
    # the forced row's candidates: the target with all the mass, then the lowest ids
    assert list(d["cand_id"][2][:4]) == [5, 0, 1, 2]
    assert list(d["cand_w"][2][:4]) == [1.0, 0.0, 0.0, 0.0]


def test_verify_with_per_position_controls(ctx):
    """Verify rows with forces: forcing each position onto its draft accepts
    every draft; a ban on a draft id ends the walk at that position."""
    from xwen_amd import sampler as xsm
    seqs, span = 4, 5
    rows = seqs * span
    rng = np.random.default_rng(44)
    x = rng.normal(0, 3, (rows, V)).astype(np.float32)
    drafts = rng.integers(0, V, (seqs, span - 1)).astype(np.int32)
    ctls = []
    for s in range(seqs):
        for i in range(span):
            if i < span - 1 and not (s == 3 and i == 2):
                ctls.append(xsm.SampleControl(force=int(drafts[s, i])))
            elif i < span - 1:
                ctls.append(xsm.SampleControl(banned=[int(drafts[s, i])]))
            else:
                ctls.append(xsm.SampleControl(force=123))
    lg = torch.as_tensor(x).cuda()
    p = xsm.params_tensor(1.0, 20, 0.95, rows, "cuda")
    u = torch.as_tensor(rng.integers(0, 1 << 23, rows).astype(np.float32) * np.float32(2.0 ** -23)).cuda()
    out = xsm.verify_batch(ctx, lg, seqs, span, p, u, torch.as_tensor(drafts).cuda(),
                           controls=xsm.controls_tensor(ctls, "cuda"))
    torch.cuda.synchronize()
    acc = out.accepted.cpu().numpy()
    ncom = out.n_committed.cpu().numpy()
    com = out.committed.cpu().numpy()
    assert list(acc) == [4, 4, 4, 2] and list(ncom) == [5, 5, 5, 3]
    for s in range(3):
        assert list(com[s]) == list(drafts[s]) + [123]
    assert list(com[3][:2]) == list(drafts[3][:2]) and com[3][2] != drafts[3][2]


@pytest.mark.parametrize("greedy", [False, True])
def test_controls_on_flat_rows(ctx, oracle, greedy):
    """Rows of one repeated value, so more than 256 of a wave's elements tie at
    the chunk bound and the chunk pass re-scans the wave exactly; the re-scan
    must see the banned, biased and pulled values, not the raw ones."""
    from xwen_amd import sampler as xsm
    S = xsm.SampleControl
    n = 8
    x = np.zeros((n, V), np.float32)
    x[2] = np.float32(1.0)
    x[3, : V // 2] = np.float32(2.0)
    x[5] = np.float32(-3.5)
    ctls = [
        S(banned=list(range(10))),                          # the lowest ids banned
        S(bias=[(50, -1.0), (7000, 0.5), (7001, 0.5)]),     # two raised ids tie on top
        S(bias=[(5, -2.0), (6, -2.0)], pull=(6, 0.5)),      # a pull half way back up
        S(banned=list(range(0, 200, 2))),                   # every other id of the plateau's start
        S(banned=list(range(2000))),                        # 2,000 bans: all of chunk 0's first slots
        S(banned=[1, 3], bias=[(0, -0.25)]),
        S(banned=list(range(1024, 1100))),                  # a block of bans in slot 1
        None,
    ]
    T = 0.0 if greedy else np.array([1.0, 0.7, 1.0, 1.3, 1.0, 0.8, 1.0, 1.0])
    K = np.array([20, 20, 50, 20, 1 if greedy else 64, 20, 30, 20])
    P = np.array([1.0, 0.9, 0.95, 1.0, 1.0, 0.5, 1.0, 0.9])
    rng = np.random.default_rng(41 + greedy)
    U = rng.integers(0, 1 << 23, n).astype(np.float32) * np.float32(2.0 ** -23)
    d = run_sample(ctx, x, T, K, P, U, ctls=ctls, cand_k=64)
    assert (d["status"] == 0).all(), d["status"]
    check_rows(oracle, x, T, K, P, U, d, ctls=ctls, margins=False, label=f"flat controls greedy={greedy}")
    for r, c in enumerate(ctls):
        if c is not None and c.banned:
            assert d["token"][r] not in set(c.banned)


def test_controls_on_flat_rows_with_an_allow_mask(ctx, oracle):
    from xwen_amd import sampler as xsm
    S = xsm.SampleControl
    n = 4
    x = np.zeros((n, V), np.float32)
    allow = np.zeros((n, V), bool)
    allow[0, 5:] = True
    allow[1, ::3] = True
    allow[2, 100:5000] = True
    allow[3, :] = True
    mask = workloads.pack_mask(allow)
    ctls = [S(banned=[5, 6, 7]), S(bias=[(3, -1.0), (9, 0.25)]), S(banned=list(range(100, 140))), S(pull=(77, 1.0))]
    T, K, P = np.array([1.0, 0.0, 1.0, 0.7]), np.array([20, 20, 40, 20]), np.array([1.0, 1.0, 0.9, 0.95])
    U = np.array([0.1, 0.0, 0.6, 0.9], np.float32)
    d = run_sample(ctx, x, T, K, P, U, mask=mask, ctls=ctls, cand_k=64)
    assert (d["status"] == 0).all(), d["status"]
    check_rows(oracle, x, T, K, P, U, d, mask=mask, ctls=ctls, margins=False, label="flat controls + mask")


def test_control_lists_longer_than_xs_ctl_max(oracle):
    """SampleControl's lists are unbounded in the reference (sampler.rs:85-121):
    a context made with xs_create_ex(ctl_max) takes rows of up to ctl_max bans
    plus biases, sorted by id in memory past XS_CTL_MAX.  Lists of 2,049 to
    20,000 entries with repeated ids (bans of biased ids, several biases of one
    id, applied in list order), with and without a mask, greedy and
    stochastic, at top_p 0.9 and 1.0, against the oracle; a list one past
    ctl_max is XS_ROW_BAD_PARAM."""
    from xwen_amd import sampler as xsm
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    cap = 20_000
    c = xsm.Context(max_rows=8, vocab=V, ctl_max=cap)
    c.bind_current_stream()
    try:
        x, spikes, rng = _rows(8, 4747)
        ctls = []
        for r in range(7):
            nb = int(rng.integers(1000, 2000)) if r == 0 else int(rng.integers(1000, 9000))
            nbias = 2049 - nb if r == 0 else int(rng.integers(1000, cap - nb))  # row 0: exactly 2,049
            banned = [int(i) for i in rng.integers(0, V + 100, nb)]  # some past the vocabulary
            if r % 2:
                banned.append(int(spikes[r][0]))                      # the top token
            ids = rng.integers(0, V, nbias)
            ids[: nbias // 4] = spikes[r][rng.integers(0, 6, nbias // 4)]  # many biases of few ids
            bias = [(int(i), float(rng.normal(0, 1.5))) for i in ids]
            pull = (int(spikes[r][3]), 0.5) if r % 3 == 0 else None
            ctls.append(xsm.SampleControl(banned=banned[: cap - len(bias)], bias=bias, pull=pull))
        ctls.append(xsm.SampleControl(banned=list(range(cap + 1))))  # one past the context's ctl_max
        T = [1.0, 0.7, 0.0, 1.3, 1.0, 0.8, 1.0, 1.0]
        K = [20, 50, 1, 20, 100, 40, 20, 20]
        P = [0.9, 1.0, 1.0, 0.95, 1.0, 0.9, 1.0, 0.9]
        U = rng.random(8).astype(np.float32)
        assert all(len(ct.banned) + len(ct.bias) > 2048 for ct in ctls)
        d = run_sample(c, x, T, K, P, U, ctls=ctls, cand_k=100)
        assert d["status"][7] == _lib_bad()
        assert (d["status"][:7] == 0).all(), d["status"]
        check_rows(oracle, x[:7], T[:7], K[:7], P[:7], U[:7],
                   {k: (None if v is None else v[:7]) for k, v in d.items()},
                   ctls=ctls[:7], label="long control lists")
        allow = rng.random((8, V)) < 0.5
        allow[np.arange(8), spikes[:, 1]] = True
        mask = workloads.pack_mask(allow)
        d = run_sample(c, x, T, K, P, U, ctls=ctls, mask=mask, cand_k=100)
        assert (d["status"][:7] == 0).all(), d["status"]
        check_rows(oracle, x[:7], T[:7], K[:7], P[:7], U[:7],
                   {k: (None if v is None else v[:7]) for k, v in d.items()},
                   ctls=ctls[:7], mask=mask[:7], label="long control lists + mask")
    finally:
        c.close()


def _lib_bad():
    from xwen_amd import _lib
    return _lib.ROW_BAD_PARAM
