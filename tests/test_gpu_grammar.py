"""The verify block under a grammar (generate.rs:2426-2461): per-position masks
and completion flags from masks_along_drafts, one xs_verify launch, against the
walk the reference makes row by row (the grammar advanced at sample time)."""
import numpy as np
import pytest

from tests import workloads
from tests.grammar_toy import ToyGrammar
from tests.test_host_grammar import _random_drafts

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


def test_verify_with_masks_along_the_drafts(ctx):
    from xwen_amd import sampler as xsm
    rng = np.random.default_rng(31)
    seqs, D = 8, 7
    span = D + 1
    x = rng.normal(0, 1, (seqs * span, V)).astype(np.float32)
    grammars = [ToyGrammar(V, n=int(rng.integers(2, 6)), dormant=(s % 2 == 0)) for s in range(seqs)]
    words = grammars[0].words
    drafts = np.zeros((seqs, D), np.int32)
    masks = np.zeros((seqs * span, words), np.uint32)
    done = np.zeros(seqs * span, np.uint8)
    for s, g in enumerate(grammars):
        d = _random_drafts(rng, g, D)
        drafts[s] = d
        m, f = xsm.masks_along_drafts(g, d, words)
        masks[s * span:(s + 1) * span] = m
        done[s * span:(s + 1) * span] = f
        for i, t in enumerate(d):
            x[s * span + i, t] = np.float32(30.0)  # the drafter's pick leads its row
    # greedy rows: each row's token is its argmax over the allowed ids
    bits = ((masks[:, :, None] >> np.arange(32, dtype=np.uint32)) & 1).reshape(len(masks), -1)[:, :V]
    tok = np.argmax(np.where(bits.astype(bool), x, -np.inf), axis=1)
    want = []
    for s in range(seqs):
        com, m = [], 0
        for i in range(span):
            t = int(tok[s * span + i])
            matched = i < D and t == drafts[s, i]
            com.append(t)
            m += matched
            if not matched or done[s * span + i]:
                break
        want.append((m, com))
    out = xsm.verify_batch(ctx, torch.as_tensor(x).cuda(), seqs, span,
                           xsm.params_tensor(0.0, 1, 1.0, seqs * span, "cuda"),
                           torch.zeros(seqs * span, dtype=torch.float32, device="cuda"),
                           torch.as_tensor(drafts).cuda(),
                           allowed=torch.as_tensor(masks.view(np.int32)).cuda(),
                           done_after=torch.as_tensor(done).cuda())
    torch.cuda.synchronize()
    acc = out.accepted.cpu().numpy()
    ncom = out.n_committed.cpu().numpy()
    com = out.committed.cpu().numpy()
    assert (out.seq_status.cpu().numpy() == 0).all()
    for s in range(seqs):
        m, c = want[s]
        assert (acc[s], ncom[s]) == (m, len(c)), (s, acc[s], ncom[s], want[s])
        assert list(com[s][:len(c)]) == c
    # the grammar ended at least one walk early, and at least one ran to the bonus row
    assert any(done[s * span:(s + 1) * span].any() for s in range(seqs))


def test_stochastic_verify_with_masks_along_the_drafts(ctx, oracle):
    """The same block drawn stochastically (T 0.7 / top_k 20 / top_p 0.8, one
    uniform per position): every row's token equals xs_sample's on the same
    row, mask and uniform, which the oracle reproduces bit for bit given the
    device's denominator; the walk equals accept_drafts over those tokens with
    the grammar's completion ending it like an EOG."""
    from tests.test_gpu_sampler import check_rows
    from xwen_amd import sampler as xsm
    rng = np.random.default_rng(47)
    seqs, D = 8, 7
    span = D + 1
    rows = seqs * span
    x = rng.normal(0, 1.5, (rows, V)).astype(np.float32)
    grammars = [ToyGrammar(V, n=int(rng.integers(2, 6)), dormant=(s % 3 == 0)) for s in range(seqs)]
    words = grammars[0].words
    drafts = np.zeros((seqs, D), np.int32)
    masks = np.zeros((rows, words), np.uint32)
    done = np.zeros(rows, np.uint8)
    for s, g in enumerate(grammars):
        d = _random_drafts(rng, g, D)
        drafts[s] = d
        m, f = xsm.masks_along_drafts(g, d, words)
        masks[s * span:(s + 1) * span] = m
        done[s * span:(s + 1) * span] = f
        for i, t in enumerate(d):
            x[s * span + i, t] += np.float32(rng.uniform(2.0, 7.0))  # likely, not certain
    T, K, P = 0.7, 20, 0.8
    U = workloads.uniforms(rng, rows)
    lg = torch.as_tensor(x).cuda()
    p = xsm.params_tensor(T, K, P, rows, "cuda")
    u = torch.as_tensor(U).cuda()
    m_dev = torch.as_tensor(masks.view(np.int32)).cuda()
    out = xsm.verify_batch(ctx, lg, seqs, span, p, u, torch.as_tensor(drafts).cuda(),
                           allowed=m_dev, done_after=torch.as_tensor(done).cuda())
    d = xsm.sample_batch(ctx, lg, p, u, allowed=m_dev, cand_k=20, stats=True)
    torch.cuda.synchronize()
    d = {k: (None if v is None else v.cpu().numpy()) for k, v in vars(d).items()}
    assert (d["status"] == 0).all()
    tok = out.row_token.cpu().numpy()
    assert (tok == d["token"]).all()
    check_rows(oracle, x, T, K, P, U, d, mask=masks, label="stochastic verify rows")
    acc = out.accepted.cpu().numpy()
    ncom = out.n_committed.cpu().numpy()
    com = out.committed.cpu().numpy()
    assert (out.seq_status.cpu().numpy() == 0).all()
    matched_any = 0
    for s in range(seqs):
        st, m, c, _calls = oracle.accept_drafts(
            list(drafts[s]), 1 << 62, list(tok[s * span:(s + 1) * span]),
            [bool(done[s * span + i]) for i in range(span)])
        assert st == 0
        assert (acc[s], ncom[s]) == (m, len(c)), (s, acc[s], ncom[s], m, len(c))
        assert list(com[s][:len(c)]) == c
        matched_any += m > 0
    assert matched_any >= 2  # the walks do go past their first row
