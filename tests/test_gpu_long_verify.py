"""Verify blocks longer than one wave: the walk over a sequence's rows runs 64
rows at a time (xs_sampler.hip, verify_walk), so its stops are checked on
either side of the 64- and 128-row group edges against the oracle's
accept_drafts (generate.rs:4020-4046): a mismatched draft, a spent budget, an
end-of-generation token, a failed (NaN) row, a draft that completes the
grammar, and a sequence that accepts every draft and commits the bonus row.
The end-of-generation list holds 71 ids."""
import numpy as np
import pytest

from tests.test_gpu_sampler import dev

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

SPAN = 130   # three groups of 64 rows: 0-63, 64-127, 128-129
ENC = 4096
EOG_ID = 4001
# an end-of-generation list longer than a fixed array would hold (the
# reference's eog is a Vec<u32>): the planted id sits in its middle
EOG_LIST = list(range(4100, 4130)) + [EOG_ID] + list(range(4200, 4240))


def test_walks_across_group_edges(oracle):
    from xwen_amd import sampler as xsm
    from xwen_amd import _lib
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    rng = np.random.default_rng(9130)
    seqs = 10
    rows = seqs * SPAN
    x = rng.normal(0, 1, (rows, ENC)).astype(np.float32)
    top = rng.integers(0, 4000, rows)  # never EOG_ID unless planted
    x[np.arange(rows), top] = 8.0
    D = SPAN - 1
    drafts = top.reshape(seqs, SPAN)[:, :D].astype(np.int32).copy()
    budgets = np.full(seqs, 1 << 30, np.int32)
    done = np.zeros((seqs, SPAN), np.uint8)
    drafts[1, 100] = (drafts[1, 100] + 1) % 4000    # mismatch in the second group
    budgets[2] = 70                                  # budget spent inside the second group
    r = 3 * SPAN + 64                                # EOG on the first row of the second group
    x[r, top[r]] = 0.0
    x[r, EOG_ID] = 8.0
    drafts[3, 64] = EOG_ID
    x[4 * SPAN + 65, 7] = np.nan                     # a failed row
    done[5, 127] = 1                                 # the last row of the second group completes the grammar
    drafts[6, 63] = (drafts[6, 63] + 1) % 4000       # mismatch on the first group's last row
    budgets[7] = 64                                  # budget stops exactly at the group edge
    budgets[8] = 128                                 # and at the third group's first row
    # sequence 0 and 9 accept all 129 drafts and commit the bonus row
    ctx = xsm.Context(max_rows=rows, vocab=ENC)
    ctx.bind_current_stream()
    try:
        p = xsm.params_tensor(0.0, 1, 1.0, rows, "cuda")
        u = dev(np.zeros(rows, np.float32))
        out = xsm.verify_batch(ctx, dev(x), seqs, SPAN, p, u, dev(drafts), budget=dev(budgets),
                               eog=EOG_LIST, done_after=dev(done.reshape(-1)))
        torch.cuda.synchronize()
        row_tok = out.row_token.cpu().numpy()
        row_st = out.row_status.cpu().numpy()
        acc = out.accepted.cpu().numpy()
        com = out.committed.cpu().numpy()
        ncom = out.n_committed.cpu().numpy()
        sst = out.seq_status.cpu().numpy()
    finally:
        ctx.close()
    assert row_st[4 * SPAN + 65] == _lib.ROW_NAN
    for s in range(seqs):
        sl = slice(s * SPAN, (s + 1) * SPAN)
        toks = row_tok[sl]
        ok = row_st[sl] == 0
        np.testing.assert_array_equal(toks[ok], top[sl][ok] if s != 3 else
                                      np.where(np.arange(SPAN) == 64, EOG_ID, top[sl])[ok])
        # a draft that completes the grammar ends the walk as an EOG would
        eog = [(t == EOG_ID) or (i < D and done[s, i] and t == drafts[s, i]) for i, t in enumerate(toks)]
        st, m, committed, _ = oracle.accept_drafts(list(drafts[s]), int(budgets[s]), list(toks), eog,
                                                   list(row_st[sl]))
        assert (sst[s], acc[s], ncom[s]) == (st, m, len(committed)), s
        assert list(com[s, :ncom[s]]) == committed, s
        assert (com[s, ncom[s]:] == -1).all(), s
    expect = {0: (130, 129), 1: (101, 100), 2: (70, 70), 3: (65, 65), 4: (65, 65),
              5: (128, 128), 6: (64, 63), 7: (64, 64), 8: (128, 128), 9: (130, 129)}
    for s, (nc, m) in expect.items():
        assert (ncom[s], acc[s]) == (nc, m), (s, ncom[s], acc[s])
    assert sst[4] == _lib.ROW_NAN and (np.delete(sst, 4) == 0).all()
