"""Argument and capacity errors of the C ABI on a live context: each case breaks
one field of an otherwise valid call and must return the documented code
without launching anything, and the context must sample correctly afterwards."""
import ctypes as C

import numpy as np
import pytest

from xwen_amd import _lib
from xwen_amd import sampler as xsm

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

ROWS, VOCAB, WIDTH = 8, 8192, 4096


@pytest.fixture(scope="module")
def setup():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    ctx = xsm.Context(max_rows=ROWS, vocab=VOCAB)
    ctx.bind_current_stream()
    rng = np.random.default_rng(7)
    t = {
        "logits": torch.as_tensor(rng.normal(0, 3, (ROWS, WIDTH + 4)).astype(np.float32)).cuda(),
        "params": xsm.params_tensor(0.8, 20, 0.9, ROWS, "cuda"),
        "u": torch.as_tensor(rng.random(ROWS).astype(np.float32)).cuda(),
        "tok": torch.empty(ROWS, dtype=torch.int32, device="cuda"),
        "st": torch.empty(ROWS, dtype=torch.int32, device="cuda"),
        "cid": torch.empty((ROWS, 32), dtype=torch.int32, device="cuda"),
        "cw": torch.empty((ROWS, 32), dtype=torch.float32, device="cuda"),
        "nc": torch.empty(ROWS, dtype=torch.int32, device="cuda"),
        "mask": torch.full((ROWS, WIDTH // 32), -1, dtype=torch.int32, device="cuda"),
        "top": torch.empty((ROWS, 8), dtype=torch.int32, device="cuda"),
        "lp": torch.empty((ROWS, 8), dtype=torch.float32, device="cuda"),
        "prob": torch.empty(ROWS, dtype=torch.float32, device="cuda"),
    }
    yield ctx, t
    torch.cuda.synchronize()
    ctx.close()


def _sample_args(t, ld=WIDTH + 4, width=WIDTH):
    a = _lib.SampleArgs()
    a.logits = t["logits"].data_ptr()
    a.rows, a.ld, a.width, a.enc = ROWS, ld, width, width
    a.params, a.uniforms = t["params"].data_ptr(), t["u"].data_ptr()
    a.token, a.status = t["tok"].data_ptr(), t["st"].data_ptr()
    a.cand_id, a.cand_w, a.n_cand, a.cand_ld = (t["cid"].data_ptr(), t["cw"].data_ptr(),
                                                t["nc"].data_ptr(), 32)
    return a


def _call(ctx, a):
    return ctx.lib.xs_sample(ctx.h, C.byref(a))


def test_valid_call_then_every_broken_field(setup):
    ctx, t = setup
    assert _call(ctx, _sample_args(t)) == _lib.XS_OK
    torch.cuda.synchronize()
    want = t["tok"].cpu().numpy().copy()
    assert (t["st"].cpu().numpy() == 0).all()

    def broken(**kw):
        a = _sample_args(t)
        for k, v in kw.items():
            setattr(a, k, v)
        return _call(ctx, a)

    E, CAP = _lib.XS_ERR_ARG, _lib.XS_ERR_CAPACITY
    assert ctx.lib.xs_sample(None, C.byref(_sample_args(t))) == E
    assert ctx.lib.xs_sample(ctx.h, None) == E
    assert broken(logits=None) == E
    assert broken(params=None) == E
    assert broken(uniforms=None) == E
    assert broken(token=None) == E
    assert broken(status=None) == E
    assert broken(rows=-1) == E
    assert broken(rows=ROWS + 1) == CAP                     # more rows than the context holds
    assert broken(enc=VOCAB + 4, width=VOCAB + 4, ld=VOCAB + 4) == CAP
    assert broken(ld=WIDTH + 2) == E                        # ld % 4 != 0
    assert broken(logits=t["logits"].data_ptr() + 4) == E   # row not 16-byte aligned
    assert broken(width=WIDTH + 8) == E                     # width > ld
    assert broken(enc=0) == E
    assert broken(cand_ld=0) == E                           # a candidate list of width 0
    assert broken(n_top=_lib.TOP_MAX + 1) == E
    assert broken(n_top=8, top_id=t["top"].data_ptr(), top_logprob=t["lp"].data_ptr(),
                  top_ld=4) == E                            # top_ld < n_top
    assert broken(allowed=t["mask"].data_ptr(), allowed_words=WIDTH // 32,
                  allowed_ld=WIDTH // 32 - 1) == E          # allowed_ld < allowed_words

    # nothing above launched: the outputs still hold the valid call's draws,
    # and the context samples the same way again
    torch.cuda.synchronize()
    assert (t["tok"].cpu().numpy() == want).all()
    t["tok"].fill_(-1)
    assert _call(ctx, _sample_args(t)) == _lib.XS_OK
    torch.cuda.synchronize()
    assert (t["tok"].cpu().numpy() == want).all()


def test_argmax_and_verify_argument_errors(setup):
    ctx, t = setup
    E, CAP = _lib.XS_ERR_ARG, _lib.XS_ERR_CAPACITY

    def am(**kw):
        a = _lib.ArgmaxArgs()
        a.logits, a.rows, a.ld, a.width = t["logits"].data_ptr(), ROWS, WIDTH + 4, WIDTH
        a.ids, a.probs = t["tok"].data_ptr(), t["prob"].data_ptr()
        for k, v in kw.items():
            setattr(a, k, v)
        return ctx.lib.xs_argmax_probs(ctx.h, C.byref(a))

    assert am() == _lib.XS_OK
    torch.cuda.synchronize()
    assert am(ids=None) == E
    assert am(probs=None) == E
    assert am(width=0) == E
    assert am(ld=WIDTH - 4) == E                             # ld < width
    assert am(rows=ROWS + 1) == CAP
    assert am(ld=WIDTH + 2) == E

    def vf(**kw):
        a = _lib.VerifyArgs()
        a.logits, a.seqs, a.span = t["logits"].data_ptr(), 2, 4
        a.ld, a.width, a.enc = WIDTH + 4, WIDTH, WIDTH
        a.params, a.uniforms = t["params"].data_ptr(), t["u"].data_ptr()
        a.drafts = t["cid"].data_ptr()
        a.row_token, a.row_status = t["tok"].data_ptr(), t["st"].data_ptr()
        a.accepted, a.committed = t["nc"].data_ptr(), t["top"].data_ptr()
        a.n_committed, a.seq_status = t["cid"].data_ptr() + 64, t["cid"].data_ptr() + 128
        for k, v in kw.items():
            setattr(a, k, v)
        return ctx.lib.xs_verify(ctx.h, C.byref(a))

    assert vf(span=0) == E
    assert vf(seqs=-1) == E
    assert vf(n_eog=2) == E                                  # two ids at a NULL list
    assert vf(n_eog=-1) == E
    assert vf(drafts=None) == E                              # span > 1 needs drafts
    assert vf(accepted=None) == E
    assert vf(seqs=ROWS, span=4) == CAP                      # 32 rows > 8


def test_top_k_above_the_contexts_k_max_is_a_row_error():
    """xs_create's k_max bounds min(top_k, enc): a context made for k_max = 20
    refuses top_k 21 (and a whole-row top_k on a wider row) per row, with
    XS_ROW_BAD_PARAM, and draws the other rows; a row narrower than k_max may
    ask for any top_k (its candidate set is the whole row)."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from xwen_amd import sampler as xsm
    rng = np.random.default_rng(77)
    ctx = xsm.Context(max_rows=4, vocab=4096, k_max=20)
    ctx.bind_current_stream()
    x = torch.as_tensor(rng.normal(0, 2, (4, 4096)).astype(np.float32)).cuda()
    p = xsm.params_tensor(1.0, np.array([20, 21, 10**9, 0]), 0.9, 4, "cuda")
    u = torch.full((4,), 0.3, dtype=torch.float32, device="cuda")
    out = xsm.sample_batch(ctx, x, p, u)
    torch.cuda.synchronize()
    assert out.status.cpu().tolist() == [_lib.ROW_OK, _lib.ROW_BAD_PARAM, _lib.ROW_BAD_PARAM,
                                         _lib.ROW_OK]
    # 16 encodable ids: top_k 10^9 is the whole 16-id row, within k_max
    small = torch.as_tensor(rng.normal(0, 2, (4, 16)).astype(np.float32)).cuda()
    out = xsm.sample_batch(ctx, small, p, u)
    torch.cuda.synchronize()
    assert out.status.cpu().tolist() == [_lib.ROW_OK, _lib.ROW_OK, _lib.ROW_OK, _lib.ROW_OK]
    ctx.close()
