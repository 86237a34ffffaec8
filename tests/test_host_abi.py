"""The host-only part of the C ABI, without a GPU: the argument checks every
device entry point makes before it touches the device (xs_host_check_*), and
the host entry points xs_select_option (select_option, batch.rs:1545-1588)
and xs_keep_confident (keep_confident, generate.rs:3898-3905).  Loads
libxsamp.so, or the sanitized host build named by XS_HOST_LIB
(tests/test_sanitized.py runs this module under AddressSanitizer and UBSan)."""
import ctypes as C
import os

import numpy as np
import pytest

from xwen_amd import _lib

E, CAP, OK = _lib.XS_ERR_ARG, _lib.XS_ERR_CAPACITY, _lib.XS_OK


class Limits(C.Structure):
    _fields_ = [("max_rows", C.c_int64), ("vocab", C.c_int64), ("max_chunks", C.c_int32)]


@pytest.fixture(scope="module")
def host():
    L = C.CDLL(os.environ.get("XS_HOST_LIB") or _lib.LIB_PATH)
    L.xs_host_check_sample.argtypes = [C.POINTER(Limits), C.POINTER(_lib.SampleArgs)]
    L.xs_host_check_verify.argtypes = [C.POINTER(Limits), C.POINTER(_lib.VerifyArgs)]
    L.xs_host_check_argmax.argtypes = [C.POINTER(Limits), C.POINTER(_lib.ArgmaxArgs)]
    for f in ("xs_host_check_sample", "xs_host_check_verify", "xs_host_check_argmax"):
        getattr(L, f).restype = C.c_int
    L.xs_select_option.restype = C.c_int32
    L.xs_select_option.argtypes = [C.c_void_p, C.c_int64, C.c_double, C.c_int64, C.c_double,
                                   C.c_double, C.POINTER(C.c_int64)]
    L.xs_keep_confident.restype = C.c_int64
    L.xs_keep_confident.argtypes = [C.c_void_p, C.c_int64, C.c_float]
    return L


LIM = Limits(8, 300_000, 19)  # 19 chunks hold 300,000 ids (293 slots of 1,024)
DEV = 0x7f0000001000          # an aligned stand-in device address: checks never dereference it


def _sample(**kw):
    a = _lib.SampleArgs()
    a.logits, a.rows, a.ld, a.width, a.enc = DEV, 4, 248_320, 248_320, 248_320
    a.params, a.uniforms, a.token, a.status = DEV, DEV, DEV, DEV
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def test_sample_argument_checks(host):
    chk = lambda **kw: host.xs_host_check_sample(C.byref(LIM), C.byref(_sample(**kw)))
    assert chk() == OK
    assert host.xs_host_check_sample(None, C.byref(_sample())) == E
    assert host.xs_host_check_sample(C.byref(LIM), None) == E
    assert chk(token=None) == E and chk(status=None) == E and chk(params=None) == E
    assert chk(uniforms=None) == E and chk(logits=None) == E
    assert chk(rows=-1) == E and chk(enc=0) == E and chk(ld=0) == E
    assert chk(rows=9) == CAP and chk(enc=300_001, ld=300_004, width=300_004) == CAP
    assert chk(ld=248_322) == E                                   # ld % 4
    assert chk(logits=DEV + 8) == E                               # 16-byte alignment
    assert chk(width=248_324) == E                                # width > ld
    assert chk(allowed=DEV, allowed_words=7760, allowed_ld=7759) == E
    assert chk(allowed=DEV, allowed_words=-1, allowed_ld=7760) == E
    assert chk(cand_id=DEV, cand_ld=0) == E
    assert chk(n_top=-1) == E and chk(n_top=_lib.TOP_MAX + 1) == E
    assert chk(top_id=DEV, n_top=20, top_ld=19) == E
    # held_row outputs over the raw row beside a masked or controlled draw
    assert chk(row_lse=DEV, allowed=DEV, allowed_words=7760, allowed_ld=7760) == OK
    assert chk(row_max=DEV, controls=DEV) == OK
    narrow = Limits(8, 300_000, 15)                               # 15 chunks < 16 needed
    assert host.xs_host_check_sample(C.byref(narrow), C.byref(_sample())) == CAP


def test_scoring_argument_checks(host):
    """The scoring reads (score_ids, class masks, probs): each output needs its
    input and room for the row's ids, and like the held_row outputs they do
    not combine with an allow-mask or controls."""
    chk = lambda **kw: host.xs_host_check_sample(C.byref(LIM), C.byref(_sample(**kw)))
    assert chk(score_ids=DEV, score_logprob=DEV, n_score=5, score_ld=5) == OK
    assert chk(score_ids=DEV, n_score=5, score_ld=5) == E            # no output
    assert chk(score_logprob=DEV, n_score=5, score_ld=5) == E        # no ids
    assert chk(score_ids=DEV, score_logprob=DEV, n_score=5, score_ld=4) == E
    assert chk(score_ids=DEV, score_logprob=DEV, n_score=_lib.SCORE_MAX + 1, score_ld=10**5) == E
    assert chk(score_ids=DEV, score_logprob=DEV, n_score=-1, score_ld=5) == E
    assert chk(class_masks=DEV, class_mass=DEV, n_class=2, class_ld=7760) == OK
    assert chk(class_masks=DEV, class_mass=DEV, n_class=2, class_ld=7759) == E
    assert chk(class_masks=DEV, n_class=2, class_ld=7760) == E
    assert chk(class_masks=DEV, class_mass=DEV, n_class=_lib.CLASS_MAX + 1, class_ld=7760) == E
    assert chk(probs=DEV, probs_ld=248_320) == OK and chk(probs=DEV, probs_ld=248_319) == E
    # the scoring reads of the raw row beside a masked or controlled draw
    assert chk(probs=DEV, probs_ld=248_320, allowed=DEV, allowed_words=7760, allowed_ld=7760) == OK
    assert chk(score_ids=DEV, score_logprob=DEV, n_score=1, score_ld=1, controls=DEV) == OK
    assert chk(top_logprob64=DEV, n_top=20, top_ld=19) == E


def test_row_order_must_be_a_permutation(host):
    def chk(order, rows=4):
        o = np.ascontiguousarray(np.asarray(order, np.int32))
        return host.xs_host_check_sample(C.byref(Limits(2000, 300_000, 19)),
                                         C.byref(_sample(rows=rows, row_order=o.ctypes.data)))
    assert chk([3, 1, 0, 2]) == OK
    assert chk([3, 1, 1, 2]) == E and chk([0, 1, 2, 4]) == E and chk([0, -1, 2, 3]) == E
    assert chk(np.arange(_lib.ORDER_MAX), rows=_lib.ORDER_MAX) == OK
    # past ORDER_MAX rows the order is checked, then not applied
    big = np.arange(_lib.ORDER_MAX + 1)[::-1]
    assert chk(big, rows=_lib.ORDER_MAX + 1) == OK
    big = big.copy()
    big[7] = big[8]
    assert chk(big, rows=_lib.ORDER_MAX + 1) == E


def test_verify_and_argmax_argument_checks(host):
    def vf(**kw):
        a = _lib.VerifyArgs()
        a.logits, a.seqs, a.span, a.ld, a.width, a.enc = DEV, 2, 4, 248_320, 248_320, 248_320
        a.params, a.uniforms, a.drafts = DEV, DEV, DEV
        a.row_token = a.row_status = a.accepted = a.committed = a.n_committed = a.seq_status = DEV
        for k, v in kw.items():
            setattr(a, k, v)
        return host.xs_host_check_verify(C.byref(LIM), C.byref(a))
    assert vf() == OK
    assert vf(span=0) == E and vf(seqs=-1) == E and vf(n_eog=-1) == E
    assert vf(n_eog=2) == E and vf(n_eog=2, eog=DEV) == OK and vf(n_eog=300, eog=DEV) == OK
    assert vf(drafts=None) == E and vf(drafts=None, span=1) == OK
    assert vf(accepted=None) == E and vf(seq_status=None) == E
    assert vf(seqs=3) == CAP                                      # 12 rows > 8
    assert vf(seqs=2**62, span=4) == CAP                          # no overflow into a small count

    def am(**kw):
        a = _lib.ArgmaxArgs()
        a.logits, a.rows, a.ld, a.width, a.ids, a.probs = DEV, 5, 248_320, 248_320, DEV, DEV
        for k, v in kw.items():
            setattr(a, k, v)
        return host.xs_host_check_argmax(C.byref(LIM), C.byref(a))
    assert am() == OK
    assert am(ids=None) == E and am(probs=None) == E and am(width=0) == E
    assert am(ld=248_316) == E and am(ld=248_322) == E and am(logits=DEV + 4) == E
    assert am(rows=9) == CAP and am(width=300_004, ld=300_004) == CAP


def test_select_option_and_keep_confident(host, golden, oracle):
    """The host entry points against the reference's known answers and, index
    for index, against the oracle over random scores and uniforms."""
    def sel(scores, T, k, p, u):
        s = np.ascontiguousarray(np.asarray(scores, np.float64))
        idx = C.c_int64(-1)
        st = host.xs_select_option(s.ctypes.data, s.size, T, k, p, u, C.byref(idx))
        return st, idx.value
    c = golden["select_option"]
    sc = c["scores"]
    for T, k, p in c["greedy"]:
        assert sel(sc, T, k, p, 0.7) == (0, c["greedy_expect"])
    T, k, p = c["tight"]
    assert sel(sc, T, k, p, 0.99) == (0, c["tight_expect"])
    rng = np.random.default_rng(5)
    for _ in range(300):
        n = int(rng.integers(1, 40))
        s = rng.normal(0, 3, n)
        T = float(rng.choice([0.0, 0.5, 1.0, 1.7]))
        k = int(rng.choice([0, 1, 2, 5, 50]))
        p = float(rng.choice([0.3, 0.9, 1.0]))
        u = float(rng.integers(0, 1 << 52)) * 2.0 ** -52
        assert sel(s, T, k, p, u) == oracle.select_option(s, T, k, p, u)
    assert sel([], 1.0, 5, 0.9, 0.1)[0] == E
    kc = golden["keep_confident"]
    for case in kc["cases"]:
        pr = np.array([float(v) for v in case["probs"]], np.float32)
        assert host.xs_keep_confident(pr.ctypes.data, pr.size, C.c_float(case["p_min"])) \
            == len(case["expect"])
