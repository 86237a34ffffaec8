"""ctypes wrapper over the CPU oracle (oracle/_build/libxs_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker.  The product never imports it.
Each wrapper names the C function it calls; the C functions cite the
reference lines they restate (xs_oracle.c).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# XS_ORACLE_LIB names another build of the same library (the sanitized one of
# `make -C oracle asan`, for tests/test_sanitized.py)
LIB_PATH = os.environ.get("XS_ORACLE_LIB") or os.path.join(HERE, "_build", "libxs_oracle.so")

OK, NAN, NO_FINITE, MASK_SHORT, FORCE_OOR, ZERO_WEIGHT, NARROW = range(7)
ID_OOR = 9
SUM_SEQ_F32, SUM_F64, SUM_GIVEN = 0, 1, 2

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")


def build(force: bool = False) -> None:
    """Compile the oracle with its Makefile (gcc; a few seconds)."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)


class Control(C.Structure):
    """xo_control: SampleControl (sampler.rs:85-121)."""

    _fields_ = [
        ("allowed", C.c_void_p), ("allowed_words", C.c_int64),
        ("banned", C.c_void_p), ("n_banned", C.c_int64),
        ("bias_id", C.c_void_p), ("bias_delta", C.c_void_p), ("n_bias", C.c_int64),
        ("has_pull", C.c_int32), ("pull_id", C.c_uint32), ("pull_alpha", C.c_float),
        ("has_force", C.c_int32), ("force_id", C.c_uint32),
    ]


class Result(C.Structure):
    _fields_ = [
        ("status", C.c_int32), ("token", C.c_uint32), ("n_cand", C.c_int64),
        ("smax", C.c_float), ("ssum", C.c_float),
        ("margin_order", C.c_double), ("margin_cut", C.c_double), ("margin_draw", C.c_double),
    ]


_lib = None


def lib():
    global _lib
    if _lib is None:
        build()
        L = C.CDLL(LIB_PATH)
        L.xo_exp.restype = C.c_float
        L.xo_exp.argtypes = [C.c_float]
        L.xo_exp_array.restype = None
        L.xo_exp_array.argtypes = [_f32p, _f32p, C.c_int64]
        L.xo_set_exp_mode.restype = None
        L.xo_set_exp_mode.argtypes = [C.c_int32]
        L.xo_argmax.restype = C.c_int32
        L.xo_argmax.argtypes = [_f32p, C.c_int64, C.POINTER(C.c_uint32)]
        L.xo_softmax_in_place.restype = None
        L.xo_softmax_in_place.argtypes = [_f32p, C.c_int64, C.c_double, C.c_int32, C.c_float,
                                          C.POINTER(C.c_float), C.POINTER(C.c_float)]
        L.xo_top_k_desc.restype = C.c_int32
        L.xo_top_k_desc.argtypes = [_f32p, C.c_int64, C.c_int64, _f32p, _u32p]
        L.xo_candidate_set.restype = C.c_int32
        L.xo_candidate_set.argtypes = [_f32p, C.c_int64, C.c_int64, C.c_float, _f32p, _u32p,
                                       C.POINTER(C.c_int64)]
        L.xo_weighted_index.restype = C.c_int32
        L.xo_weighted_index.argtypes = [_f32p, C.c_int64, C.c_float, C.POINTER(C.c_int64)]
        L.xo_sample_controlled.restype = None
        L.xo_sample_controlled.argtypes = [
            _f32p, C.c_int64, C.c_int64, C.c_double, C.c_int64, C.c_double,
            C.POINTER(Control), C.c_float, C.c_int32, C.c_float, _f32p, _f32p, _u32p,
            C.c_int32, C.POINTER(Result)]
        L.xo_sample_rows.restype = None
        L.xo_sample_rows.argtypes = [
            C.c_void_p, C.c_int64, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p,
            C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, C.c_int32, C.c_int32,
            C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
        L.xo_accept_drafts.restype = C.c_int32
        L.xo_accept_drafts.argtypes = [C.c_void_p, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p,
                                       C.c_void_p, C.POINTER(C.c_int64), C.c_void_p,
                                       C.POINTER(C.c_int64), C.POINTER(C.c_int64)]
        L.xo_draft_argmax_probs.restype = C.c_int32
        L.xo_draft_argmax_probs.argtypes = [_f32p, C.c_int64, C.c_int64, _u32p, _f32p]
        L.xo_truncate_nucleus.restype = C.c_int64
        L.xo_truncate_nucleus.argtypes = [_f64p, C.c_int64, C.c_double]
        L.xo_select_option.restype = C.c_int32
        L.xo_select_option.argtypes = [_f64p, C.c_int64, C.c_double, C.c_int64, C.c_double,
                                       C.c_double, C.POINTER(C.c_int64)]
        L.xo_keep_confident.restype = C.c_int64
        L.xo_keep_confident.argtypes = [_u32p, _f32p, C.c_int64, C.c_float]
        L.xo_held_row.restype = C.c_int32
        L.xo_held_row.argtypes = [_f32p, C.c_int64, C.c_int64, C.POINTER(C.c_float),
                                  C.POINTER(C.c_double)]
        L.xo_last_logprobs_for.restype = C.c_int32
        L.xo_last_logprobs_for.argtypes = [_f32p, C.c_int64, C.c_int64, _i64p, C.c_int64, _f64p]
        L.xo_last_probs.restype = C.c_int32
        L.xo_last_probs.argtypes = [_f32p, C.c_int64, C.c_int64, _f64p]
        L.xo_class_masses.restype = None
        L.xo_class_masses.argtypes = [_f64p, C.c_int64, _u32p, C.c_int64, C.c_int64, _f64p]
        L.xo_det_logits.restype = None
        L.xo_det_logits.argtypes = [C.c_int64, C.c_uint64, C.c_float, _f32p]
        _lib = L
    return _lib


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def u32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint32))


def exp(x: float) -> float:
    return lib().xo_exp(float(x))


def exp_array(x: np.ndarray) -> np.ndarray:
    """xo_exp_array: the correctly rounded exp of every element."""
    xx = f32(x).ravel()
    y = np.empty_like(xx)
    lib().xo_exp_array(xx, y, xx.size)
    return y


def set_exp_mode(mode: int) -> None:
    """0: correctly rounded exp (parity, default); 1: libm expf (CPU-baseline timing)."""
    lib().xo_set_exp_mode(mode)


def argmax(values) -> tuple[int, int]:
    v = f32(values)
    out = C.c_uint32(0)
    st = lib().xo_argmax(v, v.size, C.byref(out))
    return st, out.value


def softmax_in_place(values, temperature: float, sum_mode: int = SUM_SEQ_F32,
                     s_given: float = 0.0):
    v = f32(values).copy()
    mx, sm = C.c_float(0), C.c_float(0)
    lib().xo_softmax_in_place(v, v.size, temperature, sum_mode, s_given, C.byref(mx), C.byref(sm))
    return v, mx.value, sm.value


def top_k_desc(probs, k: int):
    p = f32(probs)
    w = np.zeros(k, np.float32)
    i = np.zeros(k, np.uint32)
    st = lib().xo_top_k_desc(p, p.size, k, w, i)
    return st, list(zip(w.tolist(), i.tolist()))


def candidate_set(probs, k: int, top_p: float):
    p = f32(probs)
    m = min(k, p.size) if k < p.size else p.size
    w = np.zeros(max(m, 1), np.float32)
    i = np.zeros(max(m, 1), np.uint32)
    n = C.c_int64(0)
    st = lib().xo_candidate_set(p, p.size, k, np.float32(top_p), w, i, C.byref(n))
    return st, list(zip(w[: n.value].tolist(), i[: n.value].tolist()))


def weighted_index(weights, u: float):
    w = f32(weights)
    idx = C.c_int64(0)
    st = lib().xo_weighted_index(w, w.size, np.float32(u), C.byref(idx))
    return st, idx.value


@dataclass
class Ctl:
    """SampleControl in Python form (sampler.rs:85-121)."""

    allowed: object = None
    banned: tuple = ()
    bias: tuple = ()
    pull: object = None
    force: object = None

    def to_c(self):
        keep = []
        c = Control()
        if self.allowed is not None:
            a = u32(self.allowed)
            keep.append(a)
            c.allowed, c.allowed_words = a.ctypes.data, a.size
        if self.banned:
            b = u32(self.banned)
            keep.append(b)
            c.banned, c.n_banned = b.ctypes.data, b.size
        if self.bias:
            bi = u32([x[0] for x in self.bias])
            bd = f32([x[1] for x in self.bias])
            keep += [bi, bd]
            c.bias_id, c.bias_delta, c.n_bias = bi.ctypes.data, bd.ctypes.data, bi.size
        if self.pull is not None:
            c.has_pull, c.pull_id, c.pull_alpha = 1, self.pull[0], self.pull[1]
        if self.force is not None:
            c.has_force, c.force_id = 1, self.force
        return c, keep


@dataclass
class Draw:
    status: int
    token: int
    cand: list
    smax: float
    ssum: float
    margin_order: float
    margin_cut: float
    margin_draw: float


def sample_controlled(logits, enc: int, temperature: float, top_k: int, top_p: float,
                      u: float = 0.0, ctl: Ctl | None = None, sum_mode: int = SUM_SEQ_F32,
                      s_given: float = 0.0, margins: bool = False) -> Draw:
    """xo_sample_controlled: Sampler::sample_controlled + draw (sampler.rs:190-243)."""
    v = f32(logits)
    work = np.zeros(max(enc, 1), np.float32)
    kc = max(1, min(int(top_k), enc)) if top_k > 0 else 1
    cw = np.zeros(kc, np.float32)
    ci = np.zeros(kc, np.uint32)
    c, keep = (ctl or Ctl()).to_c()
    res = Result()
    lib().xo_sample_controlled(v, v.size, enc, temperature, int(top_k), top_p, C.byref(c),
                               np.float32(u), sum_mode, np.float32(s_given), work, cw, ci,
                               1 if margins else 0, C.byref(res))
    del keep
    cand = list(zip(cw[: res.n_cand].tolist(), ci[: res.n_cand].tolist()))
    return Draw(res.status, res.token, cand, res.smax, res.ssum, res.margin_order,
                res.margin_cut, res.margin_draw)


def sample_rows(logits: np.ndarray, enc: int, temperature, top_k, top_p, u, mask=None,
                k_out: int = 0, sum_mode: int = SUM_SEQ_F32, nthreads: int = 1):
    """xo_sample_rows: the row-parallel CPU baseline (no controls but the mask)."""
    x = np.ascontiguousarray(logits, np.float32)
    rows, ld = x.shape
    T = np.ascontiguousarray(np.broadcast_to(np.asarray(temperature, np.float64), (rows,)))
    K = np.ascontiguousarray(np.broadcast_to(np.asarray(top_k, np.int64), (rows,)))
    P = np.ascontiguousarray(np.broadcast_to(np.asarray(top_p, np.float64), (rows,)))
    U = np.ascontiguousarray(np.broadcast_to(np.asarray(u, np.float32), (rows,)))
    tok = np.zeros(rows, np.uint32)
    st = np.zeros(rows, np.int32)
    smax = np.zeros(rows, np.float32)
    ssum = np.zeros(rows, np.float32)
    cw = np.zeros((rows, max(k_out, 1)), np.float32)
    ci = np.zeros((rows, max(k_out, 1)), np.uint32)
    mptr, mld = 0, 0
    if mask is not None:
        mask = np.ascontiguousarray(mask, np.uint32)
        mptr, mld = mask.ctypes.data, mask.shape[1]
    lib().xo_sample_rows(x.ctypes.data, rows, ld, enc, T.ctypes.data, K.ctypes.data,
                         P.ctypes.data, U.ctypes.data, mptr, mld, k_out, sum_mode, nthreads,
                         tok.ctypes.data, st.ctypes.data,
                         cw.ctypes.data if k_out else None, ci.ctypes.data if k_out else None,
                         smax.ctypes.data, ssum.ctypes.data)
    return dict(token=tok, status=st, cand_w=cw[:, :k_out], cand_id=ci[:, :k_out],
                smax=smax, ssum=ssum)


def accept_drafts(drafts, budget: int, row_token, row_eog, row_status=None):
    """xo_accept_drafts: the verify walk (generate.rs:4020-4046)."""
    d = u32(drafts) if len(drafts) else np.zeros(1, np.uint32)
    t = u32(row_token)
    e = np.ascontiguousarray(np.asarray(row_eog, np.uint8))
    s = None if row_status is None else np.ascontiguousarray(np.asarray(row_status, np.int32))
    com = np.zeros(len(drafts) + 1, np.uint32)
    m, nc, calls = C.c_int64(0), C.c_int64(0), C.c_int64(0)
    st = lib().xo_accept_drafts(d.ctypes.data, len(drafts), budget, t.ctypes.data,
                                None if s is None else s.ctypes.data, e.ctypes.data,
                                C.byref(m), com.ctypes.data, C.byref(nc), C.byref(calls))
    return st, m.value, com[: nc.value].tolist(), calls.value


def draft_argmax_probs(logits: np.ndarray):
    x = np.ascontiguousarray(logits, np.float32)
    n, v = x.shape
    ids = np.zeros(n, np.uint32)
    pr = np.zeros(n, np.float32)
    lib().xo_draft_argmax_probs(x, n, v, ids, pr)
    return ids, pr


def truncate_nucleus(probs, top_p: float) -> int:
    """xo_truncate_nucleus: how many of the ranked probabilities the cut keeps."""
    p = np.ascontiguousarray(probs, np.float64)
    return int(lib().xo_truncate_nucleus(p, p.size, float(top_p)))


def select_option(scores, temperature: float, top_k: int, top_p: float, u: float = 0.0):
    """xo_select_option: (status, index) of batch.rs's select_option for uniform u."""
    s = np.ascontiguousarray(scores, np.float64)
    idx = C.c_int64(-1)
    st = lib().xo_select_option(s, s.size, float(temperature), int(top_k), float(top_p),
                                float(u), C.byref(idx))
    return int(st), int(idx.value)


def keep_confident(ids, probs, p_min: float):
    i = u32(ids) if len(ids) else np.zeros(1, np.uint32)
    p = f32(probs) if len(probs) else np.zeros(1, np.float32)
    k = lib().xo_keep_confident(i, p, len(ids), np.float32(p_min))
    return list(ids[:k])


def held_row(row, enc: int):
    r = f32(row)
    mx, lse = C.c_float(0), C.c_double(0)
    st = lib().xo_held_row(r, r.size, enc, C.byref(mx), C.byref(lse))
    return st, mx.value, lse.value


def last_logprobs_for(row, enc: int, ids):
    """(status, f64 log-probs of ids): generate.rs:1871-1883."""
    r = f32(row)
    i = np.ascontiguousarray(np.asarray(ids, np.int64)) if len(ids) else np.zeros(1, np.int64)
    out = np.zeros(max(len(ids), 1), np.float64)
    st = lib().xo_last_logprobs_for(r, r.size, enc, i, len(ids), out)
    return st, out[:len(ids)]


def last_probs(row, enc: int):
    """(status, f64 probabilities of ids 0..enc-1): generate.rs:1893-1899."""
    r = f32(row)
    out = np.zeros(max(enc, 1), np.float64)
    st = lib().xo_last_probs(r, r.size, enc, out)
    return st, out[:enc]


def class_masses(probs, masks) -> np.ndarray:
    """escape_mass's per-class sums (batch.rs:1638-1662): masks [n_class, words] u32."""
    p = np.ascontiguousarray(np.asarray(probs, np.float64))
    m = np.ascontiguousarray(np.asarray(masks, np.uint32))
    out = np.zeros(max(m.shape[0], 1), np.float64)
    lib().xo_class_masses(p, p.size, m, m.shape[0], m.shape[1], out)
    return out[:m.shape[0]]


def det_logits(n: int, seed: int, scale: float) -> np.ndarray:
    out = np.zeros(n, np.float32)
    lib().xo_det_logits(n, seed, np.float32(scale), out)
    return out
