"""ctypes binding of libxsamp.so: the structs and entry points of include/xsamp.h.

The product path: every call goes through the C ABI into the HIP kernels.  A
missing library is an error (no CPU fallback exists or is wanted).
"""
from __future__ import annotations

import ctypes as C
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "libxsamp.so")
HEADER = os.path.join(ROOT, "include", "xsamp.h")

XS_OK, XS_ERR_ARG, XS_ERR_HIP, XS_ERR_CAPACITY = 0, -1, -2, -3
ROW_OK, ROW_NAN, ROW_NO_FINITE, ROW_MASK_SHORT, ROW_FORCE_OOR, ROW_ZERO_WEIGHT, ROW_NARROW, \
    ROW_BAD_PARAM, ROW_INTERNAL, ROW_ID_OOR = range(10)
K_MAX = 127
SCORE_MAX = 4096
CLASS_MAX = 8
TOP_MAX = 128
CTL_MAX = 2048
ORDER_MAX = 1024
NOALLOC_ROWS = 64
NOALLOC_VOCAB = 262144
NOALLOC_BYTES = 15030784

_vp = C.c_void_p
_i64 = C.c_int64
_i32 = C.c_int32


class RowParams(C.Structure):
    """xs_row_params: SamplerOptions minus the seed (sampler.rs:36-41)."""

    _fields_ = [("temperature", C.c_double), ("top_k", _i32), ("top_p", C.c_float)]


class RowControl(C.Structure):
    """xs_row_control: SampleControl's bans, biases, pull and force (sampler.rs:85-121)."""

    _fields_ = [("ban_off", _i32), ("n_ban", _i32), ("bias_off", _i32), ("n_bias", _i32),
                ("has_pull", _i32), ("pull_id", C.c_uint32), ("pull_alpha", C.c_float),
                ("has_force", _i32), ("force_id", C.c_uint32)]


class SampleArgs(C.Structure):
    _fields_ = [
        ("logits", _vp), ("rows", _i64), ("ld", _i64), ("width", _i64), ("enc", _i64),
        ("params", _vp), ("uniforms", _vp),
        ("allowed", _vp), ("allowed_words", _i64), ("allowed_ld", _i64),
        ("token", _vp), ("status", _vp), ("cand_id", _vp), ("cand_w", _vp), ("n_cand", _vp),
        ("cand_ld", _i64), ("soft_max", _vp), ("soft_sum", _vp),
        ("row_max", _vp), ("row_lse", _vp), ("n_top", _i32), ("top_id", _vp),
        ("top_logprob", _vp), ("top_ld", _i64),
        ("controls", _vp), ("ctl_ids", _vp), ("ctl_delta", _vp),
        ("row_order", _vp),  # host array [rows] (int32), or NULL
        ("k_max", _i32),     # this call's bound on min(top_k, enc), 0 = the context's
        ("top_logprob64", _vp),
        ("score_ids", _vp), ("n_score", _i32), ("score_ld", _i64), ("score_logprob", _vp),
        ("class_masks", _vp), ("n_class", _i32), ("class_ld", _i64), ("class_mass", _vp),
        ("probs", _vp), ("probs_ld", _i64),
    ]


class VerifyArgs(C.Structure):
    _fields_ = [
        ("logits", _vp), ("seqs", _i64), ("span", _i64), ("ld", _i64), ("width", _i64),
        ("enc", _i64), ("params", _vp), ("uniforms", _vp),
        ("allowed", _vp), ("allowed_words", _i64), ("allowed_ld", _i64),
        ("drafts", _vp), ("budget", _vp), ("n_eog", _i32), ("eog", _vp),
        ("row_token", _vp), ("row_status", _vp), ("accepted", _vp), ("committed", _vp),
        ("n_committed", _vp), ("seq_status", _vp),
        ("controls", _vp), ("ctl_ids", _vp), ("ctl_delta", _vp), ("done_after", _vp),
        ("k_max", _i32),
    ]


class ArgmaxArgs(C.Structure):
    _fields_ = [("logits", _vp), ("rows", _i64), ("ld", _i64), ("width", _i64),
                ("ids", _vp), ("probs", _vp)]


class XsError(RuntimeError):
    pass


_lib = None


def load() -> C.CDLL:
    """Load libxsamp.so (built by __graft_entry__.build()); raise if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise XsError(f"{LIB_PATH} is missing: run __graft_entry__.build() (hipcc, gfx950)")
    L = C.CDLL(LIB_PATH)
    L.xs_create.restype = C.c_int
    L.xs_create.argtypes = [C.c_int, _i64, _i64, _i32, C.POINTER(_vp)]
    L.xs_create_ex.restype = C.c_int
    L.xs_create_ex.argtypes = [C.c_int, _i64, _i64, _i32, _i32, C.POINTER(_vp)]
    L.xs_destroy.restype = C.c_int
    L.xs_destroy.argtypes = [_vp]
    L.xs_set_stream.restype = C.c_int
    L.xs_set_stream.argtypes = [_vp, _vp]
    L.xs_sample.restype = C.c_int
    L.xs_sample.argtypes = [_vp, C.POINTER(SampleArgs)]
    L.xs_sample_noalloc.restype = C.c_int
    L.xs_sample_noalloc.argtypes = [C.POINTER(SampleArgs), _vp]
    L.xs_verify.restype = C.c_int
    L.xs_verify.argtypes = [_vp, C.POINTER(VerifyArgs)]
    L.xs_argmax_probs.restype = C.c_int
    L.xs_argmax_probs.argtypes = [_vp, C.POINTER(ArgmaxArgs)]
    L.xs_select_option.restype = _i32
    L.xs_select_option.argtypes = [_vp, _i64, C.c_double, _i64, C.c_double, C.c_double,
                                   C.POINTER(_i64)]
    L.xs_keep_confident.restype = _i64
    L.xs_keep_confident.argtypes = [_vp, _i64, C.c_float]
    L.xs_version.restype = C.c_char_p
    L.xs_version.argtypes = []
    L.xs_test_exp.restype = C.c_int
    L.xs_test_exp.argtypes = [_vp, _vp, _i64, _vp]
    L.xs_test_serial_fallback.restype = C.c_int
    L.xs_test_serial_fallback.argtypes = [_vp, _i32, C.POINTER(C.c_uint32)]
    L.xs_test_xcd.restype = C.c_int
    L.xs_test_xcd.argtypes = [_vp, _i32, C.POINTER(C.c_int32)]
    _lib = L
    return L


def declared_symbols() -> list[str]:
    """Every function include/xsamp.h declares."""
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\*?\s+\*?(xs_[a-z_0-9]+)\(", text,
                                 re.M)))


def check(rc: int, what: str) -> None:
    if rc != XS_OK:
        names = {XS_ERR_ARG: "XS_ERR_ARG", XS_ERR_HIP: "XS_ERR_HIP",
                 XS_ERR_CAPACITY: "XS_ERR_CAPACITY"}
        raise XsError(f"{what} failed: {names.get(rc, rc)}")
