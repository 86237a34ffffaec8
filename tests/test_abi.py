"""The C ABI without a GPU: the library loads, exports every entry point the
header declares, its structs have the header's layout, and its host-only entry
point (keep_confident) answers the reference's known cases."""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

from tests import workloads
from xwen_amd import _lib


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _lib.declared_symbols()
    assert {"xs_create", "xs_destroy", "xs_set_stream", "xs_sample", "xs_verify",
            "xs_argmax_probs", "xs_keep_confident", "xs_version", "xs_test_exp"} <= set(declared)
    for name in declared:
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert set(declared) <= exported


def test_version_string():
    assert _lib.load().xs_version().decode().startswith("xsamp")


def _layout_from_c(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text(r'''
#include <stddef.h>
#include <stdio.h>
#include "xsamp.h"
#define F(T, m) printf(#T "." #m " %zu\n", offsetof(T, m))
int main(void) {
  printf("xs_row_params %zu\n", sizeof(xs_row_params));
  printf("xs_sample_args %zu\n", sizeof(xs_sample_args));
  printf("xs_verify_args %zu\n", sizeof(xs_verify_args));
  printf("xs_argmax_args %zu\n", sizeof(xs_argmax_args));
  printf("xs_row_control %zu\n", sizeof(xs_row_control));
  F(xs_row_params, top_k); F(xs_row_params, top_p);
  F(xs_sample_args, params); F(xs_sample_args, allowed); F(xs_sample_args, token);
  F(xs_sample_args, cand_ld); F(xs_sample_args, n_top); F(xs_sample_args, top_ld);
  F(xs_verify_args, drafts); F(xs_verify_args, n_eog); F(xs_verify_args, eog);
  F(xs_verify_args, row_token); F(xs_verify_args, seq_status);
  F(xs_argmax_args, width); F(xs_argmax_args, ids); F(xs_argmax_args, probs);
  F(xs_row_control, n_bias); F(xs_row_control, pull_alpha); F(xs_row_control, force_id);
  F(xs_sample_args, controls); F(xs_sample_args, ctl_delta);
  F(xs_verify_args, controls); F(xs_verify_args, ctl_delta); F(xs_verify_args, done_after);
  F(xs_sample_args, row_order); F(xs_sample_args, k_max); F(xs_verify_args, k_max);
  F(xs_sample_args, top_logprob64); F(xs_sample_args, n_score); F(xs_sample_args, score_logprob);
  F(xs_sample_args, class_masks); F(xs_sample_args, class_ld); F(xs_sample_args, class_mass);
  F(xs_sample_args, probs); F(xs_sample_args, probs_ld);
  return 0;
}
''')
    exe = tmp_path / "layout"
    inc = os.path.join(_lib.ROOT, "include")
    subprocess.run(["gcc", "-I", inc, str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout
    return dict(line.rsplit(" ", 1) for line in out.splitlines())


def test_ctypes_structs_match_the_header(tmp_path):
    c = {k: int(v) for k, v in _layout_from_c(tmp_path).items()}
    assert C.sizeof(_lib.RowParams) == c["xs_row_params"]
    assert C.sizeof(_lib.SampleArgs) == c["xs_sample_args"]
    assert C.sizeof(_lib.VerifyArgs) == c["xs_verify_args"]
    assert C.sizeof(_lib.ArgmaxArgs) == c["xs_argmax_args"]
    assert C.sizeof(_lib.RowControl) == c["xs_row_control"]
    for struct, cname in ((_lib.RowParams, "xs_row_params"), (_lib.SampleArgs, "xs_sample_args"),
                          (_lib.VerifyArgs, "xs_verify_args"), (_lib.ArgmaxArgs, "xs_argmax_args"),
                          (_lib.RowControl, "xs_row_control")):
        for field, _ in struct._fields_:
            key = f"{cname}.{field}"
            if key in c:
                assert getattr(struct, field).offset == c[key], key


def test_params_tensor_packs_xs_row_params():
    torch = pytest.importorskip("torch")
    from xwen_amd import sampler as xsm
    raw = xsm.params_tensor([0.7, 0.0], [20, 1], [0.8, 1.0], 2, "cpu").numpy()
    assert raw.size == 2 * C.sizeof(_lib.RowParams)
    p = (_lib.RowParams * 2).from_buffer_copy(raw.tobytes())
    assert (p[0].temperature, p[0].top_k, p[0].top_p) == (0.7, 20, np.float32(0.8))
    assert (p[1].temperature, p[1].top_k, p[1].top_p) == (0.0, 1, 1.0)
    del torch


def test_params_tensor_saturates_a_huge_top_k():
    """The reference's top_k is a usize: 2^32, 2^32 + 20 and usize::MAX are all
    at least the vocabulary (the whole-row candidate set).  Narrowing must not
    wrap them to 0 (greedy), 20 or -1."""
    pytest.importorskip("torch")
    from xwen_amd import sampler as xsm
    ks = [1 << 32, (1 << 32) + 20, (1 << 64) - 1, (1 << 31) - 1, 20]
    raw = xsm.params_tensor(1.0, ks, 0.9, len(ks), "cpu").numpy()
    p = (_lib.RowParams * len(ks)).from_buffer_copy(raw.tobytes())
    assert [p[i].top_k for i in range(len(ks))] == [2**31 - 1] * 4 + [20]
    assert not xsm.SamplerOptions(1.0, 1 << 32, 0.9).is_greedy()


def test_keep_confident_through_the_abi(golden):
    from xwen_amd import sampler as xsm
    c = golden["keep_confident"]
    for case in c["cases"]:
        assert xsm.keep_confident(c["ids"], case["probs"], case["p_min"]) == case["expect"]
    assert xsm.keep_confident([], [], c["empty"]["p_min"]) == c["empty"]["expect"]


def test_create_without_a_gpu_fails_cleanly():
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    h = C.c_void_p()
    rc = _lib.load().xs_create(0, 4, 1024, 20, C.byref(h))
    assert rc == _lib.XS_ERR_HIP and not h.value


def test_mask_packing_round_trips():
    rng = np.random.default_rng(1)
    allow = rng.random((3, 1000)) < 0.3
    words = workloads.pack_mask(allow)
    assert words.shape == (3, 32) and words.dtype == np.uint32
    for r in range(3):
        np.testing.assert_array_equal(workloads.mask_bits(words[r], 1000), allow[r])
    # the reference's own example: mask 0b0101 allows ids 0 and 2 (sampler.rs:819-833)
    w = workloads.pack_mask(np.array([[True, False, True, False]]))
    assert w[0, 0] == 0b0101


def test_select_option_through_the_abi(golden, oracle):
    """xs_select_option (host code in the library) against the oracle's
    restatement, index for index, and on the reference's own cases."""
    from xwen_amd import sampler as xsm
    rng = np.random.default_rng(6)
    for trial in range(400):
        n = int(rng.integers(1, 12))
        scores = rng.normal(0, 3, n)
        if trial % 5 == 0:
            scores[rng.integers(0, n)] = scores.max()  # a tie at the top
        T = float(rng.choice([0.0, 0.5, 1.0, 2.5]))
        k = int(rng.choice([1, 2, 3, 20]))
        p = float(rng.choice([0.3, 0.8, 0.95, 1.0]))
        u = float(rng.integers(0, 1 << 52)) * 2.0 ** -52
        st, idx = oracle.select_option(scores, T, k, p, u)
        assert st == 0
        got = xsm.select_option(scores, xsm.SamplerOptions(temperature=T, top_k=k, top_p=p), u)
        assert got == idx, (trial, scores, T, k, p, u)
    c = golden["select_option"]
    T, k, p = c["tight"]
    assert xsm.select_option(c["scores"], xsm.SamplerOptions(T, k, p), 0.99) == c["tight_expect"]
    with pytest.raises(xsm.SampleError):
        xsm.select_option([0.0, float("nan")], xsm.SamplerOptions(1.0, 20, 0.9), 0.5)
