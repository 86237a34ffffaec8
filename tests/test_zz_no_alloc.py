"""xs_sample_noalloc, the entry point that allocates nothing (its workspace is
the library's static device array), against xs_sample on a context: the same
inputs give the same tokens, statuses, candidates and statistics bit for bit.
Two calls in a row, the second smaller than the first, so the second runs on
the array the first left behind; then the limits (rows, vocabulary, k_max)."""
import numpy as np
import pytest

from tests import workloads

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

V = workloads.V


def _np(out):
    return {k: (None if v is None else v.cpu().numpy()) for k, v in vars(out).items()}


def _same(got, want, n_cand_col="n_cand"):
    assert (want["status"] == 0).all(), want["status"]
    for k in ("token", "status", "n_cand", "soft_max", "soft_sum", "row_max", "row_lse",
              "top_id", "top_logprob"):
        if want.get(k) is None:
            continue
        a, b = got[k], want[k]
        if a.dtype.kind == "f":
            a, b = a.view(np.uint32 if a.itemsize == 4 else np.uint64), \
                b.view(np.uint32 if b.itemsize == 4 else np.uint64)
        assert (a == b).all(), k
    if want.get("cand_id") is not None:
        for r in range(len(want["n_cand"])):  # entries past n_cand are not written
            n = min(int(want["n_cand"][r]), want["cand_id"].shape[1])
            assert (got["cand_id"][r, :n] == want["cand_id"][r, :n]).all(), r
            assert (got["cand_w"][r, :n].view(np.uint32)
                    == want["cand_w"][r, :n].view(np.uint32)).all(), r


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def test_noalloc_matches_xs_sample_on_two_calls_in_a_row():
    _need_gpu()
    from xwen_amd import sampler as xsm
    torch.cuda.set_device(0)
    ctx = xsm.Context(max_rows=64, vocab=V)
    ctx.bind_current_stream()

    # first call: the batch-64 configuration at full width (64 rows: the
    # XCD-local hand-off)
    wl = workloads.c2_batch()
    lg = torch.as_tensor(wl.logits).cuda()
    p = xsm.params_tensor(wl.temperature, wl.top_k, wl.top_p, 64, "cuda")
    u = torch.as_tensor(wl.u).cuda()
    print("noalloc call 1: 64 x 248320", flush=True)
    got = xsm.sample_batch_noalloc(lg, p, u, cand_k=20, stats=True)
    want = xsm.sample_batch(ctx, lg, p, u, cand_k=20, stats=True)
    torch.cuda.synchronize()
    _same(_np(got), _np(want))

    # second call, smaller: 9 rows x 65,536 ids with allow-masks and mixed k
    rng = np.random.default_rng(907)
    rows, width = 9, 65_536
    x = rng.normal(0, 3, (rows, width)).astype(np.float32)
    x[:, rng.integers(0, width, 5)] += np.float32(9.0)
    allow = rng.random((rows, width)) < 0.3
    allow[3] = False
    allow[3, 4242] = True  # one allowed id forces it
    mask = torch.as_tensor(workloads.pack_mask(allow).view(np.int32)).cuda()
    T = np.array([1.0, 0.7, 0.0, 1.3, 1.0, 0.6, 1.0, 0.9, 1.0])
    K = np.array([20, 50, 1, 20, 100, 5, 127, 20, 2])
    P = np.array([0.95, 0.8, 1.0, 0.95, 1.0, 0.5, 0.9, 1.0, 0.2])
    lg2 = torch.as_tensor(x).cuda()
    p2 = xsm.params_tensor(T, K, P, rows, "cuda")
    u2 = torch.as_tensor(workloads.uniforms(rng, rows)).cuda()
    print("noalloc call 2: 9 x 65536 masked", flush=True)
    got = xsm.sample_batch_noalloc(lg2, p2, u2, allowed=mask, cand_k=127, stats=True)
    want = xsm.sample_batch(ctx, lg2, p2, u2, allowed=mask, cand_k=127, stats=True)
    torch.cuda.synchronize()
    g, w = _np(got), _np(want)
    _same(g, w)
    assert g["token"][3] == 4242

    # third call: held_row statistics on 5 rows of the heterogeneous batch
    wl5 = workloads.c5_heterogeneous(rows=5)
    lg5 = torch.as_tensor(wl5.logits).cuda()
    p5 = xsm.params_tensor(wl5.temperature, wl5.top_k, wl5.top_p, 5, "cuda")
    u5 = torch.as_tensor(wl5.u).cuda()
    print("noalloc call 3: 5 x 248320 held_row", flush=True)
    got = xsm.sample_batch_noalloc(lg5, p5, u5, n_top=20)
    want = xsm.sample_batch(ctx, lg5, p5, u5, n_top=20)
    torch.cuda.synchronize()
    _same(_np(got), _np(want))
    ctx.close()


def test_noalloc_limits():
    _need_gpu()
    from xwen_amd import _lib, sampler as xsm
    torch.cuda.set_device(0)
    rng = np.random.default_rng(5)
    # more rows than the static workspace holds
    x = torch.as_tensor(rng.normal(0, 1, (_lib.NOALLOC_ROWS + 1, 1024)).astype(np.float32)).cuda()
    p = xsm.params_tensor(1.0, 20, 0.9, x.shape[0], "cuda")
    u = torch.zeros(x.shape[0], dtype=torch.float32, device="cuda")
    _, rc = xsm.sample_batch_noalloc(x, p, u, check=False)
    assert rc == _lib.XS_ERR_CAPACITY
    # a wider vocabulary than it holds
    x = torch.zeros((1, _lib.NOALLOC_VOCAB + 4), dtype=torch.float32, device="cuda")
    p = xsm.params_tensor(1.0, 20, 0.9, 1, "cuda")
    u = torch.zeros(1, dtype=torch.float32, device="cuda")
    _, rc = xsm.sample_batch_noalloc(x, p, u, check=False)
    assert rc == _lib.XS_ERR_CAPACITY
    # top_k past XS_K_MAX: a per-row error, the other rows drawn
    x = torch.as_tensor(rng.normal(0, 2, (2, 4096)).astype(np.float32)).cuda()
    p = xsm.params_tensor(1.0, np.array([200, 20]), 0.9, 2, "cuda")
    u = torch.full((2,), 0.5, dtype=torch.float32, device="cuda")
    out = xsm.sample_batch_noalloc(x, p, u)
    torch.cuda.synchronize()
    st = out.status.cpu().numpy()
    assert st[0] == _lib.ROW_BAD_PARAM and st[1] == _lib.ROW_OK


def test_noalloc_first_call_inside_graph_capture():
    """A fresh process whose first xs_sample_noalloc call is captured into a HIP
    graph (the entry point's one-time set-up then runs under the capture):
    three replays with new uniforms equal xs_sample bit for bit, and eager
    calls leave the device's free memory unchanged (tests/noalloc_capture_child.py)."""
    _need_gpu()
    import os
    import subprocess
    import sys
    child = os.path.join(os.path.dirname(os.path.abspath(__file__)), "noalloc_capture_child.py")
    print("starting the capture child process", flush=True)
    r = subprocess.run([sys.executable, "-u", child], capture_output=True, text=True, timeout=300)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and "noalloc-capture ok" in r.stdout
