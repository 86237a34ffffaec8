"""Child process for tests/test_zz_no_alloc.py: the first xs_sample_noalloc
call of a fresh process is made inside a HIP graph capture (its one-time
set-up, the static array's device address, then happens during the capture),
the graph is replayed with new uniforms, and every replay is compared bit for
bit with xs_sample on a context.  Then eager calls must leave the device's
free memory unchanged.  Prints one "noalloc-capture ok" line on success;
any mismatch raises (a non-zero exit)."""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def main() -> int:
    import torch

    from tests import workloads
    from xwen_amd import sampler as xsm

    torch.cuda.set_device(0)
    rows = 16
    wl = workloads.c2_batch(rows=rows)
    lg = torch.as_tensor(wl.logits).cuda()
    p = xsm.params_tensor(wl.temperature, wl.top_k, wl.top_p, rows, "cuda")
    u = torch.as_tensor(wl.u).cuda()
    out = xsm.Draws(token=torch.empty(rows, dtype=torch.int32, device="cuda"),
                    status=torch.empty(rows, dtype=torch.int32, device="cuda"),
                    n_cand=torch.empty(rows, dtype=torch.int32, device="cuda"),
                    cand_id=torch.empty((rows, 20), dtype=torch.int32, device="cuda"),
                    cand_w=torch.empty((rows, 20), dtype=torch.float32, device="cuda"))
    torch.cuda.synchronize()

    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    print("capturing the process's first xs_sample_noalloc call", flush=True)
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            xsm.sample_batch_noalloc(lg, p, u, out=out)
    torch.cuda.synchronize()

    ctx = xsm.Context(max_rows=rows, vocab=workloads.V)
    ctx.bind_current_stream()
    rng = np.random.default_rng(4711)
    for rep in range(3):
        uu = workloads.uniforms(rng, rows)
        u.copy_(torch.as_tensor(uu))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = {k: getattr(out, k).cpu().numpy().copy() for k in ("token", "status", "n_cand",
                                                                 "cand_id", "cand_w")}
        want = xsm.sample_batch(ctx, lg, p, u, cand_k=20)
        torch.cuda.synchronize()
        assert (got["status"] == 0).all(), got["status"]
        assert (got["token"] == want.token.cpu().numpy()).all(), rep
        assert (got["n_cand"] == want.n_cand.cpu().numpy()).all(), rep
        assert (got["cand_id"] == want.cand_id.cpu().numpy()).all(), rep
        assert (got["cand_w"].view(np.uint32) == want.cand_w.cpu().numpy().view(np.uint32)).all(), rep
        print(f"replay {rep}: tokens {got['token'][:4].tolist()}... equal to xs_sample", flush=True)

    # eager calls allocate nothing: the device's free memory does not move
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    for _ in range(5):
        xsm.sample_batch_noalloc(lg, p, u, out=out)
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free0 == free1, (free0, free1)
    ctx.close()
    print("noalloc-capture ok", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
