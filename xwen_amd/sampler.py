"""Host-side mirror of xwen's sampler interface over the HIP C ABI.

Names, argument meaning and error behaviour follow the reference:

  SamplerOptions / recommended      src/sampler.rs:36-71
  SampleControl (mask, bans, bias,
  pull, force)                      src/sampler.rs:85-121, :433-490
  draft_argmax_probs                src/generate.rs:4059-4087
  Sampler.new / sample /
  sample_masked / sample_controlled src/sampler.rs:123-232
  Sampler.is_eog / eog_ids /
  encodable                         src/sampler.rs:127-128, :245-253
  verify_batch (accept_drafts)      src/generate.rs:4020-4046
  masks_along_drafts                src/generate.rs:2434-2459
  keep_confident                    src/generate.rs:3898-3905
  select_option                     src/batch.rs:1545-1588
  held-row log-probs                src/generate.rs:1871-1933

Differences, all forced by the batched device design:
  * calls are batched: `logits` is [rows, width] on the GPU and every row is an
    independent draw with its own options;
  * the RNG is a seeded stream of host uniforms u = j * 2^-23 (the f32 rand
    0.9's UniformFloat builds from 23 random bits), one per stochastic row and
    none for a greedy row -- the reference's one-draw-per-committed-token
    invariant; the reference's StdRng (ChaCha12) bit stream is not reproduced;
  * row errors are reported per row (SampleError carries every status) instead
    of failing the first one.

Device memory and streams come from PyTorch (torch.cuda); the computation is the
HIP kernels in libxsamp.so.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from . import _lib

ROW_STATUS_NAMES = {
    _lib.ROW_OK: "ok",
    _lib.ROW_NAN: "the logit row holds a NaN: the forward pass produced a corrupt row",
    _lib.ROW_NO_FINITE: "every logit was excluded: there is no token to draw",
    _lib.ROW_MASK_SHORT: "allow-mask covers fewer ids than the vocabulary holds",
    _lib.ROW_FORCE_OOR: "forced token id is outside the vocabulary",
    _lib.ROW_ZERO_WEIGHT: "no candidate carries any probability mass after top-k/top-p filtering",
    _lib.ROW_NARROW: "logit row is narrower than the encodable ids the sampler draws over",
    _lib.ROW_BAD_PARAM: "top_k exceeds the sampler context's k_max (create the context with a "
                        "larger k_max), or a control list holds more entries than the context's "
                        "ctl_max (XS_CTL_MAX unless the context was created with a larger one)",
    _lib.ROW_INTERNAL: "the row's workgroups did not share one XCD (placement check); not sampled",
    _lib.ROW_ID_OOR: "a scored token id is outside the encodable ids",
}


class SampleError(RuntimeError):
    """One or more rows failed; `status` holds every row's XS_ROW_* code."""

    def __init__(self, status):
        self.status = np.asarray(status)
        bad = np.nonzero(self.status)[0]
        first = int(bad[0])
        super().__init__(f"{len(bad)} of {self.status.size} rows failed; row {first}: "
                         f"{ROW_STATUS_NAMES.get(int(self.status[first]), 'unknown')}")


@dataclass
class SamplerOptions:
    """SamplerOptions (sampler.rs:36-71): defaults are the thinking set."""

    temperature: float = 1.0
    top_k: int = 20
    top_p: float = 0.95
    seed: int = 42

    @staticmethod
    def recommended(thinking: bool) -> "SamplerOptions":
        return SamplerOptions(temperature=1.0 if thinking else 0.7, top_k=20,
                              top_p=0.95 if thinking else 0.80, seed=42)

    def is_greedy(self) -> bool:
        # Sampler::new (sampler.rs:133-145)
        return self.temperature <= 0.0 or self.top_k <= 1


@dataclass
class SampleControl:
    """SampleControl (sampler.rs:85-121), applied in the reference's order:
    allowed -> banned -> bias -> pull -> force (apply_control, sampler.rs:433-490).

    `allowed` is a packed u32 allow-mask per row on the GPU ([rows, words], bit
    t%32 of word t/32), or None.  `banned` is a list of ids, `bias` a list of
    (id, delta), `pull` an (id, alpha) pair or None, `force` an id or None; the
    same sparse controls apply to every row of the call."""

    allowed: object = None
    banned: tuple = ()
    bias: tuple = ()
    pull: object = None
    force: object = None

    def is_noop(self) -> bool:
        return (self.allowed is None and not self.banned and not self.bias
                and self.pull is None and self.force is None)

    def has_sparse(self) -> bool:
        return bool(self.banned) or bool(self.bias) or self.pull is not None \
            or self.force is not None


@dataclass
class Controls:
    """Device form of per-row sparse controls: xs_row_control [rows] plus the id
    and delta pools its offsets index."""

    rows: object
    ids: object
    delta: object


def controls_tensor(per_row, device) -> Controls:
    """Pack one SampleControl-like object (or None) per row into the xs_row_control
    array and the shared id / delta pools (device tensors)."""
    torch = _torch()
    n = len(per_row)
    arr = (_lib.RowControl * max(n, 1))()
    ids, delta = [], []
    for r, c in enumerate(per_row):
        if c is None:
            continue
        rc = arr[r]
        rc.ban_off, rc.n_ban = len(ids), len(c.banned)
        ids += [int(i) for i in c.banned]
        delta += [0.0] * len(c.banned)
        rc.bias_off, rc.n_bias = len(ids), len(c.bias)
        ids += [int(i) for i, _ in c.bias]
        delta += [float(d) for _, d in c.bias]
        if c.pull is not None:
            rc.has_pull, rc.pull_id, rc.pull_alpha = 1, int(c.pull[0]), float(c.pull[1])
        if c.force is not None:
            rc.has_force, rc.force_id = 1, int(c.force)
    raw = np.frombuffer(bytes(arr), dtype=np.uint8)[: n * C.sizeof(_lib.RowControl)].copy()
    ids_t = torch.from_numpy(np.asarray(ids + [0], np.uint32).view(np.int32)).to(device)
    delta_t = torch.from_numpy(np.asarray(delta + [0.0], np.float32)).to(device)
    return Controls(rows=torch.from_numpy(raw).to(device), ids=ids_t, delta=delta_t)


def _torch():
    import torch
    return torch


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


class Context:
    """An xs_context: the device workspace for up to max_rows rows of `vocab` ids,
    top_k up to k_max and control lists (bans plus biases of a row) up to ctl_max."""

    def __init__(self, max_rows: int, vocab: int, k_max: int = _lib.K_MAX, device: int = 0,
                 ctl_max: int = _lib.CTL_MAX):
        self.lib = _lib.load()
        torch = _torch()
        self.device = device
        torch.cuda.set_device(device)
        h = C.c_void_p()
        _lib.check(self.lib.xs_create_ex(device, max_rows, vocab, k_max, ctl_max, C.byref(h)),
                   "xs_create_ex")
        self.h = h
        self.max_rows, self.vocab, self.k_max, self.ctl_max = max_rows, vocab, k_max, ctl_max

    def eog_list(self, eog):
        """The end-of-generation ids as an int32 device tensor, uploaded once per
        distinct list (Sampler::new's eog, sampler.rs:130)."""
        key = tuple(int(e) for e in eog)
        cache = self.__dict__.setdefault("_eog", {})
        if key not in cache:
            torch = _torch()
            cache[key] = torch.as_tensor(np.asarray(key, np.int64).astype(np.int32)).to(
                torch.device("cuda", self.device))
        return cache[key]

    def bind_current_stream(self):
        torch = _torch()
        s = torch.cuda.current_stream(self.device).cuda_stream
        _lib.check(self.lib.xs_set_stream(self.h, C.c_void_p(s)), "xs_set_stream")

    def close(self):
        if getattr(self, "h", None):
            self.lib.xs_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def params_tensor(temperature, top_k, top_p, rows: int, device):
    """Pack per-row (temperature f64, top_k i32, top_p f32) as xs_row_params [rows].

    top_k is the reference's usize: values past INT32_MAX saturate (every
    such k is at least the vocabulary, the same whole-row candidate set), so
    no client k wraps into a greedy or a small k."""
    torch = _torch()
    arr = np.zeros(rows, dtype=np.dtype([("t", "<f8"), ("k", "<i4"), ("p", "<f4")]))
    arr["t"] = np.broadcast_to(np.asarray(temperature, np.float64), (rows,))
    k = np.broadcast_to(np.asarray(top_k, dtype=object), (rows,))
    arr["k"] = np.asarray([min(max(int(v), -(1 << 31)), (1 << 31) - 1) for v in k], np.int64)
    arr["p"] = np.broadcast_to(np.asarray(top_p, np.float64), (rows,)).astype(np.float32)
    raw = np.frombuffer(arr.tobytes(), dtype=np.uint8).copy()
    return torch.from_numpy(raw).to(device)


@dataclass
class Draws:
    """Device outputs of one batched draw (torch tensors on the GPU)."""

    token: object
    status: object
    n_cand: object = None
    cand_id: object = None
    cand_w: object = None
    soft_max: object = None
    soft_sum: object = None
    row_max: object = None
    row_lse: object = None
    top_id: object = None
    top_logprob: object = None
    top_logprob64: object = None
    score_logprob: object = None
    class_mass: object = None
    probs: object = None


def sample_batch(ctx: Context, logits, params, uniforms, *, enc: int | None = None,
                 width: int | None = None, allowed=None, allowed_words: int | None = None,
                 cand_k: int = 0, stats: bool = False, n_top: int = 0, out: Draws | None = None,
                 controls: Controls | None = None, order=None, k_max: int = 0,
                 score_ids=None, class_masks=None, probs: bool = False,
                 check: bool = True) -> Draws:
    """One xs_sample call.  logits: float32 [rows, ld] CUDA tensor (ld % 4 == 0);
    params: the uint8 tensor from params_tensor; uniforms: float32 [rows];
    order: an optional host permutation of the rows (see cost_order), the
    order in which the launch starts them; k_max: this call's bound on
    min(top_k, enc), 0 for the context's (127 or less skips the whole-row
    kernels of a context sized for more).  The scoring reads of the held row
    (generate.rs:1871-1899): score_ids, an int32 [rows, n] CUDA tensor of ids
    (f64 log-probs out); class_masks, a [rows, n_class, words] u32 (as int32)
    CUDA tensor of allow-mask-layout class masks (f64 class masses out);
    probs, the whole f64 distribution."""
    a, out, keep = _sample_args(logits, params, uniforms, enc=enc, width=width, allowed=allowed,
                                allowed_words=allowed_words, cand_k=cand_k, stats=stats,
                                n_top=n_top, out=out, controls=controls, order=order, k_max=k_max,
                                score_ids=score_ids, class_masks=class_masks, probs=probs)
    rc = ctx.lib.xs_sample(ctx.h, C.byref(a))
    del keep
    if check:
        _lib.check(rc, "xs_sample")
    return out


def sample_batch_noalloc(logits, params, uniforms, *, stream=None, check: bool = True,
                         **kw) -> Draws:
    """The same draw through xs_sample_noalloc: no context, the library's static
    workspace on the current device (rows <= NOALLOC_ROWS, enc <= NOALLOC_VOCAB),
    on `stream` (default: torch's current stream).  Returns (Draws, rc) when
    check is False."""
    torch = _torch()
    lib = _lib.load()
    a, out, keep = _sample_args(logits, params, uniforms, **kw)
    s = torch.cuda.current_stream(logits.device) if stream is None else stream
    rc = lib.xs_sample_noalloc(C.byref(a), C.c_void_p(s.cuda_stream))
    del keep
    if check:
        _lib.check(rc, "xs_sample_noalloc")
        return out
    return out, rc


def _sample_args(logits, params, uniforms, *, enc: int | None = None, width: int | None = None,
                 allowed=None, allowed_words: int | None = None, cand_k: int = 0,
                 stats: bool = False, n_top: int = 0, out: Draws | None = None,
                 controls: Controls | None = None, order=None, k_max: int = 0,
                 score_ids=None, class_masks=None, probs: bool = False):
    """xs_sample_args for one call, the output tensors, and the host arrays the
    call reads (kept alive by the caller through the call)."""
    torch = _torch()
    rows, ld = logits.shape
    dev = logits.device
    enc = ld if enc is None else enc
    width = ld if width is None else width
    if out is None:
        out = Draws(token=torch.empty(rows, dtype=torch.int32, device=dev),
                    status=torch.empty(rows, dtype=torch.int32, device=dev))
        if cand_k:
            out.n_cand = torch.empty(rows, dtype=torch.int32, device=dev)
            out.cand_id = torch.empty((rows, cand_k), dtype=torch.int32, device=dev)
            out.cand_w = torch.empty((rows, cand_k), dtype=torch.float32, device=dev)
        if stats:
            out.soft_max = torch.empty(rows, dtype=torch.float32, device=dev)
            out.soft_sum = torch.empty(rows, dtype=torch.float32, device=dev)
        if n_top:
            out.row_max = torch.empty(rows, dtype=torch.float32, device=dev)
            out.row_lse = torch.empty(rows, dtype=torch.float64, device=dev)
            out.top_id = torch.empty((rows, n_top), dtype=torch.int32, device=dev)
            out.top_logprob = torch.empty((rows, n_top), dtype=torch.float32, device=dev)
            out.top_logprob64 = torch.empty((rows, n_top), dtype=torch.float64, device=dev)
        if score_ids is not None:
            out.score_logprob = torch.empty(tuple(score_ids.shape), dtype=torch.float64, device=dev)
        if class_masks is not None:
            out.class_mass = torch.empty((rows, class_masks.shape[1]), dtype=torch.float64, device=dev)
        if probs:
            out.probs = torch.empty((rows, enc), dtype=torch.float64, device=dev)
    a = _lib.SampleArgs()
    a.logits = logits.data_ptr()
    a.rows, a.ld, a.width, a.enc = rows, ld, width, enc
    a.k_max = int(k_max)
    a.params = params.data_ptr()
    a.uniforms = uniforms.data_ptr()
    if allowed is not None:
        a.allowed = allowed.data_ptr()
        a.allowed_words = allowed.shape[1] if allowed_words is None else allowed_words
        a.allowed_ld = allowed.shape[1]
    a.token = out.token.data_ptr()
    a.status = out.status.data_ptr()
    if out.cand_id is not None:
        a.cand_id = out.cand_id.data_ptr()
        a.cand_w = out.cand_w.data_ptr()
        a.n_cand = out.n_cand.data_ptr()
        a.cand_ld = out.cand_id.shape[1]
    if out.soft_max is not None:
        a.soft_max = out.soft_max.data_ptr()
        a.soft_sum = out.soft_sum.data_ptr()
    if out.top_id is not None:
        a.row_max = out.row_max.data_ptr()
        a.row_lse = out.row_lse.data_ptr()
        a.n_top = out.top_id.shape[1]
        a.top_id = out.top_id.data_ptr()
        a.top_logprob = out.top_logprob.data_ptr()
        if out.top_logprob64 is not None:
            a.top_logprob64 = out.top_logprob64.data_ptr()
        a.top_ld = out.top_id.shape[1]
    if score_ids is not None:
        a.score_ids = score_ids.data_ptr()
        a.n_score = score_ids.shape[1]
        a.score_ld = score_ids.shape[1]
        a.score_logprob = out.score_logprob.data_ptr()
    if class_masks is not None:
        a.class_masks = class_masks.data_ptr()
        a.n_class = class_masks.shape[1]
        a.class_ld = class_masks.shape[2]
        a.class_mass = out.class_mass.data_ptr()
    if out.probs is not None:
        a.probs = out.probs.data_ptr()
        a.probs_ld = out.probs.shape[1]
    if controls is not None:
        a.controls = controls.rows.data_ptr()
        a.ctl_ids = controls.ids.data_ptr()
        a.ctl_delta = controls.delta.data_ptr()
    keep = None
    if order is not None:
        keep = np.ascontiguousarray(np.asarray(order, np.int32))  # alive through the call
        if keep.shape != (rows,):  # the library reads exactly `rows` entries
            raise ValueError(f"order must list each of the {rows} rows once, got shape {keep.shape}")
        a.row_order = keep.ctypes.data
    return a, out, keep


def cost_order(temperature, top_k, *, controlled=None) -> np.ndarray:
    """A row order for sample_batch that starts the rows with the costliest
    finalization first: stochastic rows by top_k, largest first (above 63 the
    general finalizer runs), then greedy rows; rows with sparse controls
    (`controlled`, a bool per row) before all others.  Stable, so equal rows
    keep their order."""
    t = np.asarray(temperature, np.float64)
    k = np.asarray(top_k, np.int64)
    rows = max(t.size, k.size)
    t = np.broadcast_to(t, (rows,))
    k = np.broadcast_to(k, (rows,))
    cost = np.where((t <= 0.0) | (k <= 1), 0, np.minimum(k, 1 << 20)).astype(np.int64)
    if controlled is not None:
        cost = cost + np.where(np.broadcast_to(np.asarray(controlled, bool), (rows,)), 1 << 21, 0)
    return np.argsort(-cost, kind="stable").astype(np.int32)


@dataclass
class Verdict:
    row_token: object
    row_status: object
    accepted: object
    committed: object
    n_committed: object
    seq_status: object
    eog_ids: object = None


def verify_batch(ctx: Context, logits, seqs: int, span: int, params, uniforms, drafts, *,
                 budget=None, eog=(), enc: int | None = None, allowed=None,
                 controls: Controls | None = None, done_after=None,
                 out: Verdict | None = None, k_max: int = 0) -> Verdict:
    """One xs_verify call over logits [seqs*span, ld]; drafts int32 [seqs, span-1].
    `allowed` / `done_after` per position come from masks_along_drafts; k_max
    as in sample_batch."""
    torch = _torch()
    rows, ld = logits.shape
    assert rows == seqs * span
    dev = logits.device
    enc = ld if enc is None else enc
    if out is None:
        out = Verdict(row_token=torch.empty(rows, dtype=torch.int32, device=dev),
                      row_status=torch.empty(rows, dtype=torch.int32, device=dev),
                      accepted=torch.empty(seqs, dtype=torch.int32, device=dev),
                      committed=torch.empty((seqs, span), dtype=torch.int32, device=dev),
                      n_committed=torch.empty(seqs, dtype=torch.int32, device=dev),
                      seq_status=torch.empty(seqs, dtype=torch.int32, device=dev))
    a = _lib.VerifyArgs()
    a.logits = logits.data_ptr()
    a.seqs, a.span, a.ld, a.width, a.enc = seqs, span, ld, ld, enc
    a.k_max = int(k_max)
    a.params = params.data_ptr()
    a.uniforms = uniforms.data_ptr()
    if allowed is not None:
        a.allowed = allowed.data_ptr()
        a.allowed_words = allowed.shape[1]
        a.allowed_ld = allowed.shape[1]
    a.drafts = drafts.data_ptr() if span > 1 else None
    a.budget = budget.data_ptr() if budget is not None else None
    a.n_eog = len(eog)
    if len(eog):
        # a device list of any length (the reference's eog is a Vec<u32>), kept
        # by the context per distinct list: a call under graph capture reuses
        # the list an earlier eager call uploaded
        out.eog_ids = ctx.eog_list(eog)
        a.eog = out.eog_ids.data_ptr()
    a.row_token = out.row_token.data_ptr()
    a.row_status = out.row_status.data_ptr()
    a.accepted = out.accepted.data_ptr()
    a.committed = out.committed.data_ptr()
    a.n_committed = out.n_committed.data_ptr()
    a.seq_status = out.seq_status.data_ptr()
    if controls is not None:
        a.controls = controls.rows.data_ptr()
        a.ctl_ids = controls.ids.data_ptr()
        a.ctl_delta = controls.delta.data_ptr()
    if done_after is not None:
        a.done_after = done_after.data_ptr()
    _lib.check(ctx.lib.xs_verify(ctx.h, C.byref(a)), "xs_verify")
    return out


def masks_along_drafts(grammar, drafts, words: int):
    """The verify block's per-position allow-masks, computed before the launch
    (generate.rs:2434-2459).  The reference advances its grammar at sample
    time, so row i's mask is the grammar state after the tokens committed at
    rows 0..i-1; row i is reached only if those were drafts[0..i), so a copy
    of the state stepped along the drafts gives every reachable row's mask.

    `grammar` is GrammarState-like (constrain.rs:192-230): mask_words() ->
    LSB-first u32 words or None (dormant: every id allowed), on_committed(id),
    is_done(), and fork() -> an independent copy.  Returns (masks uint32
    [span, words], done_after uint8 [span]): done_after[i] is 1 when
    committing drafts[i] completes the grammar, which ends the walk like an
    EOG.  Rows past a draft the grammar disallows (the sample there cannot
    match it) or past completion are unreachable and get an all-ones mask."""
    g = grammar.fork()
    span = len(drafts) + 1
    masks = np.full((span, words), 0xFFFFFFFF, np.uint32)
    done = np.zeros(span, np.uint8)
    for i in range(span):
        m = g.mask_words()
        if m is not None:
            masks[i] = np.asarray(m, np.uint32)[:words]
        if i == len(drafts):
            break
        t = int(drafts[i])
        if m is not None and not (int(masks[i][t >> 5]) >> (t & 31)) & 1:
            break  # the row's sample cannot equal this draft: the walk ends here
        g.on_committed(t)
        if g.is_done():
            done[i] = 1
            break
    return masks, done


class Sampler:
    """Sampler (sampler.rs:21-29) over the device kernels, batched by row."""

    def __init__(self, opts: SamplerOptions, eog_tokens, encodable: int, *, max_rows: int = 256,
                 device: int = 0):
        self.opts = opts
        self.eog = list(eog_tokens)
        self.encodable_ = encodable
        self.rng = np.random.default_rng(opts.seed)
        # a top_k past the streaming selection (or the whole row) needs the
        # context's whole-row buffers, which only a larger k_max allocates
        k_max = _lib.K_MAX if opts.top_k <= _lib.K_MAX else min(int(opts.top_k), encodable)
        self.ctx = Context(max_rows, encodable, k_max=max(k_max, _lib.K_MAX), device=device)
        self.device = f"cuda:{device}"

    def encodable(self) -> int:
        return self.encodable_

    def is_eog(self, token: int) -> bool:
        return token in self.eog

    def eog_ids(self):
        return list(self.eog)

    def next_uniforms(self, rows: int):
        """One uniform per stochastic row; a greedy sampler draws none."""
        if self.opts.is_greedy():
            return np.zeros(rows, np.float32)
        return (self.rng.integers(0, 1 << 23, rows) * 2.0 ** -23).astype(np.float32)

    def sample_controlled(self, logits, ctl: SampleControl | None = None, uniforms=None):
        """Draw one token per row of `logits` ([rows, width] or [width], f32, CUDA).
        Returns an int64 numpy array of ids; raises SampleError if any row fails."""
        torch = _torch()
        if logits.dim() == 1:
            logits = logits.unsqueeze(0)
        logits = logits.to(torch.float32)
        rows, width = logits.shape
        ld = (width + 3) // 4 * 4
        if ld != width or not logits.is_contiguous() or logits.data_ptr() % 16:
            padded = torch.full((rows, ld), float("-inf"), dtype=torch.float32,
                                device=logits.device)
            padded[:, :width] = logits
            logits = padded
        if uniforms is None:
            uniforms = self.next_uniforms(rows)
        u = torch.as_tensor(np.asarray(uniforms, np.float32), device=logits.device)
        p = params_tensor(self.opts.temperature, self.opts.top_k, self.opts.top_p, rows,
                          logits.device)
        allowed = None if ctl is None else ctl.allowed
        controls = None
        if ctl is not None and ctl.has_sparse():
            controls = controls_tensor([ctl] * rows, logits.device)
        self.ctx.bind_current_stream()
        out = sample_batch(self.ctx, logits, p, u, enc=self.encodable_, width=width,
                           allowed=allowed, controls=controls)
        st = out.status.cpu().numpy()
        if st.any():
            raise SampleError(st)
        return out.token.cpu().numpy().astype(np.int64)

    def sample(self, logits, uniforms=None):
        return self.sample_controlled(logits, None, uniforms)


class HeldRow:
    """The scoring reads of held logit rows (Generator::last_logprobs_for /
    last_probs, generate.rs:1871-1899) on the device: every read is normalized
    by held_row's f64 lse over the encodable ids (raw logits, no temperature),
    and nothing but the asked-for values leaves the device.  logits: float32
    [rows, ld] CUDA tensor (ld % 4 == 0).  Each call is one xs_sample launch
    with greedy rows (no uniform is drawn) and the scoring outputs."""

    def __init__(self, ctx: Context, logits, *, enc: int | None = None):
        self.ctx, self.logits = ctx, logits
        self.rows, ld = logits.shape
        self.enc = ld if enc is None else enc

    def _call(self, **kw) -> Draws:
        torch = _torch()
        dev = self.logits.device
        p = params_tensor(0.0, 1, 1.0, self.rows, dev)
        u = torch.zeros(self.rows, dtype=torch.float32, device=dev)
        self.ctx.bind_current_stream()
        out = sample_batch(self.ctx, self.logits, p, u, enc=self.enc, **kw)
        st = out.status.cpu().numpy()
        if st.any():
            raise SampleError(st)
        return out

    def lse(self) -> np.ndarray:
        return self._call(n_top=1).row_lse.cpu().numpy()

    def last_logprobs_for(self, ids) -> np.ndarray:
        """f64 log-probs [rows, n] of ids [rows, n] (one list for every row
        when 1-D); an id outside [0, enc) raises, as the reference's error."""
        torch = _torch()
        i = np.asarray(ids, np.int32)
        if i.ndim == 1:
            i = np.broadcast_to(i, (self.rows, i.size))
        t = torch.as_tensor(np.ascontiguousarray(i), device=self.logits.device)
        return self._call(score_ids=t).score_logprob.cpu().numpy()

    def last_probs(self):
        """The f64 distribution [rows, enc], left on the device."""
        return self._call(probs=True).probs

    def class_masses(self, class_masks) -> np.ndarray:
        """f64 [rows, n_class]: each class's probability mass, class_masks a
        u32 [rows, n_class, words] (or [n_class, words] for every row) array in
        the allow-mask layout."""
        torch = _torch()
        m = np.asarray(class_masks, np.uint32)
        if m.ndim == 2:
            m = np.broadcast_to(m, (self.rows,) + m.shape)
        t = torch.as_tensor(np.ascontiguousarray(m).view(np.int32), device=self.logits.device)
        return self._call(class_masks=t).class_mass.cpu().numpy()


def escape_mass(inside: float, outside: float) -> float:
    """escape_mass's ratio (batch.rs:1664-1669) from its two class masses: the
    share of the content mass outside the field's options, clamped to [0, 1],
    and 0 when every scrap of mass was formatting."""
    content = inside + outside
    if content <= 0.0:
        return 0.0
    return min(max(outside / content, 0.0), 1.0)


def argmax_probs_device(ctx: Context, logits, *, width: int | None = None):
    """argmax_probs_device (generate.rs:4059-4070) through xs_argmax_probs: per
    row the first maximal id and 1 / sum exp(l - max), left on the device as
    int32 / float32 [rows] tensors.  logits: float32 [rows, ld] CUDA tensor."""
    torch = _torch()
    rows, ld = logits.shape
    width = ld if width is None else width
    ids = torch.empty(rows, dtype=torch.int32, device=logits.device)
    probs = torch.empty(rows, dtype=torch.float32, device=logits.device)
    a = _lib.ArgmaxArgs()
    a.logits = logits.data_ptr()
    a.rows, a.ld, a.width = rows, ld, width
    a.ids = ids.data_ptr()
    a.probs = probs.data_ptr()
    _lib.check(ctx.lib.xs_argmax_probs(ctx.h, C.byref(a)), "xs_argmax_probs")
    return ids, probs


def draft_argmax_probs(ctx: Context, logits, *, width: int | None = None):
    """draft_argmax_probs (generate.rs:4075-4087): argmax_probs_device read back,
    as numpy int64 ids and float32 probabilities."""
    ids, probs = argmax_probs_device(ctx, logits, width=width)
    return ids.cpu().numpy().astype(np.int64), probs.cpu().numpy()


def select_option(scores, sampling: SamplerOptions, u: float = 0.0) -> int:
    """select_option (batch.rs:1545-1588) through the C ABI (host memory): the
    option index drawn from f64 `scores` under `sampling`, with the uniform
    u = j * 2^-52 (ignored when greedy).  Raises SampleError when no option
    carries any mass, as the reference's call fails."""
    lib = _lib.load()
    s = np.ascontiguousarray(np.asarray(scores, np.float64))
    if s.size == 0:
        raise ValueError("select_option needs at least one option")
    idx = C.c_int64(-1)
    st = lib.xs_select_option(s.ctypes.data, s.size, float(sampling.temperature),
                              int(sampling.top_k), float(sampling.top_p), float(u), C.byref(idx))
    if st < 0:
        _lib.check(st, "xs_select_option")
    if st != _lib.ROW_OK:
        raise SampleError([st])
    return int(idx.value)


def keep_confident(ids, probs, p_min: float):
    """keep_confident (generate.rs:3898-3905) through the C ABI (host memory)."""
    lib = _lib.load()
    p = np.ascontiguousarray(np.asarray(probs, np.float32))
    n = lib.xs_keep_confident(p.ctypes.data if p.size else None, p.size, C.c_float(p_min))
    return list(ids[:n])
