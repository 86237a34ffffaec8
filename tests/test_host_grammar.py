"""masks_along_drafts (the verify-path masks, generate.rs:2434-2459) against a
live sequential walk that advances the grammar at sample time, on the CPU."""
import numpy as np

from tests.grammar_toy import ToyGrammar
from xwen_amd import sampler as xsm

V = 4096


def _random_drafts(rng, g, depth):
    """Drafts that mostly follow the grammar, with the opener, closers and
    illegal ids mixed in."""
    live, out = g.fork(), []
    for _ in range(depth):
        r = rng.random()
        if live.dormant:
            t = live.open_id if r < 0.5 else int(rng.integers(0, V))
        elif r < 0.75:
            t = int(rng.choice(live.allowed()[:-1]))
        elif r < 0.85:
            t = live.close_id
        else:
            t = int(rng.integers(0, V))
        out.append(t)
        try:
            live.on_committed(t)
        except ValueError:
            pass
        if live.is_done():
            live = g.fork()
    return out


def test_masks_along_drafts_match_a_live_walk():
    rng = np.random.default_rng(21)
    for trial in range(300):
        g = ToyGrammar(V, n=int(rng.integers(1, 6)), dormant=bool(rng.random() < 0.5))
        drafts = _random_drafts(rng, g, int(rng.integers(0, 16)))
        masks, done = xsm.masks_along_drafts(g, drafts, g.words)
        assert masks.shape == (len(drafts) + 1, g.words)
        live = g.fork()
        for i in range(len(drafts) + 1):
            m = live.mask_words()
            want = np.full(g.words, 0xFFFFFFFF, np.uint32) if m is None else m
            assert (masks[i] == want).all(), (trial, i)
            if i == len(drafts):
                break
            t = drafts[i]
            ok = (int(want[t >> 5]) >> (t & 31)) & 1
            # sample == draft whenever the draft is allowed (the walk's best case)
            if not ok:
                assert done[i:].sum() == 0
                break
            live.on_committed(t)
            assert done[i] == int(live.is_done()), (trial, i)
            if live.is_done():
                assert done[i + 1:].sum() == 0
                break
