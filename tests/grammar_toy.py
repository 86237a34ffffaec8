"""A small GrammarState-like object for tests (the interface of
src/constrain.rs:192-230: mask_words / on_committed / is_done), plus fork().

Dormant (no mask: every id allowed) until OPEN is committed.  Then in state s
(0..n-1) it allows the ids of block s, [base + 64 s, base + 64 s + 48), and
CLOSE; a block id moves it to s + 1, and CLOSE or the last block completes it."""
import copy

import numpy as np


class ToyGrammar:
    def __init__(self, vocab: int, n: int = 5, base: int = 1000, open_id: int = 7,
                 close_id: int = 999, dormant: bool = True):
        self.vocab, self.n, self.base = vocab, n, base
        self.open_id, self.close_id = open_id, close_id
        self.dormant, self.state, self.done = dormant, 0, False
        self.words = (vocab + 31) // 32

    def fork(self):
        return copy.deepcopy(self)

    def allowed(self):
        lo = self.base + 64 * self.state
        return list(range(lo, lo + 48)) + [self.close_id]

    def mask_words(self):
        if self.dormant:
            return None
        w = np.zeros(self.words, np.uint32)
        for t in self.allowed():
            w[t >> 5] |= np.uint32(1 << (t & 31))
        return w

    def on_committed(self, t: int):
        if self.dormant:
            if t == self.open_id:
                self.dormant = False
            return
        if t not in self.allowed():
            raise ValueError(f"token {t} is not allowed in state {self.state}")
        if t == self.close_id:
            self.done = True
        else:
            self.state += 1
            self.done = self.state == self.n

    def is_done(self) -> bool:
        return self.done
