"""The reference's speculative driver restated over a recorded greedy stream
(test infrastructure).

generate_tokens_spec (run.c:4882-5025) with the n-gram drafter, step for
step: the first pick after prefill, the map update after it (4900), the
context and room caps (4904-4911), the map's chained drafts with the history
scan winning when longer (4925-4931), min_draft (4934), the walk (4955-4957),
the full-accept AIMD of E_cap (4968-4976), the history and map update (5000-
5003), the emission order (5006-5009) and the cooldown after three short
walks (5010).  The model is replaced by a recorded stream: stream[p + 1] is
the greedy id after position p, so a verify block keeps draft i while it
equals the stream's id at its position.  The drafts themselves come from the
reference's own ngram_draft and ng_draft_map (run.c:4533-4549, 4639-4654)
through oracle/_ref, on its own map globals.

Two details of the reference are kept as they are: the map persists across
calls (NGM is global, as in the reference's server), and so does the
full-accept streak (fa_streak is function-static, run.c:4968).
"""
from __future__ import annotations

import numpy as np


class ReferenceDriver:
    def __init__(self, R, n_key: int = 16, max_draft: int = 8, min_draft: int = 2, cooldown: int = 8,
                 use_map: bool = True):
        self.R = R
        self.n_key, self.max_draft, self.min_draft, self.cooldown = n_key, max_draft, min_draft, cooldown
        self.use_map = use_map
        if use_map:
            R.ng_init(n_key)
        self.fa_streak = 0

    def _draft(self, hist, cap):
        R = self.R
        if self.use_map:
            d = R.ng_draft(hist, cap)
            esc = R.ngram_draft(hist, self.n_key, cap)
            return esc if len(esc) > len(d) else d
        return R.ngram_draft(hist, self.n_key, cap)

    def run(self, stream, n_prompt: int, n_gen: int, max_ctx: int):
        """(emitted ids, per-cycle [(E, k)], stats dict)."""
        s = [int(t) for t in stream]
        hist = s[:n_prompt]
        pos_n = n_prompt - 1
        out, log = [], []
        cyc = drafted = full = rej = kept = 0
        g = streak = cool = 0
        upd = 0
        if n_gen > 0 and pos_n + 1 < max_ctx:
            hist.append(s[n_prompt])
            out.append(s[n_prompt])
            g = 1
        if self.use_map:
            self.R.ng_update_range(hist, upd, len(hist))
            upd = len(hist)
        cap_hard = self.max_draft
        E_cap = cap_hard
        while g < n_gen:
            if pos_n + 1 >= max_ctx:
                break
            E, d = 0, []
            if cool > 0:
                cool -= 1
            else:
                room = max_ctx - 1 - (pos_n + 1)
                d = list(self._draft(hist, min(E_cap, room)))
                E = len(d)
                if E and E < self.min_draft:
                    E = 0
            blk = [hist[-1]] + d[:E]
            p = pos_n + 1                       # the pending token's position
            k = 0
            while k < E and blk[k + 1] == s[p + 1 + k]:
                k += 1
            ustar = s[p + 1 + k]
            pos_n = p + k
            cyc += 1
            log.append((E, k))
            if E:
                drafted += 1
                kept += k
                if k == E:
                    full += 1
                    self.fa_streak += 1
                    if self.fa_streak >= 4 and E_cap < cap_hard:
                        E_cap += 1
                        self.fa_streak = 0
                else:
                    rej += 1
                    self.fa_streak = 0
                    E_cap = k if k > self.min_draft else self.min_draft
            hist += blk[1:k + 1]
            hist.append(ustar)
            if self.use_map:
                self.R.ng_update_range(hist, upd, len(hist))
                upd = len(hist)
            for i in range(k):
                if g >= n_gen:
                    break
                out.append(blk[i + 1])
                g += 1
            if g >= n_gen:
                break
            out.append(ustar)
            g += 1
            if k == E:
                streak = 0
            else:
                streak += 1
                if streak >= 3:
                    streak = 0
                    cool = self.cooldown
        stats = dict(cycles=cyc, drafted=drafted, full=full, rejected=rej, kept=kept)
        return np.array(out, np.int32), log, stats


def repetitive_stream(seed: int, n_prompt: int, n_gen: int, vocab: int = 64, extra: int = 32) -> np.ndarray:
    """A synthetic greedy stream with the structure n-gram drafting feeds on:
    the prompt holds a few phrases, and the continuation replays phrases of
    what came before, sometimes with an id changed, between short runs of
    fresh ids."""
    g = np.random.default_rng(seed)
    phrases = [g.integers(0, vocab, g.integers(6, 24)).tolist() for _ in range(6)]
    s = []
    while len(s) < n_prompt:
        s += phrases[int(g.integers(0, len(phrases)))] + g.integers(0, vocab, 2).tolist()
    s = s[:n_prompt]
    while len(s) < n_prompt + n_gen + extra:
        r = g.random()
        if r < 0.55:
            a = int(g.integers(0, len(s) - 4))
            seg = s[a:a + int(g.integers(4, 40))]
            if g.random() < 0.4 and seg:
                seg = list(seg)
                seg[int(g.integers(0, len(seg)))] = int(g.integers(0, vocab))
            s += seg
        elif r < 0.8:
            s += phrases[int(g.integers(0, len(phrases)))]
        else:
            s += g.integers(0, vocab, int(g.integers(1, 6))).tolist()
    return np.array(s[:n_prompt + n_gen + extra], np.int32)
