"""Writes tests/golden/ngram_map.npz from the reference's own counted n-gram
map (ng_update_range, ng_draft_map, ng_save; run.c:4631-4678) and
speculative driver (generate_tokens_spec, run.c:4882-5025, restated in
tests/spec_oracle.py with the reference's drafters), so the map and the
host driver stay pinned where the reference tree is absent.

    python tests/golden/make_ngram_golden.py        # needs oracle/_ref built

Inputs come from the seeded generators below; the fixture holds the drafts
after each update step, the saved NGC2 file of each key length, and, per
driver case, the cycle log (E, k), the counters and the emitted ids.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
for p in (ROOT, ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

OUT = HERE / "ngram_map.npz"
SEED = 40
KEYS = (2, 4, 16)
N_HIST = 1200
STEP = 7          # ids folded into the map per update step
MAX_D = 8
# driver cases: (seed, n_prompt, n_gen, max_ctx, n_key, max_draft, min_draft, cooldown, use_map)
DRIVER = [
    (1, 300, 400, 4096, 16, 8, 2, 8, True),
    (2, 200, 500, 4096, 4, 8, 2, 8, True),
    (3, 200, 500, 4096, 4, 8, 2, 8, False),
    (4, 120, 300, 4096, 2, 15, 1, 3, True),
    (5, 150, 400, 330, 8, 8, 2, 8, True),      # the context fills before n_gen
]


def history(seed: int, n: int, vocab: int = 96) -> np.ndarray:
    """Ids with repeats: phrases reused, some with one id changed."""
    g = np.random.default_rng(seed)
    phrases = [g.integers(0, vocab, g.integers(3, 20)) for _ in range(12)]
    s = []
    while len(s) < n:
        ph = phrases[int(g.integers(0, len(phrases)))].copy()
        if g.random() < 0.3:
            ph[int(g.integers(0, ph.size))] = g.integers(0, vocab)
        s += ph.tolist() + g.integers(0, vocab, int(g.integers(0, 3))).tolist()
    return np.array(s[:n], np.int32)


def steps(n: int):
    return range(STEP, n + 1, STEP)


def main() -> None:
    from oracle.binding import Reference
    from spec_oracle import ReferenceDriver, repetitive_stream
    R = Reference("avx2")
    out = {}
    for n_key in KEYS:
        hist = history(SEED + n_key, N_HIST)
        R.ng_init(n_key)
        drafts = []
        for b in steps(hist.size):
            R.ng_update_range(hist, max(0, b - STEP), b)
            drafts.append(np.pad(R.ng_draft(hist[:b], MAX_D), (0, MAX_D), constant_values=-1)[:MAX_D])
        out[f"drafts_{n_key}"] = np.stack(drafts).astype(np.int32)
        path = HERE / "_ngram_tmp.ngc"
        R.ng_save(path)
        out[f"file_{n_key}"] = np.frombuffer(path.read_bytes(), np.uint8).copy()
        path.unlink()
    for i, (seed, n_prompt, n_gen, max_ctx, n_key, max_draft, min_draft, cooldown, use_map) in enumerate(DRIVER):
        stream = repetitive_stream(seed, n_prompt, n_gen)
        D = ReferenceDriver(R, n_key, max_draft, min_draft, cooldown, use_map)
        toks, log, st = D.run(stream, n_prompt, n_gen, max_ctx)
        out[f"driver_{i}_out"] = toks
        out[f"driver_{i}_log"] = np.array(log, np.int32).reshape(-1, 2)
        out[f"driver_{i}_stats"] = np.array([st[k] for k in ("cycles", "drafted", "full", "rejected", "kept")],
                                            np.int64)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: " + ", ".join(f"{k} {v.shape}" for k, v in out.items()))


if __name__ == "__main__":
    main()
