"""The host library's n-gram drafter (cwen_ngram_draft, libcwen_host.so; no
GPU needed) against the oracle's orc_ngram_draft and, where the reference
tree was built, the reference's own ngram_draft (run.c:4533-4549), on
randomized histories with repeats: the drafts must be identical, id for id.
Speculative decode == serial decode cannot see a drafter bug (a wrong draft
only costs a rejected cycle), so the drafter is pinned here on its own."""
import ctypes as C

import numpy as np
import pytest


def _host_draft(hist, n_key, max_d):
    from cwen_amd import gpu
    h = np.ascontiguousarray(hist, dtype=np.int32)
    out = np.zeros(max(max_d, 1), dtype=np.int32)
    n = gpu.host_lib().cwen_ngram_draft(h.ctypes.data, h.size, out.ctypes.data, n_key, max_d)
    assert 0 <= n <= max(max_d, 0)
    return out[:n]


def _histories(seed, count):
    g = np.random.default_rng(seed)
    for _ in range(count):
        base = g.integers(0, 50, g.integers(20, 80))
        yield np.concatenate([base, base[: g.integers(5, len(base))], g.integers(0, 50, 3),
                              base[:20]]).astype(np.int32)
        # short alphabets give many earlier matches of the key
        yield g.integers(0, 3, g.integers(1, 60)).astype(np.int32)


def test_host_drafter_equals_oracle(oracle):
    for hist in _histories(12, 40):
        for n_key in (1, 2, 4, 16):
            for max_d in (0, 1, 7, 15):
                got = _host_draft(hist, n_key, max_d)
                want = oracle.ngram_draft(hist, n_key, max_d) if max_d > 0 else np.zeros(0, np.int32)
                assert np.array_equal(got, want), (hist.tolist(), n_key, max_d)


def test_host_drafter_equals_reference(ref):
    for hist in _histories(13, 40):
        for n_key in (1, 2, 4, 16):
            for max_d in (1, 7, 15):
                assert np.array_equal(_host_draft(hist, n_key, max_d), ref.ngram_draft(hist, n_key, max_d))


def test_host_drafter_edge_cases(oracle):
    # history not longer than the key, and no earlier match
    assert _host_draft(np.arange(4, dtype=np.int32), 4, 8).size == 0
    assert _host_draft(np.arange(40, dtype=np.int32), 2, 8).size == 0
    # the longest continuation wins over a more recent, shorter one
    h = np.array([1, 2, 9, 9, 9, 1, 2, 7, 1, 2], np.int32)
    assert np.array_equal(_host_draft(h, 2, 5), oracle.ngram_draft(h, 2, 5))
