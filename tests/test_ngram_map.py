"""The host library's counted n-gram map (cwen_ngmap_*, libcwen_host.so; no
GPU) against the reference's own map -- ng_update_key_n, ng_update_range,
ng_draft_map, ng_evict_one, ng_save and ng_load (run.c:4552-4723) on its
globals through oracle/_ref -- and, where the reference tree is absent,
against tests/golden/ngram_map.npz written from it.

Checked: the whole table (which keys sit in which slots, with their token
and count) after the same updates, including past a full table where
least-hit entries are evicted; the chained drafts; NGC2 files byte for byte;
loading each other's files; and every rule of ng_load (missing file, short
or foreign header, another n_key or vocabulary, records out of range, a cut
tail, merging counts into live entries).
"""
import struct
import sys
from pathlib import Path

import numpy as np
import pytest

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import make_ngram_golden as ng  # noqa: E402

VOCAB = 248320          # the reference's V, recorded in NGC2 headers


def _map(n_key, cap=0):
    from cwen_amd import gpu
    return gpu.NgMap(n_key, VOCAB, cap)


def _same_table(ours, R):
    k1, t1, c1, u1 = ours.dump()
    k2, t2, c2, u2 = R.ng_dump()
    assert np.array_equal(u1, u2), "in-use slots differ"
    used = u1.astype(bool)
    assert np.array_equal(k1[used], k2[used])
    assert np.array_equal(t1[used], t2[used])
    assert np.array_equal(c1[used], c2[used])
    assert ours.used() == R.ng_used() == int(used.sum())


@pytest.mark.parametrize("n_key", [2, 4, 16])
def test_updates_and_drafts_equal_reference(ref, n_key):
    """A history growing in uneven steps, as the driver feeds it: after each
    step the map's drafts equal the reference's, and at the end the tables
    are identical slot for slot."""
    R = ref
    R.ng_init(n_key)
    M = _map(n_key)
    hist = ng.history(7 + n_key, 3000)
    g = np.random.default_rng(n_key)
    upd = 0
    while upd < hist.size:
        b = min(hist.size, upd + int(g.integers(1, 12)))
        M.update_range(hist, upd, b)
        R.ng_update_range(hist, upd, b)
        upd = b
        for max_d in (1, 8, 15):
            assert np.array_equal(M.draft(hist[:b], max_d), R.ng_draft(hist[:b], max_d)), (b, max_d)
    _same_table(M, R)


def _fill_full(M, hist, cap):
    """Every key once up to half the table, a block of keys hit again (so the
    eviction order has counts to choose by), then fill to just short of the
    capacity."""
    for a, b in ((0, cap // 2), (1000, 5000), (cap // 2, cap - 10)):
        M.update_range(hist, a, b)


class _Both:
    def __init__(self, M, R):
        self.M, self.R = M, R

    def update_range(self, hist, a, b):
        self.M.update_range(hist, a, b)
        self.R.ng_update_range(hist, a, b)


def test_full_table_evicts_like_reference(ref):
    """More distinct keys than slots: every insertion past the capacity
    evicts one least-hit entry (equal counts taken in turn from a rotating
    hand) and closes the hole by backward shifting.  The surviving entries
    and their slots equal the reference's through every eviction up to the
    first one in which no entry shifts back into the freed slot: there the
    reference keeps its victim marked in use and writes the new entry past
    the end of its arrays, so the reference is not run into that eviction
    (our own map, run alone, finds where it falls)."""
    from cwen_amd import gpu
    R = ref
    n_key, cap, max_evictions = 2, 1 << 18, 1500
    hist = np.random.default_rng(3).integers(0, VOCAB, cap + 3000).astype(np.int32)
    # where the first eviction without a shift falls, on our own map
    probe = _map(n_key)
    _fill_full(probe, hist, cap)
    stop = cap - 10
    while stop < hist.size and probe.evictions()[1] == 0 and probe.evictions()[0] < max_evictions:
        probe.update_range(hist, stop, stop + 1)
        stop += 1
    if probe.evictions()[1]:
        stop -= 1                      # the update whose eviction shifts nothing
    # both maps through every update before it
    R.ng_init(n_key)
    M = _map(n_key)
    both = _Both(M, R)
    _fill_full(both, hist, cap)
    both.update_range(hist, cap - 10, stop)
    evicted = M.evictions()
    assert evicted[0] >= 1000 and evicted[1] == 0
    assert M.used() == cap
    _same_table(M, R)
    g = np.random.default_rng(4)
    for _ in range(50):
        e = int(g.integers(2, stop))
        assert np.array_equal(M.draft(hist[:e], 8), R.ng_draft(hist[:e], 8))


def test_counts_saturate_like_reference(ref):
    R = ref
    R.ng_init(3)
    M = _map(3)
    key = np.array([5, 6, 7], np.int32)
    for hits, tok in ((2**31 - 10, 1), (5, 2), (100, 3), (1, 4)):
        M.update(key, tok, hits)
        R.ng_update(key, tok, hits)
    _same_table(M, R)
    _, tok, cnt, used = M.dump()
    assert cnt[used.astype(bool)][0] == 2**31 - 1 and tok[used.astype(bool)][0] == 4


def test_save_is_reference_format(ref, tmp_path):
    """The same updates give byte-identical NGC2 files, and each side loads
    the other's file into an identical table."""
    R = ref
    hist = ng.history(11, 2500)
    R.ng_init(4)
    M = _map(4)
    M.update_range(hist, 0, hist.size)
    R.ng_update_range(hist, 0, hist.size)
    M.save(tmp_path / "ours.ngc")
    R.ng_save(tmp_path / "ref.ngc")
    a, b = (tmp_path / "ours.ngc").read_bytes(), (tmp_path / "ref.ngc").read_bytes()
    assert a == b
    assert struct.unpack("<4I", a[:16]) == (0x3243474E, 4, VOCAB, M.used())
    assert not (tmp_path / "ours.ngc.tmp").exists()
    # cross loads into fresh maps
    R.ng_init(4)
    R.ng_load(tmp_path / "ours.ngc")
    M2 = _map(4)
    assert M2.load(tmp_path / "ref.ngc") == M.used()
    _same_table(M2, R)
    _same_table(M, R)


def _records(path, n_key):
    raw = Path(path).read_bytes()
    return raw[:16], np.frombuffer(raw[16:], "<i4").reshape(-1, n_key + 2)


def test_load_rules_equal_reference(ref, tmp_path):
    R = ref
    n_key = 4
    hist = ng.history(12, 800)
    R.ng_init(n_key)
    R.ng_update_range(hist, 0, hist.size)
    R.ng_save(tmp_path / "base.ngc")
    head, rec = _records(tmp_path / "base.ngc", n_key)
    rec = rec.copy()
    rec[3, n_key] = -1            # token out of range
    rec[5, n_key] = VOCAB         # token = vocab
    rec[7, n_key + 1] = 0         # count below 1
    cases = {
        "missing": None,
        "short header": head[:10],
        "foreign magic": b"XXXX" + head[4:] + rec.tobytes(),
        "other n_key": struct.pack("<4I", 0x3243474E, 5, VOCAB, len(rec)) + rec.tobytes(),
        "other vocab": struct.pack("<4I", 0x3243474E, n_key, 1000, len(rec)) + rec.tobytes(),
        "bad records": head + rec.tobytes(),
        "cut tail": head + rec.tobytes()[:-7],
        "count above records": struct.pack("<4I", 0x3243474E, n_key, VOCAB, len(rec) + 50) + rec.tobytes(),
    }
    live = ng.history(13, 300)
    for name, raw in cases.items():
        p = tmp_path / f"{name.replace(' ', '_')}.ngc"
        if raw is not None:
            p.write_bytes(raw)
        # both maps hold live entries first, so loaded counts merge into them
        R.ng_init(n_key)
        R.ng_update_range(live, 0, live.size)
        R.ng_update_range(hist, 0, 200)
        M = _map(n_key)
        M.update_range(live, 0, live.size)
        M.update_range(hist, 0, 200)
        R.ng_load(p)
        M.load(p)
        _same_table(M, R)


def test_golden_drafts_and_file(tmp_path):
    """The pin without the reference tree: drafts and the NGC2 file the
    reference produced for the fixture's history."""
    fx = np.load(ng.OUT)
    for n_key in ng.KEYS:
        hist = ng.history(ng.SEED + n_key, ng.N_HIST)
        M = _map(n_key)
        got = []
        for b in ng.steps(hist.size):
            M.update_range(hist, max(0, b - ng.STEP), b)
            got.append(np.pad(M.draft(hist[:b], ng.MAX_D), (0, ng.MAX_D), constant_values=-1)[:ng.MAX_D])
        assert np.array_equal(np.stack(got), fx[f"drafts_{n_key}"])
        M.save(tmp_path / "m.ngc")
        assert np.array_equal(np.frombuffer((tmp_path / "m.ngc").read_bytes(), np.uint8), fx[f"file_{n_key}"])


def test_create_rejects_bad_arguments():
    from cwen_amd import gpu
    for n_key, cap in ((0, 0), (257, 0), (4, 3), (4, 1)):
        with pytest.raises(gpu.CwenError):
            gpu.NgMap(n_key, VOCAB, cap)


def test_small_table_keeps_probe_chains():
    """A table of 8 slots under many more keys: after every insertion the new
    key is stored, each stored key is still found from its home slot (the
    backward shift leaves no hole inside a chain), and the table stays full.
    Evictions where no entry shifts into the freed slot occur here too, and
    free the victim's own slot."""
    M = _map(1, cap=8)
    g = np.random.default_rng(9)
    seq = g.integers(0, 40, 400).astype(np.int32)
    for i in range(1, seq.size):
        M.update_range(seq, i, i + 1)
        assert M.draft(seq[:i], 1).tolist() == [seq[i]]
        keys, tok, cnt, used = M.dump()
        for s in np.flatnonzero(used):
            assert M.draft(keys[s], 1).tolist() == [tok[s]]
    assert M.used() == 8
    evicted, in_place = M.evictions()
    assert evicted > 100 and in_place > 0
