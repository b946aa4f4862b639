"""The host library's speculative driver (the loop of cwen_generate_spec,
run through cwen_spec_replay against recorded greedy streams; no GPU)
against the reference's generate_tokens_spec (run.c:4882-5025) as restated
in tests/spec_oracle.py with the reference's own drafters through
oracle/_ref, and against tests/golden/ngram_map.npz written from it.

Equal here means the same drafts proposed (E per cycle), the same walk (k per
cycle), the same counters and the same emitted ids: the cycle count, not
only the tokens, follows the reference.  Covered: with and without the
counted map, key lengths 2..16, min_draft 1, a short cooldown, max_draft 15,
the context filling before n_gen, and the map carried across requests as
the reference's server carries it.
"""
import sys
from pathlib import Path

import numpy as np
import pytest

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import make_ngram_golden as ng  # noqa: E402
from spec_oracle import ReferenceDriver, repetitive_stream  # noqa: E402

STAT_KEYS = ("cycles", "drafted", "full", "rejected", "kept")


def _ours(stream, n_prompt, n_gen, max_ctx, n_key, max_draft, min_draft, cooldown, ngmap, fa_streak=None):
    from cwen_amd import gpu
    log = np.full(2 * 4096, -1, np.int32)
    cfg = gpu.spec_cfg(n_key, max_draft, min_draft, cooldown, 0, 0, ngmap, log, fa_streak=fa_streak)
    out, st = gpu.spec_replay(stream, n_prompt, n_gen, max_ctx, cfg)
    n = st.cycles
    return out, [tuple(x) for x in log[:2 * n].reshape(-1, 2).tolist()], {k: getattr(st, k) for k in STAT_KEYS}


def _map(n_key, use):
    from cwen_amd import gpu
    return gpu.NgMap(n_key, 248320) if use else None


@pytest.mark.parametrize("case", range(len(ng.DRIVER)))
def test_driver_equals_reference(ref, case):
    seed, n_prompt, n_gen, max_ctx, n_key, max_draft, min_draft, cooldown, use_map = ng.DRIVER[case]
    stream = repetitive_stream(seed, n_prompt, n_gen)
    D = ReferenceDriver(ref, n_key, max_draft, min_draft, cooldown, use_map)
    want_out, want_log, want_st = D.run(stream, n_prompt, n_gen, max_ctx)
    got_out, got_log, got_st = _ours(stream, n_prompt, n_gen, max_ctx, n_key, max_draft, min_draft, cooldown,
                                     _map(n_key, use_map))
    assert got_log == want_log
    assert got_st == want_st
    assert np.array_equal(got_out, want_out)
    # the drafts mattered: some were kept, some cut short
    assert want_st["kept"] > 0 and (use_map is False or want_st["drafted"] > 10)


@pytest.mark.parametrize("case", range(len(ng.DRIVER)))
def test_driver_equals_golden(case):
    seed, n_prompt, n_gen, max_ctx, n_key, max_draft, min_draft, cooldown, use_map = ng.DRIVER[case]
    fx = np.load(ng.OUT)
    stream = repetitive_stream(seed, n_prompt, n_gen)
    got_out, got_log, got_st = _ours(stream, n_prompt, n_gen, max_ctx, n_key, max_draft, min_draft, cooldown,
                                     _map(n_key, use_map))
    assert np.array_equal(np.array(got_log, np.int32).reshape(-1, 2), fx[f"driver_{case}_log"])
    assert [got_st[k] for k in STAT_KEYS] == fx[f"driver_{case}_stats"].tolist()
    assert np.array_equal(got_out, fx[f"driver_{case}_out"])


def test_output_is_the_stream():
    """Whatever the drafts, the emitted ids are the stream's continuation
    (greedy-lossless), also when the context fills first.  At the cap the
    speculative loop ends with the last slot filled and still emits that
    cycle's bonus, the greedy id after it: one id more than the serial loop,
    which emits only while a slot is left (run.c:4904-4911 vs 5031)."""
    for seed in range(6):
        stream = repetitive_stream(100 + seed, 80, 200)
        for max_ctx in (4096, 150):
            out, _, st = _ours(stream, 80, 200, max_ctx, 4, 8, 2, 8, _map(4, seed % 2 == 0))
            n = min(200, max_ctx - 80 + 1)
            assert np.array_equal(out, stream[80:80 + n])


def test_map_across_requests_equals_reference(ref):
    """One map serving three requests in turn, as the reference's server keeps
    NGM across frames, and the full-accept streak carried from request to
    request, as the reference's function-static one is (run.c:4967): each
    request's cycles equal the reference's."""
    from cwen_amd import gpu
    n_key = 4
    D = ReferenceDriver(ref, n_key)
    M = gpu.NgMap(n_key, 248320)
    carry = np.zeros(1, np.int32)
    carried = []
    for r in range(3):
        # one seed: the requests share phrases, so the map's earlier entries matter
        n_prompt = 150 + 20 * r
        stream = repetitive_stream(30, n_prompt, 250)
        want_out, want_log, want_st = D.run(stream, n_prompt, 250, 4096)
        got_out, got_log, got_st = _ours(stream, n_prompt, 250, 4096, n_key, 8, 2, 8, M, carry)
        assert got_log == want_log and got_st == want_st
        assert np.array_equal(got_out, want_out)
        assert int(carry[0]) == D.fa_streak
        carried.append(int(carry[0]))
    assert M.used() == ref.ng_used()
    assert any(carried), "no request ended inside a full-accept streak: the carry was not exercised"


def test_carried_streak_equals_reference(ref):
    """A request started from a carried full-accept streak (0, 3 or 7) ends
    with the same streak as the restatement started the same way, with the
    same cycles.  Every request starts with E_cap at its cap, and the first
    short walk resets the streak, so the streak a request starts from changes
    none of its drafts: the three logs are equal."""
    from cwen_amd import gpu  # noqa: F401
    stream = repetitive_stream(7, 120, 200)
    logs = []
    for start in (0, 3, 7):
        D = ReferenceDriver(ref, 4, use_map=False)
        D.fa_streak = start
        want_out, want_log, want_st = D.run(stream, 120, 200, 4096)
        carry = np.array([start], np.int32)
        got_out, got_log, got_st = _ours(stream, 120, 200, 4096, 4, 8, 2, 8, None, carry)
        assert got_log == want_log and got_st == want_st
        assert np.array_equal(got_out, want_out)
        assert int(carry[0]) == D.fa_streak
        logs.append(got_log)
    assert logs[0] == logs[1] == logs[2]


def test_replay_rejects_a_stream_too_short():
    from cwen_amd import gpu
    stream = np.arange(50, dtype=np.int32)
    with pytest.raises(gpu.CwenError):
        gpu.spec_replay(stream, 40, 30, 4096, gpu.spec_cfg(4))
