"""The request-frame parser of the host library's server (cwen_read_frame),
no GPU: the reference's server_read_frame rules (run.c:4177-4232) on frames
written to a pipe -- valid frames, counts outside [1, max_ctx] rejected with
their payload drained, out-of-range token ids rejected, and the end of the
stream at the 0xffffffff sentinel or inside a frame.  After every rejected
frame the next one still parses: the stream stays aligned."""
import os
import struct

import numpy as np
import pytest

CTX, VOCAB = 64, 1000
OK, REJECTED, END = 1, 0, 2


def frame(prompt, n_gen, n_prompt=None) -> bytes:
    n_prompt = len(prompt) if n_prompt is None else n_prompt
    return struct.pack("<II", n_prompt, n_gen) + np.asarray(prompt, "<i4").tobytes()


def frames_from(raw: bytes):
    from cwen_amd import gpu
    r, w = os.pipe()
    os.write(w, raw)
    os.close(w)
    got = []
    try:
        while True:
            k, toks, ng = gpu.read_frame(r, CTX, VOCAB)
            got.append((k, None if toks is None else toks.tolist(), ng))
            if k == END:
                return got
    finally:
        os.close(r)


GOOD = frame([5, 6, 7], 4)
CASES = [
    ("valid", GOOD, [(OK, [5, 6, 7], 4)]),
    ("n_prompt 0", frame([], 3), [(REJECTED, None, 0)]),
    ("n_gen 0", frame([1, 2], 0), [(REJECTED, None, 0)]),
    ("n_prompt over the context", frame(list(range(CTX + 1)), 2), [(REJECTED, None, 0)]),
    ("n_gen over the context", frame([1], CTX + 1), [(REJECTED, None, 0)]),
    ("n_gen at the context", frame([1] * CTX, CTX), [(OK, [1] * CTX, CTX)]),
    ("negative token", frame([3, -1], 2), [(REJECTED, None, 0)]),
    ("token = vocab", frame([VOCAB], 2), [(REJECTED, None, 0)]),
]


@pytest.mark.parametrize("case,raw,want", CASES, ids=[c[0] for c in CASES])
def test_frame_then_a_good_one(case, raw, want):
    assert frames_from(raw + GOOD) == want + [(OK, [5, 6, 7], 4), (END, None, 0)]


ENDS = [
    ("sentinel in n_prompt", struct.pack("<II", 0xFFFFFFFF, 1) + GOOD),
    ("sentinel in n_gen", struct.pack("<II", 1, 0xFFFFFFFF) + GOOD),
    ("cut in the header", GOOD[:6]),
    ("cut in the payload", GOOD[:-1]),
]


@pytest.mark.parametrize("case,raw", ENDS, ids=[c[0] for c in ENDS])
def test_end_of_stream(case, raw):
    assert frames_from(raw) == [(END, None, 0)]


def test_drain_cut_short_ends_the_stream():
    assert frames_from(frame([1, 2], 0)[:-4]) == [(REJECTED, None, 0), (END, None, 0)]


def test_empty_stream_and_bad_arguments():
    from cwen_amd import gpu
    assert frames_from(b"") == [(END, None, 0)]
    with pytest.raises(gpu.CwenError):
        gpu.read_frame(0, 0, VOCAB)
    assert gpu.host_lib().cwen_serve(None, None, 0, 1, None, None) == -1  # CWEN_EINVAL
