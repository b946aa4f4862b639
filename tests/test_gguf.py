"""The GGUF reader of the host library (cwen_gguf_*), no GPU: it accepts
what the reference's load_gguf accepts (run.c:3230-3301) -- v2/v3, KV pairs
of every value type skipped, 1-4 dims, 32-byte aligned data section -- and
rejects, with the same conditions, what it rejects: bad magic, other
versions, truncation, long strings, deep KV nesting, unknown KV types, too
many tensors, zero or oversized dims, the reference's internal type ids,
offsets or extents beyond the file.  Tensor data is returned in place."""
import ctypes as C
import struct

import numpy as np
import pytest

from cwen_amd import synth
from gguf_writer import KV_ARR, KV_BOOL, KV_F32, KV_STR, KV_U32, gguf_bytes, gstr, kv_entry

T_F32, T_Q4_0, T_Q4_1, T_Q8_0, T_Q5_K, T_Q6_K = 0, 2, 3, 8, 13, 14


def sample():
    kv = [kv_entry(b"general.name", KV_STR, gstr(b"synthetic")),
          kv_entry(b"n.u32", KV_U32, struct.pack("<I", 7)),
          kv_entry(b"n.f32", KV_F32, struct.pack("<f", 1.5)),
          kv_entry(b"n.bool", KV_BOOL, b"\1"),
          # an array of arrays of strings
          kv_entry(b"n.nested", KV_ARR, struct.pack("<IQ", KV_ARR, 2) +
                   2 * (struct.pack("<IQ", KV_STR, 2) + gstr(b"ab") + gstr(b"cde")))]
    t = [("w.q4_0", T_Q4_0, (64, 3), synth.q4_gguf(1, 3, 64).tobytes()),
         ("w.q4_1", T_Q4_1, (64, 2), synth.q4_1(1, 2, 64).tobytes()),
         ("w.q8_0", T_Q8_0, (32, 1), synth.q8_0(1, 1, 32).tobytes()),
         ("w.q5_k", T_Q5_K, (256, 2), synth.q5_k(1, 2, 256).tobytes()),
         ("w.q6_k", T_Q6_K, (256, 1), synth.q6_k(1, 1, 256).tobytes()),
         ("v.f32", T_F32, (5,), np.arange(5, dtype=np.float32).tobytes()),
         ("v.f32.3d", T_F32, (2, 3, 1), np.arange(6, dtype=np.float32).tobytes())]
    return t, kv


def open_bytes(tmp_path, raw: bytes, name="m.gguf"):
    from cwen_amd import gpu
    p = tmp_path / name
    p.write_bytes(raw)
    return gpu.GGUF(p)


@pytest.mark.parametrize("version", [2, 3])
def test_reads_tensor_table_and_data(tmp_path, version):
    t, kv = sample()
    g = open_bytes(tmp_path, gguf_bytes(t, kv, version=version))
    assert len(g) == len(t)
    for i, (name, typ, dims, raw) in enumerate(t):
        got = g.tensor(i)
        assert got[:4] == (name, typ, dims[0], dims[1] if len(dims) > 1 else 1)
        assert C.string_at(got[4], len(raw)) == raw          # in place, at its aligned offset
        assert g.find(name) == i
    assert g.find("absent") == -1
    g.close()


def patched(raw: bytes, at: int, fmt: str, value) -> bytes:
    b = bytearray(raw)
    struct.pack_into(fmt, b, at, value)
    return bytes(b)


def info_offset(kv_bytes: bytes, tensors_before=()) -> int:
    """Byte offset of the first tensor info after the header and KV pairs."""
    return 24 + len(kv_bytes) + sum(len(x) for x in tensors_before)


def one_tensor(name=b"w", dims=(64, 3), typ=T_Q4_0, off=0, raw=None):
    raw = synth.q4_gguf(1, 3, 64).tobytes() if raw is None else raw
    info = gstr(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims) + \
        struct.pack("<IQ", typ, off)
    body = b"GGUF" + struct.pack("<IQQ", 3, 1, 0) + info
    pad = (len(body) + 31) // 32 * 32 - len(body)
    return body + b"\0" * pad + raw


REJECT = [
    ("magic", lambda: b"GGUX" + one_tensor()[4:], "not gguf"),
    ("version 1", lambda: patched(one_tensor(), 4, "<I", 1), "gguf version 1"),
    ("version 4", lambda: patched(one_tensor(), 4, "<I", 4), "gguf version 4"),
    ("under 20 bytes", lambda: b"GGUF" + struct.pack("<IQ", 3, 0), "under 20 bytes"),
    ("truncated info", lambda: one_tensor()[:40], "truncated"),
    ("reserved type", lambda: one_tensor(typ=101), "reserved type 101"),
    ("n_dims 5", lambda: one_tensor(dims=(64, 3, 1, 1, 1)), "n_dims > 4"),
    ("zero dim", lambda: one_tensor(dims=(64, 0)), "dim 1 = 0"),
    ("dim over INT_MAX", lambda: one_tensor(dims=(64, 1 << 31)), "dim 1 ="),
    ("offset past the file", lambda: one_tensor(off=1 << 20), "offset out of the file"),
    ("extent past the file", lambda: one_tensor(dims=(64, 4)), "extent beyond the file"),
    ("name of 96 bytes", lambda: one_tensor(name=b"n" * 96), "string too long"),
    ("key of 256 bytes", lambda: gguf_bytes([], [kv_entry(b"k" * 256, KV_U32, b"\0" * 4)]), "string too long"),
    ("kv nesting 65 deep", lambda: gguf_bytes([], [kv_entry(b"deep", KV_ARR, struct.pack("<IQ", KV_ARR, 1) * 65 +
                                                            struct.pack("<IQ", KV_U32, 0))]), "kv nesting too deep"),
    ("kv type 13", lambda: gguf_bytes([], [kv_entry(b"x", 13, b"")]), "kv type 13"),
    ("1025 tensors", lambda: b"GGUF" + struct.pack("<IQQ", 3, 1025, 0) + b"\0" * 64, "too many tensors"),
]


@pytest.mark.parametrize("case,make,why", REJECT, ids=[r[0] for r in REJECT])
def test_rejects_like_the_reference(tmp_path, case, make, why):
    from cwen_amd import gpu
    with pytest.raises(gpu.CwenError) as e:
        open_bytes(tmp_path, make())
    assert e.value.rc == -1
    assert why in str(e.value), str(e.value)


def test_accepts_nesting_of_64(tmp_path):
    raw = gguf_bytes([], [kv_entry(b"deep", KV_ARR, struct.pack("<IQ", KV_ARR, 1) * 64 + struct.pack("<IQ", KV_U32, 0))])
    assert len(open_bytes(tmp_path, raw)) == 0


def test_unsized_types_skip_the_extent_check(tmp_path):
    """Types row_bytes cannot size (e.g. Q5_0, id 6) are listed, not
    extent-checked, as in the reference (they are never read)."""
    g = open_bytes(tmp_path, one_tensor(typ=6, dims=(64, 1000)))
    assert g.tensor(0)[1:4] == (6, 64, 1000)
