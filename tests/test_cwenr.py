"""The CWENR sidecar reader of the host library (cwen_gguf_apply_cwenr), no
GPU: it binds what the reference's load_cwenr binds (run.c:3486-3643) -- v4
interleaved pairs and split solos, v3 splits, v2 packed blocks split on the
host -- and drops, on the same conditions, what it drops: a bad magic or
header, a stamped sidecar whose source GGUF changed size, and (one at a
time) entries with an unknown name, a non-Q4_0 tensor, another shape, or
offsets beyond the file.  Sidecars are written by tests/gguf_writer.py."""
import ctypes as C
import struct

import numpy as np
import pytest

from cwen_amd import synth
from gguf_writer import cwenr_bytes, cwenr_entry, cwenr_from_gguf, gguf_bytes

T_Q4_0, T_Q8_0, T_RS, T_RSI = 2, 8, 101, 102


def model_file(tmp_path):
    t = [("blk.0.ffn_gate.weight", T_Q4_0, (64, 3), synth.q4_gguf(1, 3, 64).tobytes()),
         ("blk.0.ffn_up.weight", T_Q4_0, (64, 3), synth.q4_gguf(2, 3, 64).tobytes()),
         ("blk.0.ffn_down.weight", T_Q4_0, (96, 2), synth.q4_gguf(3, 2, 96).tobytes()),
         ("blk.0.attn_k.weight", T_Q4_0, (32, 4), synth.q4_gguf(4, 4, 32).tobytes()),
         ("blk.0.attn_v.weight", T_Q4_0, (32, 4), synth.q4_gguf(5, 4, 32).tobytes()),
         ("blk.0.ssm_out.weight", T_Q8_0, (32, 2), synth.q8_0(6, 2, 32).tobytes())]
    p = tmp_path / "m.gguf"
    p.write_bytes(gguf_bytes(t))
    return p, t


def pages(p) -> int:
    return (p.stat().st_size + 4095) // 4096


def blocks(raw: bytes) -> np.ndarray:
    return np.frombuffer(raw, np.uint8).reshape(-1, 18)


def view(g, i, nblk):
    """(type, qs bytes, f16 scale bytes, side) of tensor i as now bound."""
    _, typ, _, _, data = g.tensor(i)
    sc, side = g.scales(i)
    w = {T_RS: 16, T_RSI: 32}[typ]
    return typ, C.string_at(data, nblk * w), C.string_at(sc, nblk * w // 8), side


@pytest.mark.parametrize("version", [4, 3, 2])
def test_binds_every_q4_tensor(tmp_path, version):
    from cwen_amd import gpu
    p, t = model_file(tmp_path)
    s = tmp_path / "m.cwenr"
    s.write_bytes(cwenr_from_gguf(t, version, src_pages=pages(p)))
    g = gpu.GGUF(p)
    assert g.apply_cwenr(s, p) == 5
    for name, typ, dims, raw in t:
        i = g.find(name)
        if typ != T_Q4_0:
            assert g.tensor(i)[1] == typ and g.scales(i) == (None, 0)
            continue
        bl = blocks(raw)
        pair = version == 4 and any(k in name for k in ("gate", "up", "attn_k", "attn_v"))
        got_t, qs, sc, side = view(g, i, len(bl))
        if pair:
            assert got_t == T_RSI and side == int("up" in name or "attn_v" in name)
            assert np.array_equal(np.frombuffer(qs, np.uint8).reshape(-1, 32)[:, 16 * side:16 * side + 16], bl[:, 2:])
            assert np.array_equal(np.frombuffer(sc, np.uint8).reshape(-1, 4)[:, 2 * side:2 * side + 2], bl[:, :2])
        else:
            assert got_t == T_RS and side == 0
            assert qs == bl[:, 2:].tobytes() and sc == bl[:, :2].tobytes()
    g.close()


def test_v2_split_rounds_to_nearest_even(tmp_path):
    """v2 stores f32 scales; the host split rounds them to f16 like
    _mm_cvtps_ph (run.c:443-470), here checked against numpy's float16
    conversion, ties and subnormals included."""
    from cwen_amd import gpu
    p, t = model_file(tmp_path)
    bl = blocks(t[2][3])
    d = np.array([1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 3e-6, -2.0 ** -25, 65519.0, -70000.0],
                 np.float32)
    packed = np.concatenate([bl[:, 2:], d.view(np.uint8).reshape(-1, 4)], axis=1).tobytes()
    s = tmp_path / "v2.cwenr"
    s.write_bytes(cwenr_bytes([cwenr_entry("blk.0.ffn_down.weight", 96, 2, 0, len(packed))], packed, 2))
    g = gpu.GGUF(p)
    assert g.apply_cwenr(s) == 1
    _, qs, sc, _ = view(g, 2, len(bl))
    assert qs == bl[:, 2:].tobytes()
    with np.errstate(over="ignore"):
        want = d.astype(np.float16).view(np.uint16)
    assert np.array_equal(np.frombuffer(sc, np.uint16), want)
    g.close()


def test_f32_to_f16_matches_numpy():
    from cwen_amd import gpu
    f = gpu.host_lib().cwen_f32_to_f16
    rng = np.random.default_rng(7)
    bits = np.concatenate([rng.integers(0, 2 ** 32, 20000, dtype=np.uint64).astype(np.uint32),
                           np.array([0x33000000, 0x33000001, 0x337fffff, 0x38800000, 0x387fc000, 0x387fe000,
                                     0x477fe000, 0x477fefff, 0x477ff000, 0x7f800000, 0xff800000, 0x7fc00000,
                                     0x80000000, 0x00000001, 0x3f800fff, 0x3f801000, 0x3f803000], np.uint32)])
    x = bits.view(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    got = np.array([f(float(v)) for v in x], np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all((got[nan] & 0x7e00) == 0x7e00) and np.array_equal(got[nan] >> 15, bits[nan] >> 31)


def test_stamp_gate(tmp_path):
    """A stamped sidecar binds only while its source GGUF keeps the size it
    was stamped with; an unstamped one is trusted."""
    from cwen_amd import gpu
    p, t = model_file(tmp_path)
    s = tmp_path / "m.cwenr"
    for stamp, src, ok in [(pages(p), p, True), (pages(p) + 1, p, False), (pages(p), None, False),
                           (None, None, True), (0, None, True)]:
        s.write_bytes(cwenr_from_gguf(t, 4, src_pages=stamp))
        g = gpu.GGUF(p)
        if ok:
            assert g.apply_cwenr(s, src) == 5
        else:
            with pytest.raises(gpu.CwenError) as e:
                g.apply_cwenr(s, src)
            assert "stale sidecar" in str(e.value) and g.tensor(0)[1] == T_Q4_0
        g.close()


def one(name="blk.0.ffn_down.weight", ne0=96, ne1=2, a=0, b=None, flags=0, version=3):
    """A sidecar with one split entry over a payload of the right size."""
    nblk = ne0 // 32 * ne1
    payload = b"\1" * (nblk * 16) + b"\0" * (-nblk * 16 % 64) + b"\2" * (nblk * 2)
    b = (nblk * 16 + 63) // 64 * 64 if b is None else b
    return cwenr_bytes([cwenr_entry(name, ne0, ne1, a, b, flags)], payload, version)


BAD_FILE = [
    ("magic", lambda: b"CWENR002" + one()[8:], "bad magic"),
    ("under 32 bytes", lambda: one()[:31], "too small"),
    ("version 5", lambda: one(version=5), "bad header ver=5"),
    ("version 1", lambda: one(version=1), "bad header ver=1"),
    ("1025 entries", lambda: b"CWENR001" + struct.pack("<IIQ", 3, 1025, 64) + b"\0" * 8 + b"\0" * 200,
     "bad header ver=3 n=1025"),
    ("directory beyond the file", lambda: (b"CWENR001" + struct.pack("<IIQ", 3, 2, 64) + b"\0" * 8 +
                                           cwenr_entry("x", 32, 1, 0, 0))[:200], "bad header"),
    ("data base beyond the file", lambda: cwenr_bytes([cwenr_entry("x", 32, 1, 0, 0)], b"", 3, data_base=4096)[:192],
     "bad header"),
]


@pytest.mark.parametrize("case,make,why", BAD_FILE, ids=[c[0] for c in BAD_FILE])
def test_rejects_bad_sidecar(tmp_path, case, make, why):
    from cwen_amd import gpu
    p, _ = model_file(tmp_path)
    s = tmp_path / "bad.cwenr"
    s.write_bytes(make())
    g = gpu.GGUF(p)
    with pytest.raises(gpu.CwenError) as e:
        g.apply_cwenr(s)
    assert e.value.rc == -1 and why in str(e.value), str(e.value)
    assert g.tensor(2)[1] == T_Q4_0
    g.close()


SKIP = [
    ("unknown name", dict(name="blk.9.ffn_down.weight")),
    ("not Q4_0 in the GGUF", dict(name="blk.0.ssm_out.weight", ne0=32, ne1=2)),
    ("other shape", dict(ne1=3)),
    ("qs beyond the file", dict(a=1 << 20)),
    ("scales beyond the file", dict(b=1 << 40)),
    ("interleaved extent beyond the file", dict(flags=1)),
]


@pytest.mark.parametrize("case,kw", SKIP, ids=[c[0] for c in SKIP])
def test_skips_entries_that_cannot_apply(tmp_path, case, kw):
    """Alone, such an entry leaves nothing to bind (0, GGUF unchanged)."""
    from cwen_amd import gpu
    p, _ = model_file(tmp_path)
    s = tmp_path / "skip.cwenr"
    s.write_bytes(one(**kw))
    g = gpu.GGUF(p)
    assert g.apply_cwenr(s) == 0 and "no usable entries" in gpu.GGUF.last_error()
    assert all(g.tensor(i)[1] in (T_Q4_0, T_Q8_0) for i in range(len(g)))
    assert g.apply_cwenr(s) == 0          # nothing was kept: a later sidecar may still apply
    g.close()


def test_skipped_entries_leave_the_others_bound(tmp_path):
    from cwen_amd import gpu
    p, t = model_file(tmp_path)
    good = cwenr_from_gguf(t, 3)
    n = struct.unpack_from("<I", good, 12)[0]
    base = struct.unpack_from("<Q", good, 16)[0]
    extra = cwenr_entry("blk.7.nothing", 32, 1, 0, 0)
    # the same payload with one more (unknown) directory entry before it
    raw = cwenr_bytes([good[32 + 128 * i:32 + 128 * (i + 1)] for i in range(n)] + [extra], good[base:], 3)
    s = tmp_path / "m.cwenr"
    s.write_bytes(raw)
    g = gpu.GGUF(p)
    assert g.apply_cwenr(s) == 5
    with pytest.raises(gpu.CwenError) as e:
        g.apply_cwenr(s)
    assert "already applied" in str(e.value)
    g.close()


def test_missing_sidecar_is_optional(tmp_path):
    from cwen_amd import gpu
    p, _ = model_file(tmp_path)
    g = gpu.GGUF(p)
    assert g.apply_cwenr(tmp_path / "absent.cwenr") == 0 and gpu.GGUF.last_error() == "no sidecar"
    g.close()


def test_sidecar_path(monkeypatch):
    from cwen_amd import gpu
    monkeypatch.delenv("CWEN_REPACK", raising=False)
    assert gpu.GGUF.cwenr_path("/m/Qwen.gguf") == "/m/Qwen.cwenr"
    assert gpu.GGUF.cwenr_path("/m/Qwen.bin") == "/m/Qwen.bin.cwenr"
    assert gpu.GGUF.cwenr_path(".gguf") == ".gguf.cwenr"
    monkeypatch.setenv("CWEN_REPACK", "/elsewhere/x.cwenr")
    assert gpu.GGUF.cwenr_path("/m/Qwen.gguf") == "/elsewhere/x.cwenr"
    monkeypatch.delenv("CWEN_REPACK")
    with pytest.raises(gpu.CwenError):
        gpu.GGUF.cwenr_path("/m/" + "a" * 5000 + ".gguf")
