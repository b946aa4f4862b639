"""Minimal GGUF v2/v3 and CWENR sidecar writers for tests (test
infrastructure only; the sidecar layout of tools/repack_q4.py:1-27, 197-262), and the
conversion of the synthetic model's CWENR tensors to the GGUF tensors the
reference binds (run.c:3366-3406 names; GGUF Q4_0 blocks for the matrices
the reference's offline repack turns into CWENR RS/RSI)."""
import struct

import numpy as np

KV_U32, KV_F32, KV_BOOL, KV_STR, KV_ARR = 4, 6, 7, 8, 9


def gstr(s: bytes) -> bytes:
    return struct.pack("<Q", len(s)) + s


def kv_entry(key: bytes, vtype: int, payload: bytes) -> bytes:
    """One KV pair: key, value type, already-encoded value."""
    return gstr(key) + struct.pack("<I", vtype) + payload


def gguf_bytes(tensors, kv=(), version: int = 3, align: int = 32) -> bytes:
    """tensors: (name, ggml type, dims, data bytes); each tensor's data is
    placed at the next `align` boundary of the data section."""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kv)) + b"".join(kv)
    infos, data, off = [], b"", 0
    for name, typ, dims, raw in tensors:
        off = (off + align - 1) // align * align
        data = data.ljust(off, b"\0") + raw
        infos.append(gstr(name.encode()) + struct.pack("<I", len(dims)) +
                     b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", typ, off))
        off += len(raw)
    body = head + b"".join(infos)
    pad = (len(body) + align - 1) // align * align - len(body)
    return body + b"\0" * pad + data


def model_gguf_tensors(tensors, cfg: dict):
    """The GGUF tensor list of a synthetic model given as cwen_model_set
    tuples (synth.model_tensors): CWENR RS matrices become GGUF Q4_0 blocks,
    RSI pairs two Q4_0 tensors (side 0 = gate / k, side 1 = up / v)."""
    from cwen_amd import gpu as G
    from cwen_amd import synth

    name = {G.ATTN_NORM: "attn_norm.weight", G.POST_NORM: "post_attention_norm.weight",
            G.FFN_DOWN: "ffn_down.weight", G.ATTN_QKV: "attn_qkv.weight", G.ATTN_GATE: "attn_gate.weight",
            G.SSM_ALPHA: "ssm_alpha.weight", G.SSM_BETA: "ssm_beta.weight", G.SSM_A: "ssm_a",
            G.SSM_DT: "ssm_dt.bias", G.SSM_NORM: "ssm_norm.weight", G.SSM_OUT: "ssm_out.weight",
            G.ATTN_Q: "attn_q.weight", G.ATTN_OUTPUT: "attn_output.weight",
            G.ATTN_Q_NORM: "attn_q_norm.weight", G.ATTN_K_NORM: "attn_k_norm.weight"}
    pairs = {G.FFN_GATE_UP: ("ffn_gate.weight", "ffn_up.weight"), G.ATTN_KV: ("attn_k.weight", "attn_v.weight")}
    NL = cfg["n_layers"]
    glob = {G.TOK_EMBD: "token_embd.weight", G.OUTPUT_NORM: "output_norm.weight", G.OUTPUT: "output.weight",
            G.NEXTN_EH_PROJ: f"blk.{NL}.nextn.eh_proj.weight", G.NEXTN_ENORM: f"blk.{NL}.nextn.enorm.weight",
            G.NEXTN_HNORM: f"blk.{NL}.nextn.hnorm.weight",
            G.NEXTN_SHEAD_NORM: f"blk.{NL}.nextn.shared_head_norm.weight"}
    C = (2 * cfg["gdn_nkh"] + cfg["gdn_nvh"]) * 128
    out = []
    for layer, tid, wtype, data, sc, ne0, ne1 in tensors:
        full = glob[tid] if layer < 0 else None
        if tid in pairs and layer >= 0:
            for side, nm in enumerate(pairs[tid]):
                q1, s1 = synth.rsi_side(data, sc, ne1, ne0, side)
                out.append((f"blk.{layer}.{nm}", G.T_Q4_0, (ne0, ne1), synth.rs_to_gguf(q1, s1).tobytes()))
            continue
        nm = full or f"blk.{layer}.{name.get(tid, 'ssm_conv1d.weight')}"
        if wtype == G.T_Q4_0RS:
            out.append((nm, G.T_Q4_0, (ne0, ne1), synth.rs_to_gguf(data, sc).tobytes()))
        elif wtype == G.T_F32:
            dims = (4, C) if tid == G.SSM_CONV and layer >= 0 else (ne0,)
            out.append((nm, G.T_F32, dims, np.ascontiguousarray(data, np.float32).tobytes()))
        else:
            out.append((nm, wtype, (ne0, ne1), np.ascontiguousarray(data).tobytes()))
    return out


CWENR_TAG = 0x4E455743  # "CWEN"
PAIRS = ((".ffn_gate.weight", ".ffn_up.weight"), (".attn_k.weight", ".attn_v.weight"))


def cwenr_entry(name: str, ne0: int, ne1: int, a: int, b: int, flags: int = 0) -> bytes:
    """One 128-byte directory entry: name[96], ne0, ne1, two u64 offsets, flags, pad."""
    nb = name.encode()
    assert len(nb) < 96
    return nb.ljust(96, b"\0") + struct.pack("<iiQQII", ne0, ne1, a, b, flags, 0)


def cwenr_bytes(entries, payload: bytes, version: int = 4, src_pages: int | None = None,
                data_base: int | None = None) -> bytes:
    """Header (magic, version, count, data_base, stamp), the entries, the
    payload at data_base (by default the next 64-byte boundary)."""
    n = len(entries)
    base = (32 + 128 * n + 63) // 64 * 64 if data_base is None else data_base
    stamp = struct.pack("<II", CWENR_TAG, src_pages) if src_pages is not None else b"\0" * 8
    head = b"CWENR001" + struct.pack("<IIQ", version, n, base) + stamp + b"".join(entries)
    return head.ljust(base, b"\0") + payload


def cwenr_from_gguf(gt, version: int = 4, src_pages: int | None = None) -> bytes:
    """The sidecar of the GGUF Q4_0 tensors in gt ((name, type, dims, raw)):
    v4 interleaves the gate/up and k/v pairs and splits the rest, v3 splits
    every tensor into qs + f16 scales, v2 packs {qs[16], f32 d} blocks."""
    q4 = {name: (dims, raw) for name, typ, dims, raw in gt if typ == 2}
    entries, payload = [], bytearray()

    def put(blob: bytes) -> int:
        payload.extend(b"\0" * (-len(payload) % 64))
        off = len(payload)
        payload.extend(blob)
        return off

    def blocks(raw):
        return np.frombuffer(raw, np.uint8).reshape(-1, 18)

    used = set()
    for name in sorted(q4):
        if name in used:
            continue
        dims, raw = q4[name]
        ne0, ne1 = dims[0], dims[1] if len(dims) > 1 else 1
        partner = next((name[:-len(a)] + b for a, b in PAIRS if name.endswith(a)), None) if version == 4 else None
        if partner in q4:
            ba, bb = blocks(raw), blocks(q4[partner][1])
            qs = np.concatenate([ba[:, 2:], bb[:, 2:]], axis=1).tobytes()
            sc = np.concatenate([ba[:, :2], bb[:, :2]], axis=1).tobytes()
            a, b = put(qs), put(sc)
            entries += [cwenr_entry(name, ne0, ne1, a, b, 1), cwenr_entry(partner, ne0, ne1, a, b, 2)]
            used |= {name, partner}
            continue
        bl = blocks(raw)
        if version == 2:
            d = bl[:, :2].copy().view(np.float16).astype(np.float32)
            packed = np.concatenate([bl[:, 2:], d.view(np.uint8).reshape(-1, 4)], axis=1).tobytes()
            entries.append(cwenr_entry(name, ne0, ne1, put(packed), len(packed)))
        else:
            a, b = put(bl[:, 2:].tobytes()), put(bl[:, :2].tobytes())
            entries.append(cwenr_entry(name, ne0, ne1, a, b))
        used.add(name)
    return cwenr_bytes(entries, bytes(payload), version, src_pages)
