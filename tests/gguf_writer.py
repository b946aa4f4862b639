"""Minimal GGUF v2/v3 writer for tests (test infrastructure only), and the
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
    glob = {G.TOK_EMBD: "token_embd.weight", G.OUTPUT_NORM: "output_norm.weight", G.OUTPUT: "output.weight"}
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
