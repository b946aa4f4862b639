"""Writes tests/golden/reference_vectors.npz: input/output vectors of the
reference engine's own kernels (run.c compiled by oracle/Makefile into
oracle/_ref, AVX2 build), so the oracle can be re-checked where the reference
tree is absent.

    python tests/golden/make_golden.py        # needs oracle/_ref built

The quantized weights and activations of the GEMV cases are stored with
their outputs.  Every other input comes from `hash_f32`, a splitmix64 stream
that any numpy reproduces exactly, and only outputs are stored (a slice of
them for the fixed-size conv over 10240 channels and gdn_step over 48
heads).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
OUT = HERE / "reference_vectors.npz"


def hash_f32(seed: int, n: int, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    """n floats uniform in [lo, hi) from splitmix64(seed * 2^32 + i)."""
    with np.errstate(over="ignore"):
        z = (np.uint64(seed) << np.uint64(32)) + np.arange(n, dtype=np.uint64)
        z = z * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    u = (z >> np.uint64(40)).astype(np.float64) / float(1 << 24)
    return (lo + (hi - lo) * u).astype(np.float32)


# fixed-size kernel inputs (reference dims: conv C = 10240; GDN 16 k-heads, 48 v-heads, dk 128)
C_CONV, NKH, NVH, DK = 10240, 16, 48, 128
CONV_KEEP = 512          # channels of the conv outputs stored
GDN_HEAD = 5             # value head whose state is stored


def conv_inputs():
    return (hash_f32(101, C_CONV), hash_f32(102, C_CONV * 3), hash_f32(103, C_CONV * 4, -0.5, 0.5))


def gdn_inputs():
    C = (2 * NKH + NVH) * DK
    S = hash_f32(201, NVH * DK * DK, -0.02, 0.02)
    qkv = hash_f32(202, C, -2, 2)
    z = hash_f32(203, NVH * DK, -2, 2)
    decay = np.log(hash_f32(204, NVH, 0.05, 1.0)).astype(np.float32)
    beta = hash_f32(205, NVH, 0.0, 1.0)
    wn = hash_f32(206, DK, 0.5, 1.5)
    return S, qkv, z, decay, beta, wn


def elementwise_inputs():
    return hash_f32(11, 4096, -8, 8), hash_f32(12, 4096, -3, 3), hash_f32(13, 5120, -3, 3), hash_f32(14, 5120, 0.5, 1.5)


def argmax_inputs():
    lg = hash_f32(41, 3 * 1000, -5, 5).reshape(3, 1000)
    lg[0, 17] = lg[0, 600] = 9.0          # tie: the first index wins
    lg[1, 0] = np.nan                      # NaN at row position 0
    lg[2, 321] = np.nan
    return lg


def walk_inputs():
    wl = hash_f32(42, 8 * 1000, -5, 5).reshape(8, 1000)
    top = wl.argmax(1).astype(np.int32)
    drafts = np.concatenate([top[:4], [(top[4] + 1) % 1000], top[5:7]]).astype(np.int32)  # mistake at 4
    return wl, drafts


def attn_inputs(NH: int, NKV: int, HD: int, T: int = 40):
    q = hash_f32(51, NH * HD, -1, 1).reshape(NH, HD)
    Kc = hash_f32(52, T * NKV * HD, -1, 1).reshape(T, NKV, HD)
    Vc = hash_f32(53, T * NKV * HD, -1, 1).reshape(T, NKV, HD)
    gate = hash_f32(54, NH * HD, -2, 2).reshape(NH, HD)
    return q, Kc, Vc, gate


NGRAM_HIST = np.tile(np.array([5, 9, 2, 7, 7, 3, 1, 4], np.int32), 6)[:-3]


def main() -> int:
    sys.path.insert(0, str(ROOT))
    from cwen_amd import synth
    from oracle.binding import Reference
    R = Reference("avx2")
    v = {}
    # batched GEMV, the seven weight formats (B = 3)
    M, K, B = 32, 512, 3
    X = synth.activations(31, B, K)
    v["gemv_X"] = X
    qs, sc = synth.q4_rs(31, M, K)
    v["gemv_rs_qs"], v["gemv_rs_sc"], v["gemv_rs_Y"] = qs, sc, R.gemvb(101, qs, sc, K, M, X)
    qs, sc = synth.q4_rsi(31, M, K)
    v["gemv_rsi_qs"], v["gemv_rsi_sc"] = qs, sc
    v["gemv_rsi_Y0"], v["gemv_rsi_Y1"] = R.gemvb(102, qs, sc, K, M, X, 0), R.gemvb(102, qs, sc, K, M, X, 1)
    blk = synth.q4_gguf(31, M, K)
    v["gemv_q4_0"], v["gemv_q4_0_Y"] = blk, R.gemvb(2, blk, None, K, M, X)
    blk = synth.q8_0(31, M, K)
    v["gemv_q8_0"], v["gemv_q8_0_Y"] = blk, R.gemvb(8, blk, None, K, M, X)
    blk = synth.q4_1(31, M, K)
    v["gemv_q4_1"], v["gemv_q4_1_Y"] = blk, R.gemvb(3, blk, None, K, M, X)
    K6 = 1024
    X6 = synth.activations(32, B, K6)
    blk = synth.q6_k(31, M, K6)
    v["gemv_q6_k_X"], v["gemv_q6_k"], v["gemv_q6_k_Y"] = X6, blk, R.gemvb(14, blk, None, K6, M, X6)
    blk = synth.q5_k(31, M, K6)
    v["gemv_q5_k"], v["gemv_q5_k_Y"] = blk, R.gemvb(13, blk, None, K6, M, X6)
    # elementwise
    a, b, x, w = elementwise_inputs()
    v["silu_out"], v["rms_out"] = R.silu_mul(a, b), R.rmsnorm(x, w)
    # conv1d_update, gdn_step
    q, h = R.conv1d_update(*conv_inputs())
    v["conv_qkv_out"], v["conv_hist_out"] = q[:CONV_KEEP], h.reshape(C_CONV, 3)[:CONV_KEEP]
    S1, _, o = R.gdn_step(*gdn_inputs())
    v["gdn_out"], v["gdn_S_head"] = o, S1.reshape(NVH, DK, DK)[GDN_HEAD]
    # argmax with ties and NaN, the walk, the n-gram drafter
    v["argmax_out"] = np.array([R.argmax(r) for r in argmax_inputs()], np.int32)
    v["walk_out"] = np.array(R.walk(*walk_inputs()), np.int32)
    for nk in (2, 4, 16):
        v[f"ngram_out_{nk}"] = np.asarray(R.ngram_draft(NGRAM_HIST, nk, 7), np.int32)
    # rope and attention at the reference's fixed head shape
    NH, NKV, HD = R.attn_dims()
    v["attn_dims"] = np.array([NH, NKV, HD], np.int32)
    q, Kc, Vc, gate = attn_inputs(NH, NKV, HD)
    v["rope_out"] = R.rope(q, 123)
    v["attn_out"] = R.attention(Kc, Vc, 0, Kc.shape[0] - 1, q, gate)
    # embedding row (GGUF Q4_0 table of 4 tokens)
    tab = synth.q4_gguf(61, 4, 5120)
    v["embed_q4_0"], v["embed_out"] = tab, R.embed(2, tab, None, 3)
    v["isa"] = np.array(R.isa)
    np.savez_compressed(OUT, **v)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(v)} arrays)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
