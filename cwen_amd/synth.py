"""Seeded synthetic inputs for the block-verify workloads (numpy, host side).

Distributions follow the workload definitions:
  * Q4_0 weights: per 32-weight block an f16 scale d = f16(|N(0, 0.02)| / 8)
    and 16 bytes of nibbles uniform over 0..15; weight = (nibble - 8) * d.
  * Q6_K weights: ql/qh bytes uniform (6-bit quants uniform), int8 sub-scales
    uniform over [-128, 127], f16 d = f16(|N(0, 0.002)|).
  * Q8_0 weights: int8 quants uniform, f16 d = f16(|N(0, 0.02)| / 64).
  * Activations: f32 N(0, 1).

Generators are numpy PCG64 streams keyed by (seed, purpose) so every array
is reproducible on any host with the same numpy.
"""
from __future__ import annotations

import numpy as np

QK4 = 32
QK_K = 256


def rng(seed: int, *key: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(np.random.SeedSequence([seed, *key])))


def _f16_bits(x: np.ndarray) -> np.ndarray:
    return x.astype(np.float32).astype(np.float16).view(np.uint16)


def q4_scales(g: np.random.Generator, n: int) -> np.ndarray:
    return _f16_bits(np.abs(g.standard_normal(n, dtype=np.float32) * np.float32(0.02)) / np.float32(8))


def q4_nibble_bytes(g: np.random.Generator, n: int) -> np.ndarray:
    return g.integers(0, 256, size=n, dtype=np.uint8)


def q4_rs(seed: int, M: int, K: int, key: int = 0) -> tuple[np.ndarray, np.ndarray]:
    """CWENR split layout: qs[M][nb][16] bytes, sc[M][nb] f16 bits."""
    nb = K // QK4
    g = rng(seed, 1, key)
    sc = q4_scales(g, M * nb)
    qs = q4_nibble_bytes(g, M * nb * 16)
    return qs, sc


def q4_rsi(seed: int, M: int, K: int, key: int = 0) -> tuple[np.ndarray, np.ndarray]:
    """CWENR interleaved pair: qs[M][nb][A16|B16], sc[M][nb][A|B]."""
    nb = K // QK4
    g = rng(seed, 2, key)
    sc = q4_scales(g, M * nb * 2)
    qs = q4_nibble_bytes(g, M * nb * 32)
    return qs, sc


def q4_gguf(seed: int, M: int, K: int, key: int = 0) -> np.ndarray:
    """GGUF Q4_0: 18-byte blocks {f16 d; u8 qs[16]} row-major."""
    nb = K // QK4
    g = rng(seed, 3, key)
    sc = q4_scales(g, M * nb)
    qs = q4_nibble_bytes(g, M * nb * 16)
    out = np.empty((M * nb, 18), dtype=np.uint8)
    out[:, 0:2] = sc.view(np.uint8).reshape(-1, 2)
    out[:, 2:] = qs.reshape(-1, 16)
    return out.reshape(-1)


def q4_1(seed: int, M: int, K: int, key: int = 0) -> np.ndarray:
    """GGUF Q4_1: 20-byte blocks {f16 d; f16 m; u8 qs[16]}, w = n*d + m.  As a
    quantiser would set them, m is near the block minimum: m = -(8 + N(0,1)/2) d."""
    nb = K // QK4
    g = rng(seed, 7, key)
    sc = q4_scales(g, M * nb)
    d = sc.view(np.float16).astype(np.float32)
    m = _f16_bits(-(np.float32(8) + g.standard_normal(M * nb, dtype=np.float32) / np.float32(2)) * d)
    qs = q4_nibble_bytes(g, M * nb * 16)
    out = np.empty((M * nb, 20), dtype=np.uint8)
    out[:, 0:2] = sc.view(np.uint8).reshape(-1, 2)
    out[:, 2:4] = m.view(np.uint8).reshape(-1, 2)
    out[:, 4:] = qs.reshape(-1, 16)
    return out.reshape(-1)


def q5_k(seed: int, M: int, K: int, key: int = 0) -> np.ndarray:
    """GGUF Q5_K: 176-byte super-blocks {f16 d; f16 dmin; u8 scales[12];
    u8 qh[32]; u8 qs[128]}: 5-bit quants and 6-bit scales/mins uniform,
    d = |N(0, 0.002)|, dmin = |N(0, 0.002)|."""
    nsb = M * (K // QK_K)
    g = rng(seed, 8, key)
    blk = g.integers(0, 256, size=(nsb, 176), dtype=np.uint8)
    blk[:, 0:2] = _f16_bits(np.abs(g.standard_normal(nsb, dtype=np.float32) * np.float32(0.002))).view(np.uint8).reshape(-1, 2)
    blk[:, 2:4] = _f16_bits(np.abs(g.standard_normal(nsb, dtype=np.float32) * np.float32(0.002))).view(np.uint8).reshape(-1, 2)
    return blk.reshape(-1)


def q6_k(seed: int, M: int, K: int, key: int = 0) -> np.ndarray:
    """GGUF Q6_K: 210-byte super-blocks {ql[128] qh[64] i8 sc[16] f16 d}."""
    nsb = M * (K // QK_K)
    g = rng(seed, 4, key)
    blk = g.integers(0, 256, size=(nsb, 210), dtype=np.uint8)
    d = _f16_bits(np.abs(g.standard_normal(nsb, dtype=np.float32) * np.float32(0.002)))
    blk[:, 208:210] = d.view(np.uint8).reshape(-1, 2)
    return blk.reshape(-1)


def q8_0(seed: int, M: int, K: int, key: int = 0) -> np.ndarray:
    """GGUF Q8_0: 34-byte blocks {f16 d; i8 qs[32]}."""
    nblk = M * (K // QK4)
    g = rng(seed, 5, key)
    blk = g.integers(0, 256, size=(nblk, 34), dtype=np.uint8)
    d = _f16_bits(np.abs(g.standard_normal(nblk, dtype=np.float32) * np.float32(0.02)) / np.float32(64))
    blk[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    return blk.reshape(-1)


def activations(seed: int, B: int, K: int, key: int = 0) -> np.ndarray:
    """f32 N(0,1) activation block [B][K]."""
    return rng(seed, 6, key).standard_normal((B, K), dtype=np.float32)


def rs_to_gguf(qs: np.ndarray, sc: np.ndarray) -> np.ndarray:
    """Re-assemble a split (RS) tensor into GGUF 18-byte blocks (the inverse of
    the reference's v3 split, tools/repack_q4.py:75-81)."""
    nblk = sc.size
    out = np.empty((nblk, 18), dtype=np.uint8)
    out[:, 0:2] = sc.view(np.uint8).reshape(-1, 2)
    out[:, 2:] = qs.reshape(-1, 16)
    return out.reshape(-1)


def rsi_side(qs: np.ndarray, sc: np.ndarray, M: int, K: int, side: int) -> tuple[np.ndarray, np.ndarray]:
    """Extract one side of an interleaved pair as a split (RS) tensor."""
    nb = K // QK4
    q = qs.reshape(M, nb, 2, 16)[:, :, side, :]
    s = sc.reshape(M, nb, 2)[:, :, side]
    return np.ascontiguousarray(q).reshape(-1), np.ascontiguousarray(s).reshape(-1)


# ---------------------------------------------------------------- whole model
def model_tensors(cfg: dict, seed: int = 0, real_types: bool = False, mtp: bool = False, only_layer=None,
                  only_linear: bool = False):
    """Seeded random-init tensors of the hybrid decoder, in the reference's
    layouts: yields (layer, tensor id, type, data, scales, ne0, ne1); layer -1
    for the global tensors.  Q4_0 matrices are CWENR (RS, or RSI for the
    gate/up and k/v pairs), the head Q6_K, the embedding Q4_0RS; norms, conv
    taps and gate parameters F32.  real_types: the GGUF types the real
    model mixes in -- ffn_down of every other layer in Q4_1, every ssm_out
    in Q5_K.  mtp: also the MTP nextn drafter -- a full-attention block at
    layer n_layers and the nextn eh_proj (Q4_0RS, [H][2H]) and norms.
    only_layer: that layer's tensors alone, as a full-attention layer, or a
    GatedDeltaNet one with only_linear (the other tensors are not
    generated)."""
    from . import gpu as G
    H, I, V = cfg["d_model"], cfg["d_ffn"], cfg["vocab"]
    nkh, nvh = cfg["gdn_nkh"], cfg["gdn_nvh"]
    C = (2 * nkh + nvh) * 128
    Zh = nvh * 128
    Qo, Ko = cfg["n_head"] * cfg["head_dim"], cfg["n_kv_head"] * cfg["head_dim"]
    f32 = np.float32

    def norm_w(key, n):
        return (1 + 0.1 * rng(seed, 20, key).standard_normal(n)).astype(f32)

    def layer(l, full, real_types):
        k0 = 100 * (l + 1)
        yield l, G.ATTN_NORM, G.T_F32, norm_w(k0 + 1, H), None, H, 1
        yield l, G.POST_NORM, G.T_F32, norm_w(k0 + 2, H), None, H, 1
        qs, sc = q4_rsi(seed, I, H, key=k0 + 3)
        yield l, G.FFN_GATE_UP, G.T_Q4_0RSI, qs, sc, H, I
        if real_types and l % 2 == 0:
            yield l, G.FFN_DOWN, G.T_Q4_1, q4_1(seed, H, I, key=k0 + 4), None, I, H
        else:
            qs, sc = q4_rs(seed, H, I, key=k0 + 4)
            yield l, G.FFN_DOWN, G.T_Q4_0RS, qs, sc, I, H
        if not full:
            for tid, M, key in ((G.ATTN_QKV, C, 5), (G.ATTN_GATE, Zh, 6), (G.SSM_ALPHA, nvh, 7),
                                (G.SSM_BETA, nvh, 8)):
                qs, sc = q4_rs(seed, M, H, key=k0 + key)
                yield l, tid, G.T_Q4_0RS, qs, sc, H, M
            if real_types:
                yield l, G.SSM_OUT, G.T_Q5_K, q5_k(seed, H, Zh, key=k0 + 9), None, Zh, H
            else:
                qs, sc = q4_rs(seed, H, Zh, key=k0 + 9)
                yield l, G.SSM_OUT, G.T_Q4_0RS, qs, sc, Zh, H
            g = rng(seed, 21, k0)
            yield l, G.SSM_A, G.T_F32, (-np.exp(g.uniform(-1, 1, nvh))).astype(f32), None, nvh, 1
            yield l, G.SSM_DT, G.T_F32, (0.5 * g.standard_normal(nvh)).astype(f32), None, nvh, 1
            yield l, G.SSM_CONV, G.T_F32, (0.3 * g.standard_normal(4 * C)).astype(f32), None, 4 * C, 1
            yield l, G.SSM_NORM, G.T_F32, norm_w(k0 + 10, 128), None, 128, 1
        else:
            qs, sc = q4_rs(seed, 2 * Qo, H, key=k0 + 11)
            yield l, G.ATTN_Q, G.T_Q4_0RS, qs, sc, H, 2 * Qo
            qs, sc = q4_rsi(seed, Ko, H, key=k0 + 12)
            yield l, G.ATTN_KV, G.T_Q4_0RSI, qs, sc, H, Ko
            qs, sc = q4_rs(seed, H, Qo, key=k0 + 13)
            yield l, G.ATTN_OUTPUT, G.T_Q4_0RS, qs, sc, Qo, H
            yield l, G.ATTN_Q_NORM, G.T_F32, norm_w(k0 + 14, cfg["head_dim"]), None, cfg["head_dim"], 1
            yield l, G.ATTN_K_NORM, G.T_F32, norm_w(k0 + 15, cfg["head_dim"]), None, cfg["head_dim"], 1

    if only_layer is not None:
        yield from layer(only_layer, not only_linear, False)
        return
    qs, sc = q4_rs(seed, V, H, key=1000)
    yield -1, G.TOK_EMBD, G.T_Q4_0RS, qs, sc, H, V
    yield -1, G.OUTPUT_NORM, G.T_F32, norm_w(1, H), None, H, 1
    yield -1, G.OUTPUT, G.T_Q6_K, q6_k(seed, V, H, key=1001), None, H, V

    for l in range(cfg["n_layers"]):
        yield from layer(l, l % cfg["full_interval"] == cfg["full_interval"] - 1, real_types)
    if mtp:
        yield from mtp_tensors(cfg, seed)


def mtp_tensors(cfg: dict, seed: int = 0):
    """The MTP nextn drafter's tensors alone (model_tensors(mtp=True) ends
    with them): the full-attention block at layer n_layers, eh_proj and the
    three nextn norms."""
    from . import gpu as G
    H = cfg["d_model"]
    NL = cfg["n_layers"]
    yield from model_tensors(cfg, seed, only_layer=NL)
    qs, sc = q4_rs(seed, H, 2 * H, key=90001)
    yield -1, G.NEXTN_EH_PROJ, G.T_Q4_0RS, qs, sc, 2 * H, H
    for tid, key in ((G.NEXTN_ENORM, 90002), (G.NEXTN_HNORM, 90003), (G.NEXTN_SHEAD_NORM, 90004)):
        yield -1, tid, G.T_F32, (1 + 0.1 * rng(seed, 20, key).standard_normal(H)).astype(np.float32), None, H, 1


def prompt_tokens(seed: int, n: int, V: int, period: int = 37, noise: float = 0.1) -> np.ndarray:
    """A seeded token history with periodic repeats: a random motif repeated,
    with a fraction `noise` of positions replaced by random ids."""
    g = rng(seed, 30)
    motif = g.integers(0, V, period)
    t = np.resize(motif, n)
    flip = g.random(n) < noise
    t[flip] = g.integers(0, V, int(flip.sum()))
    return t.astype(np.int32)
