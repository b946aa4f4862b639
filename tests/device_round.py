"""Weights and GEMV operands rounded where the device rounds them (test
infrastructure, the oracle's "device" mode).

The reference multiplies f32 activations by weights dequantized in f32
(run.c:674-1274).  The device feeds its matrix cores f16 operands:

  * each weight is rounded once to f16 from the reference's exact value
    (the device's unpack computes it in f16 with one rounding):
      Q4_0 / RS / RSI  f16((n - 8) * d)
      Q8_0             f16(q * d)
      Q6_K             f16((q6 - 32) * f16(sc * d))
      Q4_1             f16(n * d + m)                  (one fused rounding)
      Q5_K             f16(q * f16(d * sc) + f16(-dmin * m))
  * each activation operand is rounded to f16; an input that is an RMSNorm
    output (run.c:346-368) is rounded before the normalisation scale, as
    f16(x * w), and the GEMV's output is multiplied by
    s = 1 / sqrt(sum(x^2) / K + eps) afterwards.

Products of two f16 values are exact in f32 and the device accumulates in
f32, so with these roundings the only remaining difference is the f32
summation order.  Here the sums are taken in float64.
"""
import numpy as np

import dequant as dq

T_F32, T_Q4_0, T_Q4_1, T_Q8_0, T_Q5_K, T_Q6_K, T_Q4_0RS, T_Q4_0RSI = 0, 2, 3, 8, 13, 14, 101, 102


# With ROUND off the mode keeps every weight and operand exact (float64 sums
# of the reference's values): the oracle's plain forward pass, reached through
# the device mode's composition (the tests pin that composition with it).
ROUND = True


def f16r(x) -> np.ndarray:
    """Round to the nearest f16 (ties to even), returned as float64."""
    if not ROUND:
        return np.asarray(x, np.float64)
    return np.asarray(x, np.float64).astype(np.float16).astype(np.float64)


def _q4(q: np.ndarray, d_bits: np.ndarray, M: int, K: int) -> np.ndarray:
    """[nblk][16] nibble bytes + f16 scale bits -> f16((n - 8) * d) [M][K]."""
    q = np.asarray(q).reshape(-1, 16)
    n = np.concatenate([q & 0xF, q >> 4], axis=1).astype(np.float64) - 8
    return f16r(n * dq.f16(d_bits).reshape(-1)[:, None]).reshape(M, K)


def weights(wtype: int, data: np.ndarray, sc, K: int, M: int, side: int = 0) -> np.ndarray:
    """The weight matrix [M][K] (float64) as the device's f16 operands."""
    if wtype == T_F32:
        return np.asarray(data, np.float32).reshape(M, K).astype(np.float64)
    if wtype == T_Q4_0:
        b = np.asarray(data).reshape(-1, 18)
        return _q4(np.ascontiguousarray(b[:, 2:]), np.ascontiguousarray(b[:, :2]), M, K)
    if wtype == T_Q4_0RS:
        return _q4(data, sc, M, K)
    if wtype == T_Q4_0RSI:   # qs [M][nb][A16 | B16], sc [M][nb][A | B]
        q = np.asarray(data).reshape(-1, 2, 16)[:, side]
        s = np.asarray(sc).reshape(-1, 2)[:, side]
        return _q4(np.ascontiguousarray(q), np.ascontiguousarray(s), M, K)
    if wtype == T_Q8_0:
        b = np.asarray(data).reshape(-1, 34)
        q = np.ascontiguousarray(b[:, 2:]).view(np.int8).astype(np.float64)
        return f16r(q * dq.f16(np.ascontiguousarray(b[:, :2])).reshape(-1, 1)).reshape(M, K)
    if wtype == T_Q4_1:
        b = np.asarray(data).reshape(-1, 20)
        d = dq.f16(np.ascontiguousarray(b[:, 0:2])).reshape(-1, 1)
        m = dq.f16(np.ascontiguousarray(b[:, 2:4])).reshape(-1, 1)
        q = b[:, 4:]
        n = np.concatenate([q & 0xF, q >> 4], axis=1).astype(np.float64)
        return f16r(n * d + m).reshape(M, K)
    if wtype == T_Q6_K:
        b = np.asarray(data).reshape(-1, 210)
        ql = b[:, :128].reshape(-1, 2, 2, 32).astype(np.int64)
        qh = b[:, 128:192].reshape(-1, 2, 32).astype(np.int64)
        scv = np.ascontiguousarray(b[:, 192:208]).view(np.int8).astype(np.float64)
        d = dq.f16(np.ascontiguousarray(b[:, 208:210])).reshape(-1)
        q = np.empty((b.shape[0], 2, 4, 32), np.int64)
        for t in range(4):
            nib = ql[:, :, t & 1] if t < 2 else ql[:, :, t & 1] >> 4
            q[:, :, t] = (nib & 15) | (((qh >> (2 * t)) & 3) << 4)
        ds = f16r(scv * d[:, None])                    # [sb][16] f16(sc * d)
        w = f16r((q.reshape(-1, 256) - 32).astype(np.float64) * np.repeat(ds, 16, axis=1))
        return w.reshape(M, K)
    if wtype == T_Q5_K:
        return _q5_k(data, M, K)
    raise ValueError(f"type {wtype}")


def _q5_k(blk, M: int, K: int) -> np.ndarray:
    """f16(q * D + Mo), D = f16(d * sc), Mo = f16(-dmin * m) per 32-weight
    sub-block (get_scale_min_k4, run.c:426-429, as in dequant.q5_k)."""
    b = np.asarray(blk).reshape(-1, 176)
    d = dq.f16(np.ascontiguousarray(b[:, 0:2])).reshape(-1)
    dmin = dq.f16(np.ascontiguousarray(b[:, 2:4])).reshape(-1)
    s8 = b[:, 4:16].astype(np.int64)
    qh = b[:, 16:48].astype(np.int64)
    qs = b[:, 48:176].astype(np.int64).reshape(-1, 4, 32)
    W = np.empty((b.shape[0], 256))
    for jj in range(4):
        for half in range(2):
            j = 2 * jj + half
            if j < 4:
                sc, mn = s8[:, j] & 63, s8[:, j + 4] & 63
            else:
                sc = (s8[:, j + 4] & 15) | ((s8[:, j - 4] >> 6) << 4)
                mn = (s8[:, j + 4] >> 4) | ((s8[:, j] >> 6) << 4)
            q = ((qs[:, jj] >> (4 * half)) & 15) + 16 * ((qh >> j) & 1)
            D = f16r(d * sc)[:, None]
            Mo = f16r(-(dmin * mn))[:, None]
            W[:, 32 * j:32 * j + 32] = f16r(q * D + Mo)
    return W.reshape(M, K)


# Sensitivity probe: when set, operand() first perturbs its input by
# JITTER * max|x| * N(0, 1) per element (a stand-in for the device's own f32
# summation order upstream of the rounding).  Tests measure how far that moves
# a position's logits.
JITTER = 0.0
_rng = np.random.default_rng(0)


def seed_jitter(seed: int) -> None:
    """Restart the perturbation stream (each sensitivity trial seeds its own)."""
    global _rng
    _rng = np.random.default_rng(seed)


def operand(x) -> np.ndarray:
    """An f32 activation vector as the device's f16 operand (float64)."""
    x = np.asarray(x, np.float32)
    if JITTER:
        x = (x + np.float32(JITTER) * np.max(np.abs(x)) * _rng.standard_normal(x.shape)).astype(np.float32)
    return f16r(x)


def norm_scale(x, eps: float) -> np.float32:
    """The RMSNorm scale 1 / sqrt(sum(x^2) / K + eps) in f32 (run.c:346-368)."""
    x = np.asarray(x, np.float32)
    ss = np.float32(np.sum(x.astype(np.float64) ** 2))
    return np.float32(1.0) / np.sqrt(ss / np.float32(x.size) + np.float32(eps))


def gemv(W16: np.ndarray, x16: np.ndarray, scale=None) -> np.ndarray:
    """W16 @ x16 summed in float64, times the norm scale (f32), as f32."""
    y = (W16 @ x16).astype(np.float32)
    return y * np.float32(scale) if scale is not None else y
