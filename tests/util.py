"""Shared test helpers."""
import numpy as np


def rel_err(y, ref) -> float:
    """max |y - ref| / max |ref| over the whole output (norm-wise relative error).

    This is the relative tolerance the parity tests state: per-element
    relative error is meaningless for outputs near zero, whose absolute error
    is set by the magnitude of the other terms of the dot product."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.max(np.abs(ref))
    return float(np.max(np.abs(y - ref)) / (den if den > 0 else 1.0))


def q6_k_pack(q6: np.ndarray, sc: np.ndarray, d_bits: np.ndarray) -> np.ndarray:
    """GGUF Q6_K super-blocks from natural-order values: q6 [R][K] in 0..63
    (weight = d * sc * (q6 - 32)), sc [R][K/16] int8 sub-block scales, d_bits
    [R][K/256] f16 bit patterns.  Layout {ql[128] qh[64] i8 sc[16] f16 d}:
    in each half h of 128 weights, quarter j of 32 takes ql bytes
    h*64 + (j&1)*32 + l (low nibble for j < 2, high for j >= 2) and qh bits
    2j..2j+1 of byte h*32 + l."""
    R, K = q6.shape
    q = q6.reshape(R, K // 256, 2, 4, 32).astype(np.uint8)
    ql = np.empty((R, K // 256, 2, 64), np.uint8)
    ql[..., :32] = (q[:, :, :, 0] & 15) | ((q[:, :, :, 2] & 15) << 4)
    ql[..., 32:] = (q[:, :, :, 1] & 15) | ((q[:, :, :, 3] & 15) << 4)
    qh = (q[:, :, :, 0] >> 4) | ((q[:, :, :, 1] >> 4) << 2) | ((q[:, :, :, 2] >> 4) << 4) | ((q[:, :, :, 3] >> 4) << 6)
    out = np.empty((R, K // 256, 210), np.uint8)
    out[..., :128] = ql.reshape(R, K // 256, 128)
    out[..., 128:192] = qh.reshape(R, K // 256, 64)
    out[..., 192:208] = sc.reshape(R, K // 256, 16).astype(np.int8).view(np.uint8)
    out[..., 208:210] = d_bits.astype(np.uint16).reshape(R, K // 256, 1).view(np.uint8)
    return out.reshape(R, -1)
