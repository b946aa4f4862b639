"""numpy float64 dequantization of the reference's weight formats, written
from the GGUF / CWENR block definitions (run.c:93-139, 426-429), shared by
the oracle's f64 checks and the GPU tests' element-wise error bounds.

Each function returns W [M][K] (float64).  The K-quant and offset formats
also return the magnitude |scale term| + |offset term| per weight, which is
what bounds the rounding of w = q*D + M when its two terms cancel."""
import numpy as np


def f16(bits) -> np.ndarray:
    return np.ascontiguousarray(bits).view(np.float16).astype(np.float64)


def q4_blocks(qs16: np.ndarray, d_bits: np.ndarray) -> np.ndarray:
    """[nblk][16] nibble bytes + [nblk] f16 scale bits -> [nblk][32]: low
    nibbles are weights 0..15, high nibbles 16..31, w = (n - 8) * d."""
    q = np.asarray(qs16).reshape(-1, 16)
    n = np.concatenate([q & 0xF, q >> 4], axis=1).astype(np.float64) - 8
    return n * f16(d_bits).reshape(-1)[:, None]


def rs(qs, sc, M, K) -> np.ndarray:
    return q4_blocks(qs, sc).reshape(M, K)


def q4_0(blk, M, K) -> np.ndarray:
    b = np.asarray(blk).reshape(-1, 18)
    return q4_blocks(np.ascontiguousarray(b[:, 2:]), np.ascontiguousarray(b[:, :2])).reshape(M, K)


def q8_0(blk, M, K) -> np.ndarray:
    b = np.asarray(blk).reshape(-1, 34)
    return (np.ascontiguousarray(b[:, 2:]).view(np.int8).astype(np.float64)
            * f16(np.ascontiguousarray(b[:, :2])).reshape(-1, 1)).reshape(M, K)


def q4_1(blk, M, K):
    """{f16 d, f16 m, qs[16]}: w = n*d + m.  Returns (W, |n*d| + |m|)."""
    b = np.asarray(blk).reshape(-1, 20)
    d = f16(np.ascontiguousarray(b[:, 0:2])).reshape(-1, 1)
    m = f16(np.ascontiguousarray(b[:, 2:4])).reshape(-1, 1)
    q = b[:, 4:]
    n = np.concatenate([q & 0xF, q >> 4], axis=1).astype(np.float64)
    return (n * d + m).reshape(M, K), (np.abs(n * d) + np.abs(m)).reshape(M, K)


def q5_k(blk, M, K):
    """176-byte super-blocks {f16 d, f16 dmin, 12 B packed 6-bit scales and
    mins, qh[32], qs[128]}: w = d*sc*q - dmin*m per 32-weight sub-block, q 5
    bits (nibble of qs, fifth bit in qh).  Returns (W, |d*sc*q| + |dmin*m|)."""
    b = np.asarray(blk).reshape(-1, 176)
    d = f16(np.ascontiguousarray(b[:, 0:2])).reshape(-1)
    dmin = f16(np.ascontiguousarray(b[:, 2:4])).reshape(-1)
    s8 = b[:, 4:16].astype(np.int64)
    qh = b[:, 16:48].astype(np.int64)
    qs = b[:, 48:176].astype(np.int64).reshape(-1, 4, 32)
    sc = np.empty((b.shape[0], 8), np.int64)
    mn = np.empty((b.shape[0], 8), np.int64)
    for j in range(8):   # get_scale_min_k4 (run.c:426-429)
        if j < 4:
            sc[:, j], mn[:, j] = s8[:, j] & 63, s8[:, j + 4] & 63
        else:
            sc[:, j] = (s8[:, j + 4] & 15) | ((s8[:, j - 4] >> 6) << 4)
            mn[:, j] = (s8[:, j + 4] >> 4) | ((s8[:, j] >> 6) << 4)
    W = np.empty((b.shape[0], 256))
    A = np.empty((b.shape[0], 256))
    for jj in range(4):
        for half in range(2):
            sb = 2 * jj + half
            q = ((qs[:, jj] >> (4 * half)) & 15) + 16 * ((qh >> (2 * jj + half)) & 1)
            a = (d * sc[:, sb])[:, None] * q
            o = (dmin * mn[:, sb])[:, None]
            W[:, 64 * jj + 32 * half:64 * jj + 32 * half + 32] = a - o
            A[:, 64 * jj + 32 * half:64 * jj + 32 * half + 32] = np.abs(a) + np.abs(o)
    return W.reshape(M, K), A.reshape(M, K)


def q6_k(blk, M, K) -> np.ndarray:
    """210-byte super-blocks {ql[128], qh[64], i8 sc[16], f16 d}: in half h,
    quarter t of 32 weights takes ql[64h + 32(t&1) + l] (low nibble for t < 2)
    and bits 2t..2t+1 of qh[32h + l]; w = d * sc[j/16] * (q6 - 32)."""
    b = np.asarray(blk).reshape(-1, 210)
    ql = b[:, :128].reshape(-1, 2, 2, 32).astype(np.int64)     # [sb][h][t&1][l]
    qh = b[:, 128:192].reshape(-1, 2, 32).astype(np.int64)     # [sb][h][l]
    sc = np.ascontiguousarray(b[:, 192:208]).view(np.int8).astype(np.float64)
    d = f16(np.ascontiguousarray(b[:, 208:210])).reshape(-1)
    q = np.empty((b.shape[0], 2, 4, 32), np.int64)
    for t in range(4):
        nib = ql[:, :, t & 1] if t < 2 else ql[:, :, t & 1] >> 4
        q[:, :, t] = (nib & 15) | (((qh >> (2 * t)) & 3) << 4)
    w = (q.reshape(-1, 256) - 32).astype(np.float64) * np.repeat(sc, 16, axis=1) * d[:, None]
    return w.reshape(M, K)
