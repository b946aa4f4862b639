"""Element-wise error bound of the device GEMV, for the GPU tests, with the
cases they run.

With u = 2^-11 (f16's unit roundoff) and A_ik = |w_ik| (for Q4_1 and Q5_K
|n*d| + |m| and |d*sc*q| + |dmin*m|, the two terms of a weight that can
cancel):
  * each device weight is the exact one rounded c_w times to f16 (c_w = 1:
    (n - 8) d, q8 d, and n d + m with one fused rounding; c_w = 2: Q6_K's
    f16(d*sc) then the product, Q5_K's f16 scale and offset then the fused
    q*D + M), so |w' - w| <= c_w u A (1 + u);
  * each activation is rounded once to f16: |x' - x| <= u |x|, or 2^-25
    below f16's normal range;
  * w' x' is exact in f32; the output is then a chain of at most
    d = 32 + K/64 + 40 f32 additions (inside an MFMA, along one of a wave's
    two accumulator chains, the chains' sum, the split-K pieces), which
    adds at most g S_i, g = d 2^-24 / (1 - d 2^-24), S_i = sum_k A_ik |x_k|.
The product errors e_k = w'_k x'_k - w_k x_k are odd in the sign of x_k
(f16 rounding is sign-symmetric) and |e_k| <= c_k = ((c_w + 1) u + 2u^2) A_ik |x_k|.
For activations with independent symmetric signs, Hoeffding's inequality
gives |sum_k e_k| <= lam * sqrt(sum_k c_k^2) except with probability
2 exp(-lam^2 / 2); lam = 7 puts that below 1e-10 per element.  Hence
    |y_dev - y|_i <= lam sqrt(sum_k c_k^2) + g S_i + 2^-25 sum_k A_ik.
"""
import numpy as np

from cwen_amd import synth

LAM = 7.0


def elem_case(kind, K, M=256):
    """(wtype, data, scales, side, W, A, c_w) of one test case."""
    import dequant as D
    sc, side = None, 0
    if kind == "rs":
        data, sc = synth.q4_rs(121, M, K); wtype, cw = 101, 1
        W = D.rs(data, sc, M, K); A = np.abs(W)
    elif kind == "rsi":
        data, sc = synth.q4_rsi(121, M, K); wtype, cw, side = 102, 1, 1
        W = D.rs(*synth.rsi_side(data, sc, M, K, side), M, K); A = np.abs(W)
    elif kind == "q4_0":
        data = synth.q4_gguf(121, M, K); wtype, cw = 2, 1
        W = D.q4_0(data, M, K); A = np.abs(W)
    elif kind == "q8_0":
        data = synth.q8_0(121, M, K); wtype, cw = 8, 1
        W = D.q8_0(data, M, K); A = np.abs(W)
    elif kind == "q4_1":
        data = synth.q4_1(121, M, K); wtype, cw = 3, 1
        W, A = D.q4_1(data, M, K)
    elif kind == "q5_k":
        data = synth.q5_k(121, M, K); wtype, cw = 13, 2
        W, A = D.q5_k(data, M, K)
    else:
        data = synth.q6_k(121, M, K); wtype, cw = 14, 2
        W = D.q6_k(data, M, K); A = np.abs(W)
    return wtype, data, sc, side, W, A, cw


def elem_bound(W, A, X, K, cw):
    """The bound above for every output element, [B][M]."""
    u = 2.0 ** -11
    depth = 32 + K // 64 + 40
    g = depth * 2.0 ** -24 / (1 - depth * 2.0 ** -24)
    ax = np.abs(np.asarray(X, np.float64))
    ck = ((cw + 1) * u + 2 * u * u)
    rnd = LAM * ck * np.sqrt((ax ** 2) @ (A ** 2).T)
    return rnd + g * (ax @ A.T) + 2.0 ** -25 * A.sum(1)
