"""The oracle's device-rounding mode (tests/device_round.py) pinned on the
CPU; its agreement with the device itself is tests/test_device_round_gpu.py's
(every format within 1e-5 of the device's GEMV) and the model tests'.

  * weights: the formats whose device weight is one rounding of the exact
    value (Q4_0 family, Q8_0, Q4_1) equal f16(exact) bit for bit; Q6_K and
    Q5_K, rounded twice, stay within their stated bound of the exact values
    of tests/dequant.py (which the oracle's own tests pin), and differ from a
    single rounding somewhere (the formula is not the single rounding).
  * composition: with the rounding switched off, the device mode -- its
    split RMSNorm f16(x * w) * s, its float64 GEMVs, the nextn stream --
    reproduces the plain oracle's logits within 2e-5 (f32 vs float64 sums),
    so every GEMV is wired to the right input, norm weight and side.
  * size: with rounding, the device mode's logits stay within 4 x the f16
    input-rounding spread + 1e-4 of the plain oracle's (both perturb the
    same f16 points; the mode also rounds the weights).
"""
import numpy as np
import pytest

import dequant as dq
import device_round as dr
from cwen_amd import synth
from util import rel_err

CFG = dict(n_layers=4, d_model=512, d_ffn=1024, vocab=1024, n_head=4, n_kv_head=2, head_dim=256,
           n_rot_pairs=32, n_rot=64, gdn_nkh=2, gdn_nvh=4, gdn_dk=128, full_interval=4, max_ctx=64,
           rope_theta=1e7, rms_eps=1e-6)


def _is_f16(W):
    return np.array_equal(W.astype(np.float16).astype(np.float64), W)


@pytest.mark.parametrize("kind", ["q4_0", "rs", "rsi0", "rsi1", "q8_0", "q4_1"])
def test_single_rounding_formats_equal_f16_of_exact(kind):
    M, K = 48, 512
    if kind == "q4_0":
        data, sc, t, side = synth.q4_gguf(5, M, K), None, dr.T_Q4_0, 0
        exact = dq.q4_0(data, M, K)
    elif kind == "rs":
        (data, sc), t, side = synth.q4_rs(5, M, K), dr.T_Q4_0RS, 0
        exact = dq.rs(data, sc, M, K)
    elif kind.startswith("rsi"):
        (data, sc), t, side = synth.q4_rsi(5, M, K), dr.T_Q4_0RSI, int(kind[-1])
        q = np.asarray(data).reshape(-1, 2, 16)[:, side]
        exact = dq.rs(np.ascontiguousarray(q), np.ascontiguousarray(np.asarray(sc).reshape(-1, 2)[:, side]), M, K)
    elif kind == "q8_0":
        data, sc, t, side = synth.q8_0(5, M, K), None, dr.T_Q8_0, 0
        exact = dq.q8_0(data, M, K)
    else:
        data, sc, t, side = synth.q4_1(5, M, K), None, dr.T_Q4_1, 0
        exact = dq.q4_1(data, M, K)[0]
    W = dr.weights(t, data, sc, K, M, side)
    assert _is_f16(W)
    assert np.array_equal(W, exact.astype(np.float16).astype(np.float64))
    assert not np.array_equal(W, exact)          # the rounding is real


@pytest.mark.parametrize("kind", ["q6_k", "q5_k"])
def test_double_rounding_formats(kind):
    M, K = 48, 512
    if kind == "q6_k":
        data = synth.q6_k(6, M, K)
        W, exact = dr.weights(dr.T_Q6_K, data, None, K, M), dq.q6_k(data, M, K)
        mag = np.abs(exact)                    # f16(sc d) then f16((q - 32) * that): two relative roundings
    else:
        data = synth.q5_k(6, M, K)
        W = dr.weights(dr.T_Q5_K, data, None, K, M)
        exact, mag = dq.q5_k(data, M, K)       # |q D| + |Mo| bounds the cancelling terms' roundings
    assert _is_f16(W)
    u = 2.0 ** -11
    assert np.all(np.abs(W - exact) <= 2 * u * mag + u * np.abs(exact) + 2.0 ** -24)
    assert not np.array_equal(W, exact.astype(np.float16).astype(np.float64))


def _logits(oracle, tensors, toks, **kw):
    from model_oracle import OracleModel
    om = OracleModel(oracle, CFG, tensors, **kw)
    out = [om.step(int(t), p) for p, t in enumerate(toks)]
    drafts = om.mtp_draft_logits(int(toks[-1]), len(toks) - 1, [3, 5]) if om.has_mtp else None
    return np.stack(out), drafts


def test_composition_without_rounding_is_the_plain_oracle(oracle):
    tensors = list(synth.model_tensors(CFG, seed=4, mtp=True))
    toks = synth.prompt_tokens(4, 10, CFG["vocab"])
    ref, ref_d = _logits(oracle, tensors, toks)
    try:
        dr.ROUND = False
        dev, dev_d = _logits(oracle, tensors, toks, device=True)
    finally:
        dr.ROUND = True
    errs = [rel_err(dev[p], ref[p]) for p in range(len(toks))] + [rel_err(dev_d[t], ref_d[t]) for t in range(2)]
    assert max(errs) <= 2e-5, errs


def test_device_mode_is_an_f16_scale_perturbation(oracle):
    tensors = list(synth.model_tensors(CFG, seed=4))
    toks = synth.prompt_tokens(4, 10, CFG["vocab"])
    ref, _ = _logits(oracle, tensors, toks)
    ref16, _ = _logits(oracle, tensors, toks, f16_inputs=True)
    dev, _ = _logits(oracle, tensors, toks, device=True)
    for p in range(len(toks)):
        spread = rel_err(ref16[p], ref[p])
        assert 0 < rel_err(dev[p], ref[p]) <= 4 * spread + 1e-4, (p, rel_err(dev[p], ref[p]), spread)


def test_np_attention_equals_the_c_restatement(oracle):
    """np_attention (tests/model_oracle.py, for the long-context fixtures) vs
    orc_attention at the 27B shape's 24 / 4 heads of 256, with and without a
    first slot t0 > 0: within 2e-6 (f32 sums in another order)."""
    from model_oracle import np_attention
    g = np.random.default_rng(3)
    T, nkv, nh, hd = 300, 4, 24, 256
    K = g.standard_normal((T, nkv, hd)).astype(np.float32)
    V = g.standard_normal((T, nkv, hd)).astype(np.float32)
    Kg, Vg = np.ascontiguousarray(K.transpose(1, 0, 2)), np.ascontiguousarray(V.transpose(1, 0, 2))
    for t0, pos in ((0, 0), (0, 37), (0, 299), (1, 150)):
        q = (0.3 * g.standard_normal((nh, hd))).astype(np.float32)
        gate = g.standard_normal((nh, hd)).astype(np.float32)
        want = oracle.attention(K[:pos + 1], V[:pos + 1], t0, pos, q, gate)
        got = np_attention(Kg, Vg, t0, pos, q, gate)
        assert rel_err(got, want) <= 2e-6, (t0, pos, rel_err(got, want))


def test_fast_attention_model_equals_the_c_attention_model(oracle):
    """The oracle's forward with np_attention equals it with the C attention
    within 1e-5 over 40 positions (with the nextn stream), in the plain mode:
    with f16 roundings downstream, attention differences of 1e-6 flip a few
    of them and move the logits by ~1e-4 (the sensitivity the model tests
    measure)."""
    tensors = list(synth.model_tensors(CFG, seed=8, mtp=True))
    toks = synth.prompt_tokens(8, 40, CFG["vocab"])
    ref, ref_d = _logits(oracle, tensors, toks)
    fast, fast_d = _logits(oracle, tensors, toks, fast_attention=True)
    errs = [rel_err(fast[p], ref[p]) for p in range(len(toks))] + [rel_err(fast_d[t], ref_d[t]) for t in range(2)]
    assert max(errs) <= 1e-5, max(errs)
