"""The oracle against fixed vectors of the reference engine's own kernels
(tests/golden/reference_vectors.npz, written by tests/golden/make_golden.py
from run.c compiled in oracle/_ref, AVX2 build).  These run where the
reference tree is absent; the tolerances are those of the live comparisons
in test_oracle.py: bit-exact where the oracle restates a scalar path of the
AVX2 build, else the stated relative error."""
import sys
from pathlib import Path

import numpy as np
import pytest

from util import rel_err

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
import make_golden as mg  # noqa: E402


@pytest.fixture(scope="module")
def gv():
    return np.load(GOLDEN / "reference_vectors.npz")   # no pickles: allow_pickle stays False


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_fixture_is_the_avx2_build(gv):
    assert str(gv["isa"]) == "avx2"


@pytest.mark.parametrize("name,wtype,K", [("rs", 101, 512), ("q8_0", 8, 512)])
def test_gemvb_bit_exact(oracle, gv, name, wtype, K):
    if name == "rs":
        Y = oracle.gemvb(wtype, gv["gemv_rs_qs"], gv["gemv_rs_sc"], K, 32, gv["gemv_X"])
        want = gv["gemv_rs_Y"]
    else:
        Y = oracle.gemvb(wtype, gv["gemv_q8_0"], None, K, 32, gv["gemv_X"])
        want = gv["gemv_q8_0_Y"]
    assert np.array_equal(bits(Y), bits(want))


def test_gemvb_rsi_both_sides_bit_exact(oracle, gv):
    for side in (0, 1):
        Y = oracle.gemvb(102, gv["gemv_rsi_qs"], gv["gemv_rsi_sc"], 512, 32, gv["gemv_X"], side)
        assert np.array_equal(bits(Y), bits(gv[f"gemv_rsi_Y{side}"])), side


def test_gemvb_gguf_and_q6_k(oracle, gv):
    Y = oracle.gemvb(2, gv["gemv_q4_0"], None, 512, 32, gv["gemv_X"])
    assert rel_err(Y, gv["gemv_q4_0_Y"]) < 1e-5
    Y = oracle.gemvb(3, gv["gemv_q4_1"], None, 512, 32, gv["gemv_X"])   # Q4_1: the AVX2 kernel's order
    assert rel_err(Y, gv["gemv_q4_1_Y"]) < 1e-5
    Y = oracle.gemvb(14, gv["gemv_q6_k"], None, 1024, 32, gv["gemv_q6_k_X"])
    assert rel_err(Y, gv["gemv_q6_k_Y"]) < 1e-5
    Y = oracle.gemvb(13, gv["gemv_q5_k"], None, 1024, 32, gv["gemv_q6_k_X"])   # Q5_K: the AVX2 kernel's order
    assert rel_err(Y, gv["gemv_q5_k_Y"]) < 1e-5


def test_silu_mul_and_rmsnorm(oracle, gv):
    a, b, x, w = mg.elementwise_inputs()
    assert np.array_equal(bits(oracle.silu_mul(a, b)), bits(gv["silu_out"]))
    assert rel_err(oracle.rmsnorm(x, w), gv["rms_out"]) < 1e-6


def test_conv1d_update_bit_exact(oracle, gv):
    qkv, hist, kw = mg.conv_inputs()
    q, h = oracle.conv1d_update(qkv, hist.reshape(-1, 3), kw.reshape(-1, 4))
    n = mg.CONV_KEEP
    assert np.array_equal(bits(q[:n]), bits(gv["conv_qkv_out"]))
    assert np.array_equal(bits(h.reshape(-1, 3)[:n]), bits(gv["conv_hist_out"]))


def test_gdn_step(oracle, gv):
    S, qkv, z, decay, beta, wn = mg.gdn_inputs()
    S1, _, o = oracle.gdn_step(S.reshape(mg.NVH, mg.DK, mg.DK), qkv, z, decay, beta, wn, mg.NKH, mg.NVH, mg.DK)
    assert rel_err(o, gv["gdn_out"]) < 1e-5
    assert rel_err(S1.reshape(mg.NVH, mg.DK, mg.DK)[mg.GDN_HEAD], gv["gdn_S_head"]) < 1e-5


def test_argmax_walk_ngram(oracle, gv):
    assert [oracle.argmax(r) for r in mg.argmax_inputs()] == gv["argmax_out"].tolist()
    assert list(oracle.walk(*mg.walk_inputs())) == gv["walk_out"].tolist()
    for nk in (2, 4, 16):
        assert oracle.ngram_draft(mg.NGRAM_HIST, nk, 7).tolist() == gv[f"ngram_out_{nk}"].tolist(), nk


def test_rope_attention_embed(oracle, gv):
    NH, NKV, HD = gv["attn_dims"].tolist()
    q, Kc, Vc, gate = mg.attn_inputs(NH, NKV, HD)
    assert np.array_equal(bits(oracle.rope(q, 123)), bits(gv["rope_out"]))
    assert rel_err(oracle.attention(Kc, Vc, 0, Kc.shape[0] - 1, q, gate), gv["attn_out"]) < 1e-5
    assert np.array_equal(bits(oracle.embed(2, gv["embed_q4_0"], None, 3, 5120)), bits(gv["embed_out"]))
