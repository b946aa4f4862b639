"""Pins the oracle (oracle/cwen_oracle.c) before anything is checked against it.

Each oracle function is checked three ways where possible:
  * against the reference engine's own kernels compiled from its run.c
    (oracle/_ref): bit-exact where the reference AVX2 build runs the same
    scalar code path (RS/RSI/Q8_0 dots, silu_mul, conv), within f32
    reassociation tolerance where it runs SIMD (GGUF Q4_0, Q6_K, rmsnorm,
    GDN);
  * against an independent numpy float64 decode on tiny shapes;
  * against closed forms / invariants (numpy's float16 conversion, argmax
    semantics, GDN identities).
CPU only.
"""
import numpy as np
import pytest

from cwen_amd import synth
import dequant as D
from util import q6_k_pack, rel_err

T_Q4_0, T_Q4_1, T_Q8_0, T_Q5_K, T_Q6_K, T_RS, T_RSI = 2, 3, 8, 13, 14, 101, 102


# ---------------------------------------------------------------- f16
def test_f16_to_f32_exhaustive(oracle):
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.L.orc_f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_rne(oracle):
    g = np.random.default_rng(7)
    x = np.concatenate([
        g.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** g.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504.0, 65520.0, 1e9, -1e9, np.inf, -np.inf, 5.96e-8, 2.98e-8,
                  2.99e-8, 1e-8, 6.1e-5, 6.09e-5], dtype=np.float32),
        # exact halfway points between adjacent halves (ties to even)
        ((np.arange(1024, 2048, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -10)),
    ]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    got = np.array([oracle.L.orc_f32_to_f16(float(v)) for v in x], dtype=np.uint16)
    assert np.array_equal(got, want)
    assert oracle.L.orc_f32_to_f16(float("nan")) & 0x7e00 == 0x7e00


# ---------------------------------------------------------------- dequant (numpy f64, tests/dequant.py)
SMALL = [(64, 256), (48, 512)]


@pytest.mark.parametrize("M,K", SMALL)
def test_q4_rs_vs_f64(oracle, M, K):
    qs, sc = synth.q4_rs(11, M, K)
    X = synth.activations(11, 3, K)
    W = D.rs(qs, sc, M, K)
    want = X.astype(np.float64) @ W.T
    got = oracle.gemvb(T_RS, qs, sc, K, M, X)
    assert rel_err(got, want) < 2e-6


@pytest.mark.parametrize("side", [0, 1])
def test_q4_rsi_vs_f64(oracle, side):
    M, K = 40, 256
    qs, sc = synth.q4_rsi(12, M, K)
    X = synth.activations(12, 2, K)
    q1, s1 = synth.rsi_side(qs, sc, M, K, side)
    W = D.rs(q1, s1, M, K)
    got = oracle.gemvb(T_RSI, qs, sc, K, M, X, side=side)
    assert rel_err(got, X.astype(np.float64) @ W.T) < 2e-6


def test_q4_gguf_vs_f64(oracle):
    M, K = 32, 512
    blk = synth.q4_gguf(13, M, K)
    W = D.q4_0(blk, M, K)
    X = synth.activations(13, 2, K)
    got = oracle.gemvb(T_Q4_0, blk, None, K, M, X)
    assert rel_err(got, X.astype(np.float64) @ W.T) < 2e-6


def test_q4_1_vs_f64(oracle):
    """Q4_1 blocks {d, m, qs}: w = n*d + m, lo nibbles -> w[0..15], hi -> w[16..31]."""
    M, K = 24, 512
    blk = synth.q4_1(16, M, K)
    W = D.q4_1(blk, M, K)[0]
    X = synth.activations(16, 2, K)
    got = oracle.gemvb(T_Q4_1, blk, None, K, M, X)
    assert rel_err(got, X.astype(np.float64) @ W.T) < 2e-6


def test_q5_k_vs_f64(oracle):
    """Q5_K from the GGUF block definition in f64 (6-bit scale/min unpacking
    as ggml defines it, 5-bit quants split over qs nibbles and qh bits)."""
    M, K = 4, 512
    blk = synth.q5_k(17, M, K)
    W = D.q5_k(blk, M, K)[0]
    X = synth.activations(17, 2, K)
    got = oracle.gemvb(T_Q5_K, blk, None, K, M, X)
    assert rel_err(got, X.astype(np.float64) @ W.T) < 2e-6


def test_q8_0_vs_f64(oracle):
    M, K = 24, 256
    blk = synth.q8_0(14, M, K)
    W = D.q8_0(blk, M, K)
    X = synth.activations(14, 2, K)
    got = oracle.gemvb(T_Q8_0, blk, None, K, M, X)
    assert rel_err(got, X.astype(np.float64) @ W.T) < 2e-6


def test_q6_k_vs_f64(oracle):
    M, K = 6, 512
    blk = synth.q6_k(15, M, K)
    W = D.q6_k(blk, M, K)
    X = synth.activations(15, 2, K)
    got = oracle.gemvb(T_Q6_K, blk, None, K, M, X)
    assert rel_err(got, X.astype(np.float64) @ W.T) < 2e-6


# ---------------------------------------------------------------- vs reference kernels
@pytest.mark.parametrize("wtype", [T_RS, T_RSI, T_Q8_0])
def test_scalar_paths_bit_exact_vs_reference_avx2(oracle, ref_avx2, wtype):
    """The reference AVX2 build runs these dots on its scalar path: same bits."""
    M, K, B = 96, 1024, 4
    if wtype == T_RS:
        data, sc = synth.q4_rs(21, M, K)
    elif wtype == T_RSI:
        data, sc = synth.q4_rsi(21, M, K)
    else:
        data, sc = synth.q8_0(21, M, K), None
    X = synth.activations(21, B, K)
    for side in ([0, 1] if wtype == T_RSI else [0]):
        want = ref_avx2.gemvb(wtype, data, sc, K, M, X, side=side)
        got = oracle.gemvb(wtype, data, sc, K, M, X, side=side)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("isa", ["avx2", "avx512"])
@pytest.mark.parametrize("wtype", [T_Q4_0, T_Q4_1, T_RS, T_RSI, T_Q8_0, T_Q5_K, T_Q6_K])
def test_gemvb_vs_reference(oracle, isa, wtype):
    from oracle.binding import Reference, ref_lib_path, cpu_has_avx512
    if not ref_lib_path(isa).exists():
        pytest.skip("reference checker build absent")
    if isa == "avx512" and not cpu_has_avx512():
        pytest.skip("host lacks AVX-512")
    R = Reference(isa)
    M, K = 80, 2048
    if wtype == T_Q4_0:
        data, sc = synth.q4_gguf(22, M, K), None
    elif wtype == T_RS:
        data, sc = synth.q4_rs(22, M, K)
    elif wtype == T_RSI:
        data, sc = synth.q4_rsi(22, M, K)
    elif wtype == T_Q8_0:
        data, sc = synth.q8_0(22, M, K), None
    elif wtype == T_Q4_1:
        data, sc = synth.q4_1(22, M, K), None
    elif wtype == T_Q5_K:
        data, sc = synth.q5_k(22, M, K), None
    else:
        data, sc = synth.q6_k(22, M, K), None
    for B in (1, 3, 8, 16):
        X = synth.activations(22, B, K, key=B)
        for side in ([0, 1] if wtype == T_RSI else [0]):
            want = R.gemvb(wtype, data, sc, K, M, X, side=side)
            got = oracle.gemvb(wtype, data, sc, K, M, X, side=side)
            assert rel_err(got, want) < 1e-5, (B, side)


def test_silu_mul_bit_exact(oracle, ref_avx2):
    g = np.random.default_rng(3)
    a = (g.standard_normal(4099) * 4).astype(np.float32)
    b = g.standard_normal(4099).astype(np.float32)
    assert np.array_equal(oracle.silu_mul(a, b).view(np.uint32), ref_avx2.silu_mul(a, b).view(np.uint32))


def test_silu_closed_form(oracle):
    x = np.linspace(-30, 30, 1001).astype(np.float32)
    one = np.ones_like(x)
    got = oracle.silu_mul(x, one).astype(np.float64)
    xd = x.astype(np.float64)
    assert np.max(np.abs(got - xd / (1 + np.exp(-xd)))) < 1e-5


def test_rmsnorm_vs_reference(oracle, ref):
    g = np.random.default_rng(4)
    x = g.standard_normal(5120).astype(np.float32)
    w = (1 + 0.1 * g.standard_normal(5120)).astype(np.float32)
    assert rel_err(oracle.rmsnorm(x, w), ref.rmsnorm(x, w)) < 1e-6
    xd = x.astype(np.float64)
    want = w * xd / np.sqrt(np.mean(xd * xd) + 1e-6)
    assert rel_err(oracle.rmsnorm(x, w), want) < 1e-6


def test_conv1d_bit_exact(oracle, ref_avx2):
    C = 10240
    g = np.random.default_rng(5)
    qkv = g.standard_normal(C).astype(np.float32)
    hist = g.standard_normal((C, 3)).astype(np.float32)
    kw = (0.5 * g.standard_normal((C, 4))).astype(np.float32)
    o1, h1 = oracle.conv1d_update(qkv, hist, kw)
    o2, h2 = ref_avx2.conv1d_update(qkv, hist, kw)
    assert np.array_equal(o1.view(np.uint32), o2.view(np.uint32))
    assert np.array_equal(h1, h2)
    # the history shifts by one and takes the raw input
    assert np.array_equal(h1[:, :2], hist[:, 1:]) and np.array_equal(h1[:, 2], qkv)


def _gdn_inputs(seed):
    g = np.random.default_rng(seed)
    S = (0.01 * g.standard_normal((48, 128, 128))).astype(np.float32)
    qkv = g.standard_normal(10240).astype(np.float32)
    z = g.standard_normal(6144).astype(np.float32)
    decay = np.log(g.uniform(0.05, 1.0, 48)).astype(np.float32)
    beta = (1 / (1 + np.exp(-g.standard_normal(48)))).astype(np.float32)
    wn = (1 + 0.1 * g.standard_normal(128)).astype(np.float32)
    return S, qkv, z, decay, beta, wn


@pytest.mark.parametrize("isa", ["avx2", "avx512"])
def test_gdn_step_vs_reference(oracle, isa):
    from oracle.binding import Reference, ref_lib_path, cpu_has_avx512
    if not ref_lib_path(isa).exists():
        pytest.skip("reference checker build absent")
    if isa == "avx512" and not cpu_has_avx512():
        pytest.skip("host lacks AVX-512")
    R = Reference(isa)
    S, qkv, z, decay, beta, wn = _gdn_inputs(6)
    S1, q1, o1 = oracle.gdn_step(S, qkv, z, decay, beta, wn, 16, 48, 128)
    S2, q2, o2 = R.gdn_step(S, qkv, z, decay, beta, wn)
    assert rel_err(S1, S2) < 1e-5
    assert rel_err(q1, q2) < 1e-6
    assert rel_err(o1, o2) < 1e-5


def test_gdn_step_closed_form(oracle):
    """f64 restatement of the delta rule on a tiny head: S'=gS + k(beta(v - (gS)^T k))^T."""
    g = np.random.default_rng(8)
    nkh, nvh, dk = 2, 4, 8
    S = g.standard_normal((nvh, dk, dk)).astype(np.float32)
    qkv = g.standard_normal((2 * nkh + nvh) * dk).astype(np.float32)
    z = g.standard_normal(nvh * dk).astype(np.float32)
    decay = np.log(g.uniform(0.3, 1, nvh)).astype(np.float32)
    beta = g.uniform(0, 1, nvh).astype(np.float32)
    wn = g.uniform(0.5, 1.5, dk).astype(np.float32)
    S1, _, out = oracle.gdn_step(S, qkv, z, decay, beta, wn, nkh, nvh, dk)
    q = qkv[:nkh * dk].reshape(nkh, dk).astype(np.float64)
    k = qkv[nkh * dk:2 * nkh * dk].reshape(nkh, dk).astype(np.float64)
    v = qkv[2 * nkh * dk:].reshape(nvh, dk).astype(np.float64)
    q /= np.sqrt((q * q).sum(1, keepdims=True) + 1e-6)
    k /= np.sqrt((k * k).sum(1, keepdims=True) + 1e-6)
    for hv in range(nvh):
        hk = hv % nkh
        Sh = S[hv].astype(np.float64) * np.exp(float(decay[hv]))
        delta = float(beta[hv]) * (v[hv] - Sh.T @ k[hk])
        Sh = Sh + np.outer(k[hk], delta)
        assert np.allclose(S1[hv], Sh, rtol=1e-5, atol=1e-5)
        o = (Sh.T @ q[hk]) / np.sqrt(dk)
        zz = z[hv * dk:(hv + 1) * dk].astype(np.float64)
        o = wn * o / np.sqrt(np.mean(o * o) + 1e-6) * zz / (1 + np.exp(-zz))
        assert np.allclose(out[hv * dk:(hv + 1) * dk], o, rtol=1e-4, atol=1e-5)


def test_gdn_identity_gates(oracle):
    """decay = 0 (g = 1) and beta = 0 leave the state unchanged."""
    S, qkv, z, decay, beta, wn = _gdn_inputs(9)
    S1, _, _ = oracle.gdn_step(S, qkv, z, np.zeros(48, np.float32), np.zeros(48, np.float32), wn, 16, 48, 128)
    assert np.array_equal(S1, S)


# ---------------------------------------------------------------- argmax / walk / drafter
def test_argmax_semantics(oracle, ref):
    g = np.random.default_rng(10)
    V = 151936
    for t in range(20):
        lg = g.standard_normal(V).astype(np.float32)
        if t % 4 == 1:
            lg[g.integers(0, V, 5)] = lg.max()                   # ties: first index wins
        if t % 4 == 2:
            lg[g.integers(1, V, 50)] = np.nan                     # NaN never wins
        if t % 4 == 3:
            lg[:] = -np.inf
        want_np = int(np.nanargmax(lg)) if not np.all(np.isneginf(lg)) else 0
        a = oracle.argmax(lg)
        assert a == ref.argmax(lg) == want_np
    lg = g.standard_normal(1000).astype(np.float32)
    lg[0] = np.nan                                                # NaN at 0: nothing beats it
    assert oracle.argmax(lg) == ref.argmax(lg) == 0


def test_walk_vs_reference(oracle, ref):
    g = np.random.default_rng(11)
    V = 151936
    for E in (0, 1, 3, 7, 15):
        logits = g.standard_normal((E + 1, V)).astype(np.float32)
        am = logits.argmax(1)
        for trial in range(4):
            d = np.where(g.random(E) < 0.7, am[:E], g.integers(0, V, E)).astype(np.int32)
            assert oracle.walk(logits, d) == ref.walk(logits, d)


def test_ngram_draft_vs_reference(oracle, ref):
    g = np.random.default_rng(12)
    for t in range(30):
        base = g.integers(0, 50, g.integers(20, 80))
        hist = np.concatenate([base, base[: g.integers(5, len(base))], g.integers(0, 50, 3), base[:20]])
        hist = hist.astype(np.int32)
        for n_key in (2, 4, 16):
            for max_d in (1, 7, 15):
                assert np.array_equal(oracle.ngram_draft(hist, n_key, max_d), ref.ngram_draft(hist, n_key, max_d))


# ---------------------------------------------------------------- model glue
def test_embed_vs_reference_and_closed_form(oracle, ref_avx2):
    from cwen_amd import synth
    V = ref_avx2.vocab
    H = 5120
    qs, sc = synth.q4_rs(0, 64, H, key=9)          # 64 token rows are enough to index
    # the reference indexes a [V][H] table; give it a full-size view of zeros past row 63
    qfull = np.zeros((V, H // 32, 16), np.uint8)
    sfull = np.zeros((V, H // 32), np.uint16)
    qfull[:64] = qs.reshape(64, H // 32, 16)
    sfull[:64] = sc.reshape(64, H // 32)
    for tok in (0, 7, 63):
        a = oracle.embed(101, qfull, sfull, tok, H)
        b = ref_avx2.embed(101, qfull, sfull, tok)
        assert np.array_equal(a, b)
        # closed form: (n - 8) * d, low nibbles first
        q = qfull[tok].astype(np.int32)
        d = sfull[tok].view(np.float16).astype(np.float32)
        want = np.concatenate([(q & 15) - 8, (q >> 4) - 8], axis=1).astype(np.float32) * d[:, None]
        assert np.array_equal(a, want.reshape(-1))
    g = synth.q4_gguf(0, 64, H, key=3)
    gfull = np.zeros((V, H // 32 * 18), np.uint8)
    gfull[:64] = g.reshape(64, -1)
    assert np.array_equal(oracle.embed(2, gfull, None, 5, H), ref_avx2.embed(2, gfull, None, 5))


def test_embed_q6_k_vs_reference_and_gemv(oracle, ref_avx2):
    """Q6_K embedding rows (run.c:1829-1848, 1882-1883) against run.c's own
    embed_token_to, and against the Q6_K GEMV already pinned to run.c: a
    row's embedding dotted with a one-hot x is that row's weight, so the
    two unpackings of the same super-blocks must agree element for element."""
    from cwen_amd import synth
    V = ref_avx2.vocab
    H = 5120
    rows = synth.q6_k(0, 64, H, key=17)
    full = np.zeros((V, H // 256 * 210), np.uint8)
    full[:64] = rows.reshape(64, -1)
    for tok in (0, 9, 63):
        a = oracle.embed(T_Q6_K, full, None, tok, H)
        assert np.array_equal(a, ref_avx2.embed(T_Q6_K, full, None, tok))
    # closed form in natural order, from values packed by an independent
    # writer of the layout: (d * sc) * (q - 32)
    g = np.random.default_rng(5)
    q6 = g.integers(0, 64, (3, H)).astype(np.uint8)
    sc = g.integers(-128, 128, (3, H // 16)).astype(np.int8)
    d = np.abs(g.standard_normal((3, H // 256)) * 0.01).astype(np.float16)
    packed = np.zeros((V, H // 256 * 210), np.uint8)
    packed[:3] = q6_k_pack(q6, sc, d.view(np.uint16))
    for r in range(3):
        want = (np.repeat(d[r].astype(np.float32), 256) * np.repeat(sc[r].astype(np.float32), 16)) \
            * (q6[r].astype(np.float32) - 32)
        assert np.array_equal(oracle.embed(T_Q6_K, packed, None, r, H), want)
    tok = 9
    a = oracle.embed(T_Q6_K, full, None, tok, H)
    for k in (0, 31, 32, 100, 127, 128, 200, 255, 256, 4097, H - 1):
        x = np.zeros(H, np.float32)
        x[k] = 1.0
        y = oracle.gemvb(T_Q6_K, full[:64].reshape(-1), None, H, 64, x[None])
        assert y[0, tok] == a[k], (k, y[0, tok], a[k])


@pytest.mark.parametrize("pos", [0, 1, 17, 4095, 8191])
def test_rope_vs_reference(oracle, ref, pos):
    g = np.random.default_rng(pos)
    q = g.standard_normal((24, 256)).astype(np.float32)
    a = oracle.rope(q, pos)
    b = ref.rope(q, pos)
    assert np.array_equal(a, b)
    assert np.array_equal(a[:, 64:], q[:, 64:])          # only the first 32 pairs rotate
    # rotation preserves each pair's norm
    n0 = q[:, :64].reshape(24, 32, 2)
    n1 = a[:, :64].reshape(24, 32, 2)
    assert np.allclose((n0 ** 2).sum(-1), (n1 ** 2).sum(-1), rtol=1e-5)


def test_attention_vs_reference_and_f64(oracle, ref):
    nh, nkv, hd = ref.attn_dims()
    g = np.random.default_rng(21)
    T = 37
    K = g.standard_normal((T, nkv, hd)).astype(np.float32)
    V = g.standard_normal((T, nkv, hd)).astype(np.float32)
    q = g.standard_normal((nh, hd)).astype(np.float32)
    gate = g.standard_normal((nh, hd)).astype(np.float32)
    for t0, pos in ((0, 0), (0, 36), (5, 20)):
        a = oracle.attention(K, V, t0, pos, q, gate)
        b = ref.attention(K, V, t0, pos, q, gate)
        assert rel_err(a, b) < 1e-5
        # f64 softmax attention
        kvm = nh // nkv
        want = np.zeros((nh, hd))
        for h in range(nh):
            k = K[t0:pos + 1, h // kvm].astype(np.float64)
            v = V[t0:pos + 1, h // kvm].astype(np.float64)
            s = k @ q[h].astype(np.float64) / np.sqrt(hd)
            p = np.exp(s - s.max())
            p /= p.sum()
            want[h] = (p @ v) / (1 + np.exp(-gate[h].astype(np.float64)))
        assert rel_err(a, want) < 1e-5


@pytest.mark.parametrize("kind", ["rs", "q4_0", "q8_0", "q4_1", "q5_k", "q6_k"])
def test_elementwise_bound_has_teeth(kind):
    """The GPU tests' element-wise bound (tests/elembound.py) is not
    vacuous: exact outputs with one 32-weight block left out fall outside it
    for about half of the elements or more (measured 52-81 %), and with a
    single weight's sign flipped for a sixth or more (19-53 %)."""
    from elembound import elem_bound, elem_case
    K, M = (5120 if kind != "q5_k" else 6144), 256
    _, _, _, _, W, A, cw = elem_case(kind, K, M)
    X = synth.activations(121, 8, K).astype(np.float64)
    bound = elem_bound(W, A, X, K, cw)
    blk = slice(37 * 32, 38 * 32)
    assert (np.abs(X[:, blk] @ W[:, blk].T) > bound).mean() > 0.45
    assert (np.abs(2 * X[:, 100:101] * W[:, 100][None, :]) > bound).mean() > 0.15
