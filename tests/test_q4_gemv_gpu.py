"""Parity of the HIP Q4_0 batched GEMV (libcwen_gpu.so through its C ABI)
against the oracle, plus the block-invariance property the speculative path
relies on.

Tolerance (stated): rel_err = max|y - y_oracle| / max|y_oracle| <= 1e-3 on
f32 outputs.  The kernel's only rounding beyond f32 accumulation is the f16
activation operand (2^-11 relative per element), which puts the expected
error near 1e-4.
"""
import numpy as np
import pytest

from cwen_amd import synth
from util import rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3
T_Q4_0, T_RS, T_RSI = 2, 101, 102


@pytest.fixture(scope="module")
def env():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from cwen_amd import gpu
    ctx = gpu.Context(0)
    yield torch, gpu, ctx
    torch.cuda.synchronize()


def _run(env, W, X, side=0, mode="single"):
    torch, gpu, ctx = env
    B = X.shape[0]
    Xd = torch.from_numpy(np.ascontiguousarray(X)).cuda()
    if mode == "single":
        Y = torch.full((B, W.M), float("nan"), device="cuda")
        gpu.gemvb(ctx, W, Xd, Y, B, side=side)
        torch.cuda.synchronize()
        return Y.cpu().numpy()
    if mode == "pair":
        YA = torch.full((B, W.M), float("nan"), device="cuda")
        YB = torch.full((B, W.M), float("nan"), device="cuda")
        gpu.gemvb_pair(ctx, W, Xd, YA, YB, B)
        torch.cuda.synchronize()
        return YA.cpu().numpy(), YB.cpu().numpy()
    H = torch.full((B, W.M), float("nan"), device="cuda")
    gpu.gemvb_swiglu(ctx, W, Xd, H, B)
    torch.cuda.synchronize()
    return H.cpu().numpy()


SHAPES = [(16, 512), (20, 1024), (100, 512), (48, 5120), (1024, 1024), (5120, 5120), (48, 65536)]   # K up to CWEN_KMAX


@pytest.mark.parametrize("M,K", SHAPES)
def test_rs_parity(env, oracle, M, K):
    torch, gpu, ctx = env
    qs, sc = synth.q4_rs(101, M, K)
    W = gpu.Weight(ctx, T_RS, qs, sc, K, M)
    for B in (1, 3, 8, 16):
        X = synth.activations(101, B, K, key=B)
        got = _run(env, W, X)
        want = oracle.gemvb(T_RS, qs, sc, K, M, X)
        assert np.isfinite(got).all()
        assert rel_err(got, want) <= TOL, (M, K, B, rel_err(got, want))


@pytest.mark.parametrize("M,K", [(64, 512), (5120, 5120)])
def test_gguf_parity(env, oracle, M, K):
    torch, gpu, ctx = env
    blk = synth.q4_gguf(102, M, K)
    W = gpu.Weight(ctx, T_Q4_0, blk, None, K, M)
    for B in (1, 8):
        X = synth.activations(102, B, K, key=B)
        got = _run(env, W, X)
        assert rel_err(got, oracle.gemvb(T_Q4_0, blk, None, K, M, X)) <= TOL


@pytest.mark.parametrize("M,K", [(40, 512), (1000, 2048)])
def test_rsi_single_pair_swiglu(env, oracle, M, K):
    torch, gpu, ctx = env
    qs, sc = synth.q4_rsi(103, M, K)
    W = gpu.Weight(ctx, T_RSI, qs, sc, K, M)
    for B in (1, 5, 16):
        X = synth.activations(103, B, K, key=B)
        wa = oracle.gemvb(T_RSI, qs, sc, K, M, X, side=0)
        wb = oracle.gemvb(T_RSI, qs, sc, K, M, X, side=1)
        assert rel_err(_run(env, W, X, side=0), wa) <= TOL
        assert rel_err(_run(env, W, X, side=1), wb) <= TOL
        ya, yb = _run(env, W, X, mode="pair")
        assert rel_err(ya, wa) <= TOL and rel_err(yb, wb) <= TOL
        h = _run(env, W, X, mode="swiglu")
        assert rel_err(h, oracle.silu_mul(wa, wb)) <= TOL


def test_block_invariance_bitwise(env):
    """A column computed inside a block of B is bit-identical to the same
    column computed alone (B=1) and inside a different block size."""
    torch, gpu, ctx = env
    M, K = 5120, 17408
    qs, sc = synth.q4_rs(104, M, K)
    W = gpu.Weight(ctx, T_RS, qs, sc, K, M)
    X = synth.activations(104, 16, K)
    full = _run(env, W, X)
    for b in (0, 5, 15):
        one = _run(env, W, X[b:b + 1])
        assert np.array_equal(one[0].view(np.uint32), full[b].view(np.uint32))
    eight = _run(env, W, X[3:11])
    assert np.array_equal(eight.view(np.uint32), full[3:11].view(np.uint32))


def test_pair_invariance_bitwise(env):
    torch, gpu, ctx = env
    M, K = 2048, 5120
    qs, sc = synth.q4_rsi(105, M, K)
    W = gpu.Weight(ctx, T_RSI, qs, sc, K, M)
    X = synth.activations(105, 16, K)
    h16 = _run(env, W, X, mode="swiglu")
    h1 = _run(env, W, X[7:8], mode="swiglu")
    assert np.array_equal(h1[0].view(np.uint32), h16[7].view(np.uint32))
    ya, _ = _run(env, W, X, mode="pair")
    assert np.array_equal(_run(env, W, X, side=0).view(np.uint32), ya.view(np.uint32))


def test_repeat_deterministic(env):
    torch, gpu, ctx = env
    M, K = 5120, 17408
    qs, sc = synth.q4_rs(106, M, K)
    W = gpu.Weight(ctx, T_RS, qs, sc, K, M)
    X = synth.activations(106, 8, K)
    a = _run(env, W, X)
    for _ in range(3):
        assert np.array_equal(_run(env, W, X).view(np.uint32), a.view(np.uint32))


def test_strided_activations_and_outputs(env, oracle):
    torch, gpu, ctx = env
    M, K, B = 96, 512, 4
    qs, sc = synth.q4_rs(107, M, K)
    W = gpu.Weight(ctx, T_RS, qs, sc, K, M)
    X = synth.activations(107, B, K)
    Xpad = np.zeros((B, K + 64), np.float32)
    Xpad[:, :K] = X
    Xd = torch.from_numpy(Xpad).cuda()
    Y = torch.full((B, M + 32), 7.0, device="cuda")
    gpu.gemvb(ctx, W, Xd, Y, B, xs=K + 64, ys=M + 32)
    torch.cuda.synchronize()
    Yh = Y.cpu().numpy()
    assert rel_err(Yh[:, :M], oracle.gemvb(T_RS, qs, sc, K, M, X)) <= TOL
    assert np.all(Yh[:, M:] == 7.0)  # nothing written past M


def test_argument_errors(env):
    torch, gpu, ctx = env
    M, K = 32, 512
    qs, sc = synth.q4_rs(108, M, K)
    W = gpu.Weight(ctx, T_RS, qs, sc, K, M)
    X = torch.zeros(17, K, device="cuda")
    Y = torch.zeros(17, M, device="cuda")
    for B in (0, 17):
        with pytest.raises(gpu.CwenError):
            gpu.gemvb(ctx, W, X, Y, B)
    with pytest.raises(gpu.CwenError):
        gpu.gemvb(ctx, W, X.data_ptr() + 4, Y, 1)          # misaligned activations
    with pytest.raises(gpu.CwenError):
        gpu.gemvb(ctx, W, X, Y, 1, side=1)                 # RS has one side
    with pytest.raises(gpu.CwenError):
        gpu.gemvb_swiglu(ctx, W, X, Y, 1)                  # needs a pair
    qs2, sc2 = synth.q4_rs(108, M, 96)
    with pytest.raises(gpu.CwenError):
        gpu.Weight(ctx, T_RS, qs2, sc2, 80, M)             # K not whole 32-weight blocks
    with pytest.raises(gpu.CwenError):
        gpu.Weight(ctx, gpu.T_Q6_K, synth.q6_k(108, M, 512), None, 288, M)   # K-quant: whole 256s
    with pytest.raises(gpu.CwenError):
        gpu.Weight(ctx, 1, qs, sc, K, M)                   # F16 is not a supported type
    qs3, sc3 = synth.q4_rs(108, M, 65536 + 32)
    with pytest.raises(gpu.CwenError):
        gpu.Weight(ctx, T_RS, qs3, sc3, 65536 + 32, M)     # K past CWEN_KMAX


@pytest.mark.slow
def test_ffn_block_full_size(env, oracle):
    """The FFN workload at full size, B=8: RSI gate/up + SwiGLU, then RS down."""
    torch, gpu, ctx = env
    H, I, B = 5120, 17408, 8
    gq, gs = synth.q4_rsi(0, I, H)
    dq, ds = synth.q4_rs(0, H, I, key=1)
    X = synth.activations(0, B, H)
    Wgu = gpu.Weight(ctx, T_RSI, gq, gs, H, I)
    Wd = gpu.Weight(ctx, T_RS, dq, ds, I, H)
    Xd = torch.from_numpy(X).cuda()
    Hd = torch.empty(B, I, device="cuda")
    Yd = torch.empty(B, H, device="cuda")
    gpu.gemvb_swiglu(ctx, Wgu, Xd, Hd, B)
    gpu.gemvb(ctx, Wd, Hd, Yd, B)
    torch.cuda.synchronize()
    h_want = oracle.silu_mul(oracle.gemvb(T_RSI, gq, gs, H, I, X, 0), oracle.gemvb(T_RSI, gq, gs, H, I, X, 1))
    assert rel_err(Hd.cpu().numpy(), h_want) <= TOL
    y_want = oracle.gemvb(T_RS, dq, ds, I, H, h_want)
    assert rel_err(Yd.cpu().numpy(), y_want) <= TOL


@pytest.mark.parametrize("H,I", [(1024, 2048), (1024, 9216), (5120, 17408)])
def test_mlp_block(env, oracle, H, I):
    """cwen_mlp_block (f32 in, Y += down(SwiGLU(gate/up X))) is
    bit-identical to the f16 entry points run one by one (f32 -> f16,
    SwiGLU GEMV, accumulating down GEMV), repeats exactly, and matches the
    oracle's mlp_blk within TOL.  The shapes cover split gate/up tiles
    (2048), whole tiles plus split remainder tiles (9216: 288 tiles) and the
    27B FFN."""
    torch, gpu, ctx = env
    gq, gs = synth.q4_rsi(110, I, H)
    dq, ds = synth.q4_rs(110, H, I, key=1)
    Wgu = gpu.Weight(ctx, T_RSI, gq, gs, H, I)
    Wd = gpu.Weight(ctx, T_RS, dq, ds, I, H)
    for B in (1, 5, 8, 16):
        X = synth.activations(110, B, H, key=B)
        Y0 = synth.activations(111, B, H, key=B)
        Xd = torch.from_numpy(X).cuda()
        Xh = torch.empty(B, H, dtype=torch.float16, device="cuda")
        Hh = torch.empty(B, I, dtype=torch.float16, device="cuda")
        ref = torch.from_numpy(Y0).cuda()
        gpu.act_to_f16(ctx, Xd, Xh, H, B)
        gpu.gemvb_swiglu_f16(ctx, Wgu, Xh, None, B, Hh=Hh)
        gpu.gemvb_f16(ctx, Wd, Hh, ref, B, accumulate=True)
        ref = ref.cpu().numpy()
        for rep in range(2):
            Y = torch.from_numpy(Y0).cuda()
            gpu.mlp_block(ctx, Wgu, Wd, Xd, Y, B)
            torch.cuda.synchronize()
            got = Y.cpu().numpy()
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (B, rep)
        if B == 8:
            h = oracle.silu_mul(oracle.gemvb(T_RSI, gq, gs, H, I, X, 0), oracle.gemvb(T_RSI, gq, gs, H, I, X, 1))
            assert rel_err(got - Y0, oracle.gemvb(T_RS, dq, ds, I, H, h)) <= TOL


@pytest.mark.parametrize("M,K", [(16, 512), (100, 1024), (5120, 17408)])
def test_q4_1_parity(env, oracle, M, K):
    """Q4_1 (GGUF {d, m, qs}, w = n*d + m; the real model's ffn_down type):
    the same GEMV kernel with its own dequant, vs the oracle's dot_q4_1 within
    TOL, at the 27B down shape too; a column is bit-identical alone and
    inside a block."""
    torch, gpu, ctx = env
    blk = synth.q4_1(109, M, K)
    W = gpu.Weight(ctx, gpu.T_Q4_1, blk, None, K, M)
    X = synth.activations(109, 16, K)
    full = None
    for B in (1, 5, 8, 16):
        got = _run(env, W, X[:B])
        assert rel_err(got, oracle.gemvb(gpu.T_Q4_1, blk, None, K, M, X[:B])) <= TOL, B
        if B == 16:
            full = got
    one = _run(env, W, X[9:10])
    assert np.array_equal(one[0].view(np.uint32), full[9].view(np.uint32))


@pytest.mark.parametrize("M,K", [(16, 512), (100, 1024), (5120, 6144)])
def test_q5_k_parity(env, oracle, M, K):
    """Q5_K (the real model's ssm_out type, here at its 5120 x 6144 shape):
    the low nibbles in the Q4_0 layout, the fifth bits ORed in by the unpack,
    (d*sc, -dmin*m) per sub-block rounded to f16 at upload.  Within TOL of
    the oracle's dot_q5_K; a column is bit-identical alone and in a block."""
    torch, gpu, ctx = env
    blk = synth.q5_k(110, M, K)
    W = gpu.Weight(ctx, gpu.T_Q5_K, blk, None, K, M)
    X = synth.activations(110, 16, K)
    full = None
    for B in (1, 5, 8, 16):
        got = _run(env, W, X[:B])
        assert rel_err(got, oracle.gemvb(gpu.T_Q5_K, blk, None, K, M, X[:B])) <= TOL, B
        if B == 16:
            full = got
    one = _run(env, W, X[4:5])
    assert np.array_equal(one[0].view(np.uint32), full[4].view(np.uint32))


RAGGED = [("rs", 32), ("rs", 96), ("rs", 544), ("rs", 5152), ("q4_0", 480), ("rsi", 1056), ("q8_0", 608),
          ("q4_1", 800), ("q6_k", 256), ("q6_k", 768), ("q5_k", 1280)]


@pytest.mark.parametrize("kind,K", RAGGED)
def test_k_multiple_of_32(env, oracle, kind, K):
    """K in whole blocks but not a multiple of the device's 512-wide tiles,
    as the reference accepts (run.c:1293-1306): the last super-tile is
    zero-padded and the activations past K read as zeros.  Parity vs the
    oracle within TOL for B = 1, 5, 16, a column bit-identical alone and in
    a block, and column 0 unaffected by an infinite first element of column
    1 (which lies right after column 0's last element: a read past K would
    turn column 0's padded products into NaN)."""
    torch, gpu, ctx = env
    M = 40
    if kind == "rs":
        data, sc = synth.q4_rs(111, M, K); wtype = T_RS
    elif kind == "rsi":
        data, sc = synth.q4_rsi(111, M, K); wtype = T_RSI
    elif kind == "q4_0":
        data, sc = synth.q4_gguf(111, M, K), None; wtype = T_Q4_0
    elif kind == "q8_0":
        data, sc = synth.q8_0(111, M, K), None; wtype = gpu.T_Q8_0
    elif kind == "q4_1":
        data, sc = synth.q4_1(111, M, K), None; wtype = gpu.T_Q4_1
    elif kind == "q6_k":
        data, sc = synth.q6_k(111, M, K), None; wtype = gpu.T_Q6_K
    else:
        data, sc = synth.q5_k(111, M, K), None; wtype = gpu.T_Q5_K
    W = gpu.Weight(ctx, wtype, data, sc, K, M)
    X = synth.activations(111, 16, K)
    full = None
    for B in (1, 5, 16):
        got = _run(env, W, X[:B])
        want = oracle.gemvb(wtype, data, sc, K, M, X[:B])
        assert np.isfinite(got).all()
        assert rel_err(got, want) <= TOL, (kind, K, B, rel_err(got, want))
        if B == 16:
            full = got
    one = _run(env, W, X[11:12])
    assert np.array_equal(one[0].view(np.uint32), full[11].view(np.uint32))
    if kind == "rsi":
        ya, yb = _run(env, W, X[:5], mode="pair")
        wa, wb = oracle.gemvb(T_RSI, data, sc, K, M, X[:5], 0), oracle.gemvb(T_RSI, data, sc, K, M, X[:5], 1)
        assert rel_err(ya, wa) <= TOL and rel_err(yb, wb) <= TOL
        assert rel_err(_run(env, W, X[:5], mode="swiglu"), oracle.silu_mul(wa, wb)) <= TOL
    Xi = X[:2].copy()
    Xi[1, 0] = np.inf
    got = _run(env, W, Xi)
    assert np.isfinite(got[0]).all()
    assert np.array_equal(got[0].view(np.uint32), full[0].view(np.uint32))


ELEM_CASES = [("rs", 5120), ("rsi", 5120), ("q4_0", 5120), ("q8_0", 5120), ("q4_1", 5120), ("q5_k", 6144),
              ("q6_k", 5120), ("rs", 17408)]


@pytest.mark.parametrize("kind,K", ELEM_CASES)
def test_elementwise_error_bound(env, kind, K):
    """Every output element within a rounding bound of its own exact value
    (float64 from the block definitions, tests/dequant.py, which the
    oracle's tests pin) instead of a norm-wise tolerance; the bound and its
    derivation are tests/elembound.py's.  The bound has teeth: leaving out
    one 32-weight block breaks it for half of the elements or more, flipping
    one weight's sign for a sixth or more (test_oracle.py's
    test_elementwise_bound_has_teeth)."""
    from elembound import elem_bound, elem_case
    torch, gpu, ctx = env
    M = 256
    wtype, data, sc, side, Wx, A, cw = elem_case(kind, K, M)
    W = gpu.Weight(ctx, wtype, data, sc, K, M)
    X = synth.activations(121, 16, K)
    X[:, ::97] *= 1e-6      # some activations below f16's normal range
    worst = 0.0
    for B in (1, 8, 16):
        got = _run(env, W, X[:B], side=side).astype(np.float64)
        exact = X[:B].astype(np.float64) @ Wx.T
        r = np.abs(got - exact) / elem_bound(Wx, A, X[:B], K, cw)
        assert (r <= 1).all(), (kind, K, B, float(r.max()))
        worst = max(worst, float(r.max()))
    print(f"{kind} K={K}: worst error / bound {worst:.3f}")
