"""Parity of the HIP Q6_K / Q8_0 batched GEMV and of the on-device LM-head
acceptance (per-column argmax + greedy prefix walk) against the oracle.

Tolerances (stated):
  * GEMV outputs: rel_err = max|y - y_oracle| / max|y_oracle| <= 1e-3.
  * argmax, k and bonus: bit-exact, given the same logits.  The head entry
    point is checked against the oracle's argmax/walk applied to the logits the
    GPU itself produced, and the logits-only entry point against the oracle on
    identical inputs, including ties, NaN, signed zeros and infinities.
"""
import numpy as np
import pytest

from cwen_amd import synth
from util import rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3
T_Q8_0, T_Q6_K = 8, 14


@pytest.fixture(scope="module")
def env():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from cwen_amd import gpu
    ctx = gpu.Context(0)
    yield torch, gpu, ctx
    torch.cuda.synchronize()


def _weights(wtype, M, K, key=0):
    return synth.q6_k(0, M, K, key=key) if wtype == T_Q6_K else synth.q8_0(0, M, K, key=key)


def _gemvb(env, W, X):
    torch, gpu, ctx = env
    B = X.shape[0]
    Y = torch.full((B, W.M), float("nan"), device="cuda")
    gpu.gemvb(ctx, W, torch.from_numpy(np.ascontiguousarray(X)).cuda(), Y, B)
    torch.cuda.synchronize()
    return Y.cpu().numpy()


@pytest.mark.parametrize("wtype", [T_Q6_K, T_Q8_0])
@pytest.mark.parametrize("M,K", [(16, 512), (40, 1024), (300, 1024), (1000, 5120)])
def test_gemv_parity(env, oracle, wtype, M, K):
    _, gpu, ctx = env
    data = _weights(wtype, M, K)
    W = gpu.Weight(ctx, wtype, data, None, K, M)
    for B in (1, 3, 8, 16):
        X = synth.activations(1, B, K)
        y = _gemvb(env, W, X)
        ref = oracle.gemvb(wtype, data, None, K, M, X)
        assert rel_err(y, ref) <= TOL, (wtype, M, K, B, rel_err(y, ref))


@pytest.mark.parametrize("wtype", [T_Q6_K, T_Q8_0])
def test_gemv_block_invariance_bitwise(env, wtype):
    _, gpu, ctx = env
    M, K = 700, 1024
    W = gpu.Weight(ctx, wtype, _weights(wtype, M, K, key=3), None, K, M)
    X = synth.activations(2, 16, K)
    y16 = _gemvb(env, W, X)
    for b in (0, 5, 15):
        y1 = _gemvb(env, W, X[b:b + 1])
        assert np.array_equal(y1[0], y16[b])


def _drafts(rng, am, E, V):
    """draft i = argmax(row i) with probability 0.6, else uniform."""
    d = np.where(rng.random(E) < 0.6, am[:E], rng.integers(0, V, E))
    return d.astype(np.int32)


def _head(env, W, X, drafts, want_logits=True):
    torch, gpu, ctx = env
    B = X.shape[0]
    res = torch.full((2 + B,), -7, dtype=torch.int32, device="cuda")
    dd = torch.from_numpy(drafts).cuda() if drafts.size else None
    lg = torch.full((B, W.M), float("nan"), device="cuda") if want_logits else None
    gpu.head_verify(ctx, W, torch.from_numpy(np.ascontiguousarray(X)).cuda(), B, res, drafts=dd,
                    E=drafts.size, logits=lg)
    torch.cuda.synchronize()
    return res.cpu().numpy(), (lg.cpu().numpy() if want_logits else None)


def test_head_verify_parity(env, oracle):
    _, gpu, ctx = env
    V, K = 5000, 1024
    data = synth.q6_k(0, V, K, key=5)
    W = gpu.Weight(ctx, T_Q6_K, data, None, K, V)
    rng = np.random.default_rng(11)
    for B in (1, 2, 8, 16):
        X = synth.activations(3, B, K)
        ref = oracle.gemvb(T_Q6_K, data, None, K, V, X)
        for trial in range(3):
            E = int(rng.integers(0, B))
            # drafts from the GPU's own argmax so that long walks occur
            res0, lg = _head(env, W, X, np.zeros(0, np.int32))
            am = np.array([oracle.argmax(lg[b]) for b in range(B)])
            assert np.array_equal(res0[2:], am)
            assert rel_err(lg, ref) <= TOL
            drafts = _drafts(rng, am, E, V)
            res, lg2 = _head(env, W, X, drafts)
            assert np.array_equal(lg2, lg)  # deterministic
            k, bonus = oracle.walk(lg[:E + 1], drafts)
            assert (res[0], res[1]) == (k, bonus), (B, E, res[:2], k, bonus)
            # without the logits output the result is the same
            res3, _ = _head(env, W, X, drafts, want_logits=False)
            assert np.array_equal(res3, res)


def test_head_block_invariance(env):
    _, gpu, ctx = env
    V, K = 3000, 512
    W = gpu.Weight(ctx, T_Q6_K, synth.q6_k(0, V, K, key=6), None, K, V)
    X = synth.activations(4, 16, K)
    res16, lg16 = _head(env, W, X, np.zeros(0, np.int32))
    for b in (0, 7, 15):
        res1, lg1 = _head(env, W, X[b:b + 1], np.zeros(0, np.int32))
        assert np.array_equal(lg1[0], lg16[b])
        assert res1[2] == res16[2 + b]


def _argmax_walk(env, lg, drafts):
    torch, gpu, ctx = env
    B, V = lg.shape
    res = torch.full((2 + B,), -7, dtype=torch.int32, device="cuda")
    dd = torch.from_numpy(drafts).cuda() if drafts.size else None
    gpu.argmax_walk(ctx, torch.from_numpy(np.ascontiguousarray(lg)).cuda(), V, B, res, drafts=dd,
                    E=drafts.size)
    torch.cuda.synchronize()
    return res.cpu().numpy()


def test_argmax_walk_edge_cases(env, oracle):
    rng = np.random.default_rng(5)
    V = 20000
    cases = []
    base = rng.standard_normal((8, V)).astype(np.float32)
    cases.append(base.copy())
    t = base.copy(); t[:, [3, 777, 19999]] = 50.0; cases.append(t)          # ties: first wins
    t = base.copy(); t[0, 0] = np.nan; t[1, 5] = np.nan; t[1, 6] = 99; cases.append(t)  # NaN rules
    t = np.full((8, V), -np.inf, np.float32); t[2, 9] = np.nan; cases.append(t)        # all -inf
    t = np.zeros((8, V), np.float32); t[:, :100] = -0.0; t[3, 50] = 0.0; cases.append(t)  # signed zeros
    t = base.copy(); t[4, 123] = np.inf; t[4, 124] = np.inf; cases.append(t)
    t = np.full((8, V), np.nan, np.float32); cases.append(t)                  # all NaN -> 0
    t = base.copy(); t[5, V - 1] = 1e30; cases.append(t)                       # last index
    for lg in cases:
        am = np.array([oracle.argmax(lg[b]) for b in range(lg.shape[0])])
        for E in (0, 1, 4, 7):
            drafts = _drafts(rng, am, E, V)
            res = _argmax_walk(env, lg, drafts)
            assert np.array_equal(res[2:], am)
            k, bonus = oracle.walk(lg[:E + 1], drafts)
            assert (res[0], res[1]) == (k, bonus)


@pytest.mark.parametrize("B,V", [(1, 1), (1, 8193), (16, 151936), (3, 8192)])
def test_argmax_walk_shapes(env, oracle, B, V):
    rng = np.random.default_rng(V + B)
    lg = rng.standard_normal((B, V)).astype(np.float32)
    am = np.array([oracle.argmax(lg[b]) for b in range(B)])
    drafts = am[:B - 1].astype(np.int32).copy()       # full accept
    res = _argmax_walk(env, lg, drafts)
    assert np.array_equal(res[2:], am)
    assert (res[0], res[1]) == (B - 1, am[B - 1])


def test_head_argument_errors(env):
    torch, gpu, ctx = env
    W = gpu.Weight(ctx, T_Q6_K, synth.q6_k(0, 64, 512), None, 512, 64)
    X = torch.zeros(4, 512, device="cuda")
    res = torch.zeros(6, dtype=torch.int32, device="cuda")
    d = torch.zeros(4, dtype=torch.int32, device="cuda")
    with pytest.raises(gpu.CwenError):
        gpu.head_verify(ctx, W, X, 4, res, drafts=d, E=4)     # E > B - 1
    with pytest.raises(gpu.CwenError):
        gpu.head_verify(ctx, W, X, 4, res, drafts=None, E=2)  # drafts missing
    with pytest.raises(gpu.CwenError):
        gpu.Weight(ctx, T_Q6_K, synth.q6_k(0, 64, 512), None, 384, 64)  # K not whole super-blocks
    gpu.head_verify(ctx, W, X, 4, res, drafts=d, E=3)
    torch.cuda.synchronize()


@pytest.mark.slow
@pytest.mark.parametrize("V", [151936, 248320])
def test_head_full_size(env, oracle, V):
    """The Q6_K head at B=8 at the workload's vocabulary (151936) and the real
    model's (248320, run.c:84; 1.04 GB of weights): logits on a row sample vs
    the oracle, argmax and walk vs the oracle on the GPU's logits."""
    _, gpu, ctx = env
    K, B = 5120, 8
    data = synth.q6_k(0, V, K)
    W = gpu.Weight(ctx, T_Q6_K, data, None, K, V)
    X = synth.activations(0, B, K)
    rng = np.random.default_rng(0)
    res0, lg = _head(env, W, X, np.zeros(0, np.int32))
    rows = np.sort(rng.choice(V, 512, replace=False))
    sub = data.reshape(V, -1)[rows].reshape(-1)
    ref = oracle.gemvb(T_Q6_K, sub, None, K, rows.size, X)
    assert rel_err(lg[:, rows], ref) <= TOL
    am = np.array([oracle.argmax(lg[b]) for b in range(B)])
    assert np.array_equal(res0[2:], am)
    drafts = _drafts(rng, am, B - 1, V)
    res, _ = _head(env, W, X, drafts, want_logits=False)
    assert (res[0], res[1]) == oracle.walk(lg, drafts)
