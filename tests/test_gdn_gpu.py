"""Parity of the HIP GatedDeltaNet block verify (conv + delta rule over B
positions, per-position snapshots, rollback) against the oracle's
conv1d_update + gdn_step applied position by position.

Tolerances (stated): outputs and recurrent state rel_err <= 1e-3
(max|x - ref| / max|ref|); the conv history holds raw inputs and must match
bit for bit.  The serial equivalence (a block of B == B single-position
blocks committed one by one) is checked bit for bit: it is what makes the GPU
speculative decode emit the serial decode's tokens.
"""
import numpy as np
import pytest

from util import rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3


@pytest.fixture(scope="module")
def env():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from cwen_amd import gpu
    ctx = gpu.Context(0)
    yield torch, gpu, ctx
    torch.cuda.synchronize()


def _inputs(seed, B, nkh, nvh, dk=128):
    """The GDN verify workload: S ~ N(0, 0.01), raw qkv / history / z ~ N(0,1),
    alpha ~ U(0,1) -> decay = log(alpha), beta = sigmoid(N(0,1))."""
    g = np.random.default_rng(seed)
    C = (2 * nkh + nvh) * dk
    f = np.float32
    S = (0.01 * g.standard_normal((nvh, dk, dk))).astype(f)
    hist = g.standard_normal((C, 3)).astype(f)
    kw = (0.5 * g.standard_normal((C, 4))).astype(f)
    wn = (1 + 0.1 * g.standard_normal(dk)).astype(f)
    qkv = g.standard_normal((B, C)).astype(f)
    z = g.standard_normal((B, nvh * dk)).astype(f)
    decay = np.log(g.uniform(1e-3, 1.0, (B, nvh))).astype(f)
    beta = (1 / (1 + np.exp(-g.standard_normal((B, nvh))))).astype(f)
    return S, hist, kw, wn, qkv, z, decay, beta


def _oracle_run(oracle, S, hist, kw, wn, qkv, z, decay, beta, nkh, nvh, dk=128):
    """Reference order: per position conv1d_update then gdn_step; returns the
    outputs and the (S, hist) after each position."""
    outs, states = [], []
    for b in range(qkv.shape[0]):
        x, hist = oracle.conv1d_update(qkv[b], hist, kw)
        S, _, o = oracle.gdn_step(S, x, z[b], decay[b], beta[b], wn, nkh, nvh, dk)
        outs.append(o)
        states.append((S.copy(), hist.copy()))
    return np.stack(outs), states


def _gpu_block(env, G, kw, wn, qkv, z, decay, beta):
    torch, gpu, ctx = env
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    B = qkv.shape[0]
    out = torch.full((B, G.nvh * G.dk), float("nan"), device="cuda")
    G.block(t(qkv), t(z), t(decay), t(beta), t(kw), t(wn), out, B)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("nkh,nvh,B", [(16, 48, 8), (16, 48, 1), (16, 48, 16), (2, 6, 5)])
def test_gdn_block_parity_and_rollback(env, oracle, nkh, nvh, B):
    _, gpu, ctx = env
    S, hist, kw, wn, qkv, z, decay, beta = _inputs(100 + B + nvh, B, nkh, nvh)
    G = gpu.GDN(ctx, nkh, nvh)
    G.set_state(S, hist)
    out = _gpu_block(env, G, kw, wn, qkv, z, decay, beta)
    ref, states = _oracle_run(oracle, S, hist, kw, wn, qkv, z, decay, beta, nkh, nvh)
    for b in range(B):
        assert rel_err(out[b], ref[b]) <= TOL, (b, rel_err(out[b], ref[b]))
    S0, h0 = G.get_state(0)
    assert np.array_equal(S0, S) and np.array_equal(h0, hist)    # current state untouched
    for p in range(1, B + 1):
        Sp, hp = G.get_state(p)
        assert rel_err(Sp, states[p - 1][0]) <= TOL, (p, rel_err(Sp, states[p - 1][0]))
        assert np.array_equal(hp, states[p - 1][1])
    # roll back to a seeded accepted length, then continue with a new block
    L = int(np.random.default_rng(B).integers(0, B + 1))
    G.commit(L)
    Sc, hc = G.get_state(0)
    S_L, h_L = (S, hist) if L == 0 else states[L - 1]
    assert rel_err(Sc, S_L) <= TOL and np.array_equal(hc, h_L)
    _, _, kw2, wn2, qkv2, z2, decay2, beta2 = _inputs(7, 5, nkh, nvh)
    out2 = _gpu_block(env, G, kw, wn, qkv2, z2, decay2, beta2)
    ref2, _ = _oracle_run(oracle, S_L, h_L, kw, wn, qkv2, z2, decay2, beta2, nkh, nvh)
    assert rel_err(out2, ref2) <= TOL
    G.free()


@pytest.mark.parametrize("B", [8, 16])
def test_gdn_block_equals_serial_bitwise(env, B):
    """One block of B positions == B one-position blocks, each committed
    (at B = 16 each wave of the recurrence stages two positions)."""
    _, gpu, ctx = env
    nkh, nvh = 16, 48
    S, hist, kw, wn, qkv, z, decay, beta = _inputs(3, B, nkh, nvh)
    Gb = gpu.GDN(ctx, nkh, nvh)
    Gb.set_state(S, hist)
    out_b = _gpu_block(env, Gb, kw, wn, qkv, z, decay, beta)
    Gs = gpu.GDN(ctx, nkh, nvh)
    Gs.set_state(S, hist)
    for b in range(B):
        o = _gpu_block(env, Gs, kw, wn, qkv[b:b + 1], z[b:b + 1], decay[b:b + 1], beta[b:b + 1])
        assert np.array_equal(o[0], out_b[b]), b
        Gs.commit(1)
        Sb, hb = Gb.get_state(b + 1)
        Ss, hs = Gs.get_state(0)
        assert np.array_equal(Sb, Ss) and np.array_equal(hb, hs), b
    Gb.free()
    Gs.free()


def test_gdn_long_replay_then_full_block(env, oracle):
    """Commit 12 of a block of 16, then a block of 16: the second launch
    replays 12 positions (more than one per recurrence wave) before its own
    16.  Its outputs and end state equal, bit for bit, those of a state that
    took the same 12 positions as single committed blocks, and match the
    oracle continued from the 12th position (rel_err <= 1e-3)."""
    _, gpu, ctx = env
    nkh, nvh, B, L = 16, 48, 16, 12
    S, hist, kw, wn, qkv, z, decay, beta = _inputs(11, B, nkh, nvh)
    _, _, _, _, qkv2, z2, decay2, beta2 = _inputs(12, B, nkh, nvh)
    G = gpu.GDN(ctx, nkh, nvh)
    G.set_state(S, hist)
    _gpu_block(env, G, kw, wn, qkv, z, decay, beta)
    G.commit(L)
    out_r = _gpu_block(env, G, kw, wn, qkv2, z2, decay2, beta2)
    G.commit(B)
    Gs = gpu.GDN(ctx, nkh, nvh)
    Gs.set_state(S, hist)
    for b in range(L):
        _gpu_block(env, Gs, kw, wn, qkv[b:b + 1], z[b:b + 1], decay[b:b + 1], beta[b:b + 1])
        Gs.commit(1)
    out_s = _gpu_block(env, Gs, kw, wn, qkv2, z2, decay2, beta2)
    Gs.commit(B)
    assert np.array_equal(out_r.view(np.uint32), out_s.view(np.uint32))
    Sr, hr = G.get_state(0)
    Ss, hs = Gs.get_state(0)
    assert np.array_equal(Sr.view(np.uint32), Ss.view(np.uint32)) and np.array_equal(hr, hs)
    _, states = _oracle_run(oracle, S, hist, kw, wn, qkv[:L], z[:L], decay[:L], beta[:L], nkh, nvh)
    ref2, states2 = _oracle_run(oracle, *states[L - 1], kw, wn, qkv2, z2, decay2, beta2, nkh, nvh)
    assert rel_err(out_r, ref2) <= TOL, rel_err(out_r, ref2)
    assert rel_err(Sr, states2[-1][0]) <= TOL and np.array_equal(hr, states2[-1][1])
    G.free()
    Gs.free()


def test_gdn_identity_gates(env):
    """decay = 0 (g = 1) and beta = 0 leave the state unchanged."""
    _, gpu, ctx = env
    nkh, nvh, B = 16, 48, 4
    S, hist, kw, wn, qkv, z, decay, beta = _inputs(4, B, nkh, nvh)
    G = gpu.GDN(ctx, nkh, nvh)
    G.set_state(S, hist)
    _gpu_block(env, G, kw, wn, qkv, z, np.zeros_like(decay), np.zeros_like(beta))
    for p in range(1, B + 1):
        assert np.array_equal(G.get_state(p)[0], S)
    G.free()


def test_gdn_argument_errors(env):
    _, gpu, ctx = env
    with pytest.raises(gpu.CwenError):
        gpu.GDN(ctx, 16, 48, dk=64)
    with pytest.raises(gpu.CwenError):
        gpu.GDN(ctx, 16, 40)            # nvh not a multiple of nkh
    G = gpu.GDN(ctx, 2, 4)
    with pytest.raises(gpu.CwenError):
        G.commit(1)                     # no block run yet
    with pytest.raises(gpu.CwenError):
        G.get_state(1)
    G.free()
