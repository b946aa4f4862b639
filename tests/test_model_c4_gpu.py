"""The 27B shape's attention geometry at long context, on the device.

The full 27B-shape model has 24 query heads over 4 KV heads (6 per KV head),
and its benchmark prefills 4096 tokens in blocks of 16 into an 8192-slot
cache.  That geometry takes attention paths the small test config never
reaches: a block of 16 positions has 96 queries per KV head (more than four
16-query tiles, so the chunk kernel runs 8-wave workgroups), and past 2048
positions the key chunks outnumber the chunk workgroups (each takes several
chunks, landing the next while it computes the current one).

  * test_c4_geometry_vs_oracle: a 2-layer model of that geometry (one
    GatedDeltaNet layer, one full-attention layer) prefilled to 4192
    positions in blocks of 16, then a block of 16 and two blocks of 8 with
    the head.  Their logits are compared with the oracle's serial forward
    over the same 4224 tokens (tests/golden/c4_geometry_logits.npz, written
    by make_c4_geometry_golden.py).  The same over 6400 tokens
    (c4_geometry_wide_logits.npz): past 6144 positions the chunk kernel
    switches from 64 double-buffered workgroups per KV head to 128
    single-buffered ones, so the prefill crosses the switch and the
    compared blocks run the wide grid.  The reference is the oracle's
    device-rounding mode (tests/device_round.py: f16 weights and operands
    where the device rounds them, float64 sums).  Tolerance (stated), as in
    tests/test_model_gpu.py: per position, rel_err <= 1e-4 + 2 * jit, jit
    = how far the mode's own logits move when each f16 operand is perturbed
    by 1e-6 * max|x| first (the fixture's "jit"); rel_err = max|d| /
    max|ref| over the vocab.  Every row's argmax is also checked bit-exact
    against the device's own logits.
  * test_c4_geometry_long_context_vs_oracle: the same model in a 32768-slot
    cache (run.c:85 MAX_SEQ, the interface's maximum) prefilled to 16416 and
    32704 positions, then the same three blocks, against
    c4_geometry_{16k,32k}_logits.npz (make_c4_geometry_golden.py --long):
    514 and 1023 key chunks, so the chunk kernel runs its wide grid several
    chunks per workgroup and each of the merge's four groups sums 128-129
    and 255-256 chunk partials.  Same bound.
  * block == single positions bit for bit at the same geometry and context,
    and near the end of the 32768-slot cache.
  * test_27b_shape_spec_equals_serial (slow): the full 64-layer 27B shape
    (device-generated random-init weights), max_ctx 8192, a 4160-token
    prompt: a block equals its single positions bit for bit, verify blocks
    with planted draft mistakes walk and roll back to the serial stream, and
    the speculative decode emits exactly the serial decode's tokens.
"""
from pathlib import Path

import numpy as np
import pytest

from cwen_amd import synth
from util import rel_err

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "c4_geometry_logits.npz"
GOLDEN_WIDE = GOLDEN.with_name("c4_geometry_wide_logits.npz")
TOL_DEV, JIT_FACTOR = 1e-4, 2.0     # as in tests/test_model_gpu.py


def _golden_cfg():
    import sys
    sys.path.insert(0, str(GOLDEN.parent))
    import make_c4_geometry_golden as g
    return g


@pytest.fixture(scope="module")
def env():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from cwen_amd import gpu
    g = _golden_cfg()
    ctx = gpu.Context(0)
    m = gpu.Model(ctx, **g.CFG)
    for t in synth.model_tensors(g.CFG, seed=g.SEED):
        m.set(*t)
    yield gpu, ctx, m, g
    m.free()
    torch.cuda.synchronize()


def _prefill(m, toks, n, B=16):
    m.reset()
    for b0 in range(0, n, B):
        m.forward(toks[b0:min(n, b0 + B)], want_argmax=False)
    assert m.pos == n - 1


@pytest.fixture(scope="module")
def env_long():
    """The same model in a 32768-slot cache (the interface's maximum,
    run.c:85 MAX_SEQ)."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from cwen_amd import gpu
    g = _golden_cfg()
    ctx = gpu.Context(0)
    m = gpu.Model(ctx, **g.LONG_CFG)
    for t in synth.model_tensors(g.LONG_CFG, seed=g.SEED):
        m.set(*t)
    yield gpu, ctx, m, g
    m.free()
    torch.cuda.synchronize()


@pytest.mark.parametrize("golden", [GOLDEN, GOLDEN_WIDE], ids=["narrow", "wide"])
def test_c4_geometry_vs_oracle(env, oracle, golden):
    _vs_oracle(env, oracle, golden)


@pytest.mark.parametrize("which", ["16k", "32k"])
def test_c4_geometry_long_context_vs_oracle(env_long, oracle, which):
    """16448 and 32736 positions in a 32768-slot cache: 514 and 1023 key
    chunks, so each of the merge's four groups sums 128-129 and 255-256
    chunk partials.  Same comparison and tolerance as above, against
    c4_geometry_{16k,32k}_logits.npz."""
    _vs_oracle(env_long, oracle, GOLDEN.with_name(f"c4_geometry_{which}_logits.npz"))


@pytest.mark.parametrize("B", [16, 8])
def test_c4_geometry_long_context_block_equals_singles(env_long, B):
    """A block equals its single positions bit for bit near the end of the
    32768-slot cache."""
    gpu, ctx, m, g = env_long
    p0 = 32736 - B
    toks = g.tokens(32736)
    _prefill(m, toks, p0)
    m.forward(toks[p0:p0 + B])
    block = m.logits(B).copy()
    _prefill(m, toks, p0)
    for b in range(B):
        m.forward(toks[p0 + b:p0 + b + 1])
        assert np.array_equal(m.logits(1)[0].view(np.uint32), block[b].view(np.uint32)), b


def _vs_oracle(env, oracle, golden):
    gpu, ctx, m, g = env
    fx = np.load(golden)
    n_ctx, n_cmp = int(fx["n_ctx"]), int(fx["n_cmp"])
    toks = g.tokens(n_ctx)
    assert len(toks) == n_ctx
    p0 = n_ctx - n_cmp
    _prefill(m, toks, p0)
    got, b0 = [], p0
    for B in (16, 8, 8):
        am = m.forward(toks[b0:b0 + B])
        lg = m.logits(B)
        for b in range(B):
            assert am[b] == oracle.argmax(lg[b])
        got.extend(list(lg))
        b0 += B
    got = np.stack(got)
    ref, jit = fx["refdev"], fx["jit"]
    errs = [rel_err(got[i], ref[i]) for i in range(n_cmp)]
    tol = TOL_DEV + JIT_FACTOR * jit
    worst = max(range(n_cmp), key=lambda i: errs[i] / tol[i])
    print(f"c4 geometry: max rel_err vs the device-rounding oracle {max(errs):.3e}; worst err / tol "
          f"{errs[worst] / tol[worst]:.2f} at position {p0 + worst} (tol {tol[worst]:.2e}); vs the plain oracle "
          f"{max(rel_err(got[i], fx['ref'][i]) for i in range(n_cmp)):.3e}", flush=True)
    for i in range(n_cmp):
        assert errs[i] <= tol[i], (p0 + i, errs[i], tol[i])


@pytest.mark.parametrize("B", [16, 8])
@pytest.mark.parametrize("p0", [4192, 6368])
def test_c4_geometry_block_equals_singles(env, B, p0):
    gpu, ctx, m, g = env
    toks = g.tokens(g.N_CTX_WIDE)
    _prefill(m, toks, p0)
    m.forward(toks[p0:p0 + B])
    block = m.logits(B).copy()
    _prefill(m, toks, p0)
    for b in range(B):
        m.forward(toks[p0 + b:p0 + b + 1])
        assert np.array_equal(m.logits(1)[0].view(np.uint32), block[b].view(np.uint32)), b


C27 = dict(n_layers=64, d_model=5120, d_ffn=17408, vocab=151936, n_head=24, n_kv_head=4, head_dim=256,
           n_rot_pairs=32, n_rot=64, gdn_nkh=16, gdn_nvh=48, gdn_dk=128, full_interval=4, max_ctx=8192,
           rope_theta=1e7, rms_eps=1e-6)


@pytest.mark.slow
def test_27b_shape_spec_equals_serial():
    import ctypes as C
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from cwen_amd import gpu
    ctx = gpu.Context(0)
    m = gpu.Model(ctx, **C27)
    m.synth(7)
    V = C27["vocab"]
    prompt = synth.prompt_tokens(8, 4160, V, period=97, noise=0.05)
    n_gen = 48
    print("27B shape: serial decode", flush=True)
    serial, st_s = m.generate_serial(prompt, n_gen, with_stats=True)
    assert len(serial) == n_gen
    print("27B shape: speculative decode", flush=True)
    spec, st = m.generate_spec(prompt, n_gen, n_key=4)
    assert np.array_equal(spec, serial)
    print(f"27B shape: spec == serial, {st.cycles} cycles, {st.drafted} drafted, {st.kept} kept", flush=True)

    # verify blocks with planted draft mistakes reproduce the serial stream
    rng = np.random.default_rng(9)
    nxt = C.c_int()
    gpu.check("cwen_prefill", gpu.host_lib().cwen_prefill(
        m.h, np.ascontiguousarray(prompt, np.int32).ctypes.data, len(prompt), C.byref(nxt)))
    out = [nxt.value]
    seen_partial = seen_full = False
    while len(out) < n_gen:
        E = len(serial[len(out):len(out) + int(rng.integers(1, 16))])
        fut = serial[len(out):len(out) + E].astype(np.int32)
        drafts = fut.copy()
        if E and rng.random() < 0.5:
            j = int(rng.integers(0, E))
            drafts[j] = (drafts[j] + 1) % V
        k, bonus = m.verify(np.concatenate([[out[-1]], drafts]).astype(np.int32))
        assert k == next((i for i in range(E) if drafts[i] != fut[i]), E)
        seen_partial |= k < E
        seen_full |= E > 0 and k == E
        out.extend(drafts[:k].tolist())
        out.append(bonus)
    assert seen_partial and seen_full
    assert np.array_equal(np.array(out[:n_gen]), serial)
    print("27B shape: planted-mistake verify == serial", flush=True)

    # a block of 16 past 4096 positions equals its single positions bit for bit
    p0 = len(prompt)
    blk = serial[:16].astype(np.int32)
    gpu.check("cwen_prefill", gpu.host_lib().cwen_prefill(
        m.h, np.ascontiguousarray(prompt, np.int32).ctypes.data, len(prompt), C.byref(nxt)))
    m.forward(blk)
    block = m.logits(16).copy()
    gpu.check("cwen_prefill", gpu.host_lib().cwen_prefill(
        m.h, np.ascontiguousarray(prompt, np.int32).ctypes.data, len(prompt), C.byref(nxt)))
    for b in range(16):
        m.forward(blk[b:b + 1])
        assert np.array_equal(m.logits(1)[0].view(np.uint32), block[b].view(np.uint32)), (p0 + b)
    print("27B shape: block of 16 == singles", flush=True)
    m.free()
    ctx.close()
