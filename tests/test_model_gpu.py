"""The block-verify model on the device (cwen_model_* + the C host drivers)
on a small config of the same hybrid architecture.

Checked:
  * forward parity: per-position logits of the device forward pass vs the
    oracle's serial forward composed from its C restatements
    (tests/model_oracle.py) in its device-rounding mode: every weight and
    GEMV operand rounded to f16 where the device rounds it
    (tests/device_round.py), sums in float64.  Tolerance (stated), per
    position: rel_err(device, oracle_device) <= 1e-4 + 2 * jit, rel_err =
    max|d| / max|ref| over the vocab, jit = how far the mode's own logits at
    that position move when each f16 operand is perturbed by 1e-6 * max|x|
    before its rounding (the larger of two seeded trials).  What is left
    between device and mode is the order of the device's f32 sums, which
    an f16 rounding downstream can amplify by a flip; jit measures that
    amplification per position.  The device-rounding mode itself is pinned to the
    plain oracle on the CPU (tests/test_device_round.py); f16 rounding moves
    this random-init model's logits by up to ~1e-2 at ill-conditioned
    positions, so a bound against the plain oracle would have to be that
    loose.  The fixed 1e-3 bound against run.c at the native dimensions over
    all 64 layers is tests/test_model_drift_gpu.py's.
  * block == serial, bit for bit: one block of B positions gives the same
    logits as B single-position passes (the property spec == serial rests on).
  * verify with crafted drafts walks and rolls back exactly: accepted drafts
    and bonus tokens reproduce the serial token stream.
  * the speculative decode loop (n-gram drafter, host C) emits exactly the
    serial decode's tokens.
"""
import numpy as np
import pytest

from cwen_amd import synth
from util import rel_err

pytestmark = pytest.mark.gpu
CWEN_BMAX = 16
TOL_DEV = 1e-4    # device vs the oracle's device-rounding mode, plus JIT_FACTOR x the position's sensitivity
JITTER = 1e-6     # relative perturbation before each f16 rounding that the sensitivity is measured with
JIT_FACTOR = 2.0

CFG = dict(n_layers=4, d_model=1024, d_ffn=2048, vocab=4096, n_head=4, n_kv_head=2, head_dim=256,
           n_rot_pairs=32, n_rot=64, gdn_nkh=2, gdn_nvh=4, gdn_dk=128, full_interval=4, max_ctx=512,
           rope_theta=1e7, rms_eps=1e-6)


@pytest.fixture(scope="module")
def env():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from cwen_amd import gpu
    ctx = gpu.Context(0)
    tensors = list(synth.model_tensors(CFG, seed=0))
    m = gpu.Model(ctx, **CFG)
    for t in tensors:
        m.set(*t)
    yield gpu, ctx, m, tensors
    m.free()
    torch.cuda.synchronize()


def _oracle_logits(oracle, tensors, toks, cfg=None):
    """The oracle's device-rounding logits per position and the stated
    tolerance per position (module docstring)."""
    import device_round
    from model_oracle import OracleModel
    OM = OracleModel(oracle, cfg or CFG, tensors, device=True)
    ref = np.stack([OM.step(t, p) for p, t in enumerate(toks)])
    jit = np.zeros(len(toks))
    try:
        device_round.JITTER = JITTER
        for trial in (1, 2):
            device_round.seed_jitter(trial)
            OJ = OracleModel(oracle, cfg or CFG, tensors, device=True)
            jit = np.maximum(jit, [rel_err(OJ.step(t, p), ref[p]) for p, t in enumerate(toks)])
    finally:
        device_round.JITTER = 0.0
    return ref, TOL_DEV + JIT_FACTOR * jit


def _check(got, ref, tol, what=""):
    errs = [rel_err(got[p], ref[p]) for p in range(len(ref))]
    worst = max(range(len(errs)), key=lambda p: errs[p] / tol[p])
    print(f"{what}: max rel_err vs the device-rounding oracle {max(errs):.2e}; "
          f"worst err / tol {errs[worst] / tol[worst]:.2f} at position {worst} (tol {tol[worst]:.2e})", flush=True)
    for p, e in enumerate(errs):
        assert e <= tol[p], (p, e, tol[p])


def test_forward_parity_vs_oracle(env, oracle):
    gpu, ctx, m, tensors = env
    toks = synth.prompt_tokens(1, 12, CFG["vocab"])
    m.reset()
    ref, tol = _oracle_logits(oracle, tensors, toks)
    got = []
    for b0, B in ((0, 5), (5, 7)):          # two blocks of different size
        am = m.forward(toks[b0:b0 + B])
        lg = m.logits(B)
        got.append(lg)
        for b in range(B):
            assert am[b] == oracle.argmax(lg[b])   # the head's argmax is exact on its own logits
    got = np.concatenate(got)
    _check(got, ref, tol, "two blocks")
    assert m.pos == len(toks) - 1


def test_forward_parity_across_key_chunks(env, oracle):
    """70 positions in ragged blocks (16, 16, 3, 13, 16, 6): blocks cross the
    32-key chunk boundaries of the attention, so the chunk partials, their
    merge and the per-query masks inside a chunk are all exercised.  Same
    tolerance as the single-chunk parity test."""
    gpu, ctx, m, tensors = env
    toks = synth.prompt_tokens(7, 70, CFG["vocab"])
    m.reset()
    ref, tol = _oracle_logits(oracle, tensors, toks)
    got, b0 = [], 0
    for B in (16, 16, 3, 13, 16, 6):
        am = m.forward(toks[b0:b0 + B])       # with the head: logits are written
        got.append(m.logits(B))
        assert all(am[i] == oracle.argmax(got[-1][i]) for i in range(B))
        b0 += B
    got = np.concatenate(got)
    _check(got, ref, tol, "70 positions across key chunks")


def test_real_model_types(env, oracle):
    """The real model's mix of GGUF types: Q4_1 ffn_down in every other layer
    and Q5_K ssm_out in every GDN layer (the producers of the split RMSNorm's
    operand are then Q4_1 / Q5_K GEMVs).  Forward parity vs the oracle with
    the same tolerance, a block equal to single positions bit for bit, and
    speculative decode equal to serial decode."""
    gpu, ctx, _, _ = env
    tensors = list(synth.model_tensors(CFG, seed=3, real_types=True))
    assert {t[2] for t in tensors} >= {gpu.T_Q4_1, gpu.T_Q5_K}
    m = gpu.Model(ctx, **CFG)
    for t in tensors:
        m.set(*t)
    toks = synth.prompt_tokens(4, 24, CFG["vocab"])
    ref, tol = _oracle_logits(oracle, tensors, toks)
    got = []
    for b0, B in ((0, 8), (8, 16)):
        m.forward(toks[b0:b0 + B])
        got.append(m.logits(B))
    got = np.concatenate(got)
    _check(got, ref, tol, "real model types")
    m.reset()
    singles = []
    for p in range(8):
        m.forward(toks[p:p + 1])
        singles.append(m.logits(1)[0])
    assert np.array_equal(np.stack(singles).view(np.uint32), got[:8].view(np.uint32))
    prompt = synth.prompt_tokens(5, 48, CFG["vocab"], period=13, noise=0.05)
    m.reset()
    serial = m.generate_serial(prompt, 40)
    spec, st = m.generate_spec(prompt, 40, n_key=2)
    assert np.array_equal(spec, serial)
    m.free()


def test_context_not_a_multiple_of_the_chunk(env, oracle):
    """max_ctx 77: the attention's last 32-key chunk holds only positions
    64..76, and its rows past the last position (and past the cache's end)
    load as zeros.  The cache filled to its last slot in ragged blocks:
    logits vs the oracle with the stated tolerance, and single positions
    equal to the block bit for bit."""
    gpu, ctx, _, tensors = env
    cfg = {**CFG, "max_ctx": 77}
    m = gpu.Model(ctx, **cfg)
    for t in tensors:
        m.set(*t)
    toks = synth.prompt_tokens(12, 77, CFG["vocab"])
    ref, tol = _oracle_logits(oracle, tensors, toks)
    got, b0 = [], 0
    for B in (16, 16, 16, 16, 13):
        m.forward(toks[b0:b0 + B])
        got.append(m.logits(B))
        b0 += B
    got = np.concatenate(got)
    assert m.pos == 76
    _check(got, ref, tol, "max_ctx 77")
    m.reset()
    for b in range(0, 64, 16):
        m.forward(toks[b:b + 16])
    singles = []
    for p in range(64, 77):
        m.forward(toks[p:p + 1])
        singles.append(m.logits(1)[0])
    assert np.array_equal(np.stack(singles).view(np.uint32), got[64:].view(np.uint32))
    with pytest.raises(gpu.CwenError):
        m.forward(toks[:1])                 # the cache is full
    m.free()


def test_q6_k_embedding(env, oracle):
    """A Q6_K token_embd (run.c:1882-1883).  (1) Forward parity vs the oracle
    with a random Q6_K table, same tolerance as above.  (2) Exactness: a Q6_K
    table built so every row dequantizes to the same f32 values as a Q4_0RS
    table (d = 2^-12, equal scale pairs sc, q = n + 24, Q4_0RS scale sc * 2^-12)
    gives the same logits, bit for bit, as that Q4_0RS table."""
    from util import q6_k_pack
    gpu, ctx, _, tensors = env
    V, H = CFG["vocab"], CFG["d_model"]
    rest = [t for t in tensors if not (t[0] == -1 and t[1] == gpu.TOK_EMBD)]
    q6 = (-1, gpu.TOK_EMBD, gpu.T_Q6_K, synth.q6_k(9, V, H, key=77), None, H, V)
    m = gpu.Model(ctx, **CFG)
    for t in rest + [q6]:
        m.set(*t)
    toks = synth.prompt_tokens(8, 10, CFG["vocab"])
    ref, tol = _oracle_logits(oracle, rest + [q6], toks)
    m.forward(toks)
    got = m.logits(len(toks))
    _check(got, ref, tol, "Q6_K embedding")
    # (2) the same values through both layouts
    g = np.random.default_rng(10)
    n = g.integers(0, 16, (V, H)).astype(np.uint8)
    s32 = g.integers(1, 128, (V, H // 32))
    qs_rs = (n.reshape(V, H // 32, 2, 16)[:, :, 0] | (n.reshape(V, H // 32, 2, 16)[:, :, 1] << 4)).astype(np.uint8)
    sc_rs = (s32 * 2.0 ** -12).astype(np.float16).view(np.uint16)
    assert np.array_equal(sc_rs.view(np.float16).astype(np.float64), s32 * 2.0 ** -12)
    packed = q6_k_pack(n + 24, np.repeat(s32, 2, axis=1).astype(np.int8),
                       np.full((V, H // 256), np.float16(2.0 ** -12)).view(np.uint16))
    logits = {}
    for name, t in (("rs", (-1, gpu.TOK_EMBD, gpu.T_Q4_0RS, qs_rs.reshape(-1), sc_rs.reshape(-1), H, V)),
                    ("q6", (-1, gpu.TOK_EMBD, gpu.T_Q6_K, packed.reshape(-1), None, H, V))):
        m.set(*t)
        m.reset()
        m.forward(toks)
        logits[name] = m.logits(len(toks))
    assert np.array_equal(logits["rs"].view(np.uint32), logits["q6"].view(np.uint32))
    m.free()


def test_gguf_load_equals_set(env, tmp_path):
    """cwen_model_load_gguf on a GGUF file written from the synthetic model
    (the reference's tensor names, GGUF Q4_0 matrices with gate/up and k/v as
    separate tensors, F32 vectors, the Q6_K head) gives the model set tensor
    by tensor: argmaxes and logits bit for bit.  A file missing a tensor the
    reference requires is refused, naming it."""
    gpu, ctx, m, tensors = env
    from gguf_writer import gguf_bytes, model_gguf_tensors
    gt = model_gguf_tensors(tensors, CFG)
    p = tmp_path / "model.gguf"
    p.write_bytes(gguf_bytes(gt))
    g = gpu.GGUF(p)
    mg = gpu.Model(ctx, **CFG)
    mg.load_gguf(g)
    toks = synth.prompt_tokens(2, 10, CFG["vocab"])
    m.reset()
    a, la = m.forward(toks), m.logits(10)
    b, lb = mg.forward(toks), mg.logits(10)
    assert np.array_equal(a, b)
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    mg.free()
    g.close()
    p2 = tmp_path / "missing.gguf"
    p2.write_bytes(gguf_bytes([t for t in gt if t[0] != "blk.1.ffn_down.weight"]))
    g2 = gpu.GGUF(p2)
    mg2 = gpu.Model(ctx, **CFG)
    with pytest.raises(gpu.CwenError) as e:
        mg2.load_gguf(g2)
    assert "missing blk.1.ffn_down.weight" in str(e.value)
    mg2.free()
    g2.close()


@pytest.mark.parametrize("version", [4, 3, 2])
def test_cwenr_load_equals_set(env, tmp_path, version):
    """A GGUF file with a CWENR sidecar of its Q4_0 tensors (v4: gate/up and
    k/v interleaved pairs uploaded as they are; v3: split halves interleaved
    on the host; v2: packed blocks split on the host) loads into the model
    set tensor by tensor: argmaxes and logits bit for bit."""
    gpu, ctx, m, tensors = env
    from gguf_writer import cwenr_from_gguf, gguf_bytes, model_gguf_tensors
    gt = model_gguf_tensors(tensors, CFG)
    p = tmp_path / "model.gguf"
    p.write_bytes(gguf_bytes(gt))
    s = tmp_path / "model.cwenr"
    s.write_bytes(cwenr_from_gguf(gt, version, src_pages=(p.stat().st_size + 4095) // 4096))
    g = gpu.GGUF(p)
    n_q4 = sum(1 for t in gt if t[1] == gpu.T_Q4_0)
    assert g.apply_cwenr(gpu.GGUF.cwenr_path(p), p) == n_q4
    assert g.tensor(g.find("token_embd.weight"))[1] == gpu.T_Q4_0RS
    mg = gpu.Model(ctx, **CFG)
    mg.load_gguf(g)
    toks = synth.prompt_tokens(3, 10, CFG["vocab"])
    m.reset()
    a, la = m.forward(toks), m.logits(10)
    b, lb = mg.forward(toks), mg.logits(10)
    assert np.array_equal(a, b)
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    mg.free()
    g.close()


def test_serve_answers_frames_like_generate(env):
    """The frame server (cwen_serve, run.c:5063-5078) over pipes: each valid
    frame is answered with the tokens cwen_generate_serial gives for it, from
    a fresh decode, in serial and in speculative mode alike; a frame with an
    out-of-range token is answered with 0 and the stream continues."""
    import os
    import struct
    gpu, ctx, m, _ = env
    prompts = [synth.prompt_tokens(5, 48, CFG["vocab"], period=13, noise=0.05),
               synth.prompt_tokens(6, 7, CFG["vocab"]), synth.prompt_tokens(7, 33, CFG["vocab"], period=5)]
    n_gen = [30, 12, 25]
    want = []
    for p, g in zip(prompts, n_gen):
        want.append(m.generate_serial(p, g).tolist())
    req = b""
    for i, (p, g) in enumerate(zip(prompts, n_gen)):
        req += struct.pack("<II", len(p), g) + np.asarray(p, "<i4").tobytes()
        if i == 0:
            req += struct.pack("<IIi", 1, 4, CFG["vocab"])           # rejected: token out of range
    for spec in (None, gpu.SpecCfg(2, 8, 2, 8, 0, 1)):
        ri, wi = os.pipe()
        ro, wo = os.pipe()
        os.write(wi, req)
        os.close(wi)
        try:
            assert m.serve(ri, wo, spec) == 3
            os.close(wo)
            raw = b""
            while chunk := os.read(ro, 65536):
                raw += chunk
        finally:
            os.close(ri)
            os.close(ro)
        got, at = [], 0
        while at < len(raw):
            (n,) = struct.unpack_from("<I", raw, at)
            got.append(list(struct.unpack_from(f"<{n}i", raw, at + 4)))
            at += 4 + 4 * n
        assert got == [want[0], [], want[1], want[2]], spec


@pytest.mark.parametrize("B", [4, 8, 16])
def test_block_equals_serial_bitwise(env, B):
    """Every block size takes the same path (the producer writes the f16
    operand x * w of the next RMSNorm, the consuming GEMV scales its output
    columns by 1 / rms), so a block and its single positions agree bit for
    bit."""
    gpu, ctx, m, _ = env
    toks = synth.prompt_tokens(2, 12 + B, CFG["vocab"])
    m.reset()
    m.forward(toks[:12], want_argmax=False)
    m.forward(toks[12:12 + B])
    block = m.logits(B).copy()
    m.reset()
    m.forward(toks[:12], want_argmax=False)
    for b in range(B):
        m.forward(toks[12 + b:13 + b])
        assert np.array_equal(m.logits(1)[0], block[b]), b


@pytest.mark.parametrize("emax", [8, 16])
def test_verify_walk_and_rollback(env, emax):
    """Drafts built from the serial stream with planted mistakes: every
    accepted draft and bonus must equal the serial stream.  Blocks of up to
    emax positions (E < emax drafts), so with emax = 16 the accepted prefix
    the next block replays reaches 15 positions."""
    gpu, ctx, m, _ = env
    V = CFG["vocab"]
    prompt = synth.prompt_tokens(3, 40, V)
    n_gen = 60
    serial = m.generate_serial(prompt, n_gen)
    assert len(serial) == n_gen
    g = np.random.default_rng(4)
    import ctypes as C
    nxt = C.c_int()
    gpu.check("cwen_prefill", gpu.host_lib().cwen_prefill(m.h, np.ascontiguousarray(prompt, np.int32).ctypes.data,
                                                          len(prompt), C.byref(nxt)))
    out = [nxt.value]
    seen_partial = seen_full = False
    longest = 0        # longest accepted prefix of a partly rejected block
    while len(out) < n_gen:
        E = int(g.integers(0, emax))
        fut = serial[len(out):len(out) + E].astype(np.int32)
        E = len(fut)
        drafts = fut.copy()
        if E and g.random() < 0.5:
            j = int(g.integers(0, E))
            drafts[j] = (drafts[j] + 1) % V       # plant a mistake at j
        k, bonus = m.verify(np.concatenate([[out[-1]], drafts]).astype(np.int32))
        want_k = next((i for i in range(E) if drafts[i] != fut[i]), E)
        assert k == want_k, (len(out), E, k, want_k)
        seen_partial |= k < E
        seen_full |= E > 0 and k == E
        if k < E:
            longest = max(longest, k)
        out.extend(drafts[:k].tolist())
        out.append(bonus)
    assert seen_partial and seen_full
    if emax == 16:
        assert longest >= 8, longest          # a replay longer than 8 positions happened
    assert np.array_equal(np.array(out[:n_gen]), serial)


@pytest.mark.parametrize("n_key", [2, 4, 16])
def test_spec_decode_equals_serial(env, n_key):
    gpu, ctx, m, _ = env
    prompt = synth.prompt_tokens(5, 64, CFG["vocab"], period=13, noise=0.05)
    n_gen = 80
    serial = m.generate_serial(prompt, n_gen)
    spec, st = m.generate_spec(prompt, n_gen, n_key=n_key)
    assert np.array_equal(spec, serial)
    assert st.cycles <= n_gen
    if n_key <= 4:
        assert st.drafted > 0


@pytest.mark.parametrize("use_map", [True, False])
def test_spec_cycles_equal_replay_of_serial(env, use_map):
    """The device speculative driver with the counted n-gram map: its drafts
    and walk, cycle by cycle, equal the host replay of the same driver over
    the model's own serial stream (cwen_spec_replay), which the CPU tests pin
    to the reference's generate_tokens_spec.  So on the device, too, the
    cycle count follows the reference, not only the tokens."""
    gpu, ctx, m, _ = env
    prompt = synth.prompt_tokens(6, 64, CFG["vocab"], period=11, noise=0.05)
    n_gen = 120
    # the stream runs a block past n_gen: the last cycle's walk reads that far
    longer = m.generate_serial(prompt, n_gen + CWEN_BMAX)
    serial = longer[:n_gen]
    stream = np.concatenate([prompt, longer]).astype(np.int32)
    logs = []
    for replay in (False, True):
        log = np.full(2 * 1024, -1, np.int32)
        mp = gpu.NgMap(4, CFG["vocab"]) if use_map else None
        cfg = gpu.spec_cfg(4, 8, 2, 8, 0, 0, mp, log)
        if replay:
            out, st = gpu.spec_replay(stream, prompt.size, n_gen, CFG["max_ctx"], cfg)
        else:
            out, st = m.generate_spec(prompt, n_gen, n_key=4, mtp=0, ngmap=mp, cycle_log=log)
        assert np.array_equal(out, serial)
        logs.append((log[:2 * st.cycles].copy(), [st.cycles, st.drafted, st.full, st.rejected, st.kept]))
    assert np.array_equal(logs[0][0], logs[1][0])
    assert logs[0][1] == logs[1][1]
    assert logs[0][1][1] > 0


def test_chunk_mapping_changes_no_bit(env):
    """The attention's partials are per 32-key chunk and merged in chunk
    order, so which workgroup computes a chunk cannot change a bit: with
    max_ctx 4096 every chunk has a workgroup of its own, with 16384 the
    workgroups loop over chunks (the stride path); a 4000-token prompt and
    a verify block give bit-identical logits in both.  A context beyond
    CWEN_CTX_MAX (32768, the reference's MAX_SEQ) is refused."""
    gpu, ctx, m, tensors = env
    prompt = synth.prompt_tokens(9, 4000, CFG["vocab"])
    out = []
    for max_ctx in (4096, 16384):
        mm = gpu.Model(ctx, **{**CFG, "max_ctx": max_ctx})
        for t in tensors:
            mm.set(*t)
        for i in range(0, prompt.size - 8, 16):
            mm.forward(prompt[i:min(i + 16, prompt.size - 8)], want_argmax=False)
        am = mm.forward(prompt[-8:])
        out.append((am, mm.logits(8)))
        mm.free()
    assert np.array_equal(out[0][0], out[1][0])
    assert np.array_equal(out[0][1].view(np.uint32), out[1][1].view(np.uint32))
    with pytest.raises(gpu.CwenError):
        gpu.Model(ctx, **{**CFG, "max_ctx": 32769})


def test_out_of_range_operand_is_reported(env):
    """The RMSNorm is split between producer and consumer, so the f16 operand
    holds a residual element times its norm weight before normalisation.
    When that leaves f16's range the operand is infinite: verify and
    forward-with-argmax then return CWEN_ERANGE (sticky until reset) instead
    of tokens silently computed from it.  In range, the same model gives the
    ordinary result, before and after."""
    gpu, ctx, m, tensors = env
    mb = gpu.Model(ctx, **CFG)
    for t in tensors:
        mb.set(*t)
    toks = synth.prompt_tokens(6, 8, CFG["vocab"])
    ok = mb.verify(toks)
    layer, tid, wtype, w, _, ne0, ne1 = next(t for t in tensors if t[0] == 1 and t[1] == gpu.POST_NORM)
    mb.set(layer, tid, wtype, (w * 1e6).astype(np.float32), None, ne0, ne1)
    mb.reset()
    with pytest.raises(gpu.CwenError) as e:
        mb.verify(toks)
    assert e.value.rc == gpu.CWEN_ERANGE
    with pytest.raises(gpu.CwenError) as e:   # sticky: the next synchronous call reports it too
        mb.forward(toks[:1])
    assert e.value.rc == gpu.CWEN_ERANGE
    mb.set(layer, tid, wtype, w, None, ne0, ne1)
    mb.reset()
    assert mb.verify(toks) == ok
    mb.free()


def test_graph_replay_equals_eager(env, monkeypatch):
    """CWEN_GRAPHS=1: each (mode, B) block is captured once and replayed at
    later positions (position and ring slot read on the device).  Replays
    give the eager model's logits and token stream bit for bit."""
    gpu, ctx, m, tensors = env
    monkeypatch.setenv("CWEN_GRAPHS", "1")
    mg = gpu.Model(ctx, **CFG)
    monkeypatch.delenv("CWEN_GRAPHS")
    for t in tensors:
        mg.set(*t)
    toks = synth.prompt_tokens(6, 30, CFG["vocab"])
    for model in (m, mg):
        model.reset()
    for b0, B in ((0, 5), (5, 5), (10, 5), (15, 1), (16, 1), (17, 8)):   # replays of B = 5 and B = 1
        a = m.forward(toks[b0:b0 + B])
        la = m.logits(B)
        b = mg.forward(toks[b0:b0 + B])
        assert np.array_equal(a, b), b0
        assert np.array_equal(la, mg.logits(B)), b0
    prompt = synth.prompt_tokens(5, 64, CFG["vocab"], period=13, noise=0.05)
    serial = m.generate_serial(prompt, 60)
    spec, st = mg.generate_spec(prompt, 60, n_key=2)
    assert np.array_equal(spec, serial)
    assert st.drafted > 0
    mg.free()
