"""The MTP nextn drafter on the device (cwen_model_mtp_draft and the commit
pass every block runs), on the small hybrid config with a synthetic nextn
block.  Checked against the oracle's restatement of mtp_step / mtp_commit /
mtp_draft (run.c:3099-3187, tests/model_oracle.py):

  * draft logits: after a prompt in blocks, and after a history of verify
    cycles that kept all, some and none of their drafts (so the commit pass
    wrote slots past the walk that later passes rewrote), each draft step's
    logits match the device-rounding mode of the oracle
    (tests/device_round.py) -- whose nextn stream was built one position at
    a time -- with the tolerance of the forward parity tests
    (tests/test_model_gpu.py): per step, rel_err <= 1e-4 + 2 * the step's
    sensitivity (how far the oracle's logits move when each f16 operand is
    perturbed by 1e-6 * max|x| first).  The oracle is fed the device's draft
    tokens (teacher forcing), and each draft is the argmax of the device's
    own logits for that step.
  * speculative decode drafting with the MTP block emits exactly the serial
    decode's tokens.
  * a model without the MTP tensors drafts nothing.
"""
import numpy as np
import pytest

from cwen_amd import synth
from util import rel_err

pytestmark = pytest.mark.gpu
TOL_DEV, JITTER, JIT_FACTOR = 1e-4, 1e-6, 2.0     # as in tests/test_model_gpu.py

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
    tensors = list(synth.model_tensors(CFG, seed=0, mtp=True))
    m = gpu.Model(ctx, **CFG)
    for t in tensors:
        m.set(*t)
    assert m.has_mtp()
    yield gpu, ctx, m, tensors
    m.free()
    torch.cuda.synchronize()


def check_drafts(m, oracle, tensors, committed, pend, n):
    """Device drafts from pend after the committed tokens vs the oracle's
    nextn stream built serially over the same tokens."""
    from model_oracle import OracleModel
    drafts = m.mtp_draft(pend, n)
    assert len(drafts) == n
    got = m.mtp_logits(n)
    for t in range(n):
        assert drafts[t] == oracle.argmax(got[t])
    import device_round
    refs = []
    try:
        for trial, jitter in enumerate((0.0, JITTER, JITTER)):
            device_round.JITTER = jitter
            device_round.seed_jitter(trial)
            om = OracleModel(oracle, CFG, tensors, device=True)
            for p, tok in enumerate(committed):
                om.step(tok, p)
            refs.append(om.mtp_draft_logits(pend, len(committed) - 1, drafts[:-1]))
    finally:
        device_round.JITTER = 0.0
    for t in range(n):
        tol = TOL_DEV + JIT_FACTOR * max(rel_err(refs[1][t], refs[0][t]), rel_err(refs[2][t], refs[0][t]))
        e = rel_err(got[t], refs[0][t])
        print(f"draft step {t}: rel_err vs the device-rounding oracle {e:.2e} (tol {tol:.2e})", flush=True)
        assert e <= tol, (t, e, tol)
    return drafts


def test_draft_after_prompt_blocks(env, oracle):
    gpu, ctx, m, tensors = env
    toks = synth.prompt_tokens(11, 21, CFG["vocab"])
    m.reset()
    assert len(m.mtp_draft(0, 4)) == 0                 # nothing parked yet
    m.forward(toks[:16])
    am = m.forward(toks[16:])
    check_drafts(m, oracle, tensors, list(toks), int(am[-1]), 5)


def test_draft_after_verify_history(env, oracle):
    """Cycles that keep every draft, a prefix, none, and the device's own
    MTP drafts; then the drafts from the final position."""
    gpu, ctx, m, tensors = env
    prompt = synth.prompt_tokens(12, 9, CFG["vocab"])
    m.reset()
    truth = list(m.generate_serial(prompt, 40))          # the serial continuation
    m.reset()
    committed = list(prompt)
    am = m.forward(prompt)
    pend = int(am[-1])
    assert pend == truth[0]
    i = 0                                                 # truth[i] == pend
    for kind in ("all", "prefix", "none", "mtp", "all", "mtp", "prefix"):
        if kind == "mtp":
            d = list(m.mtp_draft(pend, 4))
        else:
            d = truth[i + 1:i + 5]
            if kind == "prefix":
                d[2] = (d[2] + 1) % CFG["vocab"]
            elif kind == "none":
                d[0] = (d[0] + 1) % CFG["vocab"]
        k, bonus = m.verify([pend] + d)
        if kind == "all":
            assert k == 4
        elif kind == "prefix":
            assert k == 2
        elif kind == "none":
            assert k == 0
        committed += [pend] + d[:k]
        i += k + 1
        pend = bonus
        assert pend == truth[i]
    assert m.pos == len(committed) - 1
    check_drafts(m, oracle, tensors, committed, pend, 4)


def test_spec_with_mtp_equals_serial(env):
    gpu, ctx, m, _ = env
    prompt = synth.prompt_tokens(13, 30, CFG["vocab"])
    m.reset()
    serial = m.generate_serial(prompt, 48)
    m.reset()
    spec, st = m.generate_spec(prompt, 48, mtp=1, min_draft=1)
    assert np.array_equal(spec, serial)
    assert st.drafted > 0
    m.reset()
    ng, _ = m.generate_spec(prompt, 48, n_key=2, mtp=0)
    assert np.array_equal(ng, serial)


def test_gguf_with_nextn_block_equals_set(env, tmp_path):
    """A GGUF file holding blk.N.nextn.* and blk.N's block (N = n_layers)
    loads the drafter: drafts and their logits equal the set model's, bit for
    bit; without its shared_head_norm the load is refused, naming it."""
    gpu, ctx, m, tensors = env
    from gguf_writer import gguf_bytes, model_gguf_tensors
    gt = model_gguf_tensors(tensors, CFG)
    p = tmp_path / "mtp.gguf"
    p.write_bytes(gguf_bytes(gt))
    g = gpu.GGUF(p)
    mg = gpu.Model(ctx, **CFG)
    mg.load_gguf(g)
    assert mg.has_mtp()
    toks = synth.prompt_tokens(15, 12, CFG["vocab"])
    m.reset()
    pend = int(m.forward(toks)[-1])
    assert int(mg.forward(toks)[-1]) == pend
    a, b = m.mtp_draft(pend, 4), mg.mtp_draft(pend, 4)
    assert np.array_equal(a, b)
    assert np.array_equal(m.mtp_logits(4).view(np.uint32), mg.mtp_logits(4).view(np.uint32))
    mg.free()
    g.close()
    NL = CFG["n_layers"]
    p2 = tmp_path / "partial.gguf"
    p2.write_bytes(gguf_bytes([t for t in gt if t[0] != f"blk.{NL}.nextn.shared_head_norm.weight"]))
    g2 = gpu.GGUF(p2)
    mg2 = gpu.Model(ctx, **CFG)
    with pytest.raises(gpu.CwenError) as e:
        mg2.load_gguf(g2)
    assert f"missing blk.{NL}.nextn.shared_head_norm.weight" in str(e.value)
    mg2.free()
    g2.close()


def test_no_mtp_block_drafts_nothing(env):
    gpu, ctx, _, _ = env
    tensors = list(synth.model_tensors(CFG, seed=0))
    m2 = gpu.Model(ctx, **CFG)
    for t in tensors:
        m2.set(*t)
    assert not m2.has_mtp()
    m2.forward(synth.prompt_tokens(14, 5, CFG["vocab"]))
    assert len(m2.mtp_draft(1, 4)) == 0
    m2.free()
