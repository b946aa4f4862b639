"""The oracle's serial forward (tests/model_oracle.py) pinned to the
reference engine's own model composition at its native dimensions
(H 5120, I 17408, 24/4 heads of 256, GDN 16/48 x 128):

  * a GatedDeltaNet layer (layer_linear, run.c:2323-2358) over 3 positions:
    the residual after each step, and the recurrent state and conv history
    after the last;
  * a full-attention layer (layer_full, run.c:2412-2458) over 4 positions,
    which also exercises its KV cache;
  * the head tail of forward_ex (run.c:2640-2644);
  * the MTP nextn stream: mtp_commit over positions 0..3 (slot 0 only parks,
    run.c:3146-3163) and a draft step (mtp_step, run.c:3099-3133) at slot 4
    on the parked hidden, whose attention reads every committed slot.

Against the reference's AVX2 build live (oracle/_ref, when the reference tree
was built here) and against tests/golden/model_composition.npz (written from
that build by tests/golden/make_model_golden.py), so the pin re-checks where
the reference is absent.  Tolerance (stated): rel_err <= 2e-5, rel_err =
max|d| / max|ref|; the two sides use the same scalar formulas in different
kernel variants (the reference's fused dual-matrix dots and wider
accumulators), so they differ in the last bits only.
"""
import sys
from pathlib import Path

import numpy as np
import pytest

from util import rel_err

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import make_model_golden as mg  # noqa: E402

TOL = 2e-5
GOLDEN = Path(mg.OUT)


@pytest.fixture(scope="module")
def tensors():
    return mg.tensors()


@pytest.fixture(scope="module")
def oracle_outputs(oracle, tensors):
    """The same steps through the oracle's composition."""
    from model_oracle import OracleModel
    OM = OracleModel(oracle, mg.CFG, tensors)
    out = {}
    xs = mg.residuals(mg.N_LIN, 1)
    out["linear_x"] = np.stack([OM.linear_layer(mg.LIN, xs[p]) for p in range(mg.N_LIN)])
    out["linear_S"] = OM.S[mg.LIN][mg.S_HEAD].copy()
    out["linear_hist"] = OM.hist[mg.LIN][:mg.HIST_KEEP].copy()
    xs = mg.residuals(mg.N_FULL, 2)
    out["full_x"] = np.stack([OM.full_layer(mg.FULL, xs[p], p) for p in range(mg.N_FULL)])
    out["head"] = OM.head(mg.residuals(1, 3)[0])
    toks = mg.tokens(mg.N_MTP + 2, 4)
    xs = mg.residuals(mg.N_MTP + 1, 5)
    parked = []
    for p in range(mg.N_MTP + 1):
        OM.mtp_commit(p, int(toks[p]), xs[p])
        assert OM.hpos == p
        parked.append(OM.hprev)
    out["mtp_parked"] = np.stack(parked)
    out["mtp_draft"] = OM.mtp_step(int(toks[mg.N_MTP + 1]), mg.N_MTP + 1, parked[-1])
    return out


KEYS = ["linear_x", "linear_S", "linear_hist", "full_x", "head", "mtp_parked", "mtp_draft"]


@pytest.mark.parametrize("key", KEYS)
def test_oracle_composition_vs_golden(oracle_outputs, key):
    ref = np.load(GOLDEN)[key]
    got = oracle_outputs[key]
    assert got.shape == ref.shape
    assert np.isfinite(ref).all()
    assert rel_err(got, ref) <= TOL, (key, rel_err(got, ref))


def test_oracle_composition_vs_reference(oracle_outputs, ref_avx2, tensors):
    """The live reference build gives the fixture's values (the fixture is
    current) and the oracle matches it."""
    mg.bind(ref_avx2, tensors)
    live = mg.reference_outputs(ref_avx2)
    fx = np.load(GOLDEN)
    for key in KEYS:
        assert np.array_equal(live[key], fx[key]), key
        assert rel_err(oracle_outputs[key], live[key]) <= TOL, (key, rel_err(oracle_outputs[key], live[key]))


def test_reference_block_layers_equal_serial_steps(ref_avx2, tensors):
    """run.c's per-layer block steps (layer_linear_blk / layer_full_blk,
    run.c:2685-2745, which forward_block and so bench.py's CPU verify-cycle
    leg run) give the serial layer steps' residuals on 4 positions, within
    TOL (gemvb and gemv order their sums differently)."""
    R = ref_avx2
    mg.bind(R, tensors)
    X = mg.residuals(8, 6)
    for p in range(4):                       # KV slots 0..3 hold known rows
        R.layer_step(mg.FULL, p, X[p])
    R.snap_save()
    blk = R.block_layer(mg.LIN, 4, X[4:8])
    R.snap_load()
    ser = np.stack([R.layer_step(mg.LIN, 4 + b, X[4 + b]) for b in range(4)])
    assert rel_err(blk, ser) <= TOL, rel_err(blk, ser)
    blk = R.block_layer(mg.FULL, 4, X[4:8])
    ser = np.stack([R.layer_step(mg.FULL, 4 + b, X[4 + b]) for b in range(4)])
    assert rel_err(blk, ser) <= TOL, rel_err(blk, ser)
    assert rel_err(blk, X[4:8]) > 100 * TOL          # the layer did something


def test_composition_catches_a_planted_mistake(oracle, tensors):
    """A mistake planted in the oracle's composition (the post-attention
    norm skipped before the MLP) is far outside the tolerance: the check
    has teeth."""
    from model_oracle import OracleModel

    class Broken(OracleModel):
        def mlp(self, l, x):
            from cwen_amd import gpu as G
            h = self.O.silu_mul(self.mv(l, G.FFN_GATE_UP, x, 0), self.mv(l, G.FFN_GATE_UP, x, 1))
            return (x + self.mv(l, G.FFN_DOWN, h)).astype(np.float32)

    OM = Broken(oracle, mg.CFG, tensors)
    x = OM.linear_layer(mg.LIN, mg.residuals(mg.N_LIN, 1)[0])
    assert rel_err(x, np.load(GOLDEN)["linear_x"][0]) > 100 * TOL


def test_64_layer_fixture_is_consistent():
    """tests/golden/model_64_layer_logits.npz holds run.c's own 64-layer chain
    and the oracle composition on the same weights (written by
    tests/golden/make_drift_golden.py): they agree within the composition's
    tolerance over the whole depth, and rounding only the GEMV inputs to f16
    moves the logits by less than the per-GEMV bound."""
    sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
    import make_drift_golden as dg
    fx = np.load(dg.OUT)
    for p in range(dg.N_POS):
        assert rel_err(fx["logits_oracle"][p], fx["logits_ref"][p]) <= TOL
        assert rel_err(fx["logits_f16_inputs"][p], fx["logits_ref"][p]) <= 1e-3

