"""Writes tests/golden/model_composition.npz: outputs of the reference engine's
own model composition -- layer_linear, layer_full, the head tail of
forward_ex, mtp_step and mtp_commit (run.c:2323-2358, 2412-2458, 2640-2644,
3099-3163), called through oracle/_ref's AVX2 build at the reference's native
dimensions -- so tests/test_model_composition.py can pin the oracle's serial
forward (tests/model_oracle.py) where the reference tree is absent.

    python tests/golden/make_model_golden.py        # needs oracle/_ref built

Inputs come from the seeded generators below (numpy PCG64 via cwen_amd.synth),
so only outputs are stored: the residual after every step, a slice of the
recurrent state and conv history, a prefix of the head's logits, and the
nextn block's outputs and parked hidden.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
for p in (ROOT, ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

OUT = HERE / "model_composition.npz"

# The reference's compile-time geometry (run.c:83-88); 4 layers are enough to
# hold one GatedDeltaNet layer (0) and one full-attention layer (3), the MTP
# block sits after them.  The head and the embedding keep VH rows.
CFG = dict(n_layers=4, d_model=5120, d_ffn=17408, vocab=4096, n_head=24, n_kv_head=4, head_dim=256,
           n_rot_pairs=32, n_rot=64, gdn_nkh=16, gdn_nvh=48, gdn_dk=128, full_interval=4, max_ctx=64,
           rope_theta=1e7, rms_eps=1e-6)
SEED = 31
LIN, FULL = 0, 3                 # a linear and a full-attention layer
N_LIN, N_FULL, N_MTP = 3, 4, 3   # positions stepped
REF_MTP_LAYER = 64               # the reference's nextn block (NW) after its 64 layers
S_HEAD = 5                       # value head of the recurrent state stored
HIST_KEEP = 512                  # conv channels of the history stored


def tensors():
    """The layers LIN and FULL, the globals and the MTP block, in the
    reference's layouts (cwen_amd.synth.model_tensors' generator)."""
    from cwen_amd import synth
    keep = {-1, LIN, FULL, CFG["n_layers"]}
    return [t for t in synth.model_tensors(CFG, seed=SEED, mtp=True) if t[0] in keep]


def residuals(n: int, key: int) -> np.ndarray:
    """Residual-stream inputs: f32 N(0, 1) rows scaled by 0.5."""
    from cwen_amd import synth
    return (0.5 * synth.activations(SEED, n, CFG["d_model"], key=key)).astype(np.float32)


def tokens(n: int, key: int) -> np.ndarray:
    from cwen_amd import synth
    return synth.prompt_tokens(SEED + key, n, CFG["vocab"])


def bind(R, ts) -> None:
    R.model_init(CFG["max_ctx"])
    for layer, tid, wtype, data, sc, ne0, ne1 in ts:
        R.set_tensor(REF_MTP_LAYER if layer == CFG["n_layers"] else layer, tid, wtype, data, sc, ne0, ne1)


def reference_outputs(R) -> dict:
    out = {}
    xs = residuals(N_LIN, 1)
    out["linear_x"] = np.stack([R.layer_step(LIN, p, xs[p]) for p in range(N_LIN)])
    S, hist = R.gdn_state(LIN)
    out["linear_S"] = S[S_HEAD].copy()
    out["linear_hist"] = hist[:HIST_KEEP].copy()
    xs = residuals(N_FULL, 2)
    out["full_x"] = np.stack([R.layer_step(FULL, p, xs[p]) for p in range(N_FULL)])
    out["head"] = R.head(residuals(1, 3)[0], CFG["vocab"])
    # the nextn stream: commit positions 0..N_MTP (slot 0 only parks), then a
    # draft step at slot N_MTP + 1 on the parked hidden
    toks = tokens(N_MTP + 2, 4)
    xs = residuals(N_MTP + 1, 5)
    parked = []
    for p in range(N_MTP + 1):
        hp, hprev = R.mtp_commit(p, int(toks[p]), xs[p])
        assert hp == p
        parked.append(hprev)
    out["mtp_parked"] = np.stack(parked)
    out["mtp_draft"] = R.mtp_step(int(toks[N_MTP + 1]), N_MTP + 1, parked[-1])
    return out


def main() -> None:
    from oracle.binding import Reference
    R = Reference("avx2")
    bind(R, tensors())
    out = reference_outputs(R)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: " + ", ".join(f"{k} {v.shape}" for k, v in out.items()))


if __name__ == "__main__":
    main()
