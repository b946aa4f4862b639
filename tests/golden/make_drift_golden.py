"""Writes tests/golden/model_64_layer_logits.npz: the logits of a 64-layer
model at the reference's native dimensions (H 5120, I 17408, 24/4 heads of
256, GatedDeltaNet 16/48 x 128, every 4th layer full attention) after a few
tokens, so tests/test_model_drift_gpu.py can state how far the device path
drifts from the reference over the real depth.

    python tests/golden/make_drift_golden.py        # needs oracle/_ref built; ~10 min, ~14 GB RAM

Three restatements of the same serial forward, all from the seeded weights
of cwen_amd.synth.model_tensors:
  * logits_ref: run.c's own layer chain -- layer_linear / layer_full for
    each of the 64 layers and the head tail of forward_ex (run.c:2323-2358,
    2412-2458, 2640-2644), through oracle/_ref, after the oracle's embedding
    (pinned to run.c's embed_token_to);
  * logits_oracle: the oracle composition (tests/model_oracle.py);
  * logits_f16_inputs: the oracle with every GEMV input rounded to f16 first,
    the one precision choice of the device path: how much that rounding alone
    moves the logits at this depth.
"""
from __future__ import annotations

import sys
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
for p in (ROOT, ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

OUT = HERE / "model_64_layer_logits.npz"
CFG = dict(n_layers=64, d_model=5120, d_ffn=17408, vocab=2048, n_head=24, n_kv_head=4, head_dim=256,
           n_rot_pairs=32, n_rot=64, gdn_nkh=16, gdn_nvh=48, gdn_dk=128, full_interval=4, max_ctx=64,
           rope_theta=1e7, rms_eps=1e-6)
SEED = 41
TOK_SEED = 42
N_POS = 4


def tokens() -> np.ndarray:
    from cwen_amd import synth
    return synth.prompt_tokens(TOK_SEED, N_POS, CFG["vocab"])


def main() -> None:
    from cwen_amd import gpu as G, synth
    from model_oracle import OracleModel
    from oracle.binding import Oracle, Reference
    t0 = time.time()
    ts = list(synth.model_tensors(CFG, seed=SEED))
    print(f"weights {sum(t[3].nbytes for t in ts) / 1e9:.1f} GB in {time.time() - t0:.0f} s", flush=True)
    toks = tokens()
    O = Oracle()
    out = {"tokens": toks}
    # run.c's layer chain
    R = Reference("avx2")
    R.model_init(CFG["max_ctx"])
    for layer, tid, wtype, data, sc, ne0, ne1 in ts:
        R.set_tensor(layer, tid, wtype, data, sc, ne0, ne1)
    wtype, qs, sc, H, _ = next((t[2], t[3], t[4], t[5], t[6]) for t in ts if t[0] == -1 and t[1] == G.TOK_EMBD)
    ref = []
    for p, tok in enumerate(toks):
        x = O.embed(wtype, qs, sc, int(tok), H)
        for l in range(CFG["n_layers"]):
            x = R.layer_step(l, p, x)
        ref.append(R.head(x, CFG["vocab"]))
        print(f"reference position {p} at {time.time() - t0:.0f} s", flush=True)
    out["logits_ref"] = np.stack(ref)
    for key, f16 in (("logits_oracle", False), ("logits_f16_inputs", True)):
        OM = OracleModel(O, CFG, ts, f16_inputs=f16)
        rows = []
        for p, tok in enumerate(toks):
            rows.append(OM.step(int(tok), p))
            print(f"{key} position {p} at {time.time() - t0:.0f} s", flush=True)
        out[key] = np.stack(rows)
    np.savez_compressed(OUT, **out)
    rel = lambda a, b: float(np.abs(a - b).max() / np.abs(b).max())
    for p in range(N_POS):
        print(f"position {p}: oracle vs run.c {rel(out['logits_oracle'][p], out['logits_ref'][p]):.2e}, "
              f"f16 inputs vs run.c {rel(out['logits_f16_inputs'][p], out['logits_ref'][p]):.2e}", flush=True)
    print(f"wrote {OUT}", flush=True)


if __name__ == "__main__":
    main()
