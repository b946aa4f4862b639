"""Writes tests/golden/c4_geometry_logits.npz: the oracle's logits for the
last positions of a 4224-token context on a small model with the 27B
shape's attention geometry, and c4_geometry_wide_logits.npz the same for a
6400-token context (past 6144 positions the chunk kernel takes its wide
grid) (24 query heads, 4 KV heads of dim 256: 6 query
heads per KV head), so the device's long-context attention paths can be
compared with the oracle where the GPU tests run, without re-running 4224
serial oracle steps there.

    python tests/golden/make_c4_geometry_golden.py          # a few minutes
    python tests/golden/make_c4_geometry_golden.py --wide   # about 10 minutes

The model and the tokens come from the seeded generators of cwen_amd.synth
(numpy PCG64 streams), so only the outputs are stored: for each compared
position the logits of the oracle's serial forward (tests/model_oracle.py,
composed from the C restatement), and the same with every GEMV input rounded
to f16 first (the device's operand precision), which measures how sensitive
each position is to that rounding.
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

OUT = HERE / "c4_geometry_logits.npz"
OUT_WIDE = HERE / "c4_geometry_wide_logits.npz"

# The 27B shape's attention geometry at small d_model / d_ffn / vocab: layer 0
# GatedDeltaNet, layer 1 full attention.
CFG = dict(n_layers=2, d_model=512, d_ffn=1024, vocab=2048, n_head=24, n_kv_head=4, head_dim=256,
           n_rot_pairs=32, n_rot=64, gdn_nkh=2, gdn_nvh=4, gdn_dk=128, full_interval=2, max_ctx=8192,
           rope_theta=1e7, rms_eps=1e-6)
SEED, TOK_SEED = 21, 22
N_CTX = 4224               # > 4096: 132 key chunks of 32, three per chunk workgroup (64 per KV head)
N_CTX_WIDE = 6400          # 200 key chunks: past 192 the chunk kernel takes its wide grid (128 per KV head)
N_CMP = 32                 # last positions compared: one block of 16, two of 8


def tokens(n: int = N_CTX) -> np.ndarray:
    from cwen_amd import synth
    return synth.prompt_tokens(TOK_SEED, n, CFG["vocab"], period=41, noise=0.1)


def main(n_ctx: int = N_CTX, out_path: Path = OUT) -> None:
    from cwen_amd import synth
    from model_oracle import OracleModel
    from oracle.binding import Oracle
    O = Oracle()
    tensors = list(synth.model_tensors(CFG, seed=SEED))
    toks = tokens(n_ctx)
    out = {}
    for name, f16 in (("ref", False), ("ref16", True)):
        t0 = time.time()
        om = OracleModel(O, CFG, tensors, f16_inputs=f16)
        rows = []
        for p, t in enumerate(toks):
            lg = om.step(int(t), p)
            if p >= n_ctx - N_CMP:
                rows.append(lg)
        out[name] = np.stack(rows).astype(np.float32)
        print(f"{name}: {time.time() - t0:.0f} s", flush=True)
    np.savez_compressed(out_path, n_ctx=np.int32(n_ctx), n_cmp=np.int32(N_CMP), **out)
    print(f"wrote {out_path}")


if __name__ == "__main__":
    if "--wide" in sys.argv:
        main(N_CTX_WIDE, OUT_WIDE)
    else:
        main()
