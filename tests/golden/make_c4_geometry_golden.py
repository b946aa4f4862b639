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
composed from the C restatement) -- "ref"; the same with every GEMV input
rounded to f16 first -- "ref16"; the oracle's device-rounding mode
(tests/device_round.py) -- "refdev"; and "jit", how far that mode's logits
move when each f16 operand is perturbed by 1e-6 * max|x| first (the larger of
two seeded trials), the position's sensitivity to f32-level differences.

    python tests/golden/make_c4_geometry_golden.py --device [--wide]

adds "refdev" and "jit" to an existing file (three more serial passes).
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


JITTER = 1e-6


def add_device(n_ctx: int, out_path: Path) -> None:
    """Adds the device-rounding mode's logits and their sensitivity."""
    import device_round
    from cwen_amd import synth
    from model_oracle import OracleModel
    from oracle.binding import Oracle
    sys.path.insert(0, str(ROOT / "tests"))
    from util import rel_err
    O = Oracle()
    tensors = list(synth.model_tensors(CFG, seed=SEED))
    toks = tokens(n_ctx)
    old = dict(np.load(out_path))
    runs = []
    for trial in range(3):
        t0 = time.time()
        device_round.JITTER = 0.0 if trial == 0 else JITTER
        device_round.seed_jitter(trial)
        om = OracleModel(O, CFG, tensors, device=True)
        rows = []
        for p, t in enumerate(toks):
            lg = om.step(int(t), p)
            if p >= n_ctx - N_CMP:
                rows.append(lg)
        runs.append(np.stack(rows).astype(np.float32))
        print(f"device trial {trial}: {time.time() - t0:.0f} s", flush=True)
    device_round.JITTER = 0.0
    jit = np.array([max(rel_err(runs[1][i], runs[0][i]), rel_err(runs[2][i], runs[0][i])) for i in range(N_CMP)])
    old["refdev"], old["jit"] = runs[0], jit.astype(np.float64)
    np.savez_compressed(out_path, **old)
    print(f"wrote {out_path}: jit max {jit.max():.2e}")


if __name__ == "__main__":
    n, path = (N_CTX_WIDE, OUT_WIDE) if "--wide" in sys.argv else (N_CTX, OUT)
    if "--device" in sys.argv:
        add_device(n, path)
    else:
        main(n, path)
