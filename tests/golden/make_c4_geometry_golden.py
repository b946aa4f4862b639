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

adds "refdev" and "jit" to an existing file (three more serial passes, with
the oracle's BLAS attention, np_attention).

    python tests/golden/make_c4_geometry_golden.py --long 16k|32k

writes c4_geometry_{16k,32k}_logits.npz: the same model in a 32768-slot
cache over 16448 and 32736 tokens (the attention merge then sums 128 and
256 key chunks per group), with "ref" (the plain oracle), "refdev" and
"jit", all with np_attention (the C restatement's attention would take hours
at these contexts; tests/test_device_round.py pins np_attention to it).
Roughly 10 and 40 minutes.
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
LONG_CFG = {**CFG, "max_ctx": 32768}
N_CTX_LONG = {"16k": 16448, "32k": 32736}   # 514 and 1023 key chunks of 32


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


def add_device(n_ctx: int, out_path: Path, cfg: dict = CFG, plain: bool = False) -> None:
    """Adds the device-rounding mode's logits and their sensitivity (and,
    with plain, the plain oracle's logits) to out_path, created if absent."""
    import device_round
    from cwen_amd import synth
    from model_oracle import OracleModel
    from oracle.binding import Oracle
    sys.path.insert(0, str(ROOT / "tests"))
    from util import rel_err
    O = Oracle()
    tensors = list(synth.model_tensors(cfg, seed=SEED))
    toks = tokens(n_ctx)
    old = dict(np.load(out_path)) if out_path.exists() else {"n_ctx": np.int32(n_ctx), "n_cmp": np.int32(N_CMP)}
    runs = []
    for trial in range(4 if plain else 3):
        t0 = time.time()
        device_round.JITTER = JITTER if trial in (1, 2) else 0.0
        device_round.seed_jitter(trial)
        om = OracleModel(O, cfg, tensors, device=trial < 3, fast_attention=True)
        rows = []
        for p, t in enumerate(toks):
            lg = om.step(int(t), p)
            if p >= n_ctx - N_CMP:
                rows.append(lg)
            if p % 4096 == 4095:
                print(f"  trial {trial}: {p + 1} positions, {time.time() - t0:.0f} s", flush=True)
        runs.append(np.stack(rows).astype(np.float32))
        print(f"trial {trial}: {time.time() - t0:.0f} s", flush=True)
    device_round.JITTER = 0.0
    jit = np.array([max(rel_err(runs[1][i], runs[0][i]), rel_err(runs[2][i], runs[0][i])) for i in range(N_CMP)])
    old["refdev"], old["jit"] = runs[0], jit.astype(np.float64)
    if plain:
        old["ref"] = runs[3]
    np.savez_compressed(out_path, **old)
    print(f"wrote {out_path}: jit max {jit.max():.2e}")


if __name__ == "__main__":
    if "--long" in sys.argv:
        which = sys.argv[sys.argv.index("--long") + 1]
        add_device(N_CTX_LONG[which], HERE / f"c4_geometry_{which}_logits.npz", LONG_CFG, plain=True)
        sys.exit(0)
    n, path = (N_CTX_WIDE, OUT_WIDE) if "--wide" in sys.argv else (N_CTX, OUT)
    if "--device" in sys.argv:
        add_device(n, path)
    else:
        main(n, path)
