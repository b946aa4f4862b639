"""cwen_run, the command-line front end (cwen_amd/host/cwen_run.c), against
the reference's `run` main (run.c:5080-5251): its arguments and exit codes,
its environment knobs (spec_config_init 4021-4052, CWEN_CTX 4100-4104,
strict integers and 0/1 flags 2481-2520), and -- on the GPU -- its output:
the greedy ids of the model in the GGUF file, serial or speculative, one
line on stdout; the frame server on stdin/stdout; the n-gram map kept in
CWEN_NGRAM_CACHE across runs.

The geometry the CLI reads from the tensor shapes (cwen_model_cfg_from_gguf)
is checked on the CPU against the config the file was written from.
"""
import os
import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest

from cwen_amd import synth

ROOT = Path(__file__).resolve().parent.parent
CLI = ROOT / "cwen_amd" / "cwen_run"
CFG = dict(n_layers=4, d_model=1024, d_ffn=2048, vocab=4096, n_head=4, n_kv_head=2, head_dim=256,
           n_rot_pairs=32, n_rot=64, gdn_nkh=2, gdn_nvh=4, gdn_dk=128, full_interval=4, max_ctx=512,
           rope_theta=1e7, rms_eps=1e-6)


def run(*args, env=None, stdin=None, timeout=120):
    if not CLI.exists():
        pytest.skip("cwen_run is not built")
    e = {k: v for k, v in os.environ.items() if not k.startswith("CWEN_")}
    e.update(env or {})
    return subprocess.run([str(CLI), *map(str, args)], env=e, input=stdin, capture_output=True, timeout=timeout)


@pytest.fixture(scope="module")
def model_file(tmp_path_factory):
    from gguf_writer import gguf_bytes, model_gguf_tensors
    tensors = list(synth.model_tensors(CFG, seed=0))
    p = tmp_path_factory.mktemp("cli") / "model.gguf"
    p.write_bytes(gguf_bytes(model_gguf_tensors(tensors, CFG)))
    return p, tensors


# ---------------------------------------------------------------- CPU
def test_help():
    r = run("--help")
    assert r.returncode == 0 and r.stdout.startswith(b"usage: cwen_run")
    assert run("-h").returncode == 0


@pytest.mark.parametrize("args,why", [
    (["-x"], b"unknown option"),
    (["m.gguf", "-d"], b"needs a value"),
    (["m.gguf", "-d", "0"], b"-d must be an integer in [1, 15]"),
    (["m.gguf", "--draft-tokens", "16"], b"must be an integer in [1, 15]"),
    (["m.gguf", "--spec-draft-n-max", "x"], b"must be an integer"),
    (["a", "b", "x"], b"N_PREDICT must be an integer"),
    (["a", "b", "-1"], b"unknown option '-1'"),          # a leading '-' is an option, as in the reference
    (["a", "b", "3", "d"], b"at most 3 arguments"),
])
def test_bad_arguments_exit_2(args, why):
    r = run(*args)
    assert r.returncode == 2 and why in r.stderr, r.stderr


@pytest.mark.parametrize("env,why", [
    ({"CWEN_SPEC": "2"}, b"CWEN_SPEC must be 0 or 1"),
    ({"CWEN_SERVER": "yes"}, b"CWEN_SERVER must be 0 or 1"),
    ({"CWEN_SPEC_NGRAM_N": "1"}, b"CWEN_SPEC_NGRAM_N must be an integer in [2, 256]"),
    ({"CWEN_SPEC_MAX_DRAFT": "16"}, b"CWEN_SPEC_MAX_DRAFT must be an integer in [1, 15]"),
    ({"CWEN_SPEC_MAX_DRAFT": "4", "CWEN_SPEC_MIN_DRAFT": "5"}, b"CWEN_SPEC_MIN_DRAFT must be an integer in [1, 4]"),
    # run.c:4045-4050: the default minimum draft (2) above a maximum of 1
    ({"CWEN_SPEC_MAX_DRAFT": "1"}, b"CWEN_SPEC_MIN_DRAFT (2) exceeds CWEN_SPEC_MAX_DRAFT (1)"),
    ({"CWEN_SPEC_COOLDOWN": "-1"}, b"CWEN_SPEC_COOLDOWN must be an integer"),
    ({"CWEN_CTX": "63"}, b"CWEN_CTX must be an integer in [64, 32768]"),
    ({"CWEN_CTX": "4k"}, b"CWEN_CTX must be an integer"),
    ({"CWEN_DUMP": "/tmp/x"}, b"CWEN_DUMP is not supported"),
    ({"CWEN_ROPE_YARN": "8192,4"}, b"CWEN_ROPE_YARN is not supported"),
    ({"CWEN_DFLASH": "d.spec"}, b"CWEN_DFLASH is not supported"),
])
def test_bad_knobs_exit_1_before_loading(env, why):
    r = run("does-not-exist.gguf", env=env)
    assert r.returncode == 1 and why in r.stderr, r.stderr
    assert b"cannot open" not in r.stderr      # refused before the model file is touched


def test_missing_model_exits_1():
    r = run("does-not-exist.gguf")
    assert r.returncode == 1 and b"cannot open file" in r.stderr


def test_geometry_from_tensor_shapes(model_file, tmp_path):
    """The config read back from the file's shapes is the one it was written
    from; a file without attention layers is refused, naming what is missing."""
    from cwen_amd import gpu
    from gguf_writer import gguf_bytes, model_gguf_tensors
    p, tensors = model_file
    got = gpu.GGUF(p).model_cfg(512)
    for k, v in CFG.items():
        assert got[k] == pytest.approx(v), k
    gt = [t for t in model_gguf_tensors(tensors, CFG) if "attn_q." not in t[0]]
    q = tmp_path / "noattn.gguf"
    q.write_bytes(gguf_bytes(gt))
    with pytest.raises(gpu.CwenError) as e:
        gpu.GGUF(q).model_cfg(512)
    assert "full-attention" in str(e.value)


def test_geometry_of_the_27b_shape():
    """The reference's compiled geometry (run.c:83-91) from tensor headers of
    its shapes: a file holding only the tensors the geometry reads."""
    from cwen_amd import gpu
    from gguf_writer import gguf_bytes
    F32, Q4 = 0, 2

    def t(name, ne0, ne1, typ=Q4):
        nb = ne0 * ne1 * 4 if typ == F32 else ne0 // 32 * 18 * ne1
        return (name, typ, (ne0, ne1) if ne1 > 1 else (ne0,), b"\0" * nb)
    ts = [t("token_embd.weight", 5120, 64)]   # vocab comes from ne1: kept small here, checked below
    for l in range(64):
        ts.append(t(f"blk.{l}.attn_norm.weight", 32, 1, F32))
    ts += [t("blk.0.ffn_down.weight", 17408, 1), t("blk.3.attn_q.weight", 512, 12288),
           t("blk.3.attn_q_norm.weight", 256, 1, F32), t("blk.3.attn_k.weight", 512, 1024),
           t("blk.0.ssm_norm.weight", 128, 1, F32), t("blk.0.ssm_alpha.weight", 512, 48),
           t("blk.0.attn_qkv.weight", 512, 10240), t("blk.64.attn_norm.weight", 32, 1, F32),
           t("blk.64.nextn.eh_proj.weight", 512, 1)]
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        p = Path(d) / "shape.gguf"
        p.write_bytes(gguf_bytes(ts))
        c = gpu.GGUF(p).model_cfg(4096)
    want = dict(n_layers=64, d_model=5120, d_ffn=17408, vocab=64, n_head=24, n_kv_head=4, head_dim=256,
                n_rot_pairs=32, n_rot=64, gdn_nkh=16, gdn_nvh=48, gdn_dk=128, full_interval=4, max_ctx=4096)
    for k, v in want.items():
        assert c[k] == v, k


# ---------------------------------------------------------------- GPU
def _ids_file(tmp_path, ids):
    p = tmp_path / "prompt.bin"
    p.write_bytes(np.asarray(ids, "<i4").tobytes())
    return p


def _tokens(stdout: bytes) -> list[int]:
    assert stdout.endswith(b"\n") and stdout.count(b"\n") == 1
    return [int(x) for x in stdout.split()]


@pytest.fixture(scope="module")
def reference_stream(model_file):
    """Serial greedy decode of the same model through the library."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from cwen_amd import gpu
    p, tensors = model_file
    ctx = gpu.Context(0)
    m = gpu.Model(ctx, **CFG)
    for t in tensors:
        m.set(*t)
    prompt = synth.prompt_tokens(8, 48, CFG["vocab"], period=9, noise=0.05)
    serial = m.generate_serial(prompt, 40)
    m.free()
    torch.cuda.synchronize()
    return prompt, serial


@pytest.mark.gpu
def test_cli_serial_and_speculative(model_file, reference_stream, tmp_path):
    p, _ = model_file
    prompt, serial = reference_stream
    ids = _ids_file(tmp_path, prompt)
    env = {"CWEN_CTX": "512"}
    r = run(p, ids, 40, env=env)
    assert r.returncode == 0, r.stderr
    assert _tokens(r.stdout) == serial.tolist()
    for extra, spec_env in (([], {"CWEN_SPEC": "1"}), (["-d", "4"], {}), ([], {"CWEN_SPEC": "1", "CWEN_MTP": "0"})):
        r = run(p, ids, 40, *extra, env={**env, **spec_env})
        assert r.returncode == 0, r.stderr
        assert _tokens(r.stdout) == serial.tolist()
        assert b"with drafts" in r.stderr
    r = run(p, ids, 0, env=env)            # prefill only
    assert r.returncode == 0 and r.stdout == b""


@pytest.mark.gpu
def test_cli_context_cap_and_bad_ids(model_file, reference_stream, tmp_path):
    p, _ = model_file
    prompt, serial = reference_stream
    ids = _ids_file(tmp_path, prompt)
    # room for 64 - 48 ids only; the attention's chunking follows the context
    # length, so the library model it is compared with has the same one
    from cwen_amd import gpu
    _, tensors = model_file
    m = gpu.Model(gpu.Context(0), **{**CFG, "max_ctx": 64})
    for t in tensors:
        m.set(*t)
    want = m.generate_serial(prompt, 40)
    m.free()
    assert want.size == 16
    r = run(p, ids, 40, env={"CWEN_CTX": "64"})
    assert r.returncode == 0 and _tokens(r.stdout) == want.tolist()
    assert b"filled after 16 of 40" in r.stderr
    bad = _ids_file(tmp_path, [1, 2, CFG["vocab"]])
    r = run(p, bad, 4, env={"CWEN_CTX": "512"})
    assert r.returncode == 1 and b"outside the vocabulary" in r.stderr
    r = run(p, env={"CWEN_CTX": "512"})           # the default prompt id is beyond this vocabulary
    assert r.returncode == 1 and b"give IDS_FILE" in r.stderr


@pytest.mark.gpu
def test_cli_server_frames(model_file, reference_stream):
    p, _ = model_file
    prompt, serial = reference_stream
    frame = struct.pack("<II", prompt.size, 24) + prompt.astype("<i4").tobytes()
    bad = struct.pack("<II", 2, 5) + np.array([1, CFG["vocab"]], "<i4").tobytes()
    for env in ({"CWEN_SERVER": "1", "CWEN_CTX": "512"}, {"CWEN_SERVER": "1", "CWEN_CTX": "512", "CWEN_SPEC": "1"}):
        r = run(p, env=env, stdin=frame + bad + frame)
        assert r.returncode == 0, r.stderr
        out = np.frombuffer(r.stdout, "<u4")
        want = [24] + serial[:24].tolist()
        assert out.tolist() == want + [0] + want


@pytest.mark.gpu
def test_cli_ngram_cache_persists(model_file, reference_stream, tmp_path):
    """With CWEN_NGRAM_CACHE the map is saved at the end of a run (an NGC2
    file of the run's key length and the model's vocabulary) and merged at the
    start of the next; the ids are the same either way."""
    p, _ = model_file
    prompt, serial = reference_stream
    ids = _ids_file(tmp_path, prompt)
    cache = tmp_path / "map.ngc"
    env = {"CWEN_CTX": "512", "CWEN_SPEC": "1", "CWEN_SPEC_NGRAM_N": "4", "CWEN_NGRAM_CACHE": str(cache)}
    r = run(p, ids, 40, env=env)
    assert r.returncode == 0 and _tokens(r.stdout) == serial.tolist()
    assert b"no file at" in r.stderr
    magic, nk, vocab, used = struct.unpack("<4I", cache.read_bytes()[:16])
    assert (magic, nk, vocab) == (0x3243474E, 4, CFG["vocab"]) and used > 0
    r = run(p, ids, 40, env=env)
    assert r.returncode == 0 and _tokens(r.stdout) == serial.tolist()
    assert f"{used} entries merged".encode() in r.stderr
    r = run(p, ids, 8, env={"CWEN_CTX": "512", "CWEN_NGRAM_CACHE": str(cache)})
    assert r.returncode == 0 and b"no effect without CWEN_SPEC=1" in r.stderr
