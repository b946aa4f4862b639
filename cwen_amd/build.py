"""Build recipe for the native parts of cwen_amd (in-tree, no JIT cache).

    python -m cwen_amd.build          # libcwen_gpu.so (HIP, gfx950) and the rest

Produces cwen_amd/libcwen_gpu.so from cwen_amd/csrc/*.hip with hipcc, the host
library and CLI from cwen_amd/host, and cwen_amd/libcwen_probe.so (bench.py's
read-stream probes, cwen_amd/probe) -- a measurement aid, not part of the
product library.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "libcwen_gpu.so"
HOST_LIB = PKG / "libcwen_host.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Packed-FP32 VALU ops are disabled for all device code; hipcc's host pass
# warns that it does not know the feature, which is harmless.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
    # MFMA results in VGPRs: the epilogue reads them with VALU ops directly
    # instead of a v_accvgpr_read per element.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    f"-I{ROOT / 'include'}", f"-I{CSRC}",
]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        out = "\n".join(line for line in (r.stdout + r.stderr).splitlines()
                        if "packed-fp32-ops" not in line)
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")


def build_gpu(verbose: bool = False) -> Path:
    OBJ.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    if not srcs:
        raise RuntimeError("no HIP sources")
    objs = [OBJ / (s.stem + ".o") for s in srcs]

    def comp(pair):
        s, o = pair
        _run([HIPCC, *HIP_FLAGS, "-c", str(s), "-o", str(o)])
        return o

    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        list(ex.map(comp, zip(srcs, objs)))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


def build_host(verbose: bool = False) -> Path:
    """The C host drivers (cwen_amd/host), linked against libcwen_gpu.so."""
    srcs = [PKG / "host" / f for f in ("cwen_host.c", "cwen_ngram.c", "cwen_gguf.c", "cwen_serve.c")]
    tmp = HOST_LIB.with_suffix(".so.tmp")
    _run(["gcc", "-O2", "-std=c11", "-Wall", "-Wextra", "-fPIC", "-shared", f"-I{ROOT / 'include'}",
          *map(str, srcs), f"-L{PKG}", "-lcwen_gpu", "-Wl,-rpath,$ORIGIN", "-o", str(tmp)])
    os.replace(tmp, HOST_LIB)
    if verbose:
        print(f"built {HOST_LIB}")
    return HOST_LIB


PROBE_LIB = PKG / "libcwen_probe.so"


def build_probe(verbose: bool = False) -> Path:
    """The read-stream probes bench.py times for its HBM-ceiling leg."""
    tmp = PROBE_LIB.with_suffix(".so.tmp")
    _run([HIPCC, *HIP_FLAGS, "-shared", str(PKG / "probe" / "stream_probe.hip"), "-o", str(tmp)])
    os.replace(tmp, PROBE_LIB)
    if verbose:
        print(f"built {PROBE_LIB}")
    return PROBE_LIB


CLI = PKG / "cwen_run"


def build_cli(verbose: bool = False) -> Path:
    """cwen_run, the command-line front end (cwen_amd/host/cwen_run.c), linked
    against libcwen_host.so and libcwen_gpu.so next to it."""
    tmp = CLI.with_suffix(".tmp")
    _run(["gcc", "-O2", "-std=c11", "-Wall", "-Wextra", f"-I{ROOT / 'include'}", f"-I{PKG / 'host'}",
          str(PKG / "host" / "cwen_run.c"), f"-L{PKG}", "-lcwen_host", "-lcwen_gpu", "-Wl,-rpath,$ORIGIN",
          "-o", str(tmp)])
    os.replace(tmp, CLI)
    if verbose:
        print(f"built {CLI}")
    return CLI


def build_oracle(verbose: bool = False) -> None:
    """Test infrastructure: the oracle restatement and, if the reference tree
    is present, the reference checker builds (oracle/Makefile)."""
    r = subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{r.stdout}{r.stderr}")
    if verbose:
        print("built oracle")


if __name__ == "__main__":
    build_gpu(verbose=True)
    build_host(verbose=True)
    build_cli(verbose=True)
    build_probe(verbose=True)
    if "--oracle" in sys.argv:
        build_oracle(verbose=True)
