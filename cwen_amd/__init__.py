"""cwen_amd: MI355X (gfx950) implementation of cwen's speculative
block-verify hot path.  The product is the C-ABI library libcwen_gpu.so
(include/cwen_gpu.h) built from cwen_amd/csrc; `cwen_amd.gpu` is its ctypes
binding and `cwen_amd.synth` generates the seeded synthetic workloads."""

__all__ = ["gpu", "synth", "build"]
