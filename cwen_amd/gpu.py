"""ctypes binding of libcwen_gpu.so (the C ABI in include/cwen_gpu.h).

This is plumbing for Python callers (tests, bench): every compute call goes
straight to the HIP library.  Importing it on a machine without the built
library raises; there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libcwen_gpu.so"
HOST_LIB_PATH = Path(__file__).resolve().parent / "libcwen_host.so"

CWEN_OK = 0
CWEN_ERANGE = -6
ERRORS = {-1: "EINVAL", -2: "EHIP", -3: "ENOMEM", -4: "ETYPE", -5: "ESCRATCH", -6: "ERANGE", -7: "EIO"}

T_F32, T_Q4_0, T_Q4_1, T_Q8_0, T_Q5_K, T_Q6_K, T_Q4_0RS, T_Q4_0RSI = 0, 2, 3, 8, 13, 14, 101, 102
BMAX = 16

# (name, restype, argtypes) of every exported entry point.
_VP, _I, _F = C.c_void_p, C.c_int, C.POINTER(C.c_float)
SIGNATURES = [
    ("cwen_version", C.c_char_p, []),
    ("cwen_ctx_create", _I, [_I, C.POINTER(_VP)]),
    ("cwen_ctx_destroy", _I, [_VP]),
    ("cwen_weight_upload", _I, [_VP, _I, _VP, _VP, _I, _I, C.POINTER(_VP)]),
    ("cwen_weight_free", _I, [_VP]),
    ("cwen_weight_info", _I, [_VP, C.POINTER(_I), C.POINTER(_I), C.POINTER(_I), C.POINTER(_I),
                              C.POINTER(C.c_size_t)]),
    ("cwen_gemvb", _I, [_VP, _VP, _I, _VP, _I, _VP, _I, _I, _VP]),
    ("cwen_gemvb_pair", _I, [_VP, _VP, _VP, _I, _VP, _VP, _I, _I, _VP]),
    ("cwen_gemvb_swiglu", _I, [_VP, _VP, _VP, _I, _VP, _I, _I, _VP]),
    ("cwen_mlp_block", _I, [_VP, _VP, _VP, _VP, _I, _VP, _I, _I, _VP]),
    ("cwen_mlp_block_noalloc", _I, [_VP, _VP, _VP, _I, _VP, _I, _I, _VP]),
    ("cwen_act_to_f16", _I, [_VP, _VP, _I, _VP, _I, _I, _VP]),
    ("cwen_gemvb_f16", _I, [_VP, _VP, _I, _VP, _VP, _I, _VP, _I, _I, _VP]),
    ("cwen_gemvb_swiglu_f16", _I, [_VP, _VP, _VP, _VP, _I, _VP, _I, _VP]),
    ("cwen_head_verify", _I, [_VP, _VP, _VP, _I, _I, _VP, _I, _VP, _I, _VP, _VP]),
    ("cwen_argmax_walk", _I, [_VP, _VP, _I, _I, _I, _VP, _I, _VP, _VP]),
    ("cwen_gdn_create", _I, [_VP, _I, _I, _I, C.POINTER(_VP)]),
    ("cwen_gdn_free", _I, [_VP]),
    ("cwen_gdn_set_state", _I, [_VP, _VP, _VP]),
    ("cwen_gdn_get_state", _I, [_VP, _I, _VP, _VP]),
    ("cwen_gdn_block", _I, [_VP, _VP, _VP, _I, _VP, _I, _VP, _VP, _I, _VP, _VP, _VP, _I, _I, _VP]),
    ("cwen_gdn_commit", _I, [_VP, _I]),
    ("cwen_model_create", _I, [_VP, _VP, C.POINTER(_VP)]),
    ("cwen_model_free", _I, [_VP]),
    ("cwen_model_set", _I, [_VP, _I, _I, _I, _VP, _VP, _I, _I]),
    ("cwen_model_reset", _I, [_VP]),
    ("cwen_model_synth", _I, [_VP, C.c_ulonglong]),
    ("cwen_model_pos", _I, [_VP]),
    ("cwen_model_capacity", _I, [_VP]),
    ("cwen_model_forward", _I, [_VP, _VP, _I, _I, _VP, _VP]),
    ("cwen_model_verify", _I, [_VP, _VP, _I, C.POINTER(_I), C.POINTER(_I), _VP]),
    ("cwen_model_logits", _I, [_VP, _VP, _I]),
    ("cwen_model_has_mtp", _I, [_VP]),
    ("cwen_model_mtp_draft", _I, [_VP, _I, _I, _VP, _VP]),
    ("cwen_model_mtp_logits", _I, [_VP, _VP, _I]),
]

# libcwen_host.so (include/.. cwen_amd/host/cwen_host.h)
HOST_SIGNATURES = [
    ("cwen_spec_default", None, [_VP]),
    ("cwen_ngram_draft", _I, [_VP, _I, _VP, _I, _I]),
    ("cwen_prefill", _I, [_VP, _VP, _I, C.POINTER(_I)]),
    ("cwen_generate_serial", _I, [_VP, _VP, _I, _I, _VP, _VP]),
    ("cwen_generate_spec", _I, [_VP, _VP, _I, _I, _VP, _VP, _VP]),
    ("cwen_spec_replay", _I, [_VP, _I, _I, _I, _I, _VP, _VP, _VP]),
    ("cwen_ngmap_create", _I, [_I, _I, C.c_size_t, C.POINTER(_VP)]),
    ("cwen_ngmap_free", None, [_VP]),
    ("cwen_ngmap_n_key", _I, [_VP]),
    ("cwen_ngmap_used", C.c_size_t, [_VP]),
    ("cwen_ngmap_evictions", None, [_VP, C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]),
    ("cwen_ngmap_update", None, [_VP, _VP, _I, _I]),
    ("cwen_ngmap_update_range", None, [_VP, _VP, _I, _I]),
    ("cwen_ngmap_draft", _I, [_VP, _VP, _I, _VP, _I]),
    ("cwen_ngmap_save", _I, [_VP, C.c_char_p]),
    ("cwen_ngmap_load", _I, [_VP, C.c_char_p]),
    ("cwen_ngmap_dump", _I, [_VP, _VP, _VP, _VP, _VP]),
    ("cwen_gguf_open", _I, [C.c_char_p, C.POINTER(_VP)]),
    ("cwen_gguf_close", None, [_VP]),
    ("cwen_gguf_error", C.c_char_p, []),
    ("cwen_gguf_count", _I, [_VP]),
    ("cwen_gguf_tensor", _I, [_VP, _I, C.POINTER(C.c_char_p), C.POINTER(_I), C.POINTER(_I), C.POINTER(_I),
                              C.POINTER(_VP)]),
    ("cwen_gguf_find", _I, [_VP, C.c_char_p]),
    ("cwen_gguf_tensor_scales", _I, [_VP, _I, C.POINTER(_VP), C.POINTER(_I)]),
    ("cwen_cwenr_path", _I, [C.c_char_p, C.c_char_p, C.c_size_t]),
    ("cwen_gguf_apply_cwenr", _I, [_VP, C.c_char_p, C.c_char_p]),
    ("cwen_f32_to_f16", C.c_uint16, [C.c_float]),
    ("cwen_model_load_gguf", _I, [_VP, _VP, _VP]),
    ("cwen_model_cfg_from_gguf", _I, [_VP, _I, _VP]),
    ("cwen_read_frame", _I, [_I, _VP, _I, _I, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32)]),
    ("cwen_serve", _I, [_VP, _VP, _I, _I, _VP, C.POINTER(_I)]),
]


class CwenError(RuntimeError):
    def __init__(self, fn: str, rc: int):
        super().__init__(f"{fn} failed: {rc} ({ERRORS.get(rc, '?')})")
        self.rc = rc


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run `python -m cwen_amd.build`")
        L = C.CDLL(str(LIB_PATH))
        for name, res, args in SIGNATURES:
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


_hlib = None


def host_lib() -> C.CDLL:
    global _hlib
    if _hlib is None:
        lib()  # the host library resolves libcwen_gpu.so next to it
        if not HOST_LIB_PATH.exists():
            raise RuntimeError(f"{HOST_LIB_PATH} is not built; run `python -m cwen_amd.build`")
        L = C.CDLL(str(HOST_LIB_PATH))
        for name, res, args in HOST_SIGNATURES:
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _hlib = L
    return _hlib


def check(fn: str, rc: int) -> None:
    if rc != CWEN_OK:
        raise CwenError(fn, rc)


def _ptr(t) -> int | None:
    """Device pointer of a torch tensor (or raw int, or None)."""
    if t is None:
        return None
    return t if isinstance(t, int) else t.data_ptr()


def _stream(stream) -> int | None:
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    return stream if isinstance(stream, int) else stream.cuda_stream


class Context:
    def __init__(self, device: int = 0):
        h = C.c_void_p()
        check("cwen_ctx_create", lib().cwen_ctx_create(device, C.byref(h)))
        self.h = h

    def close(self) -> None:
        if self.h:
            lib().cwen_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Weight:
    """A device-resident weight uploaded from a reference layout (host arrays)."""

    def __init__(self, ctx: Context, wtype: int, data: np.ndarray, scales: np.ndarray | None,
                 ne0: int, ne1: int):
        data = np.ascontiguousarray(data)
        sc = None if scales is None else np.ascontiguousarray(scales)
        h = C.c_void_p()
        check("cwen_weight_upload",
              lib().cwen_weight_upload(ctx.h, wtype, data.ctypes.data,
                                       None if sc is None else sc.ctypes.data,
                                       ne0, ne1, C.byref(h)))
        self.h, self.ctx, self.type, self.K, self.M = h, ctx, wtype, ne0, ne1

    def info(self) -> dict:
        t, k, m, ns = C.c_int(), C.c_int(), C.c_int(), C.c_int()
        sb = C.c_size_t()
        check("cwen_weight_info", lib().cwen_weight_info(self.h, C.byref(t), C.byref(k), C.byref(m),
                                                         C.byref(ns), C.byref(sb)))
        return {"type": t.value, "ne0": k.value, "ne1": m.value, "nside": ns.value,
                "stream_bytes": sb.value}

    def free(self) -> None:
        if self.h:
            lib().cwen_weight_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def gemvb(ctx: Context, W: Weight, X, Y, B: int, side: int = 0, xs: int | None = None,
          ys: int | None = None, stream=None) -> None:
    xs = W.K if xs is None else xs
    ys = W.M if ys is None else ys
    check("cwen_gemvb", lib().cwen_gemvb(ctx.h, W.h, side, _ptr(X), xs, _ptr(Y), ys, B, _stream(stream)))


def gemvb_pair(ctx: Context, W: Weight, X, YA, YB, B: int, xs: int | None = None,
               ys: int | None = None, stream=None) -> None:
    xs = W.K if xs is None else xs
    ys = W.M if ys is None else ys
    check("cwen_gemvb_pair", lib().cwen_gemvb_pair(ctx.h, W.h, _ptr(X), xs, _ptr(YA), _ptr(YB), ys, B,
                                                   _stream(stream)))


def gemvb_swiglu(ctx: Context, W: Weight, X, H, B: int, xs: int | None = None,
                 hs: int | None = None, stream=None) -> None:
    xs = W.K if xs is None else xs
    hs = W.M if hs is None else hs
    check("cwen_gemvb_swiglu", lib().cwen_gemvb_swiglu(ctx.h, W.h, _ptr(X), xs, _ptr(H), hs, B,
                                                       _stream(stream)))


def mlp_block(ctx: Context, Wgu: Weight, Wd: Weight, X, Y, B: int, xs: int | None = None,
              ys: int | None = None, stream=None) -> None:
    """Y += down(silu(gate X) * (up X)) -- the block FFN (mlp_blk)."""
    xs = Wgu.K if xs is None else xs
    ys = Wd.M if ys is None else ys
    check("cwen_mlp_block", lib().cwen_mlp_block(ctx.h, Wgu.h, Wd.h, _ptr(X), xs, _ptr(Y), ys, B,
                                                 _stream(stream)))


def mlp_block_noalloc(Wgu: Weight, Wd: Weight, X, Y, B: int, xs: int | None = None,
                      ys: int | None = None, stream=None) -> None:
    """mlp_block on the library's static per-GPU scratch (no allocation, no
    context scratch); raises CwenError(ESCRATCH) beyond its limits."""
    xs = Wgu.K if xs is None else xs
    ys = Wd.M if ys is None else ys
    check("cwen_mlp_block_noalloc", lib().cwen_mlp_block_noalloc(Wgu.h, Wd.h, _ptr(X), xs, _ptr(Y), ys, B,
                                                                 _stream(stream)))


def act_to_f16(ctx: Context, X, Xh, K: int, B: int, xs: int | None = None, stream=None) -> None:
    xs = K if xs is None else xs
    check("cwen_act_to_f16", lib().cwen_act_to_f16(ctx.h, _ptr(X), xs, _ptr(Xh), K, B, _stream(stream)))


def gemvb_f16(ctx: Context, W: Weight, Xh, Y, B: int, side: int = 0, Yh=None, accumulate: bool = False,
              ys: int | None = None, stream=None) -> None:
    ys = W.M if ys is None else ys
    check("cwen_gemvb_f16", lib().cwen_gemvb_f16(ctx.h, W.h, side, _ptr(Xh), _ptr(Y), ys, _ptr(Yh),
                                                 int(accumulate), B, _stream(stream)))


def gemvb_swiglu_f16(ctx: Context, W: Weight, Xh, H, B: int, Hh=None, hs: int | None = None,
                     stream=None) -> None:
    hs = W.M if hs is None else hs
    check("cwen_gemvb_swiglu_f16", lib().cwen_gemvb_swiglu_f16(ctx.h, W.h, _ptr(Xh), _ptr(H), hs, _ptr(Hh),
                                                               B, _stream(stream)))


def head_verify(ctx: Context, W: Weight, X, B: int, res, drafts=None, E: int = 0, logits=None,
                xs: int | None = None, ls: int | None = None, stream=None) -> None:
    """Head GEMV + per-column argmax + greedy walk; res (device int32 [2+B]) gets
    k, bonus, argmax of each column."""
    xs = W.K if xs is None else xs
    ls = W.M if ls is None else ls
    check("cwen_head_verify", lib().cwen_head_verify(ctx.h, W.h, _ptr(X), xs, B, _ptr(drafts), E,
                                                     _ptr(logits), ls, _ptr(res), _stream(stream)))


def argmax_walk(ctx: Context, logits, V: int, B: int, res, drafts=None, E: int = 0, ls: int | None = None,
                stream=None) -> None:
    ls = V if ls is None else ls
    check("cwen_argmax_walk", lib().cwen_argmax_walk(ctx.h, _ptr(logits), ls, V, B, _ptr(drafts), E,
                                                     _ptr(res), _stream(stream)))


class GDN:
    """One GatedDeltaNet layer's device state with its snapshot ring."""

    def __init__(self, ctx: Context, nkh: int, nvh: int, dk: int = 128):
        h = C.c_void_p()
        check("cwen_gdn_create", lib().cwen_gdn_create(ctx.h, nkh, nvh, dk, C.byref(h)))
        self.h, self.ctx, self.nkh, self.nvh, self.dk = h, ctx, nkh, nvh, dk
        self.C = (2 * nkh + nvh) * dk

    def set_state(self, S: np.ndarray | None, hist: np.ndarray | None) -> None:
        S = None if S is None else np.ascontiguousarray(S, dtype=np.float32)
        hist = None if hist is None else np.ascontiguousarray(hist, dtype=np.float32)
        check("cwen_gdn_set_state", lib().cwen_gdn_set_state(
            self.h, None if S is None else S.ctypes.data, None if hist is None else hist.ctypes.data))

    def get_state(self, pos: int = 0) -> tuple[np.ndarray, np.ndarray]:
        S = np.empty((self.nvh, self.dk, self.dk), dtype=np.float32)
        hist = np.empty((self.C, 3), dtype=np.float32)
        check("cwen_gdn_get_state", lib().cwen_gdn_get_state(self.h, pos, S.ctypes.data, hist.ctypes.data))
        return S, hist

    def block(self, qkv, z, decay, beta, kw, wn, out, B: int, qs=None, zs=None, gs=None, os_=None,
              stream=None) -> None:
        zh = self.nvh * self.dk
        check("cwen_gdn_block", lib().cwen_gdn_block(
            self.ctx.h, self.h, _ptr(qkv), self.C if qs is None else qs, _ptr(z), zh if zs is None else zs,
            _ptr(decay), _ptr(beta), self.nvh if gs is None else gs, _ptr(kw), _ptr(wn), _ptr(out),
            zh if os_ is None else os_, B, _stream(stream)))

    def commit(self, n: int) -> None:
        check("cwen_gdn_commit", lib().cwen_gdn_commit(self.h, n))

    def free(self) -> None:
        if self.h:
            lib().cwen_gdn_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ---------------------------------------------------------------- model
class ModelCfg(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_layers", "d_model", "d_ffn", "vocab", "n_head", "n_kv_head",
                                        "head_dim", "n_rot_pairs", "n_rot", "gdn_nkh", "gdn_nvh", "gdn_dk",
                                        "full_interval", "max_ctx")] + \
              [("rope_theta", C.c_float), ("rms_eps", C.c_float)]


(TOK_EMBD, OUTPUT_NORM, OUTPUT, ATTN_NORM, POST_NORM, FFN_GATE_UP, FFN_DOWN, ATTN_QKV, ATTN_GATE, SSM_ALPHA,
 SSM_BETA, SSM_A, SSM_DT, SSM_CONV, SSM_NORM, SSM_OUT, ATTN_Q, ATTN_KV, ATTN_OUTPUT, ATTN_Q_NORM,
 ATTN_K_NORM, NEXTN_EH_PROJ, NEXTN_ENORM, NEXTN_HNORM, NEXTN_SHEAD_NORM) = range(25)


class SpecCfg(C.Structure):
    _fields_ = [("n_key", C.c_int), ("max_draft", C.c_int), ("min_draft", C.c_int), ("cooldown", C.c_int),
                ("max_cycles", C.c_int), ("mtp", C.c_int), ("ngmap", C.c_void_p), ("cycle_log", C.c_void_p),
                ("cycle_log_cap", C.c_int), ("debug", C.c_int), ("fa_streak", C.c_void_p)]


def spec_cfg(n_key: int = 16, max_draft: int = 8, min_draft: int = 2, cooldown: int = 8, max_cycles: int = 0,
             mtp: int = 1, ngmap: "NgMap | None" = None, cycle_log: np.ndarray | None = None,
             debug: int = 0, fa_streak: np.ndarray | None = None) -> SpecCfg:
    """A speculation config; cycle_log (int32, even length) receives (E, k) per cycle;
    fa_streak (one int32) carries the full-accept streak from call to call."""
    if fa_streak is not None and (fa_streak.dtype != np.int32 or fa_streak.size < 1):
        raise ValueError("fa_streak must be an int32 array of at least one element")
    return SpecCfg(n_key, max_draft, min_draft, cooldown, max_cycles, mtp, None if ngmap is None else ngmap.h,
                   None if cycle_log is None else cycle_log.ctypes.data,
                   0 if cycle_log is None else cycle_log.size // 2, debug,
                   None if fa_streak is None else fa_streak.ctypes.data)


class NgMap:
    """The host library's counted n-gram map (cwen_ngmap_*; no GPU needed)."""

    def __init__(self, n_key: int = 16, vocab: int = 248320, cap: int = 0):
        h = C.c_void_p()
        check("cwen_ngmap_create", host_lib().cwen_ngmap_create(n_key, vocab, cap, C.byref(h)))
        self.h, self.n_key = h, n_key
        self.cap = cap or (1 << 18)

    def update(self, key, tok: int, hits: int = 1) -> None:
        k = np.ascontiguousarray(key, dtype=np.int32)
        host_lib().cwen_ngmap_update(self.h, k.ctypes.data, int(tok), int(hits))

    def update_range(self, hist, a: int, b: int) -> None:
        h = np.ascontiguousarray(hist, dtype=np.int32)
        host_lib().cwen_ngmap_update_range(self.h, h.ctypes.data, a, b)

    def draft(self, hist, max_d: int) -> np.ndarray:
        h = np.ascontiguousarray(hist, dtype=np.int32)
        out = np.zeros(max(max_d, 1), dtype=np.int32)
        n = host_lib().cwen_ngmap_draft(self.h, h.ctypes.data, h.size, out.ctypes.data, max_d)
        return out[:n]

    def save(self, path) -> None:
        check("cwen_ngmap_save", host_lib().cwen_ngmap_save(self.h, str(path).encode()))

    def load(self, path) -> int:
        n = host_lib().cwen_ngmap_load(self.h, str(path).encode())
        if n < 0:
            raise CwenError("cwen_ngmap_load", n)
        return n

    def used(self) -> int:
        return host_lib().cwen_ngmap_used(self.h)

    def evictions(self) -> tuple[int, int]:
        """(entries evicted, evictions that shifted no entry into the freed slot)."""
        a, b = C.c_size_t(), C.c_size_t()
        host_lib().cwen_ngmap_evictions(self.h, C.byref(a), C.byref(b))
        return a.value, b.value

    def dump(self) -> tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
        keys = np.zeros((self.cap, self.n_key), np.int32)
        tok = np.zeros(self.cap, np.int32)
        cnt = np.zeros(self.cap, np.int32)
        used = np.zeros(self.cap, np.uint8)
        check("cwen_ngmap_dump", host_lib().cwen_ngmap_dump(self.h, keys.ctypes.data, tok.ctypes.data,
                                                            cnt.ctypes.data, used.ctypes.data))
        return keys, tok, cnt, used

    def free(self) -> None:
        if self.h:
            host_lib().cwen_ngmap_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def spec_replay(stream, n_prompt: int, n_gen: int, max_ctx: int, cfg: SpecCfg) -> tuple[np.ndarray, "SpecStats"]:
    """cwen_spec_replay: the speculative driver against a recorded greedy stream."""
    s = np.ascontiguousarray(stream, dtype=np.int32)
    out = np.zeros(max(n_gen, 1), dtype=np.int32)
    st = SpecStats()
    n = host_lib().cwen_spec_replay(s.ctypes.data, s.size, n_prompt, n_gen, max_ctx, C.byref(cfg), out.ctypes.data,
                                    C.byref(st))
    if n < 0:
        raise CwenError("cwen_spec_replay", n)
    return out[:n], st


class SpecStats(C.Structure):
    _fields_ = [("cycles", C.c_longlong), ("drafted", C.c_longlong), ("full", C.c_longlong),
                ("rejected", C.c_longlong), ("kept", C.c_longlong), ("prefill_tokens", C.c_int),
                ("prefill_s", C.c_double), ("decode_s", C.c_double)]


def read_frame(fd: int, max_ctx: int, vocab: int) -> tuple[int, np.ndarray | None, int]:
    """One request frame from fd (cwen_read_frame): (1, prompt, n_gen) for a
    valid frame, (0, None, 0) for a rejected one, (2, None, 0) at the end of
    the stream."""
    toks = np.zeros(max_ctx, np.int32)
    n_p, n_g = C.c_uint32(), C.c_uint32()
    r = host_lib().cwen_read_frame(fd, toks.ctypes.data, max_ctx, vocab, C.byref(n_p), C.byref(n_g))
    if r < 0:
        raise CwenError("cwen_read_frame", r)
    return (1, toks[:n_p.value].copy(), n_g.value) if r == 1 else (r, None, 0)


class GGUF:
    """A GGUF file mapped by the host library (cwen_gguf_*); no GPU needed."""

    def __init__(self, path):
        h = C.c_void_p()
        rc = host_lib().cwen_gguf_open(str(path).encode(), C.byref(h))
        if rc != CWEN_OK:
            raise CwenError(f"cwen_gguf_open ({host_lib().cwen_gguf_error().decode()})", rc)
        self.h = h

    def __len__(self) -> int:
        return host_lib().cwen_gguf_count(self.h)

    def tensor(self, i: int) -> tuple[str, int, int, int, int]:
        """(name, GGUF type, ne0, ne1, data address)."""
        name, t, a, b, d = C.c_char_p(), _I(), _I(), _I(), C.c_void_p()
        check("cwen_gguf_tensor", host_lib().cwen_gguf_tensor(self.h, i, C.byref(name), C.byref(t), C.byref(a),
                                                              C.byref(b), C.byref(d)))
        return name.value.decode(), t.value, a.value, b.value, d.value

    def find(self, name: str) -> int:
        return host_lib().cwen_gguf_find(self.h, name.encode())

    def scales(self, i: int) -> tuple[int | None, int]:
        """(f16 scale address, pair side) of a tensor a sidecar rebound."""
        sc, side = C.c_void_p(), _I()
        check("cwen_gguf_tensor_scales", host_lib().cwen_gguf_tensor_scales(self.h, i, C.byref(sc), C.byref(side)))
        return sc.value, side.value

    def apply_cwenr(self, path, src_gguf=None) -> int:
        """Rebind the Q4_0 tensors a CWENR sidecar holds; the number rebound
        (0: no file, or no entry applies)."""
        rc = host_lib().cwen_gguf_apply_cwenr(self.h, str(path).encode(),
                                              None if src_gguf is None else str(src_gguf).encode())
        if rc < 0:
            raise CwenError(f"cwen_gguf_apply_cwenr ({host_lib().cwen_gguf_error().decode()})", rc)
        return rc

    @staticmethod
    def cwenr_path(gguf_path) -> str:
        buf = C.create_string_buffer(4096)
        check("cwen_cwenr_path", host_lib().cwen_cwenr_path(str(gguf_path).encode(), buf, len(buf)))
        return buf.value.decode()

    @staticmethod
    def last_error() -> str:
        return host_lib().cwen_gguf_error().decode()

    def model_cfg(self, max_ctx: int = 4096) -> dict:
        """The model geometry read from the tensor shapes (cwen_model_cfg_from_gguf)."""
        c = ModelCfg()
        rc = host_lib().cwen_model_cfg_from_gguf(self.h, max_ctx, C.byref(c))
        if rc != CWEN_OK:
            raise CwenError(f"cwen_model_cfg_from_gguf ({host_lib().cwen_gguf_error().decode()})", rc)
        return {name: getattr(c, name) for name, _ in ModelCfg._fields_}

    def close(self) -> None:
        if self.h:
            host_lib().cwen_gguf_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Model:
    """The block-verify model on one device (cwen_model_* of the C ABI)."""

    def __init__(self, ctx: Context, **cfg):
        self.cfg = ModelCfg(**cfg)
        h = C.c_void_p()
        check("cwen_model_create", lib().cwen_model_create(ctx.h, C.byref(self.cfg), C.byref(h)))
        self.h, self.ctx = h, ctx

    def set(self, layer: int, tid: int, wtype: int, data: np.ndarray, scales: np.ndarray | None,
            ne0: int, ne1: int) -> None:
        data = np.ascontiguousarray(data)
        sc = None if scales is None else np.ascontiguousarray(scales)
        check("cwen_model_set", lib().cwen_model_set(self.h, layer, tid, wtype, data.ctypes.data,
                                                     None if sc is None else sc.ctypes.data, ne0, ne1))

    def reset(self) -> None:
        check("cwen_model_reset", lib().cwen_model_reset(self.h))

    def synth(self, seed: int = 0) -> None:
        """Device-generated random-init weights (cwen_model_synth)."""
        check("cwen_model_synth", lib().cwen_model_synth(self.h, seed))

    @property
    def pos(self) -> int:
        return lib().cwen_model_pos(self.h)

    def forward(self, toks, want_argmax: bool = True) -> np.ndarray | None:
        t = np.ascontiguousarray(toks, dtype=np.int32)
        am = np.zeros(t.size, dtype=np.int32)
        check("cwen_model_forward", lib().cwen_model_forward(self.h, t.ctypes.data, t.size, int(want_argmax),
                                                             am.ctypes.data if want_argmax else None, None))
        return am if want_argmax else None

    def verify(self, blk) -> tuple[int, int]:
        t = np.ascontiguousarray(blk, dtype=np.int32)
        k, bonus = C.c_int(), C.c_int()
        check("cwen_model_verify", lib().cwen_model_verify(self.h, t.ctypes.data, t.size, C.byref(k),
                                                           C.byref(bonus), None))
        return k.value, bonus.value

    def logits(self, rows: int) -> np.ndarray:
        out = np.empty((rows, self.cfg.vocab), dtype=np.float32)
        check("cwen_model_logits", lib().cwen_model_logits(self.h, out.ctypes.data, rows))
        return out

    def has_mtp(self) -> bool:
        return lib().cwen_model_has_mtp(self.h) == 1

    def mtp_draft(self, pend: int, n: int) -> np.ndarray:
        """Up to n greedy drafts of the MTP block after the last filled position."""
        out = np.zeros(max(n, 1), dtype=np.int32)
        k = lib().cwen_model_mtp_draft(self.h, int(pend), n, out.ctypes.data, None)
        if k < 0:
            raise CwenError("cwen_model_mtp_draft", k)
        return out[:k]

    def mtp_logits(self, rows: int) -> np.ndarray:
        out = np.empty((rows, self.cfg.vocab), dtype=np.float32)
        check("cwen_model_mtp_logits", lib().cwen_model_mtp_logits(self.h, out.ctypes.data, rows))
        return out

    def generate_serial(self, prompt, n_gen: int, with_stats: bool = False):
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(n_gen, dtype=np.int32)
        st = SpecStats()
        n = host_lib().cwen_generate_serial(self.h, p.ctypes.data, p.size, n_gen, out.ctypes.data, C.byref(st))
        if n < 0:
            raise CwenError("cwen_generate_serial", n)
        return (out[:n], st) if with_stats else out[:n]

    def generate_spec(self, prompt, n_gen: int, n_key: int = 16, max_draft: int = 8, min_draft: int = 2,
                      cooldown: int = 8, max_cycles: int = 0, mtp: int = 1, ngmap: NgMap | None = None,
                      cycle_log: np.ndarray | None = None) -> tuple[np.ndarray, SpecStats]:
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(n_gen, dtype=np.int32)
        cfg = spec_cfg(n_key, max_draft, min_draft, cooldown, max_cycles, mtp, ngmap, cycle_log)
        st = SpecStats()
        n = host_lib().cwen_generate_spec(self.h, p.ctypes.data, p.size, n_gen, C.byref(cfg), out.ctypes.data,
                                          C.byref(st))
        if n < 0:
            raise CwenError("cwen_generate_spec", n)
        return out[:n], st

    def serve(self, fd_in: int, fd_out: int, spec: SpecCfg | None = None) -> int:
        """Answer request frames from fd_in on fd_out until the stream ends
        (cwen_serve); the number of valid frames answered."""
        n = _I()
        check("cwen_serve", host_lib().cwen_serve(self.h, C.byref(self.cfg), fd_in, fd_out,
                                                  None if spec is None else C.byref(spec), C.byref(n)))
        return n.value

    def load_gguf(self, g: "GGUF") -> None:
        """Upload the verify path's tensors from a GGUF file (cwen_model_load_gguf)."""
        rc = host_lib().cwen_model_load_gguf(self.h, C.byref(self.cfg), g.h)
        if rc != CWEN_OK:
            raise CwenError(f"cwen_model_load_gguf ({host_lib().cwen_gguf_error().decode()})", rc)

    def free(self) -> None:
        if self.h:
            lib().cwen_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
