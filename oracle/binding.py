"""ctypes binding of the oracle (liboracle.so) and of the reference checker
builds (oracle/_ref/libcwen_ref_*.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product package.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "liboracle.so"
REF_DIR = HERE / "_ref"

_VP, _I, _F = C.c_void_p, C.c_int, C.c_float


class OrcTensor(C.Structure):
    _fields_ = [("data", _VP), ("scales", _VP), ("type", _I), ("ne0", _I), ("ne1", _I),
                ("pair_side", _I)]


def _f32p(a: np.ndarray) -> int:
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data


def _i32p(a: np.ndarray) -> int:
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data


class Oracle:
    """The scalar C restatement (oracle/cwen_oracle.c)."""

    def __init__(self, path: Path = ORACLE_SO):
        if not path.exists():
            raise RuntimeError(f"{path} not built; run `make -C oracle`")
        L = C.CDLL(str(path))
        L.orc_f16_to_f32.restype = _F
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f32_to_f16.argtypes = [_F]
        L.orc_gemvb.restype = _I
        L.orc_gemvb.argtypes = [C.POINTER(OrcTensor), _VP, _I, _VP, _I, _I]
        L.orc_silu_mul.argtypes = [_VP, _VP, _I]
        L.orc_rmsnorm.argtypes = [_VP, _VP, _VP, _I]
        L.orc_conv1d_update.argtypes = [_VP, _VP, _VP, _I]
        L.orc_gdn_step.argtypes = [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _I, _I, _I]
        L.orc_argmax.restype = _I
        L.orc_argmax.argtypes = [_VP, _I]
        L.orc_walk.restype = _I
        L.orc_walk.argtypes = [_VP, C.c_long, _I, _VP, _I, C.POINTER(_I)]
        L.orc_ngram_draft.restype = _I
        L.orc_ngram_draft.argtypes = [_VP, _I, _VP, _I, _I]
        L.orc_embed.argtypes = [_VP, _VP, _I, _I, _I, _VP]
        L.orc_rope_apply.argtypes = [_VP, _I, _I, _I, _I, _I, _F]
        L.orc_attention.argtypes = [_VP, _VP, _I, _I, _I, _I, _VP, _VP, _I, _VP]
        self.L = L

    def gemvb(self, wtype: int, data: np.ndarray, scales, K: int, M: int, X: np.ndarray,
              side: int = 0) -> np.ndarray:
        X = np.ascontiguousarray(X, dtype=np.float32)
        B = X.shape[0]
        Y = np.empty((B, M), dtype=np.float32)
        t = OrcTensor(data.ctypes.data, None if scales is None else scales.ctypes.data,
                      wtype, K, M, side)
        rc = self.L.orc_gemvb(C.byref(t), _f32p(X), K, _f32p(Y), M, B)
        if rc:
            raise RuntimeError(f"orc_gemvb rc={rc}")
        return Y

    def silu_mul(self, a: np.ndarray, b: np.ndarray) -> np.ndarray:
        a = np.array(a, dtype=np.float32, copy=True)
        b = np.ascontiguousarray(b, dtype=np.float32)
        self.L.orc_silu_mul(_f32p(a), _f32p(b), a.size)
        return a

    def rmsnorm(self, x: np.ndarray, w: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        o = np.empty_like(x)
        self.L.orc_rmsnorm(_f32p(o), _f32p(x), _f32p(np.ascontiguousarray(w, np.float32)), x.size)
        return o

    def conv1d_update(self, qkv: np.ndarray, hist: np.ndarray, kw: np.ndarray):
        qkv = np.array(qkv, dtype=np.float32, copy=True)
        hist = np.array(hist, dtype=np.float32, copy=True)
        self.L.orc_conv1d_update(_f32p(qkv), _f32p(hist), _f32p(np.ascontiguousarray(kw, np.float32)),
                                 qkv.size)
        return qkv, hist

    def gdn_step(self, S, qkv, z, decay, beta, wn, nkh, nvh, dk):
        S = np.array(S, dtype=np.float32, copy=True)
        qkv = np.array(qkv, dtype=np.float32, copy=True)
        out = np.empty(nvh * dk, dtype=np.float32)
        args = [np.ascontiguousarray(a, np.float32) for a in (z, decay, beta, wn)]
        self.L.orc_gdn_step(_f32p(S), _f32p(qkv), *(_f32p(a) for a in args), _f32p(out), nkh, nvh, dk)
        return S, qkv, out

    def argmax(self, lg: np.ndarray) -> int:
        lg = np.ascontiguousarray(lg, dtype=np.float32)
        return self.L.orc_argmax(_f32p(lg), lg.size)

    def walk(self, logits: np.ndarray, drafts: np.ndarray) -> tuple[int, int]:
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        d = np.ascontiguousarray(drafts, dtype=np.int32)
        bonus = C.c_int()
        k = self.L.orc_walk(_f32p(logits), logits.shape[1], logits.shape[1], _i32p(d), d.size,
                            C.byref(bonus))
        return k, bonus.value

    def ngram_draft(self, hist: np.ndarray, n_key: int, max_d: int) -> np.ndarray:
        h = np.ascontiguousarray(hist, dtype=np.int32)
        out = np.zeros(max(max_d, 1), dtype=np.int32)
        n = self.L.orc_ngram_draft(_i32p(h), h.size, _i32p(out), n_key, max_d)
        return out[:n]

    def embed(self, wtype: int, qs: np.ndarray, sc, token: int, H: int) -> np.ndarray:
        out = np.empty(H, dtype=np.float32)
        self.L.orc_embed(qs.ctypes.data, None if sc is None else sc.ctypes.data, wtype, token, H, _f32p(out))
        return out

    def rope(self, q: np.ndarray, pos: int, npairs: int = 32, nrot: int = 64, theta: float = 1e7) -> np.ndarray:
        q = np.array(q, dtype=np.float32, copy=True)
        hd = q.shape[-1]
        self.L.orc_rope_apply(_f32p(q), q.size // hd, hd, pos, npairs, nrot, theta)
        return q

    def attention(self, K: np.ndarray, V: np.ndarray, t0: int, pos: int, q: np.ndarray,
                  gate: np.ndarray) -> np.ndarray:
        """K, V [t][nkv][hd]; q, gate [nh][hd] -> out [nh][hd]."""
        K = np.ascontiguousarray(K, np.float32)
        V = np.ascontiguousarray(V, np.float32)
        q = np.ascontiguousarray(q, np.float32)
        gate = np.ascontiguousarray(gate, np.float32)
        nkv, hd = K.shape[1], K.shape[2]
        out = np.empty_like(q)
        self.L.orc_attention(_f32p(K), _f32p(V), nkv, hd, t0, pos, _f32p(q), _f32p(gate), q.shape[0], _f32p(out))
        return out


def cpu_has_avx512() -> bool:
    try:
        flags = Path("/proc/cpuinfo").read_text()
    except OSError:
        return False
    return all(f" {x}" in flags for x in ("avx512f", "avx512bw", "avx512vl", "avx512dq", "avx512_vnni"))


def ref_lib_path(isa: str | None = None) -> Path:
    if isa is None:
        isa = "avx512" if cpu_has_avx512() else "avx2"
    return REF_DIR / f"libcwen_ref_{isa}.so"


class Reference:
    """The reference engine's own kernels, compiled from its run.c (oracle/_ref)."""

    def __init__(self, isa: str | None = None):
        path = ref_lib_path(isa)
        if not path.exists():
            raise RuntimeError(f"{path} not built (needs the reference tree; `make -C oracle`)")
        self.isa = path.stem.split("_")[-1]
        L = C.CDLL(str(path))
        L.ref_vocab.restype = _I
        L.ref_gemv.restype = _I
        L.ref_gemv.argtypes = [_I, _VP, _VP, _I, _I, _I, _VP, _VP]
        L.ref_gemvb.restype = _I
        L.ref_gemvb.argtypes = [_I, _VP, _VP, _I, _I, _I, _VP, _I, _VP, _I, _I]
        L.ref_silu_mul.argtypes = [_VP, _VP, _I]
        L.ref_rmsnorm.argtypes = [_VP, _VP, _VP, _I]
        L.ref_conv1d_update.restype = _I
        L.ref_conv1d_update.argtypes = [_VP, _VP, _VP]
        L.ref_gdn_step.restype = _I
        L.ref_gdn_step.argtypes = [_VP, _VP, _VP, _VP, _VP, _VP, _VP]
        L.ref_argmax.restype = _I
        L.ref_argmax.argtypes = [_VP, _I]
        L.ref_walk.restype = _I
        L.ref_walk.argtypes = [_VP, C.c_long, _I, _VP, _I, C.POINTER(_I)]
        L.ref_ngram_draft.restype = _I
        L.ref_ngram_draft.argtypes = [_VP, _I, _VP, _I, _I]
        L.ref_omp_threads.restype = _I
        L.ref_rope_apply.restype = _I
        L.ref_rope_apply.argtypes = [_VP, _I, _I]
        L.ref_attn_dims.argtypes = [C.POINTER(_I)] * 3
        L.ref_attention.restype = _I
        L.ref_attention.argtypes = [_VP, _VP, _I, _I, _VP, _VP, _VP]
        L.ref_embed.restype = _I
        L.ref_embed.argtypes = [_I, _VP, _VP, _I, _VP]
        L.ref_model_init.restype = _I
        L.ref_model_init.argtypes = [_I]
        L.ref_set_tensor.restype = _I
        L.ref_set_tensor.argtypes = [_I, _I, _I, _VP, _VP, _I, _I]
        L.ref_layer_step.restype = _I
        L.ref_layer_step.argtypes = [_I, _I, _VP]
        L.ref_head.restype = _I
        L.ref_head.argtypes = [_VP, _VP, _I]
        L.ref_gdn_state.restype = _I
        L.ref_gdn_state.argtypes = [_I, _VP, _VP]
        L.ref_mtp_step.restype = _I
        L.ref_mtp_step.argtypes = [_I, _I, _VP, _VP]
        L.ref_mtp_commit.restype = _I
        L.ref_mtp_commit.argtypes = [_I, _I, _VP, _VP]
        L.ref_snap_roundtrip.restype = _I
        L.ref_snap_save.restype = _I
        L.ref_snap_load.restype = _I
        L.ref_block_layer.restype = _I
        L.ref_block_layer.argtypes = [_I, _I, _I, _VP]
        L.ref_ng_init.restype = _I
        L.ref_ng_init.argtypes = [_I]
        L.ref_ng_cap.restype = C.c_long
        L.ref_ng_used.restype = C.c_long
        L.ref_ng_update_key_n.argtypes = [_VP, _I, _I]
        L.ref_ng_update_range.argtypes = [_VP, _I, _I]
        L.ref_ng_draft_map.restype = _I
        L.ref_ng_draft_map.argtypes = [_VP, _I, _VP, _I]
        L.ref_ng_save.argtypes = [C.c_char_p]
        L.ref_ng_load.argtypes = [C.c_char_p]
        L.ref_ng_dump.argtypes = [_VP, _VP, _VP, _VP]
        self.L = L
        self._model_ctx = None
        self._bound = []   # tensors the reference's globals point into, kept alive
        self.vocab = L.ref_vocab()

    def gemvb(self, wtype, data, scales, K, M, X, side=0, out: np.ndarray | None = None):
        X = np.ascontiguousarray(X, dtype=np.float32)
        B = X.shape[0]
        Y = np.empty((B, M), dtype=np.float32) if out is None else out
        rc = self.L.ref_gemvb(wtype, data.ctypes.data, None if scales is None else scales.ctypes.data,
                              K, M, side, _f32p(X), K, Y.ctypes.data, M, B)
        if rc:
            raise RuntimeError(f"ref_gemvb rc={rc}")
        return Y

    def gemv(self, wtype, data, scales, K, M, x, side=0):
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(M, dtype=np.float32)
        rc = self.L.ref_gemv(wtype, data.ctypes.data, None if scales is None else scales.ctypes.data,
                             K, M, side, _f32p(x), _f32p(y))
        if rc:
            raise RuntimeError(f"ref_gemv rc={rc}")
        return y

    def silu_mul(self, a, b):
        a = np.array(a, dtype=np.float32, copy=True)
        self.L.ref_silu_mul(_f32p(a), _f32p(np.ascontiguousarray(b, np.float32)), a.size)
        return a

    def rmsnorm(self, x, w):
        x = np.ascontiguousarray(x, dtype=np.float32)
        o = np.empty_like(x)
        self.L.ref_rmsnorm(_f32p(o), _f32p(x), _f32p(np.ascontiguousarray(w, np.float32)), x.size)
        return o

    def conv1d_update(self, qkv, hist, kw):
        qkv = np.array(qkv, dtype=np.float32, copy=True)
        hist = np.array(hist, dtype=np.float32, copy=True)
        self.L.ref_conv1d_update(_f32p(qkv), _f32p(hist), _f32p(np.ascontiguousarray(kw, np.float32)))
        return qkv, hist

    def gdn_step(self, S, qkv, z, decay, beta, wn):
        S = np.array(S, dtype=np.float32, copy=True)
        qkv = np.array(qkv, dtype=np.float32, copy=True)
        z = np.array(z, dtype=np.float32, copy=True)
        decay = np.array(decay, dtype=np.float32, copy=True)
        beta = np.array(beta, dtype=np.float32, copy=True)
        out = np.empty(48 * 128, dtype=np.float32)
        self.L.ref_gdn_step(_f32p(S), _f32p(qkv), _f32p(z), _f32p(decay), _f32p(beta),
                            _f32p(np.ascontiguousarray(wn, np.float32)), _f32p(out))
        return S, qkv, out

    def argmax(self, lg):
        lg = np.ascontiguousarray(lg, dtype=np.float32)
        return self.L.ref_argmax(_f32p(lg), lg.size)

    def walk(self, logits, drafts):
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        d = np.ascontiguousarray(drafts, dtype=np.int32)
        bonus = C.c_int()
        k = self.L.ref_walk(_f32p(logits), logits.shape[1], logits.shape[1], _i32p(d), d.size,
                            C.byref(bonus))
        return k, bonus.value

    def ngram_draft(self, hist, n_key, max_d):
        h = np.ascontiguousarray(hist, dtype=np.int32)
        out = np.zeros(max(max_d, 1), dtype=np.int32)
        n = self.L.ref_ngram_draft(_i32p(h), h.size, _i32p(out), n_key, max_d)
        return out[:n]

    def attn_dims(self) -> tuple[int, int, int]:
        a, b, c = C.c_int(), C.c_int(), C.c_int()
        self.L.ref_attn_dims(C.byref(a), C.byref(b), C.byref(c))
        return a.value, b.value, c.value

    def rope(self, q: np.ndarray, pos: int) -> np.ndarray:
        q = np.array(q, dtype=np.float32, copy=True)
        if self.L.ref_rope_apply(_f32p(q), q.size // 256, pos):
            raise RuntimeError("ref_rope_apply")
        return q

    def attention(self, K, V, t0, pos, q, gate):
        K = np.ascontiguousarray(K, np.float32)
        V = np.ascontiguousarray(V, np.float32)
        q = np.ascontiguousarray(q, np.float32)
        gate = np.ascontiguousarray(gate, np.float32)
        out = np.empty_like(q)
        if self.L.ref_attention(_f32p(K), _f32p(V), t0, pos, _f32p(q), _f32p(gate), _f32p(out)):
            raise RuntimeError("ref_attention")
        return out

    def embed(self, wtype, qs, sc, token):
        out = np.empty(5120, dtype=np.float32)
        self.L.ref_embed(wtype, qs.ctypes.data, None if sc is None else sc.ctypes.data, token, _f32p(out))
        return out

    # ---- the reference's model composition (ref_harness.c), native dims only
    def model_init(self, ctx: int = 64) -> None:
        """alloc_state with ctx slots (once per process)."""
        if self._model_ctx is None:
            if self.L.ref_model_init(ctx):
                raise RuntimeError("ref_model_init")
            self._model_ctx = ctx
        elif self._model_ctx != ctx:
            raise RuntimeError("the reference's state was allocated with another context")

    def set_tensor(self, layer: int, tid: int, wtype: int, data: np.ndarray, scales, ne0: int, ne1: int) -> None:
        data = np.ascontiguousarray(data)
        sc = None if scales is None else np.ascontiguousarray(scales)
        self._bound.append((data, sc))
        if self.L.ref_set_tensor(layer, tid, wtype, data.ctypes.data, None if sc is None else sc.ctypes.data,
                                 ne0, ne1):
            raise RuntimeError(f"ref_set_tensor({layer}, {tid})")

    def layer_step(self, layer: int, pos: int, x: np.ndarray) -> np.ndarray:
        x = np.array(x, dtype=np.float32, copy=True)
        if self.L.ref_layer_step(layer, pos, _f32p(x)):
            raise RuntimeError("ref_layer_step")
        return x

    def block_layer(self, layer: int, pbase: int, X: np.ndarray) -> np.ndarray:
        """layer_linear_blk / layer_full_blk over rows X[B][H] at positions pbase.. ."""
        X = np.array(X, dtype=np.float32, copy=True, order="C")
        if self.L.ref_block_layer(layer, X.shape[0], pbase, _f32p(X)):
            raise RuntimeError("ref_block_layer")
        return X

    def snap_save(self) -> None:
        if self.L.ref_snap_save():
            raise RuntimeError("ref_snap_save")

    def snap_load(self) -> None:
        if self.L.ref_snap_load():
            raise RuntimeError("ref_snap_load")

    def head(self, x: np.ndarray, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.float32)
        if self.L.ref_head(_f32p(np.ascontiguousarray(x, np.float32)), _f32p(out), n):
            raise RuntimeError("ref_head")
        return out

    def gdn_state(self, layer: int) -> tuple[np.ndarray, np.ndarray]:
        S = np.empty((48, 128, 128), dtype=np.float32)
        hist = np.empty((10240, 3), dtype=np.float32)
        if self.L.ref_gdn_state(layer, _f32p(S), _f32p(hist)):
            raise RuntimeError("ref_gdn_state")
        return S, hist

    def mtp_step(self, tok: int, pos: int, h: np.ndarray) -> np.ndarray:
        out = np.empty(5120, dtype=np.float32)
        if self.L.ref_mtp_step(tok, pos, _f32p(np.ascontiguousarray(h, np.float32)), _f32p(out)):
            raise RuntimeError("ref_mtp_step")
        return out

    def mtp_commit(self, pos: int, tok: int, x_pre: np.ndarray) -> tuple[int, np.ndarray]:
        hprev = np.empty(5120, dtype=np.float32)
        hp = self.L.ref_mtp_commit(pos, tok, _f32p(np.ascontiguousarray(x_pre, np.float32)), _f32p(hprev))
        if hp < -1:
            raise RuntimeError("ref_mtp_commit")
        return hp, hprev

    def snap_roundtrip(self) -> None:
        """snap_save + snap_load over the whole model's GDN state."""
        if self.L.ref_snap_roundtrip():
            raise RuntimeError("ref_snap_roundtrip")

    # ---- the counted n-gram map (run.c:4552-4723) on the reference's globals
    def ng_init(self, n_key: int) -> None:
        if self.L.ref_ng_init(n_key):
            raise RuntimeError("ref_ng_init")
        self._ng_key = n_key

    def ng_update(self, key, tok: int, hits: int = 1) -> None:
        k = np.ascontiguousarray(key, dtype=np.int32)
        self.L.ref_ng_update_key_n(_i32p(k), int(tok), int(hits))

    def ng_update_range(self, hist, a: int, b: int) -> None:
        h = np.ascontiguousarray(hist, dtype=np.int32)
        self.L.ref_ng_update_range(_i32p(h), a, b)

    def ng_draft(self, hist, max_d: int) -> np.ndarray:
        h = np.ascontiguousarray(hist, dtype=np.int32)
        out = np.zeros(max(max_d, 1), dtype=np.int32)
        n = self.L.ref_ng_draft_map(_i32p(h), h.size, _i32p(out), max_d)
        return out[:n]

    def ng_save(self, path) -> None:
        self.L.ref_ng_save(str(path).encode())

    def ng_load(self, path) -> None:
        self.L.ref_ng_load(str(path).encode())

    def ng_used(self) -> int:
        return self.L.ref_ng_used()

    def ng_dump(self) -> tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
        """(keys [cap][n_key], tokens, counts, in-use flags) of the reference's table."""
        cap = self.L.ref_ng_cap()
        keys = np.zeros((cap, self._ng_key), np.int32)
        tok = np.zeros(cap, np.int32)
        cnt = np.zeros(cap, np.int32)
        used = np.zeros(cap, np.uint8)
        self.L.ref_ng_dump(keys.ctypes.data, tok.ctypes.data, cnt.ctypes.data, used.ctypes.data)
        return keys, tok, cnt, used
