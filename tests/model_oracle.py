"""Serial forward pass of the hybrid decoder composed from the oracle's C
restatements (test infrastructure).  Mirrors forward_ex / layer_linear /
layer_full / mlp of the reference (run.c:2594-2645, 2325-2358, 2412-2458,
2205-2321) one position at a time, and, when the tensors hold an MTP block,
its nextn stream: mtp_step / mtp_commit / mtp_draft (run.c:3099-3187)."""
import numpy as np

T_F32, T_Q4_0RS, T_Q4_0RSI, T_Q6_K = 0, 101, 102, 14


def np_attention(Kg: np.ndarray, Vg: np.ndarray, t0: int, pos: int, q: np.ndarray, gate: np.ndarray) -> np.ndarray:
    """The oracle's gated attention (orc_attention, after run.c:2362-2409):
    per query head h of KV group h // (nh / nkv), softmax over keys t0..pos of
    (q . k) / sqrt(hd), the weighted sum of the values, times sigmoid(gate),
    in f32 with BLAS products.  Kg, Vg are group-major [nkv][t][hd]."""
    nkv, hd = Kg.shape[0], Kg.shape[2]
    nh = q.shape[0]
    kvm = nh // nkv
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    out = np.empty((nh, hd), np.float32)
    for g in range(nkv):
        s = (q[g * kvm:(g + 1) * kvm].astype(np.float32) @ Kg[g, t0:pos + 1].T) * scale
        e = np.exp(s - s.max(axis=1, keepdims=True))
        e /= e.sum(axis=1, keepdims=True)
        out[g * kvm:(g + 1) * kvm] = e @ Vg[g, t0:pos + 1]
    g32 = np.asarray(gate, np.float32)
    return (out * (np.float32(1.0) / (np.float32(1.0) + np.exp(-g32)))).astype(np.float32)


class OracleModel:
    """f16_inputs: round every GEMV input to f16 first, used by the tests to
    measure how sensitive a position's logits are to that rounding.

    device: round where the device rounds (tests/device_round.py) -- f16
    weights from each format's one-rounding formula, f16 GEMV operands, an
    RMSNorm input rounded as f16(x * w) with the norm scale applied to the
    GEMV's output -- and sum the GEMVs in float64; everything else is the
    C restatement, as in the other modes.  The device's logits differ from
    this mode only by the order of its f32 sums."""

    def __init__(self, O, cfg: dict, tensors, f16_inputs: bool = False, device: bool = False,
                 fast_attention: bool = False):
        self.O, self.c = O, cfg
        self.f16_inputs = f16_inputs
        self.device = device
        # fast_attention: np_attention (BLAS, f32) instead of the C restatement
        # of the attention, for contexts of tens of thousands of positions.
        self.fast_attention = fast_attention
        self.w16 = {}
        self.g = {}
        self.t = {}
        for layer, tid, wtype, data, sc, ne0, ne1 in tensors:
            self.t[(layer, tid)] = (wtype, data, sc, ne0, ne1)
        c = cfg
        self.C = (2 * c["gdn_nkh"] + c["gdn_nvh"]) * 128
        from cwen_amd import gpu as G
        self.has_mtp = (-1, G.NEXTN_EH_PROJ) in self.t
        self.reset()

    def reset(self):
        c = self.c
        self.S = {}
        self.hist = {}
        self.K = {}
        self.V = {}
        for l in range(c["n_layers"]):
            if l % c["full_interval"] == c["full_interval"] - 1:
                self.K[l] = np.zeros((c["max_ctx"], c["n_kv_head"], c["head_dim"]), np.float32)
                self.V[l] = np.zeros_like(self.K[l])
            else:
                self.S[l] = np.zeros((c["gdn_nvh"], 128, 128), np.float32)
                self.hist[l] = np.zeros((self.C, 3), np.float32)
        NL = c["n_layers"]
        self.K[NL] = np.zeros((c["max_ctx"], c["n_kv_head"], c["head_dim"]), np.float32)
        self.V[NL] = np.zeros_like(self.K[NL])
        # group-major copies [n_kv_head][max_ctx][head_dim] for np_attention
        self.Kg = {l: np.zeros((c["n_kv_head"], c["max_ctx"], c["head_dim"]), np.float32)
                   for l in self.K} if self.fast_attention else {}
        self.Vg = {l: np.zeros_like(a) for l, a in self.Kg.items()}
        self.hprev, self.hpos = None, -1

    def _w16(self, layer, tid, side):
        key = (layer, tid, side)
        if key not in self.w16:
            import device_round
            wtype, data, sc, ne0, ne1 = self.t[(layer, tid)]
            self.w16[key] = device_round.weights(wtype, data, sc, ne0, ne1, side)
        return self.w16[key]

    def mv(self, layer, tid, x, side=0):
        """GEMV of tensor (layer, tid) on input x."""
        if self.device:
            import device_round
            return device_round.gemv(self._w16(layer, tid, side), device_round.operand(x))
        wtype, data, sc, ne0, ne1 = self.t[(layer, tid)]
        if self.f16_inputs:
            x = x.astype(np.float16).astype(np.float32)
        return self.O.gemvb(wtype, data, sc, ne0, ne1, x[None, :], side)[0]

    def mvn(self, layer, tid, x, wn, side=0):
        """GEMV of tensor (layer, tid) on rmsnorm(x, wn) (run.c:346-368)."""
        if self.device:
            import device_round
            xw = np.asarray(x, np.float32) * np.asarray(wn, np.float32)
            return device_round.gemv(self._w16(layer, tid, side), device_round.operand(xw),
                                     device_round.norm_scale(x, self.c["rms_eps"]))
        return self.mv(layer, tid, self.O.rmsnorm(x, wn), side)

    def f32(self, layer, tid):
        return self.t[(layer, tid)][1]

    def step(self, tok: int, pos: int) -> np.ndarray:
        """forward_ex (run.c:2594-2645): embed, every layer, the MTP commit
        when present, the head."""
        from cwen_amd import gpu as G
        O, c = self.O, self.c
        wtype, qs, sc, H, _ = self.t[(-1, G.TOK_EMBD)]
        x = O.embed(wtype, qs, sc, int(tok), H)
        for l in range(c["n_layers"]):
            x = self.layer(l, x, pos)
        self.mtp_commit(pos, int(tok), x)
        return self.head(x)

    def layer(self, l, x, pos):
        """layer_linear (run.c:2323-2358) or layer_full (run.c:2412-2458)
        on residual x at position pos."""
        return self.linear_layer(l, x) if l in self.S else self.full_layer(l, x, pos)

    def linear_layer(self, l, x):
        """layer_linear (run.c:2323-2358): the GatedDeltaNet sublayer, then the MLP."""
        from cwen_amd import gpu as G
        O, c = self.O, self.c
        wn = self.f32(l, G.ATTN_NORM)
        qkv = self.mvn(l, G.ATTN_QKV, x, wn)
        z = self.mvn(l, G.ATTN_GATE, x, wn)
        a = self.mvn(l, G.SSM_ALPHA, x, wn)
        b = self.mvn(l, G.SSM_BETA, x, wn)
        A, dt = self.f32(l, G.SSM_A), self.f32(l, G.SSM_DT)
        xa = (a + dt).astype(np.float32)
        sp = np.where(xa > 20, xa, np.log(np.float32(1) + np.exp(xa))).astype(np.float32)
        decay = (A * sp).astype(np.float32)
        beta = (np.float32(1) / (np.float32(1) + np.exp(-b))).astype(np.float32)
        xc, self.hist[l] = O.conv1d_update(qkv, self.hist[l], self.f32(l, G.SSM_CONV).reshape(-1, 4))
        self.S[l], _, o = O.gdn_step(self.S[l], xc, z, decay, beta, self.f32(l, G.SSM_NORM),
                                     c["gdn_nkh"], c["gdn_nvh"], 128)
        x = (x + self.mv(l, G.SSM_OUT, o)).astype(np.float32)
        return self.mlp(l, x)

    def full_layer(self, l, x, pos):
        """layer_full (run.c:2412-2458): gated attention over slots 0..pos, then the MLP."""
        from cwen_amd import gpu as G
        return self.mlp(l, self.full_attn(l, x, self.f32(l, G.ATTN_NORM), pos, 0))

    def head(self, x):
        """The head tail of forward_ex (run.c:2640-2644)."""
        from cwen_amd import gpu as G
        return self.mvn(-1, G.OUTPUT, x, self.f32(-1, G.OUTPUT_NORM))

    def full_attn(self, l, x, wn, pos, t0):
        """layer_full (run.c:2412-2458): x + the gated attention over slots
        t0..pos, on rmsnorm(x, wn)."""
        from cwen_amd import gpu as G
        O, c = self.O, self.c
        NH, NKV, HD = c["n_head"], c["n_kv_head"], c["head_dim"]
        qf = self.mvn(l, G.ATTN_Q, x, wn).reshape(NH, 2, HD)
        q, gate = qf[:, 0].copy(), qf[:, 1].copy()
        k = self.mvn(l, G.ATTN_KV, x, wn, 0).reshape(NKV, HD)
        v = self.mvn(l, G.ATTN_KV, x, wn, 1).reshape(NKV, HD)
        qn, kn = self.f32(l, G.ATTN_Q_NORM), self.f32(l, G.ATTN_K_NORM)
        q = np.stack([O.rmsnorm(q[h], qn) for h in range(NH)])
        k = np.stack([O.rmsnorm(k[h], kn) for h in range(NKV)])
        q = O.rope(q, pos, c["n_rot_pairs"], c["n_rot"], c["rope_theta"])
        k = O.rope(k, pos, c["n_rot_pairs"], c["n_rot"], c["rope_theta"])
        self.K[l][pos], self.V[l][pos] = k, v
        if self.fast_attention:
            self.Kg[l][:, pos], self.Vg[l][:, pos] = k, v
            att = np_attention(self.Kg[l], self.Vg[l], t0, pos, q, gate)
        else:
            att = O.attention(self.K[l][:pos + 1], self.V[l][:pos + 1], t0, pos, q, gate)
        return (x + self.mv(l, G.ATTN_OUTPUT, att.reshape(-1))).astype(np.float32)

    def mlp(self, l, x):
        from cwen_amd import gpu as G
        O = self.O
        wn = self.f32(l, G.POST_NORM)
        h = O.silu_mul(self.mvn(l, G.FFN_GATE_UP, x, wn, 0), self.mvn(l, G.FFN_GATE_UP, x, wn, 1))
        return (x + self.mv(l, G.FFN_DOWN, h)).astype(np.float32)

    def mtp_block(self, tok: int, pos: int, h: np.ndarray) -> np.ndarray:
        """The nextn block of mtp_step (run.c:3099-3133) at stream slot pos on
        token tok and predecessor hidden h, before the shared head norm.  The
        stream's attention covers slots 1..pos."""
        from cwen_amd import gpu as G
        O, NL = self.O, self.c["n_layers"]
        wtype, qs, sc, H, _ = self.t[(-1, G.TOK_EMBD)]
        e = O.embed(wtype, qs, sc, int(tok), H)
        cat = np.concatenate([O.rmsnorm(e, self.f32(-1, G.NEXTN_ENORM)), O.rmsnorm(h, self.f32(-1, G.NEXTN_HNORM))])
        x = self.mv(-1, G.NEXTN_EH_PROJ, cat.astype(np.float32))
        x = self.full_attn(NL, x, self.f32(NL, G.ATTN_NORM), pos, 1)
        return self.mlp(NL, x)

    def mtp_step(self, tok: int, pos: int, h: np.ndarray) -> np.ndarray:
        """mtp_step (run.c:3099-3133): the shared-head-normed hidden."""
        from cwen_amd import gpu as G
        return self.O.rmsnorm(self.mtp_block(tok, pos, h), self.f32(-1, G.NEXTN_SHEAD_NORM))

    def mtp_commit(self, pos: int, tok: int, x_pre: np.ndarray) -> None:
        """mtp_commit (run.c:3150-3163): step the committed position (from
        slot 1 on) against the parked hidden of pos - 1, then park
        rmsnorm(x_pre, output_norm)."""
        from cwen_amd import gpu as G
        if not self.has_mtp:
            return
        if pos >= 1 and self.hpos == pos - 1:
            self.mtp_step(tok, pos, self.hprev)
        self.hprev = self.O.rmsnorm(x_pre, self.f32(-1, G.OUTPUT_NORM))
        self.hpos = pos

    def mtp_draft_logits(self, pend: int, pos: int, inputs) -> np.ndarray:
        """mtp_draft (run.c:3170-3187) from the hidden parked at pos, with the
        step inputs given (pend, then the previous drafts): each step's head
        logits."""
        from cwen_amd import gpu as G
        assert self.hpos == pos
        h, out = self.hprev, []
        shn = self.f32(-1, G.NEXTN_SHEAD_NORM)
        for t, tok in enumerate([pend] + list(inputs)):
            x = self.mtp_block(int(tok), pos + 1 + t, h)
            h = self.O.rmsnorm(x, shn)
            out.append(self.mvn(-1, G.OUTPUT, x, shn))
        return np.stack(out)
