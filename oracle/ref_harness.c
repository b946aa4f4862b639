/* Reference-build harness (test infrastructure only).
 *
 * Compiles the reference engine's run.c where it lies (the recipe in
 * oracle/Makefile passes -I<reference tree>; nothing is copied) with main
 * renamed, and exports a few plain-C wrappers around its static kernels so
 * tests can call them on in-memory tensors with no model file.  The built
 * library lands in oracle/_ref/ and is used only as a checker for the
 * oracle and as the CPU baseline timed by bench.py.
 */
#define main cwen_ref_main
#include "run.c"
#undef main

int ref_vocab(void) { return V; }
int ref_dims(int *h, int *qkv, int *lkh, int *lvh, int *lsd) {
  *h = H; *qkv = QKV_DIM; *lkh = LKH; *lvh = LVH; *lsd = LSD;
  return 0;
}

static Tensor mk(int type, const void *data, const void *scales, int ne0, int ne1, int side) {
  Tensor t;
  t.data = data; t.scales = scales; t.type = type; t.ne0 = ne0; t.ne1 = ne1; t.pair_side = side;
  return t;
}

/* gemv (run.c:1419) on one activation vector */
int ref_gemv(int type, const void *data, const void *scales, int ne0, int ne1, int side,
             const float *x, float *y) {
  Tensor t = mk(type, data, scales, ne0, ne1, side);
  if (!matmul_type_ok(type)) return -1;
  gemv(&t, x, y);
  return 0;
}

/* gemvb (run.c:1577) over B activation columns */
int ref_gemvb(int type, const void *data, const void *scales, int ne0, int ne1, int side,
              const float *X, int xs, float *Y, int ys, int B) {
  Tensor t = mk(type, data, scales, ne0, ne1, side);
  if (!matmul_type_ok(type) || B < 1 || B > SPEC_BMAX) return -1;
  gemvb(&t, X, xs, Y, ys, B);
  return 0;
}

void ref_silu_mul(float *a, const float *b, int n) { silu_mul(a, b, n); }
void ref_rmsnorm(float *o, const float *x, const float *w, int n) { rmsnorm(o, x, w, n); }

/* conv1d_update (run.c:2183) with the caller's [QKV_DIM][3] history and [QKV_DIM][4] taps */
int ref_conv1d_update(float *qkv, float *hist, const float *kw) {
  float *saved = Cstate;
  const void *sw = W[0].ssm_conv.data;
  Cstate = hist;
  W[0].ssm_conv.data = kw;
  conv1d_update(0, qkv);
  Cstate = saved;
  W[0].ssm_conv.data = sw;
  return 0;
}

/* gdn_step (run.c:2014) on the caller's [LVH][LSD][LSD] state */
int ref_gdn_step(float *S, float *qkv, float *z, float *decay, float *beta,
                 const float *wn, float *out) {
  float *saved = Srec;
  const void *sw = W[0].ssm_norm.data;
  Srec = S;
  W[0].ssm_norm.data = wn;
  gdn_step(0, qkv, z, decay, beta, out);
  Srec = saved;
  W[0].ssm_norm.data = sw;
  return 0;
}

/* argmax_of (run.c:2647) scans exactly V entries; shorter vocabularies are
   padded with -inf, which can never win a strict '>' scan. */
static float *pad_buf;
static const float *padded(const float *lg, int n) {
  if (n == V) return lg;
  if (!pad_buf) {
    pad_buf = aligned_alloc(64, (size_t)V * sizeof(float));
    if (!pad_buf) return NULL;
  }
  memcpy(pad_buf, lg, (size_t)n * sizeof(float));
  for (int i = n; i < V; i++) pad_buf[i] = -INFINITY;
  return pad_buf;
}
int ref_argmax(const float *lg, int n) {
  if (n < 1 || n > V) return -1;
  const float *p = padded(lg, n);
  return p ? argmax_of(p) : -1;
}

/* greedy walk exactly as generate_tokens_spec (run.c:4954-4956) */
int ref_walk(const float *logits, long ls, int n, const int *drafts, int E, int *bonus) {
  int k = 0;
  const float *cur = logits;
  while (k < E && ref_argmax(cur, n) == drafts[k]) { k++; cur = logits + (size_t)k * ls; }
  *bonus = ref_argmax(cur, n);
  return k;
}

int ref_ngram_draft(const int *h, int hn, int *out, int n_key, int max_d) {
  return ngram_draft(h, hn, out, n_key, max_d);
}

int ref_omp_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* rope_apply (run.c:1920-1948) on n_heads heads of HD at position pos */
int ref_rope_apply(float *q, int n_heads, int pos) {
  if (pos < 0 || pos >= MAX_SEQ) return -1;
  rope_apply(q, n_heads, pos);
  return 0;
}
int ref_attn_dims(int *nh, int *nkv, int *hd) {
  *nh = NH; *nkv = NKV; *hd = HD;
  return 0;
}
/* attention_heads_kv (run.c:2362) over caller K/V [t][NKV][HD] */
int ref_attention(const float *K, const float *Vv, int t0, int pos, const float *q, const float *gate,
                  float *out) {
  if (t0 < 0 || t0 > pos || pos >= MAX_SEQ) return -1;
  attention_heads_kv(K, Vv, t0, pos, q, gate, out);
  return 0;
}
/* embed_token_to (run.c:1849) with a caller token_embd of type Q4_0 / Q4_0RS */
int ref_embed(int type, const void *qs, const void *sc, int token, float *dst) {
  Tensor saved = tok_embd;
  tok_embd = mk(type, qs, sc, H, V, 0);
  embed_token_to(token, dst);
  tok_embd = saved;
  return 0;
}

/* ---- the model composition, for pinning the oracle's serial forward ----
 * The reference's own layer functions over its global state: W[l] (and NW,
 * tok_embd, output_norm, output) bound to caller tensors, the activation x,
 * pos_n, Srec / Cstate and the KV caches from alloc_state.  Dimensions are
 * the reference's compile-time ones (H 5120, I 17408, 24/4 heads of 256,
 * GDN 16/48 x 128). */

/* tensor ids of include/cwen_gpu.h (CWEN_TOK_EMBD ...) */
enum { ID_TOK_EMBD, ID_OUTPUT_NORM, ID_OUTPUT, ID_ATTN_NORM, ID_POST_NORM, ID_FFN_GATE_UP, ID_FFN_DOWN,
       ID_ATTN_QKV, ID_ATTN_GATE, ID_SSM_ALPHA, ID_SSM_BETA, ID_SSM_A, ID_SSM_DT, ID_SSM_CONV, ID_SSM_NORM,
       ID_SSM_OUT, ID_ATTN_Q, ID_ATTN_KV, ID_ATTN_OUTPUT, ID_ATTN_Q_NORM, ID_ATTN_K_NORM, ID_NEXTN_EH_PROJ,
       ID_NEXTN_ENORM, ID_NEXTN_HNORM, ID_NEXTN_SHEAD_NORM };

/* alloc_state (run.c:3928) with a context of ctx slots and the nextn stream
 * on; every layer l with l % FULL_INT != FULL_INT - 1 is linear.  Once per
 * process. */
int ref_model_init(int ctx) {
  if (ctx < 2 || ctx > MAX_SEQ || logits) return -1;
  g_ctx = ctx;
  mtp_use = 1;
  spec_enabled = 0;
  alloc_state();
  for (int l = 0; l < L; l++) W[l].is_linear = (l % FULL_INT) != FULL_INT - 1;
  mtp_hpos = -1;
  return 0;
}

/* Bind one tensor: layer -1 the globals and the nextn projection / norms,
 * layer L the nextn decoder block (NW), else W[layer].  A Q4_0RSI pair binds
 * both of its Tensors (pair_side 0 and 1), as load_cwenr does. */
int ref_set_tensor(int layer, int id, int type, const void *data, const void *scales, int ne0, int ne1) {
  const Tensor t0 = mk(type, data, scales, ne0, ne1, 0), t1 = mk(type, data, scales, ne0, ne1, 1);
  if (layer < 0) {
    switch (id) {
      case ID_TOK_EMBD: tok_embd = t0; return 0;
      case ID_OUTPUT_NORM: output_norm = t0; return 0;
      case ID_OUTPUT: output = t0; return 0;
      case ID_NEXTN_EH_PROJ: NW.eh_proj = t0; return 0;
      case ID_NEXTN_ENORM: NW.enorm = t0; return 0;
      case ID_NEXTN_HNORM: NW.hnorm = t0; return 0;
      case ID_NEXTN_SHEAD_NORM: NW.shared_head_norm = t0; return 0;
      default: return -1;
    }
  }
  if (layer == L) {
    switch (id) {
      case ID_ATTN_NORM: NW.attn_norm = t0; return 0;
      case ID_POST_NORM: NW.post_norm = t0; return 0;
      case ID_FFN_GATE_UP: NW.ffn_gate = t0; NW.ffn_up = t1; return 0;
      case ID_FFN_DOWN: NW.ffn_down = t0; return 0;
      case ID_ATTN_Q: NW.wq = t0; return 0;
      case ID_ATTN_KV: NW.wk = t0; NW.wv = t1; return 0;
      case ID_ATTN_OUTPUT: NW.wo = t0; return 0;
      case ID_ATTN_Q_NORM: NW.q_norm = t0; return 0;
      case ID_ATTN_K_NORM: NW.k_norm = t0; return 0;
      default: return -1;
    }
  }
  if (layer >= L) return -1;
  LayerW *w = &W[layer];
  switch (id) {
    case ID_ATTN_NORM: w->attn_norm = t0; return 0;
    case ID_POST_NORM: w->post_norm = t0; return 0;
    case ID_FFN_GATE_UP: w->ffn_gate = t0; w->ffn_up = t1; return 0;
    case ID_FFN_DOWN: w->ffn_down = t0; return 0;
    case ID_ATTN_QKV: w->qkv = t0; return 0;
    case ID_ATTN_GATE: w->gate_z = t0; return 0;
    case ID_SSM_ALPHA: w->ssm_alpha = t0; return 0;
    case ID_SSM_BETA: w->ssm_beta = t0; return 0;
    case ID_SSM_A: w->ssm_a = t0; return 0;
    case ID_SSM_DT: w->ssm_dt = t0; return 0;
    case ID_SSM_CONV: w->ssm_conv = t0; return 0;
    case ID_SSM_NORM: w->ssm_norm = t0; return 0;
    case ID_SSM_OUT: w->ssm_out = t0; return 0;
    case ID_ATTN_Q: w->wq = t0; return 0;
    case ID_ATTN_KV: w->wk = t0; w->wv = t1; return 0;
    case ID_ATTN_OUTPUT: w->wo = t0; return 0;
    case ID_ATTN_Q_NORM: w->q_norm = t0; return 0;
    case ID_ATTN_K_NORM: w->k_norm = t0; return 0;
    default: return -1;
  }
}

/* One decoder layer at position pos on the residual xio[H]:
 * layer_linear (run.c:2323) or layer_full (run.c:2412), in place. */
int ref_layer_step(int layer, int pos, float *xio) {
  if (!logits || layer < 0 || layer >= L || pos < 0 || pos >= g_ctx) return -1;
  memcpy(x, xio, sizeof x);
  pos_n = pos;
  if (W[layer].is_linear) layer_linear(layer);
  else layer_full(layer);
  memcpy(xio, x, sizeof x);
  return 0;
}

/* One decoder layer over a block of B positions pbase .. pbase+B-1 on the
 * residual rows xio[B][H]: layer_linear_blk (run.c:2685) or layer_full_blk
 * (run.c:2714), in place -- forward_block's per-layer step. */
int ref_block_layer(int layer, int B, int pbase, float *xio) {
  if (!logits || layer < 0 || layer >= L || B < 1 || B > SPEC_BMAX || pbase < 0 || pbase + B > g_ctx) return -1;
  memcpy(BXres, xio, (size_t)B * H * sizeof(float));
  if (W[layer].is_linear) layer_linear_blk(layer, B);
  else layer_full_blk(layer, B, pbase);
  memcpy(xio, BXres, (size_t)B * H * sizeof(float));
  return 0;
}

/* The head tail of forward_ex (run.c:2640-2644) on residual xin[H]: the
 * first n logits of output . rmsnorm(x, output_norm). */
int ref_head(const float *xin, float *out, int n) {
  if (!logits || n < 1 || n > output.ne1) return -1;
  memcpy(x, xin, sizeof x);
  rmsnorm(xb, x, (const float *)output_norm.data, H);
  gemv(&output, xb, logits);
  memcpy(out, logits, (size_t)n * sizeof(float));
  return 0;
}

/* Layer l's recurrent state [LVH][LSD][LSD] and conv history [QKV_DIM][3]. */
int ref_gdn_state(int layer, float *S, float *hist) {
  if (!Srec || layer < 0 || layer >= L) return -1;
  if (S) memcpy(S, Srec + (size_t)layer * LVH * LSD * LSD, (size_t)LVH * LSD * LSD * sizeof(float));
  if (hist) memcpy(hist, Cstate + (size_t)layer * QKV_DIM * (CONV_K - 1), (size_t)QKV_DIM * (CONV_K - 1) * sizeof(float));
  return 0;
}

/* mtp_step (run.c:3099): the nextn block at stream slot pos on token tok and
 * predecessor hidden h[H]; out[H] the shared-head-normed hidden. */
int ref_mtp_step(int tok, int pos, const float *h, float *out) {
  static float hb_[H] __attribute__((aligned(64))), ob_[H] __attribute__((aligned(64)));
  if (!NKc || pos < 1 || pos >= g_ctx || tok < 0 || tok >= V) return -1;
  memcpy(hb_, h, sizeof hb_);
  mtp_step(tok, pos, hb_, ob_);
  memcpy(out, ob_, sizeof ob_);
  return 0;
}

/* mtp_commit (run.c:3146): fold position pos (token tok, target residual
 * x_pre[H]) into the nextn stream; hprev[H] (nullable) receives the parked
 * hidden.  Returns the parked position. */
int ref_mtp_commit(int pos, int tok, const float *x_pre, float *hprev) {
  static float xb_[H] __attribute__((aligned(64)));
  if (!NKc || pos < 0 || pos >= g_ctx || tok < 0 || tok >= V) return -1;
  memcpy(xb_, x_pre, sizeof xb_);
  mtp_commit(pos, tok, xb_);
  if (hprev) memcpy(hprev, NHprev, sizeof NHprev);
  return mtp_hpos;
}

/* The rollback copies of a drafted cycle: snap_save then snap_load
 * (run.c:2802-2809) over all L layers' Srec and Cstate, allocating the
 * state (ref_model_init) and the snapshot buffers on first use. */
static int snap_alloc(void) {
  if (!logits && ref_model_init(2)) return -1;
  if (!SnapS) {
    SnapS = aligned_alloc(64, (size_t)L * LVH * LSD * LSD * sizeof(float));
    SnapC = aligned_alloc(64, (size_t)L * QKV_DIM * (CONV_K - 1) * sizeof(float));
    if (!SnapS || !SnapC) return -1;
  }
  return 0;
}
int ref_snap_roundtrip(void) {
  if (snap_alloc()) return -1;
  snap_save();
  snap_load();
  return 0;
}
/* snap_save alone: what a drafted cycle pays before its block (run.c:4952);
 * snap_load puts the saved state back. */
int ref_snap_save(void) {
  if (snap_alloc()) return -1;
  snap_save();
  return 0;
}
int ref_snap_load(void) {
  if (!SnapS) return -1;
  snap_load();
  return 0;
}

/* The counted n-gram map (run.c:204-221, 4552-4723) on the reference's own
 * globals.  ref_ng_init allocates NGM at NG_CAP as alloc_state does with
 * speculation on (run.c:3972-3978), with lookup key length n_key
 * (Scfg_n_key), and rewinds the eviction hand; the map starts empty. */
int ref_ng_init(int n_key) {
  if (n_key < 1 || n_key > 256) return -1;
  free(NGM.keys);
  free(NGM.tok);
  free(NGM.cnt);
  free(NGM.used);
  memset(&NGM, 0, sizeof NGM);
  Scfg_n_key = n_key;
  NG_evict_hand = 0;
  NGM.cap = NG_CAP;
  NGM.keys = malloc(sizeof(int) * NG_CAP * (size_t)n_key);
  NGM.tok = malloc(sizeof(int) * NG_CAP);
  NGM.cnt = calloc(NG_CAP, sizeof(int));
  NGM.used = calloc(NG_CAP, 1);
  return NGM.keys && NGM.tok && NGM.cnt && NGM.used ? 0 : -1;
}
long ref_ng_cap(void) { return (long)NG_CAP; }
long ref_ng_used(void) { return (long)NGM.used_n; }
void ref_ng_update_key_n(const int *key, int tok, int hits) { ng_update_key_n(key, tok, hits); }
void ref_ng_update_range(const int *h, int a, int b) { ng_update_range(h, a, b); }
int ref_ng_draft_map(const int *h, int hn, int *out, int max_d) { return ng_draft_map(h, hn, out, max_d); }
void ref_ng_save(const char *path) { ng_save(path); }
void ref_ng_load(const char *path) { ng_load(path); }
/* Copy the table: keys [cap][n_key], tokens, counts, in-use flags. */
void ref_ng_dump(int *keys, int *tok, int *cnt, unsigned char *used) {
  memcpy(keys, NGM.keys, sizeof(int) * NGM.cap * (size_t)Scfg_n_key);
  memcpy(tok, NGM.tok, sizeof(int) * NGM.cap);
  memcpy(cnt, NGM.cnt, sizeof(int) * NGM.cap);
  memcpy(used, NGM.used, NGM.cap);
}
