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
