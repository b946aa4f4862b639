/* cwen_gguf.c -- GGUF v2/v3 reader and model binder over the cwen_gpu C ABI.
 *
 * The reader follows the reference's load_gguf (run.c:3188-3301): the file
 * is mapped read-only, every cursor read is bounds-checked, KV pairs are
 * skipped (nesting at most 64 deep), tensor infos are read (at most 1024
 * tensors, names under 96 bytes, at most 4 dims, each in [1, INT_MAX], no
 * internal type ids >= 100), the data section starts at the next 32-byte
 * boundary, and every tensor's offset and extent (row_bytes * ne1, for the
 * types row_bytes sizes) lie inside the file.  Where the reference exits,
 * the reader returns CWEN_EINVAL and keeps the reason for cwen_gguf_error.
 *
 * The binder follows rebind_layers_from_tens (run.c:3366-3406): the
 * reference's tensor names, shapes pinned exactly for matrices and as a
 * floor for F32 vectors, tied embeddings when output.weight is absent.  The
 * device model takes gate/up and k/v as interleaved pairs (CWENR v4 RSI), so
 * two GGUF Q4_0 tensors are interleaved on the host first, as the
 * reference's offline repack does (tools/repack_q4.py).
 */
#define _GNU_SOURCE
#include "cwen_host.h"

#include <fcntl.h>
#include <limits.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

enum { G_MAX_TENSORS = 1024, G_NAME = 96, G_KEY = 256, G_ALIGN = 32, G_NEST = 64 };

typedef struct {
  char name[G_NAME];
  int type, ne0, ne1;
  uint64_t off;
  const void *data;
} gguf_tensor;

struct cwen_gguf {
  void *map;
  size_t len;
  int n;
  gguf_tensor *t;
};

static char g_err[192];

const char *cwen_gguf_error(void) { return g_err; }

static int fail(const char *why) {
  snprintf(g_err, sizeof g_err, "%s", why);
  return CWEN_EINVAL;
}

/* Bounds-checked cursor (run.c:3191-3200). */
typedef struct {
  const uint8_t *p, *end;
  int bad;
} cursor;

static const uint8_t *adv(cursor *c, uint64_t k) {
  if (c->bad || (uint64_t)(c->end - c->p) < k) {
    c->bad = 1;
    return NULL;
  }
  const uint8_t *q = c->p;
  c->p += k;
  return q;
}
static uint64_t rd_u64(cursor *c) {
  uint64_t v = 0;
  const uint8_t *q = adv(c, 8);
  if (q) memcpy(&v, q, 8);
  return v;
}
static uint32_t rd_u32(cursor *c) {
  uint32_t v = 0;
  const uint8_t *q = adv(c, 4);
  if (q) memcpy(&v, q, 4);
  return v;
}
/* A length-prefixed string into buf (cap includes the terminator). */
static int rd_str(cursor *c, char *buf, int cap) {
  const uint64_t n = rd_u64(c);
  if (c->bad) return fail("truncated");
  if (n >= (uint64_t)cap) return fail("string too long");
  const uint8_t *q = adv(c, n);
  if (!q) return fail("truncated");
  memcpy(buf, q, (size_t)n);
  buf[n] = 0;
  return CWEN_OK;
}
/* Skip one KV value of GGUF type t (run.c:3201-3216). */
static int skip_val(cursor *c, uint32_t t, int depth) {
  if (depth > G_NEST) return fail("kv nesting too deep");
  switch (t) {
    case 0: case 1: case 7: adv(c, 1); break;            /* u8 i8 bool */
    case 2: case 3: adv(c, 2); break;                    /* u16 i16 */
    case 4: case 5: case 6: adv(c, 4); break;            /* u32 i32 f32 */
    case 8: adv(c, rd_u64(c)); break;                    /* string */
    case 9: {                                            /* array */
      const uint32_t at = rd_u32(c);
      const uint64_t n = rd_u64(c);
      for (uint64_t i = 0; i < n && !c->bad; i++) {
        const int rc = skip_val(c, at, depth + 1);
        if (rc) return rc;
      }
      break;
    }
    case 10: case 11: case 12: adv(c, 8); break;         /* u64 i64 f64 */
    default: {
      char m[48];
      snprintf(m, sizeof m, "kv type %u", t);
      return fail(m);
    }
  }
  return c->bad ? fail("truncated") : CWEN_OK;
}

/* Bytes of one row of ne0 weights, 0 for types the reference cannot size
 * (run.c:1293-1308; the GGUF types only). */
static uint64_t row_bytes(int type, int ne0) {
  switch (type) {
    case CWEN_T_F32: return (uint64_t)ne0 * 4;
    case CWEN_T_Q4_0: return (uint64_t)(ne0 / 32) * 18;
    case CWEN_T_Q4_1: return (uint64_t)(ne0 / 32) * 20;
    case CWEN_T_Q8_0: return (uint64_t)(ne0 / 32) * 34;
    case CWEN_T_Q5_K: return (uint64_t)(ne0 / 256) * 176;
    case CWEN_T_Q6_K: return (uint64_t)(ne0 / 256) * 210;
    default: return 0;
  }
}

void cwen_gguf_close(cwen_gguf *g) {
  if (!g) return;
  if (g->map && g->map != MAP_FAILED) munmap(g->map, g->len);
  free(g->t);
  free(g);
}

int cwen_gguf_open(const char *path, cwen_gguf **out) {
  if (!path || !out) return fail("null argument");
  *out = NULL;
  const int fd = open(path, O_RDONLY);
  if (fd < 0) return fail("cannot open file");
  struct stat st;
  if (fstat(fd, &st) || st.st_size < 20) {
    close(fd);
    return fail("not a gguf (under 20 bytes)");
  }
  cwen_gguf *g = (cwen_gguf *)calloc(1, sizeof *g);
  if (!g) {
    close(fd);
    return CWEN_ENOMEM;
  }
  g->len = (size_t)st.st_size;
  g->map = mmap(NULL, g->len, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (g->map == MAP_FAILED) {
    g->map = NULL;
    cwen_gguf_close(g);
    return fail("mmap failed");
  }
  const uint8_t *begin = (const uint8_t *)g->map;
  cursor c = {begin, begin + g->len, 0};
  int rc = CWEN_OK;
  if (memcmp(adv(&c, 4), "GGUF", 4)) {
    rc = fail("not gguf");
    goto out;
  }
  /* v2 and v3 share this layout; v1 counted in u32 and later versions may
   * move fields (run.c:3245-3247). */
  const uint32_t ver = rd_u32(&c);
  if (ver < 2u || ver > 3u) {
    char m[48];
    snprintf(m, sizeof m, "gguf version %u", ver);
    rc = fail(m);
    goto out;
  }
  const uint64_t n_tensors = rd_u64(&c), n_kv = rd_u64(&c);
  for (uint64_t i = 0; i < n_kv && !rc; i++) {
    char key[G_KEY];
    if ((rc = rd_str(&c, key, sizeof key))) break;
    const uint32_t t = rd_u32(&c);
    rc = skip_val(&c, t, 0);
  }
  if (rc) goto out;
  if (c.bad) {
    rc = fail("truncated");
    goto out;
  }
  if (n_tensors > G_MAX_TENSORS) {
    rc = fail("too many tensors");
    goto out;
  }
  g->n = (int)n_tensors;
  g->t = (gguf_tensor *)calloc(n_tensors ? n_tensors : 1, sizeof *g->t);
  if (!g->t) {
    rc = CWEN_ENOMEM;
    goto out;
  }
  for (int i = 0; i < g->n && !rc; i++) {
    gguf_tensor *t = &g->t[i];
    if ((rc = rd_str(&c, t->name, G_NAME))) break;
    const uint32_t n_dims = rd_u32(&c);
    uint64_t dims[4] = {1, 1, 1, 1};
    if (n_dims > 4) {
      rc = fail("n_dims > 4");
      break;
    }
    for (uint32_t d = 0; d < n_dims; d++) {
      dims[d] = rd_u64(&c);
      if (!c.bad && (dims[d] == 0 || dims[d] > (uint64_t)INT_MAX)) {
        char m[160];
        snprintf(m, sizeof m, "%.100s: dim %u = %llu", t->name, d, (unsigned long long)dims[d]);
        rc = fail(m);
        break;
      }
    }
    if (rc) break;
    const uint32_t typ = rd_u32(&c);
    /* 100 and up are the reference's internal CWENR tags (run.c:3271-3277). */
    if (!c.bad && typ >= 100u) {
      char m[48];
      snprintf(m, sizeof m, "reserved type %u", typ);
      rc = fail(m);
      break;
    }
    t->off = rd_u64(&c);
    t->type = (int)typ;
    t->ne0 = (int)dims[0];
    t->ne1 = (int)(n_dims > 1 ? dims[1] : 1);
    if (c.bad) rc = fail("truncated");
  }
  if (rc) goto out;
  /* data section at the next 32-byte boundary (run.c:3286-3289) */
  const uint64_t data_off = ((uint64_t)(c.p - begin) + G_ALIGN - 1) & ~(uint64_t)(G_ALIGN - 1);
  for (int i = 0; i < g->n; i++) {
    gguf_tensor *t = &g->t[i];
    if (data_off >= g->len || t->off >= g->len - data_off) {
      rc = fail("tensor offset out of the file");
      goto out;
    }
    t->data = begin + data_off + t->off;
    const uint64_t rb = row_bytes(t->type, t->ne0);
    if (rb && rb * (uint64_t)t->ne1 > g->len - data_off - t->off) {
      char m[160];
      snprintf(m, sizeof m, "%.100s: extent beyond the file", t->name);
      rc = fail(m);
      goto out;
    }
  }
out:
  if (rc) {
    cwen_gguf_close(g);
    return rc;
  }
  g_err[0] = 0;
  *out = g;
  return CWEN_OK;
}

int cwen_gguf_count(const cwen_gguf *g) { return g ? g->n : CWEN_EINVAL; }

int cwen_gguf_tensor(const cwen_gguf *g, int i, const char **name, int *type, int *ne0, int *ne1,
                     const void **data) {
  if (!g || i < 0 || i >= g->n) return CWEN_EINVAL;
  const gguf_tensor *t = &g->t[i];
  if (name) *name = t->name;
  if (type) *type = t->type;
  if (ne0) *ne0 = t->ne0;
  if (ne1) *ne1 = t->ne1;
  if (data) *data = t->data;
  return CWEN_OK;
}

int cwen_gguf_find(const cwen_gguf *g, const char *name) {
  if (!g || !name) return CWEN_EINVAL;
  for (int i = 0; i < g->n; i++)
    if (!strcmp(g->t[i].name, name)) return i;
  return -1;
}

/* ------------------------------------------------------------------ binder */

/* Matrix types the device GEMV computes (the reference's matmul_type_ok,
 * run.c:1311-1318, minus its drafter-only T_Q8S). */
static int mat_type_ok(int ty) {
  return ty == CWEN_T_Q4_0 || ty == CWEN_T_Q4_1 || ty == CWEN_T_Q8_0 || ty == CWEN_T_Q5_K || ty == CWEN_T_Q6_K;
}

static const gguf_tensor *need(const cwen_gguf *g, const char *name, int *rc) {
  const int i = cwen_gguf_find(g, name);
  if (i < 0) {
    char m[160];
    snprintf(m, sizeof m, "missing %.100s", name);
    *rc = fail(m);
    return NULL;
  }
  return &g->t[i];
}

/* A matrix pinned to (ne0, ne1) exactly (run.c:3342-3360 must_mat_sh). */
static const gguf_tensor *mat(const cwen_gguf *g, const char *name, int ne0, int ne1, int *rc) {
  const gguf_tensor *t = need(g, name, rc);
  if (!t) return NULL;
  if (!mat_type_ok(t->type)) {
    char m[160];
    snprintf(m, sizeof m, "%.100s: unsupported weight type %d", name, t->type);
    *rc = fail(m);
    return NULL;
  }
  if (t->ne0 != ne0 || t->ne1 != ne1) {
    char m[192];
    snprintf(m, sizeof m, "%.100s: shape %dx%d, need %dx%d", name, t->ne0, t->ne1, ne0, ne1);
    *rc = fail(m);
    return NULL;
  }
  return t;
}

/* An F32 vector holding at least n floats (run.c:3329-3364 must_f32_n). */
static const gguf_tensor *vec(const cwen_gguf *g, const char *name, int n, int *rc) {
  const gguf_tensor *t = need(g, name, rc);
  if (!t) return NULL;
  if (t->type != CWEN_T_F32 || (long long)t->ne0 * t->ne1 < n) {
    char m[192];
    snprintf(m, sizeof m, "%.100s: need F32 of %d values", name, n);
    *rc = fail(m);
    return NULL;
  }
  return t;
}

static int set_vec(cwen_model *m, int layer, int id, const gguf_tensor *t, int n) {
  return cwen_model_set(m, layer, id, CWEN_T_F32, t->data, NULL, n, 1);
}
static int set_mat(cwen_model *m, int layer, int id, const gguf_tensor *t) {
  return cwen_model_set(m, layer, id, t->type, t->data, NULL, t->ne0, t->ne1);
}

/* Two GGUF Q4_0 matrices of one shape as a CWENR interleaved pair:
 * qs[row][block][a 16 | b 16], f16 sc[row][block][a | b]. */
static int set_pair(cwen_model *m, int layer, int id, const gguf_tensor *a, const gguf_tensor *b) {
  if (a->type != CWEN_T_Q4_0 || b->type != CWEN_T_Q4_0) return fail("pair halves must be Q4_0");
  const size_t nblk = (size_t)(a->ne0 / 32) * a->ne1;
  uint8_t *qs = (uint8_t *)malloc(nblk * 32);
  uint16_t *sc = (uint16_t *)malloc(nblk * 4);
  if (!qs || !sc) {
    free(qs);
    free(sc);
    return CWEN_ENOMEM;
  }
  const uint8_t *pa = (const uint8_t *)a->data, *pb = (const uint8_t *)b->data;
  for (size_t i = 0; i < nblk; i++) {
    memcpy(&sc[2 * i], pa + i * 18, 2);
    memcpy(&sc[2 * i + 1], pb + i * 18, 2);
    memcpy(qs + i * 32, pa + i * 18 + 2, 16);
    memcpy(qs + i * 32 + 16, pb + i * 18 + 2, 16);
  }
  const int rc = cwen_model_set(m, layer, id, CWEN_T_Q4_0RSI, qs, sc, a->ne0, a->ne1);
  free(qs);
  free(sc);
  return rc;
}

#define TRY(x)             \
  do {                     \
    if ((rc = (x))) return rc; \
  } while (0)
#define NEED(ptr, expr)    \
  do {                     \
    if (!((ptr) = (expr))) return rc; \
  } while (0)

int cwen_model_load_gguf(cwen_model *m, const cwen_model_cfg *c, const cwen_gguf *g) {
  if (!m || !c || !g) return fail("null argument");
  int rc = CWEN_OK;
  const int H = c->d_model, I = c->d_ffn, V = c->vocab;
  const int C = (2 * c->gdn_nkh + c->gdn_nvh) * c->gdn_dk, Zh = c->gdn_nvh * c->gdn_dk;
  const int Qo = c->n_head * c->head_dim, Ko = c->n_kv_head * c->head_dim;
  const gguf_tensor *t, *u;
  NEED(t, need(g, "token_embd.weight", &rc));
  if (t->type != CWEN_T_Q4_0) return fail("token_embd.weight: the device embedding takes Q4_0");
  if (t->ne0 != H || t->ne1 != V) return fail("token_embd.weight: shape");
  TRY(set_mat(m, -1, CWEN_TOK_EMBD, t));
  NEED(u, vec(g, "output_norm.weight", H, &rc));
  TRY(set_vec(m, -1, CWEN_OUTPUT_NORM, u, H));
  {
    const int io = cwen_gguf_find(g, "output.weight");  /* tied embeddings when absent */
    const gguf_tensor *o = io >= 0 ? &g->t[io] : t;
    if (!mat_type_ok(o->type) || o->ne0 != H || o->ne1 != V) return fail("output.weight: type or shape");
    TRY(set_mat(m, -1, CWEN_OUTPUT, o));
  }
  char n[G_NAME], n2[G_NAME];
  for (int l = 0; l < c->n_layers; l++) {
    const int linear = (l + 1) % c->full_interval != 0;
#define NM(buf, suf) snprintf(buf, sizeof buf, "blk.%d.%s", l, suf)
    NM(n, "attn_norm.weight");
    NEED(u, vec(g, n, H, &rc));
    TRY(set_vec(m, l, CWEN_ATTN_NORM, u, H));
    NM(n, "post_attention_norm.weight");
    NEED(u, vec(g, n, H, &rc));
    TRY(set_vec(m, l, CWEN_POST_NORM, u, H));
    NM(n, "ffn_gate.weight");
    NM(n2, "ffn_up.weight");
    NEED(t, mat(g, n, H, I, &rc));
    NEED(u, mat(g, n2, H, I, &rc));
    TRY(set_pair(m, l, CWEN_FFN_GATE_UP, t, u));
    NM(n, "ffn_down.weight");
    NEED(t, mat(g, n, I, H, &rc));
    TRY(set_mat(m, l, CWEN_FFN_DOWN, t));
    if (linear) {
      static const struct { const char *suf; int id; } parts[] = {
          {"attn_qkv.weight", CWEN_ATTN_QKV}, {"attn_gate.weight", CWEN_ATTN_GATE},
          {"ssm_alpha.weight", CWEN_SSM_ALPHA}, {"ssm_beta.weight", CWEN_SSM_BETA}};
      const int rows[4] = {C, Zh, c->gdn_nvh, c->gdn_nvh};
      for (int k = 0; k < 4; k++) {
        NM(n, parts[k].suf);
        NEED(t, mat(g, n, H, rows[k], &rc));
        TRY(set_mat(m, l, parts[k].id, t));
      }
      NM(n, "ssm_a");
      NEED(u, vec(g, n, c->gdn_nvh, &rc));
      TRY(set_vec(m, l, CWEN_SSM_A, u, c->gdn_nvh));
      NM(n, "ssm_dt.bias");
      NEED(u, vec(g, n, c->gdn_nvh, &rc));
      TRY(set_vec(m, l, CWEN_SSM_DT, u, c->gdn_nvh));
      NM(n, "ssm_conv1d.weight");
      NEED(u, vec(g, n, 4 * C, &rc));
      TRY(set_vec(m, l, CWEN_SSM_CONV, u, 4 * C));
      NM(n, "ssm_norm.weight");  /* one head_dim vector shared by the heads */
      NEED(u, vec(g, n, c->gdn_dk, &rc));
      TRY(set_vec(m, l, CWEN_SSM_NORM, u, c->gdn_dk));
      NM(n, "ssm_out.weight");
      NEED(t, mat(g, n, Zh, H, &rc));
      TRY(set_mat(m, l, CWEN_SSM_OUT, t));
    } else {
      NM(n, "attn_q.weight");
      NEED(t, mat(g, n, H, 2 * Qo, &rc));
      TRY(set_mat(m, l, CWEN_ATTN_Q, t));
      NM(n, "attn_k.weight");
      NM(n2, "attn_v.weight");
      NEED(t, mat(g, n, H, Ko, &rc));
      NEED(u, mat(g, n2, H, Ko, &rc));
      TRY(set_pair(m, l, CWEN_ATTN_KV, t, u));
      NM(n, "attn_output.weight");
      NEED(t, mat(g, n, Qo, H, &rc));
      TRY(set_mat(m, l, CWEN_ATTN_OUTPUT, t));
      NM(n, "attn_q_norm.weight");
      NEED(u, vec(g, n, c->head_dim, &rc));
      TRY(set_vec(m, l, CWEN_ATTN_Q_NORM, u, c->head_dim));
      NM(n, "attn_k_norm.weight");
      NEED(u, vec(g, n, c->head_dim, &rc));
      TRY(set_vec(m, l, CWEN_ATTN_K_NORM, u, c->head_dim));
    }
#undef NM
  }
  g_err[0] = 0;
  return CWEN_OK;
}
