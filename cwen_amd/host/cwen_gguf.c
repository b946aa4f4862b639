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
 *
 * The CWENR sidecar reader follows load_cwenr (run.c:3467-3643): a sidecar
 * stamped with its source GGUF's size in 4 KiB pages is dropped when the
 * GGUF no longer has that size; v3/v4 entries rebind a GGUF Q4_0 tensor of
 * the same name and shape to a split (RS) or interleaved (RSI) view of the
 * sidecar; v2's packed 20-byte blocks are split on the host, the f32 scale
 * rounded to f16 to nearest even.  Entries that cannot apply are skipped.
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
  const void *scales;  /* CWENR RS / RSI: the f16 scales */
  int side;            /* CWENR RSI: 0 = first (A), 1 = second (B) of the pair */
} gguf_tensor;

struct cwen_gguf {
  void *map;
  size_t len;
  int n;
  gguf_tensor *t;
  void *rmap;   /* a v3/v4 CWENR sidecar the tensors point into */
  size_t rlen;
  void *split;  /* v2: qs and f16 scales split on the host */
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
  if (g->rmap) munmap(g->rmap, g->rlen);
  free(g->split);
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

int cwen_gguf_tensor_scales(const cwen_gguf *g, int i, const void **scales, int *side) {
  if (!g || i < 0 || i >= g->n) return CWEN_EINVAL;
  if (scales) *scales = g->t[i].scales;
  if (side) *side = g->t[i].side;
  return CWEN_OK;
}

/* ------------------------------------------------------------ CWENR sidecar */

enum { R_HEAD = 32, R_ENT = 128, R_MAX = 1024, R_IL_A = 1, R_IL_B = 2 };
#define R_STAMP_TAG 0x4e455743u /* "CWEN" little-endian */

int cwen_cwenr_path(const char *gguf, char *out, size_t cap) {
  if (!gguf || !out || !cap) return CWEN_EINVAL;
  const char *env = getenv("CWEN_REPACK");
  int k;
  if (env && env[0]) {
    k = snprintf(out, cap, "%s", env);
  } else {
    const size_t n = strlen(gguf);
    if (n > 5 && !strcmp(gguf + n - 5, ".gguf"))
      k = snprintf(out, cap, "%.*s.cwenr", (int)(n - 5), gguf);
    else
      k = snprintf(out, cap, "%s.cwenr", gguf);
  }
  return (k < 0 || (size_t)k >= cap) ? CWEN_EINVAL : CWEN_OK;
}

/* IEEE binary32 -> binary16, round to nearest even; NaN becomes a quiet NaN
 * with the sign kept, overflow becomes infinity, and results below the
 * smallest subnormal's half become signed zero. */
static uint16_t f32_to_f16_rne(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  const uint32_t sign = (u >> 16) & 0x8000u, a = u & 0x7fffffffu;
  if (a >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (a > 0x7f800000u ? 0x0200u : 0));
  const int e = (int)(a >> 23) - 127;                    /* unbiased exponent */
  if (e < -25) return (uint16_t)sign;                    /* |x| < 2^-25 */
  const uint32_t mant = (a & 0x7fffffu) | 0x800000u;    /* 24 significant bits */
  /* the result's unit in the last place is 2^(e-10) for normals, 2^-24 below
   * 2^-14: drop `sh` low bits of the 24-bit significand */
  const int sh = e < -14 ? 13 + (-14 - e) : 13;
  uint32_t r = mant >> sh;
  const uint32_t rem = mant & ((1u << sh) - 1u), half = 1u << (sh - 1);
  if (rem > half || (rem == half && (r & 1u))) r++;
  if (e < -14) return (uint16_t)(sign | r);              /* subnormal, or the smallest normal */
  /* normal: r holds the hidden bit; a carry out of 11 bits bumps the exponent */
  uint32_t he = (uint32_t)(e + 15);
  if (r >> 11) {
    r >>= 1;
    he++;
  }
  if (he >= 31u) return (uint16_t)(sign | 0x7c00u);
  return (uint16_t)(sign | (he << 10) | (r & 0x3ffu));
}

uint16_t cwen_f32_to_f16(float x) { return f32_to_f16_rne(x); }

typedef struct {
  int t;             /* tensor index */
  int32_t ne0, ne1;
  uint64_t a, b;     /* v3/v4: qs and scale offsets; v2: offset and byte count */
  uint32_t flags;
} r_entry;

/* One directory entry and the GGUF Q4_0 tensor of the same name and shape
 * it applies to, or -1 (run.c:3472-3485). */
static int r_match(const cwen_gguf *g, const uint8_t *dir, uint32_t i, r_entry *e) {
  const uint8_t *p = dir + R_HEAD + (size_t)i * R_ENT;
  char name[G_NAME];
  memcpy(name, p, G_NAME);
  name[G_NAME - 1] = 0;
  memcpy(&e->ne0, p + 96, 4);
  memcpy(&e->ne1, p + 100, 4);
  memcpy(&e->a, p + 104, 8);
  memcpy(&e->b, p + 112, 8);
  memcpy(&e->flags, p + 120, 4);
  e->t = cwen_gguf_find(g, name);
  if (e->t < 0) return -1;
  const gguf_tensor *t = &g->t[e->t];
  if (t->type != CWEN_T_Q4_0 || t->ne0 != e->ne0 || t->ne1 != e->ne1) return -1;
  return e->t;
}

int cwen_gguf_apply_cwenr(cwen_gguf *g, const char *path, const char *src_gguf) {
  if (!g || !path) return fail("null argument");
  if (g->rmap || g->split) return fail("a sidecar is already applied");
  const int fd = open(path, O_RDONLY);
  if (fd < 0) {
    snprintf(g_err, sizeof g_err, "no sidecar");
    return 0;  /* optional */
  }
  struct stat st;
  if (fstat(fd, &st) || st.st_size < R_HEAD) {
    close(fd);
    return fail("cwenr: unusable (too small)");
  }
  const size_t len = (size_t)st.st_size;
  void *map = mmap(NULL, len, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (map == MAP_FAILED) return fail("cwenr: mmap failed");
  const uint8_t *p = (const uint8_t *)map;
  int rc = CWEN_OK;
  if (memcmp(p, "CWENR001", 8)) {
    rc = fail("cwenr: bad magic");
    goto drop;
  }
  {  /* staleness gate: a stamped sidecar must match its source's size */
    uint32_t tag, src_pages;
    memcpy(&tag, p + 24, 4);
    memcpy(&src_pages, p + 28, 4);
    if (tag == R_STAMP_TAG) {
      struct stat gs;
      const uint64_t want = (src_gguf && stat(src_gguf, &gs) == 0) ? ((uint64_t)gs.st_size + 4095) / 4096 : 0;
      if ((uint64_t)src_pages != want) {
        rc = fail("cwenr: stale sidecar (its source GGUF changed since the repack)");
        goto drop;
      }
    }
  }
  uint32_t ver, n;
  uint64_t base;
  memcpy(&ver, p + 8, 4);
  memcpy(&n, p + 12, 4);
  memcpy(&base, p + 16, 8);
  if ((ver != 2 && ver != 3 && ver != 4) || n > R_MAX || base >= len || R_HEAD + (size_t)n * R_ENT > len) {
    char m[64];
    snprintf(m, sizeof m, "cwenr: bad header ver=%u n=%u", ver, n);
    rc = fail(m);
    goto drop;
  }
  const size_t rem = len - (size_t)base;
  int bound = 0;
  if (ver >= 3) {
    for (uint32_t i = 0; i < n; i++) {
      r_entry e;
      if (r_match(g, p, i, &e) < 0) continue;
      const int il = e.flags == R_IL_A || e.flags == R_IL_B;
      const size_t nblk = (size_t)(e.ne0 / 32) * (size_t)e.ne1;
      const size_t qsb = nblk * (il ? 32u : 16u), scb = nblk * (il ? 4u : 2u);
      if (e.a > rem || e.b > rem || qsb > rem - e.a || scb > rem - e.b) continue;  /* out of the file */
      gguf_tensor *t = &g->t[e.t];
      t->data = p + base + e.a;
      t->scales = p + base + e.b;
      t->type = il ? CWEN_T_Q4_0RSI : CWEN_T_Q4_0RS;
      t->side = e.flags == R_IL_B;
      bound++;
    }
    if (!bound) goto none;
    g->rmap = map;
    g->rlen = len;
  } else {
    /* v2: packed {u8 qs[16]; f32 d} blocks, split into qs and f16 scales */
    r_entry *es = (r_entry *)calloc(n ? n : 1, sizeof *es);
    if (!es) {
      rc = CWEN_ENOMEM;
      goto drop;
    }
    size_t total = 0;
    int k = 0;
    for (uint32_t i = 0; i < n; i++) {
      r_entry e;
      if (r_match(g, p, i, &e) < 0) continue;
      const size_t nblk = (size_t)(e.ne0 / 32) * (size_t)e.ne1;
      if (e.a > rem || e.b > rem - e.a || e.b != nblk * 20u) continue;  /* out of the file, or mis-sized */
      es[k++] = e;
      total += nblk;
    }
    if (!k) {
      free(es);
      goto none;
    }
    uint8_t *arena = (uint8_t *)malloc(total * 18u);
    if (!arena) {
      free(es);
      rc = CWEN_ENOMEM;
      goto drop;
    }
    uint8_t *qd = arena;
    uint16_t *sd = (uint16_t *)(arena + total * 16u);
    for (int j = 0; j < k; j++) {
      gguf_tensor *t = &g->t[es[j].t];
      if (t->type != CWEN_T_Q4_0) continue;  /* a repeated name binds once */
      const size_t nblk = (size_t)(es[j].ne0 / 32) * (size_t)es[j].ne1;
      const uint8_t *src = p + base + es[j].a;
      for (size_t b = 0; b < nblk; b++) {
        float d;
        memcpy(qd + b * 16, src + b * 20, 16);
        memcpy(&d, src + b * 20 + 16, 4);
        sd[b] = f32_to_f16_rne(d);
      }
      t->data = qd;
      t->scales = sd;
      t->type = CWEN_T_Q4_0RS;
      t->side = 0;
      qd += nblk * 16u;
      sd += nblk;
      bound++;
    }
    free(es);
    g->split = arena;
    munmap(map, len);
  }
  g_err[0] = 0;
  return bound;
none:
  snprintf(g_err, sizeof g_err, "cwenr: no usable entries");
  munmap(map, len);
  return 0;
drop:
  munmap(map, len);
  return rc;
}

/* ------------------------------------------------------------------ binder */

/* Matrix types the device GEMV computes (the reference's matmul_type_ok,
 * run.c:1311-1318, minus its drafter-only T_Q8S). */
static int q4_family(int ty) { return ty == CWEN_T_Q4_0 || ty == CWEN_T_Q4_0RS || ty == CWEN_T_Q4_0RSI; }
static int mat_type_ok(int ty) {
  return q4_family(ty) || ty == CWEN_T_Q4_1 || ty == CWEN_T_Q8_0 || ty == CWEN_T_Q5_K || ty == CWEN_T_Q6_K;
}

/* Block i (row-major over rows, then K) of a Q4_0 tensor in any of its three
 * layouts: the f16 scale bits and the 16 nibble bytes. */
static const uint8_t *q4_block(const gguf_tensor *t, size_t i, uint16_t *d) {
  const uint8_t *q = (const uint8_t *)t->data, *sc = (const uint8_t *)t->scales;
  switch (t->type) {
    case CWEN_T_Q4_0: memcpy(d, q + i * 18, 2); return q + i * 18 + 2;
    case CWEN_T_Q4_0RS: memcpy(d, sc + i * 2, 2); return q + i * 16;
    default: memcpy(d, sc + (2 * i + t->side) * 2, 2); return q + i * 32 + 16 * t->side;
  }
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
/* A matrix as the device takes it: GGUF types and a sidecar's split (RS)
 * view as they are; one side of an interleaved (RSI) view split out first. */
static int set_mat(cwen_model *m, int layer, int id, const gguf_tensor *t) {
  if (t->type != CWEN_T_Q4_0RSI) return cwen_model_set(m, layer, id, t->type, t->data, t->scales, t->ne0, t->ne1);
  const size_t nblk = (size_t)(t->ne0 / 32) * t->ne1;
  uint8_t *qs = (uint8_t *)malloc(nblk * 18);
  if (!qs) return CWEN_ENOMEM;
  uint16_t *sc = (uint16_t *)(qs + nblk * 16);
  for (size_t i = 0; i < nblk; i++) memcpy(qs + i * 16, q4_block(t, i, &sc[i]), 16);
  const int rc = cwen_model_set(m, layer, id, CWEN_T_Q4_0RS, qs, sc, t->ne0, t->ne1);
  free(qs);
  return rc;
}

/* Two Q4_0 matrices of one shape as an interleaved pair,
 * qs[row][block][a 16 | b 16], f16 sc[row][block][a | b]: a sidecar's pair
 * as it is, any other combination of layouts interleaved on the host. */
static int set_pair(cwen_model *m, int layer, int id, const gguf_tensor *a, const gguf_tensor *b) {
  if (!q4_family(a->type) || !q4_family(b->type)) return fail("pair halves must be Q4_0");
  if (a->type == CWEN_T_Q4_0RSI && b->type == CWEN_T_Q4_0RSI && a->data == b->data && a->scales == b->scales &&
      a->side == 0 && b->side == 1)
    return cwen_model_set(m, layer, id, CWEN_T_Q4_0RSI, a->data, a->scales, a->ne0, a->ne1);
  const size_t nblk = (size_t)(a->ne0 / 32) * a->ne1;
  uint8_t *qs = (uint8_t *)malloc(nblk * 36);
  if (!qs) return CWEN_ENOMEM;
  uint16_t *sc = (uint16_t *)(qs + nblk * 32);
  for (size_t i = 0; i < nblk; i++) {
    memcpy(qs + i * 32, q4_block(a, i, &sc[2 * i]), 16);
    memcpy(qs + i * 32 + 16, q4_block(b, i, &sc[2 * i + 1]), 16);
  }
  const int rc = cwen_model_set(m, layer, id, CWEN_T_Q4_0RSI, qs, sc, a->ne0, a->ne1);
  free(qs);
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
  if (!q4_family(t->type) && t->type != CWEN_T_Q6_K) return fail("token_embd.weight: the device embedding takes Q4_0 or Q6_K");
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
  /* The MTP nextn block blk.N, N = n_layers (run.c:3409-3464): bound when
   * its eh_proj is present, and then every part with its shape pinned. */
  snprintf(n, sizeof n, "blk.%d.nextn.eh_proj.weight", c->n_layers);
  if (cwen_gguf_find(g, n) >= 0) {
    const int l = c->n_layers;
    NEED(t, mat(g, n, 2 * H, H, &rc));
    TRY(set_mat(m, -1, CWEN_NEXTN_EH_PROJ, t));
    static const struct { const char *suf; int id; } norms[] = {
        {"nextn.enorm.weight", CWEN_NEXTN_ENORM}, {"nextn.hnorm.weight", CWEN_NEXTN_HNORM},
        {"nextn.shared_head_norm.weight", CWEN_NEXTN_SHEAD_NORM}};
    for (int k = 0; k < 3; k++) {
      snprintf(n, sizeof n, "blk.%d.%s", l, norms[k].suf);
      NEED(u, vec(g, n, H, &rc));
      TRY(set_vec(m, -1, norms[k].id, u, H));
    }
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
#undef NM
  }
  g_err[0] = 0;
  return CWEN_OK;
}

/* The model geometry from the shapes of the tensors cwen_model_load_gguf
 * binds.  The reference compiles its geometry in (run.c:83-91) and pins
 * every shape to it at load; read back from the shapes of its own model
 * file, this gives those constants.  RoPE (64 rotated dimensions, theta
 * 1e7) and the norm epsilon (1e-6) leave no trace in the shapes and are the
 * reference's values. */
static int dim_of(const cwen_gguf *g, const char *name, int which, int *out) {
  const int i = cwen_gguf_find(g, name);
  if (i < 0) {
    char m[160];
    snprintf(m, sizeof m, "geometry: missing %.100s", name);
    return fail(m);
  }
  *out = which ? g->t[i].ne1 : g->t[i].ne0;
  return CWEN_OK;
}

int cwen_model_cfg_from_gguf(const cwen_gguf *g, int max_ctx, cwen_model_cfg *c) {
  if (!g || !c) return fail("null argument");
  memset(c, 0, sizeof *c);
  char n[G_NAME];
  int rc, nl = 0, first_full = -1, first_linear = -1, qkv = 0, qrows = 0, krows = 0;
  if ((rc = dim_of(g, "token_embd.weight", 0, &c->d_model)) || (rc = dim_of(g, "token_embd.weight", 1, &c->vocab)))
    return rc;
  for (;; nl++) {
    snprintf(n, sizeof n, "blk.%d.attn_norm.weight", nl);
    if (cwen_gguf_find(g, n) < 0) break;
    snprintf(n, sizeof n, "blk.%d.nextn.eh_proj.weight", nl);
    if (cwen_gguf_find(g, n) >= 0) break;   /* the MTP block follows the decoder layers */
    snprintf(n, sizeof n, "blk.%d.attn_q.weight", nl);
    const int full = cwen_gguf_find(g, n) >= 0;
    if (full && first_full < 0) first_full = nl;
    if (!full && first_linear < 0) first_linear = nl;
  }
  if (nl < 1) return fail("geometry: no decoder layers (blk.0.attn_norm.weight)");
  if (first_full < 0) return fail("geometry: no full-attention layer (blk.N.attn_q.weight)");
  c->n_layers = nl;
  c->full_interval = first_full + 1;
  if ((rc = dim_of(g, "blk.0.ffn_down.weight", 0, &c->d_ffn))) return rc;
  const int f = first_full;
#define DIM(fmt, l, which, dst)                          \
  do {                                                   \
    snprintf(n, sizeof n, fmt, l);                       \
    if ((rc = dim_of(g, n, which, dst))) return rc;      \
  } while (0)
  DIM("blk.%d.attn_q_norm.weight", f, 0, &c->head_dim);
  DIM("blk.%d.attn_q.weight", f, 1, &qrows);
  DIM("blk.%d.attn_k.weight", f, 1, &krows);
  if (c->head_dim < 1 || qrows % (2 * c->head_dim) || krows % c->head_dim)
    return fail("geometry: attention rows are not whole heads");
  c->n_head = qrows / (2 * c->head_dim);
  c->n_kv_head = krows / c->head_dim;
  if (first_linear >= 0) {
    DIM("blk.%d.ssm_norm.weight", first_linear, 0, &c->gdn_dk);
    DIM("blk.%d.ssm_alpha.weight", first_linear, 1, &c->gdn_nvh);
    DIM("blk.%d.attn_qkv.weight", first_linear, 1, &qkv);
    const int kd = qkv - c->gdn_nvh * c->gdn_dk;
    if (c->gdn_dk < 1 || kd < 0 || kd % (2 * c->gdn_dk)) return fail("geometry: GatedDeltaNet rows are not whole heads");
    c->gdn_nkh = kd / (2 * c->gdn_dk);
  }
#undef DIM
  c->n_rot = 64;
  c->n_rot_pairs = 32;
  c->rope_theta = 1e7f;
  c->rms_eps = 1e-6f;
  c->max_ctx = max_ctx;
  g_err[0] = 0;
  return CWEN_OK;
}
