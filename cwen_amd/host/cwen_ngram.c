/* Counted n-gram map for the speculative driver's drafts (see cwen_host.h).
 *
 * Reference: the NGMap of run.c:204-221 and ng_hash / ng_find /
 * ng_update_key_n / ng_evict_one / ng_update_range / ng_draft_map / ng_save /
 * ng_load, run.c:4552-4723.  A key of n_key confirmed tokens maps to the
 * token that last followed it and a hit count.  The table is open-addressed
 * with linear probing over a power-of-two capacity; a full table drops one
 * least-hit entry (equal counts taken in turn by a rotating hand) and closes
 * the hole by backward shifting, so probe chains stay unbroken.
 *
 * The hash, the probe order and the eviction order are the reference's: they
 * decide which entries survive a full table, and so which drafts the driver
 * proposes.  The NGC2 file layout is the reference's too, so maps persist
 * across the two engines.
 */
#include <limits.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "cwen_host.h"

#define NGC2_MAGIC 0x3243474eu /* "NGC2", little-endian */
#define NG_KEY_MAX 256

struct cwen_ngmap {
  int n_key, vocab;
  size_t cap, mask, used_n, hand;
  size_t evicted, evicted_in_place;   /* evictions; those where no entry shifted */
  int *keys;             /* [cap][n_key] */
  int *tok, *cnt;        /* [cap] */
  unsigned char *used;   /* [cap] */
};

/* FNV-1a-style over the key's ids with the FNV-64 prime, each step followed
 * by a xor-shift by 29 (run.c:4555-4562).  The seed is run.c's decimal
 * 1469598103934665603, which is not the FNV-64 offset basis
 * (14695981039346656037): slot placement, and with it eviction, follows the
 * reference's value. */
static uint64_t key_hash(const int *k, int n) {
  uint64_t h = 0x14650fb0739d0383ull;
  for (int i = 0; i < n; i++) {
    h = (h ^ (uint64_t)(uint32_t)k[i]) * 0x100000001b3ull;
    h ^= h >> 29;
  }
  return h;
}

static int *slot_key(const cwen_ngmap *m, size_t s) { return m->keys + s * (size_t)m->n_key; }

/* The slot holding key (*hit = 1), else the first free slot of its probe
 * chain (*hit = 0), else cap when every slot is taken. */
static size_t probe(const cwen_ngmap *m, const int *key, int *hit) {
  const size_t kb = (size_t)m->n_key * sizeof(int);
  size_t s = (size_t)key_hash(key, m->n_key) & m->mask;
  for (size_t step = 0; step < m->cap; step++, s = (s + 1) & m->mask) {
    if (!m->used[s]) { *hit = 0; return s; }
    if (memcmp(slot_key(m, s), key, kb) == 0) { *hit = 1; return s; }
  }
  *hit = 0;
  return m->cap;
}

/* Drop one entry of the lowest count: among equals, the first at or after
 * the hand; the hand then moves past it.  Entries after the hole move back
 * into it when their home slot does not lie cyclically in (hole, slot]. */
static void evict_one(cwen_ngmap *m) {
  int low = INT_MAX;
  for (size_t s = 0; s < m->cap; s++)
    if (m->used[s] && m->cnt[s] < low) low = m->cnt[s];
  size_t victim = m->cap;
  for (size_t i = 0; i < m->cap; i++) {
    const size_t s = (m->hand + i) & m->mask;
    if (m->used[s] && m->cnt[s] == low) { victim = s; break; }
  }
  if (victim == m->cap) return;   /* empty table */
  m->hand = (victim + 1) & m->mask;
  const size_t kb = (size_t)m->n_key * sizeof(int);
  size_t hole = victim;
  for (size_t i = 1; i < m->cap; i++) {
    const size_t s = (victim + i) & m->mask;
    if (!m->used[s]) break;
    const size_t home = (size_t)key_hash(slot_key(m, s), m->n_key) & m->mask;
    const size_t d_home = (home - hole) & m->mask, d_slot = (s - hole) & m->mask;
    if (d_home == 0 || d_home > d_slot) {
      memcpy(slot_key(m, hole), slot_key(m, s), kb);
      m->tok[hole] = m->tok[s];
      m->cnt[hole] = m->cnt[s];
      hole = s;
    }
  }
  /* The last slot vacated is free.  When no entry moves this is the victim
   * itself: run.c leaves that slot marked in use, so its next probe finds no
   * free slot and the insertion lands one entry past the end of its arrays. */
  m->used[hole] = 0;
  m->used_n--;
  m->evicted++;
  if (hole == victim) m->evicted_in_place++;
}

int cwen_ngmap_create(int n_key, int vocab, size_t cap, cwen_ngmap **out) {
  if (!out || n_key < 1 || n_key > NG_KEY_MAX || vocab < 1) return CWEN_EINVAL;
  if (cap == 0) cap = CWEN_NGMAP_CAP;
  if (cap < 2 || (cap & (cap - 1)) || cap > SIZE_MAX / ((size_t)n_key * sizeof(int))) return CWEN_EINVAL;
  cwen_ngmap *m = (cwen_ngmap *)calloc(1, sizeof *m);
  if (!m) return CWEN_ENOMEM;
  m->n_key = n_key;
  m->vocab = vocab;
  m->cap = cap;
  m->mask = cap - 1;
  m->keys = (int *)malloc(cap * (size_t)n_key * sizeof(int));
  m->tok = (int *)malloc(cap * sizeof(int));
  m->cnt = (int *)calloc(cap, sizeof(int));
  m->used = (unsigned char *)calloc(cap, 1);
  if (!m->keys || !m->tok || !m->cnt || !m->used) {
    cwen_ngmap_free(m);
    return CWEN_ENOMEM;
  }
  *out = m;
  return CWEN_OK;
}

void cwen_ngmap_free(cwen_ngmap *m) {
  if (!m) return;
  free(m->keys);
  free(m->tok);
  free(m->cnt);
  free(m->used);
  free(m);
}

int cwen_ngmap_n_key(const cwen_ngmap *m) { return m ? m->n_key : CWEN_EINVAL; }

size_t cwen_ngmap_used(const cwen_ngmap *m) { return m ? m->used_n : 0; }

void cwen_ngmap_evictions(const cwen_ngmap *m, size_t *evicted, size_t *in_place) {
  if (evicted) *evicted = m ? m->evicted : 0;
  if (in_place) *in_place = m ? m->evicted_in_place : 0;
}

void cwen_ngmap_update(cwen_ngmap *m, const int *key, int tok, int hits) {
  if (!m || !key) return;
  int hit;
  size_t s = probe(m, key, &hit);
  if (hit) {
    m->cnt[s] = hits < INT_MAX - m->cnt[s] ? m->cnt[s] + hits : INT_MAX;
    m->tok[s] = tok;
    return;
  }
  if (s == m->cap) {           /* full: make room, then look again */
    evict_one(m);
    s = probe(m, key, &hit);
    if (s == m->cap) return;
  }
  memcpy(slot_key(m, s), key, (size_t)m->n_key * sizeof(int));
  m->tok[s] = tok;
  m->cnt[s] = hits;
  m->used[s] = 1;
  m->used_n++;
}

void cwen_ngmap_update_range(cwen_ngmap *m, const int *h, int a, int b) {
  if (!m || !h) return;
  for (int p = a < m->n_key ? m->n_key : a; p < b; p++) cwen_ngmap_update(m, h + p - m->n_key, h[p], 1);
}

int cwen_ngmap_draft(const cwen_ngmap *m, const int *h, int hn, int *out, int max_d) {
  if (!m || !h || !out || hn < m->n_key || max_d <= 0) return 0;
  int key[NG_KEY_MAX];
  memcpy(key, h + hn - m->n_key, (size_t)m->n_key * sizeof(int));
  int n = 0;
  while (n < max_d) {
    int hit;
    const size_t s = probe(m, key, &hit);
    if (!hit) break;
    out[n] = m->tok[s];
    memmove(key, key + 1, (size_t)(m->n_key - 1) * sizeof(int));
    key[m->n_key - 1] = out[n++];
  }
  return n;
}

int cwen_ngmap_save(const cwen_ngmap *m, const char *path) {
  if (!m || !path) return CWEN_EINVAL;
  const size_t plen = strlen(path);
  char *tmp = (char *)malloc(plen + 5);
  if (!tmp) return CWEN_ENOMEM;
  memcpy(tmp, path, plen);
  memcpy(tmp + plen, ".tmp", 5);
  FILE *f = fopen(tmp, "wb");
  if (!f) {
    fprintf(stderr, "n-gram map: cannot create %s\n", tmp);
    free(tmp);
    return CWEN_EIO;
  }
  const uint32_t head[4] = {NGC2_MAGIC, (uint32_t)m->n_key, (uint32_t)m->vocab, (uint32_t)m->used_n};
  int ok = fwrite(head, sizeof head, 1, f) == 1;
  for (size_t s = 0; ok && s < m->cap; s++) {
    if (!m->used[s]) continue;
    ok = fwrite(slot_key(m, s), sizeof(int), (size_t)m->n_key, f) == (size_t)m->n_key &&
         fwrite(&m->tok[s], sizeof(int), 1, f) == 1 && fwrite(&m->cnt[s], sizeof(int), 1, f) == 1;
  }
  ok = (fclose(f) == 0) && ok;
  if (!ok || rename(tmp, path) != 0) {
    fprintf(stderr, "n-gram map: writing %s failed; nothing saved\n", path);
    remove(tmp);
    free(tmp);
    return CWEN_EIO;
  }
  free(tmp);
  return CWEN_OK;
}

int cwen_ngmap_load(cwen_ngmap *m, const char *path) {
  if (!m || !path) return CWEN_EINVAL;
  FILE *f = fopen(path, "rb");
  if (!f) {
    fprintf(stderr, "n-gram map: no file at %s; starting empty\n", path);
    return 0;
  }
  /* The map only proposes drafts, which the model verifies: a file that
   * cannot be used is reported and skipped, never fatal. */
  uint32_t head[4];
  const char *why = NULL;
  if (fread(head, sizeof head, 1, f) != 1) why = "header cut short";
  else if (head[0] != NGC2_MAGIC) why = "not an NGC2 file";
  if (why) {
    fprintf(stderr, "n-gram map: %s: %s; starting empty\n", path, why);
    fclose(f);
    return 0;
  }
  if ((int)head[1] != m->n_key || (int)head[2] != m->vocab) {
    fprintf(stderr, "n-gram map: %s holds keys of %u tokens over a vocabulary of %u, this run uses %d and %d; "
                    "starting empty\n", path, head[1], head[2], m->n_key, m->vocab);
    fclose(f);
    return 0;
  }
  int key[NG_KEY_MAX + 2];     /* key, then tok and count */
  const size_t rec = (size_t)m->n_key + 2;
  int merged = 0;
  for (uint32_t r = 0; r < head[3] && m->used_n < m->cap; r++) {
    if (fread(key, sizeof(int), rec, f) != rec) break;   /* file cut short: keep what was read */
    const int tok = key[m->n_key], cnt = key[m->n_key + 1];
    if (tok < 0 || tok >= m->vocab || cnt < 1) continue;
    cwen_ngmap_update(m, key, tok, cnt);
    merged++;
  }
  fclose(f);
  fprintf(stderr, "n-gram map: %d entries merged from %s\n", merged, path);
  return merged;
}

int cwen_ngmap_dump(const cwen_ngmap *m, int *keys, int *tok, int *cnt, unsigned char *used) {
  if (!m) return CWEN_EINVAL;
  if (keys) memcpy(keys, m->keys, m->cap * (size_t)m->n_key * sizeof(int));
  if (tok) memcpy(tok, m->tok, m->cap * sizeof(int));
  if (cnt) memcpy(cnt, m->cnt, m->cap * sizeof(int));
  if (used) memcpy(used, m->used, m->cap);
  return CWEN_OK;
}
