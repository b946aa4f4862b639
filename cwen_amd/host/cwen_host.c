/* Host decode drivers over the cwen_gpu C ABI (see cwen_host.h). */
#define _POSIX_C_SOURCE 199309L
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "cwen_host.h"

#define PREFILL_BLOCK 16

static double now_s(void) {
  struct timespec t;
  clock_gettime(CLOCK_MONOTONIC, &t);
  return (double)t.tv_sec + 1e-9 * (double)t.tv_nsec;
}

void cwen_spec_default(cwen_spec_cfg *cfg) {
  cfg->n_key = 16;
  cfg->max_draft = 8;
  cfg->min_draft = 2;
  cfg->cooldown = 8;
  cfg->max_cycles = 0;
  cfg->mtp = 1;
  cfg->ngmap = NULL;
  cfg->cycle_log = NULL;
  cfg->cycle_log_cap = 0;
  cfg->debug = 0;
  cfg->fa_streak = NULL;
}

/* run.c:4533-4549 */
int cwen_ngram_draft(const int *h, int hn, int *out, int n_key, int max_d) {
  if (hn <= n_key || max_d <= 0) return 0;
  const int *tail = h + hn - n_key;
  int best = 0;
  for (int j = hn - n_key - 1; j >= 0 && best < max_d; j--) {
    if (memcmp(h + j, tail, (size_t)n_key * sizeof(int)) != 0) continue;
    const int avail = hn - (j + n_key);
    if (avail > best) {
      const int n = avail < max_d ? avail : max_d;
      memcpy(out, h + j + n_key, (size_t)n * sizeof(int));
      best = n;
    }
  }
  return best;
}

int cwen_prefill(cwen_model *m, const int *prompt, int n_prompt, int *next) {
  if (!m || !prompt || n_prompt < 1 || !next) return CWEN_EINVAL;
  int rc = cwen_model_reset(m);
  if (rc) return rc;
  for (int i = 0; i < n_prompt;) {
    int B = n_prompt - i;
    if (B > PREFILL_BLOCK) B = PREFILL_BLOCK;
    const int last = i + B == n_prompt;
    int am[CWEN_BMAX];
    rc = cwen_model_forward(m, prompt + i, B, last, last ? am : NULL, NULL);
    if (rc) return rc;
    if (last) *next = am[B - 1];
    i += B;
  }
  return CWEN_OK;
}

/* run.c:5027-5045: one position per pass, stopping when the context fills. */
int cwen_generate_serial(cwen_model *m, const int *prompt, int n_prompt, int n_gen, int *out,
                         cwen_spec_stats *stats) {
  if (!m || !out || n_gen < 0) return CWEN_EINVAL;
  const int cap = cwen_model_capacity(m);
  cwen_spec_stats st;
  memset(&st, 0, sizeof st);
  st.prefill_tokens = n_prompt;
  int next, rc;
  double t0 = now_s();
  if ((rc = cwen_prefill(m, prompt, n_prompt, &next))) return rc;
  double t1 = now_s();
  st.prefill_s = t1 - t0;
  int n = 0;
  for (int g = 0; g < n_gen; g++) {
    if (cwen_model_pos(m) + 1 >= cap) break;
    out[n++] = next;
    if (g + 1 == n_gen) break;
    int k, bonus;
    if ((rc = cwen_model_verify(m, &next, 1, &k, &bonus, NULL))) return rc;
    st.cycles++;
    next = bonus;
  }
  st.decode_s = now_s() - t1;
  if (stats) *stats = st;
  return n;
}

/* What the speculative loop needs of a model. */
typedef struct {
  void *ud;
  int (*prefill)(void *ud, const int *prompt, int n_prompt, int *next);
  int (*pos)(void *ud);
  int (*capacity)(void *ud);
  int (*verify)(void *ud, const int *blk, int B, int *k, int *bonus);
  int (*mtp_draft)(void *ud, int pend, int n, int *out);   /* NULL: no MTP block */
} spec_model;

/* generate_tokens_spec (run.c:4882-5025) over m. */
static int spec_loop(const spec_model *M, const int *prompt, int n_prompt, int n_gen, const cwen_spec_cfg *cfg_in,
                     int *out, cwen_spec_stats *stats) {
  if (!out || n_gen < 0 || !prompt || n_prompt < 1) return CWEN_EINVAL;
  cwen_spec_cfg cfg;
  if (cfg_in) cfg = *cfg_in; else cwen_spec_default(&cfg);
  if (cfg.max_draft > CWEN_BMAX - 1) cfg.max_draft = CWEN_BMAX - 1;
  if (cfg.ngmap && cwen_ngmap_n_key(cfg.ngmap) != cfg.n_key) return CWEN_EINVAL;
  cwen_spec_stats st;
  memset(&st, 0, sizeof st);
  st.prefill_tokens = n_prompt;
  int *hist = (int *)malloc(sizeof(int) * (size_t)(n_prompt + n_gen + CWEN_BMAX));
  if (!hist) return CWEN_ENOMEM;
  int pend, rc;
  double t0 = now_s();
  if ((rc = M->prefill(M->ud, prompt, n_prompt, &pend))) { free(hist); return rc; }
  double t1 = now_s();
  st.prefill_s = t1 - t0;
  memcpy(hist, prompt, sizeof(int) * (size_t)n_prompt);
  const int cap = M->capacity(M->ud);
  int hn = n_prompt, g = 0, streak = 0, cool = 0, upd = 0;
  int fa_streak = cfg.fa_streak ? *cfg.fa_streak : 0;
  if (n_gen > 0 && M->pos(M->ud) + 1 < cap) {
    hist[hn++] = pend;
    out[g++] = pend;
  }
  if (cfg.ngmap) { cwen_ngmap_update_range(cfg.ngmap, hist, upd, hn); upd = hn; }
  const int cap_hard = cfg.max_draft;
  const int use_mtp = cfg.mtp && M->mtp_draft;
  int E_cap = cap_hard;
  int blk[CWEN_BMAX], scan[CWEN_BMAX];
  while (g > 0 && g < n_gen) {
    if (cfg.max_cycles > 0 && st.cycles >= cfg.max_cycles) break;
    const int pos = M->pos(M->ud);
    if (pos + 1 >= cap) break;                     /* same context cap as the serial loop */
    int E = 0;
    if (cool > 0) {
      cool--;
    } else {
      const int room = cap - 1 - (pos + 1);        /* block slots must stay in range */
      const int lim = E_cap < room ? E_cap : room;
      if (use_mtp) {
        E = M->mtp_draft(M->ud, hist[hn - 1], lim, blk + 1);
        if (E < 0) { free(hist); return E; }
      } else {
        /* the map's chained lookups first; the history scan wins when it
         * proposes a longer run */
        E = cfg.ngmap ? cwen_ngmap_draft(cfg.ngmap, hist, hn, blk + 1, lim) : 0;
        const int esc = cwen_ngram_draft(hist, hn, scan, cfg.n_key, lim);
        if (esc > E) {
          E = esc;
          memcpy(blk + 1, scan, sizeof(int) * (size_t)E);
        }
      }
      if (E && E < cfg.min_draft) E = 0;
    }
    blk[0] = hist[hn - 1];                         /* pend */
    if (cfg.debug)
      fprintf(stderr, "spec cycle %lld: history %d, position %d, drafts %d, pending %d\n", st.cycles, hn, pos, E,
              blk[0]);
    int k = 0, bonus;
    if ((rc = M->verify(M->ud, blk, E + 1, &k, &bonus))) { free(hist); return rc; }
    if (cfg.cycle_log && st.cycles < cfg.cycle_log_cap) {
      cfg.cycle_log[2 * st.cycles] = E;
      cfg.cycle_log[2 * st.cycles + 1] = k;
    }
    st.cycles++;
    if (E > 0) {
      st.drafted++;
      st.kept += k;
      if (k == E) {
        st.full++;
        if (++fa_streak >= 4 && E_cap < cap_hard) { E_cap++; fa_streak = 0; }
      } else {
        st.rejected++;
        fa_streak = 0;
        E_cap = k > cfg.min_draft ? k : cfg.min_draft;
      }
    }
    for (int i = 0; i < k; i++) hist[hn++] = blk[i + 1];
    hist[hn++] = bonus;
    if (cfg.ngmap) { cwen_ngmap_update_range(cfg.ngmap, hist, upd, hn); upd = hn; }
    for (int i = 0; i < k && g < n_gen; i++) out[g++] = blk[i + 1];
    if (g >= n_gen) break;
    out[g++] = bonus;
    if (k == E) streak = 0;
    else if (++streak >= 3) { streak = 0; cool = cfg.cooldown; }
  }
  st.decode_s = now_s() - t1;
  if (cfg.fa_streak) *cfg.fa_streak = fa_streak;
  free(hist);
  if (cfg.debug)
    fprintf(stderr, "spec: %lld passes, %lld with drafts (%lld kept whole, %lld cut short), %.2f drafts kept on "
                    "average\n", st.cycles, st.drafted, st.full, st.rejected,
            st.drafted ? (double)st.kept / (double)st.drafted : 0.0);
  if (stats) *stats = st;
  return g;
}

/* ---- the device model ---- */
static int dev_prefill(void *ud, const int *p, int n, int *next) { return cwen_prefill((cwen_model *)ud, p, n, next); }
static int dev_pos(void *ud) { return cwen_model_pos((cwen_model *)ud); }
static int dev_capacity(void *ud) { return cwen_model_capacity((cwen_model *)ud); }
static int dev_verify(void *ud, const int *blk, int B, int *k, int *bonus) {
  return cwen_model_verify((cwen_model *)ud, blk, B, k, bonus, NULL);
}
static int dev_mtp_draft(void *ud, int pend, int n, int *out) {
  return cwen_model_mtp_draft((cwen_model *)ud, pend, n, out, NULL);
}

int cwen_generate_spec(cwen_model *m, const int *prompt, int n_prompt, int n_gen, const cwen_spec_cfg *cfg,
                       int *out, cwen_spec_stats *stats) {
  if (!m) return CWEN_EINVAL;
  const spec_model M = {m, dev_prefill, dev_pos, dev_capacity, dev_verify,
                        cwen_model_has_mtp(m) == 1 ? dev_mtp_draft : NULL};
  return spec_loop(&M, prompt, n_prompt, n_gen, cfg, out, stats);
}

/* ---- a recorded greedy stream ---- */
typedef struct {
  const int *s;
  int n, n_prompt, max_ctx, pos;   /* pos: last filled position */
} replay_model;

static int rp_prefill(void *ud, const int *p, int n, int *next) {
  replay_model *r = (replay_model *)ud;
  if (n != r->n_prompt || n >= r->n || memcmp(p, r->s, sizeof(int) * (size_t)n) != 0) return CWEN_EINVAL;
  r->pos = n - 1;
  *next = r->s[n];
  return CWEN_OK;
}
static int rp_pos(void *ud) { return ((replay_model *)ud)->pos; }
static int rp_capacity(void *ud) { return ((replay_model *)ud)->max_ctx; }
static int rp_verify(void *ud, const int *blk, int B, int *k, int *bonus) {
  replay_model *r = (replay_model *)ud;
  /* blk[b] sits at position pos + 1 + b; the greedy id after it is s[pos + 2 + b] */
  const int p = r->pos + 1;
  if (B < 1 || p + B >= r->n || blk[0] != r->s[p]) return CWEN_EINVAL;
  int kk = 0;
  while (kk < B - 1 && blk[kk + 1] == r->s[p + 1 + kk]) kk++;
  *k = kk;
  *bonus = r->s[p + 1 + kk];
  r->pos = p + kk;
  return CWEN_OK;
}

int cwen_spec_replay(const int *stream, int n_stream, int n_prompt, int n_gen, int max_ctx,
                     const cwen_spec_cfg *cfg, int *out, cwen_spec_stats *stats) {
  if (!stream || n_prompt < 1 || n_stream <= n_prompt || max_ctx < 2) return CWEN_EINVAL;
  replay_model r = {stream, n_stream, n_prompt, max_ctx, -1};
  const spec_model M = {&r, rp_prefill, rp_pos, rp_capacity, rp_verify, NULL};
  return spec_loop(&M, stream, n_prompt, n_gen, cfg, out, stats);
}
