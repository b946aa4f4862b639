/* Host decode drivers over the cwen_gpu C ABI (see cwen_host.h). */
#define _POSIX_C_SOURCE 199309L
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

int cwen_generate_spec(cwen_model *m, const int *prompt, int n_prompt, int n_gen, const cwen_spec_cfg *cfg_in,
                       int *out, cwen_spec_stats *stats) {
  if (!m || !out || n_gen < 0) return CWEN_EINVAL;
  cwen_spec_cfg cfg;
  if (cfg_in) cfg = *cfg_in; else cwen_spec_default(&cfg);
  if (cfg.max_draft > CWEN_BMAX - 1) cfg.max_draft = CWEN_BMAX - 1;
  cwen_spec_stats st;
  memset(&st, 0, sizeof st);
  st.prefill_tokens = n_prompt;
  int *hist = (int *)malloc(sizeof(int) * (size_t)(n_prompt + n_gen + CWEN_BMAX));
  if (!hist) return CWEN_ENOMEM;
  int pend, rc;
  double t0 = now_s();
  if ((rc = cwen_prefill(m, prompt, n_prompt, &pend))) { free(hist); return rc; }
  double t1 = now_s();
  st.prefill_s = t1 - t0;
  memcpy(hist, prompt, sizeof(int) * (size_t)n_prompt);
  const int cap = cwen_model_capacity(m);
  int hn = n_prompt, g = 0, streak = 0, cool = 0, fa_streak = 0;
  if (n_gen > 0 && cwen_model_pos(m) + 1 < cap) {
    hist[hn++] = pend;
    out[g++] = pend;
  }
  const int cap_hard = cfg.max_draft;
  const int use_mtp = cfg.mtp && cwen_model_has_mtp(m) == 1;
  int E_cap = cap_hard;
  int blk[CWEN_BMAX];
  while (g > 0 && g < n_gen) {
    if (cfg.max_cycles > 0 && st.cycles >= cfg.max_cycles) break;
    const int pos = cwen_model_pos(m);
    if (pos + 1 >= cap) break;                     /* same context cap as the serial loop */
    int E = 0;
    if (cool > 0) {
      cool--;
    } else {
      const int room = cap - 1 - (pos + 1);        /* block slots must stay in range */
      const int lim = E_cap < room ? E_cap : room;
      if (use_mtp) {
        E = cwen_model_mtp_draft(m, hist[hn - 1], lim, blk + 1, NULL);
        if (E < 0) { free(hist); return E; }
      } else {
        E = cwen_ngram_draft(hist, hn, blk + 1, cfg.n_key, lim);
      }
      if (E && E < cfg.min_draft) E = 0;
    }
    blk[0] = hist[hn - 1];                         /* pend */
    int k = 0, bonus;
    st.cycles++;
    if ((rc = cwen_model_verify(m, blk, E + 1, &k, &bonus, NULL))) { free(hist); return rc; }
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
    for (int i = 0; i < k && g < n_gen; i++) out[g++] = blk[i + 1];
    if (g >= n_gen) break;
    out[g++] = bonus;
    if (k == E) streak = 0;
    else if (++streak >= 3) { streak = 0; cool = cfg.cooldown; }
  }
  st.decode_s = now_s() - t1;
  free(hist);
  if (stats) *stats = st;
  return g;
}
