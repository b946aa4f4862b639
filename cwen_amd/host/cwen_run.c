/* cwen_run -- the command-line front end of the reference engine's `run`
 * (run.c:5080-5251 main, run_usage; the knobs of spec_config_init 4021-4052,
 * rope_env_init 4096-4104 and env_int / env_bool / arg_int_range 2481-2520)
 * over the GPU library: the model is loaded from the GGUF file (and its CWENR
 * sidecar) into HBM, and every forward pass runs on the GPU.
 *
 *   cwen_run [MODEL] [IDS_FILE] [N_PREDICT] [-d N]
 *
 * Greedy ids go to stdout, space-separated, then a newline; logs go to
 * stderr.  CWEN_SERVER=1 answers binary frames on stdin/stdout instead.
 * Knobs that steer the reference's CPU kernels (thread count, weight
 * residency and prefetch) have nothing to steer here and are ignored; the
 * features the GPU path does not provide (activation dumps, YaRN scaling, the
 * DFlash drafter) are refused before the model loads.
 */
#define _POSIX_C_SOURCE 200809L
#include <errno.h>
#include <limits.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>

#include "cwen_host.h"

#define DEFAULT_MODEL "model/Qwen3.8-27B-Q4_0.gguf"
#define DEFAULT_TOKEN 248044   /* the reference's prompt when no ids file is given */
#define CTX_MAX 32768          /* the reference's MAX_SEQ */

static void usage(FILE *f) {
  fprintf(f,
          "usage: cwen_run [MODEL] [IDS_FILE] [N_PREDICT] [OPTIONS]\n"
          "Greedy-decode token ids after a prompt of raw little-endian int32 ids, on the GPU.\n"
          "Ids go to stdout; logs go to stderr.\n"
          "\n"
          "  MODEL       GGUF model (default " DEFAULT_MODEL ")\n"
          "  IDS_FILE    int32 prompt ids; without it the prompt is the single id 248044\n"
          "  N_PREDICT   ids to generate, >= 0 (default 16; 0 only prefills)\n"
          "\n"
          "  -h, --help                 this text\n"
          "  -d, --draft-tokens N       speculate with up to N drafts per verify block (1..15);\n"
          "                             turns speculation on and overrides CWEN_SPEC_MAX_DRAFT\n"
          "                             (also --spec-draft-n-max)\n"
          "\n"
          "Environment:\n"
          "  CWEN_CTX=N              context window, 64..32768 (default 4096)\n"
          "  CWEN_REPACK=FILE        CWENR sidecar (default: MODEL with .cwenr)\n"
          "  CWEN_SERVER=1           binary-frame server on stdin/stdout\n"
          "  CWEN_SPEC=1             block speculation, same ids as greedy decode; drafts from\n"
          "                          the model's MTP block when it has one, else the n-gram map\n"
          "                          and history scan\n"
          "  CWEN_MTP=0              draft with n-grams even when the model has an MTP block\n"
          "  CWEN_NGRAM_CACHE=FILE   keep the n-gram map in FILE across runs (with CWEN_SPEC=1)\n"
          "  CWEN_SPEC_NGRAM_N=N     n-gram key length, 2..256 (16)\n"
          "  CWEN_SPEC_MAX_DRAFT=N   drafts per block, 1..15 (8)\n"
          "  CWEN_SPEC_MIN_DRAFT=N   proposals shorter than N are not verified (2)\n"
          "  CWEN_SPEC_COOLDOWN=N    plain steps after three short walks in a row (8)\n"
          "  CWEN_SPEC_DEBUG=1       one stderr line per cycle\n");
}

/* An integer environment knob: unset or empty leaves *out alone (0);
 * anything but a whole integer in [lo, hi] ends the run (exit 1). */
static int env_num(const char *name, long lo, long hi, int *out) {
  const char *e = getenv(name);
  if (!e || !e[0]) return 0;
  char *end;
  errno = 0;
  const long v = strtol(e, &end, 10);
  if (end == e || *end || errno || v < lo || v > hi) {
    fprintf(stderr, "cwen_run: %s must be an integer in [%ld, %ld], got '%s'\n", name, lo, hi, e);
    exit(1);
  }
  *out = (int)v;
  return 1;
}

/* A 0/1 environment knob; any other value ends the run (exit 1). */
static int env_flag(const char *name, int *out) {
  const char *e = getenv(name);
  if (!e || !e[0]) return 0;
  if (strcmp(e, "0") != 0 && strcmp(e, "1") != 0) {
    fprintf(stderr, "cwen_run: %s must be 0 or 1, got '%s'\n", name, e);
    exit(1);
  }
  *out = e[0] == '1';
  return 1;
}

/* A command-line integer in [lo, hi]; anything else ends the run (exit 2). */
static int arg_num(const char *what, const char *s, long lo, long hi) {
  char *end;
  errno = 0;
  const long v = strtol(s, &end, 10);
  if (end == s || *end || errno || v < lo || v > hi) {
    fprintf(stderr, "cwen_run: %s must be an integer in [%ld, %ld], got '%s'\n", what, lo, hi, s);
    exit(2);
  }
  return (int)v;
}

/* Prompt ids from a file of int32; at most cap are kept. */
static int read_ids(const char *path, int *ids, int cap, int vocab) {
  FILE *f = fopen(path, "rb");
  if (!f) {
    fprintf(stderr, "cwen_run: cannot open %s\n", path);
    return -1;
  }
  int n = 0;
  while (n < cap && fread(&ids[n], sizeof(int), 1, f) == 1) {
    if (ids[n] < 0 || ids[n] >= vocab) {
      fprintf(stderr, "cwen_run: %s: id %d at %d is outside the vocabulary [0, %d)\n", path, ids[n], n, vocab);
      fclose(f);
      return -1;
    }
    n++;
  }
  const int err = ferror(f);
  struct stat st;
  const int have_size = fstat(fileno(f), &st) == 0;
  fclose(f);
  if (err) {
    fprintf(stderr, "cwen_run: %s: read error\n", path);
    return -1;
  }
  if (have_size && st.st_size > 0) {
    if (st.st_size % 4)
      fprintf(stderr, "cwen_run: %s: %lld bytes is not a whole number of ids; the last %lld are ignored\n", path,
              (long long)st.st_size, (long long)(st.st_size % 4));
    if (st.st_size / 4 > n)
      fprintf(stderr, "cwen_run: %s: the prompt is longer than CWEN_CTX=%d; using its first %d ids\n", path, cap, n);
  }
  return n;
}

int main(int argc, char **argv) {
  const char *model_path = DEFAULT_MODEL, *ids_path = NULL;
  int n_predict = 16, draft_tokens = 0, npos = 0;
  const char *pos[3];
  for (int i = 1; i < argc; i++) {
    const char *a = argv[i];
    if (!strcmp(a, "-h") || !strcmp(a, "--help")) {
      usage(stdout);
      return 0;
    }
    if (a[0] == '-' && a[1]) {
      if (strcmp(a, "-d") && strcmp(a, "--draft-tokens") && strcmp(a, "--spec-draft-n-max")) {
        fprintf(stderr, "cwen_run: unknown option '%s'\n\n", a);
        usage(stderr);
        return 2;
      }
      if (i + 1 >= argc) {
        fprintf(stderr, "cwen_run: %s needs a value\n\n", a);
        usage(stderr);
        return 2;
      }
      draft_tokens = arg_num(a, argv[++i], 1, CWEN_BMAX - 1);
      continue;
    }
    if (npos == 3) {
      fprintf(stderr, "cwen_run: at most 3 arguments, got a fourth: '%s'\n\n", a);
      usage(stderr);
      return 2;
    }
    pos[npos++] = a;
  }
  if (npos >= 1) model_path = pos[0];
  if (npos >= 2) ids_path = pos[1];
  if (npos >= 3) n_predict = arg_num("N_PREDICT", pos[2], 0, INT_MAX);

  /* every knob is checked before the model loads */
  static const char *refused[] = {"CWEN_DUMP", "CWEN_DUMP_LAYERS", "CWEN_DUMP_LOGITS", "CWEN_ROPE_YARN",
                                  "CWEN_DFLASH"};
  for (size_t k = 0; k < sizeof refused / sizeof *refused; k++) {
    const char *e = getenv(refused[k]);
    if (e && e[0]) {
      fprintf(stderr, "cwen_run: %s is not supported here\n", refused[k]);
      return 1;
    }
  }
  int spec = 0, server = 0, want_mtp = 1, ctx_len = 4096;
  cwen_spec_cfg scfg;
  cwen_spec_default(&scfg);
  env_flag("CWEN_SPEC", &spec);
  env_num("CWEN_SPEC_NGRAM_N", 2, 256, &scfg.n_key);
  env_num("CWEN_SPEC_MAX_DRAFT", 1, CWEN_BMAX - 1, &scfg.max_draft);
  env_num("CWEN_SPEC_MIN_DRAFT", 1, scfg.max_draft, &scfg.min_draft);
  env_num("CWEN_SPEC_COOLDOWN", 0, 100000, &scfg.cooldown);
  env_flag("CWEN_SPEC_DEBUG", &scfg.debug);
  env_num("CWEN_CTX", 64, CTX_MAX, &ctx_len);
  env_flag("CWEN_SERVER", &server);
  env_flag("CWEN_MTP", &want_mtp);
  /* run.c:4045-4050: the default minimum (2) above a lowered maximum is
     refused before the model loads, not left to drop every proposal */
  if (scfg.min_draft > scfg.max_draft) {
    fprintf(stderr, "cwen_run: CWEN_SPEC_MIN_DRAFT (%d) exceeds CWEN_SPEC_MAX_DRAFT (%d)\n", scfg.min_draft,
            scfg.max_draft);
    return 1;
  }
  if (draft_tokens > 0) {   /* the flag wins over the environment */
    scfg.max_draft = draft_tokens;
    spec = 1;
    if (scfg.min_draft > scfg.max_draft) scfg.min_draft = scfg.max_draft;
  }
  const char *cache_path = getenv("CWEN_NGRAM_CACHE");
  if (cache_path && !cache_path[0]) cache_path = NULL;
  if (cache_path && !spec) {
    fprintf(stderr, "cwen_run: CWEN_NGRAM_CACHE=%s has no effect without CWEN_SPEC=1\n", cache_path);
    cache_path = NULL;
  }

  /* the model */
  cwen_gguf *g = NULL;
  if (cwen_gguf_open(model_path, &g)) {
    fprintf(stderr, "cwen_run: %s: %s\n", model_path, cwen_gguf_error());
    return 1;
  }
  char side[4096];
  if (cwen_cwenr_path(model_path, side, sizeof side) == CWEN_OK) {
    const int r = cwen_gguf_apply_cwenr(g, side, model_path);
    if (r < 0) {
      fprintf(stderr, "cwen_run: %s: %s\n", side, cwen_gguf_error());
      cwen_gguf_close(g);
      return 1;
    }
    if (r > 0) fprintf(stderr, "cwen_run: %s: %d tensors from the sidecar\n", side, r);
  }
  cwen_model_cfg cfg;
  if (cwen_model_cfg_from_gguf(g, ctx_len, &cfg)) {
    fprintf(stderr, "cwen_run: %s: %s\n", model_path, cwen_gguf_error());
    cwen_gguf_close(g);
    return 1;
  }
  cwen_ctx *ctx = NULL;
  cwen_model *m = NULL;
  int rc = cwen_ctx_create(0, &ctx);
  if (!rc) rc = cwen_model_create(ctx, &cfg, &m);
  if (!rc) rc = cwen_model_load_gguf(m, &cfg, g);
  if (rc) {
    fprintf(stderr, "cwen_run: loading %s failed (%d): %s\n", model_path, rc, cwen_gguf_error());
    cwen_gguf_close(g);
    if (m) cwen_model_free(m);
    if (ctx) cwen_ctx_destroy(ctx);
    return 1;
  }
  cwen_gguf_close(g);   /* the weights now live in HBM */
  fprintf(stderr, "cwen_run: %d layers, d_model %d, vocab %d, context %d%s\n", cfg.n_layers, cfg.d_model, cfg.vocab,
          cfg.max_ctx, cwen_model_has_mtp(m) == 1 ? ", MTP block" : "");
  scfg.mtp = want_mtp;
  cwen_ngmap *map = NULL;
  if (spec) {
    /* the n-gram map learns whichever drafter proposes (run.c:3972-3978) */
    if ((rc = cwen_ngmap_create(scfg.n_key, cfg.vocab, 0, &map))) {
      fprintf(stderr, "cwen_run: cannot allocate the n-gram map\n");
      goto out;
    }
    if (cache_path) cwen_ngmap_load(map, cache_path);
    scfg.ngmap = map;
  }

  if (server) {
    fprintf(stderr, "cwen_run: serving frames on stdin\n");
    int served = 0;
    rc = cwen_serve(m, &cfg, 0, 1, spec ? &scfg : NULL, &served);
    if (rc) fprintf(stderr, "cwen_run: serving stopped (%d) after %d frames\n", rc, served);
    goto out;
  }

  {
    int *ids = (int *)malloc(sizeof(int) * (size_t)cfg.max_ctx);
    int *out = (int *)malloc(sizeof(int) * ((size_t)n_predict + 1));
    int n_ids = 0;
    if (!ids || !out) {
      rc = CWEN_ENOMEM;
    } else if (ids_path) {
      n_ids = read_ids(ids_path, ids, cfg.max_ctx, cfg.vocab);
      if (n_ids < 0) rc = CWEN_EINVAL;
      else if (n_ids == 0) {
        fprintf(stderr, "cwen_run: %s holds no ids\n", ids_path);
        rc = CWEN_EINVAL;
      }
    } else if (DEFAULT_TOKEN < cfg.vocab) {
      ids[0] = DEFAULT_TOKEN;
      n_ids = 1;
    } else {
      fprintf(stderr, "cwen_run: the default prompt id %d is outside this model's vocabulary; give IDS_FILE\n",
              DEFAULT_TOKEN);
      rc = CWEN_EINVAL;
    }
    if (!rc) {
      fprintf(stderr, "cwen_run: prefill of %d ids\n", n_ids);
      cwen_spec_stats st;
      const int n = spec ? cwen_generate_spec(m, ids, n_ids, n_predict, &scfg, out, &st)
                         : cwen_generate_serial(m, ids, n_ids, n_predict, out, &st);
      if (n < 0) {
        fprintf(stderr, "cwen_run: decoding failed (%d)\n", n);
        rc = n;
      } else {
        for (int i = 0; i < n; i++) printf(i ? " %d" : "%d", out[i]);
        if (n > 0) putchar('\n');
        if (n < n_predict)
          fprintf(stderr, "cwen_run: the context window (CWEN_CTX=%d) filled after %d of %d ids\n", cfg.max_ctx,
                  n, n_predict);
        fprintf(stderr, "cwen_run: prefill %.3f s, decode %.3f s, %lld passes", st.prefill_s, st.decode_s,
                st.cycles);
        if (spec)
          fprintf(stderr, " (%lld with drafts: %lld kept whole, %lld cut short; %.2f drafts kept on average)",
                  st.drafted, st.full, st.rejected, st.drafted ? (double)st.kept / (double)st.drafted : 0.0);
        fputc('\n', stderr);
        if (fflush(stdout) || ferror(stdout)) {
          fprintf(stderr, "cwen_run: writing the ids to stdout failed\n");
          rc = CWEN_EIO;
        }
      }
    }
    free(ids);
    free(out);
  }

out:
  if (map) {
    if (cache_path && cwen_ngmap_used(map) > 0) cwen_ngmap_save(map, cache_path);
    cwen_ngmap_free(map);
  }
  cwen_model_free(m);
  cwen_ctx_destroy(ctx);
  return rc ? 1 : 0;
}
