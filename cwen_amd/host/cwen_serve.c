/* cwen_serve.c -- the reference's binary-frame server over the cwen_gpu C ABI.
 *
 * Requests are <u32 n_prompt><u32 n_gen><n_prompt x i32>, little-endian;
 * 0xffffffff in a header word, or a stream that ends inside a frame, closes
 * the server (run.c:4177-4232).  A frame with a count outside [1, max_ctx]
 * is rejected after its declared payload is drained, so the next header
 * stays aligned; a frame with a token id outside [0, vocab) is rejected
 * after its payload is read.  A rejected frame is answered with the u32 0,
 * a valid one with <u32 n_out><n_out x i32> from a fresh decode of its
 * prompt (server_loop, run.c:5063-5078).
 */
#define _GNU_SOURCE
#include "cwen_host.h"

#include <stdio.h>
#include <stdlib.h>
#include <unistd.h>

#define END_WORD 0xffffffffu

/* Skip `words` 4-byte words of a rejected frame's payload.  Pipes cannot
 * seek, so the bytes are read into a scratch block and dropped; a stream that
 * ends early is left at its end, where the next header read sees it. */
static void skip_payload(FILE *f, uint64_t words) {
  unsigned char scratch[4096];
  uint64_t left = words * 4u;
  while (left > 0) {
    const size_t want = left < sizeof scratch ? (size_t)left : sizeof scratch;
    const size_t got = fread(scratch, 1, want, f);
    if (got != want) break;
    left -= got;
  }
}

/* One request frame; see cwen_read_frame in cwen_host.h for the outcomes. */
static int read_frame(FILE *in, int *tokens, int max_ctx, int vocab, uint32_t *np, uint32_t *ng) {
  uint32_t hdr[2];
  if (fread(hdr, sizeof hdr[0], 2, in) != 2 || hdr[0] == END_WORD || hdr[1] == END_WORD)
    return CWEN_FRAME_END;                        /* closed stream or the end marker */
  const uint32_t lim = (uint32_t)max_ctx;
  const int counts_ok = hdr[0] >= 1 && hdr[0] <= lim && hdr[1] >= 1 && hdr[1] <= lim;
  if (!counts_ok) {
    fprintf(stderr, "cwen_serve: rejecting a frame of %u prompt / %u new tokens (each must be 1..%d)\n",
            hdr[0], hdr[1], max_ctx);
    skip_payload(in, hdr[0]);                     /* keep the next header aligned */
    return CWEN_FRAME_REJECTED;
  }
  if (fread(tokens, sizeof tokens[0], hdr[0], in) != hdr[0]) return CWEN_FRAME_END;  /* cut short */
  for (uint32_t i = 0; i < hdr[0]; i++) {
    if (tokens[i] >= 0 && tokens[i] < vocab) continue;
    fprintf(stderr, "cwen_serve: rejecting a frame whose token %u is %d (vocabulary 0..%d)\n", i, tokens[i],
            vocab - 1);
    return CWEN_FRAME_REJECTED;
  }
  *np = hdr[0];
  *ng = hdr[1];
  return CWEN_FRAME_OK;
}

/* Buffered stdio over a duplicate of fd, so the caller's descriptor stays
 * open after fclose. */
static FILE *open_dup(int fd, const char *mode) {
  const int d = dup(fd);
  if (d < 0) return NULL;
  FILE *f = fdopen(d, mode);
  if (!f) close(d);
  return f;
}

int cwen_read_frame(int fd, int *tokens, int max_ctx, int vocab, uint32_t *n_prompt, uint32_t *n_gen) {
  if (!tokens || !n_prompt || !n_gen || max_ctx < 1 || vocab < 1) return CWEN_EINVAL;
  /* unbuffered, so nothing past this frame is taken from fd */
  FILE *in = open_dup(fd, "rb");
  if (!in) return CWEN_EINVAL;
  setvbuf(in, NULL, _IONBF, 0);
  const int r = read_frame(in, tokens, max_ctx, vocab, n_prompt, n_gen);
  fclose(in);
  return r;
}

static int put_reply(FILE *out, const int *tok, uint32_t n) {
  if (fwrite(&n, 4, 1, out) != 1 || (n && fwrite(tok, 4, n, out) != n) || fflush(out)) {
    fprintf(stderr, "cwen_serve: a reply could not be written\n");
    return CWEN_EIO;
  }
  return CWEN_OK;
}

int cwen_serve(cwen_model *m, const cwen_model_cfg *cfg, int fd_in, int fd_out, const cwen_spec_cfg *spec,
               int *n_served) {
  if (!m || !cfg || cfg->max_ctx < 1) return CWEN_EINVAL;
  int *tokens = (int *)malloc((size_t)cfg->max_ctx * sizeof(int));
  int *out = (int *)malloc((size_t)cfg->max_ctx * sizeof(int));
  FILE *in = open_dup(fd_in, "rb"), *wr = open_dup(fd_out, "wb");
  int rc = (!tokens || !out) ? CWEN_ENOMEM : (!in || !wr) ? CWEN_EINVAL : CWEN_OK;
  int served = 0;
  /* the full-accept streak lives across requests, as run.c's function-static
   * one does (run.c:4967), unless the caller carries its own */
  cwen_spec_cfg sc;
  int fa_carry = 0;
  if (spec) {
    sc = *spec;
    if (!sc.fa_streak) sc.fa_streak = &fa_carry;
  }
  while (!rc) {
    uint32_t np = 0, ng = 0;
    const int r = read_frame(in, tokens, cfg->max_ctx, cfg->vocab, &np, &ng);
    if (r == CWEN_FRAME_END) break;  /* a clean close */
    if (r == CWEN_FRAME_REJECTED) {
      rc = put_reply(wr, NULL, 0);
      continue;
    }
    const int n = spec ? cwen_generate_spec(m, tokens, (int)np, (int)ng, &sc, out, NULL)
                       : cwen_generate_serial(m, tokens, (int)np, (int)ng, out, NULL);
    if (n < 0) {
      rc = n;
      break;
    }
    rc = put_reply(wr, out, (uint32_t)n);
    served++;
  }
  if (in) fclose(in);
  if (wr) fclose(wr);
  free(tokens);
  free(out);
  if (n_served) *n_served = served;
  return rc;
}
