/* cwen_host.h -- host-side decode drivers over the cwen_gpu C ABI.
 *
 * Plain C: the greedy serial decode loop and the speculative block-verify
 * loop of the reference engine (maci0/cwen run.c generate_tokens 5027-5045,
 * generate_tokens_spec 4882-5025), with its history-scan n-gram drafter
 * (ngram_draft 4533-4549).  Every forward pass runs on the device through
 * cwen_model_forward / cwen_model_verify; per cycle only token ids go down
 * and (k, bonus) comes back.
 */
#ifndef CWEN_HOST_H
#define CWEN_HOST_H
#include "cwen_gpu.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Speculation knobs (run.c:193-198 Scfg_*). */
typedef struct {
  int n_key;       /* n-gram lookup key length (16)            */
  int max_draft;   /* drafts per block, <= CWEN_BMAX - 1 (8)   */
  int min_draft;   /* a proposal shorter than this is dropped (2) */
  int cooldown;    /* plain steps after 3 short walks (8)      */
  int max_cycles;  /* stop after this many verify cycles (0: no limit) */
  int mtp;         /* draft with the model's MTP block when it has one,
                      else the n-gram drafter (1; run.c CWEN_MTP)      */
} cwen_spec_cfg;

typedef struct {
  long long cycles, drafted, full, rejected, kept;  /* run.c:4891 counters; cycles = passes */
  int prefill_tokens;
  double prefill_s, decode_s;                       /* wall time of the two phases */
} cwen_spec_stats;

/* Default knobs of the reference. */
void cwen_spec_default(cwen_spec_cfg *cfg);

/* ngram_draft (run.c:4533-4549): the continuation of the most recent earlier
 * occurrence of the last n_key history tokens, preferring an older match
 * with a longer continuation; up to max_d ids into out.  Returns the count. */
int cwen_ngram_draft(const int *h, int hn, int *out, int n_key, int max_d);

/* prefill_forward (run.c:4823-4857): reset the model, score the prompt in
 * blocks of up to 16 positions and return the argmax after the last prompt
 * token in *next. */
int cwen_prefill(cwen_model *m, const int *prompt, int n_prompt, int *next);

/* generate_tokens (run.c:5027-5045): prefill, then n_gen greedy tokens, one
 * position per forward pass.  Returns the number of tokens written to out
 * (fewer than n_gen only when the context fills), or a negative status. */
int cwen_generate_serial(cwen_model *m, const int *prompt, int n_prompt, int n_gen, int *out,
                         cwen_spec_stats *stats);

/* generate_tokens_spec (run.c:4882-5025): the same token stream as
 * cwen_generate_serial, produced by block-verify cycles; the drafts come
 * from the model's MTP block (cwen_model_mtp_draft) when cfg->mtp is set and
 * the model has one, else from the n-gram drafter. */
int cwen_generate_spec(cwen_model *m, const int *prompt, int n_prompt, int n_gen, const cwen_spec_cfg *cfg,
                       int *out, cwen_spec_stats *stats);

/* ---- GGUF weights (cwen_gguf.c) ----
 * load_gguf (run.c:3188-3301): map a GGUF v2/v3 file read-only and read its
 * tensor table with the reference's bounds checks.  Malformed input returns
 * CWEN_EINVAL; cwen_gguf_error names the reason. */
typedef struct cwen_gguf cwen_gguf;
int cwen_gguf_open(const char *path, cwen_gguf **out);
void cwen_gguf_close(cwen_gguf *g);
const char *cwen_gguf_error(void);
/* Tensor count; tensor i's name, GGUF type id, ne0, ne1 and data pointer
 * (inside the mapping; any out pointer may be NULL); index of a name or -1
 * (run.c find_tensor). */
int cwen_gguf_count(const cwen_gguf *g);
int cwen_gguf_tensor(const cwen_gguf *g, int i, const char **name, int *type, int *ne0, int *ne1,
                     const void **data);
int cwen_gguf_find(const cwen_gguf *g, const char *name);
/* Tensor i's f16 scales and pair side once a CWENR sidecar rebound it
 * (type CWEN_T_Q4_0RS / CWEN_T_Q4_0RSI); NULL and 0 for GGUF types. */
int cwen_gguf_tensor_scales(const cwen_gguf *g, int i, const void **scales, int *side);

/* ---- CWENR sidecar (cwen_gguf.c) ----
 * cwenr_path_for (run.c:3310-3325): $CWEN_REPACK if set, else the GGUF
 * path with ".gguf" replaced by (or, without it, followed by) ".cwenr".
 * CWEN_EINVAL when the result does not fit in cap bytes. */
int cwen_cwenr_path(const char *gguf, char *out, size_t cap);
/* load_cwenr (run.c:3486-3643): map the sidecar at path and rebind the Q4_0
 * tensors of g it holds (same name and shape) to its split (v3, v4 solo) or
 * interleaved (v4 pairs) views; v2's packed blocks are split on the host.
 * Returns the number of tensors rebound (>= 1); 0 when there is no file or
 * no entry applies; CWEN_EINVAL for a bad magic or header, or a stamped
 * sidecar whose source size (src_gguf's, in 4 KiB pages) no longer matches.
 * Below 1, g is unchanged and the reason is in cwen_gguf_error.  The views
 * live until cwen_gguf_close. */
int cwen_gguf_apply_cwenr(cwen_gguf *g, const char *path, const char *src_gguf);
/* IEEE f32 -> f16 bits, rounded to nearest even (the v2 scale split,
 * run.c:443-470). */
uint16_t cwen_f32_to_f16(float x);
/* rebind_layers_from_tens (run.c:3366-3406): upload every tensor the verify
 * path uses, by the reference's names, with its shape pins, into model m
 * created with cfg.  ffn_gate/ffn_up and attn_k/attn_v (GGUF Q4_0) are
 * interleaved on the host into the device's pair form; output.weight falls
 * back to token_embd.weight (tied).  The embedding must be Q4_0.  Tensors a
 * sidecar rebound are uploaded from its views (an interleaved pair as it
 * is).  When blk.<n_layers>.nextn.eh_proj.weight is present the MTP nextn
 * block is bound too, every part required (run.c:3409-3464). */
int cwen_model_load_gguf(cwen_model *m, const cwen_model_cfg *cfg, const cwen_gguf *g);

/* ---- binary-frame server (cwen_serve.c) ---- */
#define CWEN_EIO (-7) /* a reply could not be written */
#define CWEN_FRAME_REJECTED 0
#define CWEN_FRAME_OK 1
#define CWEN_FRAME_END 2
/* server_read_frame (run.c:4212-4232): read one request
 * <u32 n_prompt><u32 n_gen><n_prompt x i32> from fd, unbuffered.  Returns
 * CWEN_FRAME_OK for a valid frame (counts stored, tokens filled),
 * CWEN_FRAME_REJECTED for a rejected one (a count outside [1, max_ctx]: its
 * payload drained; a token outside [0, vocab)), CWEN_FRAME_END at the end of
 * the stream (0xffffffff in a header word, or a frame cut short; the
 * reference's -1), CWEN_EINVAL for bad arguments.  tokens holds max_ctx ids. */
int cwen_read_frame(int fd, int *tokens, int max_ctx, int vocab, uint32_t *n_prompt, uint32_t *n_gen);
/* server_loop (run.c:5063-5078): answer every frame read from fd_in on
 * fd_out -- a rejected frame with the u32 0, a valid one with
 * <u32 n_out><n_out x i32> from a fresh decode of its prompt: greedy serial
 * decode when spec is NULL, else block-verify speculation with spec's knobs
 * (the same tokens).  cfg is the model's.  Returns CWEN_OK at the end of the
 * stream, CWEN_EIO when a reply cannot be written, or a decode's negative
 * status; *n_served (may be NULL) counts the valid frames answered.  The
 * descriptors stay open. */
int cwen_serve(cwen_model *m, const cwen_model_cfg *cfg, int fd_in, int fd_out, const cwen_spec_cfg *spec,
               int *n_served);

#ifdef __cplusplus
}
#endif
#endif /* CWEN_HOST_H */
