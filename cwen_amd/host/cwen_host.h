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

/* ---- counted n-gram map (cwen_ngram.c) ----
 * The reference's NGMap (run.c:204-221, 4552-4723): a key of n_key confirmed
 * tokens -> the token that last followed it and a hit count, in an
 * open-addressed table of cap entries (a power of two; the reference's is
 * 1 << 18).  A full table evicts one least-hit entry to admit a new key.
 * The hash, probe and eviction order are the reference's, so the same
 * updates leave the same entries in the same slots. */
typedef struct cwen_ngmap cwen_ngmap;
#define CWEN_NGMAP_CAP ((size_t)1 << 18)
/* n_key in [1, 256]; vocab is recorded in saved files; cap 0 means
 * CWEN_NGMAP_CAP. */
int cwen_ngmap_create(int n_key, int vocab, size_t cap, cwen_ngmap **out);
void cwen_ngmap_free(cwen_ngmap *m);
int cwen_ngmap_n_key(const cwen_ngmap *m);
size_t cwen_ngmap_used(const cwen_ngmap *m);
/* Entries evicted so far, and how many of those evictions shifted no entry
 * back into the freed slot. */
void cwen_ngmap_evictions(const cwen_ngmap *m, size_t *evicted, size_t *in_place);
/* ng_update_key_n (run.c:4579-4593): add hits to key's count (saturating at
 * INT_MAX) and make tok its continuation, inserting the key if absent. */
void cwen_ngmap_update(cwen_ngmap *m, const int *key, int tok, int hits);
/* ng_update_range (run.c:4631-4637): every position p in [a, b) with
 * p >= n_key adds key h[p - n_key .. p) -> h[p]. */
void cwen_ngmap_update_range(cwen_ngmap *m, const int *h, int a, int b);
/* ng_draft_map (run.c:4639-4654): chained lookups from the last n_key
 * history tokens, up to max_d ids into out.  Returns the count. */
int cwen_ngmap_draft(const cwen_ngmap *m, const int *h, int hn, int *out, int max_d);
/* ng_save (run.c:4659-4678): write the NGC2 file {magic "NGC2", n_key,
 * vocab, entries} then {key, tok, count} per entry in slot order, through
 * path.tmp and a rename.  CWEN_OK or CWEN_EIO (nothing written). */
int cwen_ngmap_save(const cwen_ngmap *m, const char *path);
/* ng_load (run.c:4683-4723): merge the entries of an NGC2 file (counts add
 * to live ones).  A missing file, a short or foreign header, or another
 * n_key or vocab leaves the map as it is and returns 0; records with a token
 * outside [0, vocab) or a count below 1 are skipped; reading stops at a cut
 * record or a full map.  Returns the number of entries merged. */
int cwen_ngmap_load(cwen_ngmap *m, const char *path);
/* Copy the table (keys [cap][n_key], tokens, counts, in-use flags; any may
 * be NULL) for inspection. */
int cwen_ngmap_dump(const cwen_ngmap *m, int *keys, int *tok, int *cnt, unsigned char *used);

/* Speculation knobs (run.c:193-198 Scfg_*). */
typedef struct {
  int n_key;       /* n-gram lookup key length (16)            */
  int max_draft;   /* drafts per block, <= CWEN_BMAX - 1 (8)   */
  int min_draft;   /* a proposal shorter than this is dropped (2) */
  int cooldown;    /* plain steps after 3 short walks (8)      */
  int max_cycles;  /* stop after this many verify cycles (0: no limit) */
  int mtp;         /* draft with the model's MTP block when it has one,
                      else the n-gram drafter (1; run.c CWEN_MTP)      */
  cwen_ngmap *ngmap; /* counted n-gram map (NULL: none).  Learns from the
                      history as it grows whatever the drafter; the n-gram
                      drafter asks it first and keeps the history scan's
                      proposal when that is longer (run.c:4900, 4925-4931,
                      5003).  Its n_key must equal n_key.  It persists
                      across calls, as the reference's does across frames. */
  int *cycle_log;  /* when non-NULL, cycle c < cycle_log_cap stores its
                      draft count E at [2c] and kept drafts k at [2c + 1] */
  int cycle_log_cap;
  int debug;       /* one line per cycle on stderr (run.c CWEN_SPEC_DEBUG) */
  int *fa_streak;  /* full-accept streak carried from call to call, as the
                      reference's function-static one is (run.c:4967): when
                      non-NULL a call starts from *fa_streak and leaves its
                      final value there; NULL starts every call at 0.
                      cwen_serve carries one across its requests. */
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

/* The speculative driver of cwen_generate_spec run against a recorded
 * greedy stream instead of a model, on the host: stream[0 .. n_stream) is
 * the prompt (its first n_prompt ids) followed by what greedy decode emits
 * after it, and a verify block keeps each draft while it equals the stream's
 * next id.  The drafts, the draft sizing, the cycle count and the output are
 * those the driver produces on a model whose greedy decode is that stream;
 * max_ctx plays the model's capacity.  The n-gram drafter is used (cfg->mtp
 * is ignored).  CWEN_EINVAL when a block reaches past the stream. */
int cwen_spec_replay(const int *stream, int n_stream, int n_prompt, int n_gen, int max_ctx,
                     const cwen_spec_cfg *cfg, int *out, cwen_spec_stats *stats);

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
 * back to token_embd.weight (tied).  The embedding is Q4_0 or Q6_K.  Tensors a
 * sidecar rebound are uploaded from its views (an interleaved pair as it
 * is).  When blk.<n_layers>.nextn.eh_proj.weight is present the MTP nextn
 * block is bound too, every part required (run.c:3409-3464). */
int cwen_model_load_gguf(cwen_model *m, const cwen_model_cfg *cfg, const cwen_gguf *g);
/* The geometry cwen_model_load_gguf needs, read from g's tensor shapes:
 * d_model and vocab from token_embd, the layer count up to the MTP block,
 * the full-attention interval from the first layer with attn_q, head sizes
 * and counts from the attention and GatedDeltaNet matrices.  RoPE (64
 * dimensions, theta 1e7) and the norm epsilon 1e-6 are the reference's
 * compiled values (run.c:83-91), which the shapes do not record.  max_ctx is
 * the caller's.  CWEN_EINVAL when a tensor is missing or a size does not
 * divide into heads (cwen_gguf_error names it). */
int cwen_model_cfg_from_gguf(const cwen_gguf *g, int max_ctx, cwen_model_cfg *cfg);

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
