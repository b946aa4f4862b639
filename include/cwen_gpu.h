/* cwen_gpu.h -- C ABI of the MI355X (gfx950) block-verify library.
 *
 * The reference engine (maci0/cwen run.c) is one C translation unit whose
 * hot path is a set of static functions over global state.  This header is
 * the drop-in boundary for that path: plain C types, plain pointers and
 * sizes, no C++ or torch types.  Each entry point names the reference
 * function it replaces (run.c:line).
 *
 * Conventions
 *   - Every function returns an int status: 0 on success, a negative
 *     CWEN_E* code on failure (the reference exit(1)s or asserts instead;
 *     the host wrapper maps a failure to that policy).
 *   - Activation and output pointers (X, Y, logits ...) are DEVICE pointers
 *     to f32 data.  X and Y rows must start 16-byte aligned and their
 *     strides (xs, ys, in floats) must be multiples of 4.
 *   - `stream` is a hipStream_t passed as void*; NULL means the default
 *     stream.  Calls are asynchronous on that stream unless stated.
 *   - One context drives one device.  A context and every weight created
 *     on it are not thread-safe, and calls on different streams that share
 *     a context must not overlap (they share the context's scratch).
 */
#ifndef CWEN_GPU_H
#define CWEN_GPU_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define CWEN_OK         0
#define CWEN_EINVAL   (-1)   /* bad argument or shape                    */
#define CWEN_EHIP     (-2)   /* a HIP runtime call failed                */
#define CWEN_ENOMEM   (-3)   /* device allocation failed                 */
#define CWEN_ETYPE    (-4)   /* weight type not supported by this call   */
#define CWEN_ESCRATCH (-5)   /* a shape exceeds the context's scratch    */
#define CWEN_ERANGE   (-6)   /* an f16 activation operand left f16's     */
                             /* range; the model's state is invalid      */
                             /* until cwen_model_reset                   */

/* Largest K (inputs) of a weight; sizes the context's f16 activation scratch. */
#define CWEN_KMAX 65536

/* ggml / CWENR weight type ids -- the same numeric ids as run.c:97-103 */
#define CWEN_T_F32      0
#define CWEN_T_Q4_0     2    /* GGUF 18-byte blocks {f16 d; u8 qs[16]}          */
#define CWEN_T_Q4_1     3    /* GGUF 20-byte blocks {f16 d; f16 m; u8 qs[16]},
                                w = n*d + m (run.c:111, 571-588, 1026-1099)     */
#define CWEN_T_Q8_0     8    /* GGUF 34-byte blocks {f16 d; i8 qs[32]}          */
#define CWEN_T_Q5_K    13    /* GGUF 176-byte super-blocks of 256 {f16 d, dmin;
                                u8 scales[12]; u8 qh[32]; u8 qs[128]}
                                (run.c:113-115, 426-429, 1100-1158)              */
#define CWEN_T_Q6_K    14    /* GGUF 210-byte super-blocks of 256                */
#define CWEN_T_Q4_0RS  101   /* CWENR split: qs[ne1][nb][16] + f16 sc[ne1][nb]   */
#define CWEN_T_Q4_0RSI 102   /* CWENR interleaved pair: qs[ne1][nb][A16|B16],
                                 f16 sc[ne1][nb][A|B]                            */

/* Largest verify block (SPEC_BMAX, run.c:192). */
#define CWEN_BMAX 16
/* Largest context (MAX_SEQ, run.c:85); cwen_model_create refuses more. */
#define CWEN_CTX_MAX 32768

typedef struct cwen_ctx cwen_ctx;        /* device, stream-independent scratch */
typedef struct cwen_weight cwen_weight;  /* one device-resident weight matrix  */

/* Library version string, e.g. "cwen-gpu 0.1 gfx950". */
const char *cwen_version(void);

/* Create a context on HIP device `device`: selects it and allocates the f16
 * activation scratch (2 x 16 x CWEN_KMAX halves).  Replaces the block scratch
 * part of alloc_state (run.c:3942-3963). */
int cwen_ctx_create(int device, cwen_ctx **out);
int cwen_ctx_destroy(cwen_ctx *ctx);

/* Upload one weight matrix given in a reference layout in HOST memory and
 * repack it on the device into the tile layout the kernels stream.
 * Types: Q4_0, Q4_0RS, Q4_0RSI, Q4_1, Q8_0 (ne0 = K a multiple of 32) and
 * Q6_K, Q5_K (K a multiple of 256), K at most CWEN_KMAX: whole blocks, as
 * the reference's row_bytes requires (run.c:1293-1306).  The device tiles
 * K in 512s; a last partial tile is padded with zero weights and the
 * activations past K are read as zeros.
 * `data`/`scales` are what the reference's Tensor.data / Tensor.scales point
 * at (run.c:132): for Q4_0RS and Q4_0RSI `scales` is the f16 scale channel,
 * for the self-contained GGUF types it is NULL.  ne0 = K (inputs), ne1 = M
 * (rows).  A Q4_0RSI blob is uploaded once and holds both sides of the pair
 * (the reference binds it as two Tensors with pair_side 0/1 over the same
 * data, run.c:3544-3579).  Replaces the CWENR/GGUF binding of a tensor
 * (run.c:3372-3466, 3544-3579); the reference uses it in place from mmap. */
int cwen_weight_upload(cwen_ctx *ctx, int type, const void *data, const void *scales,
                       int ne0, int ne1, cwen_weight **out);
int cwen_weight_free(cwen_weight *w);
/* Device bytes the kernels stream per full pass over the weight. */
int cwen_weight_info(const cwen_weight *w, int *type, int *ne0, int *ne1,
                     int *nside, size_t *stream_bytes);

/* Batched GEMV over a verify block: Y[b*ys + i] = row i of W . X[b*xs ...]
 * for b < B (1 <= B <= 16).  For a Q4_0RSI pair weight `side` picks A (0)
 * or B (1), as Tensor.pair_side does; other types require side 0.
 * Per output the arithmetic does not depend on B or on the other columns,
 * so a column computed in a block is bit-identical to the same column
 * computed alone.  Replaces gemvb (run.c:1577-1680) and, at B=1, gemv
 * (run.c:1419-1527).  X is converted to the f16 operand format in the
 * context's scratch first (a second, small launch on the same stream). */
int cwen_gemvb(cwen_ctx *ctx, const cwen_weight *W, int side,
               const float *X, int xs, float *Y, int ys, int B, void *stream);

/* Both sides of a Q4_0RSI pair in one pass over the interleaved stream:
 * YA = W_A . X, YB = W_B . X.  Replaces the two gemvb calls over one blob
 * in layer_full_blk (run.c:2724-2725) and gemv_dual_same_shape (run.c:1802). */
int cwen_gemvb_pair(cwen_ctx *ctx, const cwen_weight *W, const float *X, int xs,
                    float *YA, float *YB, int ys, int B, void *stream);

/* Gate/up pair with the SwiGLU epilogue fused: H[b*hs + i] =
 * silu(W_A[i] . X_b) * (W_B[i] . X_b).  Replaces mlp_blk's gate gemvb, up
 * gemvb and silu_mul (run.c:2677-2680). */
int cwen_gemvb_swiglu(cwen_ctx *ctx, const cwen_weight *W, const float *X, int xs,
                      float *H, int hs, int B, void *stream);

/* The block FFN, mlp_blk (run.c:2677-2683): Y_b += W_down . (silu(W_gate . X_b)
 * * (W_up . X_b)) for b < B, with Wgu a Q4_0RSI gate/up pair and Wd the down
 * projection.  The hidden activations never leave the device in f32: the
 * gate/up launch writes them straight into the down launch's operand format. */
int cwen_mlp_block(cwen_ctx *ctx, const cwen_weight *Wgu, const cwen_weight *Wd,
                   const float *X, int xs, float *Y, int ys, int B, void *stream);

/* cwen_mlp_block without any allocation and without the context's scratch:
 * the same kernels and launch decomposition, so Y is bit-identical to
 * cwen_mlp_block's.  No counterpart in the reference: it is for callers that
 * cannot allocate or touch a context's shared buffers (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Its scratch
 * (the f16 operands of X and of the hidden activations, split-K partials and
 * arrival counters) is one static device array of CWEN_STATIC_SCRATCH_BYTES
 * per GPU, held until the process ends; its address on a device is looked up
 * when the first context is created there (cwen_ctx_create), so Wgu and Wd
 * must come from a context, and that first cwen_ctx_create on a GPU must
 * return before any noalloc call runs there (it clears the array's arrival
 * counters; concurrent first creations on one GPU are serialised).  Limits: d_model and d_ffn (Wgu's ne0 and ne1)
 * at most CWEN_STATIC_KMAX, and launch decompositions whose split-K pieces
 * fit the array (every 27B-shape FFN does); beyond them it returns
 * CWEN_ESCRATCH before any launch.  Every call on a GPU shares that GPU's
 * array: calls that overlap on one GPU (any streams, any contexts) race and
 * must be serialised by the caller. */
#define CWEN_STATIC_KMAX 32768
#define CWEN_STATIC_SCRATCH_BYTES (2u * 2u * CWEN_BMAX * CWEN_STATIC_KMAX + 4u * 1048576u + 4u * 4096u)
int cwen_mlp_block_noalloc(const cwen_weight *Wgu, const cwen_weight *Wd, const float *X, int xs, float *Y,
                           int ys, int B, void *stream);

/* LM head + acceptance of one verify block, on the device.  logits_b = W . X_b
 * for b < B (W: the output head, M = vocab rows, any uploaded single-sided
 * type), then the per-column argmax -- argmax_of (run.c:2647-2668): the first
 * index of the maximum, NaN logits ignored, 0 when logit 0 is NaN -- and the
 * greedy prefix walk of generate_tokens_spec (run.c:4954-4956): k = the
 * longest prefix with argmax(row k) == drafts[k], k <= E, bonus =
 * argmax(row k).  `drafts` (device, E <= B-1 ids) is blk[1..E] of the
 * reference.  Writes the DEVICE int array res: res[0] = k, res[1] = bonus,
 * res[2 + b] = argmax(row b).  `logits` (device f32 [b*ls + v], nullable)
 * receives the logits; with NULL they never leave the chip.  Replaces
 * gemvb(&output, ...) of forward_block (run.c:2773-2777) + argmax_of + the
 * walk loop. */
int cwen_head_verify(cwen_ctx *ctx, const cwen_weight *W, const float *X, int xs, int B,
                     const int *drafts, int E, float *logits, int ls, int *res, void *stream);

/* The same argmax + walk over given device logits [b*ls + v], v < V: the
 * reference's argmax_of per row and the walk loop (run.c:2647-2668,
 * 4954-4956), res as for cwen_head_verify. */
int cwen_argmax_walk(cwen_ctx *ctx, const float *logits, int ls, int V, int B, const int *drafts,
                     int E, int *res, void *stream);

/* ---- GatedDeltaNet block verify ----
 * One linear-attention layer's recurrent state [nvh][dk][dk] (row = key
 * dimension) and conv history [C][3], C = (2*nkh + nvh)*dk, device-resident.
 * Replaces one layer's Srec/Cstate and the snapshot copies SnapS/SnapC
 * (run.c:171-172, 204, 3931-3932, 2787-2809): the history is kept after every
 * position of a block; the state is kept at the block's start and end, and
 * an accepted prefix is replayed (inside the next block) from the block's
 * saved inputs, as the reference replays a short walk (run.c:4975-4988).
 * dk must be 128 and nvh a multiple of nkh (key head of value head hv:
 * hv % nkh, run.c:2027). */
typedef struct cwen_gdn cwen_gdn;
int cwen_gdn_create(cwen_ctx *ctx, int nkh, int nvh, int dk, cwen_gdn **out);
int cwen_gdn_free(cwen_gdn *g);
/* Current state from HOST arrays (NULL = zeros).  Synchronous. */
int cwen_gdn_set_state(cwen_gdn *g, const float *S, const float *hist);
/* Copy state `pos` to HOST arrays (either may be NULL): 0 = the current
 * state, p >= 1 = the state after position p-1 of the last block (before
 * it is committed; replayed on the device).  Synchronous. */
int cwen_gdn_get_state(cwen_gdn *g, int pos, float *S, float *hist);
/* B positions of a verify block, in order, each exactly conv1d_update then
 * gdn_step of the reference (run.c:2183-2200, 2014-2180) as called by
 * layer_linear_blk (run.c:2700-2704): qkv (device, [b*qs + c]) is the raw
 * mixed q|k|v row before the conv, z [b*zs + i] the gate row, decay
 * [b*gs + hv] the log-domain decay (g = exp(decay)) and beta [b*gs + hv],
 * kw [C][4] the conv taps, wn [dk] the gated-norm weight; out [b*os + i]
 * receives the gated-RMSNorm output (nvh*dk per position).  kw, wn and out
 * must be 16-byte aligned and os a multiple of 4.  The state after any
 * position stays reachable (cwen_gdn_get_state); the current state does not
 * move until cwen_gdn_commit.  A block after an uncommitted one starts from
 * that block's start state (as if it had been committed with n = 0). */
int cwen_gdn_block(cwen_ctx *ctx, cwen_gdn *g, const float *qkv, int qs, const float *z, int zs,
                   const float *decay, const float *beta, int gs, const float *kw, const float *wn,
                   float *out, int os, int B, void *stream);
/* Accept the first n positions (0..B) of the last block: the current state
 * becomes the snapshot after position n-1 (n = 0 keeps the state from
 * before the block).  No state is copied: the whole block makes the end
 * state current; a prefix of n keeps the start state and the next block
 * replays the n positions first.  Waits for queued work.  Replaces snap_load
 * + the replaying forward_block of a short walk (run.c:4975-4988) for this
 * layer. */
int cwen_gdn_commit(cwen_gdn *g, int n);

/* ---- the block-verify model ----
 * The reference's hybrid decoder (run.c:80-92, 140-160) resident on one
 * device: layer l is full attention when l % full_interval ==
 * full_interval - 1 (run.c FULL_INT), otherwise GatedDeltaNet.  One model
 * replaces the reference's globals W[], tok_embd, output(_norm), Srec,
 * Cstate, Kcache/Vcache and the block scratch of alloc_state. */
typedef struct {
  int n_layers, d_model, d_ffn, vocab;        /* L, H, I, V                      */
  int n_head, n_kv_head, head_dim;            /* NH, NKV, HD (HD must be 256)    */
  int n_rot_pairs, n_rot;                     /* RoPE pairs (32) and NROT (64)   */
  int gdn_nkh, gdn_nvh, gdn_dk;               /* LKH, LVH, LSD (LSD must be 128) */
  int full_interval;                          /* FULL_INT                        */
  int max_ctx;                                /* KV / position capacity, 2..CWEN_CTX_MAX */
  float rope_theta, rms_eps;                  /* ROPE_THETA, RMS_EPS             */
} cwen_model_cfg;
typedef struct cwen_model cwen_model;

/* Tensor ids of cwen_model_set, named after the GGUF tensors the reference
 * binds (run.c:3367-3406). */
enum {
  CWEN_TOK_EMBD = 0,     /* token_embd.weight      Q4_0 / Q4_0RS / Q6_K, [V][H]   */
  CWEN_OUTPUT_NORM,      /* output_norm.weight     F32 [H]                        */
  CWEN_OUTPUT,           /* output.weight          any GEMV type, [V][H]          */
  CWEN_ATTN_NORM,        /* blk.l.attn_norm        F32 [H]                        */
  CWEN_POST_NORM,        /* blk.l.post_attention_norm F32 [H]                     */
  CWEN_FFN_GATE_UP,      /* ffn_gate + ffn_up      Q4_0RSI pair [I][H]            */
  CWEN_FFN_DOWN,         /* ffn_down               [H][I]                         */
  CWEN_ATTN_QKV,         /* attn_qkv (GDN)         [C][H], C = (2 LKH + LVH) LSD  */
  CWEN_ATTN_GATE,        /* attn_gate (GDN z)      [LVH*LSD][H]                   */
  CWEN_SSM_ALPHA,        /* ssm_alpha              [LVH][H]                       */
  CWEN_SSM_BETA,         /* ssm_beta               [LVH][H]                       */
  CWEN_SSM_A,            /* ssm_a                  F32 [LVH]                      */
  CWEN_SSM_DT,           /* ssm_dt.bias            F32 [LVH]                      */
  CWEN_SSM_CONV,         /* ssm_conv1d             F32 [C][4]                     */
  CWEN_SSM_NORM,         /* ssm_norm               F32 [LSD]                      */
  CWEN_SSM_OUT,          /* ssm_out                [H][LVH*LSD]                   */
  CWEN_ATTN_Q,           /* attn_q (q|gate per head) [2*NH*HD][H]                 */
  CWEN_ATTN_KV,          /* attn_k + attn_v        Q4_0RSI pair [NKV*HD][H]       */
  CWEN_ATTN_OUTPUT,      /* attn_output            [H][NH*HD]                     */
  CWEN_ATTN_Q_NORM,      /* attn_q_norm            F32 [HD]                       */
  CWEN_ATTN_K_NORM,      /* attn_k_norm            F32 [HD]                       */
  /* MTP nextn drafter (run.c:3087-3187, the GGUF's blk.N, N = n_layers):
   * these four at layer -1; its decoder block is layer n_layers, set with
   * the full-attention ids above (attn_norm, post_norm, ffn pair and down,
   * attn_q, the k/v pair, attn_output, q/k norms). */
  CWEN_NEXTN_EH_PROJ,    /* nextn.eh_proj          [H][2H] (input [e' | h'])      */
  CWEN_NEXTN_ENORM,      /* nextn.enorm            F32 [H]                        */
  CWEN_NEXTN_HNORM,      /* nextn.hnorm            F32 [H]                        */
  CWEN_NEXTN_SHEAD_NORM  /* nextn.shared_head_norm F32 [H]                        */
};

int cwen_model_create(cwen_ctx *ctx, const cwen_model_cfg *cfg, cwen_model **out);
int cwen_model_free(cwen_model *m);
/* Upload one tensor from HOST memory (layer ignored for the global ones);
 * quantized types go through cwen_weight_upload's repack. */
int cwen_model_set(cwen_model *m, int layer, int id, int type, const void *data, const void *scales,
                   int ne0, int ne1);
/* Fill every tensor with seeded random-init values generated on the device
 * (no host data): Q4_0 matrices CWENR RS / RSI with nibbles uniform and f16
 * scales |N(0,0.02)|/8, a Q6_K head (bytes uniform, d = |N(0,0.002)|), a
 * Q4_0RS embedding, F32 norms 1 + 0.1 N(0,1), conv taps 0.3 N(0,1), gate
 * parameters A = -exp(U(-1,1)), dt = 0.5 N(0,1).  For benchmarks of the
 * architecture; no reference counterpart (the reference maps a model file). */
int cwen_model_synth(cwen_model *m, unsigned long long seed);
/* Empty context: position -1, GDN states and conv histories zero (reset_state). */
int cwen_model_reset(cwen_model *m);
/* Last filled position (the reference's pos_n). */
int cwen_model_pos(const cwen_model *m);
/* Position capacity (max_ctx; the reference's g_ctx). */
int cwen_model_capacity(const cwen_model *m);
/* forward_block (run.c:2752-2779): score HOST token ids toks[0..B-1] at
 * positions pos+1..pos+B and advance by B.  With want_argmax the head runs
 * on every row and argmax_out (HOST, B ints, nullable) receives each row's
 * argmax_of; without it the head is skipped (prefill chunks).  Synchronous
 * when want_argmax.  Returns CWEN_ERANGE (after the block has run and been
 * committed) when any f16 activation operand written since the last reset
 * was out of f16's range, e.g. a residual element times its RMSNorm weight
 * of magnitude 65520 or more; without want_argmax the next synchronous call
 * reports it. */
int cwen_model_forward(cwen_model *m, const int *toks, int B, int want_argmax, int *argmax_out, void *stream);
/* One speculative verify cycle on the device: score blk[0..B-1] (blk[0] the
 * pending token, blk[1..B-1] the drafts), take the per-row argmax, walk the
 * drafts (run.c:4954-4956) and keep the accepted prefix: the state advances
 * by k+1 positions (GDN snapshots committed, KV slots past the prefix are
 * rewritten before any read).  Only k and the bonus token return to the
 * host.  B = 1 is the serial decode step (forward_ex + argmax_of).
 * Synchronous.  CWEN_ERANGE as for cwen_model_forward. */
int cwen_model_verify(cwen_model *m, const int *blk, int B, int *k, int *bonus, void *stream);
/* Copy the f32 logits of the last head pass (rows 0..rows-1) to HOST. */
int cwen_model_logits(cwen_model *m, float *host, int rows);

/* MTP nextn drafter.  1 when every MTP tensor is set.  From then on each
 * forward / verify block also commits its kept positions into the drafter's
 * own KV stream on the device (mtp_commit, run.c:3150-3163). */
int cwen_model_has_mtp(const cwen_model *m);
/* mtp_draft (run.c:3170-3187): up to n (<= CWEN_BMAX - 1) greedy drafts after
 * the last filled position, starting from the pending token pend, each step
 * the nextn block on the previous step's own output plus the shared head,
 * chained on the device; one synchronisation at the end.  Returns the count
 * (fewer near the end of the context; 0 without an MTP block or before the
 * first block), or a negative status.  The slots drafted are speculative:
 * the next block's commit rewrites them. */
int cwen_model_mtp_draft(cwen_model *m, int pend, int n, int *drafts, void *stream);
/* Copy the f32 logits of the last draft's steps (rows 0..rows-1) to HOST. */
int cwen_model_mtp_logits(cwen_model *m, float *host, int rows);

/* ---- f16 activation operands ----
 * The kernels read activations as IEEE half, row-major [B][K] with row stride
 * exactly K (2-byte elements, 16-byte aligned rows).  These entry points let a
 * caller keep activations in that format between GEMVs; no reference
 * counterpart (the reference keeps f32 everywhere and its AVX kernels read f32). */
int cwen_act_to_f16(cwen_ctx *ctx, const float *X, int xs, void *Xh, int K, int B,
                    void *stream);
/* Y (f32, nullable) = or += W . Xh; Yh (f16 [B][M], nullable) gets the f32 result
 * rounded to half (after accumulation when `accumulate` is set). */
int cwen_gemvb_f16(cwen_ctx *ctx, const cwen_weight *W, int side, const void *Xh,
                   float *Y, int ys, void *Yh, int accumulate, int B, void *stream);
/* SwiGLU pair from f16 operands; H (f32, nullable), Hh (f16 [B][M], nullable). */
int cwen_gemvb_swiglu_f16(cwen_ctx *ctx, const cwen_weight *W, const void *Xh,
                          float *H, int hs, void *Hh, int B, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* CWEN_GPU_H */
