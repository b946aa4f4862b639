/* cwen oracle: a scalar CPU restatement of the reference engine's
 * speculative block-verify hot path (maci0/cwen run.c).
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product library links, loads or
 * calls this code: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only to check results against.
 *
 * Every function follows the reference's *scalar* (non-SIMD) code path
 * statement by statement and in the same f32 evaluation order, so that a
 * build of run.c with SIMD disabled (oracle/_ref, scalar variant) is
 * bit-identical to it.  Citations are run.c:line in the reference tree.
 *
 * Layout conventions are the reference's:
 *   Q4_0 (GGUF)  18-byte blocks {f16 d; u8 qs[16]}, w[j]=(lo(qs[j])-8)*d,
 *                w[j+16]=(hi(qs[j])-8)*d                       run.c:109,432
 *   Q4_0RS       qs[ne1][nb][16] + f16 sc[ne1][nb]              run.c:99,1464
 *   Q4_0RSI      qs[ne1][nb][A16|B16] + f16 sc[ne1][nb][A|B]    run.c:100,1469
 *   Q8_0         34-byte blocks {f16 d; i8 qs[32]}              run.c:106
 *   Q6_K         210-byte super-blocks {ql[128] qh[64] sc[16] f16 d}  run.c:115
 */
#ifndef CWEN_ORACLE_H
#define CWEN_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml / CWENR type ids (run.c:97-103) */
enum { ORC_F32 = 0, ORC_Q4_0 = 2, ORC_Q4_1 = 3, ORC_Q8_0 = 8, ORC_Q5_K = 13, ORC_Q6_K = 14,
       ORC_Q4_0RS = 101, ORC_Q4_0RSI = 102 };

/* Mirrors the reference Tensor (run.c:132): ne0 = K (inputs), ne1 = M (rows). */
typedef struct {
  const void *data;
  const void *scales;
  int type;
  int ne0, ne1;
  int pair_side;
} orc_tensor;

float    orc_f16_to_f32(uint16_t h);                 /* run.c:293-299 */
uint16_t orc_f32_to_f16(float x);                    /* run.c:447-470 */

float orc_dot_q4_0(const uint8_t *blk18, const float *y, int K);          /* run.c:1009-1025 */
float orc_dot_q4_rs(const uint8_t *qs, const uint16_t *sc, const float *y, int K); /* run.c:753-767 */
float orc_dot_q4_rsi(const uint8_t *qs, const uint16_t *sc, int side,
                     const float *y, int K);                                 /* run.c:942-975 */
float orc_dot_q4_1(const uint8_t *blk20, const float *y, int K);            /* run.c:1087-1096 */
float orc_dot_q8_0(const uint8_t *blk34, const float *y, int K);            /* run.c:1248-1274 */
float orc_dot_q5_K(const uint8_t *blk176, const float *y, int K);           /* run.c:1142-1156 */
float orc_dot_q6_K(const uint8_t *blk210, const float *y, int K);           /* run.c:1226-1245 */

/* Y[b*ys+i] = row i of W . X[b*xs ..], b < B (run.c:1577-1680). */
int  orc_gemvb(const orc_tensor *W, const float *X, int xs, float *Y, int ys, int B);

float orc_silu(float x);                                  /* run.c:378-384 */
void  orc_silu_mul(float *a, const float *b, int n);      /* run.c:1697-1713 */
void  orc_rmsnorm(float *o, const float *x, const float *w, int n);  /* run.c:346-368 */
void  orc_l2norm_rows(float *x, int rows, int dim);       /* run.c:401-423 */
void  orc_residual_add(float *dst, const float *d, int n);/* run.c:1683-1695 */
float orc_softplus(float x);                              /* run.c:392 */
float orc_sigmoid(float x);                               /* run.c:393-399 */

/* Depthwise causal conv + SiLU over C channels (run.c:2183-2200).
 * hist: [C][3] oldest first; kw: [C][4]. */
void orc_conv1d_update(float *qkv, float *hist, const float *kw, int C);

/* One GatedDeltaNet step (run.c:2014-2180).
 * S: [nvh][dk][dk] (row = k-dim i, col = v-dim j), qkv: [q nkh*dk | k nkh*dk | v nvh*dk]
 * (q and k are L2-normalised in place), z: [nvh*dk], decay/beta: [nvh],
 * wn: [dk] shared gated-norm weight, out: [nvh*dk]. */
void orc_gdn_step(float *S, float *qkv, const float *z, const float *decay,
                  const float *beta, const float *wn, float *out,
                  int nkh, int nvh, int dk);

/* First index of the maximum, strict '>' scan from index 0 (run.c:2647-2668). */
int orc_argmax(const float *lg, int V);

/* Greedy prefix walk (run.c:4954-4956): logits rows [E+1][V] (row stride ls),
 * drafts d[0..E-1] compared against rows 0..E-1.  Returns k, writes bonus. */
int orc_walk(const float *logits, long ls, int V, const int *drafts, int E, int *bonus);

/* Prompt-lookup drafter (run.c:4533-4549). */
int orc_ngram_draft(const int *h, int hn, int *out, int n_key, int max_d);

/* run.c:1849-1887 embed_token_to for Q4_0 (18-byte blocks, scales NULL),
 * Q4_0RS rows ((n - 8) * d) and Q6_K rows (run.c:1829-1848, scales NULL):
 * dst[H] of row `token`. */
void orc_embed(const uint8_t *qs, const uint16_t *sc, int type, int token, int H, float *dst);

/* run.c:1903-1948 rope_tables + rope_apply without YaRN: on each of n_heads
 * heads of hd floats, pairs (2i, 2i+1), i < npairs, rotate by
 * pos / theta^(i/nrot). */
void orc_rope_apply(float *q, int n_heads, int hd, int pos, int npairs, int nrot, float theta);

/* run.c:2362-2409 attention_heads_kv, scalar branch: nh query heads of hd
 * against nkv key/value heads (GQA group nh/nkv), keys and values
 * [t][nkv][hd] for t in t0..pos, scale 1/sqrt(hd), softmax, output gated by
 * sigmoid(gate).  out[nh*hd]. */
void orc_attention(const float *K, const float *V, int nkv, int hd, int t0, int pos, const float *q,
                   const float *gate, int nh, float *out);

#ifdef __cplusplus
}
#endif
#endif
