// C ABI of the block-verify model: the hybrid GatedDeltaNet / gated-attention
// decoder of the reference engine (run.c) resident on one device, with the
// forward_block / verify / serial-step entry points.
//
// Reference: forward_block 2752-2779, layer_linear_blk 2685-2712,
// layer_full_blk 2714-2745, mlp_blk 2677-2683, forward_ex 2594-2645,
// prefill_forward 4823-4857, the verify walk of generate_tokens_spec
// 4950-5009.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include <new>

#include "cwen_internal.h"

namespace {

// The GEMVs that read the same normalised input are one row-concatenated
// weight, one launch: GDN layers [qkv | gate | alpha | beta] (lin_in), full
// layers [wq | wk | wv] (att_in; the k/v pair's two sides become two row
// blocks).  `parts` records which row blocks have been uploaded.
struct Layer {
  int linear;
  float *attn_norm = nullptr, *post_norm = nullptr;
  cwen_weight *ffn_gu = nullptr, *ffn_down = nullptr;
  cwen_weight *lin_in = nullptr, *ssm_out = nullptr;
  float *ssm_a = nullptr, *ssm_dt = nullptr, *ssm_conv = nullptr, *ssm_norm = nullptr;
  cwen_gdn *gdn = nullptr;
  cwen_weight *att_in = nullptr, *wo = nullptr;
  float *q_norm = nullptr, *k_norm = nullptr;
  float *K = nullptr, *V = nullptr;
  unsigned parts = 0;
};

template <class T> int dmalloc(T **p, size_t n) {
  return hipMalloc((void **)p, n * sizeof(T)) == hipSuccess ? CWEN_OK : CWEN_ENOMEM;
}

}  // namespace

struct cwen_model {
  cwen_ctx *ctx;
  cwen_model_cfg cfg;
  Layer *L;
  uint8_t *emb_qs = nullptr;
  uint16_t *emb_sc = nullptr;
  int emb_type = -1;
  float *out_norm = nullptr;
  cwen_weight *head = nullptr;
  int pos = -1;                  // last filled slot (host copy)
  int *ctl = nullptr;            // device: [0] last filled slot, [1..4] the GDN layers' control word
  // With CWEN_GRAPHS=1 each (mode, B) block is captured once into a graph
  // per attention band and replayed: the launch shapes depend on (mode, B),
  // the weight shapes and attention_wide(pos + B) only, the position and
  // ring slot are read from ctl on the device.
  // Off by default: replay measured no faster than eager launches (the
  // per-kernel cost is on the device side).
  int use_graphs = 0;
  hipStream_t cap = nullptr;     // capture stream
  hipGraphExec_t gexec[3][2][CWEN_BMAX] = {};  // [mode][attention_wide][B - 1]
  int *htok = nullptr;           // pinned token staging [BMAX]
  hipEvent_t tok_ev = nullptr;   // the last staging copy has been issued past this
  // device scratch
  int *toks = nullptr;
  int *res = nullptr;            // [0] range flag copy, [1] k, [2] bonus, [3..] argmax per column
  float *X = nullptr;            // residual stream [BMAX][H]
  float *ssq = nullptr;          // partial sums of squares of X [BMAX][CWEN_MAX_PARTS]
  _Float16 *xh = nullptr;        // f16 operand x * w of the next RMSNorm [BMAX][H]
  float *lin = nullptr;           // GDN layer input GEMV out [BMAX][lin_rows]
  _Float16 *gh = nullptr;        // GDN output f16 [BMAX][nvh*dk]
  float *att = nullptr;           // attention input GEMV out [BMAX][att_rows]
  float *qbuf = nullptr, *apart = nullptr;
  _Float16 *yh = nullptr;        // attention output f16 [BMAX][NH*HD]
  _Float16 *hh = nullptr;        // FFN hidden f16 [BMAX][I]
  float *logits = nullptr;       // [BMAX][V]
  int *hres = nullptr;           // pinned host copy of res
  // MTP nextn drafter (blk.N after the N decoder layers; its decoder block
  // is L[n_layers]).  Its KV stream starts at slot 1: slot s lives at index
  // s - 1, *mctl is the last index filled.  Every block commits its
  // positions into the stream after the target's head, pairing position
  // p's token with the target's final residual at p - 1 (hprev holds the
  // previous block's last committed row).
  cwen_weight *mtp_eh = nullptr;                       // nextn.eh_proj [H][2H]
  float *mtp_enorm = nullptr, *mtp_hnorm = nullptr, *mtp_shn = nullptr;
  int mtp_hpos = -1;                                   // hprev holds position mtp_hpos (host copy)
  int *mctl = nullptr;                                 // [0] last filled index of the MTP stream
  int *mres = nullptr;                                 // per draft step t: [4t] k, [4t+1] token, [4t+2] argmax
  int *hmres = nullptr;                                // pinned host copy of mres
  float *hprev = nullptr;                              // [H] target residual of position mtp_hpos
  float *hin = nullptr, *e2 = nullptr, *X2 = nullptr;  // [BMAX][H]
  _Float16 *cat = nullptr, *xh2 = nullptr;             // [BMAX][2H], [BMAX][H]
  float *ssq2 = nullptr;                               // [BMAX][CWEN_MAX_PARTS]
  float *mlogits = nullptr;                            // [BMAX][V] logits of the draft steps
};

namespace {

bool is_full(const cwen_model_cfg &c, int l) { return l % c.full_interval == c.full_interval - 1; }

// rocprofv3 runs its tool with ROCPROF* variables in the environment.
bool under_profiler() {
  for (char **e = environ; e && *e; ++e)
    if (strncmp(*e, "ROCPROF", 7) == 0) return true;
  return false;
}

// Row layout of the concatenated input weights.
// Row blocks start on 16-row groups (a block shorter than a multiple of 16
// is followed by zero rows).
struct Rows {
  int C, Zh, nvh, lin;        // lin_in: qkv C | gate Zh | alpha nvh | beta nvh
  int o_alpha, o_beta;        // row offsets of the alpha and beta blocks
  int Qo2, Ko, att;           // att_in: wq 2*Qo | wk Ko | wv Ko
};
Rows rows_of(const cwen_model_cfg &c) {
  Rows r;
  r.C = (2 * c.gdn_nkh + c.gdn_nvh) * 128;
  r.Zh = c.gdn_nvh * 128;
  r.nvh = c.gdn_nvh;
  r.o_alpha = r.C + r.Zh;
  r.o_beta = r.o_alpha + (r.nvh + Q4_ROWS - 1) / Q4_ROWS * Q4_ROWS;
  r.lin = r.o_beta + r.nvh;
  r.Qo2 = 2 * c.n_head * c.head_dim;
  r.Ko = c.n_kv_head * c.head_dim;
  r.att = r.Qo2 + 2 * r.Ko;
  return r;
}

int check_cfg(const cwen_model_cfg *c) {
  if (!c || c->n_layers <= 0 || c->d_model <= 0 || c->d_ffn <= 0 || c->vocab <= 0) return CWEN_EINVAL;
  if (c->d_model % Q4_K_ALIGN || c->d_ffn % Q4_K_ALIGN) return CWEN_EINVAL;
  if (c->d_model > 8192) return CWEN_EINVAL;  // <= CWEN_MAX_PARTS row-tile partials of the residual's sum of squares
  if (c->head_dim != 256 || c->n_head <= 0 || c->n_kv_head <= 0 || c->n_head % c->n_kv_head) return CWEN_EINVAL;
  // Attention takes every block size up to CWEN_BMAX: refused here rather than
  // part-way through a block.
  if (c->n_head / c->n_kv_head > attention_max_group()) return CWEN_EINVAL;
  if ((c->n_head * c->head_dim) % Q4_K_ALIGN) return CWEN_EINVAL;
  if (c->gdn_dk != 128 || c->gdn_nkh <= 0 || c->gdn_nvh % c->gdn_nkh || (c->gdn_nvh * 128) % Q4_K_ALIGN)
    return CWEN_EINVAL;
  if (c->full_interval <= 0 || c->max_ctx < 2 || c->max_ctx > CWEN_CTX_MAX || c->n_rot_pairs < 0 ||
      2 * c->n_rot_pairs > c->head_dim)
    return CWEN_EINVAL;
  return CWEN_OK;
}

int upload_f32(const void *data, size_t n, float **out) {
  if (*out) (void)hipFree(*out);
  *out = nullptr;
  if (dmalloc(out, n)) return CWEN_ENOMEM;
  CWEN_HIP_TRY(hipMemcpy(*out, data, n * sizeof(float), hipMemcpyHostToDevice));
  return CWEN_OK;
}

int upload_w(cwen_model *m, int type, const void *data, const void *scales, int ne0, int ne1,
             int want_ne0, int want_ne1, cwen_weight **out) {
  if (ne0 != want_ne0 || ne1 != want_ne1) return CWEN_EINVAL;
  if (*out) cwen_weight_free(*out);
  *out = nullptr;
  return cwen_weight_upload(m->ctx, type, data, scales, ne0, ne1, out);
}

// Device commit of a block of nmax positions: keep n, or walk[0] + 1
// (accepted drafts + bonus) when walk is given, clamped to [1, nmax].  The
// position and the GDN ring slot advance by n; the GDN base state and replay
// count follow gdn_commit_host's rule.  The sticky range flag ctl[5] is
// copied to *flag_out, next to the walk's result, for the host to read.
__global__ void advance_kernel(int *ctl, const int *walk, int n, int nmax, int nslot, int *flag_out) {
  *flag_out = ctl[5];
  if (walk) n = walk[0] + 1;
  n = n < 1 ? 1 : (n > nmax ? nmax : n);
  ctl[0] += n;
  ctl[1] = (ctl[1] + n) % nslot;
  if (n == nmax) {
    ctl[2] ^= 1;
    ctl[3] = 0;
  } else {
    ctl[3] = n;
  }
  ctl[4] ^= 1;
}

enum { MODE_FWD = 0, MODE_FWD_HEAD = 1, MODE_VERIFY = 2 };

// One block over the tokens in m->toks: positions ctl[0]+1 .. ctl[0]+B, then
// the device commit.  MODE_FWD_HEAD adds the head and per-position argmax,
// MODE_VERIFY the head and the walk over drafts toks[1..B-1] (kept = k + 1).
// The nextn input of one row (mtp_step, run.c:3099-3102): the embedding e
// and the predecessor hidden h = rmsnorm(hsrc, wpre) (the target's
// output_norm, or the MTP block's own shared_head_norm while drafting), each
// RMS-normalised with its own weight, as the f16 operand [e' | h'] of
// eh_proj.  One workgroup per row.
__global__ __launch_bounds__(256) void mtp_cat_kernel(const float *e, const float *hsrc, int hs, const float *wpre,
                                                      const float *enorm, const float *hnorm, int H, float eps,
                                                      _Float16 *cat, int *rflag) {
  __shared__ float red[3][8];
  const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const float *er = e + (size_t)r * H, *hr = hsrc + (size_t)r * hs;
  float se = 0.f, sh = 0.f;
  for (int i = tid; i < H; i += 256) {
    se += er[i] * er[i];
    sh += hr[i] * hr[i];
  }
  for (int o = 32; o; o >>= 1) {
    se += __shfl_xor(se, o);
    sh += __shfl_xor(sh, o);
  }
  if (lane == 0) { red[0][wv] = se; red[1][wv] = sh; }
  __syncthreads();
  se = red[0][0] + red[0][1] + red[0][2] + red[0][3];
  sh = red[1][0] + red[1][1] + red[1][2] + red[1][3];
  const float re = 1.f / sqrtf(se / H + eps), rh = 1.f / sqrtf(sh / H + eps);
  float s1 = 0.f;
  for (int i = tid; i < H; i += 256) {
    const float h1 = hr[i] * rh * wpre[i];
    s1 += h1 * h1;
  }
  for (int o = 32; o; o >>= 1) s1 += __shfl_xor(s1, o);
  if (lane == 0) red[2][wv] = s1;
  __syncthreads();
  s1 = red[2][0] + red[2][1] + red[2][2] + red[2][3];
  const float r1 = 1.f / sqrtf(s1 / H + eps);
  _Float16 *out = cat + (size_t)r * 2 * H;
  bool bad = false;
  for (int i = tid; i < H; i += 256) {
    const _Float16 a = (_Float16)(er[i] * re * enorm[i]);
    const _Float16 b = (_Float16)(hr[i] * rh * wpre[i] * r1 * hnorm[i]);
    out[i] = a;
    out[H + i] = b;
    bad |= f16_bad(a);
    bad |= f16_bad(b);
  }
  if (bad) raise_flag(rflag);
}

// *p = v, or *p += v (add): the MTP stream's fill mark, set on the device so
// that it stays ordered with the launches around it.
__global__ void mtp_ctl_kernel(int *p, int v, int add) { p[0] = add ? p[0] + v : v; }

// hprev = row `walk ? walk[0] : n - 1` of X (the last committed position).
__global__ void mtp_park_kernel(const float *X, int H, const int *walk, int n, float *hprev) {
  const int row = walk ? walk[0] : n - 1;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < H; i += gridDim.x * blockDim.x)
    hprev[i] = X[(size_t)row * H + i];
}

int mtp_ready(const cwen_model *m) {
  const Layer &y = m->L[m->cfg.n_layers];
  return m->mtp_eh && m->mtp_enorm && m->mtp_hnorm && m->mtp_shn && m->mctl && y.attn_norm && y.post_norm &&
         y.ffn_gu && y.ffn_down && y.parts == 3u && y.wo && y.q_norm && y.k_norm;
}

// One pass of B rows through the nextn block (mtp_step, run.c:3099-3133):
// tokens toks[0..B-1], predecessor hiddens rows of hsrc (stride hs) under
// norm weight wpre; the block's attention appends at *mctl + 1 ...  With
// head_t >= 0 (B = 1) the shared head scores the result into mlogits row
// head_t and its argmax lands in mres[4 * head_t + 1].
int mtp_pass(cwen_model *m, int B, const int *toks, const float *hsrc, int hs, const float *wpre, int head_t,
             hipStream_t st) {
  const cwen_model_cfg &c = m->cfg;
  cwen_ctx *ctx = m->ctx;
  const int H = c.d_model;
  Layer &y = m->L[c.n_layers];
  int *const rflag = m->ctl + 5;
  int rc;
  if ((rc = embed_launch(m->emb_qs, m->emb_sc, m->emb_type, toks, B, H, m->e2, H, m->ssq2, st))) return rc;
  hipLaunchKernelGGL(mtp_cat_kernel, dim3(B), dim3(256), 0, st, m->e2, hsrc, hs, wpre, m->mtp_enorm, m->mtp_hnorm,
                     H, c.rms_eps, m->cat, rflag);
  CWEN_HIP_TRY(hipGetLastError());
  GemvOut o0 = {m->X2, nullptr, m->xh2, H, 0};
  o0.ssq = m->ssq2;
  o0.nwh = y.attn_norm;
  o0.rflag = rflag;
  if ((rc = gemv_launch(ctx, m->mtp_eh, 1, 0, GEMV_EPI_STORE, m->cat, o0, B, st))) return rc;
  const Rows r = rows_of(c);
  const GemvPost n1 = {m->ssq2, gemv_row_tiles(m->mtp_eh), c.rms_eps};
  GemvOut o1 = {m->att, nullptr, nullptr, r.att, 0};
  if ((rc = gemv_launch(ctx, y.att_in, 1, 0, GEMV_EPI_STORE, m->xh2, o1, B, st, nullptr, &n1))) return rc;
  if ((rc = attention_launch(m->att, r.att, m->att + r.Qo2, m->att + r.Qo2 + r.Ko, r.att, y.q_norm, y.k_norm,
                             m->qbuf, y.K, y.V, m->mctl, B, c.n_head, c.n_kv_head, c.n_rot_pairs, c.n_rot,
                             c.rope_theta, c.rms_eps, m->apart, c.max_ctx, m->yh, st, rflag, m->pos + B)))
    return rc;
  GemvOut o5 = {m->X2, nullptr, m->xh2, H, 1};
  o5.ssq = m->ssq2;
  o5.nwh = y.post_norm;
  o5.rflag = rflag;
  if ((rc = gemv_launch(ctx, y.wo, 1, 0, GEMV_EPI_STORE, m->yh, o5, B, st))) return rc;
  const GemvPost n2 = {m->ssq2, gemv_row_tiles(y.wo), c.rms_eps};
  GemvOut f1 = {nullptr, nullptr, m->hh, 0, 0};
  f1.rflag = rflag;
  GemvOut f2 = {m->X2, nullptr, m->xh2, H, 1};
  f2.ssq = m->ssq2;
  f2.rflag = rflag;
  f2.nwh = m->mtp_shn;
  if ((rc = gemv_launch(ctx, y.ffn_gu, 2, 0, GEMV_EPI_SWIGLU, m->xh2, f1, B, st, nullptr, &n2)) ||
      (rc = gemv_launch(ctx, y.ffn_down, 1, 0, GEMV_EPI_STORE, m->hh, f2, B, st)))
    return rc;
  if (head_t < 0) return CWEN_OK;
  const GemvPost nh = {m->ssq2, gemv_row_tiles(y.ffn_down), c.rms_eps};
  GemvOut o = {m->mlogits + (size_t)head_t * c.vocab, nullptr, nullptr, c.vocab, 0,
               {ctx->amax_keys, ctx->amax_cnt, m->toks, 0, m->mres + 4 * head_t}};
  return gemv_launch(ctx, m->head, 1, 0, GEMV_EPI_ARGMAX, m->xh2, o, 1, st, nullptr, &nh);
}

// mtp_commit (run.c:3150-3163) for the B positions of a block starting at
// position P = m->pos + 1: position 0 is only parked (it has no
// predecessor), every other position p is stepped with its token and the
// target residual of p - 1.  Rows past the verify walk write MTP slots past
// the commit, which later blocks and drafts rewrite before any read; the
// parked hidden is the walk's last kept row.
int mtp_commit_pass(cwen_model *m, int B, int mode, hipStream_t st) {
  const int H = m->cfg.d_model, P = m->pos;
  const int s0 = P < 0 ? 1 : 0, Bm = B - s0;
  if (Bm > 0) {
    float *dst = m->hin;
    if (!s0) {
      CWEN_HIP_TRY(hipMemcpyAsync(dst, m->hprev, (size_t)H * sizeof(float), hipMemcpyDeviceToDevice, st));
      dst += H;
    }
    if (B > 1)
      CWEN_HIP_TRY(hipMemcpyAsync(dst, m->X, (size_t)(B - 1) * H * sizeof(float), hipMemcpyDeviceToDevice, st));
    hipLaunchKernelGGL(mtp_ctl_kernel, dim3(1), dim3(1), 0, st, m->mctl, P + s0 - 1, 0);
    CWEN_HIP_TRY(hipGetLastError());
    int rc = mtp_pass(m, Bm, m->toks + s0, m->hin, H, m->out_norm, -1, st);
    if (rc) return rc;
  }
  hipLaunchKernelGGL(mtp_park_kernel, dim3((H + 255) / 256), dim3(256), 0, st, m->X, H,
                     mode == MODE_VERIFY ? m->res + 1 : nullptr, B, m->hprev);
  CWEN_HIP_TRY(hipGetLastError());
  return CWEN_OK;
}

int block(cwen_model *m, int B, int mode, hipStream_t st) {
  const cwen_model_cfg &c = m->cfg;
  cwen_ctx *ctx = m->ctx;
  const int H = c.d_model, I = c.d_ffn;
  int rc;
  // RMSNorm of the residual stream X, split between producer and consumer:
  // each producer of X (embed, the accumulating GEMVs) also writes the f16
  // operand x * w of the next norm (weight w) to m->xh, and per-row-tile
  // sums of squares of x to m->ssq (`npart` of them); the consuming GEMV
  // scales its outputs by each column's 1 / rms.  Every block size takes
  // this one path, so blocks and single positions agree bit for bit.
  // Every f16 operand written raises the sticky flag ctl[5] when it is out
  // of f16's range.
  int *const rflag = m->ctl + 5;
  if ((rc = embed_launch(m->emb_qs, m->emb_sc, m->emb_type, m->toks, B, H, m->X, H, m->ssq, st, m->xh,
                         m->L[0].attn_norm, rflag)))
    return rc;
  int npart = 1;
  for (int l = 0; l < c.n_layers; ++l) {
    Layer &y = m->L[l];
    const GemvPost n1 = {m->ssq, npart, c.rms_eps};
    const cwen_weight *wout;
    if (y.linear) {
      const Rows r = rows_of(c);
      // A Q4 in-projection applies the causal conv to its q/k/v rows as it
      // stores them (gdn_conv_out); z and the gates are stored as they are.
      const bool fuse_conv = y.lin_in->fmt == GEMV_Q4;
      GemvOut o1 = {m->lin, nullptr, nullptr, r.lin, 0};
      if (fuse_conv) gdn_conv_out(y.gdn, y.ssm_conv, o1);
      if ((rc = gemv_launch(ctx, y.lin_in, 1, 0, fuse_conv ? GEMV_EPI_CONV : GEMV_EPI_STORE, m->xh, o1, B, st,
                            nullptr, &n1)))
        return rc;
      const float *qkv = m->lin, *z = m->lin + r.C, *ga = m->lin + r.o_alpha, *gb = m->lin + r.o_beta;
      if ((rc = gdn_block_launch(y.gdn, qkv, r.lin, z, r.lin, ga, gb, r.lin, y.ssm_conv, y.ssm_norm, nullptr, 0, B,
                                 st, m->gh, r.Zh, y.ssm_a, y.ssm_dt, 0, rflag, fuse_conv)))
        return rc;
      GemvOut o5 = {m->X, nullptr, m->xh, H, 1};
      o5.ssq = m->ssq;
      o5.nwh = y.post_norm;
      o5.rflag = rflag;
      if ((rc = gemv_launch(ctx, y.ssm_out, 1, 0, GEMV_EPI_STORE, m->gh, o5, B, st))) return rc;
      wout = y.ssm_out;
    } else {
      const Rows r = rows_of(c);
      GemvOut o1 = {m->att, nullptr, nullptr, r.att, 0};
      if ((rc = gemv_launch(ctx, y.att_in, 1, 0, GEMV_EPI_STORE, m->xh, o1, B, st, nullptr, &n1))) return rc;
      if ((rc = attention_launch(m->att, r.att, m->att + r.Qo2, m->att + r.Qo2 + r.Ko, r.att, y.q_norm, y.k_norm,
                                 m->qbuf, y.K, y.V, m->ctl, B, c.n_head, c.n_kv_head, c.n_rot_pairs, c.n_rot,
                                 c.rope_theta, c.rms_eps, m->apart, c.max_ctx, m->yh, st, rflag, m->pos + B)))
        return rc;
      GemvOut o5 = {m->X, nullptr, m->xh, H, 1};
      o5.ssq = m->ssq;
      o5.nwh = y.post_norm;
      o5.rflag = rflag;
      if ((rc = gemv_launch(ctx, y.wo, 1, 0, GEMV_EPI_STORE, m->yh, o5, B, st))) return rc;
      wout = y.wo;
    }
    const GemvPost n2 = {m->ssq, gemv_row_tiles(wout), c.rms_eps};
    GemvOut f1 = {nullptr, nullptr, m->hh, 0, 0};
    f1.rflag = rflag;
    GemvOut f2 = {m->X, nullptr, m->xh, H, 1};
    f2.ssq = m->ssq;
    f2.rflag = rflag;
    f2.nwh = l + 1 < c.n_layers ? m->L[l + 1].attn_norm : m->out_norm;
    if ((rc = gemv_launch(ctx, y.ffn_gu, 2, 0, GEMV_EPI_SWIGLU, m->xh, f1, B, st, nullptr, &n2)) ||
        (rc = gemv_launch(ctx, y.ffn_down, 1, 0, GEMV_EPI_STORE, m->hh, f2, B, st)))
      return rc;
    npart = gemv_row_tiles(y.ffn_down);
    (void)I;
  }
  if (mode != MODE_FWD) {
    const int E = mode == MODE_VERIFY ? B - 1 : 0;
    const GemvPost nh = {m->ssq, npart, c.rms_eps};
    GemvOut o = {m->logits, nullptr, nullptr, c.vocab, 0,
                 {ctx->amax_keys, ctx->amax_cnt, m->toks + 1, E, m->res + 1}};
    if ((rc = gemv_launch(ctx, m->head, 1, 0, GEMV_EPI_ARGMAX, m->xh, o, B, st, nullptr, &nh))) return rc;
  }
  if (mtp_ready(m) && (rc = mtp_commit_pass(m, B, mode, st))) return rc;
  hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(1), 0, st, m->ctl, mode == MODE_VERIFY ? m->res + 1 : nullptr, B,
                     B, CWEN_BMAX + 1, m->res);
  CWEN_HIP_TRY(hipGetLastError());
  return CWEN_OK;
}

void drop_graphs(cwen_model *m) {
  for (auto &mode : m->gexec)
    for (auto &row : mode)
      for (hipGraphExec_t &g : row)
        if (g) {
          (void)hipGraphExecDestroy(g);
          g = nullptr;
        }
}

// Stage the tokens, then run the block: replay its graph (captured on first
// use) or launch eagerly.
int run_block(cwen_model *m, const int *toks, int B, int mode, hipStream_t st) {
  for (int b = 0; b < B; ++b)
    if (toks[b] < 0 || toks[b] >= m->cfg.vocab) return CWEN_EINVAL;
  CWEN_HIP_TRY(hipEventSynchronize(m->tok_ev));  // the previous staging copy has been read
  memcpy(m->htok, toks, (size_t)B * sizeof(int));
  CWEN_HIP_TRY(hipMemcpyAsync(m->toks, m->htok, (size_t)B * sizeof(int), hipMemcpyHostToDevice, st));
  CWEN_HIP_TRY(hipEventRecord(m->tok_ev, st));
  // the MTP commit's launch shape depends on the position: eager
  if (!m->use_graphs || mtp_ready(m)) return block(m, B, mode, st);
  hipGraphExec_t &ge = m->gexec[mode][attention_wide(m->pos + B)][B - 1];
  if (!ge) {
    hipGraph_t g = nullptr;
    CWEN_HIP_TRY(hipStreamBeginCapture(m->cap, hipStreamCaptureModeThreadLocal));
    const int rc = block(m, B, mode, m->cap);
    const hipError_t e = hipStreamEndCapture(m->cap, &g);
    if (rc || e != hipSuccess) {
      if (g) (void)hipGraphDestroy(g);
      return rc ? rc : CWEN_EHIP;
    }
    const hipError_t ei = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (ei != hipSuccess) {
      ge = nullptr;
      return CWEN_EHIP;
    }
  }
  CWEN_HIP_TRY(hipGraphLaunch(ge, st));
  return CWEN_OK;
}

// Host copy of the commit the block of B made on the device.
void commit(cwen_model *m, int n, int B) {
  for (int l = 0; l < m->cfg.n_layers; ++l)
    if (m->L[l].linear) gdn_commit_host(m->L[l].gdn, n, B);
  m->pos += n;
  if (mtp_ready(m)) m->mtp_hpos = m->pos;
}

// The MTP block's buffers, on the first MTP tensor set.
int mtp_alloc(cwen_model *m) {
  if (m->mctl) return CWEN_OK;
  const cwen_model_cfg &c = m->cfg;
  const int H = c.d_model, BM = CWEN_BMAX;
  const Rows R = rows_of(c);
  Layer &y = m->L[c.n_layers];
  y.linear = 0;
  const size_t kv = (size_t)c.max_ctx * R.Ko;
  int rc = (dmalloc(&y.K, kv) || dmalloc(&y.V, kv) || dmalloc(&m->mres, 4 * BM) || dmalloc(&m->hprev, H) ||
            dmalloc(&m->hin, (size_t)BM * H) || dmalloc(&m->e2, (size_t)BM * H) || dmalloc(&m->X2, (size_t)BM * H) ||
            dmalloc(&m->cat, (size_t)BM * 2 * H) || dmalloc(&m->xh2, (size_t)BM * H) ||
            dmalloc(&m->ssq2, (size_t)CWEN_MAX_PARTS * BM) || dmalloc(&m->mlogits, (size_t)BM * c.vocab))
               ? CWEN_ENOMEM
               : CWEN_OK;
  if (!rc) rc = gemv_alloc_q4(m->ctx, H, R.att, &y.att_in);
  if (!rc && hipHostMalloc((void **)&m->hmres, 4 * BM * sizeof(int), hipHostMallocDefault) != hipSuccess)
    rc = CWEN_ENOMEM;
  if (!rc) rc = dmalloc(&m->mctl, 2);  // last: marks the buffers complete
  return rc;
}

int ready(const cwen_model *m) {
  if (!m->emb_qs || !m->out_norm || !m->head) return 0;
  for (int l = 0; l < m->cfg.n_layers; ++l) {
    const Layer &y = m->L[l];
    if (!y.attn_norm || !y.post_norm || !y.ffn_gu || !y.ffn_down) return 0;
    if (y.linear && (y.parts != 15u || !y.ssm_out || !y.ssm_a || !y.ssm_dt || !y.ssm_conv || !y.ssm_norm))
      return 0;
    if (!y.linear && (y.parts != 3u || !y.wo || !y.q_norm || !y.k_norm)) return 0;
  }
  return 1;
}


// ---- seeded synthetic tensors generated on the device (benchmarks: the
// random-init weights of the architecture without a host round trip).
// Counter-based: value i of stream `key` is a function of (seed, key, i) only.
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}
__device__ __forceinline__ uint64_t hsh(uint64_t seed, uint64_t key, uint64_t i) {
  return mix64(seed * 0x9e3779b97f4a7c15ull ^ mix64(key * 0xd1b54a32d192ed03ull + i));
}
__device__ __forceinline__ float unif(uint64_t h) { return ((h >> 40) + 0.5f) * (1.f / 16777216.f); }  // (0,1)
__device__ __forceinline__ float gauss(uint64_t seed, uint64_t key, uint64_t i) {
  const uint64_t h = hsh(seed, key, i);
  const float u1 = ((h >> 40) + 0.5f) * (1.f / 16777216.f), u2 = ((h & 0xFFFFFF) + 0.5f) * (1.f / 16777216.f);
  return sqrtf(-2.f * logf(u1)) * cosf(6.2831853f * u2);
}
// bytes uniform 0..255
__global__ void synth_bytes_kernel(uint8_t *p, size_t n, uint64_t seed, uint64_t key) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    p[i] = (uint8_t)(hsh(seed, key, i) >> 56);
}
// f16 scales |N(0, sigma)|, written at p[i * stride] (bytes) for i < n
__global__ void synth_scale_kernel(uint8_t *p, size_t n, size_t stride, float sigma, uint64_t seed, uint64_t key) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const _Float16 h = (_Float16)fabsf(gauss(seed, key, i) * sigma);
    *(uint16_t *)(p + i * stride) = __builtin_bit_cast(uint16_t, h);
  }
}
// f32 values: kind 0: mu + sigma N, kind 1: -exp(U(-1, 1))
__global__ void synth_f32_kernel(float *p, size_t n, int kind, float mu, float sigma, uint64_t seed, uint64_t key) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    p[i] = kind == 0 ? mu + sigma * gauss(seed, key, i) : -expf(2.f * unif(hsh(seed, key, i)) - 1.f);
}

int synth_launch_grid(size_t n) { return (int)((n + 255) / 256 < 65536 ? (n + 255) / 256 : 65536); }

// A quantized matrix of `type` [ne1][ne0] generated in its reference layout on
// the device (raw bytes and scale channel).
struct Raw {
  uint8_t *q = nullptr, *s = nullptr;
  ~Raw() {
    if (q) (void)hipFree(q);
    if (s) (void)hipFree(s);
  }
};
int synth_raw(int type, int ne0, int ne1, uint64_t seed, uint64_t key, Raw &r) {
  const size_t nblk = (size_t)(ne0 / 32) * ne1;
  size_t qbytes, sbytes = 0;
  switch (type) {
    case CWEN_T_Q4_0RS: qbytes = nblk * 16; sbytes = nblk * 2; break;
    case CWEN_T_Q4_0RSI: qbytes = nblk * 32; sbytes = nblk * 4; break;
    case CWEN_T_Q6_K: qbytes = (size_t)(ne0 / 256) * ne1 * 210; break;
    default: return CWEN_ETYPE;
  }
  if (dmalloc(&r.q, qbytes) || (sbytes && dmalloc(&r.s, sbytes))) return CWEN_ENOMEM;
  hipLaunchKernelGGL(synth_bytes_kernel, dim3(synth_launch_grid(qbytes)), dim3(256), 0, nullptr, r.q, qbytes, seed,
                     key * 4);
  if (type == CWEN_T_Q6_K)  // d = f16(|N(0, 0.002)|) at byte 208 of each 210-byte super-block
    hipLaunchKernelGGL(synth_scale_kernel, dim3(synth_launch_grid(qbytes / 210)), dim3(256), 0, nullptr, r.q + 208,
                       qbytes / 210, (size_t)210, 0.002f, seed, key * 4 + 1);
  else  // f16(|N(0, 0.02)| / 8)
    hipLaunchKernelGGL(synth_scale_kernel, dim3(synth_launch_grid(sbytes / 2)), dim3(256), 0, nullptr, r.s,
                       sbytes / 2, (size_t)2, 0.02f / 8.f, seed, key * 4 + 1);
  CWEN_HIP_TRY(hipGetLastError());
  return CWEN_OK;
}

int synth_weight(cwen_ctx *ctx, int type, int ne0, int ne1, uint64_t seed, uint64_t key, cwen_weight **out) {
  if (ne0 % Q4_K_ALIGN) return CWEN_EINVAL;
  Raw r;
  int rc = synth_raw(type, ne0, ne1, seed, key, r);
  if (rc) return rc;
  cwen_weight *w = (cwen_weight *)calloc(1, sizeof(cwen_weight));
  if (!w) return CWEN_ENOMEM;
  w->ctx = ctx; w->type = type; w->fmt = gemv_fmt_of(type);
  w->ne0 = ne0; w->ne1 = ne1; w->nside = type == CWEN_T_Q4_0RSI ? 2 : 1;
  w->nrg = (ne1 + Q4_ROWS - 1) / Q4_ROWS;
  w->nst = ne0 / Q4_ST_K;
  w->bytes = (size_t)w->nrg * w->nst * w->nside * gemv_st_bytes(w->fmt);
  gemv_choose_split(ctx, w);
  if (w->bytes >= ((size_t)1 << 32)) { free(w); return CWEN_EINVAL; }
  if (dmalloc(&w->dev, w->bytes)) { free(w); return CWEN_ENOMEM; }
  if ((rc = gemv_repack(w, r.q, (const uint16_t *)r.s, nullptr)) || hipDeviceSynchronize() != hipSuccess) {
    (void)hipFree(w->dev);
    free(w);
    return rc ? rc : CWEN_EHIP;
  }
  *out = w;
  return CWEN_OK;
}

// Rows row_off.. of a concatenated weight from a generated matrix (both
// sides of a generated Q4_0RSI pair when side_row_off[1] >= 0).
int synth_part(cwen_weight *w, int type, int M, const int side_row_off[2], uint64_t seed, uint64_t key) {
  Raw r;
  int rc = synth_raw(type, w->ne0, M, seed, key, r);
  if (rc) return rc;
  if (type == CWEN_T_Q4_0RSI) {
    if ((rc = gemv_repack_part(w, r.q, (const uint16_t *)r.s, type, M, side_row_off[0], 0, nullptr)) ||
        (rc = gemv_repack_part(w, r.q, (const uint16_t *)r.s, type, M, side_row_off[1], 1, nullptr)))
      return rc;
  } else if ((rc = gemv_repack_part(w, r.q, (const uint16_t *)r.s, type, M, side_row_off[0], -1, nullptr))) {
    return rc;
  }
  CWEN_HIP_TRY(hipDeviceSynchronize());
  return CWEN_OK;
}

int synth_f32(float **out, size_t n, int kind, float mu, float sigma, uint64_t seed, uint64_t key) {
  if (*out) (void)hipFree(*out);
  *out = nullptr;
  if (dmalloc(out, n)) return CWEN_ENOMEM;
  hipLaunchKernelGGL(synth_f32_kernel, dim3(synth_launch_grid(n)), dim3(256), 0, nullptr, *out, n, kind, mu, sigma,
                     seed, key * 4 + 2);
  CWEN_HIP_TRY(hipGetLastError());
  return CWEN_OK;
}

}  // namespace

extern "C" {

int cwen_model_create(cwen_ctx *ctx, const cwen_model_cfg *cfg, cwen_model **out) {
  if (!ctx || !out) return CWEN_EINVAL;
  *out = nullptr;
  int rc = check_cfg(cfg);
  if (rc) return rc;
  CWEN_HIP_TRY(hipSetDevice(ctx->device));
  cwen_model *m = new (std::nothrow) cwen_model();
  if (!m) return CWEN_ENOMEM;
  m->ctx = ctx;
  m->cfg = *cfg;
  const cwen_model_cfg &c = m->cfg;
  m->L = new (std::nothrow) Layer[c.n_layers + 1];  // + the MTP block
  if (!m->L) { delete m; return CWEN_ENOMEM; }
  const int H = c.d_model, I = c.d_ffn, BM = CWEN_BMAX;
  const Rows R = rows_of(c);
  const int Zh = R.Zh, Qo = R.Qo2 / 2, Ko = R.Ko;
  const char *ge = getenv("CWEN_GRAPHS");
  m->use_graphs = ge && ge[0] == '1';
  if (m->use_graphs && under_profiler()) {
    // A replayed graph under rocprofv3's kernel tracer crashed inside the HIP
    // runtime (a host copy in the tracer's graph-launch path); the same
    // replays are bit-identical to eager launches without it.  Eager launches
    // give the profiler the same kernels.
    fprintf(stderr, "cwen: CWEN_GRAPHS=1 ignored under a profiler (graph replay is not traced safely); "
                    "launching eagerly\n");
    m->use_graphs = 0;
  }
  const int ctl0[6] = {-1, 0, 0, 0, 0, 0};  // position, ring slot, base slot, replay count, buffer, range flag
  rc = dmalloc(&m->ctl, 6) ? CWEN_ENOMEM : CWEN_OK;
  if (!rc && (hipMemcpy(m->ctl, ctl0, sizeof(ctl0), hipMemcpyHostToDevice) != hipSuccess ||
              hipStreamCreateWithFlags(&m->cap, hipStreamNonBlocking) != hipSuccess ||
              hipEventCreateWithFlags(&m->tok_ev, hipEventDisableTiming) != hipSuccess))
    rc = CWEN_EHIP;
  if (!rc) rc = attention_init();
  for (int l = 0; l < c.n_layers && !rc; ++l) {
    Layer &y = m->L[l];
    y.linear = !is_full(c, l);
    if (y.linear) {
      if (!(rc = cwen_gdn_create(ctx, c.gdn_nkh, c.gdn_nvh, 128, &y.gdn))) {
        (void)hipFree(y.gdn->ctl);  // every layer's state moves with the model's commit
        y.gdn->ctl = m->ctl + 1;
        y.gdn->own_ctl = 0;
        rc = gemv_alloc_q4(ctx, H, R.lin, &y.lin_in);
      }
    } else {
      const size_t kv = (size_t)c.max_ctx * Ko;
      rc = dmalloc(&y.K, kv) || dmalloc(&y.V, kv) ? CWEN_ENOMEM : CWEN_OK;
      if (!rc) rc = gemv_alloc_q4(ctx, H, R.att, &y.att_in);
    }
  }
  if (!rc)
    rc = (dmalloc(&m->toks, BM) || dmalloc(&m->res, 3 + BM) ||
          dmalloc(&m->X, (size_t)BM * H) || dmalloc(&m->ssq, (size_t)CWEN_MAX_PARTS * BM) || dmalloc(&m->xh, (size_t)BM * H) ||
          dmalloc(&m->lin, (size_t)BM * R.lin) || dmalloc(&m->gh, (size_t)BM * Zh) ||
          dmalloc(&m->att, (size_t)BM * R.att) || dmalloc(&m->qbuf, (size_t)BM * Qo) ||
          dmalloc(&m->apart, attn_partial_floats(c.n_head, c.n_kv_head, c.max_ctx, BM)) ||
          dmalloc(&m->yh, (size_t)BM * Qo) || dmalloc(&m->hh, (size_t)BM * I) ||
          dmalloc(&m->logits, (size_t)BM * c.vocab))
             ? CWEN_ENOMEM
             : CWEN_OK;
  if (!rc && (hipHostMalloc((void **)&m->hres, (3 + BM) * sizeof(int), hipHostMallocDefault) != hipSuccess ||
              hipHostMalloc((void **)&m->htok, BM * sizeof(int), hipHostMallocDefault) != hipSuccess))
    rc = CWEN_ENOMEM;
  if (rc) {
    cwen_model_free(m);
    return rc;
  }
  *out = m;
  return CWEN_OK;
}

int cwen_model_free(cwen_model *m) {
  if (!m) return CWEN_EINVAL;
  (void)hipSetDevice(m->ctx->device);
  (void)hipDeviceSynchronize();
  drop_graphs(m);
  if (m->cap) (void)hipStreamDestroy(m->cap);
  if (m->tok_ev) (void)hipEventDestroy(m->tok_ev);
  for (int l = 0; m->L && l <= m->cfg.n_layers; ++l) {
    Layer &y = m->L[l];
    for (float *p : {y.attn_norm, y.post_norm, y.ssm_a, y.ssm_dt, y.ssm_conv, y.ssm_norm, y.q_norm, y.k_norm, y.K,
                     y.V})
      if (p) (void)hipFree(p);
    for (cwen_weight *w : {y.ffn_gu, y.ffn_down, y.lin_in, y.ssm_out, y.att_in, y.wo})
      if (w) cwen_weight_free(w);
    if (y.gdn) cwen_gdn_free(y.gdn);
  }
  delete[] m->L;
  for (void *p : {(void *)m->emb_qs, (void *)m->emb_sc, (void *)m->out_norm, (void *)m->toks, (void *)m->ctl,
                  (void *)m->res, (void *)m->X, (void *)m->ssq, (void *)m->xh, (void *)m->lin, (void *)m->gh, (void *)m->att,
                  (void *)m->qbuf,
                  (void *)m->apart, (void *)m->yh, (void *)m->hh, (void *)m->logits})
    if (p) (void)hipFree(p);
  for (void *p : {(void *)m->mtp_enorm, (void *)m->mtp_hnorm, (void *)m->mtp_shn, (void *)m->mctl, (void *)m->mres,
                  (void *)m->hprev, (void *)m->hin, (void *)m->e2, (void *)m->X2, (void *)m->cat, (void *)m->xh2,
                  (void *)m->ssq2, (void *)m->mlogits})
    if (p) (void)hipFree(p);
  if (m->mtp_eh) cwen_weight_free(m->mtp_eh);
  if (m->hmres) (void)hipHostFree(m->hmres);
  if (m->head) cwen_weight_free(m->head);
  if (m->hres) (void)hipHostFree(m->hres);
  if (m->htok) (void)hipHostFree(m->htok);
  delete m;
  return CWEN_OK;
}

int cwen_model_set(cwen_model *m, int layer, int id, int type, const void *data, const void *scales,
                   int ne0, int ne1) {
  if (!m || !data) return CWEN_EINVAL;
  drop_graphs(m);  // captured launches hold the weight pointers
  const cwen_model_cfg &c = m->cfg;
  const int H = c.d_model, I = c.d_ffn;
  const int C = (2 * c.gdn_nkh + c.gdn_nvh) * 128, Zh = c.gdn_nvh * 128;
  const int Qo = c.n_head * c.head_dim;
  CWEN_HIP_TRY(hipSetDevice(m->ctx->device));
  const bool f32 = type == CWEN_T_F32;
  if (id == CWEN_TOK_EMBD) {  // rows dequantised one token at a time (embed_token_to)
    if ((type != CWEN_T_Q4_0 && type != CWEN_T_Q4_0RS && type != CWEN_T_Q6_K) || ne0 != H || ne1 != c.vocab)
      return CWEN_EINVAL;
    if ((type == CWEN_T_Q4_0RS && !scales) || (type == CWEN_T_Q6_K && H % 256)) return CWEN_EINVAL;
    const size_t nblk = (size_t)(H / 32) * c.vocab;
    if (m->emb_qs) (void)hipFree(m->emb_qs);
    if (m->emb_sc) (void)hipFree(m->emb_sc);
    m->emb_qs = nullptr; m->emb_sc = nullptr;
    const size_t qb = type == CWEN_T_Q4_0 ? nblk * 18
                    : type == CWEN_T_Q6_K ? (size_t)(H / 256) * 210 * c.vocab : nblk * 16;
    if (dmalloc(&m->emb_qs, qb)) return CWEN_ENOMEM;
    CWEN_HIP_TRY(hipMemcpy(m->emb_qs, data, qb, hipMemcpyHostToDevice));
    if (type == CWEN_T_Q4_0RS) {
      if (dmalloc(&m->emb_sc, nblk)) return CWEN_ENOMEM;
      CWEN_HIP_TRY(hipMemcpy(m->emb_sc, scales, nblk * 2, hipMemcpyHostToDevice));
    }
    m->emb_type = type;
    return CWEN_OK;
  }
  if (id == CWEN_OUTPUT_NORM) return (f32 && ne0 == H) ? upload_f32(data, H, &m->out_norm) : CWEN_EINVAL;
  if (id == CWEN_OUTPUT) return f32 ? CWEN_ETYPE : upload_w(m, type, data, scales, ne0, ne1, H, c.vocab, &m->head);
  if (id >= CWEN_NEXTN_EH_PROJ && id <= CWEN_NEXTN_SHEAD_NORM) {
    int rc = mtp_alloc(m);
    if (rc) return rc;
    switch (id) {
      case CWEN_NEXTN_EH_PROJ: return upload_w(m, type, data, scales, ne0, ne1, 2 * H, H, &m->mtp_eh);
      case CWEN_NEXTN_ENORM: return (f32 && ne0 == H) ? upload_f32(data, H, &m->mtp_enorm) : CWEN_EINVAL;
      case CWEN_NEXTN_HNORM: return (f32 && ne0 == H) ? upload_f32(data, H, &m->mtp_hnorm) : CWEN_EINVAL;
      default: return (f32 && ne0 == H) ? upload_f32(data, H, &m->mtp_shn) : CWEN_EINVAL;
    }
  }
  if (layer < 0 || layer > c.n_layers) return CWEN_EINVAL;
  if (layer == c.n_layers) {
    int rc = mtp_alloc(m);
    if (rc) return rc;
  }
  Layer &y = m->L[layer];
  switch (id) {
    case CWEN_ATTN_NORM: return (f32 && ne0 == H) ? upload_f32(data, H, &y.attn_norm) : CWEN_EINVAL;
    case CWEN_POST_NORM: return (f32 && ne0 == H) ? upload_f32(data, H, &y.post_norm) : CWEN_EINVAL;
    case CWEN_FFN_GATE_UP:
      return type == CWEN_T_Q4_0RSI ? upload_w(m, type, data, scales, ne0, ne1, H, I, &y.ffn_gu) : CWEN_ETYPE;
    case CWEN_FFN_DOWN: return upload_w(m, type, data, scales, ne0, ne1, I, H, &y.ffn_down);
    default: break;
  }
  const Rows R = rows_of(c);
  auto part = [&](cwen_weight *w, int want_ne1, int row_off, int side_sel, unsigned bit) {
    if (ne0 != H || ne1 != want_ne1) return CWEN_EINVAL;
    int rc = gemv_upload_part(w, type, data, scales, ne1, row_off, side_sel);
    if (!rc) y.parts |= bit;
    return rc;
  };
  if (y.linear) {
    switch (id) {
      case CWEN_ATTN_QKV: return part(y.lin_in, R.C, 0, -1, 1u);
      case CWEN_ATTN_GATE: return part(y.lin_in, R.Zh, R.C, -1, 2u);
      case CWEN_SSM_ALPHA: return part(y.lin_in, R.nvh, R.o_alpha, -1, 4u);
      case CWEN_SSM_BETA: return part(y.lin_in, R.nvh, R.o_beta, -1, 8u);
      case CWEN_SSM_OUT: return upload_w(m, type, data, scales, ne0, ne1, Zh, H, &y.ssm_out);
      case CWEN_SSM_A: return (f32 && ne0 == c.gdn_nvh) ? upload_f32(data, ne0, &y.ssm_a) : CWEN_EINVAL;
      case CWEN_SSM_DT: return (f32 && ne0 == c.gdn_nvh) ? upload_f32(data, ne0, &y.ssm_dt) : CWEN_EINVAL;
      case CWEN_SSM_CONV: return (f32 && ne0 == 4 * C) ? upload_f32(data, ne0, &y.ssm_conv) : CWEN_EINVAL;
      case CWEN_SSM_NORM: return (f32 && ne0 == 128) ? upload_f32(data, ne0, &y.ssm_norm) : CWEN_EINVAL;
      default: return CWEN_EINVAL;
    }
  }
  switch (id) {
    case CWEN_ATTN_Q: return part(y.att_in, R.Qo2, 0, -1, 1u);
    case CWEN_ATTN_KV: {
      if (type != CWEN_T_Q4_0RSI) return CWEN_ETYPE;
      int rc = part(y.att_in, R.Ko, R.Qo2, 0, 0u);
      if (!rc) rc = part(y.att_in, R.Ko, R.Qo2 + R.Ko, 1, 2u);
      return rc;
    }
    case CWEN_ATTN_OUTPUT: return upload_w(m, type, data, scales, ne0, ne1, Qo, H, &y.wo);
    case CWEN_ATTN_Q_NORM: return (f32 && ne0 == c.head_dim) ? upload_f32(data, ne0, &y.q_norm) : CWEN_EINVAL;
    case CWEN_ATTN_K_NORM: return (f32 && ne0 == c.head_dim) ? upload_f32(data, ne0, &y.k_norm) : CWEN_EINVAL;
    default: return CWEN_EINVAL;
  }
}

int cwen_model_synth(cwen_model *m, unsigned long long seed) {
  if (!m) return CWEN_EINVAL;
  drop_graphs(m);
  const cwen_model_cfg &c = m->cfg;
  const int H = c.d_model, I = c.d_ffn;
  const int C = (2 * c.gdn_nkh + c.gdn_nvh) * 128, Zh = c.gdn_nvh * 128;
  const int Qo = c.n_head * c.head_dim, Ko = c.n_kv_head * c.head_dim;
  cwen_ctx *ctx = m->ctx;
  CWEN_HIP_TRY(hipSetDevice(ctx->device));
  int rc;
  auto W = [&](cwen_weight **w, int type, int ne0, int ne1, uint64_t key) {
    if (*w) cwen_weight_free(*w);
    *w = nullptr;
    return synth_weight(ctx, type, ne0, ne1, seed, key, w);
  };
  {  // embedding Q4_0RS rows
    const size_t nblk = (size_t)(H / 32) * c.vocab;
    if (m->emb_qs) (void)hipFree(m->emb_qs);
    if (m->emb_sc) (void)hipFree(m->emb_sc);
    m->emb_qs = nullptr; m->emb_sc = nullptr;
    if (dmalloc(&m->emb_qs, nblk * 16) || dmalloc(&m->emb_sc, nblk)) return CWEN_ENOMEM;
    hipLaunchKernelGGL(synth_bytes_kernel, dim3(synth_launch_grid(nblk * 16)), dim3(256), 0, nullptr, m->emb_qs,
                       nblk * 16, (uint64_t)seed, (uint64_t)1);
    hipLaunchKernelGGL(synth_scale_kernel, dim3(synth_launch_grid(nblk)), dim3(256), 0, nullptr,
                       (uint8_t *)m->emb_sc, nblk, (size_t)2, 0.02f / 8.f, (uint64_t)seed, (uint64_t)2);
    m->emb_type = CWEN_T_Q4_0RS;
  }
  if ((rc = synth_f32(&m->out_norm, H, 0, 1.f, 0.1f, seed, 3)) || (rc = W(&m->head, CWEN_T_Q6_K, H, c.vocab, 4)))
    return rc;
  for (int l = 0; l < c.n_layers; ++l) {
    Layer &y = m->L[l];
    const uint64_t k0 = 100 * (uint64_t)(l + 1);
    if ((rc = synth_f32(&y.attn_norm, H, 0, 1.f, 0.1f, seed, k0 + 1)) ||
        (rc = synth_f32(&y.post_norm, H, 0, 1.f, 0.1f, seed, k0 + 2)) ||
        (rc = W(&y.ffn_gu, CWEN_T_Q4_0RSI, H, I, k0 + 3)) || (rc = W(&y.ffn_down, CWEN_T_Q4_0RS, I, H, k0 + 4)))
      return rc;
    if (y.linear) {
      const Rows R = rows_of(c);
      const int o0[2] = {0, -1}, o1[2] = {R.C, -1}, o2[2] = {R.o_alpha, -1}, o3[2] = {R.o_beta, -1};
      if ((rc = synth_part(y.lin_in, CWEN_T_Q4_0RS, C, o0, seed, k0 + 5)) ||
          (rc = synth_part(y.lin_in, CWEN_T_Q4_0RS, Zh, o1, seed, k0 + 6)) ||
          (rc = synth_part(y.lin_in, CWEN_T_Q4_0RS, c.gdn_nvh, o2, seed, k0 + 7)) ||
          (rc = synth_part(y.lin_in, CWEN_T_Q4_0RS, c.gdn_nvh, o3, seed, k0 + 8)) ||
          (rc = W(&y.ssm_out, CWEN_T_Q4_0RS, Zh, H, k0 + 9)) ||
          (rc = synth_f32(&y.ssm_a, c.gdn_nvh, 1, 0.f, 0.f, seed, k0 + 10)) ||
          (rc = synth_f32(&y.ssm_dt, c.gdn_nvh, 0, 0.f, 0.5f, seed, k0 + 11)) ||
          (rc = synth_f32(&y.ssm_conv, (size_t)4 * C, 0, 0.f, 0.3f, seed, k0 + 12)) ||
          (rc = synth_f32(&y.ssm_norm, 128, 0, 1.f, 0.1f, seed, k0 + 13)))
        return rc;
      y.parts = 15u;
    } else {
      const Rows R = rows_of(c);
      const int oq[2] = {0, -1}, okv[2] = {R.Qo2, R.Qo2 + R.Ko};
      if ((rc = synth_part(y.att_in, CWEN_T_Q4_0RS, 2 * Qo, oq, seed, k0 + 14)) ||
          (rc = synth_part(y.att_in, CWEN_T_Q4_0RSI, Ko, okv, seed, k0 + 15)) ||
          (rc = W(&y.wo, CWEN_T_Q4_0RS, Qo, H, k0 + 16)) ||
          (rc = synth_f32(&y.q_norm, c.head_dim, 0, 1.f, 0.1f, seed, k0 + 17)) ||
          (rc = synth_f32(&y.k_norm, c.head_dim, 0, 1.f, 0.1f, seed, k0 + 18)))
        return rc;
      y.parts = 3u;
    }
  }
  CWEN_HIP_TRY(hipDeviceSynchronize());
  return CWEN_OK;
}

int cwen_model_reset(cwen_model *m) {
  if (!m) return CWEN_EINVAL;
  CWEN_HIP_TRY(hipSetDevice(m->ctx->device));
  CWEN_HIP_TRY(hipDeviceSynchronize());
  for (int l = 0; l < m->cfg.n_layers; ++l)
    if (m->L[l].linear) {
      cwen_gdn *g = m->L[l].gdn;
      g->cur = g->X = g->L = g->P = 0;
      int rc = cwen_gdn_set_state(g, nullptr, nullptr);
      if (rc) return rc;
    }
  const int ctl0[6] = {-1, 0, 0, 0, 0, 0};  // clears the range flag too
  CWEN_HIP_TRY(hipMemcpy(m->ctl, ctl0, sizeof(ctl0), hipMemcpyHostToDevice));
  m->pos = -1;
  m->mtp_hpos = -1;
  return CWEN_OK;
}

int cwen_model_pos(const cwen_model *m) { return m ? m->pos : CWEN_EINVAL; }

int cwen_model_capacity(const cwen_model *m) { return m ? m->cfg.max_ctx : CWEN_EINVAL; }

int cwen_model_forward(cwen_model *m, const int *toks, int B, int want_argmax, int *argmax_out, void *stream) {
  if (!m || !toks || B < 1 || B > CWEN_BMAX || !ready(m)) return CWEN_EINVAL;
  if (m->pos + B >= m->cfg.max_ctx) return CWEN_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  int rc;
  if ((rc = run_block(m, toks, B, want_argmax ? MODE_FWD_HEAD : MODE_FWD, st))) return rc;
  if (want_argmax) {
    CWEN_HIP_TRY(hipMemcpyAsync(m->hres, m->res, (3 + B) * sizeof(int), hipMemcpyDeviceToHost, st));
    CWEN_HIP_TRY(hipStreamSynchronize(st));
    if (argmax_out) memcpy(argmax_out, m->hres + 3, (size_t)B * sizeof(int));
  }
  commit(m, B, B);
  return want_argmax && m->hres[0] ? CWEN_ERANGE : CWEN_OK;
}

int cwen_model_verify(cwen_model *m, const int *blk, int B, int *k_out, int *bonus_out, void *stream) {
  if (!m || !blk || B < 1 || B > CWEN_BMAX || !ready(m)) return CWEN_EINVAL;
  if (m->pos + B >= m->cfg.max_ctx) return CWEN_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  int rc;
  if ((rc = run_block(m, blk, B, MODE_VERIFY, st))) return rc;
  CWEN_HIP_TRY(hipMemcpyAsync(m->hres, m->res, 3 * sizeof(int), hipMemcpyDeviceToHost, st));
  CWEN_HIP_TRY(hipStreamSynchronize(st));
  const int k = m->hres[1];
  if (k < 0 || k > B - 1) return CWEN_EHIP;
  commit(m, k + 1, B);
  if (k_out) *k_out = k;
  if (bonus_out) *bonus_out = m->hres[2];
  return m->hres[0] ? CWEN_ERANGE : CWEN_OK;
}

int cwen_model_has_mtp(const cwen_model *m) { return m ? mtp_ready(m) : CWEN_EINVAL; }

int cwen_model_mtp_draft(cwen_model *m, int pend, int n, int *drafts, void *stream) {
  if (!m || !drafts || n < 0 || n > CWEN_BMAX - 1 || pend < 0 || pend >= m->cfg.vocab) return CWEN_EINVAL;
  if (!mtp_ready(m) || !ready(m) || m->pos < 0 || m->mtp_hpos != m->pos || n == 0) return 0;
  if (m->pos + n >= m->cfg.max_ctx) n = m->cfg.max_ctx - 1 - m->pos;
  if (n <= 0) return 0;
  hipStream_t st = (hipStream_t)stream;
  const cwen_model_cfg &c = m->cfg;
  CWEN_HIP_TRY(hipSetDevice(m->ctx->device));
  CWEN_HIP_TRY(hipEventSynchronize(m->tok_ev));
  m->htok[0] = pend;
  CWEN_HIP_TRY(hipMemcpyAsync(m->toks, m->htok, sizeof(int), hipMemcpyHostToDevice, st));
  CWEN_HIP_TRY(hipEventRecord(m->tok_ev, st));
  // slots pos+1 .. pos+n, at indices pos .. pos+n-1
  hipLaunchKernelGGL(mtp_ctl_kernel, dim3(1), dim3(1), 0, st, m->mctl, m->pos - 1, 0);
  CWEN_HIP_TRY(hipGetLastError());
  for (int t = 0; t < n; ++t) {
    const int *tok = t ? m->mres + 4 * (t - 1) + 1 : m->toks;
    const int rc = t ? mtp_pass(m, 1, tok, m->X2, c.d_model, m->mtp_shn, t, st)
                     : mtp_pass(m, 1, tok, m->hprev, c.d_model, m->out_norm, t, st);
    if (rc) return rc;
    hipLaunchKernelGGL(mtp_ctl_kernel, dim3(1), dim3(1), 0, st, m->mctl, 1, 1);
    CWEN_HIP_TRY(hipGetLastError());
  }
  CWEN_HIP_TRY(hipMemcpyAsync(m->hmres, m->mres, (size_t)4 * n * sizeof(int), hipMemcpyDeviceToHost, st));
  CWEN_HIP_TRY(hipStreamSynchronize(st));
  for (int t = 0; t < n; ++t) {
    drafts[t] = m->hmres[4 * t + 1];
    if (drafts[t] < 0 || drafts[t] >= c.vocab) return CWEN_EHIP;
  }
  return n;
}

int cwen_model_mtp_logits(cwen_model *m, float *host, int rows) {
  if (!m || !host || rows < 1 || rows > CWEN_BMAX || !m->mlogits) return CWEN_EINVAL;
  CWEN_HIP_TRY(hipDeviceSynchronize());
  CWEN_HIP_TRY(hipMemcpy(host, m->mlogits, (size_t)rows * m->cfg.vocab * sizeof(float), hipMemcpyDeviceToHost));
  return CWEN_OK;
}

int cwen_model_logits(cwen_model *m, float *host, int rows) {
  if (!m || !host || rows < 1 || rows > CWEN_BMAX) return CWEN_EINVAL;
  CWEN_HIP_TRY(hipDeviceSynchronize());
  CWEN_HIP_TRY(hipMemcpy(host, m->logits, (size_t)rows * m->cfg.vocab * sizeof(float), hipMemcpyDeviceToHost));
  return CWEN_OK;
}

}  // extern "C"
