// C ABI entry points of libcwen_gpu: context, weight upload, GEMV dispatch.
#include <stdlib.h>
#include <string.h>
#include <atomic>
#include <mutex>
#include "cwen_internal.h"

namespace {

int env_int(const char *name, int dflt, int lo, int hi) {
  const char *s = getenv(name);
  if (!s || !*s) return dflt;
  char *end = nullptr;
  long v = strtol(s, &end, 10);
  if (*end || v < lo || v > hi) return dflt;
  return (int)v;
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

constexpr size_t kScratchHalves = (size_t)CWEN_BMAX * CWEN_KMAX;
constexpr size_t kPartialFloats = (size_t)8 << 20;   // 32 MiB of split-K partials
constexpr int kCounters = 1 << 16;

// Scratch of the allocation-free entry point, one copy per GPU, held until
// the process ends: the f16 operand of X and the f16 hidden activations
// ([CWEN_BMAX][CWEN_STATIC_KMAX] halves each), split-K partials and the
// split-tile arrival counters, in that order.
constexpr size_t kStaticHalves = (size_t)CWEN_BMAX * CWEN_STATIC_KMAX;
constexpr size_t kStaticPartialFloats = (size_t)1 << 20;
constexpr int kStaticCounters = 4096;
constexpr size_t kStaticXhOfs = 0;
constexpr size_t kStaticHhOfs = kStaticXhOfs + kStaticHalves * 2;
constexpr size_t kStaticPartOfs = kStaticHhOfs + kStaticHalves * 2;
constexpr size_t kStaticCntOfs = kStaticPartOfs + kStaticPartialFloats * 4;
constexpr size_t kStaticBytes = kStaticCntOfs + (size_t)kStaticCounters * 4;
static_assert(kStaticBytes == CWEN_STATIC_SCRATCH_BYTES, "static scratch size");
__device__ __align__(256) unsigned char scratch[kStaticBytes];

// Device address of `scratch` on each GPU, looked up once per device with
// that device current (each GPU holds its own copy at its own address).  In
// host code the array's name is not a device address: only these are passed
// to kernels.
constexpr int kMaxDevices = 64;
std::atomic<unsigned char *> g_scratch_dev[kMaxDevices];

__global__ void zero_ints_kernel(int *p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0;
}

// Look up this device's scratch address and clear its counters (first
// context on the device only; `device` is current).  One mutex per device
// serialises the first-time set-up: a second thread creating a context on
// the same GPU waits for the counters to be cleared instead of clearing them
// again under a noalloc call already running there.
std::mutex g_scratch_mu[kMaxDevices];
int static_scratch_init(int device) {
  if (device < 0 || device >= kMaxDevices) return CWEN_EINVAL;
  std::lock_guard<std::mutex> lk(g_scratch_mu[device]);
  if (g_scratch_dev[device].load(std::memory_order_acquire)) return CWEN_OK;
  unsigned char *ptr = nullptr;
  CWEN_HIP_TRY(hipGetSymbolAddress((void **)&ptr, HIP_SYMBOL(scratch)));
  if (!ptr) return CWEN_EHIP;
  hipLaunchKernelGGL(zero_ints_kernel, dim3(16), dim3(256), 0, nullptr, (int *)(ptr + kStaticCntOfs),
                     kStaticCounters);
  CWEN_HIP_TRY(hipGetLastError());
  CWEN_HIP_TRY(hipDeviceSynchronize());
  g_scratch_dev[device].store(ptr, std::memory_order_release);
  return CWEN_OK;
}

}  // namespace

int gemv_alloc_q4(cwen_ctx *ctx, int K, int M, cwen_weight **out) {
  if (K % Q4_K_ALIGN || K > CWEN_KMAX || M <= 0) return CWEN_EINVAL;
  cwen_weight *w = (cwen_weight *)calloc(1, sizeof(cwen_weight));
  if (!w) return CWEN_ENOMEM;
  w->ctx = ctx; w->type = CWEN_T_Q4_0RS; w->fmt = GEMV_Q4;
  w->ne0 = K; w->ne1 = M; w->nside = 1;
  w->nrg = (M + Q4_ROWS - 1) / Q4_ROWS;
  w->nst = K / Q4_ST_K;
  w->bytes = (size_t)w->nrg * w->nst * gemv_st_bytes(GEMV_Q4);
  w->src_bytes = (size_t)(K / 32) * M * 18;
  if (w->bytes >= ((size_t)1 << 32)) { free(w); return CWEN_EINVAL; }
  gemv_choose_split(ctx, w);
  if (hipMalloc((void **)&w->dev, w->bytes) != hipSuccess) { free(w); return CWEN_ENOMEM; }
  if (hipMemset(w->dev, 0, w->bytes) != hipSuccess) { (void)hipFree(w->dev); free(w); return CWEN_EHIP; }
  *out = w;
  return CWEN_OK;
}

int gemv_upload_part(cwen_weight *w, int type, const void *data, const void *scales, int M, int row_off,
                     int side_sel) {
  if (type != CWEN_T_Q4_0 && type != CWEN_T_Q4_0RS && type != CWEN_T_Q4_0RSI) return CWEN_ETYPE;
  if (type != CWEN_T_Q4_0 && !scales) return CWEN_EINVAL;
  const size_t nblk = (size_t)(w->ne0 / 32) * M;
  const size_t qbytes = type == CWEN_T_Q4_0 ? nblk * 18 : type == CWEN_T_Q4_0RS ? nblk * 16 : nblk * 32;
  const size_t sbytes = type == CWEN_T_Q4_0 ? 0 : type == CWEN_T_Q4_0RS ? nblk * 2 : nblk * 4;
  uint8_t *dsrc = nullptr;
  uint16_t *dsc = nullptr;
  int rc = CWEN_OK;
  if (hipMalloc((void **)&dsrc, qbytes) != hipSuccess) return CWEN_ENOMEM;
  if (sbytes && hipMalloc((void **)&dsc, sbytes) != hipSuccess) { rc = CWEN_ENOMEM; goto done; }
  if (hipMemcpy(dsrc, data, qbytes, hipMemcpyHostToDevice) != hipSuccess ||
      (sbytes && hipMemcpy(dsc, scales, sbytes, hipMemcpyHostToDevice) != hipSuccess)) {
    rc = CWEN_EHIP;
    goto done;
  }
  rc = gemv_repack_part(w, dsrc, dsc, type, M, row_off, side_sel, nullptr);
  if (!rc && hipDeviceSynchronize() != hipSuccess) rc = CWEN_EHIP;
done:
  if (dsrc) (void)hipFree(dsrc);
  if (dsc) (void)hipFree(dsc);
  return rc;
}

extern "C" {

const char *cwen_version(void) { return "cwen-gpu 0.1 gfx950"; }

int cwen_ctx_create(int device, cwen_ctx **out) {
  if (!out) return CWEN_EINVAL;
  *out = nullptr;
  int ndev = 0;
  CWEN_HIP_TRY(hipGetDeviceCount(&ndev));
  if (device < 0 || device >= ndev) return CWEN_EINVAL;
  CWEN_HIP_TRY(hipSetDevice(device));
  cwen_ctx *c = (cwen_ctx *)calloc(1, sizeof(cwen_ctx));
  if (!c) return CWEN_ENOMEM;
  c->device = device;
  c->wg_per_cu = env_int("CWEN_GEMV_WG_PER_CU", 1, 1, 16);
  if (hipDeviceGetAttribute(&c->ncu, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || c->ncu < 1) {
    free(c);
    return CWEN_EHIP;
  }
  if (hipMalloc((void **)&c->xh, kScratchHalves * 2) != hipSuccess) {
    free(c);
    return CWEN_ENOMEM;
  }
  if (hipMalloc((void **)&c->hh, kScratchHalves * 2) != hipSuccess ||
      hipMalloc((void **)&c->partials, kPartialFloats * sizeof(float)) != hipSuccess ||
      hipMalloc((void **)&c->counters, kCounters * sizeof(int)) != hipSuccess ||
      hipMalloc((void **)&c->amax_keys, CWEN_BMAX * sizeof(unsigned long long)) != hipSuccess ||
      hipMalloc((void **)&c->amax_cnt, sizeof(int)) != hipSuccess ||
      hipMalloc((void **)&c->res, (2 + CWEN_BMAX) * sizeof(int)) != hipSuccess) {
    cwen_ctx_destroy(c);
    return CWEN_ENOMEM;
  }
  c->partials_floats = kPartialFloats;
  c->ncounters = kCounters;
  if (hipMemset(c->counters, 0, kCounters * sizeof(int)) != hipSuccess ||
      hipMemset(c->amax_keys, 0, CWEN_BMAX * sizeof(unsigned long long)) != hipSuccess ||
      hipMemset(c->amax_cnt, 0, sizeof(int)) != hipSuccess ||
      hipDeviceSynchronize() != hipSuccess) {
    cwen_ctx_destroy(c);
    return CWEN_EHIP;
  }
  const int rs = static_scratch_init(device);
  if (rs) {
    cwen_ctx_destroy(c);
    return rs;
  }
  *out = c;
  return CWEN_OK;
}

int cwen_ctx_destroy(cwen_ctx *ctx) {
  if (!ctx) return CWEN_EINVAL;
  (void)hipSetDevice(ctx->device);
  (void)hipDeviceSynchronize();
  if (ctx->xh) (void)hipFree(ctx->xh);
  if (ctx->hh) (void)hipFree(ctx->hh);
  if (ctx->partials) (void)hipFree(ctx->partials);
  if (ctx->counters) (void)hipFree(ctx->counters);
  if (ctx->amax_keys) (void)hipFree(ctx->amax_keys);
  if (ctx->amax_cnt) (void)hipFree(ctx->amax_cnt);
  if (ctx->res) (void)hipFree(ctx->res);
  free(ctx);
  return CWEN_OK;
}

int cwen_weight_upload(cwen_ctx *ctx, int type, const void *data, const void *scales,
                       int ne0, int ne1, cwen_weight **out) {
  if (!ctx || !data || !out || ne0 <= 0 || ne1 <= 0) return CWEN_EINVAL;
  *out = nullptr;
  const int fmt = gemv_fmt_of(type);
  if (fmt < 0) return CWEN_ETYPE;
  // K: whole blocks, as the reference's row_bytes (run.c:1293-1306) -- 32
  // weights, 256 for the K-quants; the last super-tile is zero-padded.
  const int kq = (type == CWEN_T_Q6_K || type == CWEN_T_Q5_K) ? 256 : 32;
  if (ne0 % kq || ne0 > CWEN_KMAX) return CWEN_EINVAL;
  const bool split_scales = (type == CWEN_T_Q4_0RS || type == CWEN_T_Q4_0RSI);
  if (split_scales && !scales) return CWEN_EINVAL;
  CWEN_HIP_TRY(hipSetDevice(ctx->device));

  const size_t nblk = (size_t)(ne0 / 32) * ne1;
  size_t qbytes = 0, sbytes = 0;
  int nside = 1;
  switch (type) {
    case CWEN_T_Q4_0: qbytes = nblk * 18; break;
    case CWEN_T_Q4_0RS: qbytes = nblk * 16; sbytes = nblk * 2; break;
    case CWEN_T_Q4_0RSI: qbytes = nblk * 32; sbytes = nblk * 4; nside = 2; break;
    case CWEN_T_Q6_K: qbytes = (size_t)(ne0 / 256) * ne1 * 210; break;
    case CWEN_T_Q4_1: qbytes = nblk * 20; break;
    case CWEN_T_Q5_K: qbytes = (size_t)(ne0 / 256) * ne1 * 176; break;
    default: qbytes = nblk * 34; break;  // Q8_0
  }

  cwen_weight *w = (cwen_weight *)calloc(1, sizeof(cwen_weight));
  if (!w) return CWEN_ENOMEM;
  w->ctx = ctx;
  w->type = type;
  w->fmt = fmt;
  w->ne0 = ne0;
  w->ne1 = ne1;
  w->nside = nside;
  w->nrg = (ne1 + Q4_ROWS - 1) / Q4_ROWS;
  w->nst = (ne0 + Q4_ST_K - 1) / Q4_ST_K;
  w->bytes = (size_t)w->nrg * w->nst * nside * gemv_st_bytes(fmt);
  if (w->bytes >= ((size_t)1 << 32)) {  // kernels address weights with 32-bit buffer offsets
    free(w);
    return CWEN_EINVAL;
  }
  w->src_bytes = qbytes + sbytes;
  gemv_choose_split(ctx, w);

  uint8_t *dsrc = nullptr;
  uint16_t *dsc = nullptr;
  int rc = CWEN_OK;
  if (hipMalloc((void **)&w->dev, w->bytes) != hipSuccess) { rc = CWEN_ENOMEM; goto fail; }
  if (hipMalloc((void **)&dsrc, qbytes) != hipSuccess) { rc = CWEN_ENOMEM; goto fail; }
  if (sbytes && hipMalloc((void **)&dsc, sbytes) != hipSuccess) { rc = CWEN_ENOMEM; goto fail; }
  if (hipMemcpy(dsrc, data, qbytes, hipMemcpyHostToDevice) != hipSuccess) { rc = CWEN_EHIP; goto fail; }
  if (sbytes && hipMemcpy(dsc, scales, sbytes, hipMemcpyHostToDevice) != hipSuccess) {
    rc = CWEN_EHIP;
    goto fail;
  }
  rc = gemv_repack(w, dsrc, dsc, nullptr);
  if (rc != CWEN_OK) goto fail;
  if (hipDeviceSynchronize() != hipSuccess) { rc = CWEN_EHIP; goto fail; }
  (void)hipFree(dsrc);
  if (dsc) (void)hipFree(dsc);
  *out = w;
  return CWEN_OK;
fail:
  if (dsrc) (void)hipFree(dsrc);
  if (dsc) (void)hipFree(dsc);
  if (w->dev) (void)hipFree(w->dev);
  free(w);
  return rc;
}

int cwen_weight_free(cwen_weight *w) {
  if (!w) return CWEN_EINVAL;
  (void)hipSetDevice(w->ctx->device);
  (void)hipDeviceSynchronize();
  (void)hipFree(w->dev);
  free(w);
  return CWEN_OK;
}

int cwen_weight_info(const cwen_weight *w, int *type, int *ne0, int *ne1, int *nside,
                     size_t *stream_bytes) {
  if (!w) return CWEN_EINVAL;
  if (type) *type = w->type;
  if (ne0) *ne0 = w->ne0;
  if (ne1) *ne1 = w->ne1;
  if (nside) *nside = w->nside;
  if (stream_bytes) *stream_bytes = w->bytes;
  return CWEN_OK;
}

static int check_act(const float *X, int xs, int K, int B) {
  if (!X || B < 1 || B > CWEN_BMAX) return CWEN_EINVAL;
  if (!aligned16(X) || (xs & 3) || (B > 1 && xs < K)) return CWEN_EINVAL;
  return CWEN_OK;
}
static int check_out(const float *Y, int ys, int M, int B) {
  if (!Y || (B > 1 && ys < M) || ys < 0) return CWEN_EINVAL;
  return CWEN_OK;
}
static int check_w(const cwen_ctx *ctx, const cwen_weight *W) {
  return (!ctx || !W || W->ctx != ctx) ? CWEN_EINVAL : CWEN_OK;
}

// f32 activations of the f32 entry points: for B <= 4 the GEMV stages and
// converts them itself (one launch); for larger blocks a separate conversion
// into ctx->xh is faster (the f32 staging adds registers and L2 traffic to
// every workgroup of the GEMV), measured on the FFN shapes.
static int f32_operand(cwen_ctx *ctx, const float *X, int xs, int K, int B, hipStream_t st, GemvF32 *n,
                       const _Float16 **xh) {
  if (B <= 4) {
    *n = {X, xs};
    *xh = nullptr;
    return CWEN_OK;
  }
  *xh = ctx->xh;
  return act_to_f16(X, xs, ctx->xh, K, B, st);
}

int cwen_act_to_f16(cwen_ctx *ctx, const float *X, int xs, void *Xh, int K, int B, void *stream) {
  if (!ctx || !Xh || !aligned16(Xh) || K <= 0 || (K & 7)) return CWEN_EINVAL;
  int rc = check_act(X, xs, K, B);
  if (rc) return rc;
  return act_to_f16(X, xs, (_Float16 *)Xh, K, B, (hipStream_t)stream);
}

int cwen_gemvb(cwen_ctx *ctx, const cwen_weight *W, int side, const float *X, int xs, float *Y,
               int ys, int B, void *stream) {
  int rc = check_w(ctx, W);
  if (rc) return rc;
  if (side < 0 || side >= W->nside) return CWEN_EINVAL;
  if ((rc = check_act(X, xs, W->ne0, B)) || (rc = check_out(Y, ys, W->ne1, B))) return rc;
  hipStream_t st = (hipStream_t)stream;
  GemvF32 x;
  const _Float16 *xh;
  if ((rc = f32_operand(ctx, X, xs, W->ne0, B, st, &x, &xh))) return rc;
  GemvOut o = {Y, nullptr, nullptr, ys, 0};
  return gemv_launch(ctx, W, 1, side, GEMV_EPI_STORE, xh, o, B, st, xh ? nullptr : &x);
}

int cwen_gemvb_pair(cwen_ctx *ctx, const cwen_weight *W, const float *X, int xs, float *YA,
                    float *YB, int ys, int B, void *stream) {
  int rc = check_w(ctx, W);
  if (rc) return rc;
  if (W->nside != 2) return CWEN_EINVAL;
  if ((rc = check_act(X, xs, W->ne0, B)) || (rc = check_out(YA, ys, W->ne1, B)) ||
      (rc = check_out(YB, ys, W->ne1, B)))
    return rc;
  hipStream_t st = (hipStream_t)stream;
  GemvF32 x;
  const _Float16 *xh;
  if ((rc = f32_operand(ctx, X, xs, W->ne0, B, st, &x, &xh))) return rc;
  GemvOut o = {YA, YB, nullptr, ys, 0};
  return gemv_launch(ctx, W, 2, 0, GEMV_EPI_PAIR, xh, o, B, st, xh ? nullptr : &x);
}

int cwen_gemvb_swiglu(cwen_ctx *ctx, const cwen_weight *W, const float *X, int xs, float *H,
                      int hs, int B, void *stream) {
  int rc = check_w(ctx, W);
  if (rc) return rc;
  if (W->nside != 2) return CWEN_EINVAL;
  if ((rc = check_act(X, xs, W->ne0, B)) || (rc = check_out(H, hs, W->ne1, B))) return rc;
  hipStream_t st = (hipStream_t)stream;
  GemvF32 x;
  const _Float16 *xh;
  if ((rc = f32_operand(ctx, X, xs, W->ne0, B, st, &x, &xh))) return rc;
  GemvOut o = {H, nullptr, nullptr, hs, 0};
  return gemv_launch(ctx, W, 2, 0, GEMV_EPI_SWIGLU, xh, o, B, st, xh ? nullptr : &x);
}

int cwen_gemvb_f16(cwen_ctx *ctx, const cwen_weight *W, int side, const void *Xh, float *Y,
                   int ys, void *Yh, int accumulate, int B, void *stream) {
  int rc = check_w(ctx, W);
  if (rc) return rc;
  if (side < 0 || side >= W->nside || !Xh || !aligned16(Xh) || B < 1 || B > CWEN_BMAX)
    return CWEN_EINVAL;
  if (!Y && !Yh) return CWEN_EINVAL;
  if (Y && (rc = check_out(Y, ys, W->ne1, B))) return rc;
  if (Yh && (W->ne1 & 7)) return CWEN_EINVAL;
  GemvOut o = {Y, nullptr, (_Float16 *)Yh, ys, accumulate ? 1 : 0};
  return gemv_launch(ctx, W, 1, side, GEMV_EPI_STORE, (const _Float16 *)Xh, o, B, (hipStream_t)stream);
}

int cwen_gemvb_swiglu_f16(cwen_ctx *ctx, const cwen_weight *W, const void *Xh, float *H, int hs,
                          void *Hh, int B, void *stream) {
  int rc = check_w(ctx, W);
  if (rc) return rc;
  if (W->nside != 2 || !Xh || !aligned16(Xh) || B < 1 || B > CWEN_BMAX) return CWEN_EINVAL;
  if (!H && !Hh) return CWEN_EINVAL;
  if (H && (rc = check_out(H, hs, W->ne1, B))) return rc;
  GemvOut o = {H, nullptr, (_Float16 *)Hh, hs, 0};
  return gemv_launch(ctx, W, 2, 0, GEMV_EPI_SWIGLU, (const _Float16 *)Xh, o, B, (hipStream_t)stream);
}

int cwen_mlp_block(cwen_ctx *ctx, const cwen_weight *Wgu, const cwen_weight *Wd, const float *X,
                   int xs, float *Y, int ys, int B, void *stream) {
  int rc;
  if ((rc = check_w(ctx, Wgu)) || (rc = check_w(ctx, Wd))) return rc;
  if (Wgu->nside != 2 || Wd->nside != 1 || Wd->ne0 != Wgu->ne1 || Wd->ne1 != Wgu->ne0)
    return CWEN_EINVAL;
  if ((rc = check_act(X, xs, Wgu->ne0, B)) || (rc = check_out(Y, ys, Wd->ne1, B))) return rc;
  hipStream_t st = (hipStream_t)stream;
  GemvF32 x;
  const _Float16 *xh;
  if ((rc = f32_operand(ctx, X, xs, Wgu->ne0, B, st, &x, &xh))) return rc;
  GemvOut o1 = {nullptr, nullptr, ctx->hh, 0, 0};
  if ((rc = gemv_launch(ctx, Wgu, 2, 0, GEMV_EPI_SWIGLU, xh, o1, B, st, xh ? nullptr : &x))) return rc;
  GemvOut o2 = {Y, nullptr, nullptr, ys, 1};
  return gemv_launch(ctx, Wd, 1, 0, GEMV_EPI_STORE, ctx->hh, o2, B, st);
}

int cwen_mlp_block_noalloc(const cwen_weight *Wgu, const cwen_weight *Wd, const float *X, int xs, float *Y,
                           int ys, int B, void *stream) {
  if (!Wgu || !Wd || Wgu->ctx != Wd->ctx) return CWEN_EINVAL;
  cwen_ctx *ctx = Wgu->ctx;
  int rc;
  if (Wgu->nside != 2 || Wd->nside != 1 || Wd->ne0 != Wgu->ne1 || Wd->ne1 != Wgu->ne0) return CWEN_EINVAL;
  if ((rc = check_act(X, xs, Wgu->ne0, B)) || (rc = check_out(Y, ys, Wd->ne1, B))) return rc;
  if (Wgu->ne0 > CWEN_STATIC_KMAX || Wgu->ne1 > CWEN_STATIC_KMAX) return CWEN_ESCRATCH;
  if (ctx->device < 0 || ctx->device >= kMaxDevices) return CWEN_EINVAL;
  unsigned char *const base = g_scratch_dev[ctx->device].load(std::memory_order_acquire);
  if (!base) return CWEN_EINVAL;
  const GemvScratch scr = {(float *)(base + kStaticPartOfs), kStaticPartialFloats, (int *)(base + kStaticCntOfs),
                           kStaticCounters};
  // Both launches' decompositions are checked before the first launch.
  if (!gemv_grid_fits(Wgu->cfg[1], scr.partials_floats, scr.ncounters) ||
      !gemv_grid_fits(Wd->cfg[0], scr.partials_floats, scr.ncounters))
    return CWEN_ESCRATCH;
  hipStream_t st = (hipStream_t)stream;
  _Float16 *const xh = (_Float16 *)(base + kStaticXhOfs), *const hh = (_Float16 *)(base + kStaticHhOfs);
  GemvF32 x = {X, xs};
  const bool stage_f32 = B <= 4;  // the GEMV converts X while staging (cwen_mlp_block's rule)
  if (!stage_f32 && (rc = act_to_f16(X, xs, xh, Wgu->ne0, B, st))) return rc;
  GemvOut o1 = {nullptr, nullptr, hh, 0, 0};
  if ((rc = gemv_launch(ctx, Wgu, 2, 0, GEMV_EPI_SWIGLU, stage_f32 ? nullptr : xh, o1, B, st,
                        stage_f32 ? &x : nullptr, nullptr, &scr)))
    return rc;
  GemvOut o2 = {Y, nullptr, nullptr, ys, 1};
  return gemv_launch(ctx, Wd, 1, 0, GEMV_EPI_STORE, hh, o2, B, st, nullptr, nullptr, &scr);
}

int cwen_head_verify(cwen_ctx *ctx, const cwen_weight *W, const float *X, int xs, int B,
                     const int *drafts, int E, float *logits, int ls, int *res, void *stream) {
  int rc = check_w(ctx, W);
  if (rc) return rc;
  if (W->nside != 1 || !res) return CWEN_EINVAL;
  if ((rc = check_act(X, xs, W->ne0, B))) return rc;
  if (E < 0 || E > B - 1 || (E > 0 && !drafts)) return CWEN_EINVAL;
  if (logits && (rc = check_out(logits, ls, W->ne1, B))) return rc;
  hipStream_t st = (hipStream_t)stream;
  GemvF32 x;
  const _Float16 *xh;
  if ((rc = f32_operand(ctx, X, xs, W->ne0, B, st, &x, &xh))) return rc;
  GemvOut o = {logits, nullptr, nullptr, ls, 0, {ctx->amax_keys, ctx->amax_cnt, drafts, E, res}};
  return gemv_launch(ctx, W, 1, 0, GEMV_EPI_ARGMAX, xh, o, B, st, xh ? nullptr : &x);
}

int cwen_argmax_walk(cwen_ctx *ctx, const float *logits, int ls, int V, int B, const int *drafts,
                     int E, int *res, void *stream) {
  if (!ctx || !logits || !res || V < 1 || B < 1 || B > CWEN_BMAX) return CWEN_EINVAL;
  if ((B > 1 && ls < V) || ls < 0) return CWEN_EINVAL;
  if (E < 0 || E > B - 1 || (E > 0 && !drafts)) return CWEN_EINVAL;
  const ArgmaxOut a = {ctx->amax_keys, ctx->amax_cnt, drafts, E, res};
  return argmax_walk_launch(logits, ls, V, B, a, (hipStream_t)stream);
}

int cwen_gdn_create(cwen_ctx *ctx, int nkh, int nvh, int dk, cwen_gdn **out) {
  if (!ctx || !out || nkh <= 0 || nvh <= 0 || nvh % nkh || dk != 128) return CWEN_EINVAL;
  *out = nullptr;
  CWEN_HIP_TRY(hipSetDevice(ctx->device));
  cwen_gdn *g = (cwen_gdn *)calloc(1, sizeof(cwen_gdn));
  if (!g) return CWEN_ENOMEM;
  g->ctx = ctx;
  g->nkh = nkh; g->nvh = nvh; g->dk = dk;
  g->C = (2 * nkh + nvh) * dk;
  g->nslot = CWEN_BMAX + 1;
  const size_t sf = (size_t)nvh * dk * dk, hf = (size_t)g->C * 3;
  if (hipMalloc((void **)&g->S, sf * 2 * sizeof(float)) != hipSuccess ||
      hipMalloc((void **)&g->H, hf * g->nslot * sizeof(float)) != hipSuccess ||
      hipMalloc((void **)&g->xc, (size_t)2 * CWEN_BMAX * g->C * sizeof(float)) != hipSuccess ||
      hipMalloc((void **)&g->gates, (size_t)2 * CWEN_BMAX * 2 * nvh * sizeof(float)) != hipSuccess ||
      hipMalloc((void **)&g->ctl, 4 * sizeof(int)) != hipSuccess) {
    cwen_gdn_free(g);
    return CWEN_ENOMEM;
  }
  g->own_ctl = 1;
  if (hipMemset(g->ctl, 0, 4 * sizeof(int)) != hipSuccess || hipMemset(g->S, 0, sf * sizeof(float)) != hipSuccess ||
      hipMemset(g->H, 0, hf * sizeof(float)) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
    cwen_gdn_free(g);
    return CWEN_EHIP;
  }
  *out = g;
  return CWEN_OK;
}

int cwen_gdn_free(cwen_gdn *g) {
  if (!g) return CWEN_EINVAL;
  (void)hipSetDevice(g->ctx->device);
  (void)hipDeviceSynchronize();
  for (float *p : {g->S, g->H, g->xc, g->gates, g->S_peek})
    if (p) (void)hipFree(p);
  if (g->ctl && g->own_ctl) (void)hipFree(g->ctl);
  free(g);
  return CWEN_OK;
}

// Write the host copy of the control word to the device (after queued work).
static int gdn_sync_ctl(cwen_gdn *g) {
  CWEN_HIP_TRY(hipDeviceSynchronize());
  const int c[4] = {g->cur, g->X, g->L, g->P};
  CWEN_HIP_TRY(hipMemcpy(g->ctl, c, sizeof(c), hipMemcpyHostToDevice));
  return CWEN_OK;
}

int cwen_gdn_set_state(cwen_gdn *g, const float *S, const float *hist) {
  if (!g) return CWEN_EINVAL;
  CWEN_HIP_TRY(hipSetDevice(g->ctx->device));
  CWEN_HIP_TRY(hipDeviceSynchronize());
  const size_t sf = (size_t)g->nvh * g->dk * g->dk, hf = (size_t)g->C * 3;
  float *Sd = g->S + (size_t)g->X * sf, *Hd = g->H + (size_t)g->cur * hf;
  if (S) CWEN_HIP_TRY(hipMemcpy(Sd, S, sf * sizeof(float), hipMemcpyHostToDevice));
  else CWEN_HIP_TRY(hipMemset(Sd, 0, sf * sizeof(float)));
  if (hist) CWEN_HIP_TRY(hipMemcpy(Hd, hist, hf * sizeof(float), hipMemcpyHostToDevice));
  else CWEN_HIP_TRY(hipMemset(Hd, 0, hf * sizeof(float)));
  g->L = 0;
  g->last_B = 0;
  if (g->own_ctl) return gdn_sync_ctl(g);
  CWEN_HIP_TRY(hipDeviceSynchronize());
  return CWEN_OK;
}

int cwen_gdn_get_state(cwen_gdn *g, int pos, float *S, float *hist) {
  if (!g || pos < 0 || pos > g->last_B) return CWEN_EINVAL;
  CWEN_HIP_TRY(hipSetDevice(g->ctx->device));
  CWEN_HIP_TRY(hipDeviceSynchronize());
  const size_t sf = (size_t)g->nvh * g->dk * g->dk, hf = (size_t)g->C * 3;
  if (S) {
    // After a block (uncommitted): its start state is base X and its inputs
    // are in buffer P; otherwise the committed state is base X plus the
    // replay of L positions of buffer P ^ 1.
    const int L = g->last_B ? pos : g->L, buf = g->last_B ? g->P : (g->P ^ 1);
    if (!g->S_peek && hipMalloc((void **)&g->S_peek, sf * sizeof(float)) != hipSuccess) return CWEN_ENOMEM;
    int rc;
    if ((rc = gdn_peek_launch(g, L, buf, g->S_peek, nullptr))) return rc;
    CWEN_HIP_TRY(hipMemcpy(S, g->S_peek, sf * sizeof(float), hipMemcpyDeviceToHost));
  }
  const int slot = (g->cur + pos) % g->nslot;
  if (hist) CWEN_HIP_TRY(hipMemcpy(hist, g->H + (size_t)slot * hf, hf * sizeof(float), hipMemcpyDeviceToHost));
  return CWEN_OK;
}

int cwen_gdn_block(cwen_ctx *ctx, cwen_gdn *g, const float *qkv, int qs, const float *z, int zs,
                   const float *decay, const float *beta, int gs, const float *kw, const float *wn,
                   float *out, int os, int B, void *stream) {
  if (!ctx || !g || g->ctx != ctx || B < 1 || B > CWEN_BMAX || !g->own_ctl) return CWEN_EINVAL;
  if (!qkv || !z || !decay || !beta || !kw || !wn || !out) return CWEN_EINVAL;
  if (!aligned16(kw) || !aligned16(wn) || !aligned16(out) || (os & 3)) return CWEN_EINVAL;
  const int zh = g->nvh * g->dk;
  if ((B > 1 && (qs < g->C || zs < zh || gs < g->nvh || os < zh)) || qs < 0 || zs < 0 || gs < 0 || os < 0)
    return CWEN_EINVAL;
  // A block after an uncommitted one restarts from that block's start state
  // (commit(0)): its inputs are dropped, no replay.
  const int force_L0 = g->last_B > 0;
  int rc = gdn_block_launch(g, qkv, qs, z, zs, decay, beta, gs, kw, wn, out, os, B, (hipStream_t)stream,
                            nullptr, 0, nullptr, nullptr, force_L0);
  if (rc == CWEN_OK) {
    if (force_L0) g->L = 0;
    g->last_B = B;
  }
  return rc;
}

int cwen_gdn_commit(cwen_gdn *g, int n) {
  if (!g || n < 0 || n > g->last_B || !g->own_ctl) return CWEN_EINVAL;
  CWEN_HIP_TRY(hipSetDevice(g->ctx->device));
  gdn_commit_host(g, n, g->last_B);
  return gdn_sync_ctl(g);
}

}  // extern "C"
