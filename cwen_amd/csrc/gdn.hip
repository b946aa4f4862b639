// GatedDeltaNet block verify: the depthwise causal conv and the gated delta
// rule across the B positions of a draft block, with rollback to any
// accepted prefix.
//
// Reference semantics (run.c): conv1d_update 2183-2200, gdn_step 2014-2180
// (+ l2norm_rows 401-423), as called position by position in
// layer_linear_blk 2700-2704; snap_save / snap_load 2787-2809 and the
// short-walk replay 4975-4988 are replaced as below.
//
// Per position b (C = 2*nkh*dk + nvh*dk channels):
//   conv:  x_c = st0*w0 + st1*w1 + st2*w2 + cur*w3 (no FMA contraction, the
//          reference's scalar order), history shifts in cur, x = silu(x)
//   q, k:  l2-normalised per key head, x / sqrt(sum x^2 + 1e-6)
//   per value head hv (key head hv % nkh):
//          S *= exp(decay);  sk = S^T k;  delta = beta (v - sk);
//          S += k delta^T;   o = S^T q / sqrt(dk)
//   gated RMSNorm: out = wn * o * (1/sqrt(mean(o^2) + 1e-6)) * silu(z)
// S is [hv][i][j], row i the key dimension, as in the reference.
//
// Rollback.  The conv history (3 floats per channel) is kept after every
// position in a ring of CWEN_BMAX+1 slots; accepting n positions moves the
// ring index.  The recurrent state (3.1 MB at 48 heads) has two base slots
// and is not snapshotted per position: a block keeps its inputs (post-conv
// values, g, beta) in a pending buffer and writes its end state to the other
// slot.  Accepting the whole block makes the end state the base; accepting
// n < B keeps the start state as the base, and the next block first replays
// those n positions from the pending buffer (the same instructions as the
// block itself, so the same bits) before its own.  The device control word
// ctl = {ring slot, base slot, replay count, pending parity} is advanced by
// the commit (cwen_gdn_commit, or the model's device commit).
//
// Design (gfx950): two launches on the caller's stream (one inside the
// model, whose in-projection GEMV applies the conv in its epilogue).
//  1. conv: one thread per (channel, position): the 4-tap filter reads its
//     inputs from the block's rows or the start history slot, so every
//     position is computed at once; it writes the post-SiLU value to the
//     pending buffer and that position's history slot to the ring.
//  2. recurrence + gated RMSNorm: the delta rule is column-local (sk[j],
//     delta[j] and o[j] read only column j), so a head's 128 columns split
//     over the 8 waves of one workgroup, 16 columns each (48 workgroups of
//     512 threads at 48 heads).  A lane owns a 4-column x 8-row block of S
//     in registers for the whole block; a column sum is a 16-lane DPP
//     reduction.  The head's outputs meet in LDS and the same workgroup
//     applies the norm, one wave per position.
// Every position runs the same instructions whatever B is, so a block of B
// equals B single-position blocks bit for bit.
#include "cwen_internal.h"

namespace {

constexpr int DK = 128;
constexpr int MAXB = CWEN_BMAX;
constexpr int COLS = 16;            // columns of a head per recurrence workgroup

__device__ __forceinline__ float silu_ref(float x) { return x * (1.f / (1.f + expf(-x))); }

// Control word ctl[4] (device): ring slot, base slot X, replay count L,
// pending parity P.  Block inputs go to pending buffer P; a replay reads
// buffer P ^ 1 (the previous block's).
struct GdnParams {
  float *S_base;              // two base states [2][nvh][DK][DK]
  float *H_slots;             // conv history ring [nslot][C][3]
  size_t s_floats, h_floats;  // floats per state / history slot
  const int *ctl;
  int nslot;
  int force_L0;               // replay nothing (the previous block was not committed)
  float *S_peek;              // peek: replay peek_L positions of buffer peek_buf from base X into S_peek, no block
  int peek_L, peek_buf;
  const float *qkv; int qs;   // raw (pre-conv) qkv [B][qs]
  const float *z; int zs;     // [B][zs]
  const float *decay, *beta; int gs;  // [B][gs]
  const float *kw;            // conv weights [C][4]
  const float *wn;            // gated-norm weight [DK]
  float *out; int os;         // [B][os], nullable
  _Float16 *outh; int ohs;    // f16 copy [B][ohs], nullable
  int *rflag;                 // set to 1 when an f16 copy is out of f16's range, nullable
  const float *A, *dt;        // raw gates when non-null: decay = A*softplus(decay + dt), beta = sigmoid(beta)
  float *xc;                  // pending post-conv values [2][BMAX][C]
  float *gates;               // pending g, beta [2][BMAX][2][nvh]
  int nkh, nvh, C, B;
};

// 1. conv: thread = (channel, position); workgroup = 256 channels of one
// position (blockIdx.y).  The 4-tap filter needs no running state: the
// inputs at b-3 .. b-1 come from the block's own rows or, before the block,
// from the history slot the block starts from, so every position is
// computed at once with run.c's product/sum order.  The pending buffer
// holds the post-conv values; the recurrence l2-normalises q and k as it
// stages them, for the block and for a later replay alike.  Each position's
// thread also writes that position's history slot (inputs b-2, b-1, b).
__global__ __launch_bounds__(256) void gdn_conv_kernel(GdnParams p) {
  const int c = blockIdx.x * 256 + threadIdx.x, b = blockIdx.y;
  if (c >= p.C) return;           // whole waves (C is a multiple of 128)
  const int cur = p.ctl[0], P = p.ctl[3];
  const float *H_in = p.H_slots + (size_t)cur * p.h_floats + (size_t)c * 3;
  const float4 w = *(const float4 *)(p.kw + (size_t)c * 4);
  // inputs at positions b-3, b-2, b-1, b (history slot entries 0..2 are the
  // inputs at -3, -2, -1)
  float in[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int t = b - 3 + j;
    in[j] = t >= 0 ? p.qkv[(size_t)t * p.qs + c] : H_in[t + 3];
  }
  // ((st0*w0 + st1*w1) + st2*w2) + xin*w3, each product and sum rounded
  const float x = __fadd_rn(__fadd_rn(__fadd_rn(__fmul_rn(in[0], w.x), __fmul_rn(in[1], w.y)), __fmul_rn(in[2], w.z)),
                            __fmul_rn(in[3], w.w));
  float y = silu_ref(x);
  float *hs = p.H_slots + (size_t)((cur + 1 + b) % p.nslot) * p.h_floats + (size_t)c * 3;
  hs[0] = in[1]; hs[1] = in[2]; hs[2] = in[3];
  p.xc[((size_t)P * CWEN_BMAX + b) * p.C + c] = y;   // q and k are l2-normalised by the recurrence
}

// 2. recurrence and gated RMSNorm: workgroup hv = 8 waves, wave w the
// columns w*16 .. w*16+15 of value head hv.  Lane: row group rg = lane & 15
// (rows 8rg..8rg+7), column group cg = lane >> 4 (4 columns).  The head's
// 128 outputs of a position meet in LDS, so the norm follows a workgroup
// barrier, not another launch.  Staging is shared: wave w l2-normalises q
// and k of positions w and w + 8, each wave stages its own v columns, the
// last wave the gates.  The replay and the block's own positions share one
// LDS layout per phase.
constexpr int RW = DK / COLS;       // waves per head
__global__ __launch_bounds__(64 * RW) void gdn_rec_kernel(GdnParams p) {
  __shared__ __align__(16) float qk[MAXB][2 * DK];   // normalised q | k per position
  __shared__ __align__(16) float vs[MAXB][DK];
  __shared__ __align__(16) float ob[MAXB][DK];       // pre-norm outputs of the block
  __shared__ float s_g[MAXB], s_beta[MAXB];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hv = blockIdx.x, slice = wave;
  const int hk = hv % p.nkh;
  const bool peek = p.S_peek != nullptr;
  const int X = p.ctl[1], P = p.ctl[3];
  const int L = peek ? p.peek_L : (p.force_L0 ? 0 : p.ctl[2]);
  const int Pr = peek ? p.peek_buf : (P ^ 1);
  const int B = peek ? 0 : p.B;
  const int rg = lane & 15, cg = lane >> 4;
  const int i0 = rg * 8, j0 = slice * COLS + cg * 4;
  const size_t xstride = (size_t)CWEN_BMAX * p.C;
  const size_t gstride = (size_t)CWEN_BMAX * 2 * p.nvh;

  float4 s[8];
  {
    const float *Sh = p.S_base + (size_t)X * p.s_floats + (size_t)hv * DK * DK;
#pragma unroll
    for (int r = 0; r < 8; ++r) s[r] = *(const float4 *)(Sh + (size_t)(i0 + r) * DK + j0);
  }
  // The norm's inputs of this wave's positions (w, w + 8), requested now.
  float2 zr[MAXB / RW] = {}, wn2 = {0.f, 0.f};
  if (B > 0) {
    wn2 = *(const float2 *)(p.wn + 2 * lane);
#pragma unroll
    for (int u = 0; u < MAXB / RW; ++u) {
      const int b = wave + RW * u;
      if (b < B) {
        zr[u].x = p.z[(size_t)b * p.zs + hv * DK + 2 * lane];
        zr[u].y = p.z[(size_t)b * p.zs + hv * DK + 2 * lane + 1];
      }
    }
  }

  auto stage = [&](int nb, int buf, bool fresh) {
    const float *xc = p.xc + (size_t)buf * xstride;
    float *gs = p.gates + (size_t)buf * gstride;
    const bool gw = wave == RW - 1 && lane < nb;   // the gates' lanes
    float g_in = 0.f, b_in = 0.f;
    if (gw) {
      g_in = fresh ? p.decay[(size_t)lane * p.gs + hv] : gs[((size_t)lane * 2 + 0) * p.nvh + hv];
      b_in = fresh ? p.beta[(size_t)lane * p.gs + hv] : gs[((size_t)lane * 2 + 1) * p.nvh + hv];
    }
    // q and k of key head hk, positions wave and wave + RW
    float qkr[MAXB / RW][4];
#pragma unroll
    for (int u = 0; u < MAXB / RW; ++u) {
      const int b = min(wave + RW * u, nb - 1);
      const float *xq = xc + (size_t)b * p.C + hk * DK;
      const float *xk = xc + (size_t)b * p.C + (p.nkh + hk) * DK;
      qkr[u][0] = xq[lane]; qkr[u][1] = xq[lane + 64];
      qkr[u][2] = xk[lane]; qkr[u][3] = xk[lane + 64];
    }
    // v: this wave's COLS columns, 8 positions per group, 2 values per lane
    float vr[MAXB / 8][2];
#pragma unroll
    for (int h = 0; h < MAXB / 8; ++h)
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int e = lane + 64 * i, b = min(8 * h + e / COLS, nb - 1);
        vr[h][i] = xc[(size_t)b * p.C + 2 * p.nkh * DK + hv * DK + slice * COLS + e % COLS];
      }
#pragma unroll
    for (int u = 0; u < MAXB / RW; ++u) {   // l2 norms (run.c:401-423)
      const int b = wave + RW * u;
      if (b < nb) {
        const float rq = 1.f / sqrtf(sum64(qkr[u][0] * qkr[u][0]) + sum64(qkr[u][1] * qkr[u][1]) + 1e-6f);
        const float rk = 1.f / sqrtf(sum64(qkr[u][2] * qkr[u][2]) + sum64(qkr[u][3] * qkr[u][3]) + 1e-6f);
        qk[b][lane] = qkr[u][0] * rq; qk[b][lane + 64] = qkr[u][1] * rq;
        qk[b][DK + lane] = qkr[u][2] * rk; qk[b][DK + lane + 64] = qkr[u][3] * rk;
      }
    }
#pragma unroll
    for (int h = 0; h < MAXB / 8; ++h)
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int e = lane + 64 * i, b = 8 * h + e / COLS;
        if (b < nb) vs[b][slice * COLS + e % COLS] = vr[h][i];
      }
    if (gw) {
      float g = g_in, bt = b_in;
      if (fresh) {
        float dec = g_in;
        if (p.A) {  // run.c:2697-2698 (softplus, sigmoid: run.c:392-399)
          const float x = dec + p.dt[hv];
          dec = p.A[hv] * (x > 20.f ? x : logf(1.f + expf(x)));
          bt = 1.f / (1.f + expf(-bt));
        }
        g = expf(dec);
        gs[((size_t)lane * 2 + 0) * p.nvh + hv] = g;
        gs[((size_t)lane * 2 + 1) * p.nvh + hv] = bt;
      }
      s_g[lane] = g;
      s_beta[lane] = bt;
    }
    __syncthreads();
  };

  const float scale = 1.f / sqrtf((float)DK);
  auto run = [&](int nb, bool emit) {
    for (int b = 0; b < nb; ++b) {
      const float g = s_g[b], beta = s_beta[b];
      const float4 qa = *(const float4 *)&qk[b][i0], qb = *(const float4 *)&qk[b][i0 + 4];
      const float4 ka = *(const float4 *)&qk[b][DK + i0], kb = *(const float4 *)&qk[b][DK + i0 + 4];
      const float kr[8] = {ka.x, ka.y, ka.z, ka.w, kb.x, kb.y, kb.z, kb.w};
      const float qr[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
      float4 sk = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        s[r].x *= g; s[r].y *= g; s[r].z *= g; s[r].w *= g;
        sk.x = fmaf(s[r].x, kr[r], sk.x); sk.y = fmaf(s[r].y, kr[r], sk.y);
        sk.z = fmaf(s[r].z, kr[r], sk.z); sk.w = fmaf(s[r].w, kr[r], sk.w);
      }
      sk = (float4){sum16(sk.x), sum16(sk.y), sum16(sk.z), sum16(sk.w)};
      const float4 v4 = *(const float4 *)&vs[b][j0];
      const float4 dl = {beta * (v4.x - sk.x), beta * (v4.y - sk.y), beta * (v4.z - sk.z), beta * (v4.w - sk.w)};
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        s[r].x = fmaf(kr[r], dl.x, s[r].x); s[r].y = fmaf(kr[r], dl.y, s[r].y);
        s[r].z = fmaf(kr[r], dl.z, s[r].z); s[r].w = fmaf(kr[r], dl.w, s[r].w);
      }
      if (emit) {
        float4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          o.x = fmaf(s[r].x, qr[r], o.x); o.y = fmaf(s[r].y, qr[r], o.y);
          o.z = fmaf(s[r].z, qr[r], o.z); o.w = fmaf(s[r].w, qr[r], o.w);
        }
        o = (float4){sum16(o.x) * scale, sum16(o.y) * scale, sum16(o.z) * scale, sum16(o.w) * scale};
        if (rg == 0) *(float4 *)&ob[b][j0] = o;
      }
    }
  };
  auto store = [&](float *S) {
    float *So = S + (size_t)hv * DK * DK;
#pragma unroll
    for (int r = 0; r < 8; ++r) *(float4 *)(So + (size_t)(i0 + r) * DK + j0) = s[r];
  };

  if (L > 0) {  // the previous block's accepted prefix
    stage(L, Pr, false);
    run(L, false);
    if (peek) {
      store(p.S_peek);
      return;
    }
    store(p.S_base + (size_t)X * p.s_floats);
    __syncthreads();
  } else if (peek) {
    store(p.S_peek);
    return;
  }
  stage(B, P, true);
  run(B, true);
  store(p.S_base + (size_t)(X ^ 1) * p.s_floats);
  __syncthreads();
  // gated RMSNorm of positions wave and wave + RW: out = wn * o * (1 / sqrt(mean(o^2) + 1e-6)) * silu(z)
#pragma unroll
  for (int u = 0; u < MAXB / RW; ++u) {
    const int b = wave + RW * u;
    if (b >= B) break;
    const float2 o = *(const float2 *)&ob[b][2 * lane];
    const float ss = sum64(o.x * o.x + o.y * o.y);
    const float sc = 1.f / sqrtf(ss / DK + 1e-6f);
    float2 r;
    r.x = wn2.x * o.x * sc * silu_ref(zr[u].x);
    r.y = wn2.y * o.y * sc * silu_ref(zr[u].y);
    if (p.out) *(float2 *)(p.out + (size_t)b * p.os + hv * DK + 2 * lane) = r;
    if (p.outh) {
      const half2_t h = {(_Float16)r.x, (_Float16)r.y};
      *(half2_t *)(p.outh + (size_t)b * p.ohs + hv * DK + 2 * lane) = h;
      if (f16_bad(h[0]) || f16_bad(h[1])) raise_flag(p.rflag);
    }
  }
}

}  // namespace

static void fill_params(GdnParams &p, const cwen_gdn *g) {
  p.s_floats = (size_t)g->nvh * DK * DK;
  p.h_floats = (size_t)g->C * 3;
  p.S_base = g->S;
  p.H_slots = g->H;
  p.ctl = g->ctl;
  p.nslot = g->nslot;
  p.force_L0 = 0;
  p.S_peek = nullptr;
  p.peek_L = p.peek_buf = 0;
  p.rflag = nullptr;
  p.xc = g->xc; p.gates = g->gates;
  p.nkh = g->nkh; p.nvh = g->nvh; p.C = g->C;
}

void gdn_conv_out(const cwen_gdn *g, const float *kw, GemvOut &o) {
  o.cv_w = kw;
  o.cv_H = g->H;
  o.cv_xc = g->xc;
  o.cv_ctl = g->ctl;
  o.cv_C = g->C;
  o.cv_nslot = g->nslot;
}

int gdn_block_launch(const cwen_gdn *g, const float *qkv, int qs, const float *z, int zs,
                     const float *decay, const float *beta, int gs, const float *kw, const float *wn,
                     float *out, int os, int B, hipStream_t st, _Float16 *outh, int ohs, const float *A,
                     const float *dt, int force_L0, int *rflag, bool conv_done) {
  GdnParams p;
  fill_params(p, g);
  p.force_L0 = force_L0;
  p.qkv = qkv; p.qs = qs;
  p.z = z; p.zs = zs;
  p.decay = decay; p.beta = beta; p.gs = gs;
  p.kw = kw; p.wn = wn;
  p.out = out; p.os = os;
  p.outh = outh; p.ohs = ohs;
  p.rflag = rflag;
  p.A = A; p.dt = dt;
  p.B = B;
  if (!conv_done)
    hipLaunchKernelGGL(gdn_conv_kernel, dim3((unsigned)((g->C + 255) / 256), (unsigned)B), dim3(256), 0, st, p);
  hipLaunchKernelGGL(gdn_rec_kernel, dim3((unsigned)g->nvh), dim3(64 * RW), 0, st, p);
  CWEN_HIP_TRY(hipGetLastError());
  return CWEN_OK;
}

int gdn_peek_launch(const cwen_gdn *g, int L, int buf, float *S_out, hipStream_t st) {
  GdnParams p;
  fill_params(p, g);
  p.S_peek = S_out;
  p.peek_L = L;
  p.peek_buf = buf;
  p.qkv = nullptr; p.qs = 0; p.z = nullptr; p.zs = 0; p.decay = p.beta = nullptr; p.gs = 0;
  p.kw = p.wn = nullptr; p.out = nullptr; p.os = 0; p.outh = nullptr; p.ohs = 0; p.A = p.dt = nullptr;
  p.B = 0;
  hipLaunchKernelGGL(gdn_rec_kernel, dim3((unsigned)g->nvh), dim3(64 * RW), 0, st, p);
  CWEN_HIP_TRY(hipGetLastError());
  return CWEN_OK;
}
