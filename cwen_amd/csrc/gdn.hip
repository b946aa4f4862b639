// GatedDeltaNet block verify: the depthwise causal conv and the gated delta
// rule across the B positions of a draft block, with the recurrent state and
// the conv history snapshotted in HBM after every position.
//
// Reference semantics (run.c): conv1d_update 2183-2200, gdn_step 2014-2180
// (+ l2norm_rows 401-423), as called position by position in
// layer_linear_blk 2700-2704; snap_save / snap_load 2787-2809 and the
// short-walk replay 4975-4988 are replaced by the snapshot ring.
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
// Design (gfx950): three launches on the caller's stream.
//  1. conv: one thread per channel runs the B positions in order, writes the
//     post-SiLU values to scratch and the history after every position to
//     the snapshot ring.
//  2. recurrence: the delta rule is column-local (sk[j], delta[j] and o[j]
//     read only column j), so a head's 128 columns split over 8 single-wave
//     workgroups of 16 columns; 384 workgroups keep the per-position state
//     snapshot (3 MB per position) spread over the whole chip.  A lane owns a
//     4-column x 8-row block in registers for the whole block; a column sum
//     is a 16-lane DPP reduction.  The state after each position is stored
//     to snapshot slot (cur + 1 + b) mod NSLOT.
//  3. norm: one wave per (position, value head) applies the gated RMSNorm.
// Accepting the first n positions is then the host-side move cur += n:
// rollback reads nothing.  Every position runs the same instructions whatever
// B is, so a block of B equals B single-position blocks bit for bit.
#include "cwen_internal.h"

namespace {

constexpr int DK = 128;
constexpr int MAXB = CWEN_BMAX;
constexpr int COLS = 16;            // columns of a head per recurrence workgroup

__device__ __forceinline__ float silu_ref(float x) { return x * (1.f / (1.f + expf(-x))); }

// Slot ring: the state before the block is slot *cur; the state after
// position b is written to slot (*cur + 1 + b) % nslot.  The slot is read on
// the device, so a captured launch replays at any ring position.
struct GdnParams {
  float *S_slots;             // state ring [nslot][nvh][DK][DK]
  float *H_slots;             // conv history ring [nslot][C][3]
  size_t s_floats, h_floats;  // floats per slot
  const int *cur;             // device: current slot
  int nslot;
  const float *qkv; int qs;   // raw (pre-conv) qkv [B][qs]
  const float *z; int zs;     // [B][zs]
  const float *decay, *beta; int gs;  // [B][gs]
  const float *kw;            // conv weights [C][4]
  const float *wn;            // gated-norm weight [DK]
  float *out; int os;         // [B][os], nullable
  _Float16 *outh; int ohs;    // f16 copy [B][ohs], nullable
  const float *A, *dt;        // raw gates when non-null: decay = A*softplus(decay + dt), beta = sigmoid(beta)
  float *xc;                  // scratch: post-conv values [B][C]
  float *ob;                  // scratch: pre-norm outputs [B][nvh*DK]
  int nkh, nvh, C, B;
};

// 1. conv: thread = channel.  All loads of a channel are issued before its
// first use.
__global__ __launch_bounds__(256) void gdn_conv_kernel(GdnParams p) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= p.C) return;
  const int cur = *p.cur;
  const float *H_in = p.H_slots + (size_t)cur * p.h_floats;
  const float4 w = *(const float4 *)(p.kw + (size_t)c * 4);
  float h0 = H_in[(size_t)c * 3 + 0], h1 = H_in[(size_t)c * 3 + 1], h2 = H_in[(size_t)c * 3 + 2];
  float raw[MAXB];
#pragma unroll
  for (int b = 0; b < MAXB; ++b) raw[b] = b < p.B ? p.qkv[(size_t)b * p.qs + c] : 0.f;
#pragma unroll
  for (int b = 0; b < MAXB; ++b) {
    if (b >= p.B) break;
    const float xin = raw[b];
    // ((st0*w0 + st1*w1) + st2*w2) + xin*w3, each product and sum rounded
    const float x = __fadd_rn(__fadd_rn(__fadd_rn(__fmul_rn(h0, w.x), __fmul_rn(h1, w.y)), __fmul_rn(h2, w.z)),
                              __fmul_rn(xin, w.w));
    h0 = h1; h1 = h2; h2 = xin;
    p.xc[(size_t)b * p.C + c] = silu_ref(x);
    float *hs = p.H_slots + (size_t)((cur + 1 + b) % p.nslot) * p.h_floats + (size_t)c * 3;
    hs[0] = h0; hs[1] = h1; hs[2] = h2;
  }
}

// 2. recurrence: workgroup (hv, slice) = one wave, columns
// slice*16 .. slice*16+15 of head hv.  Lane: row group rg = lane & 15 (rows
// 8rg..8rg+7), column group cg = lane >> 4 (4 columns).
__global__ __launch_bounds__(64) void gdn_rec_kernel(GdnParams p) {
  __shared__ __align__(16) float qk[MAXB][2 * DK];   // normalised q | k per position
  __shared__ __align__(16) float vs[MAXB][COLS];
  __shared__ float s_g[MAXB], s_beta[MAXB];
  const int lane = threadIdx.x;
  const int hv = blockIdx.x / (DK / COLS);
  const int slice = blockIdx.x % (DK / COLS);
  const int hk = hv % p.nkh;
  const int B = p.B;
  const int cur = *p.cur;
  const int rg = lane & 15, cg = lane >> 4;
  const int i0 = rg * 8, j0 = slice * COLS + cg * 4;

  float4 s[8];
  {
    const float *Sh = p.S_slots + (size_t)cur * p.s_floats + (size_t)hv * DK * DK;
#pragma unroll
    for (int r = 0; r < 8; ++r) s[r] = *(const float4 *)(Sh + (size_t)(i0 + r) * DK + j0);
  }
  if (lane < B) {
    float dec = p.decay[(size_t)lane * p.gs + hv], bt = p.beta[(size_t)lane * p.gs + hv];
    if (p.A) {  // run.c:2697-2698 (softplus, sigmoid: run.c:392-399)
      const float x = dec + p.dt[hv];
      dec = p.A[hv] * (x > 20.f ? x : logf(1.f + expf(x)));
      bt = 1.f / (1.f + expf(-bt));
    }
    s_g[lane] = expf(dec);
    s_beta[lane] = bt;
  }
  for (int e = lane; e < B * COLS; e += 64)
    vs[e / COLS][e % COLS] = p.xc[(size_t)(e / COLS) * p.C + 2 * p.nkh * DK + hv * DK + slice * COLS + e % COLS];
  // q and k of key head hk, l2-normalised per position
  for (int b = 0; b < B; ++b) {
    const float *xq = p.xc + (size_t)b * p.C + hk * DK;
    const float *xk = p.xc + (size_t)b * p.C + (p.nkh + hk) * DK;
    const float q0 = xq[lane], q1 = xq[lane + 64], k0 = xk[lane], k1 = xk[lane + 64];
    const float sq = 1.f / sqrtf(sum64(q0 * q0 + q1 * q1) + 1e-6f);
    const float sk = 1.f / sqrtf(sum64(k0 * k0 + k1 * k1) + 1e-6f);
    qk[b][lane] = q0 * sq; qk[b][lane + 64] = q1 * sq;
    qk[b][DK + lane] = k0 * sk; qk[b][DK + lane + 64] = k1 * sk;
  }
  __syncthreads();

  const float scale = 1.f / sqrtf((float)DK);
  for (int b = 0; b < B; ++b) {
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
    const float4 v4 = *(const float4 *)&vs[b][cg * 4];
    const float4 dl = {beta * (v4.x - sk.x), beta * (v4.y - sk.y), beta * (v4.z - sk.z), beta * (v4.w - sk.w)};
    float4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      s[r].x = fmaf(kr[r], dl.x, s[r].x); s[r].y = fmaf(kr[r], dl.y, s[r].y);
      s[r].z = fmaf(kr[r], dl.z, s[r].z); s[r].w = fmaf(kr[r], dl.w, s[r].w);
      o.x = fmaf(s[r].x, qr[r], o.x); o.y = fmaf(s[r].y, qr[r], o.y);
      o.z = fmaf(s[r].z, qr[r], o.z); o.w = fmaf(s[r].w, qr[r], o.w);
    }
    o = (float4){sum16(o.x) * scale, sum16(o.y) * scale, sum16(o.z) * scale, sum16(o.w) * scale};
    float *So = p.S_slots + (size_t)((cur + 1 + b) % p.nslot) * p.s_floats + (size_t)hv * DK * DK;
#pragma unroll
    for (int r = 0; r < 8; ++r) *(float4 *)(So + (size_t)(i0 + r) * DK + j0) = s[r];
    if (rg == 0) *(float4 *)(p.ob + (size_t)b * p.nvh * DK + hv * DK + j0) = o;
  }
}

// 3. gated RMSNorm: one wave per (position, value head).
__global__ __launch_bounds__(64) void gdn_norm_kernel(GdnParams p) {
  const int b = blockIdx.x / p.nvh, hv = blockIdx.x % p.nvh;
  const int lane = threadIdx.x;
  const float2 o = *(const float2 *)(p.ob + (size_t)b * p.nvh * DK + hv * DK + 2 * lane);
  const float ss = sum64(o.x * o.x + o.y * o.y);
  const float sc = 1.f / sqrtf(ss / DK + 1e-6f);
  const float zx = p.z[(size_t)b * p.zs + hv * DK + 2 * lane], zy = p.z[(size_t)b * p.zs + hv * DK + 2 * lane + 1];
  const float2 w = *(const float2 *)(p.wn + 2 * lane);
  float2 r;
  r.x = w.x * o.x * sc * silu_ref(zx);
  r.y = w.y * o.y * sc * silu_ref(zy);
  if (p.out) *(float2 *)(p.out + (size_t)b * p.os + hv * DK + 2 * lane) = r;
  if (p.outh) {
    const half2_t h = {(_Float16)r.x, (_Float16)r.y};
    *(half2_t *)(p.outh + (size_t)b * p.ohs + hv * DK + 2 * lane) = h;
  }
}

}  // namespace

int gdn_block_launch(const cwen_gdn *g, const float *qkv, int qs, const float *z, int zs,
                     const float *decay, const float *beta, int gs, const float *kw, const float *wn,
                     float *out, int os, int B, hipStream_t st, _Float16 *outh, int ohs, const float *A,
                     const float *dt) {
  GdnParams p;
  p.s_floats = (size_t)g->nvh * DK * DK;
  p.h_floats = (size_t)g->C * 3;
  p.S_slots = g->S;
  p.H_slots = g->H;
  p.cur = g->dcur;
  p.nslot = g->nslot;
  p.qkv = qkv; p.qs = qs;
  p.z = z; p.zs = zs;
  p.decay = decay; p.beta = beta; p.gs = gs;
  p.kw = kw; p.wn = wn;
  p.out = out; p.os = os;
  p.outh = outh; p.ohs = ohs;
  p.A = A; p.dt = dt;
  p.xc = g->xc; p.ob = g->ob;
  p.nkh = g->nkh; p.nvh = g->nvh; p.C = g->C; p.B = B;
  hipLaunchKernelGGL(gdn_conv_kernel, dim3((unsigned)((g->C + 255) / 256)), dim3(256), 0, st, p);
  hipLaunchKernelGGL(gdn_rec_kernel, dim3((unsigned)(g->nvh * (DK / COLS))), dim3(64), 0, st, p);
  hipLaunchKernelGGL(gdn_norm_kernel, dim3((unsigned)(g->nvh * B)), dim3(64), 0, st, p);
  CWEN_HIP_TRY(hipGetLastError());
  return CWEN_OK;
}
