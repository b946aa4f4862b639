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
// Design (gfx950): one workgroup per value head, 256 threads; thread t owns
// column j = t/2 and rows 64*(t&1) .. +63 of the head's 128 x 128 state in 64
// VGPRs for the whole block.  The delta rule is column-local (sk[j], delta[j]
// and o[j] read only column j), so a position costs two lane shuffles and one
// block-wide sum (the RMSNorm).  Inputs of all B positions are staged in LDS
// up front.  After each position the state is stored to snapshot slot
// (cur + 1 + b) mod NSLOT, the conv history likewise, so accepting the first
// n positions is the host-side move cur += n: rollback reads nothing.
#include "cwen_internal.h"

namespace {

constexpr int DK = 128;
constexpr int THREADS = 256;
constexpr int MAXB = CWEN_BMAX;

struct GdnParams {
  const float *S_in;     // state slot read [nvh][DK][DK]
  float *S_slots;        // slot ring base
  const float *H_in;     // conv history slot read [C][3]
  float *H_slots;
  size_t s_floats, h_floats;  // floats per slot
  int cur, nslot;
  const float *qkv; int qs;   // raw (pre-conv) qkv [B][qs]
  const float *z; int zs;     // [B][zs]
  const float *decay, *beta; int gs;  // [B][gs]
  const float *kw;            // conv weights [C][4]
  const float *wn;            // gated-norm weight [DK]
  float *out; int os;         // [B][os]
  int nkh, nvh, C, B;
};

__device__ __forceinline__ float silu_ref(float x) { return x * (1.f / (1.f + expf(-x))); }

__global__ __launch_bounds__(THREADS) void gdn_block_kernel(GdnParams p) {
  // post-conv inputs of this head for every position: q | k | v, then z
  __shared__ float xin[MAXB][3 * DK];
  __shared__ float zin[MAXB][DK];
  __shared__ float red[THREADS / 64];
  const int tid = threadIdx.x;
  const int hv = blockIdx.x;
  const int hk = hv % p.nkh;
  const int B = p.B;

  // ---- conv over the B positions for the head's q, k, v channels.
  // Local channel lc: 0..127 q of key head hk, 128..255 k, 256..383 v of hv.
  // The q/k channels of key head hk are shared by nvh/nkh value heads; the
  // one with hv == hk owns their history.
  for (int lc = tid; lc < 3 * DK; lc += THREADS) {
    const int part = lc / DK, i = lc % DK;
    const int c = part == 0 ? hk * DK + i : part == 1 ? (p.nkh + hk) * DK + i : 2 * p.nkh * DK + hv * DK + i;
    const bool owner = part == 2 || hv == hk;
    const float w0 = p.kw[(size_t)c * 4 + 0], w1 = p.kw[(size_t)c * 4 + 1];
    const float w2 = p.kw[(size_t)c * 4 + 2], w3 = p.kw[(size_t)c * 4 + 3];
    float h0 = p.H_in[(size_t)c * 3 + 0], h1 = p.H_in[(size_t)c * 3 + 1], h2 = p.H_in[(size_t)c * 3 + 2];
    for (int b = 0; b < B; ++b) {
      const float cur = p.qkv[(size_t)b * p.qs + c];
      // ((st0*w0 + st1*w1) + st2*w2) + cur*w3, each product and sum rounded
      const float x = __fadd_rn(__fadd_rn(__fadd_rn(__fmul_rn(h0, w0), __fmul_rn(h1, w1)), __fmul_rn(h2, w2)),
                                __fmul_rn(cur, w3));
      h0 = h1; h1 = h2; h2 = cur;
      xin[b][lc] = silu_ref(x);
      if (owner) {
        float *hs = p.H_slots + (size_t)((p.cur + 1 + b) % p.nslot) * p.h_floats + (size_t)c * 3;
        hs[0] = h0; hs[1] = h1; hs[2] = h2;
      }
    }
  }
  for (int e = tid; e < B * DK; e += THREADS) zin[e / DK][e % DK] = p.z[(size_t)(e / DK) * p.zs + hv * DK + e % DK];
  __syncthreads();

  // ---- l2norm of q and k per position: wave w takes positions w, w+4, ...
  {
    const int wave = tid >> 6, lane = tid & 63;
    for (int b = wave; b < B; b += THREADS / 64) {
#pragma unroll
      for (int part = 0; part < 2; ++part) {
        float *x = &xin[b][part * DK];
        const float a = x[lane], c = x[lane + 64];
        float ss = a * a + c * c;
#pragma unroll
        for (int sh = 32; sh > 0; sh >>= 1) ss += __shfl_xor(ss, sh);
        const float s = 1.f / sqrtf(ss + 1e-6f);
        x[lane] = a * s;
        x[lane + 64] = c * s;
      }
    }
  }
  __syncthreads();

  // ---- the recurrence, state in registers
  const int j = tid >> 1, hh = tid & 1;
  const int i0 = hh * 64;
  const float *Sh = p.S_in + (size_t)hv * DK * DK;
  float s[64];
#pragma unroll
  for (int r = 0; r < 64; ++r) s[r] = Sh[(size_t)(i0 + r) * DK + j];
  const float scale = 1.f / sqrtf((float)DK);
  const float wnj = p.wn[j];

  for (int b = 0; b < B; ++b) {
    const float g = expf(p.decay[(size_t)b * p.gs + hv]);
    const float beta = p.beta[(size_t)b * p.gs + hv];
    const float *q = &xin[b][0], *k = &xin[b][DK];
    const float vj = xin[b][2 * DK + j];
    float sk = 0.f;
#pragma unroll
    for (int r = 0; r < 64; ++r) {
      s[r] *= g;
      sk = fmaf(s[r], k[i0 + r], sk);
    }
    sk += __shfl_xor(sk, 1);
    const float delta = beta * (vj - sk);
    float o = 0.f;
#pragma unroll
    for (int r = 0; r < 64; ++r) {
      s[r] = fmaf(k[i0 + r], delta, s[r]);
      o = fmaf(s[r], q[i0 + r], o);
    }
    o += __shfl_xor(o, 1);
    o *= scale;
    // snapshot after this position
    float *So = p.S_slots + (size_t)((p.cur + 1 + b) % p.nslot) * p.s_floats + (size_t)hv * DK * DK;
#pragma unroll
    for (int r = 0; r < 64; ++r) So[(size_t)(i0 + r) * DK + j] = s[r];
    // gated RMSNorm over the head's 128 outputs (each column held twice)
    float ss = hh == 0 ? o * o : 0.f;
#pragma unroll
    for (int sh = 32; sh > 0; sh >>= 1) ss += __shfl_xor(ss, sh);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    const float tot = red[0] + red[1] + red[2] + red[3];
    __syncthreads();
    const float sc = 1.f / sqrtf(tot / DK + 1e-6f);
    if (hh == 0) {
      const float zj = zin[b][j];
      p.out[(size_t)b * p.os + hv * DK + j] = wnj * o * sc * silu_ref(zj);
    }
  }
}

}  // namespace

int gdn_block_launch(const cwen_gdn *g, const float *qkv, int qs, const float *z, int zs,
                     const float *decay, const float *beta, int gs, const float *kw, const float *wn,
                     float *out, int os, int B, hipStream_t st) {
  GdnParams p;
  p.s_floats = (size_t)g->nvh * DK * DK;
  p.h_floats = (size_t)g->C * 3;
  p.S_slots = g->S;
  p.H_slots = g->H;
  p.S_in = g->S + (size_t)g->cur * p.s_floats;
  p.H_in = g->H + (size_t)g->cur * p.h_floats;
  p.cur = g->cur;
  p.nslot = g->nslot;
  p.qkv = qkv; p.qs = qs;
  p.z = z; p.zs = zs;
  p.decay = decay; p.beta = beta; p.gs = gs;
  p.kw = kw; p.wn = wn;
  p.out = out; p.os = os;
  p.nkh = g->nkh; p.nvh = g->nvh; p.C = g->C; p.B = B;
  hipLaunchKernelGGL(gdn_block_kernel, dim3((unsigned)g->nvh), dim3(THREADS), 0, st, p);
  CWEN_HIP_TRY(hipGetLastError());
  return CWEN_OK;
}
