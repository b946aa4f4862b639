// Q4_0 batched GEMV for a verify block of B = 1..16 activation columns.
//
// Reference semantics: gemvb / dot_q4_bcol / dot_q4_0rsi_2mat / mlp_blk
// (run.c:1529-1680, 886-975, 2677-2683): Y[b][i] = sum_k (n_ik - 8) * d_i,blk(k) * X[b][k].
//
// Design (gfx950):
//  * Weights are repacked once at upload into 1152-byte tiles (16 rows x 128 K)
//    laid out in MFMA operand order, so a wave streams each tile with one
//    coalesced 16-byte load per lane and no cross-lane shuffles.
//  * Nibbles become exact f16 values (n - 8) with two magic-exponent ops per
//    pair; the block's f16 scale is applied in f32 after the MFMA, so the
//    only rounding beyond f32 accumulation is the f16 activation operand.
//  * v_mfma_f32_16x16x32_f16: A = activations (16 columns x 32 K, one Q4
//    block), B = weights (32 K x 16 rows).  Columns >= B are zero operands,
//    so one kernel serves B = 1..16 and each column's arithmetic is the same
//    whatever B is (block verify == serial decode, bit for bit).
//  * A workgroup of 4 waves owns 4 row groups (64 rows) and one K range; the
//    activation chunk is staged once in LDS (f32 -> f16) and shared by all
//    4 waves.  Long K ranges are split across workgroups; the last
//    workgroup of a row tile sums the partials in fixed split order, so the
//    result is deterministic.
#include "cwen_internal.h"

namespace {

constexpr int WAVES = 4;
constexpr int CH = 4;  // K tiles per LDS chunk == weight prefetch depth

// Nibble position holding operand element e (see unpack8): unpack8 yields
// elements in nibble order 0,4,1,5,2,6,3,7.
__constant__ int kNibPos[8] = {0, 4, 1, 5, 2, 6, 3, 7};

// 8 nibbles -> 8 exact f16 values (n - 8), element e taken from nibble kNibPos[e].
__device__ __forceinline__ half8_t unpack8(uint32_t q) {
  const uint32_t q2 = q >> 8;
  const uint32_t t0 = (q & 0x000F000Fu) | 0x64006400u;   // 1024 + n0, 1024 + n4
  const uint32_t t1 = (q & 0x00F000F0u) | 0x64006400u;   // 1024 + 16 n1, 1024 + 16 n5
  const uint32_t t2 = (q2 & 0x000F000Fu) | 0x64006400u;  // 1024 + n2, 1024 + n6
  const uint32_t t3 = (q2 & 0x00F000F0u) | 0x64006400u;  // 1024 + 16 n3, 1024 + 16 n7
  const half2_t k1032 = {(_Float16)1032.0f, (_Float16)1032.0f};
  const half2_t k16 = {(_Float16)0.0625f, (_Float16)0.0625f};
  const half2_t k72 = {(_Float16)-72.0f, (_Float16)-72.0f};
  const half2_t h0 = __builtin_bit_cast(half2_t, t0) - k1032;
  const half2_t h1 = __builtin_elementwise_fma(__builtin_bit_cast(half2_t, t1), k16, k72);
  const half2_t h2 = __builtin_bit_cast(half2_t, t2) - k1032;
  const half2_t h3 = __builtin_elementwise_fma(__builtin_bit_cast(half2_t, t3), k16, k72);
  half8_t r;
  r[0] = h0[0]; r[1] = h0[1]; r[2] = h1[0]; r[3] = h1[1];
  r[4] = h2[0]; r[5] = h2[1]; r[6] = h3[0]; r[7] = h3[1];
  return r;
}

__device__ __forceinline__ float h2f(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

__device__ __forceinline__ float silu_f(float x) { return x * (1.f / (1.f + expf(-x))); }

struct Q4Params {
  const uint8_t *w;   // tiled weights
  int nsw;            // sides stored per tile position (1 or 2)
  int side0;          // first side computed
  int M, nrg, nkt;
  const float *X;
  int xs, B;
  float *Y0, *Y1;
  int ys;
  int S, tps;         // split-K
  float *part;
  int *cnt;
};

template <int NS, int EPI>
__global__ __launch_bounds__(256) void q4_gemv_kernel(Q4Params p) {
  __shared__ uint4 act[CH * 4 * 64];  // [tile][block][lane] f16 x 8
  __shared__ int s_last;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int n = lane & 15, g = lane >> 4;
  const int rt = blockIdx.x / p.S;
  const int sp = blockIdx.x - rt * p.S;
  const int rg = rt * WAVES + wave;
  const bool rows_on = rg < p.nrg;
  const int kt0 = sp * p.tps;
  const int nt = min(p.nkt, kt0 + p.tps) - kt0;
  const bool act_on = n < p.B;

  const size_t tstride = (size_t)p.nsw * Q4_TILE_BYTES;
  const uint8_t *wb[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s)
    wb[s] = p.w + (((size_t)(rows_on ? rg : 0) * p.nkt + kt0) * p.nsw + p.side0 + s) * Q4_TILE_BYTES;

  uint4 wq[CH][NS];
  uint2 wsc[CH][NS];
#pragma unroll
  for (int i = 0; i < CH; ++i)
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      if (rows_on && i < nt) {
        const uint8_t *t = wb[s] + (size_t)i * tstride;
        wq[i][s] = *(const uint4 *)(t + lane * 16);
        wsc[i][s] = *(const uint2 *)(t + Q4_TILE_QS + n * 8);
      } else {
        wq[i][s] = make_uint4(0, 0, 0, 0);
        wsc[i][s] = make_uint2(0, 0);
      }
    }

  floatx4_t acc[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) acc[s] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
  const floatx4_t zero4 = {0.f, 0.f, 0.f, 0.f};

  for (int ch0 = 0; ch0 < nt; ch0 += CH) {
    const int chn = min(CH, nt - ch0);
    __syncthreads();
    // Stage X[b][k] for this chunk as f16 MFMA A-operands: slot (tile, block, g, c).
    {
      const int nslot = chn * 16 * p.B;
      for (int i = tid; i < nslot; i += 256) {
        const int gg = i & 3, m = (i >> 2) & 3;
        const int rest = i >> 4;
        const int tt = rest % chn, c = rest / chn;
        const int k0 = ((kt0 + ch0 + tt) * 4 + m) * 32 + gg * 8;
        const float4 *src = (const float4 *)(p.X + (size_t)c * p.xs + k0);
        const float4 v0 = src[0], v1 = src[1];
        half8_t h;
        h[0] = (_Float16)v0.x; h[1] = (_Float16)v0.y; h[2] = (_Float16)v0.z; h[3] = (_Float16)v0.w;
        h[4] = (_Float16)v1.x; h[5] = (_Float16)v1.y; h[6] = (_Float16)v1.z; h[7] = (_Float16)v1.w;
        act[(tt * 4 + m) * 64 + gg * 16 + c] = __builtin_bit_cast(uint4, h);
      }
    }
    __syncthreads();
    if (!rows_on) continue;
#pragma unroll
    for (int tt = 0; tt < CH; ++tt) {
      if (tt < chn) {
        uint4 q[NS];
        uint2 sc[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s) { q[s] = wq[tt][s]; sc[s] = wsc[tt][s]; }
        const int tn = ch0 + tt + CH;
        if (tn < nt) {
#pragma unroll
          for (int s = 0; s < NS; ++s) {
            const uint8_t *t = wb[s] + (size_t)tn * tstride;
            wq[tt][s] = *(const uint4 *)(t + lane * 16);
            wsc[tt][s] = *(const uint2 *)(t + Q4_TILE_QS + n * 8);
          }
        }
        half8_t a[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          if (act_on) a[m] = __builtin_bit_cast(half8_t, act[(tt * 4 + m) * 64 + lane]);
          else a[m] = (half8_t){0, 0, 0, 0, 0, 0, 0, 0};
        }
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          const uint32_t qd[4] = {q[s].x, q[s].y, q[s].z, q[s].w};
          const float d[4] = {h2f(sc[s].x & 0xffffu), h2f(sc[s].x >> 16),
                              h2f(sc[s].y & 0xffffu), h2f(sc[s].y >> 16)};
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            const floatx4_t pm = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[m], unpack8(qd[m]), zero4, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[s][r] = __builtin_fmaf(pm[r], d[m], acc[s][r]);
          }
        }
      }
    }
  }

  // Split-K: publish partials; the last workgroup of this row tile reduces in split order.
  if (p.S > 1) {
    if (rows_on) {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        float *dst = p.part + ((((size_t)rg * p.S + sp) * NS + s) * 64 + lane) * 4;
        *(floatx4_t *)dst = acc[s];
      }
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) s_last = (atomicAdd(&p.cnt[rt], 1) == p.S - 1);
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    if (rows_on) {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        floatx4_t sum = *(volatile floatx4_t *)(p.part + ((((size_t)rg * p.S + 0) * NS + s) * 64 + lane) * 4);
        for (int k = 1; k < p.S; ++k) {
          const floatx4_t v =
              *(volatile floatx4_t *)(p.part + ((((size_t)rg * p.S + k) * NS + s) * 64 + lane) * 4);
          sum += v;
        }
        acc[s] = sum;
      }
    }
    if (tid == 0) p.cnt[rt] = 0;
  }

  if (!rows_on) return;
  const int row = rg * Q4_ROWS + n;
  if (row >= p.M) return;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int c = g * 4 + r;
    if (c < p.B) {
      if (EPI == Q4_EPI_SWIGLU) {
        p.Y0[(size_t)c * p.ys + row] = silu_f(acc[0][r]) * acc[NS - 1][r];
      } else {
        p.Y0[(size_t)c * p.ys + row] = acc[0][r];
        if (NS == 2) p.Y1[(size_t)c * p.ys + row] = acc[NS - 1][r];
      }
    }
  }
}

// One thread per (row group, K tile, side, lane): builds the lane's 16 nibble
// bytes and, for lanes 0..15, the row's 4 block scales.
__global__ void q4_repack_kernel(uint8_t *dst, const uint8_t *src, const uint16_t *sc, int type,
                                 int M, int K, int nrg, int nkt, int nsw) {
  const size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t total = (size_t)nrg * nkt * nsw * 64;
  if (id >= total) return;
  const int lane = (int)(id & 63);
  size_t t = id >> 6;
  const int side = (int)(t % nsw); t /= nsw;
  const int kt = (int)(t % nkt);
  const int rg = (int)(t / nkt);
  const int n = lane & 15, g = lane >> 4;
  const int row = rg * Q4_ROWS + n;
  const int nb = K / 32;
  uint8_t *tile = dst + (((size_t)rg * nkt + kt) * nsw + side) * Q4_TILE_BYTES;
  uint32_t out[4];
  uint16_t scl[4];
  for (int m = 0; m < 4; ++m) {
    const int blk = kt * 4 + m;
    const uint8_t *qs;
    uint16_t d;
    if (row < M) {
      const size_t bi = (size_t)row * nb + blk;
      if (type == CWEN_T_Q4_0) {
        const uint8_t *b = src + bi * 18;
        d = (uint16_t)(b[0] | (b[1] << 8));
        qs = b + 2;
      } else if (type == CWEN_T_Q4_0RS) {
        qs = src + bi * 16;
        d = sc[bi];
      } else {  // Q4_0RSI
        qs = src + bi * 32 + side * 16;
        d = sc[bi * 2 + side];
      }
    } else {
      qs = nullptr;
      d = 0;
    }
    uint32_t word = 0;
    for (int e = 0; e < 8; ++e) {
      const int k = g * 8 + e;
      uint32_t nib = 8;
      if (qs) nib = (k < 16) ? (qs[k] & 0xFu) : (qs[k - 16] >> 4);
      word |= nib << (4 * kNibPos[e]);
    }
    out[m] = word;
    scl[m] = d;
  }
  *(uint4 *)(tile + lane * 16) = make_uint4(out[0], out[1], out[2], out[3]);
  if (g == 0) {
    uint16_t *s = (uint16_t *)(tile + Q4_TILE_QS + n * 8);
    for (int m = 0; m < 4; ++m) s[m] = scl[m];
  }
}

}  // namespace

int q4_repack(cwen_weight *w, const uint8_t *dsrc, const uint16_t *dsc, hipStream_t st) {
  const size_t threads = (size_t)w->nrg * w->nkt * w->nside * 64;
  const int blk = 256;
  const size_t grid = (threads + blk - 1) / blk;
  hipLaunchKernelGGL(q4_repack_kernel, dim3((unsigned)grid), dim3(blk), 0, st, w->dev, dsrc, dsc,
                     w->type, w->ne1, w->ne0, w->nrg, w->nkt, w->nside);
  CWEN_HIP_TRY(hipGetLastError());
  return CWEN_OK;
}

// Split-K choice depends on the shape only (never on B), so every column of
// every call on this weight uses the same reduction tree.
void q4_choose_split(const cwen_ctx *ctx, cwen_weight *w) {
  const int nrt = (w->nrg + WAVES - 1) / WAVES;
  int S = (ctx->wg_target + nrt / 2) / nrt;
  const int smax = w->nkt / 4 > 1 ? w->nkt / 4 : 1;
  if (S < 1) S = 1;
  if (S > smax) S = smax;
  const int tps = (w->nkt + S - 1) / S;
  w->tps = tps;
  w->split = (w->nkt + tps - 1) / tps;
}

int q4_gemv_launch(cwen_ctx *ctx, const cwen_weight *w, int nsides, int side0, int epi,
                   const float *X, int xs, float *Y0, float *Y1, int ys, int B,
                   hipStream_t st) {
  Q4Params p;
  p.w = w->dev;
  p.nsw = w->nside;
  p.side0 = side0;
  p.M = w->ne1;
  p.nrg = w->nrg;
  p.nkt = w->nkt;
  p.X = X;
  p.xs = xs;
  p.B = B;
  p.Y0 = Y0;
  p.Y1 = Y1;
  p.ys = ys;
  p.S = w->split;
  p.tps = w->tps;
  p.part = ctx->partials;
  p.cnt = ctx->counters;
  const int nrt = (w->nrg + WAVES - 1) / WAVES;
  if (p.S > 1) {
    const size_t need = (size_t)nrt * WAVES * p.S * nsides * 256;
    if (need > ctx->partials_floats || nrt > ctx->ncounters) return CWEN_ESCRATCH;
  }
  const dim3 grid((unsigned)(nrt * p.S)), block(256);
  if (nsides == 1 && epi == Q4_EPI_STORE)
    hipLaunchKernelGGL((q4_gemv_kernel<1, Q4_EPI_STORE>), grid, block, 0, st, p);
  else if (nsides == 2 && epi == Q4_EPI_STORE)
    hipLaunchKernelGGL((q4_gemv_kernel<2, Q4_EPI_STORE>), grid, block, 0, st, p);
  else if (nsides == 2 && epi == Q4_EPI_SWIGLU)
    hipLaunchKernelGGL((q4_gemv_kernel<2, Q4_EPI_SWIGLU>), grid, block, 0, st, p);
  else
    return CWEN_EINVAL;
  CWEN_HIP_TRY(hipGetLastError());
  return CWEN_OK;
}
