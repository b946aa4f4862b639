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
//    block), B = weights (32 K x 16 rows).  Activations are f16 row-major
//    [B][K]; a lane's A operand is 16 contiguous bytes of one column, read
//    straight from L2.  Columns >= B lie past the buffer range and load as
//    zeros, so one kernel serves B = 1..16 and a column's arithmetic never
//    depends on B (block verify == serial decode, bit for bit).
//  * One workgroup owns one 16-row group (both sides of an interleaved pair)
//    and all of K; its waves split K and the partial sums are reduced through
//    LDS in wave order.  There is no cross-workgroup synchronisation, and the
//    reduction tree depends on the shape only.
//  * Each wave keeps a ring of PF tiles in flight (weights + activation
//    operands) with unconditional, fixed-order buffer loads, so the in-order
//    load counter only waits for the tile being consumed.
#include "cwen_internal.h"

namespace {

constexpr int PF = 4;  // tiles in flight per wave

// Nibble position holding operand element e (see unpack8): unpack8 yields
// elements in nibble order 0,4,1,5,2,6,3,7.
__constant__ int kNibPos[8] = {0, 4, 1, 5, 2, 6, 3, 7};

// (q & mask) | magic in one VOP3 op.  gfx9 VOP3 takes no literal and reads at
// most one scalar, so the mask comes from an SGPR and the magic from a VGPR.
__device__ __forceinline__ uint32_t and_or(uint32_t q, uint32_t mask_s, uint32_t magic_v) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(q), "s"(mask_s), "v"(magic_v));
  return r;
}

// 8 nibbles -> 8 exact f16 values (n - 8), element e taken from nibble kNibPos[e].
struct Unpack {
  uint32_t lo, hi;   // SGPR masks 0x000F000F, 0x00F000F0
  uint32_t magic;    // VGPR 0x64006400
};
// Materialise the constants once, opaque to the compiler, so the loop does
// not rebuild them per use.
__device__ __forceinline__ Unpack unpack_consts() {
  Unpack u;
  asm volatile("s_mov_b32 %0, 0x000f000f" : "=s"(u.lo));
  asm volatile("s_mov_b32 %0, 0x00f000f0" : "=s"(u.hi));
  asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(u.magic));
  return u;
}

__device__ __forceinline__ half8_t unpack8(uint32_t q, const Unpack &u) {
  const uint32_t q2 = q >> 8;
  const uint32_t t0 = and_or(q, u.lo, u.magic);    // 1024 + n0, 1024 + n4
  const uint32_t t1 = and_or(q, u.hi, u.magic);    // 1024 + 16 n1, 1024 + 16 n5
  const uint32_t t2 = and_or(q2, u.lo, u.magic);   // 1024 + n2, 1024 + n6
  const uint32_t t3 = and_or(q2, u.hi, u.magic);   // 1024 + 16 n3, 1024 + 16 n7
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

struct Q4Params {
  const uint8_t *w;    // tiled weights
  uint32_t wbytes;     // bytes of the tiled weights (buffer range)
  int nsw;             // sides stored per tile position (1 or 2)
  int side0;           // first side computed
  int M, nkt;
  const _Float16 *xh;  // activations f16 [B][K]
  uint32_t xbytes;     // B*K*2 (buffer range: columns >= B read as zero)
  int B;
  Q4Out out;
};

template <int NS, int EPI, int W>
__global__ __launch_bounds__(64 * W) void q4_gemv_kernel(Q4Params p) {
  __shared__ floatx4_t red[W][NS][64];

  const int tid = threadIdx.x;
  // Wave index as a scalar: the K range and the loop trip count are then
  // provably wave-uniform, which keeps the loop's load-counter waits exact.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int n = lane & 15, g = lane >> 4;
  const int rg = blockIdx.x;
  const int t0 = (wave * p.nkt) / W;
  const int nt = ((wave + 1) * p.nkt) / W - t0;  // >= 1 (host keeps W <= nkt)

  const __amdgpu_buffer_rsrc_t wr = make_rsrc(p.w, p.wbytes);
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.xh, p.xbytes);

  const uint32_t tstride = (uint32_t)p.nsw * Q4_TILE_BYTES;
  uint32_t wofs[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s)
    wofs[s] = (((uint32_t)rg * p.nkt + t0) * p.nsw + p.side0 + s) * Q4_TILE_BYTES;
  const uint32_t lq = lane * 16, ls = Q4_TILE_QS + n * 8;
  // A operand of block m of tile t: column n, K run 32m + 8g .. +7.
  const uint32_t xlane = ((uint32_t)n * (uint32_t)(p.nkt * Q4_TILE_K) + t0 * Q4_TILE_K + g * 8) * 2;

  uint4 wq[PF][NS];
  uint2 wsc[PF][NS];
  uint4 xa[PF][4];
#pragma unroll
  for (int i = 0; i < PF; ++i) {
    const uint32_t t = (uint32_t)(i < nt ? i : nt - 1);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      wq[i][s] = bload16(wr, wofs[s] + t * tstride + lq);
      wsc[i][s] = bload8(wr, wofs[s] + t * tstride + ls);
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) xa[i][m] = bload16(xr, xlane + t * (Q4_TILE_K * 2) + m * 64);
    // Issue the ring in slot order: the loop consumes slot 0 first.
    __builtin_amdgcn_sched_barrier(0);
  }

  floatx4_t acc[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) acc[s] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
  const floatx4_t zero4 = {0.f, 0.f, 0.f, 0.f};

  const Unpack uc = unpack_consts();

  for (int tb = 0; tb < nt; tb += PF) {
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      // Ring overrun past this wave's range (last round only): loads still
      // issue (clamped) to keep the counter schedule fixed; compute is skipped.
      if (tb + j < nt) {
        half8_t b[NS][4];
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          b[s][0] = unpack8(wq[j][s].x, uc);
          b[s][1] = unpack8(wq[j][s].y, uc);
          b[s][2] = unpack8(wq[j][s].z, uc);
          b[s][3] = unpack8(wq[j][s].w, uc);
        }
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          const half2_t d01 = __builtin_bit_cast(half2_t, wsc[j][s].x);
          const half2_t d23 = __builtin_bit_cast(half2_t, wsc[j][s].y);
          const float d[4] = {(float)d01[0], (float)d01[1], (float)d23[0], (float)d23[1]};
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            const floatx4_t pm = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                __builtin_bit_cast(half8_t, xa[j][m]), b[s][m], zero4, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[s][r] = __builtin_fmaf(pm[r], d[m], acc[s][r]);
          }
        }
      }
      // Refill this slot only after its registers are consumed, so the new
      // loads can land in the same registers.
      {
        const int tn0 = tb + j + PF;
        const uint32_t tn = (uint32_t)(tn0 < nt ? tn0 : nt - 1);
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          wq[j][s] = bload16(wr, wofs[s] + tn * tstride + lq);
          wsc[j][s] = bload8(wr, wofs[s] + tn * tstride + ls);
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) xa[j][m] = bload16(xr, xlane + tn * (Q4_TILE_K * 2) + m * 64);
      }
      // Keep slots in issue order so a later slot's decode is not hoisted
      // above this slot's loads.
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // Fixed-order reduction of the waves' K-partials.
#pragma unroll
  for (int s = 0; s < NS; ++s) red[wave][s][lane] = acc[s];
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    floatx4_t v = red[0][s][lane];
#pragma unroll
    for (int w = 1; w < W; ++w) v += red[w][s][lane];
    acc[s] = v;
  }

  const int row = rg * Q4_ROWS + n;
  if (row >= p.M) return;
  const Q4Out &o = p.out;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int c = g * 4 + r;
    if (c >= p.B) continue;
    float v = (EPI == Q4_EPI_SWIGLU) ? silu_f(acc[0][r]) * acc[NS - 1][r] : acc[0][r];
    if (o.y) {
      float *dst = o.y + (size_t)c * o.ys + row;
      if (o.accumulate) v += *dst;
      *dst = v;
    }
    if (o.yh) o.yh[(size_t)c * p.M + row] = (_Float16)v;
    if (EPI == Q4_EPI_PAIR) o.y1[(size_t)c * o.ys + row] = acc[NS - 1][r];
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

template <int NS, int EPI>
int launch_w(const Q4Params &p, int waves, int nrg, hipStream_t st) {
  const dim3 grid((unsigned)nrg);
  switch (waves) {
    case 2: hipLaunchKernelGGL((q4_gemv_kernel<NS, EPI, 2>), grid, dim3(128), 0, st, p); break;
    case 4: hipLaunchKernelGGL((q4_gemv_kernel<NS, EPI, 4>), grid, dim3(256), 0, st, p); break;
    case 8: hipLaunchKernelGGL((q4_gemv_kernel<NS, EPI, 8>), grid, dim3(512), 0, st, p); break;
    default: return CWEN_EINVAL;
  }
  return CWEN_OK;
}

__global__ void act_to_f16_kernel(const float *x, int xs, _Float16 *xh, int K, int B) {
  const int k4 = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
  const int c = blockIdx.y;
  if (k4 >= K || c >= B) return;
  const float4 v = *(const float4 *)(x + (size_t)c * xs + k4);
  const half2_t a = {(_Float16)v.x, (_Float16)v.y}, b = {(_Float16)v.z, (_Float16)v.w};
  *(uint2 *)(xh + (size_t)c * K + k4) = make_uint2(__builtin_bit_cast(uint32_t, a),
                                                   __builtin_bit_cast(uint32_t, b));
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

// Waves per workgroup: enough row groups x waves to fill the chip while each
// wave keeps several K tiles.  Shape-only, so the reduction tree (and hence
// every output bit) never depends on B.
void q4_choose_split(const cwen_ctx *ctx, cwen_weight *w) {
  int waves = 2;
  while (waves < 8 && (long)w->nrg * waves < ctx->wg_target && w->nkt / (waves * 2) >= 4) waves *= 2;
  if (waves > w->nkt) waves = 2;
  w->split = waves;
  w->tps = (w->nkt + waves - 1) / waves;
}

int q4_gemv_launch(const cwen_weight *w, int nsides, int side0, int epi, const _Float16 *xh,
                   const Q4Out &out, int B, hipStream_t st) {
  Q4Params p;
  p.w = w->dev;
  p.wbytes = (uint32_t)w->bytes;
  p.nsw = w->nside;
  p.side0 = side0;
  p.M = w->ne1;
  p.nkt = w->nkt;
  p.xh = xh;
  p.xbytes = (uint32_t)((size_t)B * w->ne0 * 2);
  p.B = B;
  p.out = out;
  int rc;
  if (nsides == 1 && epi == Q4_EPI_STORE) rc = launch_w<1, Q4_EPI_STORE>(p, w->split, w->nrg, st);
  else if (nsides == 2 && epi == Q4_EPI_PAIR) rc = launch_w<2, Q4_EPI_PAIR>(p, w->split, w->nrg, st);
  else if (nsides == 2 && epi == Q4_EPI_SWIGLU) rc = launch_w<2, Q4_EPI_SWIGLU>(p, w->split, w->nrg, st);
  else return CWEN_EINVAL;
  if (rc) return rc;
  CWEN_HIP_TRY(hipGetLastError());
  return CWEN_OK;
}

int act_to_f16(const float *x, int xs, _Float16 *xh, int K, int B, hipStream_t st) {
  const int threads = 256;
  const dim3 grid((unsigned)((K / 4 + threads - 1) / threads), (unsigned)B);
  hipLaunchKernelGGL(act_to_f16_kernel, grid, dim3(threads), 0, st, x, xs, xh, K, B);
  CWEN_HIP_TRY(hipGetLastError());
  return CWEN_OK;
}
