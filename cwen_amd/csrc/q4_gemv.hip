// Q4_0 batched GEMV for a verify block of B = 1..16 activation columns.
//
// Reference semantics: gemvb / dot_q4_bcol / dot_q4_0rsi_2mat / mlp_blk
// (run.c:1529-1680, 886-975, 2677-2683): Y[b][i] = sum_k (n_ik - 8) * d_i,blk(k) * X[b][k].
//
// Design (gfx950):
//  * Weights are repacked once at upload into 1152-byte tiles of 16 rows x
//    4 blocks (128 K).  Lane l = 16g + n of a wave owns block g of row n: its
//    16 nibble bytes (one 16-byte load) and its f16 scale (one 2-byte load),
//    so a tile streams with no duplicated bytes.
//  * v_mfma_f32_16x16x32_f16, A = activations (16 columns x 32 K), B =
//    weights (32 K x 16 rows).  MFMA j of a tile takes K run j (8 weights) of
//    each lane's block, so a lane's B operand always belongs to one block and
//    the block scale is folded into the f16 weights: w = (n - 8) * d with one
//    rounding (relative 2^-12), the same order as the f16 activation rounding.
//    The MFMA accumulates in f32; there is no per-block epilogue.
//  * Activations are f16 row-major [B][K].  A workgroup's 4 waves take
//    different rows over the same K range and share the activation chunk,
//    staged once per workgroup in LDS (double-buffered).  Columns >= B load
//    as zeros (past the buffer range), so one kernel serves B = 1..16 and a
//    column's arithmetic never depends on B (block verify == serial decode,
//    bit for bit).
//  * Long K is split across workgroups.  Each writes its partial sums with
//    agent-scope atomic stores, bumps a per-row-tile counter, and the last
//    arriver sums the partials in split order: deterministic, with no cache
//    writeback/invalidate.  The split depends on the shape only.
//  * Each wave keeps PF tiles of weights in flight; every global load in the
//    loop is unconditional and issued in a fixed order, so the in-order load
//    counter only waits for the data being consumed.
#include "cwen_internal.h"

namespace {

constexpr int PF = 4;      // tiles per round == weight tiles in flight per wave
constexpr int WAVES = 4;   // waves per workgroup

// K-run order inside a dword: unpack8 yields elements from nibbles
// 0,4,1,5,2,6,3,7, so the repack stores weight e of the run at kNibPos[e].
__constant__ int kNibPos[8] = {0, 4, 1, 5, 2, 6, 3, 7};

// (q & mask) | magic in one VOP3 op.  gfx9 VOP3 takes no literal and reads at
// most one scalar, so the mask comes from an SGPR and the magic from a VGPR.
__device__ __forceinline__ uint32_t and_or(uint32_t q, uint32_t mask_s, uint32_t magic_v) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(q), "s"(mask_s), "v"(magic_v));
  return r;
}

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

// 8 nibbles -> 8 f16 weights (n - 8) * d.  (n - 8) is exact (magic-exponent
// trick); the product with the block scale is the one rounding.
__device__ __forceinline__ half8_t unpack8(uint32_t q, const Unpack &u, half2_t dd) {
  const uint32_t q2 = q >> 8;
  const uint32_t t0 = and_or(q, u.lo, u.magic);    // 1024 + n0, 1024 + n4
  const uint32_t t1 = and_or(q, u.hi, u.magic);    // 1024 + 16 n1, 1024 + 16 n5
  const uint32_t t2 = and_or(q2, u.lo, u.magic);   // 1024 + n2, 1024 + n6
  const uint32_t t3 = and_or(q2, u.hi, u.magic);   // 1024 + 16 n3, 1024 + 16 n7
  const half2_t k1032 = {(_Float16)1032.0f, (_Float16)1032.0f};
  const half2_t k16 = {(_Float16)0.0625f, (_Float16)0.0625f};
  const half2_t k72 = {(_Float16)-72.0f, (_Float16)-72.0f};
  const half2_t h0 = (__builtin_bit_cast(half2_t, t0) - k1032) * dd;
  const half2_t h1 = __builtin_elementwise_fma(__builtin_bit_cast(half2_t, t1), k16, k72) * dd;
  const half2_t h2 = (__builtin_bit_cast(half2_t, t2) - k1032) * dd;
  const half2_t h3 = __builtin_elementwise_fma(__builtin_bit_cast(half2_t, t3), k16, k72) * dd;
  half8_t r;
  r[0] = h0[0]; r[1] = h0[1]; r[2] = h1[0]; r[3] = h1[1];
  r[4] = h2[0]; r[5] = h2[1]; r[6] = h3[0]; r[7] = h3[1];
  return r;
}

__device__ __forceinline__ uint32_t bload2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return (uint32_t)(uint16_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}

// LDS hand-off barrier: waits for this wave's LDS writes only, not for its
// outstanding global loads (unlike __syncthreads(), whose release fence
// drains the load counter).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // gfx9 encoding: lgkmcnt(0), vmcnt/expcnt unchanged
  __builtin_amdgcn_s_barrier();
}

struct Q4Params {
  const uint8_t *w;    // tiled weights
  uint32_t wbytes;     // bytes of the tiled weights (buffer range)
  int nsw;             // sides stored per tile position (1 or 2)
  int side0;           // first side computed (NS == 1)
  int M, nrg, nkt;
  int S, tps;          // K split across workgroups, tiles per split (multiple of PF)
  const _Float16 *xh;  // activations f16 [B][K]
  uint32_t xbytes;     // B*K*2 (buffer range: columns >= B read as zero)
  int B;
  float *part;         // split-K partials
  int *cnt;            // per row-tile arrival counters (zero between launches)
  Q4Out out;
};

// NS: sides per row group (2 = both halves of an interleaved pair).
// R:  row groups per wave.  Each wave carries R*NS weight streams.
template <int NS, int R, int EPI>
__global__ __launch_bounds__(64 * WAVES) void q4_gemv_kernel(Q4Params p) {
  constexpr int NSET = NS * R;
  __shared__ uint4 act[2][PF * 4 * 64];  // [buf][tile][K run][lane] f16 x 8
  __shared__ int s_last;

  const int tid = threadIdx.x;
  // Wave index as a scalar: loop bounds and addresses are then provably
  // wave-uniform, which keeps the loop's load-counter waits exact.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int n = lane & 15, g = lane >> 4;
  const int rt = blockIdx.x / p.S;
  const int sp = blockIdx.x - rt * p.S;
  const int kt0 = sp * p.tps;
  const int nt = min(p.nkt - kt0, p.tps);      // multiple of PF
  const int nround = nt / PF;

  const __amdgpu_buffer_rsrc_t wr = make_rsrc(p.w, p.wbytes);
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.xh, p.xbytes);

  // Weight streams of this wave: set q = r*NS + s is row group rgs[r], side s.
  const uint32_t tstride = (uint32_t)p.nsw * Q4_TILE_BYTES;
  uint32_t wofs[NSET];
  int rgs[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    rgs[r] = (rt * WAVES + wave) * R + r;
    const int rgc = rgs[r] < p.nrg ? rgs[r] : p.nrg - 1;  // idle streams read a valid tile
#pragma unroll
    for (int s = 0; s < NS; ++s)
      wofs[r * NS + s] = (((uint32_t)rgc * p.nkt + kt0) * p.nsw + (NS == 2 ? s : p.side0)) * Q4_TILE_BYTES;
  }
  const uint32_t lq = lane * 16, ls = Q4_TILE_QS + lane * 2;

  // Activation staging: thread (wave, lane) copies K run `wave` of block g of
  // each round tile for column n into LDS slot (tile*4 + wave)*64 + lane.
  const uint32_t xlane = ((uint32_t)n * (uint32_t)(p.nkt * Q4_TILE_K) + g * 32 + wave * 8) * 2;
  const uint32_t xtile = Q4_TILE_K * 2;

  uint4 xs[PF];
  uint4 wq[PF][NSET];
  uint32_t wsc[PF][NSET];
#pragma unroll
  for (int j = 0; j < PF; ++j) xs[j] = bload16(xr, xlane + (uint32_t)(kt0 + j) * xtile);
#pragma unroll
  for (int i = 0; i < PF; ++i) {
#pragma unroll
    for (int q = 0; q < NSET; ++q) {
      wq[i][q] = bload16(wr, wofs[q] + i * tstride + lq);
      wsc[i][q] = bload2(wr, wofs[q] + i * tstride + ls);
    }
    __builtin_amdgcn_sched_barrier(0);  // issue the ring in slot order
  }
#pragma unroll
  for (int j = 0; j < PF; ++j) act[0][(j * 4 + wave) * 64 + lane] = xs[j];
  lds_barrier();

  const Unpack uc = unpack_consts();
  floatx4_t acc[NSET][2];
#pragma unroll
  for (int q = 0; q < NSET; ++q) acc[q][0] = acc[q][1] = (floatx4_t){0.f, 0.f, 0.f, 0.f};

  for (int rd = 0; rd < nround; ++rd) {
    const int cur = rd & 1;
    {  // next round's activations (the last round re-reads its own, harmlessly)
      const int nr = rd + 1 < nround ? rd + 1 : rd;
#pragma unroll
      for (int j = 0; j < PF; ++j) xs[j] = bload16(xr, xlane + (uint32_t)(kt0 + nr * PF + j) * xtile);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      half8_t b[NSET][4];
#pragma unroll
      for (int q = 0; q < NSET; ++q) {
        const half2_t dd = __builtin_bit_cast(half2_t, wsc[j][q] * 0x10001u);
        b[q][0] = unpack8(wq[j][q].x, uc, dd);
        b[q][1] = unpack8(wq[j][q].y, uc, dd);
        b[q][2] = unpack8(wq[j][q].z, uc, dd);
        b[q][3] = unpack8(wq[j][q].w, uc, dd);
      }
      // Refill the slot once its registers are consumed, so the loads land
      // in the same registers (no loop-carried copies, no counter drain).
      {
        const int tn0 = rd * PF + j + PF;
        const uint32_t tn = (uint32_t)(tn0 < nt ? tn0 : nt - 1);
#pragma unroll
        for (int q = 0; q < NSET; ++q) {
          wq[j][q] = bload16(wr, wofs[q] + tn * tstride + lq);
          wsc[j][q] = bload2(wr, wofs[q] + tn * tstride + ls);
        }
      }
      half8_t a[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) a[m] = __builtin_bit_cast(half8_t, act[cur][(j * 4 + m) * 64 + lane]);
#pragma unroll
      for (int q = 0; q < NSET; ++q)
#pragma unroll
        for (int m = 0; m < 4; ++m)
          acc[q][m & 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[m], b[q][m], acc[q][m & 1], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);  // keep slots in issue order
    }
#pragma unroll
    for (int j = 0; j < PF; ++j) act[cur ^ 1][(j * 4 + wave) * 64 + lane] = xs[j];
    lds_barrier();
  }

  floatx4_t res[NSET];
#pragma unroll
  for (int q = 0; q < NSET; ++q) res[q] = acc[q][0] + acc[q][1];

  if (p.S > 1) {
    // Publish this split's partials.  Agent-scope atomic stores reach the
    // device coherence point; the wait makes them complete before the
    // counter bump, and the last arriver reads them the same way.
    const bool cols_on = g * 4 < p.B;
    uint64_t *part = (uint64_t *)p.part;
#pragma unroll
    for (int q = 0; q < NSET; ++q) {
      const size_t base = ((((size_t)rt * WAVES + wave) * NSET + q) * p.S + sp) * 128 + lane * 2;
      if (cols_on) {
        __hip_atomic_store(part + base, __builtin_bit_cast(uint64_t, (float2){res[q][0], res[q][1]}),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(part + base + 1, __builtin_bit_cast(uint64_t, (float2){res[q][2], res[q][3]}),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");  // stores acknowledged
    __builtin_amdgcn_s_barrier();
    if (tid == 0)
      s_last = __hip_atomic_fetch_add(p.cnt + rt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == p.S - 1;
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    if (!s_last) return;
#pragma unroll
    for (int q = 0; q < NSET; ++q) {
      const size_t base = ((((size_t)rt * WAVES + wave) * NSET + q) * p.S) * 128 + lane * 2;
      floatx4_t v = {0.f, 0.f, 0.f, 0.f};
      if (cols_on) {
        for (int k = 0; k < p.S; ++k) {
          const float2 lo = __builtin_bit_cast(
              float2, __hip_atomic_load(part + base + (size_t)k * 128, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
          const float2 hi = __builtin_bit_cast(
              float2, __hip_atomic_load(part + base + (size_t)k * 128 + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
          v += (floatx4_t){lo.x, lo.y, hi.x, hi.y};
        }
      }
      res[q] = v;
    }
    if (tid == 0) __hip_atomic_store(p.cnt + rt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  const Q4Out &o = p.out;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = rgs[r] * Q4_ROWS + n;
    if (rgs[r] >= p.nrg || row >= p.M) continue;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = g * 4 + e;
      if (c >= p.B) continue;
      const float a0 = res[r * NS][e];
      float v = (EPI == Q4_EPI_SWIGLU) ? silu_f(a0) * res[r * NS + NS - 1][e] : a0;
      if (o.y) {
        float *dst = o.y + (size_t)c * o.ys + row;
        if (o.accumulate) v += *dst;
        *dst = v;
      }
      if (o.yh) o.yh[(size_t)c * p.M + row] = (_Float16)v;
      if (EPI == Q4_EPI_PAIR) o.y1[(size_t)c * o.ys + row] = res[r * NS + NS - 1][e];
    }
  }
}

// One thread per (row group, K tile, side, lane): lane l = 16g + n gets block
// g of the tile for row n -- 4 dwords, dword j holding K run j (weights
// 8j..8j+7 of the block) in kNibPos order -- and that block's f16 scale.
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
  const int blk = kt * 4 + g;
  uint8_t *tile = dst + (((size_t)rg * nkt + kt) * nsw + side) * Q4_TILE_BYTES;
  const uint8_t *qs = nullptr;
  uint16_t d = 0;
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
  }
  uint32_t out[4];
  for (int j = 0; j < 4; ++j) {
    uint32_t word = 0;
    for (int e = 0; e < 8; ++e) {
      const int k = j * 8 + e;  // weight index inside the 32-weight block
      uint32_t nib = 8;
      if (qs) nib = (k < 16) ? (qs[k] & 0xFu) : (qs[k - 16] >> 4);
      word |= nib << (4 * kNibPos[e]);
    }
    out[j] = word;
  }
  *(uint4 *)(tile + lane * 16) = make_uint4(out[0], out[1], out[2], out[3]);
  *(uint16_t *)(tile + Q4_TILE_QS + lane * 2) = d;
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

template <int NS, int R, int EPI>
int launch_one(const Q4Params &p, int nrt, hipStream_t st) {
  hipLaunchKernelGGL((q4_gemv_kernel<NS, R, EPI>), dim3((unsigned)(nrt * p.S)), dim3(64 * WAVES), 0, st, p);
  return CWEN_OK;
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

// Launch shape from the weight's shape only (never from B), so every output
// bit is independent of the block size.  rows: row groups per wave for
// single-sided use; split: K split across workgroups; tps: K tiles per split.
void q4_choose_split(const cwen_ctx *ctx, cwen_weight *w) {
  const int R = (w->nside == 1 && w->nrg >= 2 * WAVES * 32) ? 2 : 1;
  // A pair is computed two-sided (R = 1); single-side calls on it use R = 1 too.
  const int Rs = (w->nside == 1) ? R : 1;
  const int nrt = (w->nrg + WAVES * Rs - 1) / (WAVES * Rs);
  const int nrd = w->nkt / PF;                       // rounds of K
  int S = (ctx->wg_target + nrt - 1) / nrt;
  if (S > nrd / 2) S = nrd / 2;                      // keep >= 2 rounds per split
  if (S < 1) S = 1;
  const int rps = (nrd + S - 1) / S;
  w->rows = Rs;
  w->tps = rps * PF;
  w->split = (nrd + rps - 1) / rps;
}

int q4_gemv_launch(cwen_ctx *ctx, const cwen_weight *w, int nsides, int side0, int epi,
                   const _Float16 *xh, const Q4Out &out, int B, hipStream_t st) {
  Q4Params p;
  p.w = w->dev;
  p.wbytes = (uint32_t)w->bytes;
  p.nsw = w->nside;
  p.side0 = side0;
  p.M = w->ne1;
  p.nrg = w->nrg;
  p.nkt = w->nkt;
  p.S = w->split;
  p.tps = w->tps;
  p.xh = xh;
  p.xbytes = (uint32_t)((size_t)B * w->ne0 * 2);
  p.B = B;
  p.part = ctx->partials;
  p.cnt = ctx->counters;
  p.out = out;
  const int R = w->rows;
  const int nrt = (w->nrg + WAVES * R - 1) / (WAVES * R);
  if (p.S > 1) {
    const size_t need = (size_t)nrt * WAVES * R * nsides * p.S * 256;
    if (need > ctx->partials_floats || nrt > ctx->ncounters) return CWEN_ESCRATCH;
  }
  int rc;
  if (nsides == 1 && epi == Q4_EPI_STORE)
    rc = R == 2 ? launch_one<1, 2, Q4_EPI_STORE>(p, nrt, st) : launch_one<1, 1, Q4_EPI_STORE>(p, nrt, st);
  else if (nsides == 2 && epi == Q4_EPI_PAIR)
    rc = launch_one<2, 1, Q4_EPI_PAIR>(p, nrt, st);
  else if (nsides == 2 && epi == Q4_EPI_SWIGLU)
    rc = launch_one<2, 1, Q4_EPI_SWIGLU>(p, nrt, st);
  else
    return CWEN_EINVAL;
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
