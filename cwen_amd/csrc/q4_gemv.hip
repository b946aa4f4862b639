// Q4_0 batched GEMV for a verify block of B = 1..16 activation columns.
//
// Reference semantics: gemvb / dot_q4_bcol / dot_q4_0rsi_2mat / mlp_blk
// (run.c:1529-1680, 886-975, 2677-2683): Y[b][i] = sum_k (n_ik - 8) * d_i,blk(k) * X[b][k].
//
// Design (gfx950):
//  * Weights are repacked once at upload into 4608-byte super-tiles of 16
//    rows x 16 blocks (512 K): four 1 KB nibble tiles then a 512-byte scale
//    block.  In tile u, lane l = 16g + n owns block g of row n (16 nibble
//    bytes, one 16-byte load); the scale block gives lane l the f16 scales of
//    its block in all 4 tiles (one 8-byte load).  Every nibble load moves
//    1 KB per wave, the scales of 4 tiles come in one 512-byte load, and no
//    byte is fetched twice.
//  * v_mfma_f32_16x16x32_f16, A = activations (16 columns x 32 K), B =
//    weights (32 K x 16 rows).  MFMA j of a tile takes K run j (8 weights) of
//    each lane's block, so a lane's B operand always belongs to one block and
//    the block scale is folded into the f16 weights: w = (n - 8) * d with one
//    rounding (relative 2^-12), the same order as the f16 activation rounding.
//    The MFMA accumulates in f32; there is no per-block epilogue.
//  * Activations are f16 row-major [B][K].  A workgroup's 4 waves take
//    different rows over the same K range and share the activation chunk,
//    staged once per workgroup in LDS (double-buffered).  One staging load
//    moves one column's 1 KB of a super-tile; the LDS slot of 16-byte unit u
//    of column c is c*64 + (u ^ c), which keeps both the column-wise writes
//    and the MFMA operand reads free of bank conflicts.  Only the first CB
//    columns (CB = 4, 8 or 16, the smallest >= B) are staged; columns in
//    [B, CB) lie past the buffer range and load as zeros.  Output column c
//    depends on activation column c alone, so the unstaged columns only feed
//    discarded outputs, and a column's arithmetic never depends on B (block
//    verify == serial decode, bit for bit).
//  * Long K is split across workgroups.  Each writes its partial sums with
//    agent-scope atomic stores, bumps a per-row-tile counter, and the last
//    arriver sums the partials in split order: deterministic, with no cache
//    writeback/invalidate.  The split depends on the shape only.
//  * Each wave keeps one super-tile per weight stream in flight; every global
//    load in the loop is unconditional and issued in a fixed order (scales,
//    staging, then tiles), so the in-order load counter only waits for the
//    data being consumed.
#include <type_traits>

#include "cwen_internal.h"

namespace {

constexpr int PF = Q4_ST_TILES;  // tiles per round: one super-tile per stream
constexpr int WAVES = 4;         // waves per workgroup

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

// f16 scale in the low (hi = false) or high half of `w`, broadcast to both halves.
__device__ __forceinline__ half2_t bcast_half(uint32_t w, bool hi) {
  return __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(w, w, hi ? 0x03020302u : 0x01000100u));
}

// LDS hand-off barrier: waits for this wave's LDS writes only, not for its
// outstanding global loads (unlike __syncthreads(), whose release fence
// drains the load counter).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // gfx9 encoding: lgkmcnt(0), vmcnt/expcnt unchanged
  __builtin_amdgcn_s_barrier();
}

struct Q4Params {
  const uint8_t *w;    // super-tiled weights
  uint32_t wbytes;     // bytes of the tiled weights (buffer range)
  int nsw;             // sides stored per super-tile position (1 or 2)
  int side0;           // first side computed (NS == 1)
  int M, nrg, nst;
  int S, rps;          // K split across workgroups, super-tiles (rounds) per split
  const _Float16 *xh;  // activations f16 [B][K]
  uint32_t xbytes;     // B*K*2 (buffer range: columns >= B read as zero)
  int K, B;
  float *part;         // split-K partials
  int *cnt;            // per row-tile arrival counters (zero between launches)
  Q4Out out;
};

// NS: sides per row group (2 = both halves of an interleaved pair).
// R:  row groups per wave.  Each wave carries R*NS weight streams.
// CB: activation columns staged (4, 8 or 16; >= B).
template <int NS, int R, int EPI, int CB>
__global__ __launch_bounds__(64 * WAVES) void q4_gemv_kernel(Q4Params p) {
  constexpr int NSET = NS * R;
  constexpr int XL = CB / WAVES;            // staging loads per wave per round
  __shared__ uint4 act[2][16 * 64];         // [buf][column c][unit u ^ c], f16 x 8 per unit
  __shared__ int s_last;

  const int tid = threadIdx.x;
  // Wave index as a scalar: loop bounds and addresses are then provably
  // wave-uniform, which keeps the loop's load-counter waits exact.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int n = lane & 15, g = lane >> 4;
  const int rt = blockIdx.x / p.S;
  const int sp = blockIdx.x - rt * p.S;
  const int st0 = sp * p.rps;
  const int nround = min(p.nst - st0, p.rps);

  const __amdgpu_buffer_rsrc_t wr = make_rsrc(p.w, p.wbytes);
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.xh, p.xbytes);

  // Weight streams of this wave: set q = r*NS + s is row group rgs[r], side s.
  const uint32_t sstride = (uint32_t)p.nsw * Q4_ST_BYTES;
  uint32_t wofs[NSET];
  int rgs[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    rgs[r] = (rt * WAVES + wave) * R + r;
    const int rgc = rgs[r] < p.nrg ? rgs[r] : p.nrg - 1;  // idle streams read a valid tile
#pragma unroll
    for (int s = 0; s < NS; ++s)
      wofs[r * NS + s] = (((uint32_t)rgc * p.nst + st0) * p.nsw + (NS == 2 ? s : p.side0)) * Q4_ST_BYTES;
  }
  const uint32_t lq = lane * 16, ls = Q4_ST_QS + lane * 8;

  // Activation staging: this wave copies columns c = wave + WAVES*i; lane
  // copies 16-byte unit `lane` of the column's 512-K chunk.
  const uint32_t xround = Q4_ST_K * 2;
  uint32_t xofs[XL];
  int xslot[XL];
#pragma unroll
  for (int i = 0; i < XL; ++i) {
    const int c = wave + WAVES * i;
    xofs[i] = (uint32_t)c * (uint32_t)p.K * 2 + (uint32_t)st0 * xround + lane * 16;  // per lane: range-checked
    xslot[i] = c * 64 + (lane ^ c);
  }

  uint4 xs[XL];
  uint4 wq[PF][NSET];
  uint2 sc[NSET];
#pragma unroll
  for (int q = 0; q < NSET; ++q) sc[q] = bload8(wr, ls, wofs[q]);
#pragma unroll
  for (int i = 0; i < XL; ++i) xs[i] = bload16(xr, xofs[i]);
#pragma unroll
  for (int j = 0; j < PF; ++j) {
#pragma unroll
    for (int q = 0; q < NSET; ++q) wq[j][q] = bload16(wr, lq + j * Q4_TILE_QS, wofs[q]);
    __builtin_amdgcn_sched_barrier(0);  // issue the ring in slot order
  }
#pragma unroll
  for (int i = 0; i < XL; ++i) act[0][xslot[i]] = xs[i];
  lds_barrier();

  const Unpack uc = unpack_consts();
  floatx4_t acc[NSET][2];
#pragma unroll
  for (int q = 0; q < NSET; ++q) acc[q][0] = acc[q][1] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
  // LDS unit of MFMA m of tile 0 for this lane (column n, K run 4g + m); tile
  // j adds 16 units, which stay clear of the XOR (n < 16).
  int aslot[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) aslot[m] = n * 64 + ((4 * g + m) ^ n);

  // One round = one super-tile per stream.  The LDS buffer index is a
  // template constant (the loop is unrolled by two), so every LDS address is
  // a lane base plus an immediate.
  auto round = [&](int rd, auto cur_c) __attribute__((always_inline)) {
    constexpr int cur = decltype(cur_c)::value;
    // Next round's super-tile (the last round re-reads its own, harmlessly).
    const uint32_t nr = (uint32_t)(rd + 1 < nround ? rd + 1 : rd);
    half2_t dd[NSET][PF];
#pragma unroll
    for (int q = 0; q < NSET; ++q) {
      dd[q][0] = bcast_half(sc[q].x, false);
      dd[q][1] = bcast_half(sc[q].x, true);
      dd[q][2] = bcast_half(sc[q].y, false);
      dd[q][3] = bcast_half(sc[q].y, true);
    }
#pragma unroll
    for (int q = 0; q < NSET; ++q) sc[q] = bload8(wr, ls, wofs[q] + nr * sstride);
#pragma unroll
    for (int i = 0; i < XL; ++i) xs[i] = bload16(xr, xofs[i], nr * xround);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      half8_t b[NSET][4];
#pragma unroll
      for (int q = 0; q < NSET; ++q) {
        b[q][0] = unpack8(wq[j][q].x, uc, dd[q][j]);
        b[q][1] = unpack8(wq[j][q].y, uc, dd[q][j]);
        b[q][2] = unpack8(wq[j][q].z, uc, dd[q][j]);
        b[q][3] = unpack8(wq[j][q].w, uc, dd[q][j]);
      }
      // Refill the slot once its registers are consumed, so the loads land
      // in the same registers (no loop-carried copies, no counter drain).
#pragma unroll
      for (int q = 0; q < NSET; ++q) wq[j][q] = bload16(wr, lq + j * Q4_TILE_QS, wofs[q] + nr * sstride);
      half8_t a[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) a[m] = __builtin_bit_cast(half8_t, act[cur][aslot[m] + 16 * j]);
#pragma unroll
      for (int q = 0; q < NSET; ++q)
#pragma unroll
        for (int m = 0; m < 4; ++m)
          acc[q][m & 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[m], b[q][m], acc[q][m & 1], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);  // keep slots in issue order
    }
#pragma unroll
    for (int i = 0; i < XL; ++i) act[cur ^ 1][xslot[i]] = xs[i];
    lds_barrier();
  };
  int rd = 0;
  for (; rd + 1 < nround; rd += 2) {
    round(rd, std::integral_constant<int, 0>{});
    round(rd + 1, std::integral_constant<int, 1>{});
  }
  if (rd < nround) round(rd, std::integral_constant<int, 0>{});

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
    // Sum the splits in split order.  The loads of a chunk of KCH splits are
    // all issued before the first is consumed, so the reduction costs one
    // memory round trip per chunk, not one per split.
    constexpr int KCH = 8;
#pragma unroll
    for (int q = 0; q < NSET; ++q) res[q] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
    if (cols_on) {
      for (int k0 = 0; k0 < p.S; k0 += KCH) {
        uint64_t lo[NSET][KCH], hi[NSET][KCH];
#pragma unroll
        for (int q = 0; q < NSET; ++q) {
          const size_t base = ((((size_t)rt * WAVES + wave) * NSET + q) * p.S) * 128 + lane * 2;
#pragma unroll
          for (int u = 0; u < KCH; ++u) {
            const size_t k = (size_t)min(k0 + u, p.S - 1);
            lo[q][u] = __hip_atomic_load(part + base + k * 128, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            hi[q][u] = __hip_atomic_load(part + base + k * 128 + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        }
#pragma unroll
        for (int q = 0; q < NSET; ++q)
#pragma unroll
          for (int u = 0; u < KCH; ++u)
            if (k0 + u < p.S) {
              const float2 a = __builtin_bit_cast(float2, lo[q][u]);
              const float2 b = __builtin_bit_cast(float2, hi[q][u]);
              res[q] += (floatx4_t){a.x, a.y, b.x, b.y};
            }
      }
    }
    if (tid == 0) __hip_atomic_store(p.cnt + rt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  const Q4Out &o = p.out;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = rgs[r] * Q4_ROWS + n;
    if (rgs[r] >= p.nrg || row >= p.M) continue;
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a0 = res[r * NS][e];
      v[e] = (EPI == Q4_EPI_SWIGLU) ? silu_f(a0) * res[r * NS + NS - 1][e] : a0;
    }
    if (o.y && o.accumulate) {  // all residual loads in flight together
      float old[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int c = g * 4 + e;
        old[e] = c < p.B ? o.y[(size_t)c * o.ys + row] : 0.f;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] += old[e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = g * 4 + e;
      if (c >= p.B) continue;
      if (o.y) o.y[(size_t)c * o.ys + row] = v[e];
      if (o.yh) o.yh[(size_t)c * p.M + row] = (_Float16)v[e];
      if (EPI == Q4_EPI_PAIR) o.y1[(size_t)c * o.ys + row] = res[r * NS + NS - 1][e];
    }
  }
}

// One thread per (row group, super-tile, side, lane): lane l = 16g + n gets,
// for each tile u of the super-tile, block g of that tile for row n -- 4
// dwords, dword j holding K run j (weights 8j..8j+7 of the block) in
// kNibPos order -- and the 4 blocks' f16 scales.  Rows past M get zero
// weights (nibble 8, scale 0).
__global__ void q4_repack_kernel(uint8_t *dst, const uint8_t *src, const uint16_t *sc, int type,
                                 int M, int K, int nrg, int nst, int nsw) {
  const size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t total = (size_t)nrg * nst * nsw * 64;
  if (id >= total) return;
  const int lane = (int)(id & 63);
  size_t t = id >> 6;
  const int side = (int)(t % nsw); t /= nsw;
  const int st = (int)(t % nst);
  const int rg = (int)(t / nst);
  const int n = lane & 15, g = lane >> 4;
  const int row = rg * Q4_ROWS + n;
  const int nb = K / 32;
  uint8_t *stile = dst + (((size_t)rg * nst + st) * nsw + side) * Q4_ST_BYTES;
  uint16_t d[Q4_ST_TILES];
  for (int u = 0; u < Q4_ST_TILES; ++u) {
    const int blk = (st * Q4_ST_TILES + u) * 4 + g;
    const uint8_t *qs = nullptr;
    d[u] = 0;
    if (row < M) {
      const size_t bi = (size_t)row * nb + blk;
      if (type == CWEN_T_Q4_0) {
        const uint8_t *b = src + bi * 18;
        d[u] = (uint16_t)(b[0] | (b[1] << 8));
        qs = b + 2;
      } else if (type == CWEN_T_Q4_0RS) {
        qs = src + bi * 16;
        d[u] = sc[bi];
      } else {  // Q4_0RSI
        qs = src + bi * 32 + side * 16;
        d[u] = sc[bi * 2 + side];
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
    *(uint4 *)(stile + u * Q4_TILE_QS + lane * 16) = make_uint4(out[0], out[1], out[2], out[3]);
  }
  *(uint2 *)(stile + Q4_ST_QS + lane * 8) =
      make_uint2((uint32_t)d[0] | ((uint32_t)d[1] << 16), (uint32_t)d[2] | ((uint32_t)d[3] << 16));
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

template <int NS, int R, int EPI, int CB>
int launch_one(const Q4Params &p, int nrt, hipStream_t st) {
  hipLaunchKernelGGL((q4_gemv_kernel<NS, R, EPI, CB>), dim3((unsigned)(nrt * p.S)), dim3(64 * WAVES), 0, st, p);
  return CWEN_OK;
}

template <int NS, int R, int EPI>
int launch_cb(const Q4Params &p, int nrt, hipStream_t st) {
  if (p.B <= 4) return launch_one<NS, R, EPI, 4>(p, nrt, st);
  if (p.B <= 8) return launch_one<NS, R, EPI, 8>(p, nrt, st);
  return launch_one<NS, R, EPI, 16>(p, nrt, st);
}

}  // namespace

int q4_repack(cwen_weight *w, const uint8_t *dsrc, const uint16_t *dsc, hipStream_t st) {
  const size_t threads = (size_t)w->nrg * w->nst * w->nside * 64;
  const int blk = 256;
  const size_t grid = (threads + blk - 1) / blk;
  hipLaunchKernelGGL(q4_repack_kernel, dim3((unsigned)grid), dim3(blk), 0, st, w->dev, dsrc, dsc,
                     w->type, w->ne1, w->ne0, w->nrg, w->nst, w->nside);
  CWEN_HIP_TRY(hipGetLastError());
  return CWEN_OK;
}

// Launch shape from the weight's shape only (never from B), so every output
// bit is independent of the block size.  rows: row groups per wave for
// single-sided use; split: K split across workgroups; rps: super-tiles per split.
void q4_choose_split(const cwen_ctx *ctx, cwen_weight *w) {
  const int R = (w->nside == 1 && w->nrg >= 2 * WAVES * 32) ? 2 : 1;
  // A pair is computed two-sided (R = 1); single-side calls on it use R = 1 too.
  const int Rs = (w->nside == 1) ? R : 1;
  const int nrt = (w->nrg + WAVES * Rs - 1) / (WAVES * Rs);
  const int nrd = w->nst;                            // rounds of K
  int S = (ctx->wg_target + nrt - 1) / nrt;
  if (S > nrd / 2) S = nrd / 2;                      // keep >= 2 rounds per split
  if (S < 1) S = 1;
  const int rps = (nrd + S - 1) / S;
  w->rows = Rs;
  w->rps = rps;
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
  p.nst = w->nst;
  p.S = w->split;
  p.rps = w->rps;
  p.xh = xh;
  p.xbytes = (uint32_t)((size_t)B * w->ne0 * 2);
  p.K = w->ne0;
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
    rc = R == 2 ? launch_cb<1, 2, Q4_EPI_STORE>(p, nrt, st) : launch_cb<1, 1, Q4_EPI_STORE>(p, nrt, st);
  else if (nsides == 2 && epi == Q4_EPI_PAIR)
    rc = launch_cb<2, 1, Q4_EPI_PAIR>(p, nrt, st);
  else if (nsides == 2 && epi == Q4_EPI_SWIGLU)
    rc = launch_cb<2, 1, Q4_EPI_SWIGLU>(p, nrt, st);
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
