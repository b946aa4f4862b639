// Batched quantized GEMV for a verify block of B = 1..16 activation columns:
// Q4_0 (GGUF, CWENR RS and RSI), Q6_K and Q8_0 weights.
//
// Reference semantics: gemvb / gemv_row / dot_q4_bcol / dot_q4_0rsi_2mat /
// dot_q6_K / dot_q8_0 / mlp_blk (run.c:1577-1680, 1360-1387, 1529-1571,
// 886-975, 1160-1274, 2677-2683): Y[b][i] = sum_k w_ik * X[b][k] with
//   Q4_0  w = (n - 8) * d_blk             (32-weight blocks, f16 d)
//   Q6_K  w = (q6 - 32) * d_sb * sc_sub   (256-weight super-blocks, f16 d,
//                                          int8 scale per 16 weights)
//   Q8_0  w = q8 * d_blk                  (32-weight blocks, f16 d)
// and, for the LM head, the per-column argmax and greedy prefix walk of
// argmax_of and generate_tokens_spec (run.c:2647-2668, 4954-4956).
//
// Design (gfx950):
//  * Weights are repacked once at upload into super-tiles of 16 rows x 512 K
//    per weight stream, laid out in MFMA operand order.  A super-tile holds
//    four 128-K tiles; in tile u, lane l = 16g + n of a wave owns 32-weight
//    block g of row n, so each 16-byte load of a wave moves 1 KB and no byte
//    is fetched twice.  The per-format bytes are the reference's exactly
//    (18 B / 32 Q4_0 weights, 210 B / 256 Q6_K weights, 34 B / 32 Q8_0
//    weights); only their order changes:
//      Q4_0  4608 B: 4 x 1 KB nibble tiles | 512 B scales (lane: its block's
//            f16 scale in tiles 0..3)
//      Q6_K  6720 B: 4 x 1 KB low-nibble tiles | 2 x 1 KB high-bit tile pairs
//            | 512 B int8 sub-scales, stored + 128 (lane: its 2 sub-blocks
//            in tiles 0..3) | 64 B f16 d [row][super-block]
//      Q8_0  8704 B: 4 x 2 KB int8 tiles, stored + 128 (lane: two 16-byte
//            halves) | 512 B scales
//  * v_mfma_f32_16x16x32_f16, A = activations (16 columns x 32 K), B =
//    weights (32 K x 16 rows).  MFMA m of a tile takes K run m (8 weights) of
//    each lane's block, so a lane's B operand always belongs to one scale
//    group and the scale is folded into the f16 weights.  Integers become
//    f16 exactly through the magic-exponent trick ((bits | 0x6400) is
//    1024 + bits); the product with the scale is the one rounding (relative
//    2^-12), the same order as the f16 activation rounding.  The MFMA
//    accumulates in f32.
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
//    data being consumed.  Weight loads are non-temporal (read once); the
//    staged activations use the default policy.
#include <algorithm>
#include <type_traits>
#include <vector>

#include "cwen_internal.h"

namespace {

constexpr int TILES = Q4_ST_TILES;  // tiles per round: one super-tile per stream
// A per-lane buffer offset past any activation range: the load returns zeros.
constexpr uint32_t kPastRange = 0xFFFFFFE0u;
constexpr int WAVES = 4;            // waves per workgroup

// K-run order inside a dword: the nibble unpack yields elements from nibbles
// 0,4,1,5,2,6,3,7, so the repack stores weight e of a run at kNibPos[e].
__constant__ int kNibPos[8] = {0, 4, 1, 5, 2, 6, 3, 7};

// Per-format layout of one 16-row x 512-K super-tile of one weight stream.
template <int FMT> struct Fmt;
template <> struct Fmt<GEMV_Q4> {
  static constexpr uint32_t ST_BYTES = 4608, SC_OFS = 4096;
  static constexpr int TV = 1;                 // 16-byte loads per tile per lane
};
template <> struct Fmt<GEMV_Q6K> {
  static constexpr uint32_t ST_BYTES = 6720, HI_OFS = 4096, SC_OFS = 6144, D_OFS = 6656;
  static constexpr int TV = 1;
};
template <> struct Fmt<GEMV_Q8> {
  static constexpr uint32_t ST_BYTES = 8704, SC_OFS = 8192;
  static constexpr int TV = 2;
};
// Q4_1: the Q4_0 nibble layout, then per lane the 4 blocks' (d, m) f16 pairs.
template <> struct Fmt<GEMV_Q41> {
  static constexpr uint32_t ST_BYTES = 5120, SC_OFS = 4096;
  static constexpr int TV = 1;
};
// Q5_K: the low 4 bits in the Q4_0 nibble layout, then per lane one dword
// of fifth bits per tile (kQ5HiPos), then per lane the 4 sub-blocks'
// (d*sc, -dmin*m) f16 pairs.
template <> struct Fmt<GEMV_Q5K> {
  static constexpr uint32_t ST_BYTES = 6144, HI_OFS = 4096, SC_OFS = 5120;
  static constexpr int TV = 1;
};
// Q5_K fifth bit of weight e of K run m sits at bit kQ5HiPos[e] + m of the
// tile's dword, so that the unpack's shifts (h >> m for elements 0-3,
// h >> (8 + m) for 4-5, h << (8 - m) for 6-7) bring it next to the nibble:
// to value 16 (bit 4 / 20) of a plain element, 256 (bit 8 / 24) of an
// element read as 16 * n.
__constant__ int kQ5HiPos[8] = {4, 20, 8, 24, 12, 28, 0, 16};

// (q & mask) | magic in one VOP3 op.  gfx9 VOP3 takes no literal and reads at
// most one scalar, so the mask comes from an SGPR and the magic from a VGPR.
__device__ __forceinline__ uint32_t and_or(uint32_t q, uint32_t mask_s, uint32_t magic_v) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(q), "s"(mask_s), "v"(magic_v));
  return r;
}

struct Unpack {
  uint32_t lo, hi;     // SGPR masks 0x000F000F, 0x00F000F0
  uint32_t h0, h1;     // SGPR masks 0x00300030, 0x03000300 (Q6_K high bits)
  uint32_t b4, b8;     // SGPR masks 0x00100010, 0x01000100 (Q5_K fifth bits)
  uint32_t magic;      // VGPR 0x64006400
};
// Materialise the constants once, opaque to the compiler, so the loop does
// not rebuild them per use.
__device__ __forceinline__ Unpack unpack_consts() {
  Unpack u;
  asm volatile("s_mov_b32 %0, 0x000f000f" : "=s"(u.lo));
  asm volatile("s_mov_b32 %0, 0x00f000f0" : "=s"(u.hi));
  asm volatile("s_mov_b32 %0, 0x00300030" : "=s"(u.h0));
  asm volatile("s_mov_b32 %0, 0x03000300" : "=s"(u.h1));
  asm volatile("s_mov_b32 %0, 0x00100010" : "=s"(u.b4));
  asm volatile("s_mov_b32 %0, 0x01000100" : "=s"(u.b8));
  asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(u.magic));
  return u;
}

__device__ __forceinline__ half8_t pack8(half2_t h0, half2_t h1, half2_t h2, half2_t h3) {
  half8_t r;
  r[0] = h0[0]; r[1] = h0[1]; r[2] = h1[0]; r[3] = h1[1];
  r[4] = h2[0]; r[5] = h2[1]; r[6] = h3[0]; r[7] = h3[1];
  return r;
}
__device__ __forceinline__ half2_t h2c(float v) { return (half2_t){(_Float16)v, (_Float16)v}; }

// Q4_0: 8 nibbles -> 8 f16 weights (n - 8) * d.  (n - 8) is exact; the
// product with the block scale is the one rounding.
__device__ __forceinline__ half8_t unpack8_q4(uint32_t q, const Unpack &u, half2_t dd) {
  const uint32_t q2 = q >> 8;
  const uint32_t t0 = and_or(q, u.lo, u.magic);    // 1024 + n0, 1024 + n4
  const uint32_t t1 = and_or(q, u.hi, u.magic);    // 1024 + 16 n1, 1024 + 16 n5
  const uint32_t t2 = and_or(q2, u.lo, u.magic);   // 1024 + n2, 1024 + n6
  const uint32_t t3 = and_or(q2, u.hi, u.magic);   // 1024 + 16 n3, 1024 + 16 n7
  const half2_t h0 = (__builtin_bit_cast(half2_t, t0) - h2c(1032.f)) * dd;
  const half2_t h1 = __builtin_elementwise_fma(__builtin_bit_cast(half2_t, t1), h2c(0.0625f), h2c(-72.f)) * dd;
  const half2_t h2 = (__builtin_bit_cast(half2_t, t2) - h2c(1032.f)) * dd;
  const half2_t h3 = __builtin_elementwise_fma(__builtin_bit_cast(half2_t, t3), h2c(0.0625f), h2c(-72.f)) * dd;
  return pack8(h0, h1, h2, h3);
}

// Q4_1 (w = n*d + m): the nibble extraction of unpack8_q4, n exact, then
// one fma per pair, rounded once to f16.
__device__ __forceinline__ half8_t unpack8_q41(uint32_t q, const Unpack &u, half2_t dd, half2_t mm) {
  const uint32_t q2 = q >> 8;
  const uint32_t t0 = and_or(q, u.lo, u.magic);    // 1024 + n0, 1024 + n4
  const uint32_t t1 = and_or(q, u.hi, u.magic);    // 1024 + 16 n1, 1024 + 16 n5
  const uint32_t t2 = and_or(q2, u.lo, u.magic);
  const uint32_t t3 = and_or(q2, u.hi, u.magic);
  const half2_t n0 = __builtin_bit_cast(half2_t, t0) - h2c(1024.f);
  const half2_t n1 = __builtin_elementwise_fma(__builtin_bit_cast(half2_t, t1), h2c(0.0625f), h2c(-64.f));
  const half2_t n2 = __builtin_bit_cast(half2_t, t2) - h2c(1024.f);
  const half2_t n3 = __builtin_elementwise_fma(__builtin_bit_cast(half2_t, t3), h2c(0.0625f), h2c(-64.f));
  return pack8(__builtin_elementwise_fma(n0, dd, mm), __builtin_elementwise_fma(n1, dd, mm),
               __builtin_elementwise_fma(n2, dd, mm), __builtin_elementwise_fma(n3, dd, mm));
}

// Q5_K (w = q*D + M, D = d*sc, M = -dmin*m, q = 5 bits): the nibble
// extraction of unpack8_q4 with the fifth bit ORed in (ha = h >> m,
// hb = h >> (8 + m), hc = h << (8 - m) for K run m), q exact, then one fma.
__device__ __forceinline__ half8_t unpack8_q5(uint32_t q, uint32_t ha, uint32_t hb, uint32_t hc, const Unpack &u,
                                              half2_t dd, half2_t mm) {
  const uint32_t q2 = q >> 8;
  const uint32_t t0 = and_or(ha, u.b4, and_or(q, u.lo, u.magic));    // 1024 + q0, 1024 + q4
  const uint32_t t1 = and_or(ha, u.b8, and_or(q, u.hi, u.magic));    // 1024 + 16 q1, 1024 + 16 q5
  const uint32_t t2 = and_or(hb, u.b4, and_or(q2, u.lo, u.magic));
  const uint32_t t3 = and_or(hc, u.b8, and_or(q2, u.hi, u.magic));
  const half2_t n0 = __builtin_bit_cast(half2_t, t0) - h2c(1024.f);
  const half2_t n1 = __builtin_elementwise_fma(__builtin_bit_cast(half2_t, t1), h2c(0.0625f), h2c(-64.f));
  const half2_t n2 = __builtin_bit_cast(half2_t, t2) - h2c(1024.f);
  const half2_t n3 = __builtin_elementwise_fma(__builtin_bit_cast(half2_t, t3), h2c(0.0625f), h2c(-64.f));
  return pack8(__builtin_elementwise_fma(n0, dd, mm), __builtin_elementwise_fma(n1, dd, mm),
               __builtin_elementwise_fma(n2, dd, mm), __builtin_elementwise_fma(n3, dd, mm));
}

// Q6_K: low nibbles as Q4_0 plus the 2 high bits of each weight, laid out in
// `h` so that one masked OR drops them above the nibble: weight e's bits sit
// at 4-5 / 20-21 (e = 0, 1), 8-9 / 24-25 (e = 2, 3) and, after h >> 2, the
// same places for e = 4..7.  The 6-bit value is exact in f16; q6 - 32 too.
__device__ __forceinline__ half8_t unpack8_q6(uint32_t q, uint32_t h, const Unpack &u, half2_t dd) {
  const uint32_t q2 = q >> 8, hs = h >> 2;
  const uint32_t t0 = and_or(h, u.h0, and_or(q, u.lo, u.magic));    // 1024 + q6
  const uint32_t t1 = and_or(h, u.h1, and_or(q, u.hi, u.magic));    // 1024 + 16 q6
  const uint32_t t2 = and_or(hs, u.h0, and_or(q2, u.lo, u.magic));
  const uint32_t t3 = and_or(hs, u.h1, and_or(q2, u.hi, u.magic));
  const half2_t h0 = (__builtin_bit_cast(half2_t, t0) - h2c(1056.f)) * dd;
  const half2_t h1 = __builtin_elementwise_fma(__builtin_bit_cast(half2_t, t1), h2c(0.0625f), h2c(-96.f)) * dd;
  const half2_t h2 = (__builtin_bit_cast(half2_t, t2) - h2c(1056.f)) * dd;
  const half2_t h3 = __builtin_elementwise_fma(__builtin_bit_cast(half2_t, t3), h2c(0.0625f), h2c(-96.f)) * dd;
  return pack8(h0, h1, h2, h3);
}
// The high bits of K run 2r+1 are stored rotated right by 8 in the dword of
// run 2r (their bits are exactly the ones run 2r leaves free).
__device__ __forceinline__ uint32_t rotl8(uint32_t h) { return __builtin_amdgcn_alignbit(h, h, 24); }

// Q8_0: 8 bytes (stored q + 128) -> 8 f16 weights q * d.
__device__ __forceinline__ half8_t unpack8_q8(uint32_t a, uint32_t b, uint32_t magic, half2_t dd) {
  // v_perm: bytes 0-3 come from the second operand, 4-7 from the first.
  // magic = 0x64006400: bytes 5 and 7 are 0x64, the f16 exponent of 1024.
  const uint32_t t0 = __builtin_amdgcn_perm(magic, a, 0x07010500u);  // 1024 + u0, 1024 + u1
  const uint32_t t1 = __builtin_amdgcn_perm(magic, a, 0x07030502u);
  const uint32_t t2 = __builtin_amdgcn_perm(magic, b, 0x07010500u);
  const uint32_t t3 = __builtin_amdgcn_perm(magic, b, 0x07030502u);
  const half2_t h0 = (__builtin_bit_cast(half2_t, t0) - h2c(1152.f)) * dd;
  const half2_t h1 = (__builtin_bit_cast(half2_t, t1) - h2c(1152.f)) * dd;
  const half2_t h2 = (__builtin_bit_cast(half2_t, t2) - h2c(1152.f)) * dd;
  const half2_t h3 = (__builtin_bit_cast(half2_t, t3) - h2c(1152.f)) * dd;
  return pack8(h0, h1, h2, h3);
}

// f16 in the low (hi = false) or high half of `w`, broadcast to both halves.
__device__ __forceinline__ half2_t bcast_half(uint32_t w, bool hi) {
  return __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(w, w, hi ? 0x03020302u : 0x01000100u));
}
// Two int8 (stored + 128) in bytes b, b+1 of w -> f16 pair, exactly.
__device__ __forceinline__ half2_t i8pair(uint32_t w, uint32_t magic, bool upper) {
  const uint32_t t = __builtin_amdgcn_perm(magic, w, upper ? 0x07030502u : 0x07010500u);
  return __builtin_bit_cast(half2_t, t) - h2c(1152.f);
}

// Total order on (logit, row) for the argmax: larger logit first, then the
// lower row.  NaN ranks as -inf and -0 as +0, so the maximum key is the first
// index of the maximum over the non-NaN logits -- argmax_of's strict '>' scan.
// A NaN in row 0 makes argmax_of return 0; that row gets the top key.
__device__ __forceinline__ unsigned long long amax_key(float v, int row) {
  if (row == 0 && v != v) return ~0ull;
  if (v != v) v = -__builtin_inff();
  if (v == 0.f) v = 0.f;
  uint32_t x = __builtin_bit_cast(uint32_t, v);
  x = (x & 0x80000000u) ? ~x : (x | 0x80000000u);
  return ((unsigned long long)x << 32) | (0xFFFFFFFFu - (uint32_t)row);
}
__device__ __forceinline__ int amax_row(unsigned long long key) { return (int)(0xFFFFFFFFu - (uint32_t)key); }

// Publish per-column argmax keys (atomic max, order-free), then the last
// workgroup to arrive reads the column maxima, runs the greedy walk over the
// drafts and clears the slots.  Runs with all 64*WAVES threads; `key[c]` is
// valid in threads c < 16 of the calling workgroup.
__device__ void argmax_finish(const unsigned long long *key, int B, const ArgmaxOut &a, int tid, int *s_flag) {
  if (tid < B && key[tid] != 0)
    __hip_atomic_fetch_max(a.keys + tid, key[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");  // maxima performed
  __syncthreads();
  if (tid == 0)
    *s_flag = __hip_atomic_fetch_add(a.cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (int)gridDim.x * gridDim.y - 1;
  __syncthreads();
  if (!*s_flag) return;
  if (tid == 0) {
    int am[CWEN_BMAX];
    for (int c = 0; c < B; ++c) {
      am[c] = amax_row(__hip_atomic_load(a.keys + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
      __hip_atomic_store(a.keys + c, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // run.c:4954-4956: k = longest prefix with argmax(row k) == draft k.
    int k = 0;
    while (k < a.E && am[k] == a.drafts[k]) ++k;
    a.out[0] = k;
    a.out[1] = am[k];
    for (int c = 0; c < B; ++c) a.out[2 + c] = am[c];
    __hip_atomic_store(a.cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

struct GemvParams {
  const uint8_t *w;    // super-tiled weights, round-major: super-tile (st, rg, side) at ((st*nrg + rg)*nsw + side)
  uint32_t wbytes;     // bytes of the tiled weights (buffer range)
  int nsw;             // sides stored per super-tile position (1 or 2)
  int side0;           // first side computed (NS == 1)
  int M, nrg, nst;
  // Workgroups [0, nsplit) each take one piece of a split row tile: piece
  // i % S (rounds (i % S) * rps ..) of tile tile0 + i / S.  The others take
  // whole row tiles 0, 1, ...
  int nsplit, S, rps, tile0;
  const _Float16 *xh;  // activations f16 [B][K]
  uint32_t xbytes;     // buffer range of the activations: columns >= B read as zero
  const float *xf;     // XN: f32 rows [c*xfs + k], converted to f16 while staging
  int xfs;
  // Post-scale (f16 operand w * x, x not yet normalised): output column c is
  // multiplied by 1 / sqrt(sum_p pss[p][c] / K + eps).
  const float *pss;
  int pnpart;
  float eps;
  int K, B;
  float *part;         // split-K partials
  int *cnt;            // per split-tile arrival counters (zero between launches)
  GemvOut out;
};

// 8 f32 activations -> 8 f16, rounded to nearest.
__device__ __forceinline__ uint4 cvt8(const uint4 (&x)[2]) {
  const float4 x0 = __builtin_bit_cast(float4, x[0]), x1 = __builtin_bit_cast(float4, x[1]);
  const half2_t h0 = {(_Float16)x0.x, (_Float16)x0.y}, h1 = {(_Float16)x0.z, (_Float16)x0.w};
  const half2_t h2 = {(_Float16)x1.x, (_Float16)x1.y}, h3 = {(_Float16)x1.z, (_Float16)x1.w};
  return make_uint4(__builtin_bit_cast(uint32_t, h0), __builtin_bit_cast(uint32_t, h1),
                    __builtin_bit_cast(uint32_t, h2), __builtin_bit_cast(uint32_t, h3));
}

// FMT: weight format.  NS: sides of an interleaved pair computed (2: both;
// the two waves of a wave pair take sides 0 and 1 of the same row group and
// combine them through LDS).  EPI: epilogue.  CB: activation columns staged
// (4, 8 or 16; >= B).  XN: f32 activations, converted to f16 while staging.
template <int FMT, int NS, int EPI, int CB, bool XN>
__global__ __launch_bounds__(64 * WAVES) void gemv_kernel(GemvParams p) {
  using F = Fmt<FMT>;
  constexpr int SPW = WAVES;                 // weight streams per workgroup (one per wave)
  constexpr int RPW = NS == 2 ? SPW / 2 : SPW;  // row groups per workgroup
  constexpr int TW = TILES;                  // tiles of a super-tile per wave
  constexpr int XL = CB / WAVES;             // staging loads per lane per round
  constexpr int TV = F::TV;
  // One round of weights in flight per wave: round rd + 1 is requested while
  // round rd is computed (measured: two rounds in flight were slower).
  constexpr int PD = 1;
  // The main loop's double-buffered activation chunks; the epilogue reuses
  // the same LDS for its exchanges, so a workgroup holds CB * 2 KB.
  __shared__ uint4 act[2][CB * 64];          // [buf][column c][unit u ^ c], f16 x 8 per unit
  __shared__ int s_last;

  const int tid = threadIdx.x;
  // Wave index as a scalar: loop bounds and addresses are then provably
  // wave-uniform, which keeps the loop's load-counter waits exact.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ws = wave;                             // stream of the workgroup
  const int lane = tid & 63;
  const int n = lane & 15, g = lane >> 4;
  const bool split = (int)blockIdx.x < p.nsplit;
  const int S = split ? p.S : 1;                   // pieces of this workgroup's row tile
  const int ti = split ? (int)blockIdx.x / p.S : 0;  // split tile: index of its partials and counter
  const int rt = split ? p.tile0 + ti : (int)blockIdx.x - p.nsplit;
  const int sp = split ? (int)blockIdx.x % p.S : 0;
  const int st0 = sp * p.rps;
  const int nround = split ? min(p.nst - st0, p.rps) : p.nst;

  // Post-scale: the producer's partial sums of squares of every staged
  // column, loaded first, so that waiting for them waits for nothing else
  // (see psc below).  ssq is [column][CWEN_MAX_PARTS = 128], so a wave's
  // load of 64 partials of one column is one contiguous 256-byte run, and the
  // loads need no guard.
  float pp[2][CB];
  if (p.pss) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int c = 0; c < CB; ++c) pp[j][c] = p.pss[c * CWEN_MAX_PARTS + lane + 64 * j];
  }
  __builtin_amdgcn_sched_barrier(0);
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(p.w, p.wbytes);
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(XN ? (const void *)p.xf : (const void *)p.xh, p.xbytes);

  // This wave's weight stream: row group rg, side `side`, super-tiles st0 ...
  // (round-major: consecutive rounds of a stream are nrg * nsw super-tiles
  // apart, so at any moment the launch reads one contiguous region).
  const uint32_t sstride = (uint32_t)p.nrg * p.nsw * F::ST_BYTES;
  const int side = NS == 2 ? (ws & 1) : p.side0;
  const int slot = NS == 2 ? ws >> 1 : ws;         // row-group slot of the workgroup
  const int rg = rt * RPW + slot;
  const int rgc = rg < p.nrg ? rg : p.nrg - 1;     // idle streams read a valid tile
  const uint32_t wofs = (((uint32_t)st0 * p.nrg + rgc) * p.nsw + side) * F::ST_BYTES;
  constexpr bool DM = FMT == GEMV_Q41 || FMT == GEMV_Q5K;  // per-block (scale, offset) pairs
  const uint32_t lq = lane * 16, ls = F::SC_OFS + lane * (DM ? 16 : 8);
  constexpr int jb = 0;                           // first tile of this wave

  // Activation staging: this wave copies columns c = wave + WAVES*i; lane
  // copies f16 unit `lane` (K elements 8*lane .. 8*lane+7) of the column's
  // 512-K chunk.
  constexpr uint32_t XE = XN ? 4 : 2;        // bytes per activation in memory
  const uint32_t xround = Q4_ST_K * XE;
  uint32_t xofs[XL];
  int xslot[XL];
#pragma unroll
  for (int i = 0; i < XL; ++i) {
    const int c = wave + WAVES * i;
    xofs[i] = (uint32_t)c * (uint32_t)(XN ? p.xfs : p.K) * XE + (uint32_t)st0 * xround + lane * 8 * XE;  // range-checked
    xslot[i] = c * 64 + (lane ^ c);
  }

  // Loads of one round's weight data: tile jb + t, vector v of the stream.
  auto tile_ofs = [&](int t, int v) -> uint32_t {
    return FMT == GEMV_Q8 ? lq + (jb + t) * 2048 + v * 1024 : lq + (jb + t) * 1024;
  };

  uint4 xs[XL][XN ? 2 : 1];
  uint4 wq[PD][TW][TV];
  // Scales of a round: 4 f16 (one per tile), or for Q4_1 / Q5_K 4 pairs.
  using ScT = std::conditional_t<DM, uint4, uint2>;
  ScT sc[PD];
  auto sc_load = [&](uint32_t soff) __attribute__((always_inline)) -> ScT {
    if constexpr (DM) return bload16_nt(wr, ls, soff);
    else return bload8_nt(wr, ls, soff);
  };
  uint4 h5[PD];               // Q5_K: fifth bits of the round's 4 tiles (one dword each)
  auto h5_load = [&](uint32_t soff) __attribute__((always_inline)) -> uint4 {
    if constexpr (FMT == GEMV_Q5K) return bload16_nt(wr, F::HI_OFS + lq, soff);
    else return make_uint4(0u, 0u, 0u, 0u);
  };
  uint32_t dq[PD] = {};       // Q6_K: f16 d of the round's two super-blocks
  constexpr int NHQ = (TW + 1) / 2;  // Q6_K: high-bit tile pairs of this wave
  uint4 hq[PD][NHQ];          // Q6_K: high bits of tile pairs (jb, jb+1) ...
  // Staging of round r of this piece.  K need only be a multiple of 32: the
  // last round's units past K (a lane's 8 elements lie wholly on one side)
  // get a per-lane offset beyond the buffer range and load as zeros, so they
  // meet the zero weights of the padded super-tile (never the next column's
  // activations, which could be infinite).
  auto stage_load = [&](uint32_t r) __attribute__((always_inline)) {
    const uint32_t soff = r * xround;
    const bool live = lane * 8 < p.K - (st0 + (int)r) * Q4_ST_K;
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      const uint32_t vo = live ? xofs[i] : kPastRange;
      xs[i][0] = bload16(xr, vo, soff);
      if constexpr (XN) xs[i][1] = bload16(xr, vo + 16, soff);
    }
  };
  stage_load(0);
#pragma unroll
  for (int k = 0; k < PD; ++k) {
    const uint32_t ok = wofs + (uint32_t)(k < nround ? k : nround - 1) * sstride;
    sc[k] = sc_load(ok);
    h5[k] = h5_load(ok);
    if constexpr (FMT == GEMV_Q6K) dq[k] = bload4_nt(wr, F::D_OFS + n * 4, ok);
#pragma unroll
    for (int t = 0; t < TW; ++t) {
#pragma unroll
      for (int v = 0; v < TV; ++v) wq[k][t][v] = bload16_nt(wr, tile_ofs(t, v), ok);
      if constexpr (FMT == GEMV_Q6K) {
        if (t & 1) hq[k][t >> 1] = bload16_nt(wr, F::HI_OFS + ((jb + t) >> 1) * 1024 + lq, ok);
      }
      __builtin_amdgcn_sched_barrier(0);  // issue the ring in slot order
    }
  }
  // Post-scale: the scales of this lane's output columns 4g .. 4g+3, while
  // the first round's weights are in flight.  Lane p adds partials p and
  // p + 64 in that order, then one DPP tree over the wave: a
  // fixed order, so every workgroup and every block size gets the same scale
  // for a column.  Every column index is a compile-time constant and nothing
  // branches per column (a private array indexed at run time would move to
  // LDS; a uniform branch per column reloads kernel arguments).
  float psc[4] = {1.f, 1.f, 1.f, 1.f};
  if (p.pss) {
    const float kf = (float)p.K, eps = p.eps;
    const int nb = p.B, np = p.pnpart;
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      float v = lane < np ? pp[0][c] : 0.f;
      if (lane + 64 < np) v += pp[1][c];
      const float sc1 = 1.f / sqrtf(sum64(v) / kf + eps);
      psc[c & 3] = ((c >> 2) == g && c < nb) ? sc1 : psc[c & 3];
    }
  }
  auto stage_store = [&](uint4 *buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      if constexpr (XN) buf[xslot[i]] = cvt8(xs[i]);
      else buf[xslot[i]] = xs[i][0];
    }
  };
  // CONV: the ring slot and pending buffer are read with the kernel's first
  // scalar loads; the taps and the history this lane's conv needs are
  // requested here, so only the epilogue waits for them.
  int cv_cur = 0, cv_P = 0;
  if constexpr (EPI == GEMV_EPI_CONV) {
    cv_cur = p.out.cv_ctl[0];
    cv_P = p.out.cv_ctl[3];
  }
  stage_store(act[0]);
  lds_barrier();
  float cv_h[3] = {0.f, 0.f, 0.f};
  float4 cv_w4 = {0.f, 0.f, 0.f, 0.f};
  const bool cv_rows = EPI == GEMV_EPI_CONV && rg * Q4_ROWS < p.out.cv_C;   // wave-uniform
  if constexpr (EPI == GEMV_EPI_CONV) {
    if (cv_rows) {
      const int row = rg * Q4_ROWS + n;
      cv_w4 = *(const float4 *)(p.out.cv_w + (size_t)row * 4);
      if (g == 0) {
        const float *hin = p.out.cv_H + (size_t)cv_cur * p.out.cv_C * 3 + (size_t)row * 3;
        cv_h[0] = hin[0];
        cv_h[1] = hin[1];
        cv_h[2] = hin[2];
      }
    }
  }

  const Unpack uc = unpack_consts();
  floatx4_t acc[2];
  acc[0] = acc[1] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
  // LDS unit of MFMA m of this wave's first tile for this lane (column n, K
  // run 4g + m); tile jb + t adds 16 (jb + t) units, which stay clear of the
  // XOR (n < 16).
  int aslot[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) aslot[m] = n * 64 + ((4 * g + m) ^ n) + 16 * jb;

  // One round = one super-tile of the stream.  The LDS buffer index is a
  // template constant (the loop is unrolled by two), so every LDS address is
  // a lane base plus an immediate.
  auto round = [&](int rd, auto cur_c) __attribute__((always_inline)) {
    constexpr int cur = decltype(cur_c)::value;
    // Next round's staging and the weights of round rd + PD (the last rounds
    // re-read the last super-tile, harmlessly).
    const uint32_t nr = (uint32_t)(rd + 1 < nround ? rd + 1 : rd);
    const uint32_t nw = (uint32_t)(rd + PD < nround ? rd + PD : nround - 1);
    const ScT &scc = sc[cur % PD];
    const uint32_t dqc = dq[cur % PD];
    // Scales of this round's tiles: dd[t][half] (Q4_0 / Q8_0: one per block,
    // both halves equal; Q6_K: one per 16-weight sub-block).
    half2_t dd[TW][2];
#pragma unroll
    for (int t = 0; t < TW; ++t) {
      if constexpr (FMT == GEMV_Q6K) {
        // sub-scale (exact in f16) * d, rounded once to f16
        const bool lo2 = t < 2;   // tiles 0-1: first super-block
        const uint32_t sw = lo2 ? scc.x : scc.y;
        const half2_t s2 = i8pair(sw, uc.magic, t & 1);
        const half2_t ds = s2 * bcast_half(dqc, !lo2);
        dd[t][0] = (half2_t){ds[0], ds[0]};
        dd[t][1] = (half2_t){ds[1], ds[1]};
      } else if constexpr (DM) {  // dd[t][0] = scale, dd[t][1] = offset
        const uint32_t w = t == 0 ? scc.x : t == 1 ? scc.y : t == 2 ? scc.z : scc.w;
        dd[t][0] = bcast_half(w, false);
        dd[t][1] = bcast_half(w, true);
      } else {
        const uint32_t w = t < 2 ? scc.x : scc.y;
        dd[t][0] = dd[t][1] = bcast_half(w, (t & 1) != 0);
      }
    }
    const uint4 h5c = h5[cur % PD];  // Q5_K: this round's fifth bits (the set is reloaded for round rd + PD)
    sc[cur % PD] = sc_load(wofs + nw * sstride);
    if constexpr (FMT == GEMV_Q5K) h5[cur % PD] = h5_load(wofs + nw * sstride);
    if constexpr (FMT == GEMV_Q6K) dq[cur % PD] = bload4_nt(wr, F::D_OFS + n * 4, wofs + nw * sstride);
    stage_load(nr);
    // LDS operands one tile ahead of their MFMAs: tile t + 1's reads are in
    // flight while tile t's products issue.
    half8_t an[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) an[m] = __builtin_bit_cast(half8_t, act[cur][aslot[m]]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < TW; ++t) {
      half8_t b[4];
      if constexpr (FMT == GEMV_Q4) {
        b[0] = unpack8_q4(wq[cur % PD][t][0].x, uc, dd[t][0]);
        b[1] = unpack8_q4(wq[cur % PD][t][0].y, uc, dd[t][0]);
        b[2] = unpack8_q4(wq[cur % PD][t][0].z, uc, dd[t][0]);
        b[3] = unpack8_q4(wq[cur % PD][t][0].w, uc, dd[t][0]);
      } else if constexpr (FMT == GEMV_Q5K) {
        const uint32_t h = t == 0 ? h5c.x : t == 1 ? h5c.y : t == 2 ? h5c.z : h5c.w;
        const half2_t d5 = dd[t][0], m5 = dd[t][1];
        b[0] = unpack8_q5(wq[cur % PD][t][0].x, h, h >> 8, h << 8, uc, d5, m5);
        b[1] = unpack8_q5(wq[cur % PD][t][0].y, h >> 1, h >> 9, h << 7, uc, d5, m5);
        b[2] = unpack8_q5(wq[cur % PD][t][0].z, h >> 2, h >> 10, h << 6, uc, d5, m5);
        b[3] = unpack8_q5(wq[cur % PD][t][0].w, h >> 3, h >> 11, h << 5, uc, d5, m5);
      } else if constexpr (FMT == GEMV_Q41) {
        b[0] = unpack8_q41(wq[cur % PD][t][0].x, uc, dd[t][0], dd[t][1]);
        b[1] = unpack8_q41(wq[cur % PD][t][0].y, uc, dd[t][0], dd[t][1]);
        b[2] = unpack8_q41(wq[cur % PD][t][0].z, uc, dd[t][0], dd[t][1]);
        b[3] = unpack8_q41(wq[cur % PD][t][0].w, uc, dd[t][0], dd[t][1]);
      } else if constexpr (FMT == GEMV_Q6K) {
        const uint4 &h4 = hq[cur % PD][t >> 1];
        const uint32_t ha = (t & 1) ? h4.z : h4.x;   // runs 0, 1
        const uint32_t hb = (t & 1) ? h4.w : h4.y;   // runs 2, 3
        b[0] = unpack8_q6(wq[cur % PD][t][0].x, ha, uc, dd[t][0]);
        b[1] = unpack8_q6(wq[cur % PD][t][0].y, rotl8(ha), uc, dd[t][0]);
        b[2] = unpack8_q6(wq[cur % PD][t][0].z, hb, uc, dd[t][1]);
        b[3] = unpack8_q6(wq[cur % PD][t][0].w, rotl8(hb), uc, dd[t][1]);
      } else {
        b[0] = unpack8_q8(wq[cur % PD][t][0].x, wq[cur % PD][t][0].y, uc.magic, dd[t][0]);
        b[1] = unpack8_q8(wq[cur % PD][t][0].z, wq[cur % PD][t][0].w, uc.magic, dd[t][0]);
        b[2] = unpack8_q8(wq[cur % PD][t][1].x, wq[cur % PD][t][1].y, uc.magic, dd[t][0]);
        b[3] = unpack8_q8(wq[cur % PD][t][1].z, wq[cur % PD][t][1].w, uc.magic, dd[t][0]);
      }
      // Refill the slots once their registers are consumed, so the loads
      // land in the same registers (no loop-carried copies, no counter drain).
#pragma unroll
      for (int v = 0; v < TV; ++v) wq[cur % PD][t][v] = bload16_nt(wr, tile_ofs(t, v), wofs + nw * sstride);
      if constexpr (FMT == GEMV_Q6K) {
        if (t & 1) hq[cur % PD][t >> 1] = bload16_nt(wr, F::HI_OFS + ((jb + t) >> 1) * 1024 + lq, wofs + nw * sstride);
      }
      half8_t a[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) a[m] = an[m];
      if (t + 1 < TW) {
#pragma unroll
        for (int m = 0; m < 4; ++m) an[m] = __builtin_bit_cast(half8_t, act[cur][aslot[m] + 16 * (t + 1)]);
      }
#pragma unroll
      for (int m = 0; m < 4; ++m)
        acc[m & 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[m], b[m], acc[m & 1], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);  // keep slots in issue order
    }
    stage_store(act[cur ^ 1]);
    lds_barrier();
  };
  int rd = 0;
  for (; rd + 1 < nround; rd += 2) {
    round(rd, std::integral_constant<int, 0>{});
    round(rd + 1, std::integral_constant<int, 1>{});
  }
  if (rd < nround) round(rd, std::integral_constant<int, 0>{});

  floatx4_t res = acc[0] + acc[1];
  // The epilogue's exchanges reuse the activation buffers (the main loop's
  // last barrier has passed).
  constexpr bool carry = true;

  if (EPI != GEMV_EPI_ARGMAX && S > 1) {
    // Publish this split's partials.  Agent-scope atomic stores reach the
    // device coherence point; the wait makes them complete before the
    // counter bump, and the last arriver reads them the same way.
    const bool cols_on = carry && g * 4 < p.B;
    uint64_t *part = (uint64_t *)p.part;
    const size_t base = (((size_t)ti * SPW + ws) * S + sp) * 128 + lane * 2;
    if (cols_on) {
      __hip_atomic_store(part + base, __builtin_bit_cast(uint64_t, (float2){res[0], res[1]}), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(part + base + 1, __builtin_bit_cast(uint64_t, (float2){res[2], res[3]}), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");  // stores acknowledged
    __builtin_amdgcn_s_barrier();
    if (tid == 0)
      s_last = __hip_atomic_fetch_add(p.cnt + ti, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == S - 1;
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    if (!s_last) return;   // workgroup-uniform
    // Sum the splits in split order.  The loads of a chunk of KCH splits are
    // all issued before the first is consumed, so the reduction costs one
    // memory round trip per chunk, not one per split.
    constexpr int KCH = 8;
    res = (floatx4_t){0.f, 0.f, 0.f, 0.f};
    if (cols_on) {
      const size_t b0 = (((size_t)ti * SPW + ws) * S) * 128 + lane * 2;
      for (int k0 = 0; k0 < S; k0 += KCH) {
        uint64_t lo[KCH], hi[KCH];
#pragma unroll
        for (int u = 0; u < KCH; ++u) {
          const size_t k = (size_t)min(k0 + u, S - 1);
          lo[u] = __hip_atomic_load(part + b0 + k * 128, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          hi[u] = __hip_atomic_load(part + b0 + k * 128 + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (int u = 0; u < KCH; ++u)
          if (k0 + u < S) {
            const float2 a = __builtin_bit_cast(float2, lo[u]);
            const float2 b = __builtin_bit_cast(float2, hi[u]);
            res += (floatx4_t){a.x, a.y, b.x, b.y};
          }
      }
    }
    if (tid == 0) __hip_atomic_store(p.cnt + ti, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  if (p.pss) {
#pragma unroll
    for (int e = 0; e < 4; ++e) res[e] *= psc[e];
  }
  const GemvOut &o = p.out;
  const int row = rg * Q4_ROWS + n;
  const bool row_ok = carry && rg < p.nrg && row < p.M;
  if constexpr (EPI == GEMV_EPI_ARGMAX) {
    // Logits (optional), then the per-column argmax over this workgroup's
    // rows: lane (g, n) holds row n of its row group for columns 4g..4g+3.
    unsigned long long *const s_key = (unsigned long long *)&act[1][0];   // [SPW][16]
    unsigned long long best[4] = {0, 0, 0, 0};
    if (row_ok) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int c = g * 4 + e;
        if (c < p.B && o.y) o.y[(size_t)c * o.ys + row] = res[e];
        best[e] = amax_key(res[e], row);
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
#pragma unroll
      for (int sh = 1; sh < 16; sh <<= 1) {
        const unsigned long long other = __shfl_xor(best[e], sh, 16);
        best[e] = other > best[e] ? other : best[e];
      }
    }
    if (carry && n == 0) {
#pragma unroll
      for (int e = 0; e < 4; ++e) s_key[ws * 16 + g * 4 + e] = best[e];
    }
    __syncthreads();
    unsigned long long *const s_col = s_key + SPW * 16;   // [16]
    if (tid < 16) {
      unsigned long long k = s_key[tid];
#pragma unroll
      for (int w = 1; w < SPW; ++w) k = s_key[w * 16 + tid] > k ? s_key[w * 16 + tid] : k;
      s_col[tid] = k;
    }
    __syncthreads();
    argmax_finish(s_col, p.B, o.am, tid, &s_last);
    return;
  }

  floatx4_t up = (floatx4_t){0.f, 0.f, 0.f, 0.f};  // SwiGLU: the up side from the partner wave
  bool store = row_ok;
  if constexpr (NS == 2 && EPI == GEMV_EPI_SWIGLU) {
    floatx4_t *const s_up = (floatx4_t *)&act[1][0];   // [RPW][64]
    if (carry && (ws & 1)) s_up[slot * 64 + lane] = res;
    __syncthreads();
    store = row_ok && !(ws & 1);   // the gate wave stores the pair's output
    if (store) up = s_up[slot * 64 + lane];
  }
  float *const y0 = (NS == 2 && EPI == GEMV_EPI_PAIR && (ws & 1)) ? o.y1 : o.y;  // PAIR: each side its own output

  float sq[4] = {0.f, 0.f, 0.f, 0.f};  // this lane's share of the row tile's sum of squares
  bool bad = false;                    // an f16 copy out of range
  if constexpr (NS == 1 && EPI == GEMV_EPI_CONV) {
    // GatedDeltaNet conv rows: lane (g, n) holds positions 4g .. 4g+3 of
    // channel `row`; positions 4g-3 .. 4g-1 come from lane (g-1, n), or for
    // g = 0 from the history slot the block starts from.
    if (cv_rows) {
      const float p1 = __shfl(res[1], lane - 16), p2 = __shfl(res[2], lane - 16), p3 = __shfl(res[3], lane - 16);
      if (store) {
        const int cur = cv_cur, P = cv_P;
        const size_t hf = (size_t)o.cv_C * 3;
        float a[7];
        a[0] = g == 0 ? cv_h[0] : p1;
        a[1] = g == 0 ? cv_h[1] : p2;
        a[2] = g == 0 ? cv_h[2] : p3;
#pragma unroll
        for (int e = 0; e < 4; ++e) a[3 + e] = res[e];
        const float4 w = cv_w4;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int b = g * 4 + e;
          if (b >= p.B) continue;
          // ((st0*w0 + st1*w1) + st2*w2) + xin*w3, each product and sum rounded
          const float x = __fadd_rn(__fadd_rn(__fadd_rn(__fmul_rn(a[e], w.x), __fmul_rn(a[e + 1], w.y)),
                                              __fmul_rn(a[e + 2], w.z)),
                                    __fmul_rn(a[e + 3], w.w));
          o.cv_xc[((size_t)P * CWEN_BMAX + b) * o.cv_C + row] = silu_f(x);
          float *hs = o.cv_H + (size_t)((cur + 1 + b) % o.cv_nslot) * hf + (size_t)row * 3;
          hs[0] = a[e + 1];
          hs[1] = a[e + 2];
          hs[2] = a[e + 3];
        }
      }
      store = false;
    }
  }
  if (store) {
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if constexpr (NS == 2 && EPI == GEMV_EPI_SWIGLU) v[e] = silu_f(res[e]) * up[e];
      else v[e] = res[e];
    }
    const float nwr = o.yh && o.nwh ? o.nwh[row] : 1.f;  // loaded with the residual
    if (y0 && o.accumulate) {  // all residual loads in flight together
      float old[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int c = g * 4 + e;
        old[e] = c < p.B ? y0[(size_t)c * o.ys + row] : 0.f;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] += old[e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = g * 4 + e;
      if (c >= p.B) continue;
      if (y0) y0[(size_t)c * o.ys + row] = v[e];
      if (o.yh) {
        const _Float16 h = (_Float16)(o.nwh ? v[e] * nwr : v[e]);
        o.yh[(size_t)c * p.M + row] = h;
        bad |= f16_bad(h);
      }
      sq[e] = fmaf(v[e], v[e], sq[e]);
    }
  }
  if (bad) raise_flag(o.rflag);
  if (o.ssq) {
    // Sum of squares of this row tile's outputs per column, in a fixed order
    // (rows of a wave by the DPP tree, then row groups in order): ssq[c][rt],
    // the partials a normalising consumer sums.  (STORE only: NS == 1, so
    // slot == ws.)
    float *const s_sq = (float *)&act[0][0];   // [SPW][16]
#pragma unroll
    for (int e = 0; e < 4; ++e) sq[e] = sum16(sq[e]);
    if (carry && n == 0) {
#pragma unroll
      for (int e = 0; e < 4; ++e) s_sq[ws * 16 + g * 4 + e] = sq[e];
    }
    __syncthreads();
    if (tid < 16 && tid < p.B) {
      float t = s_sq[tid];
#pragma unroll
      for (int w = 1; w < SPW; ++w) t += s_sq[w * 16 + tid];
      o.ssq[tid * CWEN_MAX_PARTS + rt] = t;
    }
  }
}

// ------------------------------------------------------------------ repack
// One thread per (row group, super-tile, side, lane).  Rows past M get zero
// weights (zero scales).

// Q4_0 family and Q4_1: lane l = 16g + n gets, for each tile u, block g of
// that tile for row n -- 4 dwords, dword j holding K run j (weights 8j..8j+7
// of the block) in kNibPos order -- and the 4 blocks' f16 scales (Q4_1: the 4
// blocks' (d, m) pairs).  The source (M rows,
// nrg row groups) lands at destination row group rg_off onward; side_sel >= 0
// takes that side of a Q4_0RSI source into a single-sided destination.
__global__ void repack_q4_kernel(uint8_t *dst, const uint8_t *src, const uint16_t *sc, int type,
                                 int M, int K, int nrg, int nst, int nsw, int rg_off, int side_sel, int nrg_dst) {
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
  const int sside = side_sel >= 0 ? side_sel : side;
  const bool q41 = type == CWEN_T_Q4_1;
  const uint32_t stb = q41 ? Fmt<GEMV_Q41>::ST_BYTES : Fmt<GEMV_Q4>::ST_BYTES;
  uint8_t *stile = dst + (((size_t)st * nrg_dst + rg + rg_off) * nsw + side) * stb;   // round-major
  uint16_t d[TILES], m[TILES];
  for (int u = 0; u < TILES; ++u) {
    const int blk = (st * TILES + u) * 4 + g;
    const uint8_t *qs = nullptr;
    d[u] = m[u] = 0;  // rows past M and blocks past K: zero weights
    if (row < M && blk < nb) {
      const size_t bi = (size_t)row * nb + blk;
      if (type == CWEN_T_Q4_0) {
        const uint8_t *b = src + bi * 18;
        d[u] = (uint16_t)(b[0] | (b[1] << 8));
        qs = b + 2;
      } else if (q41) {  // {f16 d; f16 m; u8 qs[16]}
        const uint8_t *b = src + bi * 20;
        d[u] = (uint16_t)(b[0] | (b[1] << 8));
        m[u] = (uint16_t)(b[2] | (b[3] << 8));
        qs = b + 4;
      } else if (type == CWEN_T_Q4_0RS) {
        qs = src + bi * 16;
        d[u] = sc[bi];
      } else {  // Q4_0RSI
        qs = src + bi * 32 + sside * 16;
        d[u] = sc[bi * 2 + sside];
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
    *(uint4 *)(stile + u * 1024 + lane * 16) = make_uint4(out[0], out[1], out[2], out[3]);
  }
  if (q41)
    *(uint4 *)(stile + Fmt<GEMV_Q41>::SC_OFS + lane * 16) =
        make_uint4((uint32_t)d[0] | ((uint32_t)m[0] << 16), (uint32_t)d[1] | ((uint32_t)m[1] << 16),
                   (uint32_t)d[2] | ((uint32_t)m[2] << 16), (uint32_t)d[3] | ((uint32_t)m[3] << 16));
  else
    *(uint2 *)(stile + Fmt<GEMV_Q4>::SC_OFS + lane * 8) =
        make_uint2((uint32_t)d[0] | ((uint32_t)d[1] << 16), (uint32_t)d[2] | ((uint32_t)d[3] << 16));
}

// Q6_K (run.c:115, 1212-1229): weight j of a super-block (j = 0..255) is
// q6 = (nibble of ql[64h + l + 32(t&1)], low for t < 2) | ((qh[32h + l] >> 2t) & 3) << 4
// with h = j/128, t = (j%128)/32, l = j%32, times d * sc[j/16].
__device__ inline int q6_value(const uint8_t *b, int j) {
  const int h = j >> 7, r = j & 127, t = r >> 5, l = r & 31;
  const uint8_t qlb = b[64 * h + l + 32 * (t & 1)];
  const int nib = (t < 2) ? (qlb & 0xF) : (qlb >> 4);
  const int hb = (b[128 + 32 * h + l] >> (2 * t)) & 3;
  return nib | (hb << 4);
}
// Bit position of weight e's high pair in the run's dword (see unpack8_q6).
__constant__ int kQ6HiPos[8] = {4, 20, 8, 24, 6, 22, 10, 26};

// Q5_K (GGUF 176-byte super-blocks, run.c:1142-1156): lane l = 16g + n gets,
// for each tile u, sub-block g of that tile for row n (32 weights, one
// Q5_K sub-block): the low 4 bits in the Q4_0 nibble layout, the fifth bits
// in one dword (kQ5HiPos), and (f16(d*sc), f16(-dmin*m)) of the sub-block.
__global__ void repack_q5k_kernel(uint8_t *dst, const uint8_t *src, int M, int K, int nrg, int nst) {
  const size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t total = (size_t)nrg * nst * 64;
  if (id >= total) return;
  const int lane = (int)(id & 63);
  const size_t t = id >> 6;
  const int st = (int)(t % nst);
  const int rg = (int)(t / nst);
  const int n = lane & 15, g = lane >> 4;
  const int row = rg * Q4_ROWS + n;
  const int nsb = K / 256;
  using F = Fmt<GEMV_Q5K>;
  uint8_t *stile = dst + ((size_t)st * nrg + rg) * F::ST_BYTES;   // round-major
  uint32_t hw[TILES], dm[TILES];
  for (int u = 0; u < TILES; ++u) {
    const int k0 = st * Q4_ST_K + u * Q4_TILE_K + g * 32;   // first K of the lane's sub-block
    const uint8_t *b = (row < M && k0 < K) ? src + ((size_t)row * nsb + k0 / 256) * 176 : nullptr;
    const int sb = (k0 & 255) / 32, jj = sb / 2, hs = sb & 1;
    uint32_t lo[4] = {0, 0, 0, 0};
    hw[u] = 0;
    dm[u] = 0;   // rows past M: zero weights
    if (b) {
      const uint8_t *scales = b + 4, *qh = b + 16, *ql = b + 48 + 32 * jj;
      for (int m = 0; m < 4; ++m)
        for (int e = 0; e < 8; ++e) {
          const int l = 8 * m + e;   // weight l of the sub-block
          const uint32_t nib = hs ? (ql[l] >> 4) : (ql[l] & 15u);
          const uint32_t h5 = (qh[l] >> (2 * jj + hs)) & 1u;
          lo[m] |= nib << (4 * kNibPos[e]);
          hw[u] |= h5 << (kQ5HiPos[e] + m);
        }
      // run.c:426-429 get_scale_min_k4
      int sc, mn;
      if (sb < 4) {
        sc = scales[sb] & 63;
        mn = scales[sb + 4] & 63;
      } else {
        sc = (scales[sb + 4] & 0xF) | ((scales[sb - 4] >> 6) << 4);
        mn = (scales[sb + 4] >> 4) | ((scales[sb] >> 6) << 4);
      }
      const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(b[0] | (b[1] << 8)));
      const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(b[2] | (b[3] << 8)));
      const _Float16 D = (_Float16)(d * (float)sc), Mo = (_Float16)(-(dmin * (float)mn));
      dm[u] = (uint32_t)__builtin_bit_cast(uint16_t, D) | ((uint32_t)__builtin_bit_cast(uint16_t, Mo) << 16);
    }
    *(uint4 *)(stile + u * 1024 + lane * 16) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
  }
  *(uint4 *)(stile + F::HI_OFS + lane * 16) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
  *(uint4 *)(stile + F::SC_OFS + lane * 16) = make_uint4(dm[0], dm[1], dm[2], dm[3]);
}

__global__ void repack_q6k_kernel(uint8_t *dst, const uint8_t *src, int M, int K, int nrg, int nst) {
  const size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t total = (size_t)nrg * nst * 64;
  if (id >= total) return;
  const int lane = (int)(id & 63);
  const size_t t = id >> 6;
  const int st = (int)(t % nst);
  const int rg = (int)(t / nst);
  const int n = lane & 15, g = lane >> 4;
  const int row = rg * Q4_ROWS + n;
  const int nsb = K / 256;
  using F = Fmt<GEMV_Q6K>;
  uint8_t *stile = dst + ((size_t)st * nrg + rg) * F::ST_BYTES;   // round-major
  uint8_t scb[8];
  uint32_t hiw[TILES][2];
  for (int u = 0; u < TILES; ++u) {
    const int k0 = st * Q4_ST_K + u * Q4_TILE_K + g * 32;   // first K of the lane's block
    const uint8_t *b = (row < M && k0 < K) ? src + ((size_t)row * nsb + k0 / 256) * 210 : nullptr;
    const int j0 = k0 & 255;
    uint32_t lo[4] = {0, 0, 0, 0}, hi[4] = {0, 0, 0, 0};
    for (int m = 0; m < 4; ++m)
      for (int e = 0; e < 8; ++e) {
        const int v = b ? q6_value(b, j0 + 8 * m + e) : 32;   // 32: weight 0
        lo[m] |= (uint32_t)(v & 15) << (4 * kNibPos[e]);
        hi[m] |= (uint32_t)(v >> 4) << kQ6HiPos[e];
      }
    *(uint4 *)(stile + u * 1024 + lane * 16) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    // runs 2r+1 rotated right by 8 into the free bits of run 2r
    hiw[u][0] = hi[0] | ((hi[1] >> 8) | (hi[1] << 24));
    hiw[u][1] = hi[2] | ((hi[3] >> 8) | (hi[3] << 24));
    for (int h = 0; h < 2; ++h) {
      const int sub = (j0 >> 4) + h;
      scb[u * 2 + h] = (uint8_t)((b ? (int)(int8_t)b[192 + sub] : 0) + 128);
    }
  }
  for (int p = 0; p < 2; ++p)
    *(uint4 *)(stile + F::HI_OFS + p * 1024 + lane * 16) =
        make_uint4(hiw[2 * p][0], hiw[2 * p][1], hiw[2 * p + 1][0], hiw[2 * p + 1][1]);
  uint2 scw;
  scw.x = scb[0] | (scb[1] << 8) | (scb[2] << 16) | ((uint32_t)scb[3] << 24);
  scw.y = scb[4] | (scb[5] << 8) | (scb[6] << 16) | ((uint32_t)scb[7] << 24);
  *(uint2 *)(stile + F::SC_OFS + lane * 8) = scw;
  if (g == 0) {  // d of the super-tile's two super-blocks for row n
    uint16_t d0 = 0, d1 = 0;   // super-blocks past K: zero
    if (row < M) {
      const uint8_t *b0 = src + ((size_t)row * nsb + st * 2) * 210;
      d0 = (uint16_t)(b0[208] | (b0[209] << 8));
      if (st * 2 + 1 < nsb) d1 = (uint16_t)(b0[210 + 208] | (b0[210 + 209] << 8));
    }
    *(uint32_t *)(stile + F::D_OFS + n * 4) = (uint32_t)d0 | ((uint32_t)d1 << 16);
  }
}

// Q8_0 (run.c:106, 1248-1274): lane l = 16g + n gets block g of each tile
// for row n as two 16-byte halves (bytes stored q + 128), and the 4 blocks'
// f16 scales.
__global__ void repack_q8_kernel(uint8_t *dst, const uint8_t *src, int M, int K, int nrg, int nst) {
  const size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t total = (size_t)nrg * nst * 64;
  if (id >= total) return;
  const int lane = (int)(id & 63);
  const size_t t = id >> 6;
  const int st = (int)(t % nst);
  const int rg = (int)(t / nst);
  const int n = lane & 15, g = lane >> 4;
  const int row = rg * Q4_ROWS + n;
  const int nb = K / 32;
  using F = Fmt<GEMV_Q8>;
  uint8_t *stile = dst + ((size_t)st * nrg + rg) * F::ST_BYTES;   // round-major
  uint16_t d[TILES];
  for (int u = 0; u < TILES; ++u) {
    const int blk = (st * TILES + u) * 4 + g;
    const uint8_t *b = (row < M && blk < nb) ? src + ((size_t)row * nb + blk) * 34 : nullptr;
    d[u] = b ? (uint16_t)(b[0] | (b[1] << 8)) : 0;
    uint8_t v[32];
    for (int k = 0; k < 32; ++k) v[k] = (uint8_t)((b ? (int)(int8_t)b[2 + k] : 0) + 128);
    for (int h = 0; h < 2; ++h) {
      uint32_t w4[4];
      for (int i = 0; i < 4; ++i)
        w4[i] = v[16 * h + 4 * i] | (v[16 * h + 4 * i + 1] << 8) | (v[16 * h + 4 * i + 2] << 16) |
                ((uint32_t)v[16 * h + 4 * i + 3] << 24);
      *(uint4 *)(stile + u * 2048 + h * 1024 + lane * 16) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
    }
  }
  *(uint2 *)(stile + F::SC_OFS + lane * 8) =
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

// Argmax of B rows of given logits plus the walk: grid (chunks, B); each
// workgroup scans one chunk of one row.
constexpr int AM_CHUNK = 8192;
__global__ __launch_bounds__(256) void argmax_walk_kernel(const float *lg, long ls, int V, int B, ArgmaxOut a) {
  __shared__ unsigned long long s_k[256];
  __shared__ unsigned long long s_col[CWEN_BMAX];
  __shared__ int s_flag;
  const int tid = threadIdx.x;
  const int b = blockIdx.y;
  const int i0 = blockIdx.x * AM_CHUNK;
  const int i1 = min(V, i0 + AM_CHUNK);
  const float *row = lg + (size_t)b * ls;
  unsigned long long best = 0;
  for (int i = i0 + tid; i < i1; i += 256) {
    const unsigned long long k = amax_key(row[i], i);
    best = k > best ? k : best;
  }
  s_k[tid] = best;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (tid < s) s_k[tid] = s_k[tid + s] > s_k[tid] ? s_k[tid + s] : s_k[tid];
    __syncthreads();
  }
  // Only column b carries a key; the others stay 0 (no-op maxima).
  if (tid < CWEN_BMAX) s_col[tid] = tid == b ? s_k[0] : 0ull;
  __syncthreads();
  argmax_finish(s_col, B, a, tid, &s_flag);
}

template <int FMT, int NS, int EPI, int CB, bool XN>
void launch_one(const GemvParams &p, int grid, hipStream_t st) {
  hipLaunchKernelGGL((gemv_kernel<FMT, NS, EPI, CB, XN>), dim3((unsigned)grid), dim3(64 * WAVES), 0, st, p);
}

template <int FMT, int NS, int EPI, bool XN>
void launch_xn(const GemvParams &p, int nrt, hipStream_t st) {
  if (p.B <= 4) launch_one<FMT, NS, EPI, 4, XN>(p, nrt, st);
  else if (p.B <= 8) launch_one<FMT, NS, EPI, 8, XN>(p, nrt, st);
  else launch_one<FMT, NS, EPI, 16, XN>(p, nrt, st);
}

template <int FMT, int NS, int EPI>
void launch_cb(const GemvParams &p, int nrt, hipStream_t st) {
  if (p.xf) launch_xn<FMT, NS, EPI, true>(p, nrt, st);
  else launch_xn<FMT, NS, EPI, false>(p, nrt, st);
}

template <int FMT>
int launch_fmt(const GemvParams &p, int nrt, int nsides, int epi, hipStream_t st) {
  if (nsides == 1 && epi == GEMV_EPI_STORE) {
    launch_cb<FMT, 1, GEMV_EPI_STORE>(p, nrt, st);
  } else if (nsides == 1 && epi == GEMV_EPI_ARGMAX) {
    launch_cb<FMT, 1, GEMV_EPI_ARGMAX>(p, nrt, st);
  } else {
    return CWEN_EINVAL;
  }
  return CWEN_OK;
}

}  // namespace

int gemv_fmt_of(int type) {
  switch (type) {
    case CWEN_T_Q4_0: case CWEN_T_Q4_0RS: case CWEN_T_Q4_0RSI: return GEMV_Q4;
    case CWEN_T_Q6_K: return GEMV_Q6K;
    case CWEN_T_Q8_0: return GEMV_Q8;
    case CWEN_T_Q4_1: return GEMV_Q41;
    case CWEN_T_Q5_K: return GEMV_Q5K;
    default: return -1;
  }
}

size_t gemv_st_bytes(int fmt) {
  return fmt == GEMV_Q4 ? Fmt<GEMV_Q4>::ST_BYTES : fmt == GEMV_Q6K ? Fmt<GEMV_Q6K>::ST_BYTES
       : fmt == GEMV_Q41  ? Fmt<GEMV_Q41>::ST_BYTES : fmt == GEMV_Q5K ? Fmt<GEMV_Q5K>::ST_BYTES
                          : Fmt<GEMV_Q8>::ST_BYTES;
}

int gemv_repack(cwen_weight *w, const uint8_t *dsrc, const uint16_t *dsc, hipStream_t st) {
  const size_t threads = (size_t)w->nrg * w->nst * w->nside * 64;
  const int blk = 256;
  const size_t grid = (threads + blk - 1) / blk;
  if (w->fmt == GEMV_Q4 || w->fmt == GEMV_Q41)
    hipLaunchKernelGGL(repack_q4_kernel, dim3((unsigned)grid), dim3(blk), 0, st, w->dev, dsrc, dsc,
                       w->type, w->ne1, w->ne0, w->nrg, w->nst, w->nside, 0, -1, w->nrg);
  else if (w->fmt == GEMV_Q6K)
    hipLaunchKernelGGL(repack_q6k_kernel, dim3((unsigned)grid), dim3(blk), 0, st, w->dev, dsrc, w->ne1,
                       w->ne0, w->nrg, w->nst);
  else if (w->fmt == GEMV_Q5K)
    hipLaunchKernelGGL(repack_q5k_kernel, dim3((unsigned)grid), dim3(blk), 0, st, w->dev, dsrc, w->ne1,
                       w->ne0, w->nrg, w->nst);
  else
    hipLaunchKernelGGL(repack_q8_kernel, dim3((unsigned)grid), dim3(blk), 0, st, w->dev, dsrc, w->ne1,
                       w->ne0, w->nrg, w->nst);
  CWEN_HIP_TRY(hipGetLastError());
  return CWEN_OK;
}

int gemv_repack_part(cwen_weight *w, const uint8_t *dsrc, const uint16_t *dsc, int type, int M, int row_off,
                     int side_sel, hipStream_t st) {
  if (w->fmt != GEMV_Q4 || w->nside != 1 || row_off % Q4_ROWS || row_off + M > w->ne1) return CWEN_EINVAL;
  if ((side_sel >= 0) != (type == CWEN_T_Q4_0RSI) || side_sel > 1) return CWEN_EINVAL;
  const int nrg = (M + Q4_ROWS - 1) / Q4_ROWS;
  const size_t threads = (size_t)nrg * w->nst * 64;
  const int blk = 256;
  hipLaunchKernelGGL(repack_q4_kernel, dim3((unsigned)((threads + blk - 1) / blk)), dim3(blk), 0, st, w->dev, dsrc,
                     dsc, type, M, w->ne0, nrg, w->nst, 1, row_off / Q4_ROWS, side_sel, w->nrg);
  CWEN_HIP_TRY(hipGetLastError());
  return CWEN_OK;
}

// Split-K scratch of a decomposition: WAVES x 256 partial floats per piece
// at most (one 16-row stream per wave) and one arrival counter per split
// tile.
bool gemv_grid_fits(const GemvGrid &g, size_t partials_floats, int ncounters) {
  return g.nsplit == 0 || ((size_t)g.nsplit * WAVES * 256 <= partials_floats && g.nsplit / g.S <= ncounters);
}

namespace {
// Row groups of one workgroup (its row tile): one 16-row stream per wave; a
// pair computed whole puts its two sides on a wave pair.
int tile_rows(int nsides) { return nsides == 2 ? WAVES / 2 : WAVES; }

// Estimated length of a launch (microseconds at the 27B FFN shape's rates).
// Workgroup i runs on CU i mod ncu (dispatch fills every CU's first slot,
// then every second slot, ...).  A workgroup's work is its rounds plus one
// round of start-up.  The workgroups on a CU share it evenly, at a total
// rate that grows with how many are still running (a lone four-wave
// workgroup is latency-bound), so a short piece slows a whole tile on its
// CU only while both run; the busiest CU sets the length.  Rates from
// 16480 x 5120 at B = 8 (258 tiles of 10 rounds): 12.0-12.4 us for a lone
// tile per CU, 15.6 us with two whole tiles on two CUs, 14.5 / 13.2 / 13.2
// us with the two last tiles split in 2 / 5 / 10 pieces.
// Split remainder tiles add their partial-sum hand-off, early in the launch:
// their pieces are dispatched first, so they are the oldest workgroups on
// their CUs, which the hardware serves first.
constexpr double kSplitEarly = 0.3;
double cu_rate(int wgs) {  // rounds per microsecond, all of a CU's workgroups together
  return wgs <= 1 ? 0.77 : wgs == 2 ? 1.2 : wgs == 3 ? 1.35 : wgs == 4 ? 1.45 : 1.5;
}
// Time for one CU to finish workgroups of the given lengths (in rounds),
// shared evenly among those still running.
double cu_time(std::vector<double> &len) {
  std::sort(len.begin(), len.end());
  double t = 0.0, done = 0.0;
  const int n = (int)len.size();
  for (int i = 0; i < n; ++i) {
    t += (len[(size_t)i] - done) * (n - i) / cu_rate(n - i);
    done = len[(size_t)i];
  }
  return t;
}
double grid_cost(int ncu, int nst, const GemvGrid &c, double extra) {
  std::vector<std::vector<double>> len((size_t)ncu);
  for (int i = 0; i < c.grid; ++i) {
    const int nr = i < c.nsplit ? std::min(nst - (i % c.S) * c.rps, c.rps) : nst;
    len[(size_t)(i % ncu)].push_back(nr + 1.0);
  }
  double worst = 0.0;
  for (auto &l : len)
    if (!l.empty()) worst = std::max(worst, cu_time(l));
  return worst + extra;
}

// Decomposition of ntile row tiles of nst rounds.  A launch with fewer tiles
// than CUs splits every tile into S pieces (at least two rounds each)
// for at most wg_per_cu workgroups per CU.  A larger one takes whole tiles,
// except that the ntile mod ncu remainder tiles are split into the pieces
// (chosen by grid_cost) that spread them over the CUs: without that, the
// CUs that get one whole tile more than the others would set the launch's
// length.
// split_basis: the tile count that sizes the split (the single-side one for
// both launch kinds, so a pair launch splits K as its single sides do).
GemvGrid choose_grid(const cwen_ctx *ctx, int ntile, int nst, int split_basis) {
  GemvGrid best = {ntile, 0, 1, nst, 0};
  // More than half as many tiles as CUs: whole tiles, one per CU.  Split in
  // two, most CUs would get two pieces of the same total length plus the
  // partials' round trip (measured at 224 tiles of 10 rounds: 10.7 us whole,
  // 12.1 us split).
  if (ntile < ctx->ncu && 2 * ntile > ctx->ncu) return best;
  if (ntile < ctx->ncu) {
    const int target = ctx->wg_per_cu * ctx->ncu;
    // At most wg_per_cu workgroups per CU for a single-side launch (one more
    // on some CUs than on the others would set the launch's length); a pair
    // launch, twice the tiles, takes the same pieces.
    int S = std::min(std::max(target / split_basis, 1), std::max(nst / 2, 1));
    const int rps = (nst + S - 1) / S;
    S = (nst + rps - 1) / rps;
    const GemvGrid cand = {ntile * S, ntile * S, S, rps, 0};
    if (S > 1 && gemv_grid_fits(cand, ctx->partials_floats, ctx->ncounters)) best = cand;
    return best;
  }
  const int rem = ntile % ctx->ncu;
  if (rem == 0) return best;
  double best_cost = grid_cost(ctx->ncu, nst, best, 0.0);
  for (int s = 2; s <= nst / 2; ++s) {
    const int r = (nst + s - 1) / s, se = (nst + r - 1) / r;
    const GemvGrid part = {rem * se + ntile - rem, rem * se, se, r, ntile - rem};
    if (se != s || !gemv_grid_fits(part, ctx->partials_floats, ctx->ncounters)) continue;
    const double c = grid_cost(ctx->ncu, nst, part, kSplitEarly);
    if (c < best_cost) {
      best = part;
      best_cost = c;
    }
  }
  return best;
}
}  // namespace

// Launch shape from the weight's shape only (never from B), so every output
// bit is independent of the block size.  One row group (16 rows) per wave;
// an interleaved pair computed whole puts its two sides on a wave pair.
void gemv_choose_split(const cwen_ctx *ctx, cwen_weight *w) {
  w->rows = 1;
  const int single = (w->nrg + tile_rows(1) - 1) / tile_rows(1);
  for (int ns = 1; ns <= w->nside; ++ns) {
    const int rpw = tile_rows(ns);
    w->cfg[ns - 1] = choose_grid(ctx, (w->nrg + rpw - 1) / rpw, w->nst, single);
  }
}

int gemv_row_tiles(const cwen_weight *w) { return (w->nrg + WAVES - 1) / WAVES; }

int gemv_launch(cwen_ctx *ctx, const cwen_weight *w, int nsides, int side0, int epi,
                const _Float16 *xh, const GemvOut &out, int B, hipStream_t st, const GemvF32 *xf,
                const GemvPost *post, const GemvScratch *scr) {
  if (post && (xf || !xh || !post->ssq || post->npart < 1 || post->npart > CWEN_MAX_PARTS)) return CWEN_EINVAL;
  if (xf && (xh || !xf->x || ((uintptr_t)xf->x & 15) || (xf->xs & 3) || (B > 1 && xf->xs < w->ne0)))
    return CWEN_EINVAL;
  if (out.ssq && (epi != GEMV_EPI_STORE || gemv_row_tiles(w) > CWEN_MAX_PARTS)) return CWEN_EINVAL;
  GemvParams p;
  p.w = w->dev;
  p.wbytes = (uint32_t)w->bytes;
  p.nsw = w->nside;
  p.side0 = side0;
  p.M = w->ne1;
  p.nrg = w->nrg;
  p.nst = w->nst;
  GemvGrid cfg = w->cfg[nsides - 1];
  p.xh = xh;
  const int xfs = xf ? (B > 1 ? xf->xs : w->ne0) : 0;
  p.xbytes = xf ? (uint32_t)(((size_t)(B - 1) * xfs + w->ne0) * 4) : (uint32_t)((size_t)B * w->ne0 * 2);
  p.xf = xf ? xf->x : nullptr;
  p.xfs = xfs;
  p.pss = post ? post->ssq : nullptr;
  p.pnpart = post ? post->npart : 0;
  p.eps = post ? post->eps : 0.f;
  p.K = w->ne0;
  p.B = B;
  p.part = scr ? scr->partials : ctx->partials;
  p.cnt = scr ? scr->counters : ctx->counters;
  p.out = out;
  const int rpw = tile_rows(nsides);
  const int ntile = (w->nrg + rpw - 1) / rpw;
  if (epi == GEMV_EPI_ARGMAX) cfg = {ntile, 0, 1, w->nst, 0};  // final row values in one workgroup
  if (scr && !gemv_grid_fits(cfg, scr->partials_floats, scr->ncounters)) return CWEN_ESCRATCH;
  p.nsplit = cfg.nsplit;
  p.S = cfg.S;
  p.rps = cfg.rps;
  p.tile0 = cfg.tile0;
  const int nrt = cfg.grid;
  int rc = CWEN_EINVAL;
  if (w->fmt == GEMV_Q4) {
    if (nsides == 2 && epi == GEMV_EPI_PAIR) {
      launch_cb<GEMV_Q4, 2, GEMV_EPI_PAIR>(p, nrt, st);
      rc = CWEN_OK;
    } else if (nsides == 2 && epi == GEMV_EPI_SWIGLU) {
      launch_cb<GEMV_Q4, 2, GEMV_EPI_SWIGLU>(p, nrt, st);
      rc = CWEN_OK;
    } else if (nsides == 1 && epi == GEMV_EPI_CONV) {
      if (!out.cv_w || !out.cv_H || !out.cv_xc || !out.cv_ctl || out.cv_C < 0 || out.cv_C > w->ne1 || out.cv_C % Q4_ROWS ||
          out.cv_nslot < 1)
        return CWEN_EINVAL;
      launch_cb<GEMV_Q4, 1, GEMV_EPI_CONV>(p, nrt, st);
      rc = CWEN_OK;
    } else {
      rc = launch_fmt<GEMV_Q4>(p, nrt, nsides, epi, st);
    }
  } else if (w->fmt == GEMV_Q6K) {
    rc = launch_fmt<GEMV_Q6K>(p, nrt, nsides, epi, st);
  } else if (w->fmt == GEMV_Q8) {
    rc = launch_fmt<GEMV_Q8>(p, nrt, nsides, epi, st);
  } else if (w->fmt == GEMV_Q41) {
    rc = launch_fmt<GEMV_Q41>(p, nrt, nsides, epi, st);
  } else if (w->fmt == GEMV_Q5K) {
    rc = launch_fmt<GEMV_Q5K>(p, nrt, nsides, epi, st);
  }
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

int argmax_walk_launch(const float *lg, long ls, int V, int B, const ArgmaxOut &a, hipStream_t st) {
  const dim3 grid((unsigned)((V + AM_CHUNK - 1) / AM_CHUNK), (unsigned)B);
  hipLaunchKernelGGL(argmax_walk_kernel, grid, dim3(256), 0, st, lg, ls, V, B, a);
  CWEN_HIP_TRY(hipGetLastError());
  return CWEN_OK;
}
