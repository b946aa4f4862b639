// Per-position glue kernels of the block-verify forward pass: token
// embedding, RMSNorm, and the gated full-attention layer (q/k norm, partial
// RoPE, KV-cache write, causal attention with a sigmoid output gate).
//
// Reference semantics (run.c): embed_token_to 1849-1887, rmsnorm 346-368,
// rope_tables / rope_apply 1903-1948, layer_full_blk 2714-2745,
// attention_heads_kv 2362-2409.
//
// Every kernel computes each position (block column) with the same
// instructions whatever B is, so a block of B positions produces exactly the
// values of B single-position passes.
#include "cwen_internal.h"

namespace {

constexpr int HD = 128 * 2;          // full-attention head dim
constexpr int TC = 32;               // keys per attention chunk

__device__ __forceinline__ float max64(float v) {
  auto mx = [](float a, float b) { return a > b ? a : b; };
  v = mx(v, dpp<0xB1>(v));
  v = mx(v, dpp<0x4E>(v));
  v = mx(v, dpp<0x141>(v));
  v = mx(v, dpp<0x140>(v));
  const int b = __builtin_bit_cast(int, v);
  const float a0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
  const float a1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
  const float a2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
  const float a3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
  return mx(mx(a0, a1), mx(a2, a3));
}
// Block-wide sum for 256 threads (4 waves); `red` holds 4 floats.
__device__ __forceinline__ float sum256(float v, float *red) {
  const float w = sum64(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = w;
  __syncthreads();
  const float t = red[0] + red[1] + red[2] + red[3];
  __syncthreads();
  return t;
}
__device__ __forceinline__ float f16f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// ---- embedding: Q4_0 (GGUF blocks), Q4_0RS (split scales) or Q6_K rows,
// exact f32 dequant: w = (n - 8) * d, or for Q6_K (d * sc) * (q6 - 32) in
// the reference's order (run.c:1829-1848).  Grid: B, 256 threads, thread =
// 32-weight block.
__device__ __forceinline__ void embed_block_q6k(const uint8_t *row, int i, float *w) {
  // block i = weights 32 i .. 32 i + 31 = quarter q of half h of super-block sb
  const int sb = i >> 3, h = (i >> 2) & 1, q = i & 3;
  const uint8_t *b = row + (size_t)sb * 210;
  const uint8_t *ql = b + h * 64 + (q & 1) * 32, *qh = b + 128 + h * 32;
  const int8_t *sc = (const int8_t *)(b + 192) + h * 8 + 2 * q;
  const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(b[208] | (b[209] << 8)));
  const int shift = q >= 2 ? 4 : 0;
#pragma unroll 4
  for (int l = 0; l < 32; ++l) {
    const int v = ((ql[l] >> shift) & 0xF) | (((qh[l] >> (2 * q)) & 3) << 4);
    w[l] = __fmul_rn(__fmul_rn(d, (float)sc[l >> 4]), (float)(v - 32));
  }
}

__global__ __launch_bounds__(256) void embed_kernel(const uint8_t *qs, const uint16_t *sc, int type,
                                                    const int *toks, int H, float *X, int xs, float *ssq,
                                                    _Float16 *xh, const float *nw, int *rflag) {
  __shared__ float red[4];
  const int b = blockIdx.x;
  const size_t tok = (size_t)toks[b];
  const int nb = H / 32;
  float sq = 0.f;
  for (int i = threadIdx.x; i < nb; i += 256) {
    float w[32];
    if (type == CWEN_T_Q6_K) {
      embed_block_q6k(qs + tok * (size_t)(H / 256) * 210, i, w);
    } else {
      const uint8_t *q;
      float d;
      if (type == CWEN_T_Q4_0) {
        const uint8_t *blk = qs + (tok * nb + i) * 18;
        d = f16f((uint16_t)(blk[0] | (blk[1] << 8)));
        q = blk + 2;
      } else {
        q = qs + (tok * nb + i) * 16;
        d = f16f(sc[tok * nb + i]);
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        w[j] = (float)((int)(q[j] & 0xF) - 8) * d;
        w[j + 16] = (float)((int)(q[j] >> 4) - 8) * d;
      }
    }
    float *dst = X + (size_t)b * xs + i * 32;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float lo = w[j], hi = w[j + 16];
      dst[j] = lo;
      dst[j + 16] = hi;
      if (xh) {
        const _Float16 h0 = (_Float16)(lo * nw[i * 32 + j]), h1 = (_Float16)(hi * nw[i * 32 + j + 16]);
        xh[(size_t)b * H + i * 32 + j] = h0;
        xh[(size_t)b * H + i * 32 + j + 16] = h1;
        if (f16_bad(h0) || f16_bad(h1)) raise_flag(rflag);
      }
      sq = fmaf(lo, lo, sq);
      sq = fmaf(hi, hi, sq);
    }
  }
  // The row's sum of squares: the one partial a normalising GEMV reads.
  const float t = sum256(sq, red);
  if (threadIdx.x == 0) ssq[(size_t)b * CWEN_MAX_PARTS] = t;   // ssq[column][partial]: one partial
}

// ---- full attention, part 1: per (position, head) q/k RMSNorm (one shared
// [HD] weight each), partial RoPE on pairs (2i, 2i+1), i < npairs, and the
// KV-cache write.  Grid: (B, NH + NKV), 256 threads = head dims.
struct AttnParams {
  const float *qfull; int qfs;  // [B][qfs]: per head q (HD) then gate (HD)
  const float *kx, *vx; int kvs;  // [B][kvs]: NKV*HD each
  const float *qn, *kn;
  float *q;            // [B][NH][HD] normed + roped queries
  float *K, *V;        // this layer's cache [ctx][NKV][HD]
  const int *last;     // device: last filled cache slot before the block
  int max_ctx;         // cache slots; positions at or past it are not touched
  int B, NH, NKV, npairs, nrot;
  float theta, eps;
  // attention
  float *po;           // partial outputs [NKV][nchunk][B*kvm][HD]
  float *pm, *pl;      // partial max / sum [NKV][nchunk][B*kvm]
  int nchunk;
  int nbuf;            // chunk buffers in LDS: 2 lands the next chunk during the current one
  _Float16 *yh;        // gated outputs f16 [B][NH*HD]
  int *rflag;          // set to 1 when a gated output is out of f16's range, nullable
};

__global__ __launch_bounds__(256) void attn_prep_kernel(AttnParams p) {
  __shared__ float red[4];
  __shared__ float v[HD];
  const int b = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
  const int pos = *p.last + 1 + b;
  if (pos < 0 || pos >= p.max_ctx) return;   // workgroup-uniform
  const bool isq = h < p.NH;
  const int hk = h - p.NH;
  const float x = isq ? p.qfull[(size_t)b * p.qfs + (size_t)h * 2 * HD + d]
                      : p.kx[(size_t)b * p.kvs + hk * HD + d];
  const float s = 1.f / sqrtf(sum256(x * x, red) / (float)HD + p.eps);
  float y = (isq ? p.qn[d] : p.kn[d]) * x * s;
  v[d] = y;
  __syncthreads();
  if (d < 2 * p.npairs) {
    const int idx = d >> 1;
    const float freq = 1.f / powf(p.theta, (float)idx / (float)p.nrot);
    const float ang = (float)pos * freq;
    const float c = cosf(ang), sn = sinf(ang);
    const float a = v[idx * 2], bb = v[idx * 2 + 1];
    y = (d & 1) ? a * sn + bb * c : a * c - bb * sn;
  }
  if (isq) {
    p.q[((size_t)b * p.NH + h) * HD + d] = y;
  } else {
    p.K[((size_t)pos * p.NKV + hk) * HD + d] = y;
    p.V[((size_t)pos * p.NKV + hk) * HD + d] = p.vx[(size_t)b * p.kvs + hk * HD + d];
  }
}

// ---- full attention, part 2: per (key chunk, kv head), the kvm x B queries
// of the group (each masked to keys t <= its position) against the chunk's
// TC keys on f32 matrix cores (v_mfma_f32_16x16x4f32):
//   S[q][t] = (Q[q] . K[t]) / sqrt(HD);  P[q][t] = exp(S - m_q), m_q = max_t S,
//   l_q = sum_t P;  O[q] = sum_t P[q][t] V[t]   -> partials po, pm, pl.
// In a product's k-th step lane group g (lanes 16g..16g+15) supplies
// element g*run + k of the reduction dimension, so a lane reads 4 steps with
// one 16-byte LDS read; the summation order is fixed and the same for every
// query row, whatever B is.  Scores: wave w takes 16-query tile w (both
// 16-key halves, so the chunk softmax stays in the wave); workgroups have 8
// waves (NW = 8), so a wave never holds more than one tile, and with fewer
// tiles the idle waves still share the K/V landing and the P.V products
// (8-wave workgroups measured 0.7 % faster per verify cycle than 4-wave ones
// at 1-3 tiles).  K and V rows land in LDS straight from the cache by
// 16-byte buffer loads (one 1 KB row per instruction; rows past the block's
// last position load as zeros), in their natural [key][dim] layout.  P.V:
// wave w takes head-dim tiles (16/NW)w .. of every query tile, reading V's 8
// k-steps of a tile once for all query tiles.  Every output takes the same
// instruction sequence for NW = 4 and 8.  A fixed grid of workgroups per kv head takes
// chunks blockIdx.x, + gridDim.x, ... up to the block's last position (the
// partials are per chunk, so the mapping does not change the arithmetic).
typedef float f32x4_t __attribute__((ext_vector_type(4)));
constexpr int KROW = HD + 4, PROW = TC + 4;   // K and V rows: 1040 bytes, 16-byte aligned
constexpr int NW_MAX = 8;    // waves of the largest workgroup: 16-query tiles per block (nq <= 128)
constexpr int KV_FLOATS = 2 * TC * KROW;     // K [TC][KROW] then V [TC][KROW]
typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __forceinline__ float max16(float m) {
  m = fmaxf(m, dpp<0xB1>(m)); m = fmaxf(m, dpp<0x4E>(m));
  m = fmaxf(m, dpp<0x141>(m)); return fmaxf(m, dpp<0x140>(m));
}

// NW: waves per workgroup (4, or 8 when the block has more than 4 query tiles).
template <int NW>
__global__ __launch_bounds__(64 * NW) void attn_chunk_kernel(AttnParams p) {
  extern __shared__ __align__(16) float sm[];
  const int hkv = blockIdx.y;
  const int kvm = p.NH / p.NKV;
  const int nq = p.B * kvm;
  const int MT = (nq + 15) / 16;               // 16-query tiles
  // nbuf chunk buffers, K [TC][KROW] then V [TC][KROW] each; with two, the
  // next chunk's rows land in one while the current chunk is computed from
  // the other.
  const bool two = p.nbuf == 2;
  float *Ps = sm + (two ? 2 : 1) * KV_FLOATS;  // [MT*16][PROW]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const float scale = 1.f / sqrtf((float)HD);
  // The score phase's queries stay in registers: wave w holds 16-query tile
  // w, lane (lr, lg) the HD/4 dims lg*HD/4 .. of query row lr.  Keeping them
  // out of LDS leaves room for several workgroups per CU.  They are requested
  // first, before the block's position is known: query row qi belongs to
  // position qi / kvm, so rows >= nq lie past the buffer range and load as
  // zeros.
  float4 qreg[HD / 16];
  {
    const __amdgpu_buffer_rsrc_t qr = make_rsrc(p.q, (uint32_t)((size_t)p.B * p.NH * HD * 4));
    const int qi = wave * 16 + lr;
    const uint32_t qo = (uint32_t)((((qi / kvm) * p.NH + hkv * kvm + qi % kvm) * HD + lg * (HD / 4)) * 4);
#pragma unroll
    for (int k = 0; k < HD / 16; ++k) qreg[k] = __builtin_bit_cast(float4, bload16(qr, qo + 16 * k));
  }
  constexpr int KV_R = TC / NW;                     // K (and V) rows each wave lands per chunk
  constexpr int DT = 16 / NW;                       // head-dim tiles of P.V per wave
  const __amdgpu_buffer_rsrc_t kr = make_rsrc(p.K, (uint32_t)((size_t)p.max_ctx * p.NKV * HD * 4));
  const __amdgpu_buffer_rsrc_t vr = make_rsrc(p.V, (uint32_t)((size_t)p.max_ctx * p.NKV * HD * 4));
  // The position is read after the queries are requested (a scalar load
  // issued first would hold their address computation behind it).
  __builtin_amdgcn_sched_barrier(0);
  const int pbase = *p.last + 1;
  const int tlast = min(pbase + p.B - 1, p.max_ctx - 1);  // last position of the block
  if ((int)blockIdx.x * TC > tlast) return;
  // Lands chunk c's K and V rows in LDS buffer `bf` (rows past the block's
  // last position as zeros): 2 * KV_R loads per wave.  The first chunk's
  // rows are requested with the queries in flight, so both arrive in one
  // memory round trip.
  auto land = [&](int c, int bf) __attribute__((always_inline)) {
    const int t0 = c * TC;
    const int tn = min(TC, tlast + 1 - t0);     // keys of this chunk that exist
    float *Kd = sm + bf * KV_FLOATS, *Vd = Kd + TC * KROW;
#pragma unroll
    for (int u = 0; u < KV_R; ++u) {            // row t = wave + NW u: 64 lanes x 16 bytes
      const int t = wave + NW * u;
      const uint32_t row = (uint32_t)(((size_t)(t0 + t) * p.NKV + hkv) * HD * 4);
      const uint32_t vo = t < tn ? (uint32_t)lane * 16 : 0xFFFFFFE0u;   // past the last key: zeros
      __builtin_amdgcn_raw_ptr_buffer_load_lds(kr, (lds_void_t *)(Kd + t * KROW), 16, vo, row, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(vr, (lds_void_t *)(Vd + t * KROW), 16, vo, row, 0, 0);
    }
  };
  int c = blockIdx.x, bf = 0;
  land(c, bf);
  for (;;) {
    const int t0 = c * TC;
    const int tn = min(TC, tlast + 1 - t0);     // keys of this chunk that exist
    const int cn = c + (int)gridDim.x;
    const bool more = cn * TC <= tlast;
    // The next chunk's rows go to the other buffer (its readers finished at
    // the previous barrier); the wait then leaves just those in flight.
    if (more && two) {
      land(cn, bf ^ 1);
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * KV_R) : "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    lds_barrier();                                       // every wave's rows of chunk c
    const float *Ks = sm + bf * KV_FLOATS, *Vs = Ks + TC * KROW;
    // scores and the chunk softmax, one 16-query tile per wave
    if (wave < MT) {
      const int mt = wave;
      // Four independent accumulators per 16 keys: s over the first half of
      // the lane group's K run, u over the second, summed at the end.  The
      // K rows of step k + 4 are read from LDS while step k's products issue
      // (the scheduling barriers keep the reads ahead of the products).
      f32x4_t s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
      f32x4_t u0 = {0.f, 0.f, 0.f, 0.f}, u1 = {0.f, 0.f, 0.f, 0.f};
      const float *k0 = Ks + lr * KROW + lg * (HD / 4), *k1 = k0 + 16 * KROW;
      float4 kb[2][4];
      auto kread = [&](int k, float4 (&d)[4]) __attribute__((always_inline)) {
        d[0] = *(const float4 *)(k0 + k);
        d[1] = *(const float4 *)(k1 + k);
        d[2] = *(const float4 *)(k0 + k + HD / 8);
        d[3] = *(const float4 *)(k1 + k + HD / 8);
      };
      kread(0, kb[0]);
#pragma unroll
      for (int k = 0; k < HD / 8; k += 4) {
        if (k + 4 < HD / 8) kread(k + 4, kb[((k >> 2) + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
        const float4 a = qreg[k / 4], cq = qreg[(k + HD / 8) / 4];
        const float4 b0 = kb[(k >> 2) & 1][0], b1 = kb[(k >> 2) & 1][1];
        const float4 e0 = kb[(k >> 2) & 1][2], e1 = kb[(k >> 2) & 1][3];
        s0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b0.x, s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b1.x, s1, 0, 0, 0);
        u0 = __builtin_amdgcn_mfma_f32_16x16x4f32(cq.x, e0.x, u0, 0, 0, 0);
        u1 = __builtin_amdgcn_mfma_f32_16x16x4f32(cq.x, e1.x, u1, 0, 0, 0);
        s0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b0.y, s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b1.y, s1, 0, 0, 0);
        u0 = __builtin_amdgcn_mfma_f32_16x16x4f32(cq.y, e0.y, u0, 0, 0, 0);
        u1 = __builtin_amdgcn_mfma_f32_16x16x4f32(cq.y, e1.y, u1, 0, 0, 0);
        s0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b0.z, s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b1.z, s1, 0, 0, 0);
        u0 = __builtin_amdgcn_mfma_f32_16x16x4f32(cq.z, e0.z, u0, 0, 0, 0);
        u1 = __builtin_amdgcn_mfma_f32_16x16x4f32(cq.z, e1.z, u1, 0, 0, 0);
        s0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b0.w, s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b1.w, s1, 0, 0, 0);
        u0 = __builtin_amdgcn_mfma_f32_16x16x4f32(cq.w, e0.w, u0, 0, 0, 0);
        u1 = __builtin_amdgcn_mfma_f32_16x16x4f32(cq.w, e1.w, u1, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
      s0 += u0;
      s1 += u1;
      // s0[r], s1[r]: query row mt*16 + 4*lg + r, keys lr and 16 + lr
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int qi = mt * 16 + 4 * lg + r;
        const int tq = pbase + qi / kvm;       // the query's position
        const bool v0 = qi < nq && lr < tn && t0 + lr <= tq;
        const bool v1 = qi < nq && 16 + lr < tn && t0 + 16 + lr <= tq;
        const float a0 = v0 ? s0[r] * scale : -__builtin_inff(), a1 = v1 ? s1[r] * scale : -__builtin_inff();
        const float m = max16(fmaxf(a0, a1));
        const float e0 = v0 ? expf(a0 - m) : 0.f, e1 = v1 ? expf(a1 - m) : 0.f;
        const float l = sum16(e0 + e1);
        Ps[(mt * 16 + 4 * lg + r) * PROW + lr] = e0;
        Ps[(mt * 16 + 4 * lg + r) * PROW + 16 + lr] = e1;
        if (lr == 0 && qi < nq) {
          const size_t pi = ((size_t)hkv * p.nchunk + c) * nq + qi;
          p.pm[pi] = m;
          p.pl[pi] = l;
        }
      }
    }
    lds_barrier();                              // P written (the max / sum stores need not land)
    // P.V: head-dim tiles DT*wave .. DT*wave + DT-1 of every query tile.  In
    // step k of a product, lane group g supplies key g*8 + k: P[q][g*8 + k]
    // (two 16-byte reads per query tile) and V[g*8 + k][d] (read once, shared
    // by the query tiles).  The DT products of a query tile run interleaved,
    // each still summing its steps k = 0 .. 7 in order.
    float vk[DT][8];
#pragma unroll
    for (int q = 0; q < DT; ++q) {
      const float *vb = Vs + (lg * (TC / 4)) * KROW + (wave * DT + q) * 16 + lr;
#pragma unroll
      for (int k = 0; k < 8; ++k) vk[q][k] = vb[k * KROW];
    }
    for (int mt = 0; mt < MT; ++mt) {
      const float *pa = Ps + (mt * 16 + lr) * PROW + lg * (TC / 4);
      const float4 pa0 = *(const float4 *)pa, pa1 = *(const float4 *)(pa + 4);
      const float pk[8] = {pa0.x, pa0.y, pa0.z, pa0.w, pa1.x, pa1.y, pa1.z, pa1.w};
      f32x4_t o[DT];
#pragma unroll
      for (int q = 0; q < DT; ++q) o[q] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < 8; ++k)
#pragma unroll
        for (int q = 0; q < DT; ++q) o[q] = __builtin_amdgcn_mfma_f32_16x16x4f32(pk[k], vk[q][k], o[q], 0, 0, 0);
#pragma unroll
      for (int q = 0; q < DT; ++q) {
        const int nd = wave * DT + q;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int qi = mt * 16 + 4 * lg + r;
          if (qi < nq) p.po[(((size_t)hkv * p.nchunk + c) * nq + qi) * HD + nd * 16 + lr] = o[q][r];
        }
      }
    }
    if (!more) break;
    lds_barrier();                              // this chunk's reads of K, V and P done
    c = cn;
    if (two) bf ^= 1;
    else land(c, 0);
  }
}

// ---- full attention, part 3: merge the chunks of each (position, head),
// normalise, apply the sigmoid gate, write f16.  Grid: (B, NH); MGR groups
// of HD threads (thread = head dim d) each take a contiguous quarter of the
// chunks in order, and the groups' sums are added in group order: a fixed
// order per position, whatever B is.
constexpr int MGR = 4;
__global__ __launch_bounds__(HD * MGR) void attn_merge_kernel(AttnParams p) {
  const int b = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const int d = tid % HD, grp = tid / HD;
  const int kvm = p.NH / p.NKV;
  const int hkv = h / kvm, m = h % kvm;
  const int nq = p.B * kvm;
  const int qi = b * kvm + m;
  const int pos = *p.last + 1 + b;
  if (pos < 0 || pos >= p.max_ctx) return;
  const int nc = pos / TC + 1;
  __shared__ float red[HD * MGR / 64], s_w[HD * MGR], s_l[HD * MGR], s_lo[2][MGR][HD];
  const size_t base = (size_t)hkv * p.nchunk * nq + qi;  // statistics of chunk c at base + c * nq
  float mx = -__builtin_inff();
  for (int c = tid; c < nc; c += HD * MGR) mx = fmaxf(mx, p.pm[base + (size_t)c * nq]);
  mx = max64(mx);
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  float M = red[0];
#pragma unroll
  for (int w = 1; w < HD * MGR / 64; ++w) M = fmaxf(M, red[w]);
  // Chunks HD*MGR at a time: thread j weighs chunk c0 + j into LDS; group g
  // then accumulates its quarter of them in order, its partial outputs
  // loaded MG at a time.
  float L = 0.f, O = 0.f;
  for (int c0 = 0; c0 < nc; c0 += HD * MGR) {
    __syncthreads();  // previous tile's weights read
    if (c0 + tid < nc) {
      const size_t pi = base + (size_t)(c0 + tid) * nq;
      s_w[tid] = expf(p.pm[pi] - M);
      s_l[tid] = p.pl[pi];
    }
    __syncthreads();
    const int n = min(HD * MGR, nc - c0);
    const int per = (n + MGR - 1) / MGR;
    const int j1 = min(n, (grp + 1) * per);
    constexpr int MG = 8;
    for (int j0 = grp * per; j0 < j1; j0 += MG) {
      float pv[MG];
#pragma unroll
      for (int u = 0; u < MG; ++u)
        pv[u] = j0 + u < j1 ? p.po[(base + (size_t)(c0 + j0 + u) * nq) * HD + d] : 0.f;
#pragma unroll
      for (int u = 0; u < MG; ++u) {
        if (j0 + u >= j1) break;
        L = fmaf(s_w[j0 + u], s_l[j0 + u], L);
        O = fmaf(s_w[j0 + u], pv[u], O);
      }
    }
  }
  s_lo[0][grp][d] = L;
  s_lo[1][grp][d] = O;
  __syncthreads();
  if (grp != 0) return;
  L = s_lo[0][0][d];
  O = s_lo[1][0][d];
#pragma unroll
  for (int g2 = 1; g2 < MGR; ++g2) {
    L += s_lo[0][g2][d];
    O += s_lo[1][g2][d];
  }
  const float g = p.qfull[(size_t)b * p.qfs + (size_t)h * 2 * HD + HD + d];
  const float y = (O / L) * (1.f / (1.f + expf(-g)));
  const _Float16 yh = (_Float16)y;
  p.yh[(size_t)b * p.NH * HD + (size_t)h * HD + d] = yh;
  if (f16_bad(yh)) raise_flag(p.rflag);
}

}  // namespace

int embed_launch(const uint8_t *qs, const uint16_t *sc, int type, const int *toks, int B, int H, float *X,
                 int xs, float *ssq, hipStream_t st, _Float16 *xh, const float *nw, int *rflag) {
  if ((xh == nullptr) != (nw == nullptr)) return CWEN_EINVAL;
  hipLaunchKernelGGL(embed_kernel, dim3((unsigned)B), dim3(256), 0, st, qs, sc, type, toks, H, X, xs, ssq, xh, nw, rflag);
  CWEN_HIP_TRY(hipGetLastError());
  return CWEN_OK;
}

size_t attn_partial_floats(int NH, int NKV, int max_ctx, int B) {
  const int nchunk = (max_ctx + TC - 1) / TC;
  return (size_t)NKV * nchunk * B * (NH / NKV) * (HD + 2);
}

// Dynamic LDS above 64 KB (B = 16 blocks) needs the attribute; set once per
// process before any launch (not inside a graph capture).
int attention_max_group() { return NW_MAX * 16 / CWEN_BMAX; }

int attention_init() {
  static bool done = false;
  if (!done) {
    CWEN_HIP_TRY(hipFuncSetAttribute((const void *)attn_chunk_kernel<NW_MAX>,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
    done = true;
  }
  return CWEN_OK;
}

// Chunk workgroups per kv head and chunk buffers, by the block's context.
// Up to ATTN_NARROW_CHUNKS chunks: 64 workgroups per head (one per CU at the
// 27B shape's 4 kv heads), each landing its next chunk while it computes the
// current one; two workgroups' chunks on one CU do not overlap, so more
// workgroups only add idle ones at short contexts.  Past that, 128 per head
// with one buffer each (two resident per CU), whose per-chunk cost grows
// more slowly.  Measured at 24/4 heads, B = 8, contexts 1024 / 4096 / 8000:
// 64 x 2 buffers 9.5 / 25.9 / 37.2 us, 128 x 1 buffer 14.0 / 28.0 / 34.0 us,
// 128 x 2 buffers (one workgroup per CU) 12.7 / 29.4 / 43.7 us.
constexpr int ATTN_NARROW_CHUNKS = 192, ATTN_NARROW_WGS = 64, ATTN_WIDE_WGS = 128;

bool attention_wide(int last_pos) { return last_pos >= 0 && last_pos / TC + 1 > ATTN_NARROW_CHUNKS; }

int attention_launch(const float *qfull, int qfs, const float *kx, const float *vx, int kvs, const float *qn,
                     const float *kn, float *qbuf, float *K, float *V, const int *last, int B, int NH, int NKV,
                     int npairs, int nrot, float theta, float eps, float *part, int max_ctx, _Float16 *yh,
                     hipStream_t st, int *rflag, int last_hint) {
  AttnParams p;
  p.qfull = qfull; p.qfs = qfs; p.kx = kx; p.vx = vx; p.kvs = kvs;
  p.qn = qn; p.kn = kn;
  p.q = qbuf; p.K = K; p.V = V;
  p.last = last; p.max_ctx = max_ctx; p.B = B; p.NH = NH; p.NKV = NKV; p.npairs = npairs; p.nrot = nrot;
  p.theta = theta; p.eps = eps;
  p.nchunk = (max_ctx + TC - 1) / TC;
  const int nq = B * (NH / NKV);
  p.po = part;
  p.pm = part + (size_t)NKV * p.nchunk * nq * HD;
  p.pl = p.pm + (size_t)NKV * p.nchunk * nq;
  p.yh = yh;
  p.rflag = rflag;
  // Every check before the first launch: a block never stops half-way.
  const bool wide = attention_wide(last_hint);
  const int wgs = wide ? ATTN_WIDE_WGS : ATTN_NARROW_WGS;
  const int nwg = p.nchunk < wgs ? p.nchunk : wgs;
  p.nbuf = wide ? 1 : 2;
  const int MT = (nq + 15) / 16;
  if (NH % NKV || MT > NW_MAX) return CWEN_EINVAL;   // one 16-query tile per wave
  const size_t lds = ((size_t)MT * 16 * PROW + p.nbuf * KV_FLOATS) * sizeof(float);
  if (lds > 160 * 1024) return CWEN_EINVAL;
  int rc;
  if ((rc = attention_init())) return rc;
  hipLaunchKernelGGL(attn_prep_kernel, dim3((unsigned)B, (unsigned)(NH + NKV)), dim3(HD), 0, st, p);
  hipLaunchKernelGGL(attn_chunk_kernel<NW_MAX>, dim3((unsigned)nwg, (unsigned)NKV), dim3(64 * NW_MAX), lds, st, p);
  hipLaunchKernelGGL(attn_merge_kernel, dim3((unsigned)B, (unsigned)NH), dim3(HD * MGR), 0, st, p);
  CWEN_HIP_TRY(hipGetLastError());
  return CWEN_OK;
}
