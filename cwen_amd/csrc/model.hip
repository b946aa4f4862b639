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

// ---- embedding: Q4_0 (GGUF blocks) or Q4_0RS (split scales) rows, exact
// f32 dequant w = (n - 8) * d.  Grid: B, 256 threads, thread = block.
__global__ __launch_bounds__(256) void embed_kernel(const uint8_t *qs, const uint16_t *sc, int type,
                                                    const int *toks, int H, float *X, int xs, float *ssq) {
  __shared__ float red[4];
  const int b = blockIdx.x;
  const size_t tok = (size_t)toks[b];
  const int nb = H / 32;
  float sq = 0.f;
  for (int i = threadIdx.x; i < nb; i += 256) {
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
    float *dst = X + (size_t)b * xs + i * 32;
    for (int j = 0; j < 16; ++j) {
      const float lo = (float)((int)(q[j] & 0xF) - 8) * d, hi = (float)((int)(q[j] >> 4) - 8) * d;
      dst[j] = lo;
      dst[j + 16] = hi;
      sq = fmaf(lo, lo, sq);
      sq = fmaf(hi, hi, sq);
    }
  }
  // The row's sum of squares: the one partial a normalising GEMV reads.
  const float t = sum256(sq, red);
  if (threadIdx.x == 0) ssq[b] = t;
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
  _Float16 *yh;        // gated outputs f16 [B][NH*HD]
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

// ---- full attention, part 2: per (key chunk, kv head) score the chunk
// against every query of the group (kvm heads x B positions, each masked to
// t <= its position), then accumulate exp(s - m_chunk) * V.  A fixed grid of
// workgroups per kv head takes chunks blockIdx.x, + gridDim.x, ... up to the
// block's last position (the partials are per chunk, so the mapping does not
// change the arithmetic).  The
// chunk's K rows, then its V rows, are staged in LDS with a padded row
// stride (KROW floats: the float4 reads of 16 consecutive rows hit distinct
// banks).  Scores: lane = key, queries strided over 8 groups.  P.V: thread =
// head dim, 8 queries at a time.
constexpr int KROW = HD + 4;
__global__ __launch_bounds__(256) void attn_chunk_kernel(AttnParams p) {
  extern __shared__ __align__(16) float sm[];  // Kt [TC][KROW] | Q [nq][HD] | S [nq][TC]
  const int hkv = blockIdx.y;
  const int kvm = p.NH / p.NKV;
  const int nq = p.B * kvm;
  const int pbase = *p.last + 1;
  const int tlast = min(pbase + p.B - 1, p.max_ctx - 1);  // last position of the block
  if ((int)blockIdx.x * TC > tlast) return;
  float *Kt = sm;
  float *Q = sm + TC * KROW;
  float *S = Q + nq * HD;
  const int tid = threadIdx.x;
  const float scale = 1.f / sqrtf((float)HD);
  for (int e = tid; e < nq * (HD / 4); e += 256) {  // queries: (b, m) -> head hkv*kvm + m
    const int qi = e / (HD / 4), d4 = e % (HD / 4);
    const int b = qi / kvm, m = qi % kvm;
    *(float4 *)(Q + qi * HD + d4 * 4) = *(const float4 *)(p.q + ((size_t)b * p.NH + hkv * kvm + m) * HD + d4 * 4);
  }
  for (int c = blockIdx.x; c * TC <= tlast; c += gridDim.x) {
    const int t0 = c * TC;
    const int tn = min(TC, tlast + 1 - t0);     // keys of this chunk that exist
    __syncthreads();                            // previous chunk's P.V reads done
    for (int e = tid; e < TC * (HD / 4); e += 256) {
      const int t = e / (HD / 4), d4 = e % (HD / 4);
      *(float4 *)(Kt + t * KROW + d4 * 4) =
          t < tn ? *(const float4 *)(p.K + ((size_t)(t0 + t) * p.NKV + hkv) * HD + d4 * 4) : (float4){0.f, 0.f, 0.f, 0.f};
    }
    __syncthreads();
    {  // scores and chunk softmax statistics
      const int key = tid & (TC - 1), qg = tid / TC;   // TC = 32: 8 query groups
      const int t = t0 + key;
      const float *kr = Kt + key * KROW;
      for (int qi = qg; qi < nq; qi += 256 / TC) {
        const int b = qi / kvm;
        const float *q = Q + qi * HD;
        float sc = -__builtin_inff();
        if (t <= pbase + b && key < tn) {
          float a = 0.f;
          for (int d = 0; d < HD; d += 4) {
            const float4 k4 = *(const float4 *)(kr + d), q4 = *(const float4 *)(q + d);
            a = fmaf(q4.x, k4.x, a); a = fmaf(q4.y, k4.y, a); a = fmaf(q4.z, k4.z, a); a = fmaf(q4.w, k4.w, a);
          }
          sc = a * scale;
        }
        // max / sum over the 32 keys (lanes 0-31 or 32-63 of the wave)
        float m = sc;
        m = fmaxf(m, dpp<0xB1>(m)); m = fmaxf(m, dpp<0x4E>(m)); m = fmaxf(m, dpp<0x141>(m)); m = fmaxf(m, dpp<0x140>(m));
        m = fmaxf(m, __shfl_xor(m, 16));
        const float e = (sc == -__builtin_inff()) ? 0.f : expf(sc - m);
        float l = sum16(e);
        l += __shfl_xor(l, 16);
        S[qi * TC + key] = e;
        if (key == 0) {
          const size_t pi = ((size_t)hkv * p.nchunk + c) * nq + qi;
          p.pm[pi] = m;
          p.pl[pi] = l;
        }
      }
    }
    __syncthreads();
    for (int e = tid; e < TC * (HD / 4); e += 256) {  // V rows replace K
      const int t = e / (HD / 4), d4 = e % (HD / 4);
      *(float4 *)(Kt + t * KROW + d4 * 4) =
          t < tn ? *(const float4 *)(p.V + ((size_t)(t0 + t) * p.NKV + hkv) * HD + d4 * 4) : (float4){0.f, 0.f, 0.f, 0.f};
    }
    __syncthreads();
    {  // P.V: thread = head dim
      const int d = tid;
      for (int q0 = 0; q0 < nq; q0 += 8) {
        const int nqq = min(8, nq - q0);
        float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (int t = 0; t < TC; t += 4) {
          const float v0 = Kt[(t + 0) * KROW + d], v1 = Kt[(t + 1) * KROW + d];
          const float v2 = Kt[(t + 2) * KROW + d], v3 = Kt[(t + 3) * KROW + d];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            if (j >= nqq) break;
            const float4 pr = *(const float4 *)(S + (q0 + j) * TC + t);
            o[j] = fmaf(pr.x, v0, o[j]); o[j] = fmaf(pr.y, v1, o[j]);
            o[j] = fmaf(pr.z, v2, o[j]); o[j] = fmaf(pr.w, v3, o[j]);
          }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (j >= nqq) break;
          p.po[(((size_t)hkv * p.nchunk + c) * nq + q0 + j) * HD + d] = o[j];
        }
      }
    }
  }
}

// ---- full attention, part 3: merge the chunks of each (position, head) in
// chunk order, normalise, apply the sigmoid gate, write f16.  Grid: (B, NH).
__global__ __launch_bounds__(256) void attn_merge_kernel(AttnParams p) {
  const int b = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
  const int kvm = p.NH / p.NKV;
  const int hkv = h / kvm, m = h % kvm;
  const int nq = p.B * kvm;
  const int qi = b * kvm + m;
  const int pos = *p.last + 1 + b;
  if (pos < 0 || pos >= p.max_ctx) return;
  const int nc = pos / TC + 1;
  float M = -__builtin_inff();
  for (int c = 0; c < nc; ++c) M = fmaxf(M, p.pm[((size_t)hkv * p.nchunk + c) * nq + qi]);
  float L = 0.f, O = 0.f;
  for (int c = 0; c < nc; ++c) {
    const size_t pi = ((size_t)hkv * p.nchunk + c) * nq + qi;
    const float w = expf(p.pm[pi] - M);
    L = fmaf(w, p.pl[pi], L);
    O = fmaf(w, p.po[pi * HD + d], O);
  }
  const float g = p.qfull[(size_t)b * p.qfs + (size_t)h * 2 * HD + HD + d];
  const float y = (O / L) * (1.f / (1.f + expf(-g)));
  p.yh[(size_t)b * p.NH * HD + (size_t)h * HD + d] = (_Float16)y;
}

}  // namespace

int embed_launch(const uint8_t *qs, const uint16_t *sc, int type, const int *toks, int B, int H, float *X,
                 int xs, float *ssq, hipStream_t st) {
  hipLaunchKernelGGL(embed_kernel, dim3((unsigned)B), dim3(256), 0, st, qs, sc, type, toks, H, X, xs, ssq);
  CWEN_HIP_TRY(hipGetLastError());
  return CWEN_OK;
}

size_t attn_partial_floats(int NH, int NKV, int max_ctx, int B) {
  const int nchunk = (max_ctx + TC - 1) / TC;
  return (size_t)NKV * nchunk * B * (NH / NKV) * (HD + 2);
}

// Dynamic LDS above 64 KB (B = 16 blocks) needs the attribute; set once per
// process before any launch (not inside a graph capture).
int attention_init() {
  static bool done = false;
  if (!done) {
    CWEN_HIP_TRY(hipFuncSetAttribute((const void *)attn_chunk_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                     160 * 1024));
    done = true;
  }
  return CWEN_OK;
}

// Chunk workgroups per kv head: enough to cover the chip at long contexts;
// more chunks than this are looped over.
constexpr int ATTN_CHUNK_WGS = 128;

int attention_launch(const float *qfull, int qfs, const float *kx, const float *vx, int kvs, const float *qn,
                     const float *kn, float *qbuf, float *K, float *V, const int *last, int B, int NH, int NKV,
                     int npairs, int nrot, float theta, float eps, float *part, int max_ctx, _Float16 *yh,
                     hipStream_t st) {
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
  hipLaunchKernelGGL(attn_prep_kernel, dim3((unsigned)B, (unsigned)(NH + NKV)), dim3(HD), 0, st, p);
  const int nwg = p.nchunk < ATTN_CHUNK_WGS ? p.nchunk : ATTN_CHUNK_WGS;
  const size_t lds = ((size_t)TC * KROW + (size_t)nq * (TC + HD)) * sizeof(float);
  int rc;
  if ((rc = attention_init())) return rc;
  hipLaunchKernelGGL(attn_chunk_kernel, dim3((unsigned)nwg, (unsigned)NKV), dim3(256), lds, st, p);
  hipLaunchKernelGGL(attn_merge_kernel, dim3((unsigned)B, (unsigned)NH), dim3(HD), 0, st, p);
  CWEN_HIP_TRY(hipGetLastError());
  return CWEN_OK;
}
