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
constexpr int TC = 64;               // keys per attention chunk

template <int CTRL> __device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float sum16(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  return v + dpp<0x140>(v);
}
__device__ __forceinline__ float sum64(float v) {
  const int b = __builtin_bit_cast(int, sum16(v));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
}
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
                                                    const int *toks, int H, float *X, int xs) {
  const int b = blockIdx.x;
  const size_t tok = (size_t)toks[b];
  const int nb = H / 32;
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
      dst[j] = (float)((int)(q[j] & 0xF) - 8) * d;
      dst[j + 16] = (float)((int)(q[j] >> 4) - 8) * d;
    }
  }
}

// ---- RMSNorm of B rows: y = w * x * (1/sqrt(mean(x^2) + eps)), f32 and/or
// f16 out.  Grid: B, 256 threads.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float *X, int xs, const float *w, int n, float eps,
                                                      float *Y, int ys, _Float16 *Yh, int yhs) {
  __shared__ float red[4];
  const int b = blockIdx.x;
  const float *x = X + (size_t)b * xs;
  float ss = 0.f;
  for (int i = threadIdx.x; i < n; i += 256) ss = fmaf(x[i], x[i], ss);
  const float s = 1.f / sqrtf(sum256(ss, red) / (float)n + eps);
  for (int i = threadIdx.x; i < n; i += 256) {
    const float v = w[i] * x[i] * s;
    if (Y) Y[(size_t)b * ys + i] = v;
    if (Yh) Yh[(size_t)b * yhs + i] = (_Float16)v;
  }
}

// ---- full attention, part 1: per (position, head) q/k RMSNorm (one shared
// [HD] weight each), partial RoPE on pairs (2i, 2i+1), i < npairs, and the
// KV-cache write.  Grid: (B, NH + NKV), 256 threads = head dims.
struct AttnParams {
  const float *qfull;  // [B][NH*2*HD]: per head q (HD) then gate (HD)
  const float *kx, *vx; int kvs;  // [B][kvs]: NKV*HD each
  const float *qn, *kn;
  float *q;            // [B][NH][HD] normed + roped queries
  float *K, *V;        // this layer's cache [ctx][NKV][HD]
  int pbase, B, NH, NKV, npairs, nrot;
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
  const int pos = p.pbase + b;
  const bool isq = h < p.NH;
  const int hk = h - p.NH;
  const float x = isq ? p.qfull[(size_t)b * p.NH * 2 * HD + (size_t)h * 2 * HD + d]
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

// ---- full attention, part 2: one workgroup per (key chunk, kv head) scores
// the chunk against every query of the group (kvm heads x B positions, each
// masked to t <= its position), then accumulates exp(s - m_chunk) * V.
// Lane = key within the chunk for the scores; thread = head dim for P.V.
__global__ __launch_bounds__(256) void attn_chunk_kernel(AttnParams p) {
  extern __shared__ float sm[];      // S / P [nq][TC], then q rows [nq][HD]
  const int c = blockIdx.x, hkv = blockIdx.y;
  const int kvm = p.NH / p.NKV;
  const int nq = p.B * kvm;
  const int t0 = c * TC;
  const int tlast = p.pbase + p.B - 1;       // last position of the block
  if (t0 > tlast) return;
  float *S = sm;                             // [nq][TC]
  float *Q = sm + nq * TC;                   // [nq][HD]
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const float scale = 1.f / sqrtf((float)HD);
  // queries of this group: (b, m) -> head hkv*kvm + m
  for (int e = tid; e < nq * HD; e += 256) {
    const int qi = e / HD, d = e % HD;
    const int b = qi / kvm, m = qi % kvm;
    Q[e] = p.q[((size_t)b * p.NH + hkv * kvm + m) * HD + d];
  }
  __syncthreads();
  // scores: wave w takes queries w, w+4, ...; lane = key t0 + lane
  {
    const int t = t0 + lane;
    const float *kr = p.K + ((size_t)t * p.NKV + hkv) * HD;
    const bool tv = t <= tlast;
    for (int qi = wave; qi < nq; qi += 4) {
      const int b = qi / kvm;
      const float *q = Q + qi * HD;
      float s = 0.f;
      if (tv && t <= p.pbase + b) {
        for (int d = 0; d < HD; d += 4) {
          const float4 k4 = *(const float4 *)(kr + d);
          s = fmaf(q[d], k4.x, s); s = fmaf(q[d + 1], k4.y, s);
          s = fmaf(q[d + 2], k4.z, s); s = fmaf(q[d + 3], k4.w, s);
        }
        s *= scale;
      } else {
        s = -__builtin_inff();
      }
      const float m = max64(s);
      const float e = (s == -__builtin_inff()) ? 0.f : expf(s - m);
      const float l = sum64(e);
      S[qi * TC + lane] = e;
      if (lane == 0) {
        const size_t pi = ((size_t)hkv * p.nchunk + c) * nq + qi;
        p.pm[pi] = m;
        p.pl[pi] = l;
      }
    }
  }
  __syncthreads();
  // P.V: thread = head dim
  {
    const int d = tid;
    const int tn = min(TC, tlast + 1 - t0);
    for (int qi = 0; qi < nq; ++qi) {
      const float *pr = S + qi * TC;
      float o = 0.f;
      for (int j = 0; j < tn; ++j) o = fmaf(pr[j], p.V[((size_t)(t0 + j) * p.NKV + hkv) * HD + d], o);
      p.po[(((size_t)hkv * p.nchunk + c) * nq + qi) * HD + d] = o;
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
  const int pos = p.pbase + b;
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
  const float g = p.qfull[(size_t)b * p.NH * 2 * HD + (size_t)h * 2 * HD + HD + d];
  const float y = (O / L) * (1.f / (1.f + expf(-g)));
  p.yh[(size_t)b * p.NH * HD + (size_t)h * HD + d] = (_Float16)y;
}

}  // namespace

int embed_launch(const uint8_t *qs, const uint16_t *sc, int type, const int *toks, int B, int H, float *X,
                 int xs, hipStream_t st) {
  hipLaunchKernelGGL(embed_kernel, dim3((unsigned)B), dim3(256), 0, st, qs, sc, type, toks, H, X, xs);
  CWEN_HIP_TRY(hipGetLastError());
  return CWEN_OK;
}

int rmsnorm_launch(const float *X, int xs, const float *w, int n, float eps, float *Y, int ys, _Float16 *Yh,
                   int yhs, int B, hipStream_t st) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)B), dim3(256), 0, st, X, xs, w, n, eps, Y, ys, Yh, yhs);
  CWEN_HIP_TRY(hipGetLastError());
  return CWEN_OK;
}

size_t attn_partial_floats(int NH, int NKV, int max_ctx, int B) {
  const int nchunk = (max_ctx + TC - 1) / TC;
  return (size_t)NKV * nchunk * B * (NH / NKV) * (HD + 2);
}

int attention_launch(const float *qfull, const float *kx, const float *vx, int kvs, const float *qn,
                     const float *kn, float *qbuf, float *K, float *V, int pbase, int B, int NH, int NKV,
                     int npairs, int nrot, float theta, float eps, float *part, int max_ctx, _Float16 *yh,
                     hipStream_t st) {
  AttnParams p;
  p.qfull = qfull; p.kx = kx; p.vx = vx; p.kvs = kvs;
  p.qn = qn; p.kn = kn;
  p.q = qbuf; p.K = K; p.V = V;
  p.pbase = pbase; p.B = B; p.NH = NH; p.NKV = NKV; p.npairs = npairs; p.nrot = nrot;
  p.theta = theta; p.eps = eps;
  p.nchunk = (max_ctx + TC - 1) / TC;
  const int nq = B * (NH / NKV);
  p.po = part;
  p.pm = part + (size_t)NKV * p.nchunk * nq * HD;
  p.pl = p.pm + (size_t)NKV * p.nchunk * nq;
  p.yh = yh;
  hipLaunchKernelGGL(attn_prep_kernel, dim3((unsigned)B, (unsigned)(NH + NKV)), dim3(HD), 0, st, p);
  const int nc = (pbase + B - 1) / TC + 1;
  const size_t lds = (size_t)nq * (TC + HD) * sizeof(float);
  static bool lds_set = false;  // allow the dynamic LDS of B = 16 blocks (above 64 KB)
  if (!lds_set) {
    CWEN_HIP_TRY(hipFuncSetAttribute((const void *)attn_chunk_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                     160 * 1024));
    lds_set = true;
  }
  hipLaunchKernelGGL(attn_chunk_kernel, dim3((unsigned)nc, (unsigned)NKV), dim3(256), lds, st, p);
  hipLaunchKernelGGL(attn_merge_kernel, dim3((unsigned)B, (unsigned)NH), dim3(HD), 0, st, p);
  CWEN_HIP_TRY(hipGetLastError());
  return CWEN_OK;
}
