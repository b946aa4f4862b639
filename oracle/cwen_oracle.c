/* cwen oracle: scalar CPU restatement of the reference hot path.
 *
 * TEST INFRASTRUCTURE ONLY (the tests check results against it; it is never
 * the thing measured or shipped).  Each function restates the scalar branch of the cited run.c
 * function with the same f32 evaluation order; it must be compiled with
 * -std=c11 (gcc: no FP contraction) so rounding matches the reference's
 * scalar build bit for bit.
 */
#include "cwen_oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>

static const float ORC_EPS = 1e-6f;              /* RMS_EPS, run.c:89 */

/* run.c:293-299 -- exact half->float incl. denormals, Inf, NaN */
float orc_f16_to_f32(uint16_t h) {
  uint32_t s = (h >> 15) & 1u, e = (h >> 10) & 0x1fu, f = h & 0x3ffu, u;
  if (e == 0) {
    if (!f) return s ? -0.f : 0.f;
    float v = ldexpf((float)f, -24);
    return s ? -v : v;
  }
  if (e == 31) return f ? NAN : (s ? -INFINITY : INFINITY);
  u = (s << 31) | ((e - 15 + 127) << 23) | (f << 13);
  float r;
  memcpy(&r, &u, 4);
  return r;
}

/* run.c:447-470 -- float->half, round to nearest even, NaN -> quiet NaN */
uint16_t orc_f32_to_f16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  uint32_t sign = (u >> 16) & 0x8000u, rest = u & 0x7fffffffu;
  if (rest >= 0x7f800000u)
    return (uint16_t)(sign | 0x7c00u | (rest > 0x7f800000u ? 0x0200u : 0));
  if (rest < 0x33000000u) return (uint16_t)sign;
  uint32_t e = rest >> 23, m = rest & 0x7fffffu;
  if (e < 113) {
    uint32_t t = 0x800000u | m, sh = 126u - e, half = 1u << (sh - 1);
    uint32_t r = t >> sh, rem = t & ((half << 1) - 1u);
    if (rem > half || (rem == half && (r & 1u))) r++;
    return (uint16_t)(sign + r);
  }
  uint32_t he = e - 112u, r = m >> 13u, rem = m & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) {
    if (++r == 0x400u) { r = 0; he++; }
  }
  if (he >= 31u) return (uint16_t)(sign | 0x7c00u);
  return (uint16_t)(sign | (he << 10) | r);
}

static uint16_t ld16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* run.c:432-437 dot_nib16: one 16-byte Q4 block, lo nibble -> y[j], hi -> y[j+16] */
static float nib16(const uint8_t *q, float d, const float *yy) {
  float s = 0;
  for (int j = 0; j < 16; j++)
    s += ((int)(q[j] & 0xF) - 8) * d * yy[j] + ((int)(q[j] >> 4) - 8) * d * yy[j + 16];
  return s;
}

/* run.c:1009-1025 scalar branch (GGUF 18-byte blocks) */
float orc_dot_q4_0(const uint8_t *blk18, const float *y, int K) {
  int nb = K / 32;
  float sum = 0;
  for (int i = 0; i < nb; i++) {
    const uint8_t *b = blk18 + (size_t)i * 18;
    float d = orc_f16_to_f32(ld16(b));
    sum += nib16(b + 2, d, y + i * 32);
  }
  return sum;
}

/* run.c:753-767 scalar branch (split stream + f16 scale channel) */
float orc_dot_q4_rs(const uint8_t *qs, const uint16_t *sc, const float *y, int K) {
  int nb = K / 32;
  float sum = 0;
  for (int i = 0; i < nb; i++) {
    float d = orc_f16_to_f32(sc[i]);
    sum += nib16(qs + (size_t)i * 16, d, y + i * 32);
  }
  return sum;
}

/* run.c:942-975 scalar branch (one side of an interleaved pair) */
float orc_dot_q4_rsi(const uint8_t *qs, const uint16_t *sc, int side, const float *y, int K) {
  int nb = K / 32;
  float sum = 0;
  for (int i = 0; i < nb; i++) {
    float d = orc_f16_to_f32(sc[2 * i + side]);
    sum += nib16(qs + (size_t)i * 32 + side * 16, d, y + i * 32);
  }
  return sum;
}

/* run.c:1087-1096 scalar branch (GGUF 20-byte blocks {d, m, qs}): w = n*d + m,
 * lo nibble -> y[j], hi -> y[j+16] */
float orc_dot_q4_1(const uint8_t *blk20, const float *y, int K) {
  int nb = K / 32;
  float sum = 0;
  for (int i = 0; i < nb; i++) {
    const uint8_t *b = blk20 + (size_t)i * 20;
    float d = orc_f16_to_f32(ld16(b)), m = orc_f16_to_f32(ld16(b + 2));
    const float *yy = y + i * 32;
    for (int j = 0; j < 16; j++) {
      int x0 = b[4 + j] & 0xF, x1 = b[4 + j] >> 4;
      sum += (x0 * d + m) * yy[j] + (x1 * d + m) * yy[j + 16];
    }
  }
  return sum;
}

/* run.c:426-429 get_scale_min_k4: the 6-bit scale and min of sub-block j */
static void scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
  if (j < 4) {
    *d = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

/* run.c:1142-1156 scalar branch.  Super-block {f16 d; f16 dmin; u8 scales[12];
 * u8 qh[32]; u8 qs[128]} (176 B per 256): for 64-group jj, weight l < 32 is
 * (qs[32jj+l] & 15) + 16*(qh[l] bit 2jj), scale/min of sub-block 2jj; weight
 * 32 + l is (qs[32jj+l] >> 4) + 16*(qh[l] bit 2jj+1), sub-block 2jj+1;
 * w = d*sc*q - dmin*m. */
float orc_dot_q5_K(const uint8_t *blk176, const float *y, int K) {
  float sum = 0;
  const float *yy = y;
  for (int i = 0, nb = K / 256; i < nb; i++) {
    const uint8_t *b = blk176 + (size_t)i * 176;
    const uint8_t *scales = b + 4, *qh = b + 16, *ql = b + 48;
    float d = orc_f16_to_f32(ld16(b)), min = orc_f16_to_f32(ld16(b + 2));
    int is = 0;
    uint8_t u1 = 1, u2 = 2;
    for (int j = 0; j < 256; j += 64) {
      uint8_t sc, m;
      scale_min_k4(is + 0, scales, &sc, &m);
      float d1 = d * sc, m1 = min * m;
      scale_min_k4(is + 1, scales, &sc, &m);
      float d2 = d * sc, m2 = min * m;
      for (int l = 0; l < 32; l++) sum += (d1 * ((ql[l] & 0xF) + (qh[l] & u1 ? 16 : 0)) - m1) * yy[l];
      for (int l = 0; l < 32; l++) sum += (d2 * ((ql[l] >> 4) + (qh[l] & u2 ? 16 : 0)) - m2) * yy[32 + l];
      yy += 64; ql += 32; is += 2; u1 <<= 2; u2 <<= 2;
    }
  }
  return sum;
}

/* run.c:1248-1274 scalar branch */
float orc_dot_q8_0(const uint8_t *blk34, const float *y, int K) {
  int nb = K / 32;
  float sum = 0;
  for (int i = 0; i < nb; i++) {
    const uint8_t *b = blk34 + (size_t)i * 34;
    float d = orc_f16_to_f32(ld16(b));
    const float *yy = y + i * 32;
    for (int j = 0; j < 32; j++) sum += (float)(int8_t)b[2 + j] * d * yy[j];
  }
  return sum;
}

/* run.c:1226-1245 scalar branch. Super-block: ql[128] qh[64] sc[16] d */
float orc_dot_q6_K(const uint8_t *blk210, const float *y, int K) {
  float sum = 0;
  const float *yy = y;
  for (int i = 0, nb = K / 256; i < nb; i++) {
    const uint8_t *b = blk210 + (size_t)i * 210;
    float d = orc_f16_to_f32(ld16(b + 208));
    const uint8_t *ql = b, *qh = b + 128;
    const int8_t *sc = (const int8_t *)(b + 192);
    for (int n0 = 0; n0 < 256; n0 += 128) {
      for (int l = 0; l < 32; l++) {
        int is = l / 16;
        int8_t q1 = (int8_t)((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
        int8_t q2 = (int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
        int8_t q3 = (int8_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
        int8_t q4 = (int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
        sum += d * sc[is + 0] * q1 * yy[l] + d * sc[is + 2] * q2 * yy[l + 32]
             + d * sc[is + 4] * q3 * yy[l + 64] + d * sc[is + 6] * q4 * yy[l + 96];
      }
      yy += 128; ql += 64; qh += 32; sc += 8;
    }
  }
  return sum;
}

/* run.c:1364-1387 gemv_row: one output row of W against activation y */
static float row_dot(const orc_tensor *W, const float *y, int i) {
  int K = W->ne0, nb = K / 32;
  const uint8_t *d = (const uint8_t *)W->data;
  switch (W->type) {
    case ORC_Q4_0:   return orc_dot_q4_0(d + (size_t)i * nb * 18, y, K);
    case ORC_Q4_0RS: return orc_dot_q4_rs(d + (size_t)i * nb * 16,
                                          (const uint16_t *)W->scales + (size_t)i * nb, y, K);
    case ORC_Q4_0RSI:return orc_dot_q4_rsi(d + (size_t)i * nb * 32,
                                           (const uint16_t *)W->scales + (size_t)i * nb * 2,
                                           W->pair_side, y, K);
    case ORC_Q8_0:   return orc_dot_q8_0(d + (size_t)i * nb * 34, y, K);
    case ORC_Q4_1:   return orc_dot_q4_1(d + (size_t)i * nb * 20, y, K);
    case ORC_Q5_K:   return orc_dot_q5_K(d + (size_t)i * (K / 256) * 176, y, K);
    case ORC_Q6_K:   return orc_dot_q6_K(d + (size_t)i * (K / 256) * 210, y, K);
    case ORC_F32: {
      const float *w = (const float *)W->data + (size_t)i * K;
      float s = 0;
      for (int k = 0; k < K; k++) s += w[k] * y[k];  /* run.c:1288 */
      return s;
    }
    default: return NAN;
  }
}

/* run.c:1577-1680 gemvb; per-column dots (the generic path, run.c:1666-1679) */
int orc_gemvb(const orc_tensor *W, const float *X, int xs, float *Y, int ys, int B) {
  if (!W || W->ne0 <= 0 || W->ne1 <= 0 || B < 1) return -1;
  if (W->ne0 % (W->type == ORC_Q6_K || W->type == ORC_Q5_K ? 256 : 32) != 0 && W->type != ORC_F32) return -1;
  for (int i = 0; i < W->ne1; i++)
    for (int b = 0; b < B; b++)
      Y[(size_t)b * ys + i] = row_dot(W, X + (size_t)b * xs, i);
  return 0;
}

/* run.c:378-384 */
float orc_silu(float x) { return x * (1.f / (1.f + expf(-x))); }

/* run.c:1697-1713 scalar branch: a = silu(a) * b */
void orc_silu_mul(float *a, const float *b, int n) {
  for (int i = 0; i < n; i++) a[i] = orc_silu(a[i]) * b[i];
}

/* run.c:346-368 scalar branch */
void orc_rmsnorm(float *o, const float *x, const float *w, int n) {
  float ss = 0;
  for (int i = 0; i < n; i++) ss += x[i] * x[i];
  float s = 1.f / sqrtf(ss / n + ORC_EPS);
  for (int i = 0; i < n; i++) o[i] = w[i] * x[i] * s;
}

/* run.c:401-423 scalar branch */
void orc_l2norm_rows(float *x, int rows, int dim) {
  for (int r = 0; r < rows; r++) {
    float *p = x + (size_t)r * dim;
    float ss = 0;
    for (int i = 0; i < dim; i++) ss += p[i] * p[i];
    float s = 1.f / sqrtf(ss + ORC_EPS);
    for (int i = 0; i < dim; i++) p[i] *= s;
  }
}

/* run.c:1683-1695 scalar branch */
void orc_residual_add(float *dst, const float *d, int n) {
  for (int i = 0; i < n; i++) dst[i] += d[i];
}

/* run.c:392-399 */
float orc_softplus(float x) { return x > 20.f ? x : logf(1.f + expf(x)); }
float orc_sigmoid(float x) { return 1.f / (1.f + expf(-x)); }

/* run.c:2183-2200: out = st0*w0+st1*w1+st2*w2+cur*w3, shift history, then SiLU */
void orc_conv1d_update(float *qkv, float *hist, const float *kw, int C) {
  for (int c = 0; c < C; c++) {
    const float *w = kw + (size_t)c * 4;
    float *st = hist + (size_t)c * 3;
    float cur = qkv[c];
    qkv[c] = st[0] * w[0] + st[1] * w[1] + st[2] * w[2] + cur * w[3];
    st[0] = st[1]; st[1] = st[2]; st[2] = cur;
  }
  for (int c = 0; c < C; c++) qkv[c] = orc_silu(qkv[c]);   /* silu_vec, run.c:386-391 */
}

/* run.c:2014-2180 gdn_step, scalar branches */
void orc_gdn_step(float *S, float *qkv, const float *z, const float *decay,
                  const float *beta, const float *wn, float *out,
                  int nkh, int nvh, int dk) {
  float scale = 1.f / sqrtf((float)dk);
  float *q0 = qkv, *k0 = qkv + nkh * dk, *v0 = qkv + 2 * nkh * dk;
  orc_l2norm_rows(q0, nkh, dk);
  orc_l2norm_rows(k0, nkh, dk);
  float sk[512], delta[512];
  for (int hv = 0; hv < nvh; hv++) {
    int hk = hv % nkh;                                   /* run.c:2027 */
    float *q = q0 + hk * dk, *k = k0 + hk * dk, *v = v0 + hv * dk;
    float *Sh = S + (size_t)hv * dk * dk;
    float g = expf(decay[hv]);
    float bh = beta[hv];
    for (int i = 0; i < dk * dk; i++) Sh[i] *= g;
    for (int j = 0; j < dk; j++) {
      float s = 0;
      for (int i = 0; i < dk; i++) s += Sh[i * dk + j] * k[i];
      sk[j] = s;
    }
    for (int j = 0; j < dk; j++) delta[j] = bh * (v[j] - sk[j]);
    for (int i = 0; i < dk; i++) {
      float ki = k[i];
      for (int j = 0; j < dk; j++) Sh[i * dk + j] += ki * delta[j];
    }
    float *o = out + hv * dk;
    for (int j = 0; j < dk; j++) {
      float s = 0;
      for (int i = 0; i < dk; i++) s += Sh[i * dk + j] * q[i];
      o[j] = s * scale;
    }
  }
  for (int hv = 0; hv < nvh; hv++) {                     /* gated RMSNorm, run.c:2165-2176 */
    float *o = out + hv * dk;
    const float *zz = z + hv * dk;
    float ss = 0;
    for (int i = 0; i < dk; i++) ss += o[i] * o[i];
    float s = 1.f / sqrtf(ss / dk + ORC_EPS);
    for (int i = 0; i < dk; i++) {
      float gz = zz[i] * (1.f / (1.f + expf(-zz[i])));
      o[i] = wn[i] * o[i] * s * gz;
    }
  }
}

/* run.c:2647-2668: first index of the max; NaN never wins a strict '>' */
int orc_argmax(const float *lg, int V) {
  int bi = 0;
  float bv = lg[0];
  for (int i = 1; i < V; i++)
    if (lg[i] > bv) { bv = lg[i]; bi = i; }
  return bi;
}

/* run.c:4954-4956 */
int orc_walk(const float *logits, long ls, int V, const int *drafts, int E, int *bonus) {
  int k = 0;
  const float *cur = logits;
  while (k < E && orc_argmax(cur, V) == drafts[k]) { k++; cur = logits + (size_t)k * ls; }
  *bonus = orc_argmax(cur, V);
  return k;
}

/* run.c:4533-4549 */
int orc_ngram_draft(const int *h, int hn, int *out, int n_key, int max_d) {
  if (hn <= n_key || max_d <= 0) return 0;
  const int *tail = h + hn - n_key;
  int best = 0;
  for (int j = hn - n_key - 1; j >= 0 && best < max_d; j--) {
    if (memcmp(h + j, tail, (size_t)n_key * sizeof(int))) continue;
    int avail = hn - (j + n_key);
    if (avail > best) {
      int n = avail < max_d ? avail : max_d;
      memcpy(out, h + j + n_key, (size_t)n * sizeof(int));
      best = n;
    }
  }
  return best;
}

/* run.c:1829-1848 embed_q6_k: per 256-weight super-block {ql[128], qh[64],
 * i8 scales[16], f16 d}, each half of 128 weights taking 64 ql bytes, 32 qh
 * bytes and 8 scales; weight n0 + 32 q + l (quarter q, l < 32) is
 * (d * sc[2q + l/16]) * (q6 - 32), the 6-bit value from the low (q = 0, 1)
 * or high (q = 2, 3) nibble of ql[32 (q & 1) + l] and bits 2q, 2q+1 of qh[l]. */
static void embed_q6_k_row(const uint8_t *row, int H, float *dst) {
  for (int i = 0; i < H / 256; i++) {
    const uint8_t *b = row + (size_t)i * 210;
    const uint8_t *ql = b, *qh = b + 128;
    const int8_t *sc = (const int8_t *)(b + 192);
    const float d = orc_f16_to_f32(ld16(b + 208));
    float *o = dst + (size_t)i * 256;
    for (int n0 = 0; n0 < 256; n0 += 128) {
      for (int l = 0; l < 32; l++) {
        const int is = l / 16;
        o[n0 + l] = d * sc[is + 0] * ((int8_t)((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32);
        o[n0 + l + 32] = d * sc[is + 2] * ((int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32);
        o[n0 + l + 64] = d * sc[is + 4] * ((int8_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
        o[n0 + l + 96] = d * sc[is + 6] * ((int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
      }
      ql += 64; qh += 32; sc += 8;
    }
  }
}

/* run.c:1849-1887 embed_token_to: the Q4_0RS, Q4_0 and Q6_K branches */
void orc_embed(const uint8_t *qs, const uint16_t *sc, int type, int token, int H, float *dst) {
  if (type == ORC_Q6_K) {
    embed_q6_k_row(qs + (size_t)token * (H / 256) * 210, H, dst);
    return;
  }
  int nb = H / 32;
  for (int i = 0; i < nb; i++) {
    const uint8_t *q;
    float d;
    if (type == ORC_Q4_0) {
      const uint8_t *b = qs + ((size_t)token * nb + i) * 18;
      d = orc_f16_to_f32(ld16(b));
      q = b + 2;
    } else {
      q = qs + ((size_t)token * nb + i) * 16;
      d = orc_f16_to_f32(sc[(size_t)token * nb + i]);
    }
    for (int j = 0; j < 16; j++) {
      dst[i * 32 + j] = (float)((q[j] & 0xF) - 8) * d;
      dst[i * 32 + j + 16] = (float)((q[j] >> 4) - 8) * d;
    }
  }
}

/* run.c:1903-1948, mscale = 1 (no YaRN) */
void orc_rope_apply(float *q, int n_heads, int hd, int pos, int npairs, int nrot, float theta) {
  for (int h = 0; h < n_heads; h++) {
    float *v = q + (size_t)h * hd;
    for (int idx = 0; idx < npairs; idx++) {
      float freq = 1.f / powf(theta, (float)idx / (float)nrot);
      float ang = (float)pos * freq;
      float c = cosf(ang) * 1.f, s = sinf(ang) * 1.f;
      float a = v[idx * 2], b = v[idx * 2 + 1];
      v[idx * 2] = a * c - b * s;
      v[idx * 2 + 1] = a * s + b * c;
    }
  }
}

/* run.c:2362-2409, scalar branches (dot_f32 scalar: run.c:1275-1289) */
void orc_attention(const float *K, const float *V, int nkv, int hd, int t0, int pos, const float *q,
                   const float *gate, int nh, float *out) {
  float scale = 1.f / sqrtf((float)hd);
  int kv_mul = nh / nkv;
  float *at = (float *)malloc(sizeof(float) * (size_t)(pos + 1));
  memset(out, 0, sizeof(float) * (size_t)nh * hd);
  for (int hkv = 0; hkv < nkv; hkv++) {
    for (int m = 0; m < kv_mul; m++) {
      int h = hkv * kv_mul + m;
      const float *qh = q + (size_t)h * hd;
      for (int t = t0; t <= pos; t++) {
        const float *k = K + ((size_t)t * nkv + hkv) * hd;
        float s = 0;
        for (int i = 0; i < hd; i++) s += qh[i] * k[i];
        at[t] = s * scale;
      }
      float mx = at[t0];
      for (int t = t0 + 1; t <= pos; t++) if (at[t] > mx) mx = at[t];
      float sum = 0;
      for (int t = t0; t <= pos; t++) { at[t] = expf(at[t] - mx); sum += at[t]; }
      float inv = 1.f / sum;
      for (int t = t0; t <= pos; t++) at[t] *= inv;
      float *o = out + (size_t)h * hd;
      for (int t = t0; t <= pos; t++) {
        const float *vv = V + ((size_t)t * nkv + hkv) * hd;
        float a = at[t];
        for (int i = 0; i < hd; i++) o[i] += a * vv[i];
      }
      for (int i = 0; i < hd; i++) o[i] *= orc_sigmoid(gate[(size_t)h * hd + i]);
    }
  }
  free(at);
}
