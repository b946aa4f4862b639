// Internal declarations shared by the HIP translation units of libcwen_gpu.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "cwen_gpu.h"

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

// Weight super-tile: 16 rows x 512 K of one weight stream, four 128-K tiles
// in MFMA operand order (lane l = 16*g + n of a wave owns 32-weight block g of
// row n in each tile) followed by the format's scales.  The per-format byte
// layouts are described in gemv.hip.
constexpr int Q4_TILE_K = 128;
constexpr int Q4_ST_TILES = 4;
constexpr int Q4_ST_K = Q4_ST_TILES * Q4_TILE_K;            // 512
constexpr int Q4_ROWS = 16;
// K must be a whole number of super-tiles.
constexpr int Q4_K_ALIGN = Q4_ST_K;

enum { GEMV_Q4 = 0, GEMV_Q6K = 1, GEMV_Q8 = 2, GEMV_Q41 = 3, GEMV_Q5K = 4 };

struct cwen_ctx {
  int device;
  int ncu;                  // compute units of the device
  int wg_per_cu;            // GEMV workgroups per CU a split launch aims for
  _Float16 *xh;             // f16 activation scratch [BMAX][KMAX]
  _Float16 *hh;             // second f16 scratch (FFN hidden) [BMAX][KMAX]
  float *partials;          // split-K partial sums
  size_t partials_floats;
  int *counters;            // per split-tile arrival counters, zero between launches
  int ncounters;
  unsigned long long *amax_keys;  // per-column argmax keys [CWEN_BMAX], zero between launches
  int *amax_cnt;            // argmax arrival counter, zero between launches
  int *res;                 // device result slots of the verify entry points [2 + CWEN_BMAX]
};

// A GEMV launch's work decomposition (gemv.hip): grid workgroups, the first
// nsplit of which take pieces (S per tile, rps rounds each) of row tiles
// tile0 .. tile0 + nsplit / S - 1; the others take whole row tiles.
struct GemvGrid {
  int grid, nsplit, S, rps, tile0;
};

struct cwen_weight {
  cwen_ctx *ctx;
  int type;                 // CWEN_T_*
  int fmt;                  // GEMV_Q4 / GEMV_Q6K / GEMV_Q8 / GEMV_Q41 / GEMV_Q5K
  int ne0, ne1;             // K, M
  int nside;                // 2 for an interleaved pair, else 1
  int nrg, nst;             // 16-row groups, 512-wide K super-tiles
  uint8_t *dev;             // tiled device data
  size_t bytes;             // device bytes of the tiled data
  size_t src_bytes;         // bytes of the reference layout (qs + scales)
  GemvGrid cfg[2];          // decomposition for one side / both sides of a pair (shape-only)
  int rows;                 // row groups per wave (shape-only)
};

// GatedDeltaNet layer state (gdn.hip): the recurrent state [nvh][dk][dk] in
// two base slots, the conv history [C][3] in a ring of nslot slots, and the
// pending inputs of the last block for a replay.  The device control word
// ctl[4] = {ring slot, base slot X, replay count L, pending parity P} is what
// the kernels read; the host keeps a copy.
struct cwen_gdn {
  cwen_ctx *ctx;
  int nkh, nvh, dk, C;
  int nslot;
  int cur, X, L, P;         // host copy of ctl
  int *ctl;                 // device control word
  int own_ctl;              // ctl allocated by this object (else part of a model's)
  int last_B;               // positions of the last, uncommitted block (0: none)
  float *S, *H;             // device: base states [2][nvh][dk][dk], history ring [nslot][C][3]
  float *xc, *gates;        // pending post-conv values [2][BMAX][C], g and beta [2][BMAX][2][nvh]
  float *S_peek;            // scratch for cwen_gdn_get_state (allocated on first use)
};
// Host copy of committing n positions of a block of B (0: no block, no-op):
// the ring slot moves by n; a whole block makes its end state (the other
// base slot) current, a prefix leaves the start state current with n
// positions to replay; the pending parity flips.  The model's device commit
// (advance_kernel) applies the same rule to the device word.
inline void gdn_commit_host(cwen_gdn *g, int n, int B) {
  if (B == 0) return;
  g->cur = (g->cur + n) % g->nslot;
  if (n == B) {
    g->X ^= 1;
    g->L = 0;
  } else {
    g->L = n;
  }
  g->P ^= 1;
  g->last_B = 0;
}

#define CWEN_HIP_TRY(expr)                                   \
  do {                                                       \
    hipError_t _e = (expr);                                  \
    if (_e != hipSuccess) return CWEN_EHIP;                  \
  } while (0)

// ------------------------------------------------------------ device helpers
// gfx9 raw buffer resource: 32-bit offsets; loads past num_records return
// zero without touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
// `voff` is the per-lane offset (the part the range check sees); `soff` a
// wave-uniform offset carried in a scalar register.
__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff = 0) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
__device__ __forceinline__ uint2 bload8(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff = 0) {
  return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
}
// Non-temporal variants (cache policy nt) for data read once per launch: the
// weight stream.  They keep the stream from displacing what is reused from
// the caches (the staged activations), and a plain 100 MB read with them
// ran 5 % faster on this part than with default loads.
constexpr int kNT = 2;
__device__ __forceinline__ uint4 bload16_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff = 0) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kNT));
}
__device__ __forceinline__ uint2 bload8_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff = 0) {
  return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, kNT));
}
__device__ __forceinline__ uint32_t bload4_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff = 0) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, kNT);
}

// Cross-lane sums on DPP row permutes (no LDS round trip).  The reduction
// tree is fixed, so a sum is bit-reproducible.
template <int CTRL> __device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// Sum over each aligned row of 16 lanes: quad xor 1, quad xor 2, half-row
// mirror, row mirror.
__device__ __forceinline__ float sum16(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  return v + dpp<0x140>(v);
}
// Sum over the wave (wave-uniform result).
__device__ __forceinline__ float sum64(float v) {
  const int b = __builtin_bit_cast(int, sum16(v));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
}

// LDS hand-off barrier: waits for this wave's LDS writes only, not for its
// outstanding global loads (unlike __syncthreads(), whose release fence
// drains the memory counter: loads and stores in flight).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // gfx9 encoding: lgkmcnt(0), vmcnt/expcnt unchanged
  __builtin_amdgcn_s_barrier();
}
// run.c:378-384 silu_one: x * (1 / (1 + exp(-x)))
__device__ __forceinline__ float silu_f(float x) { return x * (1.f / (1.f + expf(-x))); }

// An f16 operand that is not finite: the f32 value left f16's range (or was
// not finite itself).  Writers of f16 operands raise a sticky flag, which the
// model's entry points report.
__device__ __forceinline__ bool f16_bad(_Float16 h) { return !(__builtin_fabsf((float)h) <= 65504.f); }
__device__ __forceinline__ void raise_flag(int *flag) {
  if (flag) __hip_atomic_store(flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Row-tile partials of a column's sum of squares: at most 128 per column.
constexpr int CWEN_MAX_PARTS = 128;

// ------------------------------------------------------------ gemv.hip
enum { GEMV_EPI_STORE = 0, GEMV_EPI_PAIR = 1, GEMV_EPI_SWIGLU = 2, GEMV_EPI_ARGMAX = 3, GEMV_EPI_CONV = 4 };
struct ArgmaxOut {
  unsigned long long *keys;  // per-column keys, zero between launches
  int *cnt;                  // arrival counter, zero between launches
  const int *drafts;         // device draft ids [E]
  int E;
  int *out;                  // device: k, bonus, argmax of columns 0..B-1
};
struct GemvOut {
  float *y;          // f32 result (side A, or silu(A)*B, or logits) [c*ys + row], nullable
  float *y1;         // f32 side B of a pair [c*ys + row] (PAIR only)
  _Float16 *yh;      // f16 copy of the (accumulated) result [c*M + row], nullable
  int ys;
  int accumulate;    // y += result
  ArgmaxOut am;      // ARGMAX only
  float *ssq;        // STORE: per row tile, the sum of squares of the final y per column [CWEN_BMAX][CWEN_MAX_PARTS]
  const float *nwh;  // with yh: the f16 copy holds y * nwh[row] (the next RMSNorm's weight), nullable
  // CONV (a STORE whose rows < cv_C are GatedDeltaNet q/k/v channels): they get the
  // depthwise causal conv + SiLU (run.c conv1d_update) instead of a store:
  // position b of channel c goes to the pending buffer, cv_xc[(P*BMAX + b)*
  // cv_C + c], and its inputs b-2, b-1, b to history slot (cur + 1 + b) %
  // cv_nslot, cv_H[slot*3*cv_C + 3c ..], with cur = cv_ctl[0], P = cv_ctl[3];
  // positions before the block come from slot cur.  cv_w: [cv_C][4] taps.
  const float *cv_w;
  float *cv_H, *cv_xc;
  const int *cv_ctl;
  int cv_C, cv_nslot;
  int *rflag;        // with yh: set to 1 when an f16 value written is not finite (out of f16's range), nullable
};
// f32 activations that the GEMV converts to its f16 operand while staging.
struct GemvF32 {
  const float *x;    // [c*xs + k], 16-byte aligned, xs % 4 == 0
  int xs;            // row stride of x in floats (>= K when B > 1)
};
// RMSNorm split between producer and consumer: the f16 operand holds w * x
// (x not yet normalised) and output column c is multiplied by
// 1 / sqrt(sum_p ssq[c][p] / K + eps), the partials summed in a fixed order.
struct GemvPost {
  const float *ssq;  // [CWEN_BMAX][CWEN_MAX_PARTS], partials 0 .. npart - 1 of each column
  int npart;         // 1 .. CWEN_MAX_PARTS
  float eps;
};
int gemv_fmt_of(int type);
size_t gemv_st_bytes(int fmt);
int gemv_repack(cwen_weight *w, const uint8_t *dsrc, const uint16_t *dsc, hipStream_t st);
// Repack a Q4 source of M rows (side side_sel of a Q4_0RSI source, else -1)
// into rows row_off.. of a single-sided Q4 weight (row-concatenated weights).
int gemv_repack_part(cwen_weight *w, const uint8_t *dsrc, const uint16_t *dsc, int type, int M, int row_off,
                     int side_sel, hipStream_t st);
// A zero-filled single-sided Q4 weight of K x M to receive parts.
int gemv_alloc_q4(cwen_ctx *ctx, int K, int M, cwen_weight **out);
// Upload a Q4 source from HOST memory into rows row_off.. of w.
int gemv_upload_part(cwen_weight *w, int type, const void *data, const void *scales, int M, int row_off,
                     int side_sel);
void gemv_choose_split(const cwen_ctx *ctx, cwen_weight *w);
// Split-K scratch of a launch: partial sums and per-split-tile arrival
// counters (zero between launches; the last arriver of a tile resets its own).
struct GemvScratch {
  float *partials;
  size_t partials_floats;
  int *counters;
  int ncounters;
};
// Whether a decomposition's split pieces fit the given scratch.
bool gemv_grid_fits(const GemvGrid &g, size_t partials_floats, int ncounters);
// Row tiles of a launch over w: the number of ssq partials it writes.
int gemv_row_tiles(const cwen_weight *w);
// post (f16 operand only): the operand is w * x with x not yet normalised;
// each output column c is scaled by 1 / sqrt(sum_p post->ssq[c][p] / K +
// post->eps), completing the RMSNorm (post->x, post->w unused).
// scr (nullable) replaces the context's split-K scratch; a decomposition that
// does not fit it returns CWEN_ESCRATCH before any launch.
int gemv_launch(cwen_ctx *ctx, const cwen_weight *w, int nsides, int side0, int epi,
                const _Float16 *xh, const GemvOut &out, int B, hipStream_t st, const GemvF32 *xf = nullptr,
                const GemvPost *post = nullptr, const GemvScratch *scr = nullptr);
int act_to_f16(const float *x, int xs, _Float16 *xh, int K, int B, hipStream_t st);
int argmax_walk_launch(const float *lg, long ls, int V, int B, const ArgmaxOut &a, hipStream_t st);

// ------------------------------------------------------------ gdn.hip
int gdn_block_launch(const cwen_gdn *g, const float *qkv, int qs, const float *z, int zs,
                     const float *decay, const float *beta, int gs, const float *kw, const float *wn,
                     float *out, int os, int B, hipStream_t st, _Float16 *outh = nullptr, int ohs = 0,
                     const float *A = nullptr, const float *dt = nullptr, int force_L0 = 0,
                     int *rflag = nullptr, bool conv_done = false);
// The conv's part of a GemvOut for the block's in-projection (its output
// rows < g->C): the GEMV then does what gdn_conv_kernel would, and
// gdn_block_launch is called with conv_done.
void gdn_conv_out(const cwen_gdn *g, const float *kw, GemvOut &o);
// The state after replaying L positions of pending buffer buf from base slot
// X into S_out (device, [nvh][dk][dk]).
int gdn_peek_launch(const cwen_gdn *g, int L, int buf, float *S_out, hipStream_t st);

// ------------------------------------------------------------ model.hip
// Also writes each row's sum of squares to ssq[b][0] (one partial per column)
// and, when xh is given, the f16 operand x * nw of the first RMSNorm.
// rflag (nullable) is set to 1 when an f16 value written is not finite.
int embed_launch(const uint8_t *qs, const uint16_t *sc, int type, const int *toks, int B, int H, float *X,
                 int xs, float *ssq, hipStream_t st, _Float16 *xh = nullptr, const float *nw = nullptr,
                 int *rflag = nullptr);
size_t attn_partial_floats(int NH, int NKV, int max_ctx, int B);
int attention_init();
// Largest query heads per KV head the attention kernels take at every block
// size up to CWEN_BMAX (the block's queries of one KV head stay in registers).
int attention_max_group();
// `last` is a device int: the last filled cache slot before the block (the
// block's positions are last+1 .. last+B).  The launch shape depends on
// (B, NH, NKV, max_ctx) and attention_wide(last_hint) only, so a captured
// graph replays at any position of the same band; any hint gives the same
// result.
int attention_launch(const float *qfull, int qfs, const float *kx, const float *vx, int kvs, const float *qn,
                     const float *kn, float *qbuf, float *K, float *V, const int *last, int B, int NH, int NKV,
                     int npairs, int nrot, float theta, float eps, float *part, int max_ctx, _Float16 *yh,
                     hipStream_t st, int *rflag = nullptr, int last_hint = -1);
// Whether a block whose last position is last_pos takes the wide chunk grid
// (attention_launch's last_hint; -1 = not known, narrow).  Only the launch
// shape depends on it, never the result.
bool attention_wide(int last_pos);
