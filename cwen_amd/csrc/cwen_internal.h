// Internal declarations shared by the HIP translation units of libcwen_gpu.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "cwen_gpu.h"

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

// Q4 tile: 16 rows x 4 blocks of 32 weights (128 K).  1024 bytes of nibbles
// in MFMA operand order (lane l = 16*g + n holds 16 bytes; dword m carries
// the 8 weights k = 8g..8g+7 of block m of row n) followed by 128 bytes of
// f16 scales laid out [n][m].
constexpr int Q4_TILE_QS = 1024;
constexpr int Q4_TILE_BYTES = 1152;
constexpr int Q4_TILE_K = 128;
constexpr int Q4_ROWS = 16;
// K must be a multiple of 4 tiles (one staging round of the GEMV).
constexpr int Q4_K_ALIGN = 4 * Q4_TILE_K;

struct cwen_ctx {
  int device;
  int wg_target;            // workgroups a GEMV launch aims for
  _Float16 *xh;             // f16 activation scratch [BMAX][KMAX]
  _Float16 *hh;             // second f16 scratch (FFN hidden) [BMAX][KMAX]
  float *partials;          // split-K partial sums
  size_t partials_floats;
  int *counters;            // per row-tile arrival counters, zero between launches
  int ncounters;
};

struct cwen_weight {
  cwen_ctx *ctx;
  int type;                 // CWEN_T_*
  int ne0, ne1;             // K, M
  int nside;                // 2 for an interleaved pair, else 1
  int nrg, nkt;             // 16-row groups, 128-wide K tiles
  uint8_t *dev;             // tiled device data
  size_t bytes;             // device bytes of the tiled data
  size_t src_bytes;         // bytes of the reference layout (qs + scales)
  int split, tps;           // K split across workgroups, K tiles per split (shape-only)
  int rows;                 // row groups per wave (shape-only)
};

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
__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ uint2 bload8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}

// run.c:378-384 silu_one: x * (1 / (1 + exp(-x)))
__device__ __forceinline__ float silu_f(float x) { return x * (1.f / (1.f + expf(-x))); }

// ------------------------------------------------------------ q4_gemv.hip
enum { Q4_EPI_STORE = 0, Q4_EPI_PAIR = 1, Q4_EPI_SWIGLU = 2 };
struct Q4Out {
  float *y;          // f32 result (side A, or silu(A)*B) [c*ys + row], nullable
  float *y1;         // f32 side B of a pair [c*ys + row] (PAIR only)
  _Float16 *yh;      // f16 copy of the (accumulated) result [c*M + row], nullable
  int ys;
  int accumulate;    // y += result
};
int q4_repack(cwen_weight *w, const uint8_t *dsrc, const uint16_t *dsc, hipStream_t st);
void q4_choose_split(const cwen_ctx *ctx, cwen_weight *w);
int q4_gemv_launch(cwen_ctx *ctx, const cwen_weight *w, int nsides, int side0, int epi,
                   const _Float16 *xh, const Q4Out &out, int B, hipStream_t st);
int act_to_f16(const float *x, int xs, _Float16 *xh, int K, int B, hipStream_t st);
