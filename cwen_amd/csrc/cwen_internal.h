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

struct cwen_ctx {
  int device;
  float *partials;          // split-K partial sums
  size_t partials_floats;
  int *counters;            // per row-tile arrival counters, kept at zero between calls
  int ncounters;
  int wg_target;            // workgroups a split-K launch aims for
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
  int split, tps;           // split-K factor and K tiles per split (shape-only)
};

#define CWEN_HIP_TRY(expr)                                   \
  do {                                                       \
    hipError_t _e = (expr);                                  \
    if (_e != hipSuccess) return CWEN_EHIP;                  \
  } while (0)

// q4_gemv.hip
int q4_repack(cwen_weight *w, const uint8_t *dsrc, const uint16_t *dsc, hipStream_t st);
void q4_choose_split(const cwen_ctx *ctx, cwen_weight *w);
enum { Q4_EPI_STORE = 0, Q4_EPI_SWIGLU = 1 };
int q4_gemv_launch(cwen_ctx *ctx, const cwen_weight *w, int nsides, int side0, int epi,
                   const float *X, int xs, float *Y0, float *Y1, int ys, int B,
                   hipStream_t st);
