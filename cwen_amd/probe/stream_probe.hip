// Read-stream probes: the HBM read rate a kernel with no arithmetic reaches on
// this GPU, for the HBM-ceiling leg of bench.py.  Measurement aid only; the
// product library (libcwen_gpu.so) does not contain or call this code.
//
//  * cwen_probe_gemv_grid: the Q4 GEMV's weight stream without its arithmetic.
//    Same grid (the split pieces of the remainder tiles dispatched first, then
//    the whole tiles), same round-major super-tile layout (a 16-row x 512-K
//    super-tile of Q4_0 is 4096 B of nibbles + 512 B of scales; round r of
//    stream s starts at (r * nstream + s) * 4608), the same per-round loads per
//    wave (8 B of scales and 4 x 16 B of nibbles per lane, non-temporal, one
//    round in flight) and the activation staging loads from a small
//    cache-resident buffer.  What it does not do: dequantise, stage in LDS,
//    multiply, hand off partials or store outputs.
//  * cwen_probe_read: a plain read of `bytes` by 512 workgroups of 4 waves,
//    each wave reading 4 KB per step (round-major over the grid), 4 KB in
//    flight per wave.
// Every load goes through a buffer resource whose range is the buffer's size,
// so the probes read nothing outside the buffers they are given.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32;
constexpr int kNT = 2;   // non-temporal (read once), as the GEMV's weight loads

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *p, u32 n) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)n, 0x00020000);
}
__device__ __forceinline__ uint4 ld16(__amdgpu_buffer_rsrc_t r, u32 vo, u32 so, int aux) {
  return aux == kNT ? __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, kNT))
                    : __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, 0));
}
__device__ __forceinline__ uint2 ld8nt(__amdgpu_buffer_rsrc_t r, u32 vo, u32 so) {
  return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, vo, so, kNT));
}

constexpr u32 kTile = 4608;   // bytes of one 16-row x 512-K Q4_0 super-tile
constexpr u32 kStage = 8192;  // activation bytes staged per round (8 f16 columns x 512 K)

template <int XL>
__global__ __launch_bounds__(256) void gemv_grid_probe(const unsigned char *w, u32 wbytes, const unsigned char *x,
                                                       u32 xbytes, u32 *sink, int rounds, int nstream, int nwhole,
                                                       int npieces, int prs) {
  const __amdgpu_buffer_rsrc_t wr = rsrc(w, wbytes);
  const __amdgpu_buffer_rsrc_t xr = rsrc(x, xbytes);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const u32 rstride = (u32)nstream * kTile;
  u32 acc = 0;
  auto job = [&](int tile, int r0, int nr) {
    const u32 s = (u32)tile * 4 + wave;
    uint4 a[4], xs[XL > 0 ? XL : 1];
    uint2 sc;
    u32 o = (u32)r0 * rstride + s * kTile;
    sc = ld8nt(wr, 4096 + lane * 8, o);
#pragma unroll
    for (int i = 0; i < XL; ++i) xs[i] = ld16(xr, (wave * XL + i) * 1024 + lane * 16, (u32)r0 * kStage, 0);
#pragma unroll
    for (int d = 0; d < 4; ++d) a[d] = ld16(wr, d * 1024 + lane * 16, o, kNT);
    for (int it = 1; it <= nr; ++it) {
      const int rr = r0 + (it < nr ? it : nr - 1);   // the last step re-requests a round already read
      const u32 no = (u32)rr * rstride + s * kTile;
      acc ^= sc.x + sc.y;
      sc = ld8nt(wr, 4096 + lane * 8, no);
#pragma unroll
      for (int i = 0; i < XL; ++i) {
        acc ^= xs[i].x + xs[i].y + xs[i].z + xs[i].w;
        xs[i] = ld16(xr, (wave * XL + i) * 1024 + lane * 16, (u32)rr * kStage, 0);
      }
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        acc ^= a[d].x + a[d].y + a[d].z + a[d].w;
        a[d] = ld16(wr, d * 1024 + lane * 16, no, kNT);
      }
    }
    acc ^= sc.x;
#pragma unroll
    for (int d = 0; d < 4; ++d) acc ^= a[d].x;
  };
  const int b = blockIdx.x;
  const int ppt = (rounds + prs - 1) / prs;   // pieces per remainder tile
  if (b < npieces) {
    const int r0 = (b % ppt) * prs;
    job(nwhole + b / ppt, r0, min(prs, rounds - r0));
  } else {
    job(b - npieces, 0, rounds);
  }
  if (acc == 0x9E3779B9u) sink[0] = acc;   // keeps the loads; practically never taken
}

__global__ __launch_bounds__(256) void read_probe(const unsigned char *p, u32 bytes, u32 *sink, int iters) {
  const __amdgpu_buffer_rsrc_t r = rsrc(p, bytes);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const u32 gw = blockIdx.x * 4 + wave, nw = gridDim.x * 4;
  uint4 a[4];
  u32 acc = 0;
#pragma unroll
  for (int d = 0; d < 4; ++d) a[d] = ld16(r, gw * 4096 + d * 1024 + lane * 16, 0, kNT);
  for (int it = 1; it <= iters; ++it) {
    const u32 nb = (it < iters ? (it * nw + gw) : gw) * 4096 + lane * 16;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      acc ^= a[d].x + a[d].y + a[d].z + a[d].w;
      a[d] = ld16(r, nb + d * 1024, 0, kNT);
    }
  }
#pragma unroll
  for (int d = 0; d < 4; ++d) acc ^= a[d].x;
  if (acc == 0x9E3779B9u) sink[0] = acc;
}

}  // namespace

// Returns 0, or -1 for arguments the grid does not fit (nothing is launched).
extern "C" int cwen_probe_gemv_grid(const void *w, size_t wbytes, const void *x, size_t xbytes, void *sink,
                                    int nstream, int rounds, int nwhole, int npieces, int prs, int xl,
                                    void *stream) {
  if (!w || !x || !sink || nstream <= 0 || nstream % 4 || rounds <= 0 || prs <= 0 || nwhole < 0 || npieces < 0)
    return -1;
  const int ppt = (rounds + prs - 1) / prs;
  if (npieces % ppt || (nwhole + npieces / ppt) * 4 != nstream) return -1;
  if (wbytes < (size_t)rounds * nstream * kTile || wbytes > 0x7fffffffu) return -1;
  if (xbytes < (size_t)rounds * kStage || xbytes > 0x7fffffffu || (xl != 0 && xl != 2)) return -1;
  const dim3 grid((unsigned)(nwhole + npieces));
  const hipStream_t st = (hipStream_t)stream;
  if (xl == 2)
    hipLaunchKernelGGL(gemv_grid_probe<2>, grid, dim3(256), 0, st, (const unsigned char *)w, (u32)wbytes,
                       (const unsigned char *)x, (u32)xbytes, (u32 *)sink, rounds, nstream, nwhole, npieces, prs);
  else
    hipLaunchKernelGGL(gemv_grid_probe<0>, grid, dim3(256), 0, st, (const unsigned char *)w, (u32)wbytes,
                       (const unsigned char *)x, (u32)xbytes, (u32 *)sink, rounds, nstream, nwhole, npieces, prs);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Reads iters * 512 workgroups * 4 waves * 4 KB bytes (returned in *read_bytes).
extern "C" int cwen_probe_read(const void *p, size_t bytes, void *sink, int iters, size_t *read_bytes,
                               void *stream) {
  const size_t per = (size_t)512 * 4 * 4096;
  if (!p || !sink || iters <= 0 || bytes < per * iters || bytes > 0x7fffffffu) return -1;
  hipLaunchKernelGGL(read_probe, dim3(512), dim3(256), 0, (hipStream_t)stream, (const unsigned char *)p, (u32)bytes,
                     (u32 *)sink, iters);
  if (read_bytes) *read_bytes = per * iters;
  return hipGetLastError() == hipSuccess ? 0 : -1;
}
