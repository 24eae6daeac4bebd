// HBM calibration streams for gfx950: the traffic patterns of the ops with no
// arithmetic. Timed exactly like the ops (bench.py's `ceilings`), they give the
// practical ceiling of each pattern on the machine at hand, which is what an
// op's fraction of the 8 TB/s peak should be read against. Diagnostics only:
// no op calls them.
//
// Patterns, on 16-byte vectors with nontemporal loads and stores (the ops'
// access width and cache policy); n_vec counts the vectors of one input
// stream:
//   0  copy:                   c[i] = a[i]
//   1  two reads, one write:   c[i] = a[i] ^ b[i]              (SwiGLU's traffic)
//   2  rows of 512 vectors (8 KB), one 512-thread workgroup per row, two reads
//      and two writes with a workgroup barrier between the stores:
//      c[i] = a[i] + b[i]; barrier; d[i] = a[i] ^ b[i] ^ (another wave's word)
//      (RMSNorm + residual's traffic and row structure)
//   3  read 16 bytes, write 8:  c64[i] = fold(a[i])             (per-token FP8's traffic)
//   4  rows of 1792 vectors (14336 bf16), one 1024-thread workgroup per row,
//      two 16-byte reads and one 8-byte write per vector, a barrier between
//      the loads and the stores        (SwiGLU + per-token FP8's traffic)
//   5  rows of 512 vectors, 256 threads x 2 vectors, two 16-byte reads, a
//      16-byte write, a barrier, an 8-byte write
//                                       (RMSNorm + residual + FP8's traffic)
#include "launch.hpp"

namespace cck {
namespace {

constexpr int kCalThreads = 256;
constexpr int kCalRowVecs = 512;
constexpr int kCalLongRowVecs = 1792;

__global__ __launch_bounds__(kCalThreads) void hbm_copy(const u32x4* __restrict__ a, u32x4* __restrict__ c,
                                                        int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * kCalThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kCalThreads)
    st_stream(ld_stream(a + i), c + i);
}

__global__ __launch_bounds__(kCalThreads) void hbm_2r1w(const u32x4* __restrict__ a, const u32x4* __restrict__ b,
                                                        u32x4* __restrict__ c, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * kCalThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kCalThreads)
    st_stream(ld_stream(a + i) ^ ld_stream(b + i), c + i);
}

__global__ __launch_bounds__(kCalRowVecs) void hbm_rows_2r2w(const u32x4* __restrict__ a,
                                                             const u32x4* __restrict__ b, u32x4* __restrict__ c,
                                                             u32x4* __restrict__ d, int64_t rows) {
  __shared__ uint32_t word[kCalRowVecs / 64];
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const int64_t i = row * kCalRowVecs + threadIdx.x;
    const u32x4 x = ld_stream(a + i), y = ld_stream(b + i);
    st_stream(x + y, c + i);
    if ((threadIdx.x & 63) == 0) word[threadIdx.x >> 6] = x.x;
    __syncthreads();
    st_stream(x ^ y ^ word[(threadIdx.x >> 6) ^ 1], d + i);
    __syncthreads();  // the next row rewrites word[]
  }
}

__global__ __launch_bounds__(kCalThreads) void hbm_r16w8(const u32x4* __restrict__ a, u32x2* __restrict__ c,
                                                         int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * kCalThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kCalThreads) {
    const u32x4 v = ld_stream(a + i);
    st_stream((u32x2){v.x ^ v.y, v.z ^ v.w}, c + i);
  }
}

__global__ __launch_bounds__(1024) void hbm_rows_2r_w8(const u32x4* __restrict__ a, const u32x4* __restrict__ b,
                                                      u32x2* __restrict__ c, int64_t rows) {
  __shared__ uint32_t word[16];
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const int64_t base = row * kCalLongRowVecs;
    u32x4 x[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int v = threadIdx.x + 1024 * k;
      x[k] = v < kCalLongRowVecs ? ld_stream(a + base + v) ^ ld_stream(b + base + v) : (u32x4){0u, 0u, 0u, 0u};
    }
    if ((threadIdx.x & 63) == 0) word[threadIdx.x >> 6] = x[0].x;
    __syncthreads();
    const uint32_t w = word[(threadIdx.x >> 6) ^ 1];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int v = threadIdx.x + 1024 * k;
      if (v < kCalLongRowVecs) st_stream((u32x2){x[k].x ^ w, x[k].z}, c + base + v);
    }
    __syncthreads();  // the next row rewrites word[]
  }
}

__global__ __launch_bounds__(256) void hbm_rows_2r_w16_w8(const u32x4* __restrict__ a, const u32x4* __restrict__ b,
                                                          u32x4* __restrict__ c, u32x2* __restrict__ d, int64_t rows) {
  __shared__ uint32_t word[4];
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const int64_t i0 = row * kCalRowVecs + threadIdx.x, i1 = i0 + 256;
    const u32x4 x0 = ld_stream(a + i0), y0 = ld_stream(b + i0), x1 = ld_stream(a + i1), y1 = ld_stream(b + i1);
    st_stream(x0 + y0, c + i0);
    st_stream(x1 + y1, c + i1);
    if ((threadIdx.x & 63) == 0) word[threadIdx.x >> 6] = x0.x;
    __syncthreads();
    const uint32_t w = word[(threadIdx.x >> 6) ^ 1];
    st_stream((u32x2){x0.x ^ w, y0.y}, d + i0);
    st_stream((u32x2){x1.x ^ w, y1.y}, d + i1);
    __syncthreads();  // the next row rewrites word[]
  }
}

}  // namespace
}  // namespace cck

using namespace cck;

extern "C" int32_t cck_hbm_stream(int32_t pattern, const void* a, const void* b, void* c, void* d, int64_t n_vec,
                                  void* stream) {
  if (n_vec <= 0) return (int32_t)hipSuccess;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned g = flat_grid(n_vec, kCalThreads, 1 << 20);
  switch (pattern) {
    case 0:
      hbm_copy<<<g, kCalThreads, 0, st>>>(static_cast<const u32x4*>(a), static_cast<u32x4*>(c), n_vec);
      break;
    case 1:
      hbm_2r1w<<<g, kCalThreads, 0, st>>>(static_cast<const u32x4*>(a), static_cast<const u32x4*>(b),
                                          static_cast<u32x4*>(c), n_vec);
      break;
    case 2:
      if (n_vec % kCalRowVecs != 0) return (int32_t)hipErrorInvalidValue;
      hbm_rows_2r2w<<<row_grid(n_vec / kCalRowVecs), kCalRowVecs, 0, st>>>(
          static_cast<const u32x4*>(a), static_cast<const u32x4*>(b), static_cast<u32x4*>(c),
          static_cast<u32x4*>(d), n_vec / kCalRowVecs);
      break;
    case 3:
      hbm_r16w8<<<g, kCalThreads, 0, st>>>(static_cast<const u32x4*>(a), static_cast<u32x2*>(c), n_vec);
      break;
    case 4:
      if (n_vec % kCalLongRowVecs != 0) return (int32_t)hipErrorInvalidValue;
      hbm_rows_2r_w8<<<row_grid(n_vec / kCalLongRowVecs), 1024, 0, st>>>(
          static_cast<const u32x4*>(a), static_cast<const u32x4*>(b), static_cast<u32x2*>(c), n_vec / kCalLongRowVecs);
      break;
    case 5:
      if (n_vec % kCalRowVecs != 0) return (int32_t)hipErrorInvalidValue;
      hbm_rows_2r_w16_w8<<<row_grid(n_vec / kCalRowVecs), 256, 0, st>>>(
          static_cast<const u32x4*>(a), static_cast<const u32x4*>(b), static_cast<u32x4*>(c),
          static_cast<u32x2*>(d), n_vec / kCalRowVecs);
      break;
    default:
      return (int32_t)hipErrorInvalidValue;
  }
  return launch_status();
}
