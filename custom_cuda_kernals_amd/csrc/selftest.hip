// Diagnostic entry points (no counterpart in the reference): checks of the
// two arithmetic shortcuts the FP8 kernels rely on, run on the device itself
// over exhaustive or caller-chosen input sets, with mismatch counters.
//
//   cck_fp8_cvt_selftest  - v_cvt_pk_fp8/bf8_f32 (used on the fast path)
//                           against the exact software encoder for every
//                           fp32 bit pattern in [start, start + count);
//   cck_div_selftest      - div_by_scale (three-op division) against IEEE
//                           division x / s for caller-given x and s sets;
//   cck_scale_selftest    - scale_from_amax (fma-corrected / 7) against
//                           clamp(amax / FP8_MAX, 1e-12) with IEEE division.
#include "launch.hpp"

namespace cck {
namespace {

// counters (unsigned long long[8]):
//   [0] mismatches with finite |v| <= kFastLimit   (the fast-path domain)
//   [1] mismatches with finite |v| >  kFastLimit
//   [2] mismatches with v = +-inf
//   [3] mismatches with v = NaN
//   [4..7] lowest mismatching bit pattern of classes 0..3 (init to ~0)
template <int FMT>
__global__ __launch_bounds__(256) void cvt_selftest(uint64_t start, uint64_t count,
                                                    unsigned long long* counters) {
  unsigned long long n[4] = {0, 0, 0, 0};
  unsigned long long lo[4] = {~0ull, ~0ull, ~0ull, ~0ull};
  const uint64_t stride = (uint64_t)gridDim.x * 256;
  for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < count; i += stride) {
    const uint32_t bits = (uint32_t)(start + i);
    const float v = bits_f32(bits);
    const uint32_t hw = Fp8<FMT>::cvt4(v, 0.0f, 0.0f, 0.0f) & 0xffu;
    const uint32_t sw = Fp8<FMT>::encode(v);
    if (hw != sw) {
      const uint32_t a = bits & 0x7fffffffu;
      int cls;
      if (a > 0x7f800000u) cls = 3;
      else if (a == 0x7f800000u) cls = 2;
      else cls = (__builtin_fabsf(v) <= Fp8<FMT>::kFastLimit) ? 0 : 1;
      n[cls] += 1;
      lo[cls] = lo[cls] < bits ? lo[cls] : bits;
    }
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    if (n[c]) {
      atomicAdd(&counters[c], n[c]);
      atomicMin(&counters[4 + c], lo[c]);
    }
  }
}

// counters: [0] fp32 quotient mismatches (bitwise), [1] fp8 e4m3 code
// mismatches, [2] fp8 e5m2 code mismatches, [3] lowest flat index with a
// bitwise mismatch, [4] pairs checked. Only pairs inside the fast-path domain
// (finite normal s and 1/s, |x| / s <= 65536) are checked.
__global__ __launch_bounds__(256) void div_selftest(const float* __restrict__ xs, int64_t nx,
                                                    const float* __restrict__ ss, int64_t ns,
                                                    unsigned long long* counters) {
  unsigned long long n0 = 0, n1 = 0, n2 = 0, checked = 0, first = ~0ull;
  const int64_t total = nx * ns;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += stride) {
    const float x = xs[i % nx];
    const float s = ss[i / nx];
    const float r = 1.0f / s;
    if (!fast_path_ok<kF8E5M2>(s, r, 0.0f) || !(__builtin_fabsf(x) * r <= 65536.0f)) continue;
    checked += 1;
    const float fast = div_by_scale(x, s, r);
    const float exact = x / s;
    if (f32_bits(fast) != f32_bits(exact)) {
      n0 += 1;
      first = first < (unsigned long long)i ? first : (unsigned long long)i;
    }
    n1 += encode_e4m3fn(fast) != encode_e4m3fn(exact);
    n2 += encode_e5m2(fast) != encode_e5m2(exact);
  }
  if (n0) atomicAdd(&counters[0], n0);
  if (n1) atomicAdd(&counters[1], n1);
  if (n2) atomicAdd(&counters[2], n2);
  if (first != ~0ull) atomicMin(&counters[3], first);
  if (checked) atomicAdd(&counters[4], checked);
}

// counters: [0] scale mismatches (bitwise, NaN == NaN), [1] lowest mismatching
// amax bit pattern. amax = every non-negative fp32 pattern in [start, start+count).
template <int FMT>
__global__ __launch_bounds__(256) void scale_selftest(uint64_t start, uint64_t count,
                                                      unsigned long long* counters) {
  unsigned long long n = 0, lo = ~0ull;
  const uint64_t stride = (uint64_t)gridDim.x * 256;
  for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < count; i += stride) {
    const uint32_t bits = (uint32_t)(start + i) & 0x7fffffffu;
    const float amax = bits_f32(bits);
    const float a = scale_from_amax<FMT>(amax), b = scale_from_amax_ieee<FMT>(amax);
    const bool same = (f32_bits(a) == f32_bits(b)) || (a != a && b != b);
    if (!same) {
      n += 1;
      lo = lo < bits ? lo : bits;
    }
  }
  if (n) {
    atomicAdd(&counters[0], n);
    atomicMin(&counters[1], lo);
  }
}

}  // namespace
}  // namespace cck

using namespace cck;

extern "C" int32_t cck_scale_selftest(uint64_t start, uint64_t count, int32_t fp8_format,
                                      unsigned long long* counters, void* stream) {
  if (count == 0) return (int32_t)hipSuccess;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned g = flat_grid((int64_t)(count / 64), 256, 8192);
  return with_fp8(fp8_format, [&](auto f) {
    scale_selftest<decltype(f)::value><<<g, 256, 0, st>>>(start, count, counters);
    return launch_status();
  });
}

extern "C" int32_t cck_fp8_cvt_selftest(uint64_t start, uint64_t count, int32_t fp8_format,
                                        unsigned long long* counters, void* stream) {
  if (count == 0) return (int32_t)hipSuccess;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned g = flat_grid((int64_t)(count / 64), 256, 8192);
  return with_fp8(fp8_format, [&](auto f) {
    cvt_selftest<decltype(f)::value><<<g, 256, 0, st>>>(start, count, counters);
    return launch_status();
  });
}

extern "C" int32_t cck_div_selftest(const float* xs, int64_t nx, const float* ss, int64_t ns,
                                    unsigned long long* counters, void* stream) {
  if (nx <= 0 || ns <= 0) return (int32_t)hipSuccess;
  hipStream_t st = static_cast<hipStream_t>(stream);
  div_selftest<<<flat_grid(nx * ns / 16, 256, 8192), 256, 0, st>>>(xs, nx, ss, ns, counters);
  return launch_status();
}
