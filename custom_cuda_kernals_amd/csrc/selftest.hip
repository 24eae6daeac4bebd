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
//                           clamp(amax / FP8_MAX, 1e-12) with IEEE division;
//   cck_silu_table_selftest - both fills of the bf16 SiLU table against the
//                           arithmetic SiLU entry by entry, and the table
//                           lookup against the arithmetic path for all 2^16
//                           bf16 gates.
//   cck_sigmoid_selftest  - the fp32 SwiGLU's sigmoid (SLEEF's expf with
//                           its scaling as one ldexp, and a reciprocal in
//                           place of the division) against the
//                           operation-for-operation form, for every fp32
//                           bit pattern in [start, start + count).
#include "launch.hpp"
#include "silu.hpp"

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

// counters (unsigned long long[6]):
//   [0] fill_single entries that differ (bitwise) from CodecBF16::round(silu_one(g))
//   [1] fill_pairs entries that differ likewise
//   [2] lowest table index counted in [0] or [1] (init ~0)
//   [3] gates whose silu_vec<CodecBF16, true> (table of fill_pairs) differs
//       bitwise from silu_vec<CodecBF16, false>, over all 2^16 bf16 patterns in
//       two groupings into 8-gate vectors: ascending, and permuted by an odd
//       multiplier mod 2^16 (mixes in-range and out-of-range gates)
//   [4] vectors of [3] served by the table (all 8 gates in range)
//   [5] gates checked in [3] (2^17)
// One workgroup of 1024 threads.
__global__ __launch_bounds__(1024) void silu_table_selftest(unsigned long long* counters) {
  using T = SiluTableBF16;
  __shared__ __attribute__((aligned(16))) float tab[T::kEntries];
  unsigned long long bad[2] = {0, 0}, lo = ~0ull;
#pragma unroll
  for (int f = 0; f < 2; ++f) {
    if (f == 0) {
      T::fill_single(tab, threadIdx.x, 1024);
    } else {
      T::fill_pairs(tab, threadIdx.x, 1024);
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < T::kEntries; i += 1024) {
      const uint32_t key = i + 2 * T::kLo;
      const float g = bits_f32((((key & 1u) << 15) | (key >> 1)) << 16);
      const float want = CodecBF16::round(silu_one<CodecBF16>(g));
      if (f32_bits(tab[i]) != f32_bits(want)) {
        bad[f] += 1;
        lo = lo < i ? lo : i;
      }
    }
    __syncthreads();
  }
  constexpr uint32_t kVecs = 65536 / 8;
  unsigned long long diff = 0, hits = 0, checked = 0;
  for (uint32_t v = threadIdx.x; v < 2 * kVecs; v += 1024) {
    const bool permuted = v >= kVecs;
    const uint32_t first = (v % kVecs) * 8;
    u32x4 w;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t p0 = first + 2 * j, p1 = p0 + 1;
      if (permuted) {
        p0 = (p0 * 40503u) & 0xffffu;
        p1 = (p1 * 40503u) & 0xffffu;
      }
      w[j] = p0 | (p1 << 16);
    }
    float a[8], b[8], t[8];
    silu_vec<CodecBF16, true>(w, tab, a);
    silu_vec<CodecBF16, false>(w, nullptr, b);
    hits += T::lookup8(w, tab, t) ? 1 : 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) diff += f32_bits(a[i]) != f32_bits(b[i]);
    checked += 8;
  }
  if (bad[0]) atomicAdd(&counters[0], bad[0]);
  if (bad[1]) atomicAdd(&counters[1], bad[1]);
  if (lo != ~0ull) atomicMin(&counters[2], lo);
  if (diff) atomicAdd(&counters[3], diff);
  if (hits) atomicAdd(&counters[4], hits);
  if (checked) atomicAdd(&counters[5], checked);
}

// counters (unsigned long long[7]), g = every fp32 pattern in [start, start + count):
//   [0] SleefExpf::eval_ldexp(g) != SleefExpf::eval(g)       (bitwise, NaN == NaN)
//   [1] sigmoid_sleef(g) != sigmoid_sleef_ref(g)             (bitwise, NaN == NaN)
//   [2] recip_refined(g) != 1 / g, for g in [1, kRecipRnLimit)
//   [3] patterns checked in [2]
//   [4..6] lowest mismatching pattern of [0..2] (init to ~0)
__global__ __launch_bounds__(256) void sigmoid_selftest(uint64_t start, uint64_t count,
                                                        unsigned long long* counters) {
  unsigned long long n[3] = {0, 0, 0}, lo[3] = {~0ull, ~0ull, ~0ull}, checked = 0;
  const uint64_t stride = (uint64_t)gridDim.x * 256;
  auto differ = [](float a, float b) {
    return f32_bits(a) != f32_bits(b) && !(__builtin_isnan(a) && __builtin_isnan(b));
  };
  for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < count; i += stride) {
    const uint64_t bits = start + i;
    const float g = bits_f32((uint32_t)bits);
    const bool bad[3] = {differ(SleefExpf::eval_ldexp(g), SleefExpf::eval(g)),
                         differ(sigmoid_sleef(g), sigmoid_sleef_ref(g)),
                         g >= 1.0f && g < kRecipRnLimit && differ(recip_refined(g), 1.0f / g)};
    checked += g >= 1.0f && g < kRecipRnLimit;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      if (bad[c]) {
        n[c] += 1;
        lo[c] = lo[c] < bits ? lo[c] : bits;
      }
    }
  }
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    if (n[c]) atomicAdd(&counters[c], n[c]);
    if (lo[c] != ~0ull) atomicMin(&counters[4 + c], lo[c]);
  }
  if (checked) atomicAdd(&counters[3], checked);
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

extern "C" int32_t cck_silu_table_selftest(unsigned long long* counters, void* stream) {
  hipStream_t st = static_cast<hipStream_t>(stream);
  silu_table_selftest<<<1, 1024, 0, st>>>(counters);
  return launch_status();
}

extern "C" int32_t cck_sigmoid_selftest(uint64_t start, uint64_t count, unsigned long long* counters,
                                        void* stream) {
  if (count == 0) return (int32_t)hipSuccess;
  if (start > 0xffffffffull || count > (1ull << 32) - start) return (int32_t)hipErrorInvalidValue;
  hipStream_t st = static_cast<hipStream_t>(stream);
  sigmoid_selftest<<<flat_grid((int64_t)(count / 64), 256, 8192), 256, 0, st>>>(start, count, counters);
  return launch_status();
}
