// SiLU for the SwiGLU kernels and their device self-test, for gfx950.
//
// silu(g) = g * sigmoid(g), sigmoid = 1 / (1 + exp(-g)), in fp32 as the eager
// formula (baselines/swiglu.py:107-112).
//
// fp32 gates (no storage rounding after the SiLU to absorb differences)
// follow torch-CPU's float32 sigmoid exactly, as its vectorised loop
// computes it: 1 / (1 + exp(0 - g)) with SLEEF's single-precision expf of
// 1.0-ulp accuracy (the published xexpf algorithm: Cody-Waite reduction by
// ln 2 in two parts, a degree-5 polynomial by Horner's rule, all with fused
// multiply-adds, scaled by 2^q in two halves), an add and an IEEE division.
// The kernels evaluate the same bits with fewer operations: the scaling as
// one ldexp and the division as a Newton-refined reciprocal where that is
// correctly rounded (both checked for every fp32 gate by
// cck_sigmoid_selftest).
//
// bf16 / fp16 gates are rounded to their storage type after the SiLU, so
// there sigmoid is built for instruction count (the op is close to
// VALU-bound): exp(-g) = 2^th * (1 + c) with one v_exp_f32, and 1/(1+e) = one
// v_rcp_f32 plus a Newton step. For bf16 inputs, th = -g*HI is exact (8-bit g
// times a 16-bit HI), so only the tiny c = -g*LO*ln2 is rounded; fp16 splits
// the product with an fma. Gates outside the fast range (exp(-g) near
// overflow, sigmoid subnormal, the first-order correction no longer within an
// ulp, inf / NaN) use the IEEE expf / division path.
//
// Everything here is compiled with fp contraction off (the pragma below also
// holds for the rest of every file that includes this header).
#pragma once

#include <type_traits>

#include "cdna4.hpp"

#pragma clang fp contract(off)

namespace cck {

// log2(e) = HI + LO; HI has 16 significant bits so g * HI is exact for bf16 g.
template <class C>
struct SiluConsts {
  static constexpr bool kExactHi = false;
  static constexpr float kHi = 1.44269502162933349609375f;  // RN32(log2 e)
  static constexpr float kLo = 1.925963033500011e-08f;       // log2 e - kHi
  static constexpr float kFastAbs = 87.0f;                   // sigmoid stays normal
};
template <>
struct SiluConsts<CodecBF16> {
  static constexpr bool kExactHi = true;
  static constexpr float kHi = 1.44268798828125f;
  static constexpr float kLoLn2 = 4.888495368504664e-06f;  // (log2 e - kHi) * ln 2
  // First-order correction 1 + c is within an ulp for |c| < 1e-4 (|g| < 20).
  static constexpr float kFastAbs = 20.0f;
};

constexpr float kLn2 = 0.693147182464599609375f;

template <class C>
__device__ inline float exp_neg_fast(float g) {
  using K = SiluConsts<C>;
  if constexpr (K::kExactHi) {
    const float th = g * -K::kHi;  // exact
    const float c = g * -K::kLoLn2;
    const float p = __builtin_amdgcn_exp2f(th);
    return __builtin_fmaf(p, c, p);
  } else {
    const float th = g * -K::kHi;
    const float rem = __builtin_fmaf(g, -K::kHi, -th);  // exact remainder of the product
    const float tl = __builtin_fmaf(g, -K::kLo, rem);
    const float p = __builtin_amdgcn_exp2f(th);
    return __builtin_fmaf(p, tl * kLn2, p);
  }
}

// 1 / d to within an ulp: v_rcp_f32 then one Newton step with a fused remainder.
__device__ inline float recip_refined(float d) {
  const float r0 = __builtin_amdgcn_rcpf(d);
  const float e = __builtin_fmaf(-d, r0, 1.0f);
  return __builtin_fmaf(e, r0, r0);
}

__device__ inline float silu_exact(float g) { return g * (1.0f / (1.0f + __builtin_expf(-g))); }

// SLEEF's xexpf (u10), operation for operation: q = rint(d / ln 2) as the
// rounded product with RN(1 / ln 2), d - q ln 2 with ln 2 split in two
// (L2U exact in a float with 16 trailing zero bits, L2L the rest), the
// polynomial, 1 + (s^2 p(s) + s), and the scaling by 2^(q >> 1) 2^(q - (q >> 1))
// (two steps, so no intermediate overflows); 0 below -104, +inf above 100.
struct SleefExpf {
  static constexpr float kRLn2 = 1.442695040888963407359924681001892137426645954152985934135449406931f;
  static constexpr float kL2U = 0.693145751953125f;
  static constexpr float kL2L = 1.428606765330187045e-06f;
  static constexpr float kC0 = 0.000198527617612853646278381f, kC1 = 0.00139304355252534151077271f,
                         kC2 = 0.00833336077630519866943359f, kC3 = 0.0416664853692054748535156f,
                         kC4 = 0.166666671633720397949219f, kC5 = 0.5f;
  __device__ static float pow2i(int e) { return bits_f32((uint32_t)(e + 127) << 23); }
  __device__ static float eval(float d) {
    // |d / ln 2| <= 151 wherever the result is not replaced below; the clamp
    // keeps the conversion to int defined elsewhere (NaN d still gives NaN s).
    const int q = (int)__builtin_rintf(__builtin_fminf(__builtin_fmaxf(d * kRLn2, -200.0f), 200.0f));
    const float qf = (float)q;
    float s = __builtin_fmaf(qf, -kL2U, d);
    s = __builtin_fmaf(qf, -kL2L, s);
    float u = kC0;
    u = __builtin_fmaf(u, s, kC1);
    u = __builtin_fmaf(u, s, kC2);
    u = __builtin_fmaf(u, s, kC3);
    u = __builtin_fmaf(u, s, kC4);
    u = __builtin_fmaf(u, s, kC5);
    u = 1.0f + __builtin_fmaf(s * s, u, s);
    const int h = q >> 1;
    u = u * pow2i(h);
    u = u * pow2i(q - h);
    u = d < -104.0f ? 0.0f : u;
    return 100.0f < d ? __builtin_inff() : u;
  }
  // The same result with the scaling as one v_ldexp_f32. u * 2^(q >> 1) is
  // exact (u is in [0.7, 1.5] and |q| <= 200), so eval rounds u * 2^q once,
  // as ldexp does; cck_sigmoid_selftest compares the two for every float d.
  __device__ static float eval_ldexp(float d) {
    const float qf = __builtin_rintf(__builtin_fminf(__builtin_fmaxf(d * kRLn2, -200.0f), 200.0f));
    float s = __builtin_fmaf(qf, -kL2U, d);
    s = __builtin_fmaf(qf, -kL2L, s);
    float u = kC0;
    u = __builtin_fmaf(u, s, kC1);
    u = __builtin_fmaf(u, s, kC2);
    u = __builtin_fmaf(u, s, kC3);
    u = __builtin_fmaf(u, s, kC4);
    u = __builtin_fmaf(u, s, kC5);
    u = 1.0f + __builtin_fmaf(s * s, u, s);
    u = __builtin_amdgcn_ldexpf(u, (int)qf);
    u = d < -104.0f ? 0.0f : u;
    return 100.0f < d ? __builtin_inff() : u;
  }
};

// Below this, recip_refined(d) for d >= 1 is the correctly rounded 1 / d
// (cck_sigmoid_selftest compares it with IEEE division for every float in
// [1, 2^64)).
constexpr float kRecipRnLimit = 18446744073709551616.0f;  // 2^64

// torch-CPU's float32 vectorised sigmoid, 1 / (1 + xexpf(0 - g)), with the
// division as a correctly rounded reciprocal where that is checked (g above
// about -44.4) and IEEE division elsewhere; the lanes that need the division
// take it in a branch that a wave skips when none does.
__device__ inline float sigmoid_sleef(float g) {
  const float d = 1.0f + SleefExpf::eval_ldexp(0.0f - g);
  float r = recip_refined(d);
  if (!(d < kRecipRnLimit)) r = 1.0f / d;
  return r;
}

// The operation-for-operation form (two-step scaling, IEEE division), the
// reference of cck_sigmoid_selftest.
__device__ inline float sigmoid_sleef_ref(float g) { return 1.0f / (1.0f + SleefExpf::eval(0.0f - g)); }

// g * sigmoid(g) with torch-CPU's float32 vectorised sigmoid.
__device__ inline float silu_sleef(float g) { return g * sigmoid_sleef(g); }

template <class C>
constexpr bool kSleefSilu = std::is_same_v<C, CodecF32>;

template <class C>
__device__ inline float silu_fast(float g) {
  return g * recip_refined(1.0f + exp_neg_fast<C>(g));
}

// SiLU of one element: the fast form inside its range, the exact form
// elsewhere. Every path below computes exactly this per element, whatever
// the neighbouring elements are.
template <class C>
__device__ inline float silu_one(float g) {
  if constexpr (kSleefSilu<C>) {
    return silu_sleef(g);
  } else {
    return __builtin_fabsf(g) <= SiluConsts<C>::kFastAbs ? silu_fast<C>(g) : silu_exact(g);
  }
}

// ---------------------------------------------------------------------------
// bf16 SiLU table in LDS.
//
// A bf16 gate has only 2^16 values, so T(silu(g)) is a function of its 16
// bits. The common range 2^-14 <= |g| < 32 (4864 values) is tabulated per
// workgroup in LDS (19 KB of fp32, filled with silu_one at workgroup start),
// which replaces the two transcendental instructions and the Newton step per
// element by one ds_read_b32. Vectors with a gate outside the range (zeros,
// tiny or huge values, inf/NaN) fall back to silu_one, so results are
// bit-identical to the arithmetic path.
//
// Key of a bf16 pattern b with magnitude field m = b & 0x7fff and sign s:
// 2 * (m - kLo) + s, i.e. the 16-bit pattern rotated left by one minus
// 2 * kLo; two keys are formed per packed word with one v_pk_sub_u16.
// ---------------------------------------------------------------------------
struct SiluTableBF16 {
  static constexpr uint32_t kLo = 0x3880;                    // 2^-14
  static constexpr uint32_t kHi = 0x4200;                    // 32.0
  static constexpr uint32_t kEntries = 2 * (kHi - kLo);      // 4864

  // Rounded SiLU of every tabulated value. Two fills of identical contents:
  // each entry equals CodecBF16::round(silu_one(g)), which cck_silu_table_selftest
  // checks entry by entry on the device; which fill a kernel uses was measured
  // on MI355X.
  // * |g| < 2^-9: sigmoid(g) = 1/2 + g/4 + O(g^3), so g*sigmoid(g) = (g/2)(1 + d)
  //   with |d| < 2^-10, inside half a bf16 ulp of the exactly representable g/2:
  //   those entries are g/2 without evaluating the SiLU (a wave-uniform branch).
  // * g > kFastAbs: silu(g) = g exactly (exp(-g) < 2^-25, so 1 + exp(-g) rounds
  //   to 1 in silu_exact).
  //
  // fill_single: one entry per thread and step, silu_one otherwise.
  static constexpr uint32_t kTinyKeys = 2 * (0x3b00 - kLo);  // |g| < 2^-9
  __device__ static void fill_single(float* tab, int tid, int nthreads) {
    for (uint32_t i = tid; i < kEntries; i += nthreads) {
      const uint32_t key = i + 2 * kLo;
      const float g = bits_f32((((key & 1u) << 15) | (key >> 1)) << 16);
      float v;
      if (i < kTinyKeys) {
        v = g * 0.5f;
      } else if (g > SiluConsts<CodecBF16>::kFastAbs) {
        v = g;
      } else {
        v = CodecBF16::round(silu_one<CodecBF16>(g));
      }
      tab[i] = v;
    }
  }

  // fill_pairs: the (+a, -a) pair of adjacent keys 2p, 2p + 1 (magnitude field
  // kLo + p) per thread and step. For a <= kFastAbs, e = exp(-a) and
  // r = 1/(1+e) serve both signs, since sigmoid(-a) = e * r:
  // silu(+a) = a*r, silu(-a) = -a*(e*r); rounded to bf16 this equals silu_one
  // on both signs for every bf16 magnitude in range (cck_silu_table_selftest),
  // at one exp and one reciprocal per pair instead of per entry.
  static constexpr uint32_t kPairs = kHi - kLo;
  static constexpr uint32_t kTinyPairs = 0x3b00 - kLo;  // a < 2^-9
  __device__ static void fill_pairs(float* tab, int tid, int nthreads) {
    using K = SiluConsts<CodecBF16>;
    for (uint32_t p = tid; p < kPairs; p += nthreads) {
      const float a = bits_f32((kLo + p) << 16);
      float pos, neg;
      if (p < kTinyPairs) {
        pos = a * 0.5f;
        neg = -a * 0.5f;
      } else if (a <= K::kFastAbs) {
        const float e = exp_neg_fast<CodecBF16>(a);
        const float r = recip_refined(1.0f + e);
        pos = CodecBF16::round(a * r);
        neg = CodecBF16::round(-a * (e * r));
      } else {
        pos = a;
        neg = CodecBF16::round(silu_one<CodecBF16>(-a));
      }
      *reinterpret_cast<f32x2*>(tab + 2 * p) = (f32x2){pos, neg};
    }
  }

  __device__ static uint32_t keys2(uint32_t w) {
    const uint32_t rot = ((w << 1) & 0xfffefffeu) | ((w >> 15) & 0x00010001u);
    const u16x2 k = __builtin_bit_cast(u16x2, rot) - (u16x2){(uint16_t)(2 * kLo), (uint16_t)(2 * kLo)};
    return __builtin_bit_cast(uint32_t, k);
  }

  // a[i] <- T(silu(g[i])) for the 8 gates of w; false (a untouched) when any
  // gate is outside the table.
  __device__ static bool lookup8(const u32x4& w, const float* tab, float (&a)[8]) {
    uint32_t key[4];
    uint32_t mx = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      key[j] = keys2(w[j]);
      mx = pk_max_u16(mx, key[j]);
    }
    if (max(mx & 0xffffu, mx >> 16) >= kEntries) return false;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      a[2 * j] = tab[key[j] & 0xffffu];
      a[2 * j + 1] = tab[key[j] >> 16];
    }
    return true;
  }
};

// T(silu(g[i])) for one 16-byte vector of gates, from the table when given.
template <class C, bool TAB>
__device__ inline void silu_vec(const u32x4& gw, const float* tab, float (&a)[C::VEC]) {
  if constexpr (TAB) {
    if (SiluTableBF16::lookup8(gw, tab, a)) return;
  }
  C::unpack(gw, a);
  if constexpr (kSleefSilu<C>) {
    // sigmoid_sleef per element, with one branch for the vector: the lanes
    // where any 1 + e is at or above the reciprocal's checked range redo
    // the four divisions in IEEE form (the same results where both apply).
    float d[C::VEC], r[C::VEC];
    bool wide = false;
#pragma unroll
    for (int i = 0; i < C::VEC; ++i) {
      d[i] = 1.0f + SleefExpf::eval_ldexp(0.0f - a[i]);
      r[i] = recip_refined(d[i]);
      wide |= !(d[i] < kRecipRnLimit);
    }
    if (wide) {
#pragma unroll
      for (int i = 0; i < C::VEC; ++i) r[i] = 1.0f / d[i];
    }
#pragma unroll
    for (int i = 0; i < C::VEC; ++i) a[i] = a[i] * r[i];
    return;
  }
  float mx = 0.0f;
#pragma unroll
  for (int i = 0; i < C::VEC; i += 2) mx = absmax2(mx, a[i], a[i + 1]);
  if (mx <= SiluConsts<C>::kFastAbs) {
#pragma unroll
    for (int i = 0; i < C::VEC; ++i) a[i] = silu_fast<C>(a[i]);
  } else {
#pragma unroll
    for (int i = 0; i < C::VEC; ++i) a[i] = silu_one<C>(a[i]);
  }
#pragma unroll
  for (int i = 0; i < C::VEC; i += 2) C::round2(a[i], a[i + 1]);
}

}  // namespace cck
