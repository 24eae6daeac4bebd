// Device building blocks for the gfx950 (CDNA4, wave64) activation kernels:
//
//   * element codecs: one 16-byte global access <-> VEC floats for fp32,
//     fp16 and bf16 storage, with round-to-nearest-even stores
//     (v_cvt_pk_bf16_f32 for bf16);
//   * wave64 all-reduce through DPP (quad_perm, row_half_mirror, row_mirror,
//     row_bcast:15/31) and one readlane, and a one-barrier LDS stage for
//     multi-wave workgroups;
//   * correctly rounded division by a per-row scale at three VALU ops per
//     element, and the PyTorch-compatible slow path for non-finite cases;
//   * FP8 packing with gfx950's v_cvt_pk_fp8_f32 / v_cvt_pk_bf8_f32.
//
// The dtype tags mirror the reference ABI (csrc/includes/common.cuh:28-34,
// src/kernels/dtype.rs:5-25).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fp8_codec.hpp"

namespace cck {

enum : int32_t { kF32 = 0, kF16 = 1, kBF16 = 2, kF8E4M3 = 3, kF8E5M2 = 4 };

using u32x4 = uint32_t __attribute__((ext_vector_type(4)));
using u32x2 = uint32_t __attribute__((ext_vector_type(2)));
using f32x2 = float __attribute__((ext_vector_type(2)));
using f32x4 = float __attribute__((ext_vector_type(4)));
using bf16x2 = __bf16 __attribute__((ext_vector_type(2)));
using f16x2 = _Float16 __attribute__((ext_vector_type(2)));
using u16x2 = uint16_t __attribute__((ext_vector_type(2)));

constexpr float kMinScale = 1e-12f;  // baselines/fp8_quant.py:59 (_EPS), as float32

// ---------------------------------------------------------------------------
// Element codecs. A "vector" is one 16-byte global access.
// ---------------------------------------------------------------------------

__device__ inline uint32_t pack2_bf16(float lo, float hi) {
  bf16x2 h = __builtin_convertvector((f32x2){lo, hi}, bf16x2);
  return __builtin_bit_cast(uint32_t, h);
}
// The fp32 value v itself, opaque to the optimiser. Before an fp32 -> fp16
// conversion this keeps the fp32 rounding of the expression that produced v:
// otherwise the compiler may fold a preceding fp32 multiply into
// v_fma_mixlo_f16, which rounds the exact product once, straight to fp16,
// where the eager oracle rounds it to fp32 first (the two differ at rare
// double-rounding ties). No instruction is emitted.
__device__ inline float keep_f32(float v) {
  asm("" : "+v"(v));
  return v;
}

__device__ inline uint32_t pack2_f16(float lo, float hi) {
  f16x2 h = __builtin_convertvector((f32x2){keep_f32(lo), keep_f32(hi)}, f16x2);
  return __builtin_bit_cast(uint32_t, h);
}
__device__ inline float bf16_lo(uint32_t w) { return bits_f32(w << 16); }
__device__ inline float bf16_hi(uint32_t w) { return bits_f32(w & 0xffff0000u); }
__device__ inline float f16_lo(uint32_t w) { return (float)__builtin_bit_cast(f16x2, w).x; }
__device__ inline float f16_hi(uint32_t w) { return (float)__builtin_bit_cast(f16x2, w).y; }

// Per-lane max of two packed u16 pairs (v_pk_max_u16).
__device__ inline uint32_t pk_max_u16(uint32_t a, uint32_t b) {
  u16x2 r = __builtin_elementwise_max(__builtin_bit_cast(u16x2, a), __builtin_bit_cast(u16x2, b));
  return __builtin_bit_cast(uint32_t, r);
}

struct CodecF32 {
  static constexpr int kTag = kF32;
  static constexpr int VEC = 4;
  static constexpr int kBytes = 4;
  __device__ static void unpack(const u32x4& w, float (&f)[VEC]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = bits_f32(w[i]);
  }
  __device__ static u32x4 pack(const float (&f)[VEC]) {
    return (u32x4){f32_bits(f[0]), f32_bits(f[1]), f32_bits(f[2]), f32_bits(f[3])};
  }
  // Round-trip through storage precision (identity for fp32).
  __device__ static float round(float v) { return v; }
  __device__ static void round2(float& a, float& b) {}
  __device__ static float load1(const void* p, int64_t i) { return static_cast<const float*>(p)[i]; }
  __device__ static void store1(void* p, int64_t i, float v) { static_cast<float*>(p)[i] = v; }
  // |x| as order-preserving bits (NaN > inf > finite), accumulated with max.
  __device__ static uint32_t absmax_vec(const u32x4& w, uint32_t acc) {
#pragma unroll
    for (int i = 0; i < 4; ++i) acc = max(acc, w[i] & 0x7fffffffu);
    return acc;
  }
  __device__ static uint32_t absmax1(const void* p, int64_t i, uint32_t acc) {
    return max(acc, f32_bits(load1(p, i)) & 0x7fffffffu);
  }
  __device__ static float absmax_to_float(uint32_t acc) { return bits_f32(acc); }
};

struct CodecBF16 {
  static constexpr int kTag = kBF16;
  static constexpr int VEC = 8;
  static constexpr int kBytes = 2;
  __device__ static void unpack(const u32x4& w, float (&f)[VEC]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = bf16_lo(w[i]);
      f[2 * i + 1] = bf16_hi(w[i]);
    }
  }
  __device__ static u32x4 pack(const float (&f)[VEC]) {
    return (u32x4){pack2_bf16(f[0], f[1]), pack2_bf16(f[2], f[3]), pack2_bf16(f[4], f[5]),
                   pack2_bf16(f[6], f[7])};
  }
  // RN to bf16, returned as the fp32 value: v_cvt_pk_bf16_f32 with a zero low
  // half yields the widened value directly (one instruction).
  __device__ static float round(float v) { return bits_f32(pack2_bf16(0.0f, v)); }
  __device__ static void round2(float& a, float& b) {
    a = round(a);
    b = round(b);
  }
  __device__ static float load1(const void* p, int64_t i) {
    return bits_f32((uint32_t) static_cast<const uint16_t*>(p)[i] << 16);
  }
  __device__ static void store1(void* p, int64_t i, float v) {
    static_cast<uint16_t*>(p)[i] = (uint16_t)(pack2_bf16(v, 0.0f) & 0xffffu);
  }
  // Packed accumulator: two u16 lanes of |bf16| bits, folded at the end.
  __device__ static uint32_t absmax_vec(const u32x4& w, uint32_t acc) {
#pragma unroll
    for (int i = 0; i < 4; ++i) acc = pk_max_u16(acc, w[i] & 0x7fff7fffu);
    return acc;
  }
  __device__ static uint32_t absmax1(const void* p, int64_t i, uint32_t acc) {
    return pk_max_u16(acc, (uint32_t) static_cast<const uint16_t*>(p)[i] & 0x7fffu);
  }
  __device__ static float absmax_to_float(uint32_t acc) {
    return bits_f32(max(acc & 0xffffu, acc >> 16) << 16);
  }
};

struct CodecF16 {
  static constexpr int kTag = kF16;
  static constexpr int VEC = 8;
  static constexpr int kBytes = 2;
  __device__ static void unpack(const u32x4& w, float (&f)[VEC]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = f16_lo(w[i]);
      f[2 * i + 1] = f16_hi(w[i]);
    }
  }
  __device__ static u32x4 pack(const float (&f)[VEC]) {
    return (u32x4){pack2_f16(f[0], f[1]), pack2_f16(f[2], f[3]), pack2_f16(f[4], f[5]),
                   pack2_f16(f[6], f[7])};
  }
  __device__ static float round(float v) { return (float)(_Float16)keep_f32(v); }
  __device__ static void round2(float& a, float& b) {
    const uint32_t w = pack2_f16(a, b);
    a = f16_lo(w);
    b = f16_hi(w);
  }
  __device__ static float load1(const void* p, int64_t i) {
    return (float)static_cast<const _Float16*>(p)[i];
  }
  __device__ static void store1(void* p, int64_t i, float v) {
    static_cast<_Float16*>(p)[i] = (_Float16)keep_f32(v);
  }
  __device__ static uint32_t absmax_vec(const u32x4& w, uint32_t acc) {
#pragma unroll
    for (int i = 0; i < 4; ++i) acc = pk_max_u16(acc, w[i] & 0x7fff7fffu);
    return acc;
  }
  __device__ static uint32_t absmax1(const void* p, int64_t i, uint32_t acc) {
    return pk_max_u16(acc, (uint32_t) static_cast<const uint16_t*>(p)[i] & 0x7fffu);
  }
  __device__ static float absmax_to_float(uint32_t acc) {
    const uint32_t h = max(acc & 0xffffu, acc >> 16);
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
  }
};

// ---------------------------------------------------------------------------
// wave64 / workgroup all-reduce.
// ---------------------------------------------------------------------------

constexpr int kDppQuadXor1 = 0xB1;   // quad_perm:[1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;   // quad_perm:[2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;
constexpr int kDppRowBcast15 = 0x142;  // lane 15 of each row to the next row
constexpr int kDppRowBcast31 = 0x143;  // lane 31 to rows 2 and 3

struct MaxU32 {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return max(a, b); }
};
struct MaxPkU16 {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return pk_max_u16(a, b); }
};
// IEEE-754-2019 maximum on float bits: NaN-propagating (v_maximum3_f32).
struct MaxF32 {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const {
    return f32_bits(__builtin_elementwise_maximum(bits_f32(a), bits_f32(b)));
  }
};
// acc = maximum(acc, |a|, |b|), NaN-propagating.
__device__ inline float absmax2(float acc, float a, float b) {
  return __builtin_elementwise_maximum(acc, __builtin_elementwise_maximum(__builtin_fabsf(a), __builtin_fabsf(b)));
}
struct AddF32 {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const {
    return f32_bits(bits_f32(a) + bits_f32(b));
  }
};

template <int CTRL>
__device__ inline uint32_t dpp(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

// DPP on the rows in ROW_MASK; the other rows keep `old`.
template <int CTRL, int ROW_MASK>
__device__ inline uint32_t dpp_rows(uint32_t old, uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROW_MASK, 0xF, false);
}

// Every lane of the wave must be active. Returns the wave-uniform result.
// Four butterfly steps give every lane its row's result; row_bcast:15 then
// combines rows 0 into 1 and 2 into 3, and row_bcast:31 row 1 into row 3, so
// lane 63 holds op over the wave: (row3 op row2) op (row1 op row0). For the
// commutative ops used here that is the same value, bit for bit, as
// (row0 op row1) op (row2 op row3). All in VALU: no LDS-path ds_swizzle and
// its wait. The MoE router (two reductions per top-k round) measured 5.0-5.1
// vs 5.3-5.4 us for 2048 tokens x 160 experts, top 6, on MI355X; the row
// kernels, one reduction per row, did not change beyond noise.
template <class Op>
__device__ inline uint32_t wave_allreduce(uint32_t v, Op op) {
  v = op(v, dpp<kDppQuadXor1>(v));
  v = op(v, dpp<kDppQuadXor2>(v));
  v = op(v, dpp<kDppRowHalfMirror>(v));
  v = op(v, dpp<kDppRowMirror>(v));
  v = op(v, dpp_rows<kDppRowBcast15, 0xA>(v, v));
  v = op(v, dpp_rows<kDppRowBcast31, 0xC>(v, v));
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Workgroup all-reduce over NW waves (1-D workgroup of NW*64 threads).
// `lds` holds 2*NW words; `parity` alternates between consecutive calls so a
// wave that runs ahead into the next call never overwrites a slot that a
// slower wave is still reading (one barrier per call).
template <int NW, class Op>
__device__ inline uint32_t block_allreduce(uint32_t v, Op op, uint32_t* lds, int parity) {
  v = wave_allreduce(v, op);
  if constexpr (NW == 1) {
    return v;
  } else {
    uint32_t* slot = lds + parity * NW;
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) slot[w] = v;
    __syncthreads();
    uint32_t r = slot[0];
#pragma unroll
    for (int i = 1; i < NW; ++i) r = op(r, slot[i]);
    return r;
  }
}

// ---------------------------------------------------------------------------
// Division by a scale, bit-identical to IEEE fp32 x / s.
// ---------------------------------------------------------------------------

// Markstein's correction: with r = RN(1/s) and q0 = RN(x*r), the remainder
// e = x - q0*s is exact in one fma and RN(q0 + e*r) is the correctly rounded
// quotient (valid for normal s, r and quotients; the exhaustive checks cover
// the domains used here). The negated form makes signed zeros come out as
// IEEE division's: x = -0 -> -0.
__device__ inline float neg_div_by_scale(float x, float s, float r) {
  const float q0 = x * r;
  const float e = __builtin_fmaf(-q0, s, x);
  return __builtin_fmaf(-e, r, -q0);  // -(x / s)
}

__device__ inline float div_by_scale(float x, float s, float r) { return -neg_div_by_scale(x, s, r); }

// x / s with the NaN results of the x86 SSE/AVX division the CPU oracle (and
// the reference's eager path) runs on: a NaN operand is returned quieted,
// x first; invalid operations (0/0, inf/inf) give the "indefinite" -NaN.
__device__ inline float div_x86(float x, float s) {
  const uint32_t xb = f32_bits(x), sb = f32_bits(s);
  if ((xb & 0x7fffffffu) > 0x7f800000u) return bits_f32(xb | 0x00400000u);
  if ((sb & 0x7fffffffu) > 0x7f800000u) return bits_f32(sb | 0x00400000u);
  const bool x_inf = (xb & 0x7fffffffu) == 0x7f800000u, s_inf = (sb & 0x7fffffffu) == 0x7f800000u;
  const bool x_zero = (xb & 0x7fffffffu) == 0u, s_zero = (sb & 0x7fffffffu) == 0u;
  if ((x_inf && s_inf) || (x_zero && s_zero)) return bits_f32(0xffc00000u);
  return x / s;
}

// ---------------------------------------------------------------------------
// FP8 formats.
// ---------------------------------------------------------------------------

template <int FMT>
struct Fp8;

template <>
struct Fp8<kF8E4M3> {
  static constexpr float kMax = 448.0f;  // torch.finfo(torch.float8_e4m3fn).max
  // Rows / tiles whose quotients satisfy |x| * (1/s) <= kFastLimit use the
  // three-op division and v_cvt_pk_fp8_f32. Both were checked exhaustively on
  // gfx950 over this range (the conversion for every finite fp32, including
  // the NaN-for-overflow rounding above 464; the division for every finite
  // bf16 x against a large scale set), so it spans the dynamic-scale case
  // (|q| <= 448 * (1 + 2^-23)) with margin.
  static constexpr float kFastLimit = 65536.0f;
  __device__ static uint32_t cvt4(float a, float b, float c, float d) {
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  }
  // Codes of -a, -b, -c, -d (see cvt4_neg below).
  __device__ static uint32_t cvt4_of_neg(float a, float b, float c, float d) {
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, __builtin_bit_cast(int, a), false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
    return (uint32_t)w ^ 0x80808080u;
  }
  __host__ __device__ static uint32_t encode(float v) { return encode_e4m3fn(v); }
};

template <>
struct Fp8<kF8E5M2> {
  static constexpr float kMax = 57344.0f;  // torch.finfo(torch.float8_e5m2).max
  static constexpr float kFastLimit = 65536.0f;  // as above (infinity above 61440)
  __device__ static uint32_t cvt4(float a, float b, float c, float d) {
    int w = __builtin_amdgcn_cvt_pk_bf8_f32(a, b, 0, false);
    return (uint32_t)__builtin_amdgcn_cvt_pk_bf8_f32(c, d, w, true);
  }
  __device__ static uint32_t cvt4_of_neg(float a, float b, float c, float d) {
    int w = __builtin_amdgcn_cvt_pk_bf8_f32(a, b, __builtin_bit_cast(int, a), false);
    w = __builtin_amdgcn_cvt_pk_bf8_f32(c, d, w, true);
    return (uint32_t)w ^ 0x80808080u;
  }
  __host__ __device__ static uint32_t encode(float v) { return encode_e5m2(v); }
};

// Dynamic scale from an amax: clamp(amax / FP8_MAX, min=1e-12) with NaN
// propagating through the clamp as torch.clamp does (baselines/fp8_quant.py:169,175).
// FP8_MAX = 7 * 2^k (448 = 7 * 2^6, 57344 = 7 * 2^13), so amax / FP8_MAX =
// (amax * 2^-k) / 7 with an exact first step, and the division by 7 is the
// fma-corrected product with RN(1/7), correctly rounded for normal quotients
// (checked exhaustively against IEEE division on the device). Quotients too
// small to be normal are clamped to 1e-12 anyway; +inf is patched.
template <int FMT>
__device__ inline float scale_from_amax(float amax) {
  constexpr float kPow2 = Fp8<FMT>::kMax / 7.0f;
  constexpr float kR7 = 1.0f / 7.0f;
  const float a = amax * (1.0f / kPow2);
  const float q0 = a * kR7;
  const float e = __builtin_fmaf(-q0, 7.0f, a);
  float s = __builtin_fmaf(e, kR7, q0);
  s = (amax == __builtin_inff()) ? amax : s;
  return (s < kMinScale) ? kMinScale : s;
}

// Reference form of the same scale (IEEE division), for the device self-test.
template <int FMT>
__device__ inline float scale_from_amax_ieee(float amax) {
  const float s = amax / Fp8<FMT>::kMax;
  return (s < kMinScale) ? kMinScale : s;
}

// A row/tile/tensor may use the fast conversion when the scale is a normal
// positive number with a normal reciprocal and every |x| / s stays within the
// verified range of the hardware conversion.
template <int FMT>
__device__ inline bool fast_path_ok(float s, float r, float amax) {
  const bool s_ok = s >= 1.1754944e-38f && s <= 1.0e30f;  // also false for NaN
  const bool r_ok = r >= 1.1754944e-38f && r <= 1.0e30f;
  return s_ok && r_ok && (amax * r <= Fp8<FMT>::kFastLimit);
}

// Quantise N values (N % 4 == 0) to N fp8 bytes packed little-endian into
// N/4 words. The quotients are formed negated (saving the negation per value)
// and converted with cvt4_of_neg: an fp8 code's top bit is its sign and the
// hardware conversion is sign-symmetric for every non-NaN fp32 (it matches the
// sign-symmetric software encoders on every finite input, overflow codes
// included), so flipping the four sign bits of the packed word gives the
// codes of the true quotients. Inputs here are finite (fast_path_ok).
template <int FMT, int N>
__device__ inline void quant_fast(const float (&v)[N], float s, float r, uint32_t (&out)[N / 4]) {
#pragma unroll
  for (int i = 0; i < N / 4; ++i) {
    out[i] = Fp8<FMT>::cvt4_of_neg(neg_div_by_scale(v[4 * i], s, r), neg_div_by_scale(v[4 * i + 1], s, r),
                                   neg_div_by_scale(v[4 * i + 2], s, r), neg_div_by_scale(v[4 * i + 3], s, r));
  }
}

template <int FMT, int N>
__device__ inline void quant_exact(const float (&v)[N], float s, uint32_t (&out)[N / 4]) {
#pragma unroll
  for (int i = 0; i < N / 4; ++i) {
    uint32_t w = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) w |= Fp8<FMT>::encode(div_x86(v[4 * i + j], s)) << (8 * j);
    out[i] = w;
  }
}

__device__ inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Streaming global accesses (data touched once per launch). Nontemporal by
// default; CCK_STREAM_NT_LOAD / CCK_STREAM_NT_STORE = 0 select cached accesses.
#ifndef CCK_STREAM_NT_LOAD
#define CCK_STREAM_NT_LOAD 1
#endif
#ifndef CCK_STREAM_NT_STORE
#define CCK_STREAM_NT_STORE 1
#endif

// Cache-policy immediate of gfx950 vector memory instructions (the aux
// operand of the buffer builtins): SC0 = 1, NT = 2, SC1 = 16. On stores,
// SC1 / SC0 select the scope the write is made visible at (write-through
// beyond the CU's caches) and NT marks it as streaming.
constexpr int kPolSC0 = 1, kPolNT = 2, kPolSC1 = 16;
constexpr int kBufLoadPolicy = CCK_STREAM_NT_LOAD ? kPolNT : 0;
constexpr int kBufStorePolicy = CCK_STREAM_NT_STORE ? kPolNT : 0;

template <class T>
__device__ inline T ld_stream(const T* p) {
  if constexpr (CCK_STREAM_NT_LOAD) {
    return __builtin_nontemporal_load(p);
  } else {
    return *p;
  }
}
template <class T>
__device__ inline void st_stream(T v, T* p) {
  if constexpr (CCK_STREAM_NT_STORE) {
    __builtin_nontemporal_store(v, p);
  } else {
    *p = v;
  }
}

// One row of a tensor, addressed by 32-bit byte offsets. RowBuf<true> is a
// raw buffer resource (base and size in SGPRs, no per-lane 64-bit address
// arithmetic, accesses past `bytes` read 0 / are dropped by the hardware range
// check); RowBuf<false> is a plain global pointer. Which one a row kernel uses
// was measured per kernel on MI355X. Rows are at most a few hundred KB here.
// SPOL is the cache policy of the row's stores (buffer resources only).
constexpr int kBufDword3 = 0x00020000;  // gfx9 family: DATA_FORMAT_32, no swizzle

template <bool RSRC, int SPOL = kBufStorePolicy>
struct RowBuf;

template <int SPOL>
struct RowBuf<true, SPOL> {
  __amdgpu_buffer_rsrc_t r;
  __device__ RowBuf(const void* base, uint32_t bytes)
      : r(__builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufDword3)) {}
  __device__ u32x4 ld16(uint32_t off) const {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kBufLoadPolicy));
  }
  __device__ void st16(const u32x4& v, uint32_t off) const {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, SPOL);
  }
  __device__ void st8(const u32x2& v, uint32_t off) const {
    __builtin_amdgcn_raw_buffer_store_b64(v, r, off, 0, SPOL);
  }
  __device__ void st4(uint32_t v, uint32_t off) const {
    __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, SPOL);
  }
};

// The same interface over global pointers (callers guard the row end).
template <int SPOL>
struct RowBuf<false, SPOL> {
  static_assert(SPOL == kBufStorePolicy, "global-pointer rows store with the streaming policy");
  char* p;
  __device__ RowBuf(const void* base, uint32_t) : p(static_cast<char*>(const_cast<void*>(base))) {}
  __device__ u32x4 ld16(uint32_t off) const { return ld_stream(reinterpret_cast<const u32x4*>(p + off)); }
  __device__ void st16(const u32x4& v, uint32_t off) const { st_stream(v, reinterpret_cast<u32x4*>(p + off)); }
  __device__ void st8(const u32x2& v, uint32_t off) const { st_stream(v, reinterpret_cast<u32x2*>(p + off)); }
  __device__ void st4(uint32_t v, uint32_t off) const { st_stream(v, reinterpret_cast<uint32_t*>(p + off)); }
};

}  // namespace cck
