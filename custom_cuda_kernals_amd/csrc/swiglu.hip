// SwiGLU activation y = silu(gate) * up, optionally fused with FP8
// quantisation of y, for gfx950.
//
// Semantics follow the eager oracle's rounding points
// (baselines/swiglu.py:107-112):
//   silu = g * sigmoid(g)        with g = float(gate), sigmoid = 1 / (1 + exp(-g))
//   y    = T( T(silu) * float(up) )
// The FP8 variant quantises y (as stored in T) per row of the last dimension
// (dynamic, per token) or with a static scale and does not write y itself.
//
// Design: the plain op is a flat grid-stride stream of 16-byte vectors (two
// loads, one store per vector). The FP8 variant is row-resident: one
// workgroup per row keeps y in registers while it reduces the row amax, so
// gate/up are read once and only the codes and the scale are written.
//
// The op is close to VALU-bound on gfx950 (no packed fp32 here), so sigmoid is
// built for instruction count: exp(-g) = 2^th * (1 + c) with one v_exp_f32,
// and 1/(1+e) = one v_rcp_f32 plus a Newton step. For bf16 inputs, th = -g*HI
// is exact (8-bit g times a 16-bit HI), so only the tiny c = -g*LO*ln2 is
// rounded; other input types split the product with an fma. Vectors with a
// gate outside the fast range (exp(-g) near overflow, sigmoid subnormal, the
// first-order correction no longer within an ulp, inf / NaN) use the IEEE
// expf / division path.
#include "launch.hpp"

namespace cck {
namespace {

#pragma clang fp contract(off)

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

// In place: g[i] <- T(silu(g[i])) * u[i], i.e. y before its final rounding.
// The fast path needs every |g| <= kFastAbs (one v_maximum3_f32 per two
// elements, NaN-propagating, so NaN and +-inf take the exact path too).
template <class C>
__device__ inline void swiglu_math(float (&g)[C::VEC], const float (&u)[C::VEC]) {
  constexpr int VEC = C::VEC;
  float mx = 0.0f;
#pragma unroll
  for (int i = 0; i < VEC; i += 2) mx = absmax2(mx, g[i], g[i + 1]);
  if (mx <= SiluConsts<C>::kFastAbs) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) g[i] = g[i] * recip_refined(1.0f + exp_neg_fast<C>(g[i]));
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) g[i] = silu_exact(g[i]);
  }
#pragma unroll
  for (int i = 0; i < VEC; i += 2) C::round2(g[i], g[i + 1]);
#pragma unroll
  for (int i = 0; i < VEC; ++i) g[i] = g[i] * u[i];
}

template <class C>
__device__ inline u32x4 swiglu_vec(const u32x4& gw, const u32x4& uw) {
  float g[C::VEC], u[C::VEC];
  C::unpack(gw, g);
  C::unpack(uw, u);
  swiglu_math<C>(g, u);
  return C::pack(g);
}

template <class C, int UNROLL>
__global__ __launch_bounds__(256) void swiglu_flat(const u32x4* __restrict__ gate,
                                                   const u32x4* __restrict__ up,
                                                   u32x4* __restrict__ y, int64_t nvec) {
  const int64_t stride = (int64_t)gridDim.x * 256 * UNROLL;
  for (int64_t base = (int64_t)blockIdx.x * 256 * UNROLL + threadIdx.x; base < nvec; base += stride) {
    u32x4 g[UNROLL], u[UNROLL];
#pragma unroll
    for (int k = 0; k < UNROLL; ++k) {
      const int64_t v = base + k * 256;
      if (v < nvec) {
        g[k] = ld_stream(gate + v);
        u[k] = ld_stream(up + v);
      }
    }
#pragma unroll
    for (int k = 0; k < UNROLL; ++k) {
      const int64_t v = base + k * 256;
      if (v < nvec) st_stream(swiglu_vec<C>(g[k], u[k]), y + v);
    }
  }
}

template <class C>
__device__ inline float swiglu1(float g, float u) {
  const float a = C::round(__builtin_fabsf(g) <= SiluConsts<C>::kFastAbs
                               ? g * recip_refined(1.0f + exp_neg_fast<C>(g))
                               : silu_exact(g));
  return a * u;
}

template <class C>
__global__ __launch_bounds__(256) void swiglu_scalar(const void* __restrict__ gate,
                                                     const void* __restrict__ up,
                                                     void* __restrict__ y, int64_t begin, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = begin + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
    C::store1(y, i, swiglu1<C>(C::load1(gate, i), C::load1(up, i)));
  }
}

// Static-scale FP8 variant: no row reduction is needed, so it streams like
// swiglu_flat; each 16-byte vector takes the fast conversion when its own
// max |y| * (1/s) is inside the fast range, the exact path otherwise.
template <class C, int FMT, int UNROLL>
__global__ __launch_bounds__(256) void swiglu_fp8_static_flat(const u32x4* __restrict__ gate,
                                                             const u32x4* __restrict__ up,
                                                             uint8_t* __restrict__ yq, float s,
                                                             int64_t nvec) {
  constexpr int VEC = C::VEC;
  const float r = 1.0f / s;
  const bool scale_ok = fast_path_ok<FMT>(s, r, 0.0f);
  const int64_t stride = (int64_t)gridDim.x * 256 * UNROLL;
  for (int64_t base = (int64_t)blockIdx.x * 256 * UNROLL + threadIdx.x; base < nvec; base += stride) {
    u32x4 g[UNROLL], u[UNROLL];
#pragma unroll
    for (int k = 0; k < UNROLL; ++k) {
      const int64_t v = base + k * 256;
      if (v < nvec) {
        g[k] = ld_stream(gate + v);
        u[k] = ld_stream(up + v);
      }
    }
#pragma unroll
    for (int k = 0; k < UNROLL; ++k) {
      const int64_t v = base + k * 256;
      if (v < nvec) {
        float y[VEC], uf[VEC];
        C::unpack(g[k], y);
        C::unpack(u[k], uf);
        swiglu_math<C>(y, uf);
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < VEC; i += 2) {
          C::round2(y[i], y[i + 1]);
          amax = absmax2(amax, y[i], y[i + 1]);
        }
        uint32_t wq[VEC / 4];
        if (scale_ok && amax * r <= Fp8<FMT>::kFastLimit) {
          quant_fast<FMT, VEC>(y, s, r, wq);
        } else {
          quant_exact<FMT, VEC>(y, s, wq);
        }
        if constexpr (VEC == 8) {
          st_stream((u32x2){wq[0], wq[1]}, reinterpret_cast<u32x2*>(yq + v * 8));
        } else {
          st_stream(wq[0], reinterpret_cast<uint32_t*>(yq + v * 4));
        }
      }
    }
  }
}

template <class C, int FMT>
__global__ __launch_bounds__(256) void swiglu_fp8_static_scalar(const void* __restrict__ gate,
                                                               const void* __restrict__ up,
                                                               uint8_t* __restrict__ yq, float s,
                                                               int64_t begin, int64_t n) {
  const float r = 1.0f / s;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = begin + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
    const float yv = C::round(swiglu1<C>(C::load1(gate, i), C::load1(up, i)));
    const bool fast = fast_path_ok<FMT>(s, r, __builtin_fabsf(yv));
    const float qv = fast ? div_by_scale(yv, s, r) : div_x86(yv, s);
    yq[i] = (uint8_t)(fast ? (Fp8<FMT>::cvt4(qv, 0.0f, 0.0f, 0.0f) & 0xffu) : Fp8<FMT>::encode(qv));
  }
}

// FP8 variant, register-resident rows; y is kept as floats (already rounded
// to T) between the amax reduction and the quantisation. STATIC selects the
// static scale.
template <class C, int THREADS, int ITEMS, bool STATIC, int FMT>
__global__ __launch_bounds__(THREADS) void swiglu_fp8_resident(
    const void* __restrict__ gate, const void* __restrict__ up, uint8_t* __restrict__ yq,
    float* __restrict__ scale, int64_t rows, int64_t cols, float static_scale) {
  constexpr int NW = THREADS / 64;
  constexpr int VEC = C::VEC;
  __shared__ uint32_t lds[2 * NW];
  const int nvec = (int)(cols / VEC);
  int parity = 0;
  // Global-pointer row access: for this kernel's 1024 x 2 shape it measured
  // faster than buffer resources on MI355X (96 vs 119 us at [8192, 14336]).
  const uint32_t row_bytes = (uint32_t)(cols * C::kBytes);
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const int64_t off = row * cols * C::kBytes;
    const RowBuf<false> bg(static_cast<const char*>(gate) + off, row_bytes);
    const RowBuf<false> bu(static_cast<const char*>(up) + off, row_bytes);
    u32x4 graw[ITEMS], uraw[ITEMS];
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      const uint32_t v = threadIdx.x + k * THREADS;
      if (v < (uint32_t)nvec) {
        graw[k] = bg.ld16(v * 16u);
        uraw[k] = bu.ld16(v * 16u);
      }
    }
    float y[ITEMS][VEC];
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      const int v = threadIdx.x + k * THREADS;
      if (v < nvec) {
        float u[VEC];
        C::unpack(graw[k], y[k]);
        C::unpack(uraw[k], u);
        swiglu_math<C>(y[k], u);
#pragma unroll
        for (int i = 0; i < VEC; i += 2) {
          C::round2(y[k][i], y[k][i + 1]);
          amax = absmax2(amax, y[k][i], y[k][i + 1]);
        }
      }
    }
    // amax >= 0 (or NaN), so unsigned max on its bits is the float maximum.
    amax = bits_f32(block_allreduce<NW>(f32_bits(amax), MaxU32{}, lds, parity));
    parity ^= 1;
    float s;
    if constexpr (STATIC) {
      s = static_scale;
    } else {
      s = scale_from_amax<FMT>(amax);
      if (threadIdx.x == 0) scale[row] = s;
    }
    const float r = 1.0f / s;
    const bool fast = fast_path_ok<FMT>(s, r, amax);
    const RowBuf<false> bq(yq + row * cols, (uint32_t)cols);
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      const uint32_t v = threadIdx.x + k * THREADS;
      if (v < (uint32_t)nvec) {
        uint32_t wq[VEC / 4];
        if (fast) {
          quant_fast<FMT, VEC>(y[k], s, r, wq);
        } else {
          quant_exact<FMT, VEC>(y[k], s, wq);
        }
        if constexpr (VEC == 8) {
          bq.st8((u32x2){wq[0], wq[1]}, v * 8u);
        } else {
          bq.st4(wq[0], v * 4u);
        }
      }
    }
  }
}

// FP8 variant, any alignment / row length: y is recomputed in the second pass.
template <class C, bool STATIC, int FMT>
__global__ __launch_bounds__(256) void swiglu_fp8_generic(
    const void* __restrict__ gate, const void* __restrict__ up, uint8_t* __restrict__ yq,
    float* __restrict__ scale, int64_t rows, int64_t cols, float static_scale) {
  __shared__ uint32_t lds[2 * 4];
  int parity = 0;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const int64_t base = row * cols;
    float amax = 0.0f;
    for (int64_t j = threadIdx.x; j < cols; j += 256) {
      const float yv = C::round(swiglu1<C>(C::load1(gate, base + j), C::load1(up, base + j)));
      amax = absmax2(amax, yv, 0.0f);
    }
    amax = bits_f32(block_allreduce<4>(f32_bits(amax), MaxF32{}, lds, parity));
    parity ^= 1;
    float s;
    if constexpr (STATIC) {
      s = static_scale;
    } else {
      s = scale_from_amax<FMT>(amax);
      if (threadIdx.x == 0) scale[row] = s;
    }
    const float r = 1.0f / s;
    const bool fast = fast_path_ok<FMT>(s, r, amax);
    for (int64_t j = threadIdx.x; j < cols; j += 256) {
      const float yv = C::round(swiglu1<C>(C::load1(gate, base + j), C::load1(up, base + j)));
      const float qv = fast ? div_by_scale(yv, s, r) : div_x86(yv, s);
      yq[base + j] = (uint8_t)(fast ? (Fp8<FMT>::cvt4(qv, 0.0f, 0.0f, 0.0f) & 0xffu) : Fp8<FMT>::encode(qv));
    }
  }
}

template <class C, bool STATIC, int FMT>
int32_t launch_swiglu_fp8(const void* gate, const void* up, uint8_t* yq, float* scale, int64_t rows,
                          int64_t cols, float static_scale, hipStream_t st) {
  const bool vec_ok = (cols % C::VEC == 0) && host_aligned(gate, 16) && host_aligned(up, 16) &&
                      host_aligned(yq, C::VEC);
  const int64_t nvec = cols / C::VEC;
  const unsigned g = row_grid(rows);
  auto run = [&](auto shape) {
    using S = decltype(shape);
    swiglu_fp8_resident<C, S::kThreads, S::kItems, STATIC, FMT><<<g, S::kThreads, 0, st>>>(
        gate, up, yq, scale, rows, cols, static_scale);
  };
  // At most two vectors per thread keeps the kernel under 64 VGPRs of row
  // state; 1024-thread rows measured fastest on MI355X at cols = 14336 bf16.
  const bool done = vec_ok && pick_row_shape<RowShape<64, 1>, RowShape<64, 2>, RowShape<128, 2>, RowShape<256, 2>,
                                             RowShape<512, 2>, RowShape<1024, 2>, RowShape<1024, 4>>(nvec, run);
  if (!done) {
    swiglu_fp8_generic<C, STATIC, FMT><<<g, 256, 0, st>>>(gate, up, yq, scale, rows, cols, static_scale);
  }
  return launch_status();
}

}  // namespace
}  // namespace cck

using namespace cck;

extern "C" int32_t launch_swiglu_fwd(const void* gate, const void* up, void* y, int64_t n, int32_t dtype,
                                     void* stream) {
  if (n <= 0) return (int32_t)hipSuccess;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_codec(dtype, [&](auto codec) {
    using C = decltype(codec);
    const bool vec_ok = host_aligned(gate, 16) && host_aligned(up, 16) && host_aligned(y, 16);
    int64_t done = 0;
    if (vec_ok) {
      const int64_t nvec = n / C::VEC;
      if (nvec > 0) {
        constexpr int UNROLL = 4;
        const unsigned g = flat_grid((nvec + UNROLL - 1) / UNROLL, 256, 1 << 20);
        swiglu_flat<C, UNROLL><<<g, 256, 0, st>>>(static_cast<const u32x4*>(gate),
                                                   static_cast<const u32x4*>(up),
                                                   static_cast<u32x4*>(y), nvec);
      }
      done = nvec * C::VEC;
    }
    if (done < n) {
      swiglu_scalar<C><<<flat_grid(n - done, 256, 4096), 256, 0, st>>>(gate, up, y, done, n);
    }
    return launch_status();
  });
}

extern "C" int32_t launch_swiglu_fp8_fwd(const void* gate, const void* up, uint8_t* y_fp8, float* scale,
                                         int64_t rows, int64_t cols, float static_scale,
                                         int32_t scale_mode, int32_t dtype, int32_t fp8_format,
                                         void* stream) {
  if (scale_mode != 0 && scale_mode != 1) return (int32_t)hipErrorInvalidValue;
  if (rows <= 0 || cols <= 0) return (int32_t)hipSuccess;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_codec(dtype, [&](auto codec) {
    using C = decltype(codec);
    return with_fp8(fp8_format, [&](auto f) {
      constexpr int FMT = decltype(f)::value;
      if (scale_mode == 0) return launch_swiglu_fp8<C, false, FMT>(gate, up, y_fp8, scale, rows, cols, 0.0f, st);
      // Static scale: one flat stream over rows * cols elements.
      const int64_t n = rows * cols;
      int64_t done = 0;
      if (host_aligned(gate, 16) && host_aligned(up, 16) && host_aligned(y_fp8, C::VEC)) {
        const int64_t nvec = n / C::VEC;
        if (nvec > 0) {
          constexpr int UNROLL = 4;
          swiglu_fp8_static_flat<C, FMT, UNROLL><<<flat_grid((nvec + UNROLL - 1) / UNROLL, 256, 1 << 20), 256, 0, st>>>(
              static_cast<const u32x4*>(gate), static_cast<const u32x4*>(up), y_fp8, static_scale, nvec);
        }
        done = nvec * C::VEC;
      }
      if (done < n) {
        swiglu_fp8_static_scalar<C, FMT><<<flat_grid(n - done, 256, 4096), 256, 0, st>>>(gate, up, y_fp8, static_scale,
                                                                                         done, n);
      }
      return launch_status();
    });
  });
}
