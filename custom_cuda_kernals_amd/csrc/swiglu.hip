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
// loads, one store per vector, nontemporal so the 1.4 GB stream does not
// evict anything useful). The FP8 variant is row-resident: one workgroup per
// row keeps y packed in registers while it reduces the row amax, so gate/up
// are read once and only the codes and the scale are written.
#include "launch.hpp"

namespace cck {
namespace {

#pragma clang fp contract(off)

// sigmoid(g) = 1 / (1 + exp(-g)): exp to ~1 ulp (ocml), reciprocal refined by
// one Newton step with a fused remainder, i.e. within an ulp of the
// correctly rounded 1/d.
__device__ inline float silu(float g) {
  const float d = 1.0f + __builtin_expf(-g);
  const float r0 = __builtin_amdgcn_rcpf(d);
  const float e = __builtin_fmaf(-d, r0, 1.0f);
  const float sig = __builtin_fmaf(e, r0, r0);
  return g * sig;
}

template <class C>
__device__ inline u32x4 swiglu_vec(const u32x4& gw, const u32x4& uw) {
  float g[C::VEC], u[C::VEC];
  C::unpack(gw, g);
  C::unpack(uw, u);
#pragma unroll
  for (int i = 0; i < C::VEC; ++i) g[i] = C::round(silu(g[i])) * u[i];
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
        g[k] = __builtin_nontemporal_load(gate + v);
        u[k] = __builtin_nontemporal_load(up + v);
      }
    }
#pragma unroll
    for (int k = 0; k < UNROLL; ++k) {
      const int64_t v = base + k * 256;
      if (v < nvec) __builtin_nontemporal_store(swiglu_vec<C>(g[k], u[k]), y + v);
    }
  }
}

template <class C>
__global__ __launch_bounds__(256) void swiglu_scalar(const void* __restrict__ gate,
                                                     const void* __restrict__ up,
                                                     void* __restrict__ y, int64_t begin, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = begin + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
    C::store1(y, i, C::round(silu(C::load1(gate, i))) * C::load1(up, i));
  }
}

template <class C>
struct AmaxOp3 {
  using type = MaxPkU16;
};
template <>
struct AmaxOp3<CodecF32> {
  using type = MaxU32;
};

// FP8 variant, register-resident rows. STATIC selects the static scale.
template <class C, int THREADS, int ITEMS, bool STATIC, int FMT>
__global__ __launch_bounds__(THREADS) void swiglu_fp8_resident(
    const void* __restrict__ gate, const void* __restrict__ up, uint8_t* __restrict__ yq,
    float* __restrict__ scale, int64_t rows, int64_t cols, float static_scale) {
  constexpr int NW = THREADS / 64;
  constexpr int VEC = C::VEC;
  __shared__ uint32_t lds[2 * NW];
  const int nvec = (int)(cols / VEC);
  int parity = 0;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const int64_t off = row * cols * C::kBytes;
    const u32x4* gr = reinterpret_cast<const u32x4*>(static_cast<const char*>(gate) + off);
    const u32x4* ur = reinterpret_cast<const u32x4*>(static_cast<const char*>(up) + off);
    u32x4 yv[ITEMS];
    uint32_t acc = 0;
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      const int v = threadIdx.x + k * THREADS;
      if (v < nvec) {
        yv[k] = swiglu_vec<C>(__builtin_nontemporal_load(gr + v), __builtin_nontemporal_load(ur + v));
        acc = C::absmax_vec(yv[k], acc);
      }
    }
    acc = block_allreduce<NW>(acc, typename AmaxOp3<C>::type{}, lds, parity);
    parity ^= 1;
    const float amax = C::absmax_to_float(acc);
    float s;
    if constexpr (STATIC) {
      s = static_scale;
    } else {
      s = scale_from_amax<FMT>(amax);
      if (threadIdx.x == 0) scale[row] = s;
    }
    const float r = 1.0f / s;
    const bool fast = fast_path_ok<FMT>(s, r, amax);
    uint8_t* qr = yq + row * cols;
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      const int v = threadIdx.x + k * THREADS;
      if (v < nvec) {
        float fy[VEC];
        C::unpack(yv[k], fy);
        uint32_t wq[VEC / 4];
        if (fast) {
          quant_fast<FMT, VEC>(fy, s, r, wq);
        } else {
          quant_exact<FMT, VEC>(fy, s, wq);
        }
        if constexpr (VEC == 8) {
          __builtin_nontemporal_store((u32x2){wq[0], wq[1]}, reinterpret_cast<u32x2*>(qr + (int64_t)v * 8));
        } else {
          __builtin_nontemporal_store(wq[0], reinterpret_cast<uint32_t*>(qr + (int64_t)v * 4));
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
    uint32_t acc = 0;
    for (int64_t j = threadIdx.x; j < cols; j += 256) {
      const float yv = C::round(C::round(silu(C::load1(gate, base + j))) * C::load1(up, base + j));
      acc = max(acc, f32_bits(yv) & 0x7fffffffu);
    }
    acc = block_allreduce<4>(acc, MaxU32{}, lds, parity);
    parity ^= 1;
    const float amax = bits_f32(acc);
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
      const float yv = C::round(C::round(silu(C::load1(gate, base + j))) * C::load1(up, base + j));
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
#define CCK_SWF(T_, I_) \
  swiglu_fp8_resident<C, T_, I_, STATIC, FMT><<<g, T_, 0, st>>>(gate, up, yq, scale, rows, cols, static_scale)
  if (vec_ok && nvec <= 64) {
    CCK_SWF(64, 1);
  } else if (vec_ok && nvec <= 256) {
    CCK_SWF(256, 1);
  } else if (vec_ok && nvec <= 512) {
    CCK_SWF(256, 2);
  } else if (vec_ok && nvec <= 1024) {
    CCK_SWF(256, 4);
  } else if (vec_ok && nvec <= 1792) {
    CCK_SWF(256, 7);
  } else if (vec_ok && nvec <= 2048) {
    CCK_SWF(256, 8);
  } else if (vec_ok && nvec <= 4096) {
    CCK_SWF(512, 8);
  } else {
    swiglu_fp8_generic<C, STATIC, FMT><<<g, 256, 0, st>>>(gate, up, yq, scale, rows, cols, static_scale);
  }
#undef CCK_SWF
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
        constexpr int UNROLL = 2;
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
      return launch_swiglu_fp8<C, true, FMT>(gate, up, y_fp8, nullptr, rows, cols, static_scale, st);
    });
  });
}
