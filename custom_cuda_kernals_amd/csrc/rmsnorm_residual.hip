// Fused residual-add + RMSNorm, optionally fused with FP8 quantisation of the
// normalised output, for gfx950.
//
// Semantics follow the eager oracle's rounding points exactly
// (baselines/rmsnorm_residual.py:123-136):
//   residual_out = T(x + residual)                       (rounded to storage)
//   variance     = sum(float(residual_out)^2) / cols     (fp32)
//   inv          = 1 / sqrt(variance + eps)              (both correctly rounded)
//   y            = T( T(float(residual_out) * inv) * weight )
// The FP8 variant quantises y (as stored in T) per row (dynamic, the
// baselines/fp8_quant.py:162-178 formula applied per token) or with a static
// scale, and does not write y itself.
//
// Design: one workgroup per row; each thread keeps its ITEMS 16-byte vectors
// of residual_out in registers between the sum-of-squares reduction and the
// normalisation, so x and residual are read from HBM exactly once and
// residual_out / y (or the FP8 codes) written once.
#include "launch.hpp"

namespace cck {
namespace {

#pragma clang fp contract(off)

template <class C>
struct AmaxOp2 {
  using type = MaxPkU16;
};
template <>
struct AmaxOp2<CodecF32> {
  using type = MaxU32;
};

// MODE: 0 = write y in T; 1 = FP8 codes with a per-row dynamic scale;
// 2 = FP8 codes with a static scale.
template <class C, int THREADS, int ITEMS, int MODE, int FMT>
__global__ __launch_bounds__(THREADS) void rmsnorm_resident(
    const void* __restrict__ x, const void* __restrict__ res, const void* __restrict__ w,
    void* __restrict__ y, uint8_t* __restrict__ yq, float* __restrict__ scale,
    void* __restrict__ ro, int64_t rows, int64_t cols, float eps, float static_scale) {
  constexpr int NW = THREADS / 64;
  constexpr int VEC = C::VEC;
  __shared__ uint32_t lds[2 * NW];
  const int nvec = (int)(cols / VEC);
  const u32x4* wv = static_cast<const u32x4*>(w);
  int parity = 0;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const int64_t off = row * cols * C::kBytes;
    const u32x4* xr = reinterpret_cast<const u32x4*>(static_cast<const char*>(x) + off);
    const u32x4* rr = reinterpret_cast<const u32x4*>(static_cast<const char*>(res) + off);
    u32x4* ror = reinterpret_cast<u32x4*>(static_cast<char*>(ro) + off);
    u32x4 rov[ITEMS];
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      const int v = threadIdx.x + k * THREADS;
      if (v < nvec) {
        float fx[VEC], fr[VEC], fo[VEC];
        C::unpack(__builtin_nontemporal_load(xr + v), fx);
        C::unpack(__builtin_nontemporal_load(rr + v), fr);
#pragma unroll
        for (int i = 0; i < VEC; ++i) fo[i] = fx[i] + fr[i];
        rov[k] = C::pack(fo);
        __builtin_nontemporal_store(rov[k], ror + v);
        C::unpack(rov[k], fo);
#pragma unroll
        for (int i = 0; i < VEC; ++i) acc += fo[i] * fo[i];
      }
    }
    const float total = bits_f32(block_allreduce<NW>(f32_bits(acc), AddF32{}, lds, parity));
    parity ^= 1;
    const float variance = total / (float)cols;
    const float inv = 1.0f / __builtin_sqrtf(variance + eps);

    if constexpr (MODE == 0) {
      u32x4* yr = reinterpret_cast<u32x4*>(static_cast<char*>(y) + off);
#pragma unroll
      for (int k = 0; k < ITEMS; ++k) {
        const int v = threadIdx.x + k * THREADS;
        if (v < nvec) {
          float fo[VEC], fw[VEC];
          C::unpack(rov[k], fo);
          C::unpack(wv[v], fw);
#pragma unroll
          for (int i = 0; i < VEC; ++i) fo[i] = C::round(fo[i] * inv) * fw[i];
          __builtin_nontemporal_store(C::pack(fo), yr + v);
        }
      }
    } else {
      // y rounded to T, kept packed; amax over |y| for the dynamic scale.
      uint32_t amax_acc = 0;
#pragma unroll
      for (int k = 0; k < ITEMS; ++k) {
        const int v = threadIdx.x + k * THREADS;
        if (v < nvec) {
          float fo[VEC], fw[VEC];
          C::unpack(rov[k], fo);
          C::unpack(wv[v], fw);
#pragma unroll
          for (int i = 0; i < VEC; ++i) fo[i] = C::round(fo[i] * inv) * fw[i];
          rov[k] = C::pack(fo);
          amax_acc = C::absmax_vec(rov[k], amax_acc);
        }
      }
      float s, amax;
      if constexpr (MODE == 1) {
        amax_acc = block_allreduce<NW>(amax_acc, typename AmaxOp2<C>::type{}, lds, parity);
        parity ^= 1;
        amax = C::absmax_to_float(amax_acc);
        s = scale_from_amax<FMT>(amax);
        if (threadIdx.x == 0) scale[row] = s;
      } else {
        // Static scale: the fast/exact choice only needs this row's amax.
        amax_acc = block_allreduce<NW>(amax_acc, typename AmaxOp2<C>::type{}, lds, parity);
        parity ^= 1;
        amax = C::absmax_to_float(amax_acc);
        s = static_scale;
      }
      const float r = 1.0f / s;
      const bool fast = fast_path_ok<FMT>(s, r, amax);
      uint8_t* qr = yq + row * cols;
#pragma unroll
      for (int k = 0; k < ITEMS; ++k) {
        const int v = threadIdx.x + k * THREADS;
        if (v < nvec) {
          float fy[VEC];
          C::unpack(rov[k], fy);
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
}

// Any alignment / row length: scalar accesses; residual_out is re-read by the
// thread that wrote it.
template <class C, int MODE, int FMT>
__global__ __launch_bounds__(256) void rmsnorm_generic(
    const void* __restrict__ x, const void* __restrict__ res, const void* __restrict__ w,
    void* __restrict__ y, uint8_t* __restrict__ yq, float* __restrict__ scale,
    void* __restrict__ ro, int64_t rows, int64_t cols, float eps, float static_scale) {
  __shared__ uint32_t lds[2 * 4];
  int parity = 0;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const int64_t base = row * cols;
    float acc = 0.0f;
    for (int64_t j = threadIdx.x; j < cols; j += 256) {
      const float o = C::round(C::load1(x, base + j) + C::load1(res, base + j));
      C::store1(ro, base + j, o);
      acc += o * o;
    }
    const float total = bits_f32(block_allreduce<4>(f32_bits(acc), AddF32{}, lds, parity));
    parity ^= 1;
    const float inv = 1.0f / __builtin_sqrtf(total / (float)cols + eps);
    if constexpr (MODE == 0) {
      for (int64_t j = threadIdx.x; j < cols; j += 256) {
        C::store1(y, base + j, C::round(C::load1(ro, base + j) * inv) * C::load1(w, j));
      }
    } else {
      uint32_t amax_acc = 0;
      for (int64_t j = threadIdx.x; j < cols; j += 256) {
        const float yv = C::round(C::round(C::load1(ro, base + j) * inv) * C::load1(w, j));
        amax_acc = max(amax_acc, f32_bits(yv) & 0x7fffffffu);
      }
      amax_acc = block_allreduce<4>(amax_acc, MaxU32{}, lds, parity);
      parity ^= 1;
      const float amax = bits_f32(amax_acc);
      float s;
      if constexpr (MODE == 1) {
        s = scale_from_amax<FMT>(amax);
        if (threadIdx.x == 0) scale[row] = s;
      } else {
        s = static_scale;
      }
      const float r = 1.0f / s;
      const bool fast = fast_path_ok<FMT>(s, r, amax);
      for (int64_t j = threadIdx.x; j < cols; j += 256) {
        const float yv = C::round(C::round(C::load1(ro, base + j) * inv) * C::load1(w, j));
        const float qv = fast ? div_by_scale(yv, s, r) : div_x86(yv, s);
        yq[base + j] = (uint8_t)(fast ? (Fp8<FMT>::cvt4(qv, 0.0f, 0.0f, 0.0f) & 0xffu) : Fp8<FMT>::encode(qv));
      }
    }
  }
}

template <class C, int MODE, int FMT>
int32_t launch_rmsnorm(const void* x, const void* res, const void* w, void* y, uint8_t* yq,
                       float* scale, void* ro, int64_t rows, int64_t cols, float eps,
                       float static_scale, hipStream_t st) {
  const bool vec_ok = (cols % C::VEC == 0) && host_aligned(x, 16) && host_aligned(res, 16) &&
                      host_aligned(w, 16) && host_aligned(ro, 16) &&
                      (MODE == 0 ? host_aligned(y, 16) : host_aligned(yq, C::VEC));
  const int64_t nvec = cols / C::VEC;
  const unsigned g = row_grid(rows);
#define CCK_RMS(T_, I_) \
  rmsnorm_resident<C, T_, I_, MODE, FMT><<<g, T_, 0, st>>>(x, res, w, y, yq, scale, ro, rows, cols, eps, static_scale)
  if (vec_ok && nvec <= 64) {
    CCK_RMS(64, 1);
  } else if (vec_ok && nvec <= 256) {
    CCK_RMS(256, 1);
  } else if (vec_ok && nvec <= 512) {
    CCK_RMS(256, 2);
  } else if (vec_ok && nvec <= 1024) {
    CCK_RMS(256, 4);
  } else if (vec_ok && nvec <= 2048) {
    CCK_RMS(256, 8);
  } else if (vec_ok && nvec <= 4096) {
    CCK_RMS(512, 8);
  } else {
    rmsnorm_generic<C, MODE, FMT><<<g, 256, 0, st>>>(x, res, w, y, yq, scale, ro, rows, cols, eps, static_scale);
  }
#undef CCK_RMS
  return launch_status();
}

}  // namespace
}  // namespace cck

using namespace cck;

extern "C" int32_t launch_rmsnorm_residual_fwd(const void* x, const void* residual, const void* weight,
                                               void* y, void* residual_out, int64_t rows, int64_t cols,
                                               float eps, int32_t dtype, void* stream) {
  if (rows <= 0 || cols <= 0) return (int32_t)hipSuccess;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_codec(dtype, [&](auto codec) {
    using C = decltype(codec);
    return launch_rmsnorm<C, 0, kF8E4M3>(x, residual, weight, y, nullptr, nullptr, residual_out, rows,
                                         cols, eps, 0.0f, st);
  });
}

extern "C" int32_t launch_rmsnorm_residual_fp8_fwd(const void* x, const void* residual,
                                                   const void* weight, uint8_t* y_fp8, float* scale,
                                                   void* residual_out, int64_t rows, int64_t cols,
                                                   float eps, float static_scale, int32_t scale_mode,
                                                   int32_t dtype, int32_t fp8_format, void* stream) {
  if (scale_mode != 0 && scale_mode != 1) return (int32_t)hipErrorInvalidValue;
  if (rows <= 0 || cols <= 0) return (int32_t)hipSuccess;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_codec(dtype, [&](auto codec) {
    using C = decltype(codec);
    return with_fp8(fp8_format, [&](auto f) {
      constexpr int FMT = decltype(f)::value;
      if (scale_mode == 0) {
        return launch_rmsnorm<C, 1, FMT>(x, residual, weight, nullptr, y_fp8, scale, residual_out, rows,
                                         cols, eps, 0.0f, st);
      }
      return launch_rmsnorm<C, 2, FMT>(x, residual, weight, nullptr, y_fp8, nullptr, residual_out, rows,
                                       cols, eps, static_scale, st);
    });
  });
}
