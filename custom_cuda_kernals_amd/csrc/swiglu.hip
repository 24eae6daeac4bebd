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
// loads, one store per vector) with the arithmetic SiLU of silu.hpp. The FP8
// variants add the FP8 conversion per element, which makes them VALU-bound
// with the arithmetic SiLU; for bf16 they look the SiLU up in the LDS table
// instead (silu.hpp). The per-token FP8 variant is row-resident: one
// workgroup per row keeps y in registers while it reduces the row amax, so
// gate/up are read once and only the codes and the scale are written.
#include "launch.hpp"
#include "silu.hpp"

namespace cck {
namespace {

// The plain op: a grid-stride stream of 16-byte vectors, UNROLL per thread
// per step, the next step's loads issued before this step's math. It uses the
// arithmetic SiLU for every dtype: with the LDS table (and its per-workgroup
// fill) the bf16 stream measured slower on MI355X (111.4 vs 109.9 us at
// 8192 x 14336, 233.8 vs 218.8 us at 16384 x 14336).
template <class C, int THREADS, int UNROLL>
__global__ __launch_bounds__(THREADS) void swiglu_flat(const u32x4* __restrict__ gate,
                                                       const u32x4* __restrict__ up,
                                                       u32x4* __restrict__ y, int64_t nvec) {
  const int64_t stride = (int64_t)gridDim.x * THREADS * UNROLL;
  int64_t base = (int64_t)blockIdx.x * THREADS * UNROLL + threadIdx.x;
  u32x4 g[UNROLL], u[UNROLL];
  auto load = [&](int64_t b) {
#pragma unroll
    for (int k = 0; k < UNROLL; ++k) {
      const int64_t v = b + k * THREADS;
      if (v < nvec) {
        g[k] = ld_stream(gate + v);
        u[k] = ld_stream(up + v);
      }
    }
  };
  load(base);
  for (; base < nvec; base += stride) {
#pragma unroll
    for (int k = 0; k < UNROLL; ++k) {
      const int64_t v = base + k * THREADS;
      if (v < nvec) {
        float a[C::VEC], uf[C::VEC];
        silu_vec<C, false>(g[k], nullptr, a);
        C::unpack(u[k], uf);
#pragma unroll
        for (int i = 0; i < C::VEC; ++i) a[i] = a[i] * uf[i];
        st_stream(C::pack(a), y + v);
      }
    }
    load(base + stride);
  }
}

template <class C>
__device__ inline float swiglu1(float g, float u) {
  return C::round(silu_one<C>(g)) * u;
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
// max |y| * (1/s) is inside the fast range, the exact path otherwise. The
// static kernels also store s into scale_out[0] when given one (the scale
// tensor the Python API returns), so a static call is one launch.
template <class C, int FMT, int THREADS, int UNROLL, bool TAB>
__global__ __launch_bounds__(THREADS) void swiglu_fp8_static_flat(const u32x4* __restrict__ gate,
                                                                 const u32x4* __restrict__ up,
                                                                 uint8_t* __restrict__ yq, float s,
                                                                 int64_t nvec, float* __restrict__ scale_out) {
  constexpr int VEC = C::VEC;
  if (scale_out != nullptr && blockIdx.x == 0 && threadIdx.x == 0) scale_out[0] = s;
  __shared__ __attribute__((aligned(16))) float tab[TAB ? SiluTableBF16::kEntries : 1];
  const float r = 1.0f / s;
  const bool scale_ok = fast_path_ok<FMT>(s, r, 0.0f);
  const int64_t stride = (int64_t)gridDim.x * THREADS * UNROLL;
  int64_t base = (int64_t)blockIdx.x * THREADS * UNROLL + threadIdx.x;
  u32x4 g[UNROLL], u[UNROLL];
  auto load = [&](int64_t b) {
#pragma unroll
    for (int k = 0; k < UNROLL; ++k) {
      const int64_t v = b + k * THREADS;
      if (v < nvec) {
        g[k] = ld_stream(gate + v);
        u[k] = ld_stream(up + v);
      }
    }
  };
  load(base);
  if constexpr (TAB) {
    SiluTableBF16::fill_single(tab, threadIdx.x, THREADS);
    __syncthreads();
  }
  for (; base < nvec; base += stride) {
#pragma unroll
    for (int k = 0; k < UNROLL; ++k) {
      const int64_t v = base + k * THREADS;
      if (v < nvec) {
        float y[VEC], uf[VEC];
        silu_vec<C, TAB>(g[k], tab, y);
        C::unpack(u[k], uf);
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < VEC; i += 2) {
          y[i] = y[i] * uf[i];
          y[i + 1] = y[i + 1] * uf[i + 1];
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
    load(base + stride);
  }
}

template <class C, int FMT>
__global__ __launch_bounds__(256) void swiglu_fp8_static_scalar(const void* __restrict__ gate,
                                                               const void* __restrict__ up,
                                                               uint8_t* __restrict__ yq, float s,
                                                               int64_t begin, int64_t n,
                                                               float* __restrict__ scale_out) {
  if (scale_out != nullptr && blockIdx.x == 0 && threadIdx.x == 0) scale_out[0] = s;
  const float r = 1.0f / s;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = begin + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
    const float yv = C::round(swiglu1<C>(C::load1(gate, i), C::load1(up, i)));
    const bool fast = fast_path_ok<FMT>(s, r, __builtin_fabsf(yv));
    const float qv = fast ? div_by_scale(yv, s, r) : div_x86(yv, s);
    yq[i] = (uint8_t)(fast ? (Fp8<FMT>::cvt4(qv, 0.0f, 0.0f, 0.0f) & 0xffu) : Fp8<FMT>::encode(qv));
  }
}

// Code stores of the per-token variant: a buffer resource with SC1|NT, measured
// on MI355X against global-pointer NT stores: 90.4 vs 90.8 us at
// [8192, 14336], 177.8 vs 179.2 us at [16384, 14336].
constexpr bool kRsrcQ = true;
constexpr int kPolQ = kPolSC1 | kPolNT;

// FP8 variant with register-resident rows; y is kept as floats (already
// rounded to T) between the amax reduction and the quantisation. TAB (bf16)
// selects the LDS SiLU table, filled while the first row's loads are in
// flight. STATIC uses static_scale and skips the row reduction; each thread's
// own max |y| then selects the fast or exact conversion for its vectors.
// LDSY (rows of more than four vectors per thread, and most bf16 per-token
// rows of three or four): y is parked in LDS, in slots only its own thread
// reads back, instead of registers; 1024 x 8
// vectors hold rows of 65536 bf16 / fp16 (32768 fp32) elements in 128 KB.
// The raw registers are then free after the SiLU, so the next row's loads go
// out before the amax reduction.
template <class C, int THREADS, int ITEMS, int FMT, bool TAB, bool STATIC, bool LDSY = false>
__global__ __launch_bounds__(THREADS) void swiglu_fp8_resident(
    const void* __restrict__ gate, const void* __restrict__ up, uint8_t* __restrict__ yq,
    float* __restrict__ scale, float static_scale, int64_t rows, int64_t cols) {
  constexpr int NW = THREADS / 64;
  __shared__ u32x4 ylds[LDSY ? THREADS * ITEMS : 1];
  constexpr int VEC = C::VEC;
  __shared__ uint32_t lds[2 * NW];
  __shared__ __attribute__((aligned(16))) float tab[TAB ? SiluTableBF16::kEntries : 1];
  const int nvec = (int)(cols / VEC);
  int parity = 0;
  // A static scale goes to scale[0] when the caller passed a scale word.
  if (STATIC && scale != nullptr && blockIdx.x == 0 && threadIdx.x == 0) scale[0] = static_scale;
  // Global-pointer row access: for this kernel's 1024 x 2 shape it measured
  // faster than buffer resources on MI355X (96 vs 119 us at [8192, 14336]).
  const uint32_t row_bytes = (uint32_t)(cols * C::kBytes);
  u32x4 graw[ITEMS], uraw[ITEMS];
  auto load = [&](int64_t row) {
    const int64_t off = row * cols * C::kBytes;
    const RowBuf<false> bg(static_cast<const char*>(gate) + off, row_bytes);
    const RowBuf<false> bu(static_cast<const char*>(up) + off, row_bytes);
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      const uint32_t v = threadIdx.x + k * THREADS;
      if (v < (uint32_t)nvec) {
        graw[k] = bg.ld16(v * 16u);
        uraw[k] = bu.ld16(v * 16u);
      }
    }
  };
  int64_t row = blockIdx.x;
  if (row < rows) load(row);
  if constexpr (TAB) {
    // Pair fill: measured 0.3-1.6 % faster than fill_single in this kernel
    // on MI355X (and 1.7 % slower in the static-scale flat kernel).
    SiluTableBF16::fill_pairs(tab, threadIdx.x, THREADS);
    __syncthreads();
  }
  for (; row < rows; row += gridDim.x) {
    float y[LDSY ? 1 : ITEMS][VEC];
    float amax = 0.0f;
    uint32_t pacc = 0;  // bf16 parked rows: max |y| as packed bf16 bits
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      const int v = threadIdx.x + k * THREADS;
      if (v < nvec) {
        float u[VEC];
        float(&yk)[VEC] = y[LDSY ? 0 : k];
        silu_vec<C, TAB>(graw[k], tab, yk);
        C::unpack(uraw[k], u);
        if constexpr (LDSY && std::is_same_v<C, CodecBF16>) {
          // Parked bf16 rows: y rounded once, straight into its packed LDS
          // form, and max |y| taken on the packed bits (v_pk_max_u16; exact,
          // y being bf16 already, and NaN-propagating): one VALU operation
          // per element less than rounding, unpacking and re-packing, for
          // these rows that are bound by issue. Same bits; 188.5 vs 190.5 us
          // at [8192, 28672], 98.0 vs 99.7 at [4096, 28672], 294.4 vs 297.2
          // at [8192, 40960] on MI355X.
          u32x4 w;
#pragma unroll
          for (int i = 0; i < VEC / 2; ++i) {
            w[i] = pack2_bf16(yk[2 * i] * u[2 * i], yk[2 * i + 1] * u[2 * i + 1]);
            pacc = pk_max_u16(pacc, w[i] & 0x7fff7fffu);
          }
          ylds[k * THREADS + threadIdx.x] = w;
        } else {
#pragma unroll
          for (int i = 0; i < VEC; i += 2) {
            yk[i] = yk[i] * u[i];
            yk[i + 1] = yk[i + 1] * u[i + 1];
            C::round2(yk[i], yk[i + 1]);
            amax = absmax2(amax, yk[i], yk[i + 1]);
          }
          if constexpr (LDSY) ylds[k * THREADS + threadIdx.x] = C::pack(y[0]);
        }
      }
    }
    if constexpr (LDSY && std::is_same_v<C, CodecBF16>) amax = C::absmax_to_float(pacc);
    if constexpr (LDSY) {
      if (row + gridDim.x < rows) load(row + gridDim.x);
    }
    float s;
    if constexpr (STATIC) {
      // A scheduling fence where the reduction would be: without it the
      // compiler interleaves the conversion with the SiLU and needs 96 VGPRs
      // (one 1024-thread workgroup per CU instead of two).
      __builtin_amdgcn_sched_barrier(0);
      s = static_scale;
    } else {
      // amax >= 0 (or NaN), so unsigned max on its bits is the float maximum.
      amax = bits_f32(block_allreduce<NW>(f32_bits(amax), MaxU32{}, lds, parity));
      parity ^= 1;
      s = scale_from_amax<FMT>(amax);
      if (threadIdx.x == 0) scale[row] = s;
    }
    const float r = 1.0f / s;
    const bool fast = fast_path_ok<FMT>(s, r, amax);
    const RowBuf<kRsrcQ, kPolQ> bq(yq + row * cols, (uint32_t)cols);
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      const uint32_t v = threadIdx.x + k * THREADS;
      if (v < (uint32_t)nvec) {
        uint32_t wq[VEC / 4];
        float(&yk)[VEC] = y[LDSY ? 0 : k];
        if constexpr (LDSY) C::unpack(ylds[k * THREADS + threadIdx.x], y[0]);
        if (fast) {
          quant_fast<FMT, VEC>(yk, s, r, wq);
        } else {
          quant_exact<FMT, VEC>(yk, s, wq);
        }
        if constexpr (VEC == 8) {
          bq.st8((u32x2){wq[0], wq[1]}, v * 8u);
        } else {
          bq.st4(wq[0], v * 4u);
        }
      }
    }
    if constexpr (!LDSY) {
      if (row + gridDim.x < rows) load(row + gridDim.x);
    }
  }
}

// Per-token FP8 variant, any alignment / row length: y is recomputed in the
// second pass.
template <class C, int FMT>
__global__ __launch_bounds__(256) void swiglu_fp8_generic(
    const void* __restrict__ gate, const void* __restrict__ up, uint8_t* __restrict__ yq,
    float* __restrict__ scale, int64_t rows, int64_t cols) {
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
    const float s = scale_from_amax<FMT>(amax);
    if (threadIdx.x == 0) scale[row] = s;
    const float r = 1.0f / s;
    const bool fast = fast_path_ok<FMT>(s, r, amax);
    for (int64_t j = threadIdx.x; j < cols; j += 256) {
      const float yv = C::round(swiglu1<C>(C::load1(gate, base + j), C::load1(up, base + j)));
      const float qv = fast ? div_by_scale(yv, s, r) : div_x86(yv, s);
      yq[base + j] = (uint8_t)(fast ? (Fp8<FMT>::cvt4(qv, 0.0f, 0.0f, 0.0f) & 0xffu) : Fp8<FMT>::encode(qv));
    }
  }
}

// Register-resident rows: one workgroup per row for the row-length buckets
// below; false (nothing launched) when no bucket holds the row or the
// buffers are not aligned for 16-byte access. STATIC rows are used only with
// the bf16 table and 768 or more threads per row.
template <class C, int FMT, bool STATIC>
bool launch_swiglu_fp8_rows(const void* gate, const void* up, uint8_t* yq, float* scale, float static_scale,
                            int64_t rows, int64_t cols, hipStream_t st) {
  const bool vec_ok = (cols % C::VEC == 0) && host_aligned(gate, 16) && host_aligned(up, 16) &&
                      host_aligned(yq, C::VEC);
  const int64_t nvec = cols / C::VEC;
  const unsigned g = row_grid(rows);
  bool launched = false;
  auto run = [&](auto shape) {
    using S = decltype(shape);
    // The table pays for its per-workgroup fill only on long rows. Static
    // scales use these rows only from 768 threads (the flat stream otherwise).
    constexpr bool kTab = std::is_same_v<C, CodecBF16> && S::kThreads * S::kItems >= 1152;
    auto go = [&](auto ldsy) {
      constexpr bool kLdsY = decltype(ldsy)::value;
      constexpr auto kernel = swiglu_fp8_resident<C, S::kThreads, S::kItems, FMT, kTab, STATIC, kLdsY>;
      // bf16 rows with y in LDS run on a grid of the workgroups the device
      // holds at once, each looping over rows: one SiLU table fill per
      // workgroup instead of per row, no idle CU between rows, and the next
      // row's loads in flight across the amax reduction (4096 rows: 194.5
      // against 209.8 us at 53248 columns, 239.8 against 263.6 at 65536).
      // The same grid loses on register-resident rows (config 3v 100.5
      // against 89.8 us) and on fp16 LDS rows (5-18 %).
      constexpr bool kLoop = kTab && kLdsY;
      const int64_t resident = kLoop ? resident_groups<kernel>(S::kThreads) : 0;
      const unsigned grid = resident > 0 && resident < (int64_t)g ? (unsigned)resident : g;
      kernel<<<grid, S::kThreads, 0, st>>>(gate, up, yq, scale, static_scale, rows, cols);
      launched = true;
    };
    if constexpr (S::kItems > 4) {
      if constexpr (!STATIC) go(std::true_type{});
    } else if constexpr (kTab && !STATIC && S::kThreads == 1024 && S::kItems >= 3) {
      // bf16 per-token rows of three and four vectors per thread park y in
      // LDS (48 / 64 KB) on the looping grid too, where the grid loops (more
      // rows than resident workgroups) and at most 3/4 of the threads hold
      // a last vector. Same-run A/B against y in registers with one
      // workgroup per row, 8192 rows: 16896 columns 119.1 against 125.7 us,
      // 18944 127.3 / 140.7, 22016 146.4 / 156.4, 25600 180.6 / 186.6,
      // 28672 190.6 / 202.1, 30720 204.5 / 216.2; 1024 rows of 28672 29.0 /
      // 31.4. Past that fill it lost: 23040 168.6 / 163.9, 23552 172.2 /
      // 168.5, 31744 236.0 / 231.3, 32768 238.0 / 230.5 (24576 tied); so
      // did a grid that does not loop (256 rows of 28672: 9.5 / 9.0) and
      // fp16 and fp32 rows (1-4 %).
      constexpr auto kParked = swiglu_fp8_resident<C, S::kThreads, S::kItems, FMT, kTab, STATIC, true>;
      const int64_t last = nvec - (int64_t)(S::kItems - 1) * S::kThreads;  // threads holding a last vector
      const int64_t resident = resident_groups<kParked>(S::kThreads);
      if (4 * last <= 3 * S::kThreads && resident > 0 && resident < rows) {
        go(std::true_type{});
      } else {
        go(std::false_type{});
      }
    } else if constexpr (!STATIC || (kTab && S::kThreads >= 768)) {
      go(std::false_type{});
    }
  };
  // bf16 rows from a sweep over THREADS 256..1024 (step 128) x ITEMS 1..4,
  // with and without the table, on MI355X at 8192 rows of 5632..29568
  // elements (graph-replayed, 2 GiB rotation): 512 x 2 at 5632 (37.1 us);
  // 384 x 3 with the table at 8192, 53.4 against 57.6 for 512 x 2; 768 x 2
  // at 11008, 69.5 against 70.4 for 1024 x 2; 1024 x 2 at 14336 (89.8);
  // 1024 x 3 at 18944 and 22016, 140.6 / 156.3 against 142.2 / 159.7 for
  // 1024 x 4 (static scale 122.5 / 137.5 against 128.7 / 148.9). fp16 rows
  // (no table, VALU-bound, and at 68 VGPRs a 1024 x 2 workgroup is alone on
  // its CU) from the same sweep: 768 x 2 at 11008, 78.9 against 113.2 us for
  // 1024 x 2; 512 x 4 at 14336, 100.6 against 125.9; 1024 x 3 at 18944,
  // 166.3 against 170.7; 256 x 3 at 5632, 39.5 against 41.0; 512 x 2 at 8192
  // (57.5; 62.8 for 384 x 3). fp32 rows keep two vectors per thread up to
  // 1024 x 2. Wider rows of every type take 1024 x 6 or 8 with y in LDS.
  if (vec_ok) {
    if constexpr (std::is_same_v<C, CodecBF16>) {
      if (nvec > 896 && nvec <= 1152) {
        run(RowShape<384, 3>{});
      } else {
        pick_row_shape<RowShape<64, 1>, RowShape<64, 2>, RowShape<128, 2>, RowShape<256, 2>, RowShape<512, 2>,
                       RowShape<768, 2>, RowShape<1024, 2>, RowShape<1024, 3>, RowShape<1024, 4>,
                       RowShape<1024, 6>, RowShape<1024, 8>>(nvec, run);
      }
    } else if constexpr (std::is_same_v<C, CodecF16>) {
      pick_row_shape<RowShape<64, 1>, RowShape<64, 2>, RowShape<128, 2>, RowShape<256, 2>, RowShape<256, 3>,
                     RowShape<512, 2>, RowShape<768, 2>, RowShape<512, 4>, RowShape<1024, 3>,
                     RowShape<1024, 4>, RowShape<1024, 6>, RowShape<1024, 8>>(nvec, run);
    } else {
      pick_row_shape<RowShape<64, 1>, RowShape<64, 2>, RowShape<128, 2>, RowShape<256, 2>, RowShape<512, 2>,
                     RowShape<1024, 2>, RowShape<1024, 4>, RowShape<1024, 6>, RowShape<1024, 8>>(nvec, run);
    }
  }
  return launched;
}

template <class C, int FMT>
int32_t launch_swiglu_fp8_token(const void* gate, const void* up, uint8_t* yq, float* scale, int64_t rows,
                                int64_t cols, hipStream_t st) {
  if (!launch_swiglu_fp8_rows<C, FMT, false>(gate, up, yq, scale, 0.0f, rows, cols, st)) {
    swiglu_fp8_generic<C, FMT><<<row_grid(rows), 256, 0, st>>>(gate, up, yq, scale, rows, cols);
  }
  return launch_status();
}

// Static-scale FP8 streams of at least this many 16-byte vectors (1M bf16
// elements) use the SiLU table: 1024-thread workgroups of two vectors per
// thread, so one table fill serves 16384 elements.
constexpr int64_t kTabMinVec = int64_t(1) << 17;
constexpr int kTabThreads = 1024, kTabUnroll = 2;

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
      const u32x4* g4 = static_cast<const u32x4*>(gate);
      const u32x4* u4 = static_cast<const u32x4*>(up);
      u32x4* y4 = static_cast<u32x4*>(y);
      if (nvec > 0) {
        // 512 threads x 2 vectors: 108.9 us at [8192, 14336] bf16 on MI355X,
        // against 109.8 at 256 x 4 and 111.4-116 for the other shapes tried;
        // at most 3 workgroups per CU (4 fit): 107.3-107.9 vs 108.0-108.5 us
        // (fp16 107.4 vs 108.4, fp32 216.1 vs 218.4).
        constexpr int THREADS = 512, UNROLL = 2;
        swiglu_flat<C, THREADS, UNROLL>
            <<<flat_grid((nvec + UNROLL - 1) / UNROLL, THREADS, 1 << 20), THREADS, kLdsForGroupsPerCu<3>, st>>>(
                g4, u4, y4, nvec);
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
      if (scale_mode == 0) return launch_swiglu_fp8_token<C, FMT>(gate, up, y_fp8, scale, rows, cols, st);
      if (launch_swiglu_fp8_rows<C, FMT, true>(gate, up, y_fp8, scale, static_scale, rows, cols, st)) {
        return launch_status();
      }
      // Otherwise one flat stream over rows * cols elements.
      const int64_t n = rows * cols;
      int64_t done = 0;
      if (host_aligned(gate, 16) && host_aligned(up, 16) && host_aligned(y_fp8, C::VEC)) {
        const int64_t nvec = n / C::VEC;
        const u32x4* g4 = static_cast<const u32x4*>(gate);
        const u32x4* u4 = static_cast<const u32x4*>(up);
        bool tab = false;
        if constexpr (std::is_same_v<C, CodecBF16>) {
          if (nvec >= kTabMinVec) {
            constexpr int kPer = kTabThreads * kTabUnroll;
            swiglu_fp8_static_flat<C, FMT, kTabThreads, kTabUnroll, true>
                <<<flat_grid((nvec + kPer - 1) / kPer, 1, 1 << 20), kTabThreads, 0, st>>>(g4, u4, y_fp8,
                                                                                          static_scale, nvec, scale);
            tab = true;
          }
        }
        if (!tab && nvec > 0) {
          constexpr int UNROLL = 4;
          swiglu_fp8_static_flat<C, FMT, 256, UNROLL, false>
              <<<flat_grid((nvec + UNROLL - 1) / UNROLL, 256, 1 << 20), 256, 0, st>>>(g4, u4, y_fp8, static_scale,
                                                                                      nvec, scale);
        }
        done = nvec * C::VEC;
      }
      if (done < n) {
        swiglu_fp8_static_scalar<C, FMT><<<flat_grid(n - done, 256, 4096), 256, 0, st>>>(gate, up, y_fp8, static_scale,
                                                                                         done, n, scale);
      }
      return launch_status();
    });
  });
}
