// Dynamic and static FP8 quantisation for gfx950.
//
// Semantics (baselines/fp8_quant.py:162-189): scale = clamp(amax / FP8_MAX,
// min=1e-12); codes = (x.float() / scale).to(fp8). Four granularities:
//
//   token  - one scale per row ([M]); not in the reference, it is
//            eager_fp8_quant's "tensor" formula applied to each row;
//   block  - one scale per 128x128 tile (fp8_quant.cu:59-152 in the reference);
//   tensor - one dynamic scale for the matrix (fp8_quant.cu:159-234);
//   static - a caller-given scale, no reduction.
//
// Design: a row (token mode) or tile (block mode) is read from HBM once with
// 16-byte loads and kept in registers while the workgroup reduces |x| with
// integer max on the magnitude bits (NaN-propagating, like torch's max); the
// division by the scale is the three-op correctly rounded form
// (div_by_scale) and the conversion is v_cvt_pk_fp8/bf8_f32. Rows or tiles
// whose scale is non-finite, or whose quotients leave the verified range of
// the hardware conversion, take the exact path (x86-compatible division +
// software encoder) as a workgroup-uniform branch.
#include <atomic>
#include <mutex>

#include "launch.hpp"

namespace cck {
namespace {

// Store VEC fp8 bytes (4 or 8) at byte offset `off` of `q` (VEC-aligned),
// as a streaming store.
template <int VEC>
__device__ inline void store_codes(uint8_t* q, int64_t off, const uint32_t (&w)[VEC / 4]) {
  if constexpr (VEC == 8) {
    st_stream((u32x2){w[0], w[1]}, reinterpret_cast<u32x2*>(q + off));
  } else {
    st_stream(w[0], reinterpret_cast<uint32_t*>(q + off));
  }
}

template <class C, int FMT>
__device__ inline void quant_vec(const u32x4& raw, float s, float r, bool fast, uint8_t* q, int64_t off) {
  float f[C::VEC];
  C::unpack(raw, f);
  uint32_t w[C::VEC / 4];
  if (fast) {
    quant_fast<FMT, C::VEC>(f, s, r, w);
  } else {
    quant_exact<FMT, C::VEC>(f, s, w);
  }
  store_codes<C::VEC>(q, off, w);
}

template <int FMT>
__device__ inline uint8_t quant1(float v, float s, float r, bool fast) {
  if (fast) {
    return (uint8_t)(Fp8<FMT>::cvt4(div_by_scale(v, s, r), 0.0f, 0.0f, 0.0f) & 0xffu);
  }
  return (uint8_t)Fp8<FMT>::encode(div_x86(v, s));
}

template <class C>
struct AmaxOp {
  using type = MaxPkU16;
};
template <>
struct AmaxOp<CodecF32> {
  using type = MaxU32;
};

// Cache policy of the per-token kernel's code stores.
constexpr int kPolTokenQ = kBufStorePolicy;

// ---------------------------------------------------------------------------
// Token granularity, register-resident rows: one workgroup per row, each
// thread holds ITEMS 16-byte vectors. Requires cols % VEC == 0 and 16-byte
// aligned x, VEC-aligned q.
// ---------------------------------------------------------------------------
template <class C, int FMT, int THREADS, int ITEMS>
__global__ __launch_bounds__(THREADS) void fp8_token_resident(const void* __restrict__ x,
                                                              uint8_t* __restrict__ q,
                                                              float* __restrict__ scale,
                                                              int64_t rows, int64_t cols) {
  constexpr int NW = THREADS / 64;
  __shared__ uint32_t lds[2 * NW];
  const int nvec = (int)(cols / C::VEC);
  int parity = 0;
  // Buffer-resource row access (no per-lane 64-bit addressing): 6.6 vs 6.8 us
  // at [2048, 4096] bf16 on MI355X.
  const uint32_t row_bytes = (uint32_t)(cols * C::kBytes);
  // A row's loads are issued one iteration ahead: the first row's at kernel
  // entry, before the loop set-up, and each next row's before the current
  // one is reduced. 6.0 vs 6.3-6.5 us at [2048, 4096] bf16 on MI355X against
  // loading inside the loop (where each load also waited for the one before
  // it to feed the max). Rows of more than four vectors per thread issue the
  // next row's loads after the current row's stores instead, so the two rows
  // do not hold registers at once.
  constexpr bool kAhead = ITEMS <= 4;
  u32x4 nxt[ITEMS];
  auto issue = [&](int64_t row) {
    const RowBuf<true> bx(static_cast<const char*>(x) + row * cols * C::kBytes, row_bytes);
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      const uint32_t v = threadIdx.x + k * THREADS;
      if (v < (uint32_t)nvec) nxt[k] = bx.ld16(v * 16u);
    }
  };
  if ((int64_t)blockIdx.x < rows) issue(blockIdx.x);
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    u32x4 raw[ITEMS];
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) raw[k] = nxt[k];
    if (kAhead && row + gridDim.x < rows) issue(row + gridDim.x);
    uint32_t acc = 0;
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      const uint32_t v = threadIdx.x + k * THREADS;
      if (v < (uint32_t)nvec) acc = C::absmax_vec(raw[k], acc);
    }
    acc = block_allreduce<NW>(acc, typename AmaxOp<C>::type{}, lds, parity);
    parity ^= 1;
    const float amax = C::absmax_to_float(acc);
    const float s = scale_from_amax<FMT>(amax);
    const float r = 1.0f / s;
    if (threadIdx.x == 0) scale[row] = s;
    const bool fast = fast_path_ok<FMT>(s, r, amax);
    const RowBuf<true, kPolTokenQ> bq(q + row * cols, (uint32_t)cols);
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      const uint32_t v = threadIdx.x + k * THREADS;
      if (v < (uint32_t)nvec) {
        float f[C::VEC];
        C::unpack(raw[k], f);
        uint32_t w[C::VEC / 4];
        if (fast) {
          quant_fast<FMT, C::VEC>(f, s, r, w);
        } else {
          quant_exact<FMT, C::VEC>(f, s, w);
        }
        if constexpr (C::VEC == 8) {
          bq.st8((u32x2){w[0], w[1]}, v * 8u);
        } else {
          bq.st4(w[0], v * 4u);
        }
      }
    }
    if (!kAhead && row + gridDim.x < rows) issue(row + gridDim.x);
  }
}

// Token granularity, any alignment / row length: scalar loads, the row is
// read twice (the second read is served by L2 for rows up to a few MB).
template <class C, int FMT>
__global__ __launch_bounds__(256) void fp8_token_generic(const void* __restrict__ x,
                                                         uint8_t* __restrict__ q,
                                                         float* __restrict__ scale, int64_t rows,
                                                         int64_t cols) {
  __shared__ uint32_t lds[2 * 4];
  int parity = 0;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const int64_t base = row * cols;
    uint32_t acc = 0;
    for (int64_t j = threadIdx.x; j < cols; j += 256) acc = C::absmax1(x, base + j, acc);
    acc = block_allreduce<4>(acc, typename AmaxOp<C>::type{}, lds, parity);
    parity ^= 1;
    const float amax = C::absmax_to_float(acc);
    const float s = scale_from_amax<FMT>(amax);
    const float r = 1.0f / s;
    if (threadIdx.x == 0) scale[row] = s;
    const bool fast = fast_path_ok<FMT>(s, r, amax);
    for (int64_t j = threadIdx.x; j < cols; j += 256) {
      q[base + j] = quant1<FMT>(C::load1(x, base + j), s, r, fast);
    }
  }
}

// ---------------------------------------------------------------------------
// Block granularity: one workgroup of THREADS per 128x128 tile, tile kept in
// registers. Vector path needs n % VEC == 0 and aligned pointers. RSRC loads
// through a buffer resource based at the tile's first element (32-bit
// offsets: the launcher checks that 128 rows fit in 2 GiB) and codes are
// stored as streaming stores; measured on MI355X against 256 threads with
// global-pointer loads and cached stores: 6.55 vs 9.8 us at [2048, 4096]
// bf16, 35.0 vs 38.0 us at [16384, 4096].
// ---------------------------------------------------------------------------
constexpr int kTile = 128;
constexpr int64_t kBlockPairMinTiles = 16384;
constexpr int64_t kBlockSplitMaxTiles = 1024;  // one round of 512-thread workgroups (4 per CU)

template <class C, int FMT, int THREADS, bool RSRC, int TW, bool SPLIT = false>
__global__ __launch_bounds__(THREADS * TW) void fp8_block_resident(const void* __restrict__ x,
                                                                   uint8_t* __restrict__ q,
                                                                   float* __restrict__ scale, int64_t m,
                                                                   int64_t n) {
  constexpr int VPR = kTile / C::VEC;  // vectors per tile row
  constexpr int RPP = THREADS / VPR;   // tile rows per pass
  constexpr int ITEMS = kTile / RPP;
  constexpr int NW = THREADS / 64;     // waves per tile
  __shared__ uint32_t lds[2 * NW * TW];
  const int tile = TW == 1 ? 0 : (int)(threadIdx.x / THREADS);  // which of the workgroup's tiles
  const int t = TW == 1 ? (int)threadIdx.x : (int)(threadIdx.x % THREADS);
  const int cv = t % VPR;
  const int rr = t / VPR;
  const int64_t tiles_x = (n + kTile - 1) / kTile;
  const int64_t tx = (int64_t)blockIdx.x * TW + tile;
  // The workgroup's first element; its TW tiles sit side by side from there.
  const int64_t origin = (int64_t)blockIdx.y * kTile * n + (int64_t)blockIdx.x * TW * kTile;
  const int64_t col = tx * kTile + cv * C::VEC;
  const int64_t row0 = (int64_t)blockIdx.y * kTile + rr;
  const bool col_ok = tx < tiles_x && col < n;
  const int64_t left = (m * n - origin) * C::kBytes;
  const RowBuf<true> bx(static_cast<const char*>(x) + origin * C::kBytes,
                        (uint32_t)(left < 0x7fffffff ? left : 0x7fffffff));
  u32x4 raw[ITEMS];
  uint32_t acc = 0;
  // Loads without branches: an element outside the matrix reads the
  // workgroup's first element (always inside it) and is replaced by zeros.
  // Loading under a branch instead made the compiler copy the whole of raw[]
  // at every join and wait on each load before the next: 232 VGPRs for fp32
  // tiles (8 vectors per thread, one workgroup per CU), 111.2 vs 55.4 us at
  // [8192, 8192] fp32, 6.29 vs 6.01 us at [2048, 4096] bf16 on MI355X.
  const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int k = 0; k < ITEMS; ++k) {
    const int64_t row = row0 + k * RPP;
    const bool ok = col_ok && row < m;
    if constexpr (RSRC) {
      const uint32_t off = (uint32_t)(((int64_t)(rr + k * RPP) * n + tile * kTile + cv * C::VEC) * C::kBytes);
      raw[k] = bx.ld16(ok ? off : 0u);
    } else {
      raw[k] = ld_stream(
          reinterpret_cast<const u32x4*>(static_cast<const char*>(x) + (ok ? row * n + col : origin) * C::kBytes));
    }
    raw[k] = ok ? raw[k] : zero;
    if constexpr (!SPLIT) acc = C::absmax_vec(raw[k], acc);
  }
  // SPLIT: every load is issued before the first max, instead of each max
  // waiting on its own load (see the launcher for when each pays).
  if constexpr (SPLIT) {
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) acc = C::absmax_vec(raw[k], acc);
  }
  if constexpr (TW == 1) {
    acc = block_allreduce<NW>(acc, typename AmaxOp<C>::type{}, lds, 0);
  } else {
    // One LDS slot per wave; each tile combines its own NW waves.
    acc = wave_allreduce(acc, typename AmaxOp<C>::type{});
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = acc;
    __syncthreads();
    acc = lds[tile * NW];
#pragma unroll
    for (int i = 1; i < NW; ++i) acc = typename AmaxOp<C>::type{}(acc, lds[tile * NW + i]);
  }
  const float amax = C::absmax_to_float(acc);
  const float s = scale_from_amax<FMT>(amax);
  const float r = 1.0f / s;
  if (t == 0 && tx < tiles_x) scale[(int64_t)blockIdx.y * tiles_x + tx] = s;
  const bool fast = fast_path_ok<FMT>(s, r, amax);
#pragma unroll
  for (int k = 0; k < ITEMS; ++k) {
    const int64_t row = row0 + k * RPP;
    if (col_ok && row < m) quant_vec<C, FMT>(raw[k], s, r, fast, q, row * n + col);
  }
}

template <class C, int FMT>
__global__ __launch_bounds__(256) void fp8_block_generic(const void* __restrict__ x,
                                                         uint8_t* __restrict__ q,
                                                         float* __restrict__ scale, int64_t m,
                                                         int64_t n) {
  __shared__ uint32_t lds[2 * 4];
  const int64_t r0 = (int64_t)blockIdx.y * kTile, c0 = (int64_t)blockIdx.x * kTile;
  const int64_t rh = (m - r0 < kTile) ? m - r0 : kTile;
  const int64_t cw = (n - c0 < kTile) ? n - c0 : kTile;
  uint32_t acc = 0;
  for (int64_t t = threadIdx.x; t < rh * cw; t += 256) {
    acc = C::absmax1(x, (r0 + t / cw) * n + c0 + t % cw, acc);
  }
  acc = block_allreduce<4>(acc, typename AmaxOp<C>::type{}, lds, 0);
  const float amax = C::absmax_to_float(acc);
  const float s = scale_from_amax<FMT>(amax);
  const float r = 1.0f / s;
  if (threadIdx.x == 0) scale[(int64_t)blockIdx.y * gridDim.x + blockIdx.x] = s;
  const bool fast = fast_path_ok<FMT>(s, r, amax);
  for (int64_t t = threadIdx.x; t < rh * cw; t += 256) {
    const int64_t i = (r0 + t / cw) * n + c0 + t % cw;
    q[i] = quant1<FMT>(C::load1(x, i), s, r, fast);
  }
}

// ---------------------------------------------------------------------------
// Tensor granularity. The reference's ABI passes one caller-zeroed int32 that
// must end up holding the amax bits (fp8_quant.cu:159-234 atomicMax-es every
// block's maximum into it). Same-address device-scope atomics serialise (one
// per workgroup took 26.7 us of a 33.7 us launch at [2048, 4096] bf16 on
// MI355X), so the maximum travels through plain stores into slots inside the
// codes buffer, in three launches:
//   fp8_tensor_partial - each of gp workgroups stores the max |x| bits of its
//                        share into its slot;
//   fp8_tensor_finish  - one workgroup reduces the slots, does the single
//                        atomicMax into the caller's int32 and stores the scale;
//   fp8_tensor_cast    - the flat cast pass (fp8_tensor_cast<kScaleWord>, which
//                        reads that scale), shared with static scales.
// Small inputs save the middle launch: the partial pass stores its maximum
// into a slot array at the start of every cast chunk (fp8_tensor_partial
// <REPLICATE>), each cast workgroup reduces the array in its own chunk, which
// no other workgroup reads or writes, before overwriting the chunk with codes,
// and cast workgroup 0 does the atomicMax and stores the scale
// (fp8_tensor_cast<kAmaxChunk>). Inputs too small for one slot array use
// fp8_tensor_amax (one workgroup) in the partial and finish's place.
//
// The caller's int32 may be null (an addition: the Python API has no use for
// it). Otherwise it ends up holding max(its initial value, amax bits) and the
// scale follows from that maximum, as in the reference. Max |x| is taken on
// non-negative fp32 bits, so integer max is float max with NaN above +inf.
// ---------------------------------------------------------------------------
constexpr int kPartialThreads = 512, kPartialUnroll = 4, kPartialMaxGroups = 512;

// Where the cast takes the dynamic scale from.
enum AmaxSource : int {
  kScaleWord = 0,  // scale_out[0], stored by fp8_tensor_finish / fp8_tensor_amax
  kAmaxSlots = 1,  // `nslots` partial maxima at `slots` (the no-allocation entry point's scratch)
  kAmaxChunk = 2,  // `nslots` partial maxima at the start of the workgroup's own chunk of codes
};

// Slot of partial workgroup p in a slot array: the slots of one XCD's
// workgroups (p % 8; workgroups are dealt to the XCDs round-robin) are
// contiguous, so each cache line of a replicated array is written from one L2.
__device__ inline int partial_slot(int p, int groups) {
  return groups % 8 == 0 ? (p % 8) * (groups / 8) + p / 8 : p;
}

// Each workgroup's max |x| bits go to partial[blockIdx.x] or, with REPLICATE,
// to its slot of each of the `chunks` slot arrays at q + c * chunk_bytes.
template <class C, bool VECTOR, bool REPLICATE = false>
__global__ __launch_bounds__(kPartialThreads) void fp8_tensor_partial(const void* __restrict__ x, int64_t total,
                                                                      uint32_t* __restrict__ partial,
                                                                      uint8_t* __restrict__ q = nullptr,
                                                                      int64_t chunk_bytes = 0, int chunks = 0) {
  constexpr int T = kPartialThreads, U = kPartialUnroll;
  __shared__ uint32_t lds[2 * (T / 64)];
  uint32_t acc = 0;
  int64_t done = 0;
  if constexpr (VECTOR) {
    const int64_t nvec = total / C::VEC;
    const u32x4* xv = static_cast<const u32x4*>(x);
    for (int64_t b = (int64_t)blockIdx.x * T * U + threadIdx.x; b < nvec; b += (int64_t)gridDim.x * T * U) {
      u32x4 v[U];
#pragma unroll
      for (int k = 0; k < U; ++k) {
        // Cached loads (not streaming): x is then more often still on chip
        // when the cast pass reads it again, 54.0 vs 57.0 us for the whole op
        // at [16384, 4096] bf16 and 13.6 vs 13.7 at [2048, 4096] on MI355X.
        if (b + k * T < nvec) v[k] = xv[b + k * T];
      }
#pragma unroll
      for (int k = 0; k < U; ++k) {
        if (b + k * T < nvec) acc = C::absmax_vec(v[k], acc);
      }
    }
    done = nvec * C::VEC;
  }
  for (int64_t i = done + (int64_t)blockIdx.x * T + threadIdx.x; i < total; i += (int64_t)gridDim.x * T) {
    acc = C::absmax1(x, i, acc);
  }
  acc = block_allreduce<T / 64>(acc, typename AmaxOp<C>::type{}, lds, 0);
  const uint32_t bits = f32_bits(C::absmax_to_float(acc));
  if constexpr (REPLICATE) {
    const int64_t off = 4 * (int64_t)partial_slot((int)blockIdx.x, (int)gridDim.x);
    for (int c = threadIdx.x; c < chunks; c += T) *reinterpret_cast<uint32_t*>(q + c * chunk_bytes + off) = bits;
  } else {
    if (threadIdx.x == 0) partial[blockIdx.x] = bits;
  }
}

// The tensor's amax into the caller's int32 (if any; `initial` is its value
// before the op) and the scale of max(initial, amax) into scale_out[0]. The
// atomicMax's result is not waited for.
template <int FMT>
__device__ inline void publish_amax(uint32_t amax_bits, int32_t initial, int32_t* amax_scratch, float* scale_out) {
  if (amax_scratch != nullptr) {
    atomicMax(amax_scratch, (int32_t)amax_bits);
    amax_bits = (uint32_t)max(initial, (int32_t)amax_bits);
  }
  scale_out[0] = scale_from_amax<FMT>(bits_f32(amax_bits));
}

template <int FMT>
__global__ __launch_bounds__(256) void fp8_tensor_finish(const uint32_t* __restrict__ partial, int n_partial,
                                                         int32_t* __restrict__ amax_scratch,
                                                         float* __restrict__ scale_out) {
  __shared__ uint32_t lds[2 * 4];
  // Only this launch writes the caller's int32, so its value now is the initial one.
  const int32_t initial = (amax_scratch != nullptr && threadIdx.x == 0) ? *amax_scratch : 0;
  uint32_t acc = 0;
  for (int i = threadIdx.x; i < n_partial; i += 256) acc = max(acc, partial[i]);
  acc = block_allreduce<4>(acc, MaxU32{}, lds, 0);
  if (threadIdx.x == 0) publish_amax<FMT>(acc, initial, amax_scratch, scale_out);
}

template <class C, int FMT, bool VECTOR>
__global__ __launch_bounds__(256) void fp8_tensor_amax(const void* __restrict__ x, int64_t total,
                                                       int32_t* __restrict__ amax_scratch,
                                                       float* __restrict__ scale_out) {
  __shared__ uint32_t lds[2 * 4];
  const int32_t initial = (amax_scratch != nullptr && threadIdx.x == 0) ? *amax_scratch : 0;
  uint32_t acc = 0;
  const int64_t stride = (int64_t)gridDim.x * 256;
  const int64_t tid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if constexpr (VECTOR) {
    const int64_t nvec = total / C::VEC;
    const u32x4* xv = static_cast<const u32x4*>(x);
    for (int64_t v = tid; v < nvec; v += stride) acc = C::absmax_vec(ld_stream(xv + v), acc);
    for (int64_t i = nvec * C::VEC + tid; i < total; i += stride) acc = C::absmax1(x, i, acc);
  } else {
    for (int64_t i = tid; i < total; i += stride) acc = C::absmax1(x, i, acc);
  }
  acc = block_allreduce<4>(acc, typename AmaxOp<C>::type{}, lds, 0);
  if (threadIdx.x == 0) publish_amax<FMT>(f32_bits(C::absmax_to_float(acc)), initial, amax_scratch, scale_out);
}

// STATIC: scale is `static_scale`; otherwise it comes from SRC. VECTOR:
// CAST_THREADS threads with CAST_UNROLL 16-byte vectors each, loaded before
// any is converted; measured on MI355X against 256 threads with one vector per
// grid-stride step and cached code stores: 32.3 vs 35.7 us at [16384, 4096]
// bf16, 248 vs 338 us at [65536, 8192].
constexpr int kCastThreads = 512, kCastUnroll = 2;
static_assert(kPartialThreads * kPartialUnroll == 2 * kCastThreads * kCastUnroll,
              "the XCD-aligned cast order takes halves of the partial pass's chunks");

// Codes bytes of one vector-path cast chunk (the first chunk of workgroup b
// starts at b times this).
template <class C>
constexpr int64_t kCastChunkBytes = (int64_t)kCastThreads * kCastUnroll * C::VEC;

// Replicated slot arrays cost gp x g scattered 4-byte stores (gp partial
// workgroups, g cast chunks), each its own cache-line write at the L2, against
// the one launch they save. Measured per op on MI355X (bf16, graph-replayed,
// with the caller's zero-fill): [512, 4096] 8.7 vs 9.4 us (32 K stores),
// [1024, 4096] 10.0 vs 10.6 us (128 K), [2048, 4096] 13.7 vs 12.5 us (512 K),
// [4096, 4096] 24.2 vs 19.1 us (1 M).
constexpr int64_t kMaxReplicatedSlots = 1 << 17;

template <class C, int FMT, bool STATIC, bool VECTOR, int SRC = kScaleWord>
__global__ __launch_bounds__(VECTOR ? kCastThreads : 256) void fp8_tensor_cast(
    const void* __restrict__ x, uint8_t* __restrict__ q, float* __restrict__ scale_out,
    int32_t* __restrict__ amax_scratch, float static_scale, int64_t total, bool xcd_aligned = false,
    const uint32_t* __restrict__ slots = nullptr, int nslots = 0) {
  constexpr int T = VECTOR ? kCastThreads : 256;
  constexpr int U = VECTOR ? kCastUnroll : 1;
  static_assert(VECTOR || SRC != kAmaxChunk, "chunk slot arrays belong to the vector path");
  const int64_t nvec = VECTOR ? total / C::VEC : 0;
  const u32x4* xv = static_cast<const u32x4*>(x);
  int64_t bid = blockIdx.x;
  if constexpr (!STATIC) {
    // After the partial pass. When both passes cover x in one round of
    // workgroups (the partial's grid a multiple of 8, this one a multiple
    // of 16), workgroup 8a + c re-reads a half of partial chunk
    // 8 (a / 2) + c: workgroups are dealt to the 8 XCDs round-robin, so
    // that half is re-read by the XCD that read it (12.4-12.7 vs 13.4-13.6 us
    // for the whole reference-ABI op at [2048, 4096] bf16 on MI355X; the
    // FETCH_SIZE counter shows the re-read still leaves the L2, so the gain
    // is on the path beyond it). Otherwise the chunks are walked last-first,
    // starting on the most recently read part of x.
    if (xcd_aligned) {
      const int64_t a = blockIdx.x / 8, c = blockIdx.x % 8;
      bid = 2 * (8 * (a / 2) + c) + (a % 2);
    } else {
      bid = gridDim.x - 1 - blockIdx.x;
    }
  }
  int64_t b = bid * T * U + threadIdx.x;
  u32x4 raw[U];
  auto load = [&](int64_t b0) {
#pragma unroll
    for (int k = 0; k < U; ++k) {
      if (b0 + k * T < nvec) raw[k] = ld_stream(xv + b0 + k * T);
    }
  };
  if constexpr (VECTOR) load(b);
  float s;
  if constexpr (STATIC) {
    s = static_scale;
    // The static scale goes to scale_out[0] when the caller passed a scale word.
    if (scale_out != nullptr && blockIdx.x == 0 && threadIdx.x == 0) scale_out[0] = s;
  } else if constexpr (SRC == kScaleWord) {
    s = scale_out[0];
  } else {
    // The maximum of the slots (loaded after this workgroup's first vectors),
    // and for chunk slot arrays the caller's int32, read before workgroup 0's
    // atomicMax (its initial value) or after it (the same overall maximum).
    __shared__ uint32_t lds[2 * (T / 64)];
    const uint32_t* sl = slots;
    if constexpr (SRC == kAmaxChunk) sl = reinterpret_cast<const uint32_t*>(q + bid * kCastChunkBytes<C>);
    const bool word = SRC == kAmaxChunk && amax_scratch != nullptr;
    const int32_t seen = word ? __hip_atomic_load(amax_scratch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
    uint32_t m = 0;
    for (int i = threadIdx.x; i < nslots; i += T) m = max(m, sl[i]);
    m = block_allreduce<T / 64>(m, MaxU32{}, lds, 0);
    s = scale_from_amax<FMT>(bits_f32(word ? (uint32_t)max(seen, (int32_t)m) : m));
    if (blockIdx.x == 0 && threadIdx.x == 0) {
      if (word) atomicMax(amax_scratch, (int32_t)m);
      scale_out[0] = s;
    }
  }
  const float r = 1.0f / s;
  // A dynamic scale s = amax / FP8_MAX (or the clamp) keeps |x| * (1/s) within
  // the conversion's verified range, so only s and 1/s need checking.
  const bool fast_t = fast_path_ok<FMT>(s, r, 0.0f);
  int64_t done = 0;
  if constexpr (VECTOR) {
    const int64_t stride = (int64_t)gridDim.x * T * U;
    for (; b < nvec; b += stride) {
      if (b != bid * T * U + threadIdx.x) load(b);
#pragma unroll
      for (int k = 0; k < U; ++k) {
        const int64_t v = b + k * T;
        if (v < nvec) {
          bool fast = fast_t;
          if constexpr (STATIC) fast = fast_path_ok<FMT>(s, r, C::absmax_to_float(C::absmax_vec(raw[k], 0)));
          quant_vec<C, FMT>(raw[k], s, r, fast, q, v * C::VEC);
        }
      }
    }
    done = nvec * C::VEC;
  }
  const int64_t stride = (int64_t)gridDim.x * T;
  for (int64_t i = done + (int64_t)blockIdx.x * T + threadIdx.x; i < total; i += stride) {
    const float v = C::load1(x, i);
    bool fast = fast_t;
    if constexpr (STATIC) fast = fast_path_ok<FMT>(s, r, __builtin_fabsf(v));
    q[i] = quant1<FMT>(v, s, r, fast);
  }
}

// Cast grid for a dynamic-scale tensor after the partial pass over `gp`
// workgroups, and whether the XCD-aligned chunk order applies (both passes
// one round of workgroups, grids multiples of 8 and 16).
inline unsigned tensor_cast_grid(int64_t nvec, unsigned gp, bool* xcd_aligned) {
  const unsigned g = flat_grid(nvec, kCastThreads * kCastUnroll, 1 << 20);
  *xcd_aligned = nvec <= (int64_t)kPartialMaxGroups * kPartialThreads * kPartialUnroll && g == 2 * gp &&
                 gp % 8 == 0;
  return g;
}

// Row-length buckets of the register-resident token kernel.
template <class C, int FMT>
int32_t launch_token(const void* x, uint8_t* q, float* scale, int64_t m, int64_t n,
                     hipStream_t st) {
  const bool vec_ok = (n % C::VEC == 0) && host_aligned(x, 16) && host_aligned(q, C::VEC);
  const int64_t nvec = n / C::VEC;
  const unsigned g = row_grid(m);
  auto run = [&](auto shape) {
    using S = decltype(shape);
    fp8_token_resident<C, FMT, S::kThreads, S::kItems><<<g, S::kThreads, 0, st>>>(x, q, scale, m, n);
  };
  // 16-byte rows (f16 / bf16) from a sweep over THREADS 64..1024 x ITEMS
  // 1..4 on MI355X at 8192 bf16 rows of 2048..28672 elements (graph-replayed,
  // 2 GiB rotation): three or four vectors per thread from 2560 elements on,
  // e.g. 21.4 us for 256 x 3 at 5120 against 24.2 for 512 x 2, 39.8 for
  // 512 x 3 at 10240 against 49.0 for 1024 x 2, 63.2 for 512 x 4 at 16384
  // against 66.3 for 1024 x 2; 1024 x 6 at 36864, 74.5 against 91.3 for
  // 1024 x 8. fp32 rows keep two vectors per thread up to 1024 x 2 (27.4
  // against 28.8 us at [8192, 4096] for 256 x 4).
  bool done = false;
  if constexpr (C::VEC == 8) {
    done = vec_ok && pick_row_shape<RowShape<64, 1>, RowShape<64, 2>, RowShape<128, 2>, RowShape<128, 3>,
                                    RowShape<256, 2>, RowShape<256, 3>, RowShape<256, 4>, RowShape<512, 3>,
                                    RowShape<512, 4>, RowShape<1024, 3>, RowShape<1024, 4>, RowShape<1024, 6>,
                                    RowShape<1024, 8>>(nvec, run);
  } else {
    done = vec_ok && pick_row_shape<RowShape<64, 1>, RowShape<64, 2>, RowShape<128, 2>, RowShape<256, 2>,
                                    RowShape<512, 2>, RowShape<1024, 2>, RowShape<1024, 4>,
                                    RowShape<1024, 8>>(nvec, run);
  }
  if (!done) fp8_token_generic<C, FMT><<<g, 256, 0, st>>>(x, q, scale, m, n);
  return launch_status();
}

// ---------------------------------------------------------------------------
// Tensor granularity in one read of x (fp8_tensor_onepass). Each workgroup of
// 1024 threads keeps its share of x in registers (U 16-byte vectors per
// thread) and takes its max |x|. Workgroup 0 is the reducer: every other
// workgroup b stores its maximum into slot b and then waits for the scale;
// workgroup 0 waits until every slot is filled, reduces them with its own
// maximum, does the caller's atomicMax (if any), and publishes the scale in
// the caller's `scale` word. Every workgroup then converts what it holds.
//
// All of the exchange lives in memory the call owns: the slots are words
// 1 .. g-1 of the codes buffer, inside workgroup 0's own share of the codes
// (the launcher checks 4 g <= that share), and the result is the scale
// output. fp8_onepass_init (one small launch on the same stream, before the
// one-pass launch, for grids of two or more) marks the slots empty
// (kSlotEmpty, never the bits of a maximum |x|: those have the sign bit
// clear) and the scale unpublished (kScaleEmpty, a signalling NaN, never a
// computed scale: arithmetic on a NaN quiets it). Nothing persists between
// calls, so calls on different streams may overlap freely, and graph replays
// need nothing cleared. Each slot is written once, before its workgroup
// waits, so once workgroup 0 has seen every slot no slot is written again
// and its codes may land on them.
//
// Every shared word is written and read only by agent-scope atomics, which
// gfx950 performs beyond the per-XCD L2s, and a slot's store completes
// before its workgroup starts to wait.
//
// Waiting needs the grid resident at once: the launcher sizes it to the
// occupancy the runtime reports for the device. A workgroup other than 0
// whose wait runs past its poll limit (other work holding CUs) reads all of
// x and takes the maximum itself (and the caller's int32), then converts:
// the same scale, so the result never depends on residency. Those
// workgroups leave, so the ones not yet running get CUs and fill their
// slots: workgroup 0's wait, the only one without a limit, always ends.
// ---------------------------------------------------------------------------
constexpr int kOnePassThreads = 1024;
constexpr uint32_t kSlotEmpty = 0xffffffffu;
constexpr uint32_t kScaleEmpty = 0x7f800001u;
// Polls (about 1 us each: a short sleep and a load from beyond the L2) a
// waiting workgroup makes before it reads all of x itself; the exchange
// itself takes about 3 us.
constexpr int kDefaultPollLimit = 2048;

__device__ inline uint32_t agent_load(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void agent_store(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until this thread's memory operations have completed (s_waitcnt with
// every counter at zero); the compiler moves no memory access across it.
__device__ inline void wait_memory_ops() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

__global__ __launch_bounds__(256) void fp8_onepass_init(uint32_t* __restrict__ slots, int groups,
                                                        float* __restrict__ scale) {
  for (int i = 1 + (int)threadIdx.x; i < groups; i += 256) agent_store(slots + i, kSlotEmpty);
  if (threadIdx.x == 0) agent_store(reinterpret_cast<uint32_t*>(scale), kScaleEmpty);
}

// The scale of amax bits m together with the caller's int32 (if any; its
// value before or after the reducer's atomicMax gives the same maximum).
template <int FMT>
__device__ inline float tensor_scale(uint32_t m, const int32_t* amax_scratch) {
  if (amax_scratch != nullptr) {
    const int32_t seen = (int32_t)agent_load(reinterpret_cast<const uint32_t*>(amax_scratch));
    m = (uint32_t)max(seen, (int32_t)m);
  }
  return scale_from_amax<FMT>(bits_f32(m));
}

// U 16-byte vectors per thread and at least WPE waves per SIMD (the register
// budget: 512 / WPE VGPRs, no spills); requires 16-byte aligned x,
// VEC-aligned q, total % VEC == 0, 4 * gridDim.x <= 1024 * U * VEC (the slots
// fit in workgroup 0's codes) and fp8_onepass_init on the same stream first
// when gridDim.x > 1.
//
// SPILL: inputs larger than the grid holds. Workgroup i takes the `chunk`
// vectors from i * chunk (chunk a multiple of the workgroup size, at least
// U per thread), holds the first U per thread in registers as above and
// streams the rest twice: once, with cached loads, into its maximum, and
// again after the exchange, last-read first, converting. x is read once plus
// the part that did not fit, instead of twice. Same-run A/B on MI355X
// against the two passes (bf16, no amax word): [4097, 8200] 21.1 vs 28.2 us,
// [8192, 8192] 47.4 vs 51.1, [32768, 4096] 94.2 vs 98.9, [65536, 4096] 200.3
// vs 202.2; the re-read in ascending order measured 1-4 % slower up to
// 256 MiB, and 8 vectors per thread held with 8 streamed 3-15 % slower.
constexpr int kSpillUnroll = 4;

template <class C, int FMT, int U, int WPE, bool SPILL = false>
__global__ __launch_bounds__(kOnePassThreads, WPE) void fp8_tensor_onepass(
    const void* __restrict__ x, uint8_t* __restrict__ q, float* __restrict__ scale_out,
    int32_t* __restrict__ amax_scratch, int64_t nvec, int poll_limit, int64_t chunk) {
  constexpr int T = kOnePassThreads, NW = T / 64, R = kSpillUnroll;
  __shared__ uint32_t lds[2 * NW];
  __shared__ uint32_t scale_s, late_s;
  const u32x4* xv = static_cast<const u32x4*>(x);
  uint32_t* slots = reinterpret_cast<uint32_t*>(q);
  uint32_t* scale_bits = reinterpret_cast<uint32_t*>(scale_out);
  const int64_t c0 = (int64_t)blockIdx.x * (SPILL ? chunk : (int64_t)T * U);
  const int64_t c1 = SPILL ? min(c0 + chunk, nvec) : nvec;  // the streamed part: [c0 + T * U, c1)
  const int64_t b0 = c0 + threadIdx.x;
  const u32x4 zero = {0u, 0u, 0u, 0u};
  u32x4 raw[U];
#pragma unroll
  for (int k = 0; k < U; ++k) {
    if (b0 + k * T < nvec) raw[k] = ld_stream(xv + b0 + k * T);
  }
  uint32_t acc = 0;
  if constexpr (SPILL) {
    // Out-of-chunk lanes read the chunk's first vector and count zeros.
    for (int64_t v = b0 + (int64_t)T * U; v < c1; v += (int64_t)T * R) {
      u32x4 t[R];
#pragma unroll
      for (int j = 0; j < R; ++j) t[j] = xv[v + j * T < c1 ? v + j * T : c0];
#pragma unroll
      for (int j = 0; j < R; ++j) acc = C::absmax_vec(v + j * T < c1 ? t[j] : zero, acc);
    }
  }
#pragma unroll
  for (int k = 0; k < U; ++k) {
    if (b0 + k * T < nvec) acc = C::absmax_vec(raw[k], acc);
  }
  const uint32_t mine =
      f32_bits(C::absmax_to_float(block_allreduce<NW>(acc, typename AmaxOp<C>::type{}, lds, 0)));
  if (blockIdx.x == 0) {
    uint32_t m = mine;
    for (unsigned i = 1 + threadIdx.x; i < gridDim.x; i += T) {
      uint32_t v = agent_load(slots + i);
      while (v == kSlotEmpty) {
        __builtin_amdgcn_s_sleep(1);
        v = agent_load(slots + i);
      }
      m = max(m, v);
    }
    m = block_allreduce<NW>(m, MaxU32{}, lds, 1);
    if (threadIdx.x == 0) {
      if (amax_scratch != nullptr) m = (uint32_t)max(atomicMax(amax_scratch, (int32_t)m), (int32_t)m);
      const uint32_t sb = f32_bits(scale_from_amax<FMT>(bits_f32(m)));
      agent_store(scale_bits, sb);
      scale_s = sb;
    }
  } else {
    if (threadIdx.x == 0) {
      agent_store(slots + blockIdx.x, mine);
      wait_memory_ops();
      uint32_t v = agent_load(scale_bits);
      for (int i = 0; v == kScaleEmpty && i < poll_limit; ++i) {
        __builtin_amdgcn_s_sleep(2);
        v = agent_load(scale_bits);
      }
      scale_s = v;
      late_s = v == kScaleEmpty;
    }
    __syncthreads();
    if (late_s) {
      // The wait ran past its limit: the maximum over all of x, read by this workgroup.
      uint32_t a = 0;
      for (int64_t v = threadIdx.x; v < nvec; v += T) a = C::absmax_vec(ld_stream(xv + v), a);
      const uint32_t m = f32_bits(C::absmax_to_float(block_allreduce<NW>(a, typename AmaxOp<C>::type{}, lds, 1)));
      if (threadIdx.x == 0) scale_s = f32_bits(tensor_scale<FMT>(m, amax_scratch));
    }
  }
  __syncthreads();
  const float s = bits_f32(scale_s);
  const float r = 1.0f / s;
  // s >= amax / FP8_MAX keeps |x| * (1/s) within the conversion's verified
  // range, so only s and 1/s need checking.
  const bool fast = fast_path_ok<FMT>(s, r, 0.0f);
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const int64_t v = b0 + k * T;
    if (v < nvec) quant_vec<C, FMT>(raw[k], s, r, fast, q, v * C::VEC);
  }
  if constexpr (SPILL) {
    // Last-read first: the end of the streamed part is likeliest still on chip.
    const int64_t steps = (c1 - (c0 + (int64_t)T * U) + (int64_t)T * R - 1) / ((int64_t)T * R);
    for (int64_t st = steps - 1; st >= 0; --st) {
      const int64_t v = b0 + (int64_t)T * U + st * (int64_t)T * R;
      u32x4 t[R];
#pragma unroll
      for (int j = 0; j < R; ++j) t[j] = ld_stream(xv + (v + j * T < c1 ? v + j * T : c0));
#pragma unroll
      for (int j = 0; j < R; ++j) {
        if (v + j * T < c1) quant_vec<C, FMT>(t[j], s, r, fast, q, (v + j * T) * C::VEC);
      }
    }
  }
}

constexpr int kMaxDevices = 64;
std::mutex onepass_mu;
std::atomic<int> poll_limit{kDefaultPollLimit};

// Workgroups of fp8_tensor_onepass<C, FMT, U, WPE> the current device holds
// at once (occupancy per CU x CUs; 0 if unknown).
template <class C, int FMT, int U, int WPE, bool SPILL = false>
int onepass_groups() {
  static int groups[kMaxDevices] = {};  // per instantiation; -1 = the query failed
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    return 0;
  }
  std::lock_guard<std::mutex> lock(onepass_mu);
  if (groups[dev] == 0) {
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fp8_tensor_onepass<C, FMT, U, WPE, SPILL>,
                                                     kOnePassThreads, 0) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
      (void)hipGetLastError();
      groups[dev] = -1;
    } else {
      groups[dev] = per_cu * cus > 0 ? per_cu * cus : -1;
    }
  }
  return std::max(groups[dev], 0);
}

// Inputs from this many vectors up take the one-pass form when it fits;
// below it (and above one workgroup's worth) the init launch and the
// exchange cost more than the second read of x saves. Measured on MI355X,
// bf16 rows of 4096, graph-replayed, one-pass against the two-pass forms
// (reference ABI with the caller's zero-fill / no amax word): [1024, 4096]
// 9.73 / 7.78 against 9.32 / 7.50 us; [2048, 4096] (2^20 vectors) 11.54 /
// 9.58 against 11.67 / 9.92; [4096, 4096] 14.83 / 12.92 against 18.52 /
// 16.67; [8192, 4096] 24.04 / 22.12 against 29.66 / 27.76.
constexpr int64_t kOnePassMinVecs = int64_t(1) << 20;
constexpr int64_t kOnePassSoloVecs = (int64_t)kOnePassThreads * 2;  // one workgroup: no exchange

// Launches the one-pass form where it pays: inputs one workgroup holds
// (no exchange and no init launch: the fewest vectors per thread that
// hold x), and inputs of at least kOnePassMinVecs vectors whose grid the
// device holds at once, with the fewest vectors per thread that allow it:
// U = 1, 2 or 4 at two workgroups per CU (64 VGPRs), then U = 16 at one
// (128 VGPRs), after fp8_onepass_init; larger inputs take the SPILL form
// (U = 16 held, the rest of each chunk streamed). False otherwise.
template <class C, int FMT>
bool launch_onepass(const void* x, uint8_t* q, float* scale, int32_t* amax_scratch, int64_t nvec,
                    hipStream_t st) {
  if (nvec > kOnePassSoloVecs && nvec < kOnePassMinVecs) return false;
  const int polls = poll_limit.load(std::memory_order_relaxed);
  auto attempt = [&](auto u, auto wpe) {
    constexpr int U = decltype(u)::value, WPE = decltype(wpe)::value;
    constexpr int64_t per_group = (int64_t)kOnePassThreads * U;
    const int64_t g = (nvec + per_group - 1) / per_group;
    if (nvec <= kOnePassSoloVecs ? g > 1 : (g > onepass_groups<C, FMT, U, WPE>() || 4 * g > per_group * C::VEC)) {
      return false;
    }
    if (g > 1) {
      fp8_onepass_init<<<1, 256, 0, st>>>(reinterpret_cast<uint32_t*>(q), (int)g, scale);
    }
    fp8_tensor_onepass<C, FMT, U, WPE><<<(unsigned)g, kOnePassThreads, 0, st>>>(x, q, scale, amax_scratch, nvec,
                                                                              polls, per_group);
    return true;
  };
  if (attempt(IntC<1>{}, IntC<8>{}) || attempt(IntC<2>{}, IntC<8>{}) || attempt(IntC<4>{}, IntC<8>{}) ||
      attempt(IntC<16>{}, IntC<4>{})) {
    return true;
  }
  if (nvec <= kOnePassSoloVecs) return false;
  // Beyond what the grid holds: every resident workgroup takes an equal
  // chunk, 16 vectors per thread of it in registers and the rest streamed.
  constexpr int U = 16, WPE = 4;
  const int64_t groups = onepass_groups<C, FMT, U, WPE, true>();
  if (groups <= 0 || 4 * groups > (int64_t)kOnePassThreads * U * C::VEC) return false;
  int64_t chunk = (nvec + groups - 1) / groups;
  chunk = (chunk + kOnePassThreads - 1) / kOnePassThreads * kOnePassThreads;
  if (chunk < (int64_t)kOnePassThreads * U) return false;  // the held form fits: not reached
  const int64_t g = (nvec + chunk - 1) / chunk;
  fp8_onepass_init<<<1, 256, 0, st>>>(reinterpret_cast<uint32_t*>(q), (int)g, scale);
  fp8_tensor_onepass<C, FMT, U, WPE, true><<<(unsigned)g, kOnePassThreads, 0, st>>>(x, q, scale, amax_scratch,
                                                                                    nvec, polls, chunk);
  return true;
}

// The no-allocation entry point's two-pass form (inputs between one
// workgroup's worth and 2^20 vectors, or unaligned) keeps its partial maxima in `scratch`, a file-scope
// device array of kPartialMaxGroups words (2 KiB), one per GPU, held until
// the process ends. Each call writes every slot it reads, so nothing needs
// clearing; calls of this form that overlap on one GPU race on the array.
constexpr int kScratchWords = kPartialMaxGroups;
static __device__ __align__(256) uint32_t scratch[kScratchWords];
std::mutex scratch_mu;
uint32_t* scratch_dev[kMaxDevices] = {};

// The current device's address of `scratch`, looked up once per device. The
// host-side name of the array is only a handle for the runtime: kernels are
// given this address.
int32_t scratch_address(uint32_t** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int32_t)e;
  if (dev < 0 || dev >= kMaxDevices) return (int32_t)hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int32_t)e;
    scratch_dev[dev] = static_cast<uint32_t*>(p);
  }
  *out = scratch_dev[dev];
  return (int32_t)hipSuccess;
}

}  // namespace
}  // namespace cck

using namespace cck;

extern "C" int32_t launch_fp8_quant_token_fwd(const void* x, uint8_t* x_fp8, float* scale, int64_t m,
                                              int64_t n, int32_t dtype, int32_t fp8_format,
                                              void* stream) {
  if (m <= 0 || n <= 0) return (int32_t)hipSuccess;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_codec(dtype, [&](auto codec) {
    using C = decltype(codec);
    return with_fp8(fp8_format, [&](auto f) {
      return launch_token<C, decltype(f)::value>(x, x_fp8, scale, m, n, st);
    });
  });
}

extern "C" int32_t launch_fp8_quant_block_fwd(const void* x, uint8_t* x_fp8, float* scale, int64_t m,
                                              int64_t n, int32_t dtype, int32_t fp8_format,
                                              void* stream) {
  if (m <= 0 || n <= 0) return (int32_t)hipSuccess;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t nrb = (m + kTile - 1) / kTile, ncb = (n + kTile - 1) / kTile;
  if (nrb > 65535 || ncb > (int64_t)0x7fffffff) return (int32_t)hipErrorInvalidValue;
  const dim3 grid((unsigned)ncb, (unsigned)nrb);
  return with_codec(dtype, [&](auto codec) {
    using C = decltype(codec);
    return with_fp8(fp8_format, [&](auto f) {
      constexpr int FMT = decltype(f)::value;
      const bool vec_ok = (n % C::VEC == 0) && host_aligned(x, 16) && host_aligned(x_fp8, C::VEC);
      const bool rsrc_ok = (int64_t)kTile * n * C::kBytes <= 0x7fffffff;
      if constexpr (C::VEC == 8) {
        if (vec_ok && rsrc_ok && nrb * ncb >= kBlockPairMinTiles) {
          // Two tiles side by side per 1024-thread workgroup: 128.0 vs 131.0 us
          // at [32768, 8192] bf16, 254.5 vs 265.1 us at [65536, 8192]; no gain
          // below 16384 tiles (65.7 vs 66.3 us at [16384, 8192] for one tile).
          // fp32 tiles (8 vectors per thread) do not fit two to a workgroup's
          // registers and keep one.
          const dim3 grid2((unsigned)((ncb + 1) / 2), (unsigned)nrb);
          fp8_block_resident<C, FMT, 512, true, 2><<<grid2, 1024, 0, st>>>(x, x_fp8, scale, m, n);
          return launch_status();
        }
      }
      if (vec_ok && rsrc_ok && nrb * ncb <= kBlockSplitMaxTiles) {
        // All tiles resident at once: issuing every load of a tile before
        // its max measured 6.44 vs 6.56 us at [2048, 4096] bf16 on MI355X,
        // but 35.9 vs 35.1 us at [16384, 4096], where tiles run in rounds.
        fp8_block_resident<C, FMT, 512, true, 1, true><<<grid, 512, 0, st>>>(x, x_fp8, scale, m, n);
      } else if (vec_ok && rsrc_ok) {
        fp8_block_resident<C, FMT, 512, true, 1><<<grid, 512, 0, st>>>(x, x_fp8, scale, m, n);
      } else if (vec_ok) {
        fp8_block_resident<C, FMT, 512, false, 1><<<grid, 512, 0, st>>>(x, x_fp8, scale, m, n);
      } else {
        fp8_block_generic<C, FMT><<<grid, 256, 0, st>>>(x, x_fp8, scale, m, n);
      }
      return launch_status();
    });
  });
}

extern "C" int32_t launch_fp8_quant_tensor_fwd(const void* x, uint8_t* x_fp8, float* scale,
                                               int32_t* amax_scratch, int64_t m, int64_t n,
                                               int32_t dtype, int32_t fp8_format, void* stream) {
  if (m <= 0 || n <= 0) return (int32_t)hipSuccess;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t total = m * n;
  return with_codec(dtype, [&](auto codec) {
    using C = decltype(codec);
    return with_fp8(fp8_format, [&](auto f) {
      constexpr int FMT = decltype(f)::value;
      const bool vec_ok = host_aligned(x, 16) && host_aligned(x_fp8, C::VEC);
      const int64_t nvec = total / C::VEC;
      // One read of x where the registers of a resident grid hold it.
      if (vec_ok && total % C::VEC == 0 && launch_onepass<C, FMT>(x, x_fp8, scale, amax_scratch, nvec, st)) {
        return launch_status();
      }
      const unsigned gp = vec_ok ? flat_grid(nvec, kPartialThreads * kPartialUnroll, kPartialMaxGroups)
                                 : flat_grid(total, kPartialThreads * 16, kPartialMaxGroups);
      if (vec_ok) {
        bool aligned = false;
        const unsigned g = tensor_cast_grid(nvec, gp, &aligned);
        // Every cast chunk, the last one included, holds a slot array.
        const int64_t cb = kCastChunkBytes<C>;
        if ((int64_t)gp * g <= kMaxReplicatedSlots && nvec * C::VEC - (int64_t)(g - 1) * cb >= 4 * (int64_t)gp) {
          fp8_tensor_partial<C, true, true><<<gp, kPartialThreads, 0, st>>>(x, total, nullptr, x_fp8, cb, (int)g);
          fp8_tensor_cast<C, FMT, false, true, kAmaxChunk><<<g, kCastThreads, 0, st>>>(
              x, x_fp8, scale, amax_scratch, 0.0f, total, aligned, nullptr, (int)gp);
          return launch_status();
        }
      }
      // One slot array: 4-byte words at the first aligned word of the codes buffer.
      const uintptr_t slots = (reinterpret_cast<uintptr_t>(x_fp8) + 3) & ~uintptr_t(3);
      uint32_t* partial = reinterpret_cast<uint32_t*>(slots);
      const bool slots_fit = (int64_t)(slots - reinterpret_cast<uintptr_t>(x_fp8)) + 4 * (int64_t)gp <= total;
      if (slots_fit) {
        if (vec_ok) {
          fp8_tensor_partial<C, true><<<gp, kPartialThreads, 0, st>>>(x, total, partial);
        } else {
          fp8_tensor_partial<C, false><<<gp, kPartialThreads, 0, st>>>(x, total, partial);
        }
        fp8_tensor_finish<FMT><<<1, 256, 0, st>>>(partial, (int)gp, amax_scratch, scale);
      } else if (vec_ok) {
        fp8_tensor_amax<C, FMT, true><<<1, 256, 0, st>>>(x, total, amax_scratch, scale);
      } else {
        fp8_tensor_amax<C, FMT, false><<<1, 256, 0, st>>>(x, total, amax_scratch, scale);
      }
      if (vec_ok) {
        bool aligned = false;
        const unsigned g = tensor_cast_grid(nvec, slots_fit ? gp : 0u, &aligned);
        fp8_tensor_cast<C, FMT, false, true><<<g, kCastThreads, 0, st>>>(x, x_fp8, scale, nullptr, 0.0f, total,
                                                                          aligned);
      } else {
        const unsigned g = flat_grid(nvec, 256, 2048);
        fp8_tensor_cast<C, FMT, false, false><<<g, 256, 0, st>>>(x, x_fp8, scale, nullptr, 0.0f, total);
      }
      return launch_status();
    });
  });
}

extern "C" int32_t launch_fp8_quant_static_fwd(const void* x, uint8_t* x_fp8, float scale, float* scale_out,
                                               int64_t m, int64_t n, int32_t dtype, int32_t fp8_format,
                                               void* stream) {
  if (m <= 0 || n <= 0) return (int32_t)hipSuccess;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t total = m * n;
  return with_codec(dtype, [&](auto codec) {
    using C = decltype(codec);
    return with_fp8(fp8_format, [&](auto f) {
      constexpr int FMT = decltype(f)::value;
      const bool vec_ok = host_aligned(x, 16) && host_aligned(x_fp8, C::VEC);
      if (vec_ok) {
        const unsigned g = flat_grid(total / C::VEC, kCastThreads * kCastUnroll, 1 << 20);
        fp8_tensor_cast<C, FMT, true, true><<<g, kCastThreads, 0, st>>>(x, x_fp8, scale_out, nullptr, scale, total);
      } else {
        const unsigned g = flat_grid(total / C::VEC, 256, 8192);
        fp8_tensor_cast<C, FMT, true, false><<<g, 256, 0, st>>>(x, x_fp8, scale_out, nullptr, scale, total);
      }
      return launch_status();
    });
  });
}

extern "C" int32_t launch_fp8_quant_tensor_noalloc_fwd(const void* x, uint8_t* x_fp8, float* scale, int64_t m,
                                                       int64_t n, int32_t dtype, int32_t fp8_format,
                                                       void* stream) {
  if (m <= 0 || n <= 0) return (int32_t)hipSuccess;
  if (m > INT64_MAX / n) return (int32_t)hipErrorInvalidValue;  // m * n does not fit int64
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t total = m * n;
  return with_codec(dtype, [&](auto codec) {
    using C = decltype(codec);
    return with_fp8(fp8_format, [&](auto f) {
      constexpr int FMT = decltype(f)::value;
      uint32_t* scr = nullptr;
      const int32_t rc = scratch_address(&scr);
      if (rc != 0) return rc;
      const bool vec_ok = host_aligned(x, 16) && host_aligned(x_fp8, C::VEC);
      if (vec_ok && total % C::VEC == 0 && launch_onepass<C, FMT>(x, x_fp8, scale, nullptr, total / C::VEC, st)) {
        return launch_status();
      }
      if (vec_ok) {
        const unsigned gp = flat_grid(total / C::VEC, kPartialThreads * kPartialUnroll, kPartialMaxGroups);
        fp8_tensor_partial<C, true><<<gp, kPartialThreads, 0, st>>>(x, total, scr);
        bool aligned = false;
        const unsigned g = tensor_cast_grid(total / C::VEC, gp, &aligned);
        fp8_tensor_cast<C, FMT, false, true, kAmaxSlots><<<g, kCastThreads, 0, st>>>(x, x_fp8, scale, nullptr, 0.0f, total,
                                                                                aligned, scr, (int)gp);
      } else {
        const unsigned gp = flat_grid(total, kPartialThreads * 16, kPartialMaxGroups);
        fp8_tensor_partial<C, false><<<gp, kPartialThreads, 0, st>>>(x, total, scr);
        const unsigned g = flat_grid(total / C::VEC, 256, 2048);
        fp8_tensor_cast<C, FMT, false, false, kAmaxSlots><<<g, 256, 0, st>>>(x, x_fp8, scale, nullptr, 0.0f, total, false,
                                                                        scr, (int)gp);
      }
      return launch_status();
    });
  });
}

extern "C" int32_t cck_fp8_tensor_noalloc_poll_limit(int32_t polls) {
  return polls < 0 ? cck::poll_limit.load() : cck::poll_limit.exchange(polls);
}
