// Fused residual-add + RMSNorm, optionally fused with FP8 quantisation of the
// normalised output, for gfx950.
//
// Semantics follow the eager oracle's rounding points exactly
// (baselines/rmsnorm_residual.py:123-136):
//   residual_out = T(x + residual)                       (rounded to storage)
//   variance     = sum(float(residual_out)^2) / cols     (fp32, in torch-CPU's
//                                                         summation order)
//   inv          = 1 / sqrt(variance + eps)              (both correctly rounded)
//   y            = T( T(float(residual_out) * inv) * weight )
// so y equals the eager y bit for bit. The FP8 variant quantises y (as stored
// in T) per row (dynamic, the baselines/fp8_quant.py:162-178 formula applied
// per token) or with a static scale, and does not write y itself.
//
// Design: one workgroup per row; each thread keeps its ITEMS 16-byte vectors
// of residual_out in registers between the sum-of-squares reduction and the
// normalisation, so x and residual are read from HBM exactly once and
// residual_out / y (or the FP8 codes) written once.
#include "aten_sum.hpp"
#include "launch.hpp"

namespace cck {
namespace {

#pragma clang fp contract(off)

// Cache policies of the row stores, per MODE (below), measured on MI355X
// against NT on both streams at the config shapes:
//   MODE 0, [8192, 4096] bf16: residual_out SC1|NT and y SC1, 43.7 vs 44.1-44.7 us;
//   MODE 1, [16384, 4096]: NT on both (every SC1 combination 0.3-1 % slower);
//   MODE 2, [16384, 4096]: SC1|NT on both, 74.4 vs 75.4 us.
constexpr int ro_store_policy(int mode) { return mode == 1 ? kPolNT : (kPolSC1 | kPolNT); }
constexpr int out_store_policy(int mode) {
  return mode == 0 ? kPolSC1 : mode == 1 ? kPolNT : (kPolSC1 | kPolNT);
}

// f[i] <- T(f[i] * inv) * w[i]  (the product is rounded by the caller's store).
template <class C>
__device__ inline void scale_round_mul(float (&f)[C::VEC], float inv, const float (&w)[C::VEC]) {
#pragma unroll
  for (int i = 0; i < C::VEC; ++i) f[i] = f[i] * inv;
#pragma unroll
  for (int i = 0; i < C::VEC; i += 2) C::round2(f[i], f[i + 1]);
#pragma unroll
  for (int i = 0; i < C::VEC; ++i) f[i] = f[i] * w[i];
}

// MODE: 0 = write y in T; 1 = FP8 codes with a per-row dynamic scale;
// 2 = FP8 codes with a static scale. One row per workgroup (rows beyond the
// grid limit loop with a stride of gridDim.x). A persistent grid (a few
// workgroups per CU, each prefetching its next row while reducing the
// current one) measured about 3 % slower on MI355X than a workgroup per row.
//
// FULL: the row is exactly THREADS * ITEMS vectors and a whole number of
// 512-addend regions (bf16 / fp16 at 4096 columns: configs 2 and 5a), so the
// row length, the per-vector bounds checks and the whole summation plan are
// compile-time constants. Measured on MI355X at [16384, 4096] bf16,
// per-token FP8: see the launcher.
template <class C, int THREADS, int ITEMS, int MODE, int FMT, bool FULL>
__global__ __launch_bounds__(THREADS) void rmsnorm_resident(
    const void* __restrict__ x, const void* __restrict__ res, const void* __restrict__ w,
    void* __restrict__ y, uint8_t* __restrict__ yq, float* __restrict__ scale,
    void* __restrict__ ro, int64_t rows, int64_t cols_arg, float eps, float static_scale) {
  constexpr int NW = THREADS / 64;
  constexpr int VEC = C::VEC;
  constexpr int NREG = (THREADS * ITEMS * VEC + kRegionAddends - 1) / kRegionAddends;
  __shared__ uint32_t lds[2 * NW];
  using RowSum = ResidentRowSum<VEC, THREADS, ITEMS, FULL>;
  __shared__ float sum_stage[RowSum::kStageFloats];
  __shared__ float sum_blocks[2 * NREG * kFoldLanes];
  __shared__ float sum_tail[FULL ? 1 : 2 * kTailWords];
  const int64_t cols = FULL ? (int64_t)THREADS * ITEMS * VEC : cols_arg;
  const int nvec = (int)(cols / VEC);
  // Vector v of the row exists (always, for a full row).
  auto in_row = [&](uint32_t v) { return FULL || v < (uint32_t)nvec; };
  const AtenSumPlan plan(cols);
  const u32x4* wv = static_cast<const u32x4*>(w);
  const uint32_t row_bytes = (uint32_t)(cols * C::kBytes);
  auto load_row = [&](int64_t row, u32x4 (&xa)[ITEMS], u32x4 (&ra)[ITEMS]) {
    const int64_t off = row * cols * C::kBytes;
    const RowBuf<true> bx(static_cast<const char*>(x) + off, row_bytes);
    const RowBuf<true> br(static_cast<const char*>(res) + off, row_bytes);
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      const uint32_t v = threadIdx.x + k * THREADS;
      if (in_row(v)) {
        xa[k] = bx.ld16(v * 16u);
        ra[k] = br.ld16(v * 16u);
      }
    }
  };
  // The weight row is the same for every row: with few vectors per thread,
  // load this thread's slice once, ahead of the first row; otherwise re-read
  // it from L2 in the normalise phase (keeps wide rows within the VGPR budget).
  // Loading it after the row's x / residual loads instead, so that the first
  // row loads do not wait for it, measured 1.5-5 % slower on MI355X.
  constexpr bool kHoistW = ITEMS <= 2;
  u32x4 wreg[kHoistW ? ITEMS : 1];
  if constexpr (kHoistW) {
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      const int v = threadIdx.x + k * THREADS;
      if (in_row(v)) wreg[k] = wv[v];
    }
  }
  // A workgroup's first row is loaded at kernel entry, ahead of the loop
  // set-up; later rows load in the loop, or, in the per-token FP8 rows that
  // the launcher runs on a looping grid (PREFETCH), as soon as the current
  // row's y is built, so they are in flight across its amax reduction and
  // quantisation. Measured on MI355X, 8192 rows, against loading at the top
  // of the loop: bf16 12288 columns 121.7 vs 125.5 us, 16384 160.1 vs 165.0,
  // 24576 277.3 vs 288.0; fp16 16384 161.5 vs 167.3; fp32 8192 146.7 vs
  // 160.1. Issuing them before the row sum instead (x and residual are dead
  // once residual_out is stored) lost at 16384 (167.1) and with 512 threads.
  constexpr bool kPrefetch = MODE == 1 && THREADS * ITEMS >= 1536;
  u32x4 xa[ITEMS], ra[ITEMS];
  if ((int64_t)blockIdx.x < rows) load_row(blockIdx.x, xa, ra);
  // A static scale goes to scale[0] when the caller passed a scale word.
  if (MODE == 2 && scale != nullptr && blockIdx.x == 0 && threadIdx.x == 0) scale[0] = static_scale;
  int parity = 0;
  // Rows go to workgroups in blockIdx order, which the dispatcher deals to the
  // 8 XCDs round-robin; measured on MI355X, this beats giving each XCD a
  // contiguous block of rows (65 % vs 75 % of peak at [8192, 4096] bf16).
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x, parity ^= 1) {
    const int64_t off = row * cols * C::kBytes;
    const RowBuf<true, ro_store_policy(MODE)> bro(static_cast<char*>(ro) + off, row_bytes);
    if (!kPrefetch && row != (int64_t)blockIdx.x) load_row(row, xa, ra);
    u32x4 rov[ITEMS];
    // torch-CPU's summation order, which does not depend on the launch
    // shape either: the plain and the FP8 variants (different shapes) give
    // the same residual_out -> y bits.
    RowSum rs(plan, sum_stage, sum_blocks, sum_tail, parity);
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      const int v = threadIdx.x + k * THREADS;
      float sq[VEC];
#pragma unroll
      for (int i = 0; i < VEC; ++i) sq[i] = 0.0f;
      if (in_row(v)) {
        float fx[VEC], fr[VEC], fo[VEC];
        C::unpack(xa[k], fx);
        C::unpack(ra[k], fr);
#pragma unroll
        for (int i = 0; i < VEC; ++i) fo[i] = fx[i] + fr[i];
        rov[k] = C::pack(fo);
        bro.st16(rov[k], (uint32_t)v * 16u);
        C::unpack(rov[k], fo);
#pragma unroll
        for (int i = 0; i < VEC; ++i) sq[i] = fo[i] * fo[i];
      }
      rs.item(k, sq);
    }
    const float total = rs.total();
    // Dividing by a power of two is exact scaling: the product with its
    // reciprocal is the same correctly rounded quotient, without the IEEE
    // division sequence (the common case; the branch is wave-uniform).
    float variance;
    if ((cols & (cols - 1)) == 0) {
      variance = total * (1.0f / (float)cols);
    } else {
      variance = total / (float)cols;
    }
    const float inv = 1.0f / __builtin_sqrtf(variance + eps);

    if constexpr (MODE == 0) {
      const RowBuf<true, out_store_policy(MODE)> by(static_cast<char*>(y) + off, row_bytes);
#pragma unroll
      for (int k = 0; k < ITEMS; ++k) {
        const int v = threadIdx.x + k * THREADS;
        if (in_row(v)) {
          float fo[VEC], fw[VEC];
          C::unpack(rov[k], fo);
          // Opaque to the optimiser, so the unpacking of the hoisted weight
          // is not hoisted above the loop as well: that made every
          // workgroup wait for its weight load before issuing its row loads
          // (43.4 vs 43.9 us at [8192, 4096] bf16 on MI355X).
          u32x4 wk = kHoistW ? wreg[kHoistW ? k : 0] : wv[v];
          asm("" : "+v"(wk));
          C::unpack(wk, fw);
          scale_round_mul<C>(fo, inv, fw);
          by.st16(C::pack(fo), (uint32_t)v * 16u);
        }
      }
    } else {
      // y rounded to T; NaN-propagating amax over |y|. Held as floats, or
      // packed in T (exact: the values are rounded to T already), which
      // measured on MI355X, bf16, 8192 rows, floats vs packed: per-token
      // 512 x 4 at 16384 202.3 vs 171.8 us (but 512 x 3 at 12288 135.7 vs
      // 137.4, 256 x 3 at 5120 53.4 vs 54.1); static 256 x 3 at 5120 54.1 vs
      // 52.5, 512 x 3 at 12288 124.1 vs 122.1 (but 512 x 4 at 16384 163.5 vs
      // 166.8).
      constexpr bool kPackY =
          (MODE == 1 && ITEMS >= 4) || (MODE == 2 && (ITEMS == 3 || (ITEMS == 4 && THREADS == 1024)));
      float yv[kPackY ? 1 : ITEMS][VEC];
      u32x4 yp[kPackY ? ITEMS : 1];
      float amax = 0.0f;
#pragma unroll
      for (int k = 0; k < ITEMS; ++k) {
        const int v = threadIdx.x + k * THREADS;
        if (in_row(v)) {
          float fw[VEC];
          float f[VEC];
          C::unpack(rov[k], f);
          // Where the hoisted weight is unpacked above the row loop (the
          // optimiser's choice) or kept packed until here (opaque, as in
          // MODE 0) is picked per shape, measured on MI355X, bf16, unpacked
          // vs opaque: 512 x 2 per-token 92.9 vs 80.2 us at [8192, 8192],
          // 64.4 vs 60.1 at [8192, 5120], static 86.6 vs 79.0 at
          // [8192, 8192]; 1024 x 2 at [4096, 16384] per-token 107.3 vs 105.2,
          // static 96.9 vs 98.3; 256 x 2 at [16384, 4096] per-token 76.6 vs
          // 77.0, static 74.6 vs 75.5.
          constexpr bool kOpaqueW = THREADS == 512 || (THREADS > 512 && MODE == 1);
          u32x4 wk = kHoistW ? wreg[kHoistW ? k : 0] : wv[v];
          if constexpr (kOpaqueW) asm("" : "+v"(wk));
          C::unpack(wk, fw);
          scale_round_mul<C>(f, inv, fw);
#pragma unroll
          for (int i = 0; i < VEC; i += 2) {
            C::round2(f[i], f[i + 1]);
            amax = absmax2(amax, f[i], f[i + 1]);
          }
          if constexpr (kPackY) {
            yp[k] = C::pack(f);
          } else {
#pragma unroll
            for (int i = 0; i < VEC; ++i) yv[kPackY ? 0 : k][i] = f[i];
          }
        }
      }
      if (kPrefetch && row + gridDim.x < rows) load_row(row + gridDim.x, xa, ra);
      float s;
      if constexpr (MODE == 1) {
        amax = bits_f32(block_allreduce<NW>(f32_bits(amax), MaxU32{}, lds, parity));  // amax >= 0 or NaN
        s = scale_from_amax<FMT>(amax);
        if (threadIdx.x == 0) scale[row] = s;
      } else {
        // Static scale: no reduction; this thread's own max |y| selects the
        // fast or exact path for its vectors.
        s = static_scale;
      }
      const float r = 1.0f / s;
      const bool fast = fast_path_ok<FMT>(s, r, amax);
      const RowBuf<true, out_store_policy(MODE)> bq(yq + row * cols, (uint32_t)cols);
#pragma unroll
      for (int k = 0; k < ITEMS; ++k) {
        const int v = threadIdx.x + k * THREADS;
        if (in_row(v)) {
          uint32_t wq[VEC / 4];
          float f[VEC];
          if constexpr (kPackY) {
            C::unpack(yp[k], f);
          } else {
#pragma unroll
            for (int i = 0; i < VEC; ++i) f[i] = yv[kPackY ? 0 : k][i];
          }
          if (fast) {
            quant_fast<FMT, VEC>(f, s, r, wq);
          } else {
            quant_exact<FMT, VEC>(f, s, wq);
          }
          if constexpr (VEC == 8) {
            bq.st8((u32x2){wq[0], wq[1]}, (uint32_t)v * 8u);
          } else {
            bq.st4(wq[0], (uint32_t)v * 4u);
          }
        }
      }
    }
  }
}

// Any alignment / row length: scalar accesses, four waves. The sum of squares
// follows torch-CPU's order exactly (aten_sum.hpp), so this path gives the
// same bits as the register-resident kernel for any alignment or row length:
// the row is cut into blocks of 2^P steps (4 * 2^P vectors of 8 addends,
// one 64-vector region for P = 4); in each round wave w takes block
// b0 + w, computes and stores residual_out for it, stages its squares one
// region at a time in LDS and continues the 32 sequential folds over them;
// after the round's barrier every wave adds the round's block folds to its
// copy of the cascade in block order. The last block of a row whose length
// is not whole blocks is its tail (trailing steps, leftover vectors, trailing
// scalars). residual_out is re-read in the second pass, after the rounds'
// barriers, by other threads than the ones that wrote it.
template <class C, int MODE, int FMT>
__global__ __launch_bounds__(256) void rmsnorm_generic(
    const void* __restrict__ x, const void* __restrict__ res, const void* __restrict__ w,
    void* __restrict__ y, uint8_t* __restrict__ yq, float* __restrict__ scale,
    void* __restrict__ ro, int64_t rows, int64_t cols, float eps, float static_scale) {
  __shared__ uint32_t lds[2 * 4];
  __shared__ float stage[4 * kRegionAddends];
  __shared__ float blocks[2 * 4 * kFoldLanes];
  __shared__ float tail[2 * kTailWords];
  int parity = 0, rpar = 0;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const AtenSumPlan pl(cols);
  const int64_t nsub = int64_t(1) << (pl.p - 4);  // regions per block
  const int64_t bvecs = kRegionVecs * nsub;       // vectors per block
  const int64_t nblk = pl.nfull + (pl.has_tail() ? 1 : 0);
  float* a = stage + wave * kRegionAddends;
  if (MODE == 2 && scale != nullptr && blockIdx.x == 0 && threadIdx.x == 0) scale[0] = static_scale;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const int64_t base = row * cols;
    FoldCascade cs;
    int tpar = 0;
    for (int64_t b0 = 0; b0 < nblk; b0 += 4) {
      const int64_t blk = b0 + wave;
      float* bs = blocks + rpar * 4 * kFoldLanes;
      float* tl = tail + rpar * kTailWords;
      if (blk < nblk) {
        const bool full = blk < pl.nfull;
        float fold = 0.0f;
        for (int64_t sb = 0; sb < nsub; ++sb) {
          const int64_t first = blk * bvecs + sb * kRegionVecs;
          if (first * kSumLanes >= cols) break;
          const int64_t v = first + lane;
#pragma unroll
          for (int i = 0; i < kSumLanes; ++i) {
            const int64_t j = v * kSumLanes + i;
            float sqv = 0.0f;
            if (j < cols) {
              const float o = C::round(C::load1(x, base + j) + C::load1(res, base + j));
              C::store1(ro, base + j, o);
              sqv = o * o;
            }
            a[lane * kSumLanes + i] = sqv;
          }
          __builtin_amdgcn_wave_barrier();
          int nst = 16;
          if (!full) {
            const int64_t left = pl.ntrail - sb * 16;
            nst = left < 0 ? 0 : (left > 16 ? 16 : (int)left);
          }
          fold = fold_region(a, nst, lane & 31, fold);
          if (!full) stage_tail_parts(pl, a, first, lane, tl);
          __builtin_amdgcn_wave_barrier();
        }
        if (lane < kFoldLanes) {
          if (full) {
            bs[wave * kFoldLanes + lane] = fold;
          } else {
            tl[lane] = fold;
          }
        }
      }
      __syncthreads();
      if (lane < kFoldLanes) {
        for (int i = 0; i < 4; ++i) {
          if (b0 + i < pl.nfull) cs.add(bs[i * kFoldLanes + lane], b0 + i, pl.p);
        }
      }
      tpar = rpar;
      rpar ^= 1;
    }
    const float* tl = tail + tpar * kTailWords;
    const float total = pl.nv == 0 ? aten_scalar_row(pl, tl)
                                   : aten_combine(pl, lane < kFoldLanes ? cs.slot_sum(pl, tl, lane) : 0.0f, tl, lane);
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
  auto run = [&](auto shape) {
    using S = decltype(shape);
    // Wide FP8 rows run on a grid of the workgroups the device holds at once,
    // each looping over rows (no idle CU between rows, one weight load per
    // workgroup): per-token from 1536 vectors of capacity (8192 bf16 rows:
    // 126.9 against 134.6 us at 12288 columns, 286.1 against 301.5 at 24576;
    // fp16 172.8 against 184.9 at 16384), static from 3072 (273.3 against
    // 297.7 at 24576). Plain RMSNorm rows lose 3-6 % on such a grid, and so
    // do narrower per-token rows even with the next-row prefetch: from 1024
    // vectors, 81.0 against 76.1 us at [8192, 8192]; from 512, 84.0 against
    // 74.9 at [16384, 4096].
    constexpr int kCap = S::kThreads * S::kItems;
    constexpr bool kLoop = (MODE == 1 && kCap >= 1536) || (MODE == 2 && kCap >= 3072);
    auto go = [&](auto full) {
      constexpr auto kernel = rmsnorm_resident<C, S::kThreads, S::kItems, MODE, FMT, decltype(full)::value>;
      const int64_t resident = kLoop ? resident_groups<kernel>(S::kThreads) : 0;
      const unsigned grid = resident > 0 && resident < (int64_t)g ? (unsigned)resident : g;
      kernel<<<grid, S::kThreads, 0, st>>>(x, res, w, y, yq, scale, ro, rows, cols, eps, static_scale);
    };
    // A row that fills the shape exactly in whole 512-addend regions takes
    // the compile-time-planned kernel (no per-vector bounds checks, no tail).
    if constexpr (C::VEC == 8 && (kCap * 8) % kRegionAddends == 0) {
      if (nvec == kCap) return go(std::true_type{});
    }
    go(std::false_type{});
  };
  // 16-byte rows (f16 / bf16): the shapes come from a sweep over every
  // THREADS in 64..1024 (step 64) x ITEMS in 1..4 holding the row, on MI355X
  // at 8192 bf16 rows of 2048..16384 elements (graph-replayed, 2 GiB
  // rotation). The plain op wants up to 768 threads with one vector each,
  // then 512 or 768 x 2 and 512 x 4: no 1024-thread shape wins, e.g. 55.5 us
  // for 768 x 1 at 5120 elements against 81.4 for 1024 x 1, 90.1 for 512 x 2
  // at 8192 against 108.3, 130.3 for 768 x 2 at 12288 against 155.4. The FP8
  // variants hold y across the amax reduction and want few waves per row: 256
  // threads x 1..3 vectors, then 512 x 2..4 (5120 elements: 53.9 us for
  // 256 x 3 against 60.3 for 512 x 2; 12288: 136.6 for 512 x 3 against 161.3
  // for 1024 x 2; static 16384: 163.4 for 512 x 4 against 187.4).
  // fp32 rows stage their squares whole in LDS (aten_sum.hpp): up to
  // 1024 x 4 vectors (16384 elements, 64 KB of the 160 KB a gfx950
  // workgroup may hold); longer ones loop. Their plain-op shapes: 512 x 2
  // for rows of 513-1024 vectors, 512 x 4 up to 2048 (same-run A/B on
  // MI355X against 1024 x 1 and 1024 x 2: 172.8 vs 196.3 us at [16384, 4096],
  // 44.2 vs 53.5 at [4096, 4096], 58.2 vs 63.4 at [4096, 5120], 177.2 vs
  // 184.6 at [8192, 8192]; 256 x 2 lost to 512 x 1 at 2048 columns).
  bool done;
  if constexpr (MODE == 0 && C::VEC == 8) {
    done = vec_ok && pick_row_shape<RowShape<64, 1>, RowShape<128, 1>, RowShape<256, 1>, RowShape<320, 1>,
                                    RowShape<384, 1>, RowShape<448, 1>, RowShape<512, 1>, RowShape<768, 1>,
                                    RowShape<512, 2>, RowShape<768, 2>, RowShape<512, 4>,
                                    RowShape<1024, 4>>(nvec, run);
  } else if constexpr (MODE == 0) {
    done = vec_ok && pick_row_shape<RowShape<64, 1>, RowShape<128, 1>, RowShape<256, 1>, RowShape<512, 1>,
                                    RowShape<512, 2>, RowShape<512, 4>, RowShape<1024, 3>,
                                    RowShape<1024, 4>>(nvec, run);
  } else if constexpr (C::VEC == 8) {
    done = vec_ok && pick_row_shape<RowShape<64, 1>, RowShape<64, 2>, RowShape<256, 1>, RowShape<192, 2>,
                                    RowShape<256, 2>, RowShape<256, 3>, RowShape<512, 2>, RowShape<512, 3>,
                                    RowShape<512, 4>, RowShape<1024, 4>>(nvec, run);
  } else {
    // fp32 FP8 rows of 1025-2048 vectors: 512 x 4 against 1024 x 2, per-token
    // 53.7 vs 62.1 us at [4096, 5120], 117.6 vs 127.4 at [8192, 6144] (159.2
    // vs 157.4 at [8192, 8192]); static 147.4 vs 157.5 at [8192, 8192].
    done = vec_ok && pick_row_shape<RowShape<64, 1>, RowShape<64, 2>, RowShape<128, 2>, RowShape<256, 2>,
                                    RowShape<512, 2>, RowShape<512, 4>, RowShape<1024, 3>,
                                    RowShape<1024, 4>>(nvec, run);
  }
  if (!done) {
    rmsnorm_generic<C, MODE, FMT><<<g, 256, 0, st>>>(x, res, w, y, yq, scale, ro, rows, cols, eps, static_scale);
  }
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
      return launch_rmsnorm<C, 2, FMT>(x, residual, weight, nullptr, y_fp8, scale, residual_out, rows,
                                       cols, eps, static_scale, st);
    });
  });
}
