// MoE token permute (row gather) and unpermute (weighted combine), for gfx950.
//
// Semantics (baselines/token_permute.py:215-217, 237-251):
//   gather:   dst[i] = src[indices[i]]
//   combine:  out[t] = T( sum_j  float(w[t,j]) * float(eo[unpermute_index[t,j]]) )
// The combine rounds every product to fp32 and sums them per output column
// in the order torch-CPU's (gathered.float() * w).sum(dim=1) uses (ATen's
// reduction of a contiguous [T, k, h] tensor over its middle dimension):
//   * the leading columns it reduces as vector lanes (32-column chunks, the
//     first 4 of rows of 4 to 7): one running sum over j = 0..k-1 from +0.0
//     in ATen's block cascade (AtenCascade), which is plain j order for
//     k <= 16;
//   * the other columns: ATen's scalar form, four slots of every fourth j
//     (aten_scalar_sum);
//   * h == 1, where the reduced dimension is contiguous: ATen's row sum
//     (aten_row_sum).
//
// Design: one workgroup per output row (64-512 threads, sized to the row).
// The row's index (and weight) is workgroup-uniform and read once into SGPRs;
// the row then moves as 16-byte vectors (one per thread for the gather; 2-4
// per thread times two expert rows in flight for the combine), nontemporal. Gather is byte movement
// (dtype-agnostic); combine unpacks to fp32, accumulates and packs.
//
// Index hygiene: an index outside [0, n_src) makes a gathered row all zeros
// and drops that (t, j) term from a combine, instead of reading out of bounds.
// The reference-ABI launchers do not know n_src (the reference passes no
// source row count) and only reject negative indices; the *_checked
// launchers take the bound.
#include "launch.hpp"

namespace cck {
namespace {

#pragma clang fp contract(off)

// Rows of at most THREADS vectors: each workgroup takes R consecutive
// destination rows per step (grid-stride over groups of R). The R source
// indices are read first, then every row's vector is in flight at once, so
// the index load is paid once per R rows.
template <int THREADS, int R>
__global__ __launch_bounds__(THREADS) void token_gather_rows(const u32x4* __restrict__ src,
                                                             const int64_t* __restrict__ idx,
                                                             u32x4* __restrict__ dst, int64_t n_dst,
                                                             int64_t row_vecs, int64_t n_src) {
  const int64_t t = threadIdx.x;
  for (int64_t row0 = (int64_t)blockIdx.x * R; row0 < n_dst; row0 += (int64_t)gridDim.x * R) {
    int64_t s[R];
#pragma unroll
    for (int r = 0; r < R; ++r) s[r] = row0 + r < n_dst ? idx[row0 + r] : -1;  // uniform: scalar loads
    u32x4 v[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      v[r] = (u32x4){0u, 0u, 0u, 0u};
      if (s[r] >= 0 && s[r] < n_src && t < row_vecs) v[r] = ld_stream(src + s[r] * row_vecs + t);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (row0 + r < n_dst && t < row_vecs) st_stream(v[r], dst + (row0 + r) * row_vecs + t);
    }
  }
}

// token_gather_rows on a grid that the GPU holds at once: each workgroup
// loops over its groups of R rows and loads the next group's R indices while
// the current rows are in flight, so only the first group waits for its
// indices before its row loads.
template <int THREADS, int R>
__global__ __launch_bounds__(THREADS) void token_gather_rows_pf(const u32x4* __restrict__ src,
                                                                const int64_t* __restrict__ idx,
                                                                u32x4* __restrict__ dst, int64_t n_dst,
                                                                int64_t row_vecs, int64_t n_src) {
  const int64_t t = threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * R;
  int64_t row0 = (int64_t)blockIdx.x * R;
  int64_t s[R];
#pragma unroll
  for (int r = 0; r < R; ++r) s[r] = row0 + r < n_dst ? idx[row0 + r] : -1;  // uniform: scalar loads
  for (; row0 < n_dst; row0 += stride) {
    u32x4 v[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      v[r] = (u32x4){0u, 0u, 0u, 0u};
      if (s[r] >= 0 && s[r] < n_src && t < row_vecs) v[r] = ld_stream(src + s[r] * row_vecs + t);
    }
    const int64_t next = row0 + stride;
#pragma unroll
    for (int r = 0; r < R; ++r) s[r] = next + r < n_dst ? idx[next + r] : -1;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (row0 + r < n_dst && t < row_vecs) st_stream(v[r], dst + (row0 + r) * row_vecs + t);
    }
  }
}

// Large gathers: one 16-byte vector per thread, waves of 64 consecutive
// destination vectors, on a grid of up to 2^20 workgroups, the shape of a flat
// copy. A wave's rows and source indices are wave-uniform (scalar loads); rows
// of at least 64 vectors put a wave in at most two rows.
__global__ __launch_bounds__(256) void token_gather_flat(const u32x4* __restrict__ src,
                                                         const int64_t* __restrict__ idx,
                                                         u32x4* __restrict__ dst, int64_t n_dst,
                                                         int64_t row_vecs, int64_t n_src) {
  const int64_t total = n_dst * row_vecs;
  const int lane = threadIdx.x & 63;
  const int64_t wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  for (int64_t base = (int64_t)blockIdx.x * 256 + wave * 64; base < total; base += (int64_t)gridDim.x * 256) {
    const int64_t row = base / row_vecs;
    const int64_t col0 = base - row * row_vecs;
    int64_t s = idx[row];
    int64_t col = col0 + lane;
    if (col0 + 64 > row_vecs) {  // the wave ends in the next row
      const int64_t s1 = row + 1 < n_dst ? idx[row + 1] : -1;
      if (col >= row_vecs) {
        s = s1;
        col -= row_vecs;
      }
    }
    const bool in = base + lane < total;
    u32x4 v = (u32x4){0u, 0u, 0u, 0u};
    if (in && s >= 0 && s < n_src) v = ld_stream(src + s * row_vecs + col);
    if (in) st_stream(v, dst + base + lane);
  }
}

// Any row length / alignment: element-wise (E = 1-, 2- or 4-byte element).
template <class E>
__global__ __launch_bounds__(256) void token_gather_elems(const E* __restrict__ src,
                                                          const int64_t* __restrict__ idx,
                                                          E* __restrict__ dst, int64_t n_dst,
                                                          int64_t h, int64_t n_src) {
  for (int64_t row = blockIdx.x; row < n_dst; row += gridDim.x) {
    const int64_t s = idx[row];
    const bool valid = s >= 0 && s < n_src;
    for (int64_t c = threadIdx.x; c < h; c += 256) dst[row * h + c] = valid ? src[s * h + c] : E(0);
  }
}

// ATen's block cascade of one float running sum (the fp32 sum kernel's
// accumulation, also stated in oracle/rowsum.py): the steps fold into a0 in
// blocks of 2^p; after each whole block a1 += a0 and a0 = 0, after every 2^p
// blocks a2 += a1 and a1 = 0, after every 2^(2p) blocks a3 += a2 and a2 = 0;
// the total is ((a0 + a1) + a2) + a3.
struct AtenCascade {
  float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
  // x is step number `step` (1-based) of the sum.
  __device__ void add(float x, int64_t step, int p) {
    a0 = a0 + x;
    const int64_t m = (int64_t(1) << p) - 1;
    if ((step & m) == 0) {
      a1 = a1 + a0;
      a0 = 0.0f;
      if (((step >> p) & m) == 0) {
        a2 = a2 + a1;
        a1 = 0.0f;
        if (((step >> (2 * p)) & m) == 0) {
          a3 = a3 + a2;
          a2 = 0.0f;
        }
      }
    }
  }
  __device__ float total() const { return ((a0 + a1) + a2) + a3; }
};

// ATen's block size exponent for a sum of `steps` steps: max(4, ceil(log2
// steps) / 4), with ceil(log2 m) taken as 1 for m <= 2.
inline int aten_level_power(int64_t steps) {
  int c = 1;
  while (steps > 2 && (int64_t(1) << c) < steps) ++c;
  return c / 4 > 4 ? c / 4 : 4;
}

// ATen's scalar form of a sum of n terms (term(j) gives term j): four slots
// of every fourth term, each an AtenCascade with block exponent p, the n mod
// 4 leftovers added to slot 0, then ((s0 + s1) + s2) + s3.
template <class F>
__device__ inline float aten_scalar_sum(int64_t n, int p, F&& term) {
  AtenCascade sl[4];
  const int64_t steps = n / 4;
  for (int64_t i = 0; i < steps; ++i) {
#pragma unroll
    for (int q = 0; q < 4; ++q) sl[q].add(term(4 * i + q), i + 1, p);
  }
  float s0 = sl[0].total();
  for (int64_t j = 4 * steps; j < n; ++j) s0 = s0 + term(j);
  return ((s0 + sl[1].total()) + sl[2].total()) + sl[3].total();
}

// ATen's row sum of n contiguous terms (oracle/rowsum.py): under 8 terms the
// scalar form; otherwise 8-lane vectors in the scalar form's four slots per
// lane (block exponent p8 for n / 32 steps), then 0 + the n mod 8 trailing
// terms in order + the 8 lane totals in order. One thread, a pass per lane.
template <class F>
__device__ inline float aten_row_sum(int64_t n, int p4, int p8, F&& term) {
  if (n < 8) return 0.0f + aten_scalar_sum(n, p4, term);
  const int64_t nv = n / 8, steps = nv / 4;
  float total = 0.0f;
  for (int64_t e = nv * 8; e < n; ++e) total = total + term(e);
  for (int l = 0; l < 8; ++l) {
    AtenCascade sl[4];
    for (int64_t i = 0; i < steps; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) sl[q].add(term((4 * i + q) * 8 + l), i + 1, p8);
    }
    float s0 = sl[0].total();
    for (int64_t v = 4 * steps; v < nv; ++v) s0 = s0 + term(v * 8 + l);
    total = total + (((s0 + sl[1].total()) + sl[2].total()) + sl[3].total());
  }
  return total;
}

// The order parameters of one combine (host side).
struct CombineOrder {
  int64_t main_cols;  // leading columns summed as vector lanes
  int p_main, p_slot, p_row;
};

inline CombineOrder combine_order(int64_t k, int64_t h) {
  CombineOrder o;
  o.main_cols = h >= 32 ? h - h % 32 : (h >= 4 && h < 8 ? 4 : 0);
  o.p_main = aten_level_power(k);
  o.p_slot = aten_level_power(k / 4);
  o.p_row = aten_level_power(k / 32);
  return o;
}

// One tail column of one token in ATen's scalar form (h == 1: the row sum).
template <class C>
__device__ inline float combine_scalar_column(const void* eo, const int64_t* it, const float* wt, int64_t k,
                                              int64_t h, int64_t c, int64_t n_rows, const CombineOrder& o) {
  auto term = [&](int64_t j) {
    const int64_t r = it[j];
    return r >= 0 && r < n_rows ? wt[j] * C::load1(eo, r * h + c) : 0.0f;
  };
  return h == 1 ? aten_row_sum(k, o.p_slot, o.p_row, term) : aten_scalar_sum(k, o.p_slot, term);
}

// Weighted combine on 16-byte vectors: one workgroup per token, VPL vectors
// per thread per step; JU expert rows are loaded together before they are
// accumulated in j order (CASC: in ATen's block cascade, for k > 16). That is
// torch's order for the main columns; the launcher then rewrites the other
// (at most 31) columns with token_combine_elems on the same stream. Bounding
// this kernel by the main columns instead measured 3 % slower at 4096 tokens
// x hidden 7168 (76.0 against 73.5 us, k = 6) for the same instructions. A
// dropped term (index outside the source rows) adds +0.0, which changes no
// sum that starts at +0.0.
template <class C, int THREADS, int VPL, int JU, bool CASC>
__global__ __launch_bounds__(THREADS) void token_combine_vec(const u32x4* __restrict__ eo,
                                                             const int64_t* __restrict__ uidx,
                                                             const float* __restrict__ w,
                                                             u32x4* __restrict__ out, int64_t n_tokens,
                                                             int64_t k, int64_t row_vecs, int64_t n_rows,
                                                             int p_main) {
  constexpr int VEC = C::VEC;
  for (int64_t t = blockIdx.x; t < n_tokens; t += gridDim.x) {
    const int64_t* it = uidx + t * k;
    const float* wt = w + t * k;
    for (int64_t base = threadIdx.x; base < row_vecs; base += THREADS * VPL) {
      float acc[VPL][VEC];
      AtenCascade cas[CASC ? VPL : 1][CASC ? VEC : 1];
#pragma unroll
      for (int v = 0; v < VPL; ++v)
#pragma unroll
        for (int i = 0; i < VEC; ++i) acc[v][i] = 0.0f;
      for (int64_t j0 = 0; j0 < k; j0 += JU) {
        u32x4 raw[JU][VPL];
        float wj[JU];
        bool ok[JU];
#pragma unroll
        for (int u = 0; u < JU; ++u) {
          const int64_t j = j0 + u;
          const int64_t r = j < k ? it[j] : -1;  // uniform: scalar loads
          ok[u] = r >= 0 && r < n_rows;
          wj[u] = j < k ? wt[j] : 0.0f;
#pragma unroll
          for (int v = 0; v < VPL; ++v) {
            const int64_t c = base + THREADS * v;
            if (ok[u] && c < row_vecs) raw[u][v] = ld_stream(eo + r * row_vecs + c);
          }
        }
#pragma unroll
        for (int u = 0; u < JU; ++u) {
          if constexpr (CASC) {
            if (j0 + u >= k) continue;
#pragma unroll
            for (int v = 0; v < VPL; ++v) {
              const int64_t c = base + THREADS * v;
              if (c < row_vecs) {
                float x[VEC];
                C::unpack(raw[u][v], x);
#pragma unroll
                for (int i = 0; i < VEC; ++i) cas[v][i].add(ok[u] ? wj[u] * x[i] : 0.0f, j0 + u + 1, p_main);
              }
            }
          } else {
            if (!ok[u]) continue;
#pragma unroll
            for (int v = 0; v < VPL; ++v) {
              const int64_t c = base + THREADS * v;
              if (c < row_vecs) {
                float x[VEC];
                C::unpack(raw[u][v], x);
#pragma unroll
                for (int i = 0; i < VEC; ++i) acc[v][i] = acc[v][i] + wj[u] * x[i];
              }
            }
          }
        }
      }
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        const int64_t c = base + THREADS * v;
        if constexpr (CASC) {
#pragma unroll
          for (int i = 0; i < VEC; ++i) acc[v][i] = cas[v][i].total();
        }
        if (c < row_vecs) st_stream(C::pack(acc[v]), out + t * row_vecs + c);
      }
    }
  }
}

// Columns c0..h-1 one per thread (any alignment): the main columns with
// ATen's block cascade, the others in the scalar form (or h == 1: the row
// sum).
template <class C, int THREADS>
__global__ __launch_bounds__(THREADS) void token_combine_elems(const void* __restrict__ eo,
                                                               const int64_t* __restrict__ uidx,
                                                               const float* __restrict__ w,
                                                               void* __restrict__ out, int64_t n_tokens,
                                                               int64_t k, int64_t h, int64_t c0, int64_t n_rows,
                                                               CombineOrder o) {
  for (int64_t t = blockIdx.x; t < n_tokens; t += gridDim.x) {
    const int64_t* it = uidx + t * k;
    const float* wt = w + t * k;
    for (int64_t c = c0 + threadIdx.x; c < h; c += THREADS) {
      float v;
      if (c < o.main_cols) {
        AtenCascade acc;
        for (int64_t j = 0; j < k; ++j) {
          const int64_t r = it[j];
          acc.add(r >= 0 && r < n_rows ? wt[j] * C::load1(eo, r * h + c) : 0.0f, j + 1, o.p_main);
        }
        v = acc.total();
      } else {
        v = combine_scalar_column<C>(eo, it, wt, k, h, c, n_rows, o);
      }
      C::store1(out, t * h + c, v);
    }
  }
}

// Threads per row-workgroup: enough 64-lane waves to cover the row at VPL
// vectors per thread, up to MAXT.
template <int VPL, int MAXT, class Fn>
inline void with_row_threads(int64_t row_vecs, Fn&& fn) {
  if (row_vecs <= 64 * VPL || MAXT == 64) {
    fn(std::integral_constant<int, 64>{});
  } else if (row_vecs <= 128 * VPL || MAXT == 128) {
    fn(std::integral_constant<int, 128>{});
  } else if (row_vecs <= 256 * VPL || MAXT == 256) {
    fn(std::integral_constant<int, 256>{});
  } else {
    fn(std::integral_constant<int, 512>{});
  }
}

inline int32_t elem_bytes(int32_t dtype) {
  switch (dtype) {
    case kF32: return 4;
    case kF16:
    case kBF16: return 2;
    case kF8E4M3:
    case kF8E5M2: return 1;
    default: return 0;
  }
}

// Destination rows from which the short-row gather takes 8 rows per
// workgroup step instead of 4: same-run A/B on MI355X, bf16 rows of 8 KB,
// 11.5 vs 12.5 us at 2048 -> 4096 rows and 4096 -> 4096, 47.3 vs 48.6 us at
// 16384 rows, 191.3 vs 194.7 at 65536 (with the index prefetch below);
// 1024 -> 2048 rows took 7.5 vs 6.9 us with 8 (a grid of 256 workgroups).
constexpr int64_t kGatherR8Min = 4096;
// Rows of more than 512 vectors take token_gather_flat at every size, and
// rows of 64 to 512 vectors from 2^22 destination vectors (64 MiB) on.
// Same-run A/B on MI355X, bf16 (fp32) rows, against the row kernels below
// (and, past 512 vectors, one 512-thread workgroup per row walking it with
// one or four vectors per thread in flight): 65536 -> 65536 rows of 4096
// 171.9 vs 190.8 us, 16384 rows 43.6 vs 46.8, 8192 rows 23.0 vs 24.0, 32768
// rows of 2048 44.1 vs 47.1, 65536 rows of 1024 44.4 vs 47.3, 16384 -> 32768
// rows of 7168 149.3 vs 152.3; fp32 16384 rows of 4096 85.6 vs 89.1, 65536
// rows 348.3 vs 358.7. Past 512 vectors: 256 rows of 7168 3.30 vs 3.84, 2048
// rows 11.19 vs 11.93, 1024 -> 2048 rows of 11008 15.93 vs 17.09; fp32 512
// rows of 4096 4.64 vs 4.92, 1024 -> 2048 rows of 7168 19.95 vs 21.39. Up to
// 512 vectors and below 2^22 the row kernels win: 4096 rows of 4096, 11.6
// vs 12.1 us; 8192 -> 16384 rows of 1024, 11.8 vs 12.6; 4096 rows of 2048,
// 6.8 vs 7.4.
constexpr int64_t kGatherFlatMin = int64_t(1) << 22;

int32_t gather(const void* src, const int64_t* indices, void* dst, int64_t n_dst, int64_t h,
               int32_t dtype, int64_t n_src, hipStream_t st) {
  if (n_dst <= 0 || h <= 0) return (int32_t)hipSuccess;
  const int32_t es = elem_bytes(dtype);
  if (es == 0) return (int32_t)hipErrorInvalidValue;
  const unsigned grid = row_grid(n_dst);
  const int64_t row_bytes = h * es;
  if (row_bytes % 16 == 0 && host_aligned(src, 16) && host_aligned(dst, 16)) {
    const int64_t rv = row_bytes / 16;
    if (rv > 512 || (rv >= 64 && n_dst * rv >= kGatherFlatMin)) {
      token_gather_flat<<<flat_grid(n_dst * rv, 256, 1 << 20), 256, 0, st>>>(
          static_cast<const u32x4*>(src), indices, static_cast<u32x4*>(dst), n_dst, rv, n_src);
    } else {
      // One vector per thread, up to 512 threads, R rows per workgroup step:
      // with R = 4, 12.3 vs 12.6 us for one row per workgroup at 2048 -> 4096
      // rows of 8 KB on MI355X (13.0-13.5 with 2-8 vectors per thread).
      // When there are more groups of R rows than the GPU holds at once, a
      // resident grid loops over them with the next indices prefetched
      // (without the prefetch, 8 rows per step lost at 16384 rows: 50.7 us).
      auto run = [&](auto rows) {
        constexpr int R = decltype(rows)::value;
        const unsigned groups = row_grid((n_dst + R - 1) / R);
        with_row_threads<1, 512>(rv, [&](auto threads) {
          constexpr int TH = decltype(threads)::value;
          const int64_t res = resident_groups<token_gather_rows_pf<TH, R>>(TH);
          if (res > 0 && res < (int64_t)groups) {
            token_gather_rows_pf<TH, R><<<(unsigned)res, TH, 0, st>>>(static_cast<const u32x4*>(src), indices,
                                                                      static_cast<u32x4*>(dst), n_dst, rv, n_src);
          } else {
            token_gather_rows<TH, R><<<groups, TH, 0, st>>>(static_cast<const u32x4*>(src), indices,
                                                           static_cast<u32x4*>(dst), n_dst, rv, n_src);
          }
        });
      };
      if (n_dst >= kGatherR8Min) {
        run(std::integral_constant<int, 8>{});
      } else {
        run(std::integral_constant<int, 4>{});
      }
    }
  } else if (es == 4) {
    token_gather_elems<uint32_t><<<grid, 256, 0, st>>>(static_cast<const uint32_t*>(src), indices,
                                                       static_cast<uint32_t*>(dst), n_dst, h, n_src);
  } else if (es == 2) {
    token_gather_elems<uint16_t><<<grid, 256, 0, st>>>(static_cast<const uint16_t*>(src), indices,
                                                       static_cast<uint16_t*>(dst), n_dst, h, n_src);
  } else {
    token_gather_elems<uint8_t><<<grid, 256, 0, st>>>(static_cast<const uint8_t*>(src), indices,
                                                      static_cast<uint8_t*>(dst), n_dst, h, n_src);
  }
  return launch_status();
}

constexpr int64_t kCombineWideTokens = 4096;
constexpr int64_t kCombineFewTokens = 1024;

int32_t combine(const void* eo, const int64_t* uidx, const float* w, void* out, int64_t n_tokens,
                int64_t k, int64_t h, int32_t dtype, int64_t n_rows, hipStream_t st) {
  if (n_tokens <= 0 || k <= 0 || h <= 0) return (int32_t)hipSuccess;
  const CombineOrder order = combine_order(k, h);
  return with_codec(dtype, [&](auto codec) {
    using C = decltype(codec);
    const unsigned grid = row_grid(n_tokens);
    if (h % C::VEC == 0 && host_aligned(eo, 16) && host_aligned(out, 16)) {
      // Two expert rows in flight per step. Top-1/2 rows: 4 vectors per thread
      // (9.4 us at T=2048, k=2, hidden 4096 bf16); deeper top-k: 2 per thread
      // (20.5 us at k=6); both measured on MI355X against 1-8 vectors and 1-8 rows.
      const int64_t rv = h / C::VEC;
      const int64_t mv = order.main_cols / C::VEC;
      auto wide = [&](auto vpl) {
        constexpr int V = decltype(vpl)::value;
        token_combine_vec<C, 512, V, 2, false><<<grid, 512, 0, st>>>(
            static_cast<const u32x4*>(eo), uidx, w, static_cast<u32x4*>(out), n_tokens, k, rv, n_rows, order.p_main);
      };
      // Many tokens, rows of 512 to 2048 vectors (4096 to 16384 bf16):
      // 512-thread workgroups holding the row in one pass, measured on MI355X
      // (graph-replayed) against the shapes below: 35.0 vs 38.1 us at T=8192,
      // k=2, hidden 4096 (fp16 34.8 vs 37.2, fp32 66.6 vs 71.5); 186.5 vs
      // 194.3 at T=8192, k=8, hidden 7168; 412.7 vs 437.2 at hidden 16384 (but
      // 27.2 vs 26.3 at T=4096, k=8, hidden 2048, and 159.5 vs 158.5 at
      // T=16384, k=6, hidden 4096).
      const bool many = n_tokens >= kCombineWideTokens && (k <= 2 ? mv >= 512 : mv > 512) && mv <= 4 * 512;
      // Few tokens, so few workgroups, and rows of 512 vectors or more: the
      // same form, now for the loads it keeps in flight. Same-run A/B against
      // the shapes below: bf16 hidden 4096 top-2 at 512 tokens 4.2 vs 5.7 us,
      // top-6 at 256 6.1 vs 8.9, hidden 7168 top-6 at 512 11.6 vs 17.1; fp32
      // hidden 4096 top-6 at 256 6.9 vs 14.9, top-2 at 1024 9.9 vs 11.5. From
      // 1536 tokens it ties or loses (8.3 vs 7.9 us at bf16 hidden 4096, top 2),
      // and shorter rows lose (6.1 vs 5.3 us at 512 tokens, hidden 2048 bf16,
      // top 6).
      const bool few = n_tokens <= kCombineFewTokens && k <= 16 && mv >= 512;
      if (mv == 0) {
        // Rows of 8 to 31 elements: scalar columns only.
      } else if (k > 16) {
        // Deeper sums take ATen's block cascade: one vector per thread.
        with_row_threads<1, 512>(mv, [&](auto threads) {
          constexpr int TH = decltype(threads)::value;
          token_combine_vec<C, TH, 1, 2, true><<<grid, TH, 0, st>>>(
              static_cast<const u32x4*>(eo), uidx, w, static_cast<u32x4*>(out), n_tokens, k, rv, n_rows, order.p_main);
        });
      } else if (many || few) {
        if (mv <= 512) {
          wide(IntC<1>{});
        } else if (mv <= 1024) {
          wide(IntC<2>{});
        } else {
          wide(IntC<4>{});
        }
      } else if (k <= 2 && mv >= 1024) {
        // Rows of 1024 vectors and more (fp32 hidden 4096, bf16 8192) in one
        // pass of 256 threads: 12.8 vs 15.6 us at 1536 tokens, 17.6 vs 19.7 at
        // 2048 (fp32 hidden 4096, top 2); 27.9 vs 30.0 at 3072 tokens (bf16
        // hidden 8192); two passes of 128 threads for bf16 hidden 7168 stay
        // faster (14.0 vs 15.3 us at 1536 tokens).
        with_row_threads<4, 256>(mv, [&](auto threads) {
          constexpr int TH = decltype(threads)::value;
          token_combine_vec<C, TH, 4, 2, false><<<grid, TH, 0, st>>>(
              static_cast<const u32x4*>(eo), uidx, w, static_cast<u32x4*>(out), n_tokens, k, rv, n_rows, order.p_main);
        });
      } else if (k <= 2) {
        with_row_threads<4, 128>(mv, [&](auto threads) {
          constexpr int TH = decltype(threads)::value;
          token_combine_vec<C, TH, 4, 2, false><<<grid, TH, 0, st>>>(
              static_cast<const u32x4*>(eo), uidx, w, static_cast<u32x4*>(out), n_tokens, k, rv, n_rows, order.p_main);
        });
      } else {
        with_row_threads<2, 256>(mv, [&](auto threads) {
          constexpr int TH = decltype(threads)::value;
          token_combine_vec<C, TH, 2, 2, false><<<grid, TH, 0, st>>>(
              static_cast<const u32x4*>(eo), uidx, w, static_cast<u32x4*>(out), n_tokens, k, rv, n_rows, order.p_main);
        });
      }
      if (order.main_cols < h) {
        // The h mod 32 scalar columns (at most 31) rewritten in a launch of
        // their own, so the vector kernel keeps its registers (in the kernel,
        // their code took 90 SGPRs instead of 64 and a second round of
        // workgroups at 2048 tokens: 24.1 against 20.4 us, k = 6).
        token_combine_elems<C, 64><<<grid, 64, 0, st>>>(eo, uidx, w, out, n_tokens, k, h, order.main_cols, n_rows,
                                                        order);
      }
    } else {
      token_combine_elems<C, 256><<<grid, 256, 0, st>>>(eo, uidx, w, out, n_tokens, k, h, 0, n_rows, order);
    }
    return launch_status();
  });
}

constexpr int64_t kNoBound = INT64_MAX;

// ---------------------------------------------------------------------------
// The permutation bookkeeping between the router and the gather
// (baselines/token_permute.py:55-70, there a stable torch.argsort of the
// flattened [T, k] expert ids and its inverse):
//   permute_index[p]   = i / k for the i-th entry in (expert, i) order
//   unpermute_index[i] = p, its position in that order.
// Expert ids are bounded, so this is a stable counting sort: one launch
// below kPermSplitMin entries, three from there on. Entries whose id lies
// outside [0, n_experts) go to one extra bucket after every expert (so the
// outputs stay a permutation of [0, n)).
// ---------------------------------------------------------------------------
constexpr int kPermThreads = 1024, kPermWaves = kPermThreads / 64;
constexpr int kPermMaxExperts = 256, kPermBuckets = kPermMaxExperts + 1;
constexpr int kPermMaxGroups = 64, kPermUnroll = 16;
constexpr int kPermPerLane = (kPermBuckets + 63) / 64;

__device__ inline uint32_t lanes_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

__device__ inline int perm_bucket(int64_t id, int n_experts) {
  return (id >= 0 && id < n_experts) ? (int)id : n_experts;
}

// hist[key] += 1 for every active lane, in one LDS atomic per wave. The lanes
// whose key equals the first active lane's add once, through that lane: a
// skewed routing puts most of a wave's ids on one expert, and LDS atomics on
// one address serialise.
__device__ inline void perm_count(uint32_t* hist, int key) {
  const int key0 = __builtin_amdgcn_readfirstlane(key);
  const unsigned long long same = __ballot(key == key0);
  const bool other = key != key0;
  if (other || lanes_below(same) == 0u) atomicAdd(&hist[key], other ? 1u : (uint32_t)__popcll(same));
}

// Wave 0 turns the bucket counts (before + after this workgroup's chunk)
// into each bucket's first position for the chunk:
// base[b] = (entries in buckets below b) + before[b].
// Lane l holds buckets [l * kPermPerLane, (l + 1) * kPermPerLane).
__device__ inline void perm_bases(const uint32_t* after, const uint32_t* before, uint32_t* base, int nb, int lane) {
  uint32_t loc[kPermPerLane], sum = 0u;
#pragma unroll
  for (int i = 0; i < kPermPerLane; ++i) {
    const int b = lane * kPermPerLane + i;
    loc[i] = b < nb ? before[b] + after[b] : 0u;
    sum += loc[i];
  }
  uint32_t incl = sum;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t o = __shfl_up(incl, d);
    if (lane >= d) incl += o;
  }
  uint32_t run = incl - sum;
#pragma unroll
  for (int i = 0; i < kPermPerLane; ++i) {
    const int b = lane * kPermPerLane + i;
    if (b < nb) base[b] = run + before[b];
    run += loc[i];
  }
}

// Stable ranking of the entries [c0, c1) from base[]: per tile, every lane
// ORs its lane bit into its wave's mask of its bucket; the bits below a lane
// in its own mask rank it among the wave's lanes of the same bucket, the
// popcounts of the lower waves' masks offset it, so ties keep index order; a
// running count per bucket carries the order from tile to tile.
// lane_mask must be zero on entry and is zero on return.
template <bool kWritePermute>
__device__ inline void perm_rank_chunk(const int64_t* __restrict__ ids, int64_t k, int n_experts, int64_t c0,
                                       int64_t c1, uint32_t* base, unsigned long long (*lane_mask)[kPermBuckets],
                                       int64_t* __restrict__ permute_index, int64_t* __restrict__ unpermute_index) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nb = n_experts + 1;
  for (int64_t t0 = c0; t0 < c1; t0 += kPermThreads) {
    const int64_t j = t0 + tid;
    const bool valid = j < c1;
    const int b = valid ? perm_bucket(ids[j], n_experts) : 0;
    if (valid) atomicOr(&lane_mask[wave][b], 1ull << lane);
    __syncthreads();
    if (valid) {
      uint32_t pos = base[b] + lanes_below(lane_mask[wave][b]);
      for (int w = 0; w < wave; ++w) pos += (uint32_t)__popcll(lane_mask[w][b]);
      if constexpr (kWritePermute) permute_index[pos] = j / k;
      unpermute_index[j] = pos;
    }
    __syncthreads();
    // Carry this tile's counts into base and clear the masks for the next tile.
    for (int i = tid; i < nb; i += kPermThreads) {
      uint32_t c = 0u;
#pragma unroll
      for (int w = 0; w < kPermWaves; ++w) {
        c += (uint32_t)__popcll(lane_mask[w][i]);
        lane_mask[w][i] = 0ull;
      }
      base[i] += c;
    }
    __syncthreads();
  }
}

// One launch: workgroup c owns the entries [c * chunk, (c + 1) * chunk) in
// tiles of kPermThreads, and counts all n ids per bucket in LDS, those before
// its chunk (before) and the others (after), one LDS atomic per id. Each
// workgroup reads all n ids once more than a per-chunk count would, so the
// grid is capped: at n = 12288 (2048 tokens, top 6) that is 12 workgroups and
// 1.2 MB of L2 reads. kCombine counts through perm_count; it is used for
// k <= 2 only: with more picks per token (distinct experts per token), a
// wave's 64 entries hold at most 64 / k of any one expert, and the combining
// step costs more than it saves (6.9 against 6.0 us at 2048 tokens x top 6).
template <bool kCombine>
__global__ __launch_bounds__(kPermThreads) void moe_permutation(const int64_t* __restrict__ ids, int64_t n, int64_t k,
                                                                int n_experts, int64_t chunk,
                                                                int64_t* __restrict__ permute_index,
                                                                int64_t* __restrict__ unpermute_index) {
  // before = sides[0], after = sides[1]
  __shared__ uint32_t sides[2 * kPermBuckets], base[kPermBuckets];
  __shared__ unsigned long long lane_mask[kPermWaves][kPermBuckets];
  uint32_t* before = sides;
  uint32_t* after = sides + kPermBuckets;
  const int tid = threadIdx.x;
  const int nb = n_experts + 1;
  for (int i = tid; i < 2 * kPermBuckets; i += kPermThreads) sides[i] = 0u;
  for (int i = tid; i < kPermWaves * kPermBuckets; i += kPermThreads) (&lane_mask[0][0])[i] = 0ull;
  __syncthreads();
  const int64_t c0 = (int64_t)blockIdx.x * chunk;
  const int64_t c1 = c0 + chunk < n ? c0 + chunk : n;
  // kPermUnroll ids per thread in flight before their LDS atomics (one DRAM
  // round trip per kPermUnroll ids instead of per id).
  for (int64_t j0 = tid; j0 < n; j0 += (int64_t)kPermThreads * kPermUnroll) {
    int64_t v[kPermUnroll];
#pragma unroll
    for (int u = 0; u < kPermUnroll; ++u) {
      const int64_t j = j0 + (int64_t)u * kPermThreads;
      v[u] = j < n ? ids[j] : 0;
    }
#pragma unroll
    for (int u = 0; u < kPermUnroll; ++u) {
      const int64_t j = j0 + (int64_t)u * kPermThreads;
      if (j < n) {
        const int key = perm_bucket(v[u], n_experts) + (j < c0 ? 0 : kPermBuckets);
        if constexpr (kCombine) {
          perm_count(sides, key);
        } else {
          atomicAdd(&sides[key], 1u);
        }
      }
    }
  }
  __syncthreads();
  if (tid < 64) perm_bases(after, before, base, nb, tid);
  __syncthreads();
  perm_rank_chunk<true>(ids, k, n_experts, c0, c1, base, lane_mask, permute_index, unpermute_index);
}

// Three launches from kPermSplitMin entries on, so that each id is counted
// once: the cost of the one-launch kernel grows with n x workgroups (uniform
// ids, top 8 of 256: 14.0 against 22.9 us at 16384 tokens, 26.4 against 81.2
// at 65536; the one launch is faster up to 49152 entries). The output
// buffers carry the intermediate results between the launches (stream order
// separates them):
//   1. moe_permutation_count: workgroup c counts its own chunk per bucket and
//      stores the counts in permute_index's memory as uint32 [G][nb];
//   2. moe_permutation_rank: workgroup c sums the counts of the chunks before
//      its own (before) and of the others (after), then ranks its chunk as the
//      one-launch kernel does and writes unpermute_index only;
//   3. moe_permutation_invert: permute_index[unpermute_index[i]] = i / k,
//      overwriting the counts.
// The G x nb x 4 bytes of counts fit in permute_index's n x 8 bytes, since
// G <= n / kPermSplitChunk + 1 and nb <= kPermBuckets.
constexpr int64_t kPermSplitMin = 65536, kPermSplitChunk = 2048;
constexpr int kPermSplitMaxGroups = 256;

__global__ __launch_bounds__(kPermThreads) void moe_permutation_count(const int64_t* __restrict__ ids, int64_t n,
                                                                      int n_experts, int64_t chunk,
                                                                      uint32_t* __restrict__ counts) {
  __shared__ uint32_t hist[kPermBuckets];
  const int tid = threadIdx.x;
  const int nb = n_experts + 1;
  for (int i = tid; i < nb; i += kPermThreads) hist[i] = 0u;
  __syncthreads();
  const int64_t c0 = (int64_t)blockIdx.x * chunk;
  const int64_t c1 = c0 + chunk < n ? c0 + chunk : n;
  for (int64_t j0 = c0 + tid; j0 < c1; j0 += (int64_t)kPermThreads * kPermUnroll) {
    int64_t v[kPermUnroll];
#pragma unroll
    for (int u = 0; u < kPermUnroll; ++u) {
      const int64_t j = j0 + (int64_t)u * kPermThreads;
      v[u] = j < c1 ? ids[j] : 0;
    }
#pragma unroll
    for (int u = 0; u < kPermUnroll; ++u) {
      if (j0 + (int64_t)u * kPermThreads < c1) perm_count(hist, perm_bucket(v[u], n_experts));
    }
  }
  __syncthreads();
  for (int i = tid; i < nb; i += kPermThreads) counts[(int64_t)blockIdx.x * nb + i] = hist[i];
}

__global__ __launch_bounds__(kPermThreads) void moe_permutation_rank(const int64_t* __restrict__ ids, int64_t n,
                                                                     int64_t k, int n_experts, int64_t chunk,
                                                                     const uint32_t* __restrict__ counts,
                                                                     int64_t* __restrict__ unpermute_index) {
  __shared__ uint32_t after[kPermBuckets], before[kPermBuckets], base[kPermBuckets];
  __shared__ unsigned long long lane_mask[kPermWaves][kPermBuckets];
  const int tid = threadIdx.x;
  const int nb = n_experts + 1;
  for (int i = tid; i < nb; i += kPermThreads) {
    after[i] = 0u;
    before[i] = 0u;
  }
  for (int i = tid; i < kPermWaves * kPermBuckets; i += kPermThreads) (&lane_mask[0][0])[i] = 0ull;
  __syncthreads();
  // counts[g][b] for every chunk g: flat index i = g * nb + b, coalesced
  // (at most kPermSplitMaxGroups x kPermBuckets of them, so 32-bit).
  const uint32_t n_counts = gridDim.x * (uint32_t)nb, mine = blockIdx.x * (uint32_t)nb;
  for (uint32_t i0 = tid; i0 < n_counts; i0 += kPermThreads * kPermUnroll) {
    uint32_t v[kPermUnroll];
#pragma unroll
    for (int u = 0; u < kPermUnroll; ++u) {
      const uint32_t i = i0 + u * kPermThreads;
      v[u] = i < n_counts ? counts[i] : 0u;
    }
#pragma unroll
    for (int u = 0; u < kPermUnroll; ++u) {
      const uint32_t i = i0 + u * kPermThreads;
      if (i < n_counts && v[u] != 0u) atomicAdd(i < mine ? &before[i % nb] : &after[i % nb], v[u]);
    }
  }
  __syncthreads();
  if (tid < 64) perm_bases(after, before, base, nb, tid);
  __syncthreads();
  const int64_t c0 = (int64_t)blockIdx.x * chunk;
  const int64_t c1 = c0 + chunk < n ? c0 + chunk : n;
  perm_rank_chunk<false>(ids, k, n_experts, c0, c1, base, lane_mask, nullptr, unpermute_index);
}

__global__ __launch_bounds__(256) void moe_permutation_invert(const int64_t* __restrict__ unpermute_index, int64_t n,
                                                              int64_t k, int64_t* __restrict__ permute_index) {
  // n < 2^31 (the launcher's bound), so the token index is a 32-bit quotient.
  const uint32_t kk = (uint32_t)k;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    permute_index[unpermute_index[i]] = (int64_t)((uint32_t)i / kk);
  }
}

}  // namespace
}  // namespace cck

using namespace cck;

extern "C" int32_t launch_token_gather_fwd(const void* src, const int64_t* indices, void* dst,
                                           int64_t n_dst_rows, int64_t hidden_dim, int32_t dtype,
                                           void* stream) {
  return gather(src, indices, dst, n_dst_rows, hidden_dim, dtype, kNoBound, static_cast<hipStream_t>(stream));
}

extern "C" int32_t launch_token_gather_checked_fwd(const void* src, const int64_t* indices, void* dst,
                                                   int64_t n_src_rows, int64_t n_dst_rows,
                                                   int64_t hidden_dim, int32_t dtype, void* stream) {
  if (n_src_rows < 0) return (int32_t)hipErrorInvalidValue;
  return gather(src, indices, dst, n_dst_rows, hidden_dim, dtype, n_src_rows, static_cast<hipStream_t>(stream));
}

extern "C" int32_t launch_token_combine_fwd(const void* expert_output, const int64_t* unpermute_index,
                                            const float* weights, void* combined, int64_t n_tokens,
                                            int64_t k, int64_t hidden_dim, int32_t dtype, void* stream) {
  return combine(expert_output, unpermute_index, weights, combined, n_tokens, k, hidden_dim, dtype, kNoBound,
                 static_cast<hipStream_t>(stream));
}

extern "C" int32_t launch_token_combine_checked_fwd(const void* expert_output, const int64_t* unpermute_index,
                                                    const float* weights, void* combined,
                                                    int64_t n_expert_rows, int64_t n_tokens, int64_t k,
                                                    int64_t hidden_dim, int32_t dtype, void* stream) {
  if (n_expert_rows < 0) return (int32_t)hipErrorInvalidValue;
  return combine(expert_output, unpermute_index, weights, combined, n_tokens, k, hidden_dim, dtype,
                 n_expert_rows, static_cast<hipStream_t>(stream));
}

extern "C" int32_t launch_moe_permutation_fwd(const int64_t* topk_indices, int64_t* permute_index,
                                              int64_t* unpermute_index, int64_t n_tokens, int64_t k,
                                              int64_t num_experts, void* stream) {
  if (n_tokens < 0 || k < 0 || num_experts < 1 || num_experts > kPermMaxExperts) return (int32_t)hipErrorInvalidValue;
  if (k > 0 && n_tokens > INT32_MAX / k) return (int32_t)hipErrorInvalidValue;  // positions are 32-bit
  const int64_t n = n_tokens * k;
  if (n == 0) return (int32_t)hipSuccess;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (n >= kPermSplitMin) {
    int64_t chunk = kPermSplitChunk;
    if ((n + chunk - 1) / chunk > kPermSplitMaxGroups) {
      chunk = (n + kPermSplitMaxGroups - 1) / kPermSplitMaxGroups;
      chunk = (chunk + kPermThreads - 1) / kPermThreads * kPermThreads;
    }
    const unsigned groups = (unsigned)((n + chunk - 1) / chunk);
    // The counts ([groups][nb] uint32) live in permute_index until the last launch.
    uint32_t* counts = reinterpret_cast<uint32_t*>(permute_index);
    moe_permutation_count<<<groups, kPermThreads, 0, st>>>(topk_indices, n, (int)num_experts, chunk, counts);
    moe_permutation_rank<<<groups, kPermThreads, 0, st>>>(topk_indices, n, k, (int)num_experts, chunk, counts,
                                                          unpermute_index);
    const int64_t blocks = (n + 255) / 256;
    moe_permutation_invert<<<(unsigned)(blocks < 2048 ? blocks : 2048), 256, 0, st>>>(unpermute_index, n, k,
                                                                                     permute_index);
    return launch_status();
  }
  const int64_t tiles = (n + kPermThreads - 1) / kPermThreads;
  const int64_t groups = tiles < kPermMaxGroups ? tiles : kPermMaxGroups;
  const int64_t chunk = (tiles + groups - 1) / groups * kPermThreads;
  const unsigned grid = (unsigned)((n + chunk - 1) / chunk);
  if (k <= 2) {
    moe_permutation<true><<<grid, kPermThreads, 0, st>>>(topk_indices, n, k, (int)num_experts, chunk, permute_index,
                                                         unpermute_index);
  } else {
    moe_permutation<false><<<grid, kPermThreads, 0, st>>>(topk_indices, n, k, (int)num_experts, chunk,
                                                          permute_index, unpermute_index);
  }
  return launch_status();
}
