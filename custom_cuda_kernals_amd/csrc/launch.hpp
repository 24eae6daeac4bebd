// Host-side helpers shared by the launchers: dtype / format dispatch and the
// error convention of the C ABI (0 == hipSuccess; hipErrorInvalidValue for an
// unknown tag, returned before any device call; the launch status otherwise).
#pragma once

#include <atomic>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "cdna4.hpp"
#include "../../include/custom_kernels_amd.h"

namespace cck {

template <int V>
using IntC = std::integral_constant<int, V>;

template <class Fn>
inline int32_t with_codec(int32_t dtype, Fn&& fn) {
  switch (dtype) {
    case kF32: return fn(CodecF32{});
    case kF16: return fn(CodecF16{});
    case kBF16: return fn(CodecBF16{});
    default: return (int32_t)hipErrorInvalidValue;
  }
}

template <class Fn>
inline int32_t with_fp8(int32_t fmt, Fn&& fn) {
  switch (fmt) {
    case kF8E4M3: return fn(IntC<kF8E4M3>{});
    case kF8E5M2: return fn(IntC<kF8E5M2>{});
    default: return (int32_t)hipErrorInvalidValue;
  }
}

// Workgroup shape of a register-resident row kernel: THREADS threads, each
// holding up to ITEMS 16-byte vectors of the row.
template <int T, int I>
struct RowShape {
  static constexpr int kThreads = T;
  static constexpr int kItems = I;
};

// Calls fn(S{}) for the first shape S that holds a row of nvec vectors;
// returns false when none does (the caller then uses its looping kernel).
template <class S, class... Rest, class Fn>
inline bool pick_row_shape(int64_t nvec, Fn&& fn) {
  if (nvec <= (int64_t)S::kThreads * S::kItems) {
    fn(S{});
    return true;
  }
  if constexpr (sizeof...(Rest) > 0) {
    return pick_row_shape<Rest...>(nvec, fn);
  } else {
    return false;
  }
}

inline int32_t launch_status() { return (int32_t)hipGetLastError(); }

inline bool host_aligned(const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }

// Workgroup cap of the row-per-workgroup kernels (rows, tokens, MoE rows):
// one workgroup per row up to it, and beyond it each workgroup loops over
// rows blockIdx.x, blockIdx.x + gridDim.x, ... 65536 workgroups fill the
// 256 CUs many times over, so large inputs lose nothing, and the looping
// path is reachable at test sizes (a few MB).
constexpr int64_t kMaxRowGroups = 65536;

inline unsigned row_grid(int64_t rows) {
  return (unsigned)(rows < kMaxRowGroups ? rows : kMaxRowGroups);
}

// Dynamic LDS to reserve per workgroup (the kernel never touches it) so that
// at most N workgroups are resident on a CU: gfx950 has 160 KB of LDS per
// CU, and N * bytes <= 160 KB < (N + 1) * bytes. Some streaming kernels run
// faster with fewer workgroups in flight than their registers allow.
template <int N>
constexpr unsigned kLdsForGroupsPerCu = (160u * 1024u * 2u) / (2u * N + 1u);
static_assert(3 * kLdsForGroupsPerCu<3> <= 160u * 1024u && 4 * kLdsForGroupsPerCu<3> > 160u * 1024u);
static_assert(6 * kLdsForGroupsPerCu<6> <= 160u * 1024u && 7 * kLdsForGroupsPerCu<6> > 160u * 1024u);
static_assert(kLdsForGroupsPerCu<3> <= 64u * 1024u);  // within the default per-workgroup limit

// Workgroups of KERNEL (launched with `threads` threads and no dynamic LDS)
// that the current device holds at once: occupancy per CU x CUs, looked up
// once per kernel and device; 0 when a query fails.
template <auto KERNEL>
int64_t resident_groups(int threads) {
  constexpr int kDevices = 64;
  static std::atomic<int> cache[kDevices] = {};  // -1 = the query failed
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kDevices) {
    (void)hipGetLastError();
    return 0;
  }
  int g = cache[dev].load(std::memory_order_relaxed);
  if (g == 0) {
    int per_cu = 0, cus = 0;
    const bool ok = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, KERNEL, threads, 0) == hipSuccess &&
                    hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess;
    if (!ok) (void)hipGetLastError();  // a failed query must not surface as the launch's status
    g = ok && per_cu * cus > 0 ? per_cu * cus : -1;
    cache[dev].store(g, std::memory_order_relaxed);
  }
  return g > 0 ? g : 0;
}

inline unsigned flat_grid(int64_t work_items, int threads, int64_t cap) {
  int64_t g = (work_items + threads - 1) / threads;
  if (g < 1) g = 1;
  return (unsigned)(g < cap ? g : cap);
}

}  // namespace cck
