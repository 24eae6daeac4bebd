// Row sums of fp32 addends in the fixed order of PyTorch's CPU float sum over
// a contiguous last dimension: the order behind the variance
// `upcast.pow(2).mean(dim=-1)` of the reference's eager RMSNorm
// (baselines/rmsnorm_residual.py:133), whose last bits reach every output
// element through rsqrt. Reproducing it makes the kernel's y equal the eager
// y bit for bit.
//
// The order, for a row of n addends:
//   * vectors of 8 lanes: element e is lane e % 8 of vector V = e / 8, for the
//     nv = n / 8 whole vectors;
//   * vector V = 4 i + k is step i of slot k, for i < steps = nv / 4;
//   * per (slot, lane) the steps fold into acc0 from zero in blocks of 2^P
//     steps, P = max(4, ceil_log2(steps) / 4); after each whole block
//     acc1 += acc0; after every 2^P blocks acc2 += acc1 (acc1 = 0), after
//     every 2^(2P) blocks acc3 += acc2 (acc2 = 0); the steps % 2^P trailing
//     steps fold into acc0; p = ((acc0 + acc1) + acc2) + acc3;
//   * the nv % 4 leftover vectors are added to slot 0 in order, then
//     p0 = ((p0 + p1) + p2) + p3 lane by lane;
//   * total = ((0 + the n % 8 trailing scalars in order) + p0[0]) + ... + p0[7].
// Rows under 8 addends are 4 slots of single elements (leftovers into slot 0).
//
// On the device a "region" is 64 consecutive vectors (512 addends): with
// P = 4 that is one whole block, so a region's 16 steps x 4 slots x 8 lanes
// are 32 independent sequential folds of 16 addends. The addends of a region
// are staged in LDS as a[64][8] (vector-major), and lane c < 32 of the
// folding wave (slot c / 8, lane c % 8) reads a[4 j + c / 8][c % 8] =
// a_flat[32 j + c] for step j: consecutive lanes, consecutive words.
#pragma once

#include "cdna4.hpp"

namespace cck {

constexpr int kSumLanes = 8;
constexpr int kRegionVecs = 64;                     // vectors per region
constexpr int kRegionAddends = kRegionVecs * kSumLanes;
constexpr int kFoldLanes = 32;                      // 4 slots x 8 lanes

struct AtenSumPlan {
  int64_t nv;     // whole 8-lane vectors
  int64_t steps;  // nv / 4
  int p;          // log2 of the block length in steps
  int64_t nfull;  // whole blocks
  int ntrail;     // steps % 2^p
  int nleft;      // nv % 4
  int ntail;      // n % 8
  __device__ explicit AtenSumPlan(int64_t n) {
    nv = n / kSumLanes;
    steps = nv / 4;
    const int cl = steps <= 2 ? 1 : 64 - __builtin_clzll((unsigned long long)(steps - 1));
    p = cl / 4 > 4 ? cl / 4 : 4;
    nfull = steps >> p;
    ntrail = (int)(steps & ((1 << p) - 1));
    nleft = (int)(nv & 3);
    ntail = (int)(n & 7);
  }
  __device__ bool has_tail() const { return (ntrail | nleft | ntail) != 0; }
};

__device__ inline float readlane_f32(float v, int lane) {
  return bits_f32((uint32_t)__builtin_amdgcn_readlane((int)f32_bits(v), lane));
}


// Continue the folds of lanes c < 32 over `nsteps` steps of a staged region.
__device__ inline float fold_region(const float* a, int nsteps, int c, float acc) {
  for (int j = 0; j < nsteps; ++j) acc = acc + a[kFoldLanes * j + c];
  return acc;
}
__device__ inline float fold_region16(const float* a, int c) {
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < 16; ++j) acc = acc + a[kFoldLanes * j + c];
  return acc;
}

// Tail data of a row, staged by the wave that holds the last region:
//   [0, 32)  the folds of the trailing steps (acc0), fold c at word c;
//   [32, 56) the squares of the leftover vectors, 8 per vector;
//   [56, 64) the trailing scalars.
constexpr int kTailWords = 64;

// The addends here are squares, never -0, so every partial sum is +0, a
// positive number, +inf or NaN, and adding a +0 leaves it unchanged. Where
// the order adds a level that is still zero (or a zero acc0), the addition
// is skipped without changing a bit.

// The cascade of fold c (slot c / 8, lane c % 8) of one row, in lane c < 32.
struct FoldCascade {
  float a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
  bool has2 = false, has3 = false;
  // Add the fold f of whole block b of a row with block exponent p.
  __device__ void add(float f, int64_t b, int p) {
    a1 = a1 + f;
    const int64_t done = b + 1;
    if ((done & ((int64_t(1) << p) - 1)) == 0) {
      a2 = a2 + a1;
      a1 = 0.0f;
      has2 = true;
      if ((done & ((int64_t(1) << (2 * p)) - 1)) == 0) {
        a3 = a3 + a2;
        a2 = 0.0f;
        has3 = true;
      }
    }
  }
  // ((acc0 + acc1) + acc2) + acc3 with acc0 the trailing steps' fold.
  __device__ float slot_sum(const AtenSumPlan& pl, const float* tail, int c) const {
    float q = a1;
    if (pl.ntrail) q = tail[c] + q;
    if (has2) q = q + a2;
    if (has3) q = q + a3;
    return q;
  }
};

// Bitmask-mode ds_swizzle within 32-lane halves: lane i reads lane i ^ X.
template <int X>
__device__ inline float swizzle_xor(float v) {
  return bits_f32((uint32_t)__builtin_amdgcn_ds_swizzle((int)f32_bits(v), (X << 10) | 0x1f));
}

// From the slot sums q of lanes c < 32 (0 elsewhere) to the row total: the
// leftover vectors into slot 0, the slots combined in order in lanes 0..7,
// then ((0 + trailing scalars) + lane 0) + ... + lane 7. Every lane of the
// wave must be active; the result is wave-uniform.
__device__ inline float aten_combine(const AtenSumPlan& pl, float q, const float* tail, int lane) {
  if (lane < kSumLanes) {
    for (int i = 0; i < pl.nleft; ++i) q = q + tail[32 + kSumLanes * i + lane];
  }
  const float q1 = swizzle_xor<8>(q), q2 = swizzle_xor<16>(q), q3 = swizzle_xor<24>(q);
  const float p = ((q + q1) + q2) + q3;
  float t = 0.0f;
  for (int e = 0; e < pl.ntail; ++e) t = t + tail[56 + e];
  t = t + readlane_f32(p, 0);
#pragma unroll
  for (int l = 1; l < kSumLanes; ++l) t = t + readlane_f32(p, l);
  return t;
}

// Rows under 8 addends: four slots of single elements, leftovers into slot
// 0, slots combined in order (the scalars are tail words 56..).
__device__ inline float aten_scalar_row(const AtenSumPlan& pl, const float* tail) {
  const int n = pl.ntail;
  const int s = n / 4;
  float p0 = s ? tail[56] : 0.0f;
  for (int e = 4 * s; e < n; ++e) p0 = p0 + tail[56 + e];
  for (int k = 1; k < 4; ++k) p0 = p0 + (s ? tail[56 + k] : 0.0f);
  return p0;
}

// Finish the row sum from all its block folds `bs` (nfull blocks of 32
// words) and the staged tail, for rows with 16-step blocks (P = 4). MAXB
// bounds nfull at compile time. Up to 16 blocks the level-2 promotion can
// only happen after the 16th and last block, where it moves acc1 to acc2
// unchanged, so the cascade is one running sum; its loads are all issued
// before the first addition (blocks past the row are read and not used).
template <int MAXB>
__device__ inline float aten_finish(const AtenSumPlan& pl, const float* bs, const float* tail, int lane) {
  if (pl.nv == 0) return aten_scalar_row(pl, tail);
  float q = 0.0f;
  if (lane < kFoldLanes) {
    if constexpr (MAXB <= 16) {
      float f[MAXB];
#pragma unroll
      for (int b = 0; b < MAXB; ++b) f[b] = bs[b * kFoldLanes + lane];
      q = pl.nfull ? f[0] : 0.0f;
#pragma unroll
      for (int b = 1; b < MAXB; ++b) q = (b < pl.nfull) ? q + f[b] : q;
      if (pl.ntrail) q = tail[lane] + q;
    } else {
      FoldCascade cs;
      for (int b = 0; b < pl.nfull; ++b) cs.add(bs[b * kFoldLanes + lane], b, 4);
      q = cs.slot_sum(pl, tail, lane);
    }
  }
  return aten_combine(pl, q, tail, lane);
}

// The same finish for a row of exactly NB whole regions (n = 512 * NB, so
// nv = 64 NB, steps = 16 NB, P = 4 up to 2^24 addends, and no trailing
// steps, leftover vectors or trailing scalars), with every count known at
// compile time: the cascade is unrolled and no tail words are read. The
// result is the same bits as aten_finish for that n.
template <int NB>
__device__ inline float aten_finish_full(const float* bs, int lane) {
  float q = 0.0f;
  if (lane < kFoldLanes) {
    if constexpr (NB <= 16) {
      float f[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) f[b] = bs[b * kFoldLanes + lane];
      q = f[0];
#pragma unroll
      for (int b = 1; b < NB; ++b) q = q + f[b];
    } else {
      // FoldCascade's operations, a group of 16 blocks (acc1 from zero, then
      // promoted into acc2) at a time, so at most 16 folds are held at once.
      float a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll 1
      for (int j = 0; j < NB / 16; ++j) {
        float f[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) f[i] = bs[(16 * j + i) * kFoldLanes + lane];
        a1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) a1 = a1 + f[i];
        a2 = a2 + a1;
        a1 = 0.0f;
        if ((16 * (j + 1)) % 256 == 0) {
          a3 = a3 + a2;
          a2 = 0.0f;
        }
      }
#pragma unroll
      for (int b = NB / 16 * 16; b < NB; ++b) a1 = a1 + bs[b * kFoldLanes + lane];
      q = a1;
      q = q + a2;
      if constexpr (NB >= 256) q = q + a3;
    }
  }
  const float q1 = swizzle_xor<8>(q), q2 = swizzle_xor<16>(q), q3 = swizzle_xor<24>(q);
  const float p = ((q + q1) + q2) + q3;
  float t = readlane_f32(p, 0);
#pragma unroll
  for (int l = 1; l < kSumLanes; ++l) t = t + readlane_f32(p, l);
  return t;
}

// Copy the leftover vectors and trailing scalars that fall in a staged region
// (first vector `first_vec` of the row) to the tail words.
__device__ inline void stage_tail_parts(const AtenSumPlan& pl, const float* a, int64_t first_vec, int lane,
                                        float* tail) {
  if (lane < kSumLanes * pl.nleft) {
    const int64_t v = pl.steps * 4 + lane / kSumLanes;
    if (v >= first_vec && v < first_vec + kRegionVecs) {
      tail[32 + lane] = a[(v - first_vec) * kSumLanes + lane % kSumLanes];
    }
  }
  if (lane < pl.ntail) {
    const int64_t e = pl.nv * kSumLanes + lane - first_vec * kSumLanes;
    if (e >= 0 && e < kRegionAddends) tail[56 + lane] = a[e];
  }
}

// Row sum for the register-resident row kernels: thread t holds 16-byte
// vectors u = t + k * THREADS of the row (VEC addends each), P = 4 (rows of at
// most 2^23 addends). The kernel hands each vector's squares to item(k, sq)
// as soon as it has them (zeros past the row), then calls total().
//   VEC == 8: one 16-byte vector is one 8-lane vector, so item k of wave w
//     is region w + NW * k whole. The wave stages its regions in its own part
//     of `stage` and folds them without waiting for the other waves; a fold
//     needs 32 lanes, so the two halves of the wave fold two regions at once
//     (SLOTS = 2 staged regions per wave) where the shape has two or more
//     items per thread;
//   VEC == 4: two waves share a region, so the row is staged whole in `stage`
//     (THREADS * ITEMS * 4 floats) and folded behind a barrier.
// `bsum` holds 2 x NREG x 32 floats and `tail` 2 x 64, alternated by `parity`
// so a wave running ahead into the next row never overwrites words that a
// slower wave still reads.
//   FULL (VEC == 8 only): the row is exactly THREADS * ITEMS vectors and a
//     whole number of regions, so every count is a compile-time constant and
//     no tail is staged (aten_finish_full).
template <int VEC, int THREADS, int ITEMS, bool FULL = false>
struct ResidentRowSum {
  static constexpr int NW = THREADS / 64;
  static constexpr int NREG = (THREADS * ITEMS * VEC + kRegionAddends - 1) / kRegionAddends;
  static constexpr int SLOTS = (ITEMS >= 2 && NW <= 8) ? 2 : 1;
  static constexpr int kStageFloats = VEC == 8 ? NW * SLOTS * kRegionAddends : THREADS * ITEMS * VEC;
  static_assert(!FULL || (VEC == 8 && (THREADS * ITEMS * VEC) % kRegionAddends == 0),
                "a full row is whole regions of 8-lane vectors");
  const AtenSumPlan& pl;
  float* stage;
  float* bs;
  float* tl;
  int lane, w, nreg;
  __device__ ResidentRowSum(const AtenSumPlan& plan, float* stage_, float* bsum, float* tail, int parity)
      : pl(plan), stage(stage_), bs(bsum + parity * NREG * kFoldLanes), tl(tail + parity * kTailWords) {
    lane = threadIdx.x & 63;
    w = threadIdx.x >> 6;
    nreg = FULL ? NREG : (int)pl.nfull + (pl.has_tail() ? 1 : 0);
  }
  // Fold region `reg` staged at `a`, as fold c (c < 32) of this lane.
  __device__ void fold_one(const float* a, int reg, int c) {
    if (FULL || reg < pl.nfull) {
      bs[reg * kFoldLanes + c] = fold_region16(a, c);
    } else {
      tl[c] = fold_region(a, pl.ntrail, c, 0.0f);
      stage_tail_parts(pl, a, (int64_t)reg * kRegionVecs, c, tl);
    }
  }
  __device__ void item(int k, const float (&sq)[VEC]) {
    if constexpr (VEC == 8) {
      if (FULL || w + NW * k < nreg) {
        float* a = stage + (w * SLOTS + k % SLOTS) * kRegionAddends;
#pragma unroll
        for (int i = 0; i < VEC; ++i) a[lane * VEC + i] = sq[i];
      }
      if (k % SLOTS == SLOTS - 1 || k == ITEMS - 1) {
        // LDS accesses of one wave complete in order; the wave barriers only
        // keep the compiler from moving the fold's reads above the staging
        // writes, or the next staging writes above the fold's reads.
        __builtin_amdgcn_wave_barrier();
        const int h = lane >> 5;
        const int kk = k - k % SLOTS + h;  // the item this half folds
        if (kk < ITEMS && (SLOTS == 2 || h == 0) && (FULL || w + NW * kk < nreg)) {
          fold_one(stage + (w * SLOTS + h) * kRegionAddends, w + NW * kk, lane & 31);
        }
        __builtin_amdgcn_wave_barrier();
      }
    } else {
      const int u = threadIdx.x + k * THREADS;
#pragma unroll
      for (int i = 0; i < VEC; ++i) stage[u * VEC + i] = sq[i];
    }
  }
  // Wave-uniform row total (all threads of the workgroup must call it).
  __device__ float total() {
    if constexpr (VEC != 8) {
      __syncthreads();
      for (int reg = 2 * w + (lane >> 5); reg < nreg; reg += 2 * NW) {
        fold_one(stage + reg * kRegionAddends, reg, lane & 31);
      }
    }
    __syncthreads();
    if constexpr (FULL) {
      return aten_finish_full<NREG>(bs, lane);
    } else {
      return aten_finish<NREG>(pl, bs, tl, lane);
    }
  }
};

}  // namespace cck
