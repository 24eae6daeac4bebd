// MoE top-k router (softmax gating), for gfx950.
//
// Semantics (baselines/moe_router.py:117-128):
//   probs = softmax(float(logits), dim=-1)                      fp32
//   topk_weights, topk_indices = topk(probs, k)                 descending
//   if renormalize: topk_weights /= topk_weights.sum(-1)
// with every fp32 step as torch-CPU computes it on an AVX-512 host, so the
// weights are bit for bit the eager baseline's there:
//   * softmax (ATen's vectorised last-dim kernel, 16-float vectors):
//     m = max(x) (NaN-propagating); e_i = xexpf(x_i - m) with SLEEF's 1-ulp
//     expf (the same steps as the fp32 SwiGLU's sigmoid, silu.hpp); the sum
//     of e in 16 lane classes, lane L adding e_L, e_{L+16}, ... in order over
//     the whole vectors and then the tail element of its class, combined as
//     L + (L xor 8), then xor 4, 2, 1 (lane 0's value); below 16 experts the
//     sum is e_0 + e_1 + ... in order; p_i = e_i * RN(1 / sum);
//   * the renormalising sum in ATen's row-sum order (aten_small_row_sum
//     below), then an IEEE division.
// Ties between equal probabilities go to the lower expert index (torch's
// topk orders exact ties its own way).
//
// Three forms, by expert count E (and token count T), the same steps and
// results in each:
//   * E <= 8: one lane per token (moe_router_lanes);
//   * 9 <= E <= 32, and E <= 64 from T = 4096 on: four lanes per token, each
//     holding its quarter of every 16-expert stripe (moe_router_groups);
//     65 <= E <= 256 from T = 8192 (E <= 128) or 12288 on: eight lanes;
//   * otherwise one wave per token (moe_router_waves), below.
// One wave64 per token holds up to 256 experts (4 per lane, expert
// e = lane + 64 * slot). The max is a wave all-reduction (DPP). The
// exponentials go to a per-wave LDS row; every lane then runs its lane
// class's ordered sum (lanes 16-63 repeat lanes 0-15), and the xor tree is
// four DPP row shifts (lane 0 reads lanes 8, 4, 2, 1 above it). Each of the k
// selection rounds is a wave arg-max in two all-reductions: the largest
// probability (as integer bits; probabilities are >= +0) and then the
// smallest expert index holding it. The selected weights go to the same LDS
// row for the renormalising sum; round i's result is kept by lane i % 64, so
// the weights are stored with one coalesced pass at the end.
#include "launch.hpp"
#include "silu.hpp"

namespace cck {
namespace {

#pragma clang fp contract(off)

constexpr int kWavesPerGroup = 4;
constexpr int kSlots = 4;                // experts per lane
constexpr int kMaxExperts = 64 * kSlots;  // 256, as the reference (moe_router.cu kMaxLocal * 32)
constexpr int kSoftmaxLanes = 16;        // ATen's AVX-512 float vector

constexpr int kDppRowShl8 = 0x108, kDppRowShl4 = 0x104, kDppRowShl2 = 0x102, kDppRowShl1 = 0x101;

// torch-CPU's softmax sum over the n values of this wave's LDS row (header
// comment); wave-uniform. LDS accesses of one wave complete in order, so the
// caller only needs a wave barrier between its writes of e and this call.
__device__ inline float softmax_sum_avx512(const float* e, int n, int lane) {
  if (n < kSoftmaxLanes) {
    float s = e[0];
    for (int i = 1; i < n; ++i) s = s + e[i];
    return s;
  }
  const int full = n / kSoftmaxLanes;
  const int cls = lane & (kSoftmaxLanes - 1);
  float acc = e[cls];
  for (int v = 1; v < full; ++v) acc = acc + e[cls + kSoftmaxLanes * v];
  if (cls < n - full * kSoftmaxLanes) acc = acc + e[full * kSoftmaxLanes + cls];
  // Lane L adds lane L + 8, then + 4, + 2, + 1 (within its 16-lane row): for
  // lane 0 that is the xor tree, as addition is commutative.
  acc = acc + bits_f32(dpp<kDppRowShl8>(f32_bits(acc)));
  acc = acc + bits_f32(dpp<kDppRowShl4>(f32_bits(acc)));
  acc = acc + bits_f32(dpp<kDppRowShl2>(f32_bits(acc)));
  acc = acc + bits_f32(dpp<kDppRowShl1>(f32_bits(acc)));
  return bits_f32((uint32_t)__builtin_amdgcn_readfirstlane((int)f32_bits(acc)));
}

// ATen's float32 row sum of n < 512 non-negative addends v[0], v[STRIDE],
// v[2 * STRIDE], ..., serially: 8-lane vectors in 4 slots, each slot one
// running sum from zero (no 16-step block of a slot completes below 512
// addends, so the cascade's other levels stay zero), the leftover vectors
// into slot 0, then the trailing scalars and the 8 lanes in order; rows under
// 8 addends as scalars in 4 slots. Adding the zero levels (or a leading zero)
// changes no non-negative sum, so they are left out.
template <int STRIDE>
__device__ inline float aten_small_row_sum(const float* v, int n) {
  if (n < 8) {
    const int s = n >> 2;
    float p0 = s ? v[0] : 0.0f, p1 = s ? v[STRIDE] : 0.0f, p2 = s ? v[2 * STRIDE] : 0.0f,
          p3 = s ? v[3 * STRIDE] : 0.0f;
    for (int u = 4 * s; u < n; ++u) p0 = p0 + v[u * STRIDE];
    return ((p0 + p1) + p2) + p3;
  }
  const int nv = n >> 3, s = nv >> 2;
  float total = 0.0f;
  for (int e = nv * 8; e < n; ++e) total = total + v[e * STRIDE];
  for (int l = 0; l < 8; ++l) {
    float p0 = 0.0f, p1 = 0.0f, p2 = 0.0f, p3 = 0.0f;
    for (int i = 0; i < s; ++i) {
      p0 = p0 + v[((4 * i + 0) * 8 + l) * STRIDE];
      p1 = p1 + v[((4 * i + 1) * 8 + l) * STRIDE];
      p2 = p2 + v[((4 * i + 2) * 8 + l) * STRIDE];
      p3 = p3 + v[((4 * i + 3) * 8 + l) * STRIDE];
    }
    for (int vec = 4 * s; vec < nv; ++vec) p0 = p0 + v[(vec * 8 + l) * STRIDE];
    total = total + (((p0 + p1) + p2) + p3);
  }
  return total;
}

struct MaxI32 {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return (int32_t)a > (int32_t)b ? a : b; }
};
struct MinU32 {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return min(a, b); }
};

template <class C>
__global__ __launch_bounds__(256) void moe_router_waves(const void* __restrict__ logits,
                                                        float* __restrict__ topk_w,
                                                        int64_t* __restrict__ topk_i, int64_t n_tokens,
                                                        int n_experts, int k, int renormalize) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  __shared__ float rows[kWavesPerGroup][kMaxExperts];
  float* row = rows[wave];
  for (int64_t t = (int64_t)blockIdx.x * kWavesPerGroup + wave; t < n_tokens;
       t += (int64_t)gridDim.x * kWavesPerGroup) {
    float p[kSlots];
    bool live[kSlots];
    float mloc = -__builtin_inff();
#pragma unroll
    for (int s = 0; s < kSlots; ++s) {
      const int e = lane + 64 * s;
      live[s] = e < n_experts;
      p[s] = live[s] ? C::load1(logits, t * n_experts + e) : -__builtin_inff();
      mloc = __builtin_elementwise_maximum(mloc, p[s]);
    }
    const float m = bits_f32(wave_allreduce(f32_bits(mloc), MaxF32{}));
    // The previous token's reads of the row are done before it is rewritten.
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int s = 0; s < kSlots; ++s) {
      if (live[s]) {
        p[s] = SleefExpf::eval_ldexp(p[s] - m);
        row[lane + 64 * s] = p[s];
      }
    }
    __builtin_amdgcn_wave_barrier();
    const float inv = 1.0f / softmax_sum_avx512(row, n_experts, lane);
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int s = 0; s < kSlots; ++s) {
      if (live[s]) p[s] = p[s] * inv;
    }

    float sel_w[kSlots];
    uint32_t sel_e[kSlots];
    for (int i = 0; i < k; ++i) {
      // This lane's best remaining expert: slots ascend with the expert index,
      // so a strict > keeps the lower index on ties.
      int32_t key = -1;
      uint32_t mine = 0xffffffffu;
#pragma unroll
      for (int s = 0; s < kSlots; ++s) {
        if (live[s] && (int32_t)f32_bits(p[s]) > key) {
          key = (int32_t)f32_bits(p[s]);
          mine = (uint32_t)(lane + 64 * s);
        }
      }
      const uint32_t best = wave_allreduce((uint32_t)key, MaxI32{});
      const uint32_t sel = wave_allreduce((int32_t)best == key ? mine : 0xffffffffu, MinU32{});
#pragma unroll
      for (int s = 0; s < kSlots; ++s) {
        if ((uint32_t)(lane + 64 * s) == sel) live[s] = false;
      }
      const float val = bits_f32(best);
      if (lane == 0) row[i] = val;
      if (lane == (i & 63)) {
#pragma unroll
        for (int s = 0; s < kSlots; ++s) {
          if ((i >> 6) == s) {
            sel_w[s] = val;
            sel_e[s] = sel;
          }
        }
      }
    }
    float wsum = 1.0f;
    if (renormalize) {
      __builtin_amdgcn_wave_barrier();
      wsum = aten_small_row_sum<1>(row, k);
    }
#pragma unroll
    for (int s = 0; s < kSlots; ++s) {
      const int i = lane + 64 * s;
      if (i < k) {
        topk_w[t * k + i] = renormalize ? sel_w[s] / wsum : sel_w[s];
        topk_i[t * k + i] = (int64_t)sel_e[s];
      }
    }
  }
}

// One lane per token, for up to EMAX <= 8 experts: the same steps as
// moe_router_waves, each done serially in the lane's registers (the max over
// the row, the exponentials and their sum in index order, the k arg-max
// rounds over a live-expert mask with the lower index kept on ties). A wave
// holds 64 consecutive tokens, whose rows are contiguous, so VEC's 16-byte
// row loads are coalesced across the wave. The selected weights go to LDS in
// [round][thread] order (no bank conflicts, no barrier: each thread reads
// back only its own column) for the renormalising sum.
constexpr int kLaneThreads = 64;
constexpr int kLaneMaxExperts = 8;

template <class C, int EMAX, bool VEC>
__global__ __launch_bounds__(kLaneThreads) void moe_router_lanes(const void* __restrict__ logits,
                                                                 float* __restrict__ topk_w,
                                                                 int64_t* __restrict__ topk_i, int64_t n_tokens,
                                                                 int n_experts, int k, int renormalize) {
  static_assert(EMAX <= kLaneMaxExperts && EMAX < kSoftmaxLanes && (!VEC || EMAX % C::VEC == 0),
                "lane router shape");
  __shared__ float sel[EMAX][kLaneThreads];
  const int tid = threadIdx.x;
  const int64_t t = (int64_t)blockIdx.x * kLaneThreads + tid;
  if (t >= n_tokens) return;  // nothing below synchronises
  const int n = n_experts;
  float x[EMAX];
  if constexpr (VEC) {
    // n is a multiple of C::VEC and the rows are 16-byte aligned.
    const u32x4* r = reinterpret_cast<const u32x4*>(static_cast<const char*>(logits) + t * n * C::kBytes);
#pragma unroll
    for (int v = 0; v < EMAX / C::VEC; ++v) {
      float f[C::VEC];
      if (v * C::VEC < n) {
        C::unpack(__builtin_nontemporal_load(r + v), f);
      } else {
#pragma unroll
        for (int j = 0; j < C::VEC; ++j) f[j] = -__builtin_inff();
      }
#pragma unroll
      for (int j = 0; j < C::VEC; ++j) x[v * C::VEC + j] = f[j];
    }
  } else {
#pragma unroll
    for (int e = 0; e < EMAX; ++e) x[e] = e < n ? C::load1(logits, t * n + e) : -__builtin_inff();
  }
  float m = -__builtin_inff();
#pragma unroll
  for (int e = 0; e < EMAX; ++e) m = __builtin_elementwise_maximum(m, x[e]);
  float p[EMAX];
#pragma unroll
  for (int e = 0; e < EMAX; ++e) p[e] = e < n ? SleefExpf::eval_ldexp(x[e] - m) : 0.0f;
  float total = p[0];
#pragma unroll
  for (int e = 1; e < EMAX; ++e) {
    if (e < n) total = total + p[e];
  }
  const float inv = 1.0f / total;
#pragma unroll
  for (int e = 0; e < EMAX; ++e) p[e] = p[e] * inv;

  uint32_t live = (1u << n) - 1u;
  for (int i = 0; i < k; ++i) {
    int32_t key = -1;
    uint32_t best = 0xffffffffu;
#pragma unroll
    for (int e = 0; e < EMAX; ++e) {
      const int32_t b = (int32_t)f32_bits(p[e]);
      if (((live >> e) & 1u) && b > key) {
        key = b;
        best = (uint32_t)e;
      }
    }
    if (best < (uint32_t)EMAX) live &= ~(1u << best);
    sel[i][tid] = bits_f32((uint32_t)key);
    topk_i[t * k + i] = (int64_t)best;
  }
  const float wsum = renormalize ? aten_small_row_sum<kLaneThreads>(&sel[0][tid], k) : 1.0f;
  for (int i = 0; i < k; ++i) topk_w[t * k + i] = renormalize ? sel[i][tid] / wsum : sel[i][tid];
}

// G lanes per token (G = 2, 4 or 8), for n <= 16 * NS experts. The row is
// cut into stripes of 16 experts (the AVX-512 vector), and lane r of a group
// holds the CW = 16 / G experts [16 s + r CW, 16 s + (r + 1) CW) of every
// stripe s, so each of the 16 lane classes of the softmax sum lives in one
// lane, in stripe order. The xor tree's steps 8, 4, 2, 1 pair class L with
// L ^ step: across lanes (a DPP exchange with the lane r ^ (step / CW)) while
// step >= CW, in the lane's registers below. Every lane computes the tree
// for its own classes; floating-point addition is commutative, so after the
// cross-lane steps the lanes of a group hold the same values and all end
// with class 0's total. Below 16 experts (one stripe) the sum is a running
// sum handed from lane to lane instead (G = 2 or 4). The max and each top-k
// round's arg-max are group all-reductions (xor 1 and xor 2 quad
// permutations, then for G = 8 the half-row mirror, which pairs each lane
// with one of the other quad). Lane r of a group writes the outputs of the
// rounds i = r mod G.
constexpr int kDppRowShr1 = 0x111;     // lane i reads lane i - 1 of its row
constexpr int kDppQuadBcast3 = 0xFF;  // quad_perm:[3,3,3,3]
constexpr int kDppQuadBcast1 = 0xF5;  // quad_perm:[1,1,3,3]
constexpr int kDppRowShr4 = 0x114;  // lane i reads lane i - 4 of its row

template <int G, class Op>
__device__ inline uint32_t group_allreduce(uint32_t v, Op op) {
  static_assert(G == 2 || G == 4 || G == 8, "group size");
  v = op(v, dpp<kDppQuadXor1>(v));
  if constexpr (G >= 4) v = op(v, dpp<kDppQuadXor2>(v));
  // For an idempotent op, lane i combined with lane 7 - i (the other quad of
  // its 8) completes the group.
  if constexpr (G == 8) v = op(v, dpp<kDppRowHalfMirror>(v));
  return v;
}

// The value of lane r ^ D of this lane's group (D = 1, 2 or 4; groups of 8
// lanes are aligned within the 16-lane DPP rows).
template <int D>
__device__ inline uint32_t lane_xor(uint32_t v, int r) {
  if constexpr (D == 1) {
    return dpp<kDppQuadXor1>(v);
  } else if constexpr (D == 2) {
    return dpp<kDppQuadXor2>(v);
  } else {
    static_assert(D == 4, "lane distance");
    const uint32_t up = dpp<kDppRowShl4>(v), down = dpp<kDppRowShr4>(v);
    return (r & 4) ? down : up;
  }
}

// VB: bytes per row load, 16 (whole 16-byte vectors of a chunk), 8 or 4 (a
// chunk of CW experts in one 8- or 4-byte load) or 0 (one element at a time).
template <class C, int G, int NS, int VB>
__global__ __launch_bounds__(kLaneThreads) void moe_router_groups(const void* __restrict__ logits,
                                                                  float* __restrict__ topk_w,
                                                                  int64_t* __restrict__ topk_i, int64_t n_tokens,
                                                                  int n_experts, int k, int renormalize) {
  constexpr int CW = kSoftmaxLanes / G;  // experts of one stripe per lane
  constexpr int PER = NS * CW;           // experts per lane
  constexpr int TPB = kLaneThreads / G;  // tokens per workgroup
  static_assert(PER <= 32 && (VB != 16 || CW % C::VEC == 0) && (VB != 8 || CW * C::kBytes == 8) &&
                    (VB != 4 || CW * C::kBytes == 4) && (G != 8 || NS >= 2),
                "group router shape");
  __shared__ float sel[NS * kSoftmaxLanes][TPB];
  const int tid = threadIdx.x, r = tid % G, slot = tid / G;
  const int64_t t = (int64_t)blockIdx.x * TPB + slot;
  if (t >= n_tokens) return;  // whole groups leave together; nothing below synchronises
  const int n = n_experts;
  float x[PER];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int e0 = kSoftmaxLanes * s + r * CW;
    if constexpr (VB == 8 || VB == 4) {
      // n is a multiple of CW and the rows are VB-byte aligned.
      float f[C::VEC];
      if (e0 < n) {
        const char* a = static_cast<const char*>(logits) + (t * n + e0) * C::kBytes;
        if constexpr (VB == 8) {
          const u32x2 w = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(a));
          C::unpack((u32x4){w.x, w.y, 0u, 0u}, f);
        } else {
          const uint32_t w = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(a));
          C::unpack((u32x4){w, 0u, 0u, 0u}, f);
        }
      } else {
#pragma unroll
        for (int j = 0; j < CW; ++j) f[j] = -__builtin_inff();
      }
#pragma unroll
      for (int j = 0; j < CW; ++j) x[s * CW + j] = f[j];
    } else if constexpr (VB == 16) {
      // n is a multiple of C::VEC and the rows are 16-byte aligned.
      const u32x4* v = reinterpret_cast<const u32x4*>(static_cast<const char*>(logits) + (t * n + e0) * C::kBytes);
#pragma unroll
      for (int q = 0; q < CW / C::VEC; ++q) {
        float f[C::VEC];
        if (e0 + q * C::VEC < n) {
          C::unpack(__builtin_nontemporal_load(v + q), f);
        } else {
#pragma unroll
          for (int j = 0; j < C::VEC; ++j) f[j] = -__builtin_inff();
        }
#pragma unroll
        for (int j = 0; j < C::VEC; ++j) x[s * CW + q * C::VEC + j] = f[j];
      }
    } else {
#pragma unroll
      for (int j = 0; j < CW; ++j) x[s * CW + j] = e0 + j < n ? C::load1(logits, t * n + e0 + j) : -__builtin_inff();
    }
  }
  float mloc = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < PER; ++i) mloc = __builtin_elementwise_maximum(mloc, x[i]);
  const float m = bits_f32(group_allreduce<G>(f32_bits(mloc), MaxF32{}));
  float p[PER];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
#pragma unroll
    for (int j = 0; j < CW; ++j) {
      const int e = kSoftmaxLanes * s + r * CW + j;
      p[s * CW + j] = e < n ? SleefExpf::eval_ldexp(x[s * CW + j] - m) : 0.0f;
    }
  }
  float total;
  if (NS == 1 && n < kSoftmaxLanes) {
    // e_0 + e_1 + ... in order: lane 0 starts the running sum, and each lane
    // in turn takes it from the lane below (row_shr:1) and adds its own
    // experts; the last lane's sum goes to the whole group.
    float run = p[0];
#pragma unroll
    for (int j = 1; j < CW; ++j) {
      if (j < n) run = run + p[j];
    }
#pragma unroll
    for (int g = 1; g < G; ++g) {
      const float below = bits_f32(dpp<kDppRowShr1>(f32_bits(run)));
      if (r == g) {
        run = below;
#pragma unroll
        for (int j = 0; j < CW; ++j) {
          if (g * CW + j < n) run = run + p[j];
        }
      }
    }
    total = bits_f32(dpp<G == 4 ? kDppQuadBcast3 : kDppQuadBcast1>(f32_bits(run)));
  } else {
    // Lane classes r CW + j: stripe 0 is whole (n >= 16), the others add in order.
    float acc[CW];
#pragma unroll
    for (int j = 0; j < CW; ++j) acc[j] = p[j];
#pragma unroll
    for (int s = 1; s < NS; ++s) {
#pragma unroll
      for (int j = 0; j < CW; ++j) {
        if (kSoftmaxLanes * s + r * CW + j < n) acc[j] = acc[j] + p[s * CW + j];
      }
    }
#pragma unroll
    for (int step = kSoftmaxLanes / 2; step >= CW; step >>= 1) {
#pragma unroll
      for (int j = 0; j < CW; ++j) {
        const uint32_t a = f32_bits(acc[j]);
        const uint32_t o = step / CW == 1 ? lane_xor<1>(a, r) : step / CW == 2 ? lane_xor<2>(a, r) : lane_xor<4>(a, r);
        acc[j] = acc[j] + bits_f32(o);
      }
    }
#pragma unroll
    for (int step = CW / 2; step > 0; step >>= 1) {
#pragma unroll
      for (int j = 0; j < step; ++j) acc[j] = acc[j] + acc[j + step];
    }
    total = acc[0];
  }
  const float inv = 1.0f / total;
#pragma unroll
  for (int i = 0; i < PER; ++i) p[i] = p[i] * inv;

  uint32_t live = 0u;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
#pragma unroll
    for (int j = 0; j < CW; ++j) {
      if (kSoftmaxLanes * s + r * CW + j < n) live |= 1u << (s * CW + j);
    }
  }
  for (int i = 0; i < k; ++i) {
    int32_t key = -1;
    uint32_t mine = 0xffffffffu;
    int bit = -1;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
#pragma unroll
      for (int j = 0; j < CW; ++j) {
        const int32_t b = (int32_t)f32_bits(p[s * CW + j]);
        if (((live >> (s * CW + j)) & 1u) && b > key) {
          key = b;
          mine = (uint32_t)(kSoftmaxLanes * s + r * CW + j);
          bit = s * CW + j;
        }
      }
    }
    const uint32_t best = group_allreduce<G>((uint32_t)key, MaxI32{});
    const uint32_t pick = group_allreduce<G>((int32_t)best == key ? mine : 0xffffffffu, MinU32{});
    if (pick == mine && bit >= 0) live &= ~(1u << bit);
    sel[i][slot] = bits_f32(best);
    if (i % G == r) topk_i[t * k + i] = (int64_t)pick;
  }
  const float wsum = renormalize ? aten_small_row_sum<TPB>(&sel[0][slot], k) : 1.0f;
  for (int i = r; i < k; i += G) topk_w[t * k + i] = renormalize ? sel[i][slot] / wsum : sel[i][slot];
}

}  // namespace
}  // namespace cck

using namespace cck;

namespace {

template <class C, int EMAX>
void launch_router_lanes(const void* logits, float* w, int64_t* idx, int64_t t, int n, int k, int renorm,
                         hipStream_t st) {
  const unsigned grid = (unsigned)((t + kLaneThreads - 1) / kLaneThreads);
  const bool vec = n % C::VEC == 0 && (reinterpret_cast<uintptr_t>(logits) & 15u) == 0;
  if (vec) {
    moe_router_lanes<C, EMAX, true><<<grid, kLaneThreads, 0, st>>>(logits, w, idx, t, n, k, renorm);
  } else {
    moe_router_lanes<C, EMAX, false><<<grid, kLaneThreads, 0, st>>>(logits, w, idx, t, n, k, renorm);
  }
}

template <class C, int G, int NS>
void launch_router_groups(const void* logits, float* w, int64_t* idx, int64_t t, int n, int k, int renorm,
                          hipStream_t st) {
  constexpr int TPB = kLaneThreads / G, CW = kSoftmaxLanes / G;
  const unsigned grid = (unsigned)((t + TPB - 1) / TPB);
  const uintptr_t a = reinterpret_cast<uintptr_t>(logits);
  if constexpr (CW % C::VEC == 0) {
    if (n % C::VEC == 0 && (a & 15u) == 0) {
      moe_router_groups<C, G, NS, 16><<<grid, kLaneThreads, 0, st>>>(logits, w, idx, t, n, k, renorm);
      return;
    }
  } else if constexpr (CW * C::kBytes == 8) {
    if (n % CW == 0 && (a & 7u) == 0) {
      moe_router_groups<C, G, NS, 8><<<grid, kLaneThreads, 0, st>>>(logits, w, idx, t, n, k, renorm);
      return;
    }
  } else if constexpr (CW * C::kBytes == 4) {
    if (n % CW == 0 && (a & 3u) == 0) {
      moe_router_groups<C, G, NS, 4><<<grid, kLaneThreads, 0, st>>>(logits, w, idx, t, n, k, renorm);
      return;
    }
  }
  moe_router_groups<C, G, NS, 0><<<grid, kLaneThreads, 0, st>>>(logits, w, idx, t, n, k, renorm);
}

// Group kernels serve up to 64 experts; from 33 on only with enough tokens,
// where the wave kernel's one wave per token no longer fits the GPU at once.
constexpr int kGroupMaxExperts = 64;
constexpr int64_t kGroupWideMinTokens = 4096;
// Eight lanes per token (32 experts each at most) for 65 to 256 experts, from
// enough tokens that the wave kernel's one wave per token takes several
// rounds of the GPU: same-run A/B against it, fp32 / bf16, top-8 of 96 at
// 8192 tokens 7.4 / 9.2 vs 13.5 / 13.6 us, top-6 of 160 at 12288 8.6 / 11.8
// vs 14.6 / 15.7, at 16384 9.1 / 12.1 vs 18.3 / 19.6; top-8 of 256 at 16384
// 14.7 / 18.5 vs 24.0 / 26.1. Below those counts the wave kernel's shorter
// chain wins (top-6 of 160 at 2048 tokens: 5.4 vs 6.8 us fp32).
constexpr int kGroup8MaxExperts = 256;
inline int64_t group8_min_tokens(int n) { return n <= 128 ? 8192 : 12288; }

}  // namespace

extern "C" int32_t launch_moe_router_fwd(const void* logits, float* topk_weights, int64_t* topk_indices,
                                         int64_t num_tokens, int64_t num_experts, int64_t k, int32_t dtype,
                                         int32_t renormalize, void* stream) {
  if (num_tokens <= 0) return (int32_t)hipSuccess;
  if (num_experts > kMaxExperts || k > num_experts || k < 0) return (int32_t)hipErrorInvalidValue;
  if (k == 0) return (int32_t)hipSuccess;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int n = (int)num_experts, kk = (int)k, rn = renormalize != 0;
  // One workgroup per 64 / G tokens: every grid below fits for any token count this guard lets through.
  const bool small_grid = num_tokens <= (int64_t)kLaneThreads * (INT32_MAX / 4);
  const bool groups = n <= 2 * kSoftmaxLanes || (n <= kGroupMaxExperts && num_tokens >= kGroupWideMinTokens);
  return with_codec(dtype, [&](auto codec) {
    using C = decltype(codec);
    if (small_grid && n <= kLaneMaxExperts) {
      launch_router_lanes<C, kLaneMaxExperts>(logits, topk_weights, topk_indices, num_tokens, n, kk, rn, st);
      return launch_status();
    }
    if (small_grid && n > kGroupMaxExperts && n <= kGroup8MaxExperts && num_tokens >= group8_min_tokens(n)) {
      if (n <= 8 * kSoftmaxLanes) {
        launch_router_groups<C, 8, 8>(logits, topk_weights, topk_indices, num_tokens, n, kk, rn, st);
      } else if (n <= 10 * kSoftmaxLanes) {
        launch_router_groups<C, 8, 10>(logits, topk_weights, topk_indices, num_tokens, n, kk, rn, st);
      } else {
        launch_router_groups<C, 8, 16>(logits, topk_weights, topk_indices, num_tokens, n, kk, rn, st);
      }
      return launch_status();
    }
    if (small_grid && groups) {
      if (n <= kSoftmaxLanes) {
        launch_router_groups<C, 4, 1>(logits, topk_weights, topk_indices, num_tokens, n, kk, rn, st);
      } else if (n <= 2 * kSoftmaxLanes) {
        launch_router_groups<C, 4, 2>(logits, topk_weights, topk_indices, num_tokens, n, kk, rn, st);
      } else {
        launch_router_groups<C, 4, 4>(logits, topk_weights, topk_indices, num_tokens, n, kk, rn, st);
      }
      return launch_status();
    }
    moe_router_waves<C><<<flat_grid(num_tokens, kWavesPerGroup, kMaxRowGroups), 256, 0, st>>>(
        logits, topk_weights, topk_indices, num_tokens, n, kk, rn);
    return launch_status();
  });
}
