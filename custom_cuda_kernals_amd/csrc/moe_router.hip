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
// Design: one wave64 per token, up to 256 experts (4 per lane, expert
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

// ATen's float32 row sum of n < 512 non-negative addends, serially
// (wave-uniform): 8-lane vectors in 4 slots, each slot one running sum from
// zero (no 16-step block of a slot completes below 512 addends, so the
// cascade's other levels stay zero), the leftover vectors into slot 0, then
// the trailing scalars and the 8 lanes in order; rows under 8 addends as
// scalars in 4 slots. Adding the zero levels (or a leading zero) changes no
// non-negative sum, so they are left out.
__device__ inline float aten_small_row_sum(const float* v, int n) {
  if (n < 8) {
    const int s = n >> 2;
    float p0 = s ? v[0] : 0.0f, p1 = s ? v[1] : 0.0f, p2 = s ? v[2] : 0.0f, p3 = s ? v[3] : 0.0f;
    for (int u = 4 * s; u < n; ++u) p0 = p0 + v[u];
    return ((p0 + p1) + p2) + p3;
  }
  const int nv = n >> 3, s = nv >> 2;
  float total = 0.0f;
  for (int e = nv * 8; e < n; ++e) total = total + v[e];
  for (int l = 0; l < 8; ++l) {
    float p0 = 0.0f, p1 = 0.0f, p2 = 0.0f, p3 = 0.0f;
    for (int i = 0; i < s; ++i) {
      p0 = p0 + v[(4 * i + 0) * 8 + l];
      p1 = p1 + v[(4 * i + 1) * 8 + l];
      p2 = p2 + v[(4 * i + 2) * 8 + l];
      p3 = p3 + v[(4 * i + 3) * 8 + l];
    }
    for (int vec = 4 * s; vec < nv; ++vec) p0 = p0 + v[vec * 8 + l];
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
      wsum = aten_small_row_sum(row, k);
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

}  // namespace
}  // namespace cck

using namespace cck;

extern "C" int32_t launch_moe_router_fwd(const void* logits, float* topk_weights, int64_t* topk_indices,
                                         int64_t num_tokens, int64_t num_experts, int64_t k, int32_t dtype,
                                         int32_t renormalize, void* stream) {
  if (num_tokens <= 0) return (int32_t)hipSuccess;
  if (num_experts > kMaxExperts || k > num_experts || k < 0) return (int32_t)hipErrorInvalidValue;
  if (k == 0) return (int32_t)hipSuccess;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_codec(dtype, [&](auto codec) {
    using C = decltype(codec);
    moe_router_waves<C><<<flat_grid(num_tokens, kWavesPerGroup, kMaxRowGroups), 256, 0, st>>>(
        logits, topk_weights, topk_indices, num_tokens, (int)num_experts, (int)k, renormalize != 0);
    return launch_status();
  });
}
