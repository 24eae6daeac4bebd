// MoE top-k router (softmax gating), for gfx950.
//
// Semantics (baselines/moe_router.py:117-128):
//   probs = softmax(float(logits), dim=-1)                      fp32
//   topk_weights, topk_indices = topk(probs, k)                 descending
//   if renormalize: topk_weights /= topk_weights.sum(-1)
// Ties between equal probabilities go to the lower expert index.
//
// Design: one wave64 per token, up to 256 experts (4 per lane, expert
// e = lane + 64 * slot). The max and the sum of the softmax are wave
// all-reductions (DPP); each of the k selection rounds is a
// wave arg-max in two all-reductions: the largest probability (as integer
// bits; probabilities are >= +0) and then the smallest expert index holding
// it. Round i's result is kept by lane i % 64, so the weights are renormalised
// and stored with one coalesced pass at the end.
#include "launch.hpp"

namespace cck {
namespace {

#pragma clang fp contract(off)

constexpr int kWavesPerGroup = 4;
constexpr int kSlots = 4;                // experts per lane
constexpr int kMaxExperts = 64 * kSlots;  // 256, as the reference (moe_router.cu kMaxLocal * 32)

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
    float sloc = 0.0f;
#pragma unroll
    for (int s = 0; s < kSlots; ++s) {
      if (live[s]) {
        p[s] = __builtin_expf(p[s] - m);
        sloc = sloc + p[s];
      }
    }
    const float sum = bits_f32(wave_allreduce(f32_bits(sloc), AddF32{}));
#pragma unroll
    for (int s = 0; s < kSlots; ++s) {
      if (live[s]) p[s] = p[s] / sum;
    }

    float sel_w[kSlots];
    uint32_t sel_e[kSlots];
    float wsum = 0.0f;
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
      wsum = wsum + val;
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
