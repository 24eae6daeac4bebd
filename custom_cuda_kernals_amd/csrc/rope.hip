// Half-split rotary position embedding on q [B,S,Hq,D] and k [B,S,Hkv,D] with
// fp32 cos/sin tables [S, D/2], for gfx950. Out-of-place or in place
// (q_out == q, k_out == k): every thread reads both halves of its pairs
// before writing them.
//
// Semantics (baselines/rope.py:129-145), with every product and sum rounded
// separately in fp32 (no fma contraction) and the result rounded once to T:
//   out[:D/2] = T(x1*cos - x2*sin),  out[D/2:] = T(x2*cos + x1*sin)
// so the output is bit-identical to the eager oracle given the same tables.
//
// Design: a workgroup owns TOK tokens. Within a token, a thread is pinned to
// one VEC-wide chunk of the half dimension and walks the heads (q heads
// first, then k heads) with a stride of the number of head lanes, so its
// cos/sin chunk is loaded once per token and reused for every head it takes.
// Workgroups are 256 threads, or, for one token of more heads than 256
// threads cover at once, a thread per (head, chunk) of the token; while the
// grid fits one round of resident workgroups, a thread per (head, chunk)
// with the token's cos/sin row staged in LDS.
// All accesses are 16 bytes; a wave covers whole 128-byte cache lines.
#include "launch.hpp"

namespace cck {
namespace {

#pragma clang fp contract(off)

// Stores of a one-token-per-workgroup launch (TOK == 1) go through per-token
// buffer resources with SC1|NT: 104.0 vs 104.7 us with global-pointer NT
// stores at config 4 on MI355X. With several tokens per workgroup the row
// base is not wave-uniform, so those use global pointers.
template <int TOK>
using RopeRow = RowBuf<TOK == 1, TOK == 1 ? (kPolSC1 | kPolNT) : kBufStorePolicy>;

// q / k and q_out / k_out may be the same buffers (in place), so none of
// the four is declared __restrict__; each element is loaded before the
// element is stored, by the same thread.
template <class C, int CHUNKS, int TOK, int NT = 256>
__global__ __launch_bounds__(NT) void rope_tokens(const void* q, const void* k,
                                                   const float* __restrict__ cos_t,
                                                   const float* __restrict__ sin_t, void* q_out,
                                                   void* k_out, int64_t tokens, int64_t seq_len,
                                                   int hq, int hkv, int head_dim) {
  constexpr int VEC = C::VEC;
  constexpr int LANES = NT / TOK;           // threads per token
  constexpr int HLANES = LANES / CHUNKS;    // head lanes per token
  const int t_local = TOK == 1 ? 0 : threadIdx.x / LANES;
  const int c = threadIdx.x % CHUNKS;
  const int hl = (threadIdx.x % LANES) / CHUNKS;
  const int half = head_dim / 2;
  const int heads = hq + hkv;
  // Token rows are below 2 GiB (checked by the launcher), so 32-bit offsets hold.
  const uint32_t q_bytes = (uint32_t)((int64_t)hq * head_dim * C::kBytes);
  const uint32_t k_bytes = (uint32_t)((int64_t)hkv * head_dim * C::kBytes);
  for (int64_t tok = (int64_t)blockIdx.x * TOK + t_local; tok < tokens; tok += (int64_t)gridDim.x * TOK) {
    const int64_t s = tok % seq_len;
    float cs[VEC], sn[VEC];
    const float4* cp = reinterpret_cast<const float4*>(cos_t + s * half + c * VEC);
    const float4* sp = reinterpret_cast<const float4*>(sin_t + s * half + c * VEC);
#pragma unroll
    for (int i = 0; i < VEC / 4; ++i) {
      const float4 a = cp[i], b = sp[i];
      cs[4 * i] = a.x; cs[4 * i + 1] = a.y; cs[4 * i + 2] = a.z; cs[4 * i + 3] = a.w;
      sn[4 * i] = b.x; sn[4 * i + 1] = b.y; sn[4 * i + 2] = b.z; sn[4 * i + 3] = b.w;
    }
    // Head hh of one tensor's token row: both halves are read before either
    // is written, so the rotation works in place.
    auto rotate = [&](const char* src, const RopeRow<TOK>& dst, int hh) {
      const uint32_t off = (uint32_t)((hh * head_dim + c * VEC) * C::kBytes);
      float x1[VEC], x2[VEC], o1[VEC], o2[VEC];
      C::unpack(ld_stream(reinterpret_cast<const u32x4*>(src + off)), x1);
      C::unpack(ld_stream(reinterpret_cast<const u32x4*>(src + off + half * C::kBytes)), x2);
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        o1[i] = x1[i] * cs[i] - x2[i] * sn[i];
        o2[i] = x2[i] * cs[i] + x1[i] * sn[i];
      }
      dst.st16(C::pack(o1), off);
      dst.st16(C::pack(o2), off + half * C::kBytes);
    };
    const RopeRow<TOK> qo(static_cast<char*>(q_out) + tok * q_bytes, q_bytes);
    const RopeRow<TOK> ko(static_cast<char*>(k_out) + tok * k_bytes, k_bytes);
    // Heads h = hl, hl + HLANES, ...: the q heads, then the k heads (separate
    // loops keep each loop's row resource uniform).
    int h = hl;
    for (; h < hq; h += HLANES) rotate(static_cast<const char*>(q) + tok * q_bytes, qo, h);
    for (; h < heads; h += HLANES) rotate(static_cast<const char*>(k) + tok * k_bytes, ko, h - hq);
  }
}

// Any head_dim / alignment: one thread per (token, head, pair).
template <class C>
__global__ __launch_bounds__(256) void rope_scalar(const void* q, const void* k,
                                                   const float* __restrict__ cos_t,
                                                   const float* __restrict__ sin_t, void* q_out,
                                                   void* k_out, int64_t tokens, int64_t seq_len,
                                                   int hq, int hkv, int head_dim) {
  const int half = head_dim / 2;
  const int heads = hq + hkv;
  const int64_t total = tokens * heads * half;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += stride) {
    const int j = (int)(i % half);
    const int64_t th = i / half;
    const int h = (int)(th % heads);
    const int64_t tok = th / heads;
    const int64_t s = tok % seq_len;
    const bool is_q = h < hq;
    const void* src = is_q ? q : k;
    void* dst = is_q ? q_out : k_out;
    const int64_t e0 = (is_q ? tok * hq + h : tok * hkv + (h - hq)) * head_dim + j;
    const float c = cos_t[s * half + j], sn = sin_t[s * half + j];
    const float x1 = C::load1(src, e0), x2 = C::load1(src, e0 + half);
    C::store1(dst, e0, x1 * c - x2 * sn);
    C::store1(dst, e0 + half, x2 * c + x1 * sn);
  }
}

// One token per workgroup, a thread per (head, chunk) of it, with the token's
// cos / sin row loaded once by the first threads and shared through LDS
// (instead of every thread loading its chunk of both tables). Used where the
// grid fits one round of resident workgroups; see the launcher.
template <class C, int CHUNKS, int NT>
__global__ __launch_bounds__(NT) void rope_heads_staged(const void* q, const void* k,
                                                        const float* __restrict__ cos_t,
                                                        const float* __restrict__ sin_t, void* q_out,
                                                        void* k_out, int64_t tokens, int64_t seq_len,
                                                        int hq, int hkv, int head_dim) {
  constexpr int VEC = C::VEC;
  constexpr int F4 = CHUNKS * VEC / 4;  // float4s in one table row (half = CHUNKS * VEC)
  static_assert(2 * F4 <= NT, "the first 2 * F4 threads load the cos and sin rows");
  __shared__ float4 tab[2 * F4];
  const int c = threadIdx.x % CHUNKS;
  const int hh = threadIdx.x / CHUNKS;
  const int half = head_dim / 2;
  const int heads = hq + hkv;
  const bool live = hh < heads;
  const bool isq = hh < hq;
  const int idx = live ? (isq ? hh : hh - hq) : 0;  // lanes past the last head read head 0 and store nothing
  const uint32_t q_bytes = (uint32_t)((int64_t)hq * head_dim * C::kBytes);
  const uint32_t k_bytes = (uint32_t)((int64_t)hkv * head_dim * C::kBytes);
  const uint32_t off = (uint32_t)((idx * head_dim + c * VEC) * C::kBytes);
  for (int64_t tok = blockIdx.x; tok < tokens; tok += gridDim.x) {
    const int64_t s = tok % seq_len;
    const char* src = (live && !isq) ? static_cast<const char*>(k) + tok * k_bytes
                                     : static_cast<const char*>(q) + tok * q_bytes;
    const u32x4 ra = ld_stream(reinterpret_cast<const u32x4*>(src + off));
    const u32x4 rb = ld_stream(reinterpret_cast<const u32x4*>(src + off + half * C::kBytes));
    if (threadIdx.x < 2 * F4) {
      const float* t = threadIdx.x < F4 ? cos_t : sin_t;
      tab[threadIdx.x] = reinterpret_cast<const float4*>(t + s * half)[threadIdx.x % F4];
    }
    __syncthreads();
    float cs[VEC], sn[VEC];
#pragma unroll
    for (int i = 0; i < VEC / 4; ++i) {
      const float4 u = tab[c * (VEC / 4) + i], w = tab[F4 + c * (VEC / 4) + i];
      cs[4 * i] = u.x; cs[4 * i + 1] = u.y; cs[4 * i + 2] = u.z; cs[4 * i + 3] = u.w;
      sn[4 * i] = w.x; sn[4 * i + 1] = w.y; sn[4 * i + 2] = w.z; sn[4 * i + 3] = w.w;
    }
    float x1[VEC], x2[VEC], o1[VEC], o2[VEC];
    C::unpack(ra, x1);
    C::unpack(rb, x2);
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      o1[i] = x1[i] * cs[i] - x2[i] * sn[i];
      o2[i] = x2[i] * cs[i] + x1[i] * sn[i];
    }
    if (live) {
      if (isq) {
        const RopeRow<1> qo(static_cast<char*>(q_out) + tok * q_bytes, q_bytes);
        qo.st16(C::pack(o1), off);
        qo.st16(C::pack(o2), off + half * C::kBytes);
      } else {
        const RopeRow<1> ko(static_cast<char*>(k_out) + tok * k_bytes, k_bytes);
        ko.st16(C::pack(o1), off);
        ko.st16(C::pack(o2), off + half * C::kBytes);
      }
    }
    __syncthreads();  // the next token rewrites tab
  }
}

// One token per workgroup of 64 * W threads for the W in WS that equals
// `waves`: a thread per (head, chunk) of the token, so no thread rotates a
// second head after its first. Up to one round of the workgroups the device
// holds at once the tables are staged in LDS (rope_heads_staged): 3.51 vs
// 3.95 us at 512 tokens of 32 / 8 heads of 128 bf16, 5.13 vs 5.61 at 1024;
// with more tokens the per-token barrier lost (15.75 vs 15.29 us at 4096,
// 105.4 vs 103.2 at config 4). With min_rounds > 0, not when the tokens fill
// more than one but fewer than min_rounds rounds. false (nothing launched)
// otherwise.
template <class C, int CHUNKS, int... WS>
bool launch_rope_per_head(int waves, int min_rounds, std::integer_sequence<int, WS...>, const void* q,
                          const void* k, const float* ct, const float* sn, void* q_out, void* k_out,
                          int64_t tokens, int64_t seq_len, int hq, int hkv, int d, hipStream_t st) {
  const unsigned grid = flat_grid(tokens, 1, kMaxRowGroups);
  auto one = [&](auto w) {
    constexpr int W = decltype(w)::value;
    if (waves != W) return false;
    constexpr auto staged = rope_heads_staged<C, CHUNKS, 64 * W>;
    if (tokens <= resident_groups<staged>(64 * W)) {
      staged<<<grid, 64 * W, 0, st>>>(q, k, ct, sn, q_out, k_out, tokens, seq_len, hq, hkv, d);
      return true;
    }
    constexpr auto kernel = rope_tokens<C, CHUNKS, 1, 64 * W>;
    if (min_rounds > 0) {
      const int64_t resident = resident_groups<kernel>(64 * W);
      if (tokens > resident && tokens < min_rounds * resident) return false;
    }
    kernel<<<grid, 64 * W, 0, st>>>(q, k, ct, sn, q_out, k_out, tokens, seq_len, hq, hkv, d);
    return true;
  };
  return (one(std::integral_constant<int, WS>{}) || ...);
}

// Tokens of at most 256 / CHUNKS heads while the grid fits one round of the
// workgroups the device holds at once: rope_heads_staged in one workgroup of
// 64 * W threads (W in WS equal to `waves`). false (nothing launched)
// otherwise. Same-run A/B on MI355X against the 256-thread workgroups below,
// bf16: 28 / 4 heads of 128 at 512 tokens 3.24 vs 3.86 us, 1024 4.64 vs
// 5.34; 12 / 12 heads of 64 at 512 tokens 2.69 vs 3.33 (fp32 2.94 vs 3.38);
// 16 / 16 heads of 64 at 1024 3.55 vs 3.79; 8 / 8 heads of 128 at 256
// tokens 2.54 vs 2.50 (fp32 2.73 vs 2.60).
template <class C, int CHUNKS, int... WS>
bool launch_rope_staged_small(int waves, std::integer_sequence<int, WS...>, const void* q, const void* k,
                              const float* ct, const float* sn, void* q_out, void* k_out, int64_t tokens,
                              int64_t seq_len, int hq, int hkv, int d, hipStream_t st) {
  auto one = [&](auto w) {
    constexpr int W = decltype(w)::value;
    if (waves != W) return false;
    constexpr auto staged = rope_heads_staged<C, CHUNKS, 64 * W>;
    if (tokens > resident_groups<staged>(64 * W)) return false;
    staged<<<flat_grid(tokens, 1, kMaxRowGroups), 64 * W, 0, st>>>(q, k, ct, sn, q_out, k_out, tokens, seq_len,
                                                                    hq, hkv, d);
    return true;
  };
  return (one(std::integral_constant<int, WS>{}) || ...);
}

}  // namespace
}  // namespace cck

using namespace cck;

extern "C" int32_t launch_rope_fwd(const void* q, const void* k, const void* cos_table,
                                   const void* sin_table, void* q_out, void* k_out, int64_t batch,
                                   int64_t seq_len, int64_t n_q_heads, int64_t n_kv_heads,
                                   int64_t head_dim, int32_t dtype, void* stream) {
  if (batch <= 0 || seq_len <= 0 || head_dim <= 0) return (int32_t)hipSuccess;
  if (n_q_heads < 0 || n_kv_heads < 0 || head_dim % 2 != 0) return (int32_t)hipErrorInvalidValue;
  if (n_q_heads + n_kv_heads == 0) return (int32_t)hipSuccess;
  if (n_q_heads + n_kv_heads > 0x7fffffff || head_dim > 0x7fffffff) return (int32_t)hipErrorInvalidValue;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t tokens = batch * seq_len;
  const float* ct = static_cast<const float*>(cos_table);
  const float* sn = static_cast<const float*>(sin_table);
  const int hq = (int)n_q_heads, hkv = (int)n_kv_heads, d = (int)head_dim;
  return with_codec(dtype, [&](auto codec) {
    using C = decltype(codec);
    const int half = d / 2;
    const bool vec_ok = (half % C::VEC == 0) && host_aligned(q, 16) && host_aligned(k, 16) &&
                        host_aligned(q_out, 16) && host_aligned(k_out, 16) &&
                        host_aligned(ct, 16) && host_aligned(sn, 16);
    const int64_t max_row_bytes = (int64_t)(hq > hkv ? hq : hkv) * d * C::kBytes;
    const int chunks = vec_ok && max_row_bytes <= 0x7fffffff ? half / C::VEC : 0;
    // TOK tokens per workgroup, 256/TOK threads per token, CHUNKS chunk lanes,
    // LDS_ bytes reserved to cap the workgroups resident per CU.
#define CCK_ROPE(CH_, TOK_, LDS_)                                                            \
  rope_tokens<C, CH_, TOK_><<<flat_grid(tokens, TOK_, kMaxRowGroups), 256, LDS_, st>>>(    \
      q, k, ct, sn, q_out, k_out, tokens, seq_len, hq, hkv, d)
    // Tokens of more than 256 / CHUNKS heads (and at most 1024 / CHUNKS) get a
    // thread per (head, chunk) in one workgroup of that many threads, rounded
    // up to whole waves, instead of 256 threads that take the heads in
    // rounds. Same-run A/B on MI355X, bf16 head_dim 128, graph-replayed:
    // 32 / 8 heads (320 threads) 15.30 vs 15.72 us at [2, 2048], 52.40 vs
    // 52.85 at [16, 1024], 103.55 vs 103.43 at config 4; 64 / 8 heads (576)
    // 25.47 vs 26.29 at [1, 4096], 48.20 vs 49.53 at [1, 8192]; 32 / 32
    // heads (512) 82.62 vs 84.41 at [4, 4096]. Capping these at 4, 5 or 6
    // workgroups per CU (LDS reserved) measured no different. With 16 chunk
    // lanes (fp32 head_dim 128: 640 threads for 40 heads) a grid of more
    // than one and fewer than four rounds of resident workgroups lost to
    // the 256-thread rounds (9.49 vs 8.71 us at 1024 tokens, 15.79 vs 15.29
    // at 2048), so those keep them; fewer tokens (2.90 vs 4.05 us at 128,
    // 5.16 vs 5.79 at 512) and more (103.9 vs 108.4 us at 16384) do not.
    const int heads = hq + hkv;
    const int waves = chunks > 0 ? (heads * chunks + 63) / 64 : 0;
    using Waves = std::integer_sequence<int, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16>;
    if ((chunks == 8 || chunks == 16) && heads * chunks > 256 && waves <= 16 &&
        (chunks == 8 ? launch_rope_per_head<C, 8>(waves, 0, Waves{}, q, k, ct, sn, q_out, k_out, tokens, seq_len,
                                                  hq, hkv, d, st)
                     : launch_rope_per_head<C, 16>(waves, 4, Waves{}, q, k, ct, sn, q_out, k_out, tokens, seq_len,
                                                   hq, hkv, d, st))) {
    } else if (heads * chunks <= 256 &&
               ((chunks == 8 && launch_rope_staged_small<C, 8>(waves, std::integer_sequence<int, 1, 2, 3, 4>{}, q, k,
                                                                ct, sn, q_out, k_out, tokens, seq_len, hq, hkv, d, st)) ||
                (chunks == 4 && launch_rope_staged_small<C, 4>(waves, std::integer_sequence<int, 1, 2, 3, 4>{}, q, k,
                                                                ct, sn, q_out, k_out, tokens, seq_len, hq, hkv, d, st)) ||
                (chunks == 16 && launch_rope_staged_small<C, 16>(waves, std::integer_sequence<int, 1, 2, 3, 4>{}, q,
                                                                  k, ct, sn, q_out, k_out, tokens, seq_len, hq, hkv, d,
                                                                  st)))) {
    } else if (chunks == 8) {
      // Tokens of at most 32 heads (and more than 128): with at most 6
      // workgroups per CU (8 fit) this 256-thread shape measured 102.0 vs
      // 103.8 us on MI355X at config 4's size when that took it too.
      CCK_ROPE(8, 1, kLdsForGroupsPerCu<6>);
    } else if (chunks == 4) {
      // bf16 head_dim 64: 64.1 vs 67.8 us for eight tokens per workgroup;
      // 61.7 vs 64.1 us with at most 6 workgroups per CU.
      CCK_ROPE(4, 1, kLdsForGroupsPerCu<6>);
    } else if (chunks == 16) {
      // fp32 head_dim 128: 219.7 vs 231.5 us for two tokens per workgroup (a
      // cap of 5 or 6 workgroups per CU measured no different).
      CCK_ROPE(16, 1, 0);
    } else if (chunks == 2) {
      CCK_ROPE(2, 16, 0);
    } else if (chunks == 1) {
      CCK_ROPE(1, 32, 0);
    } else if (chunks == 32) {
      CCK_ROPE(32, 1, 0);
    } else {
      const int64_t total = tokens * (int64_t)(hq + hkv) * half;
      rope_scalar<C><<<flat_grid(total, 256, 1 << 20), 256, 0, st>>>(q, k, ct, sn, q_out, k_out,
                                                                   tokens, seq_len, hq, hkv, d);
    }
#undef CCK_ROPE
    return launch_status();
  });
}
