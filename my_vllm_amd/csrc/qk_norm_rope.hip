// Attention prologue for gfx950: per-head q/k RMSNorm, neox rotary embedding
// and the slot_mapping KV store in one launch.
//
// Semantics follow the reference's separate native ops, in their order
// (nanovllm/models/qwen3.py:96-100, then Attention.forward's store,
// nanovllm/layers/attention.py:140-141):
//   x  = T(T(x32 * rsqrt(mean(x32^2) + eps)) * w)      q_norm / k_norm
//        (layernorm.py:31-40; skipped when no weight is given)
//   y1 = T(x1 * cos - x2 * sin), y2 = T(x2 * cos + x1 * sin)   fp32 products,
//        x1 / x2 the two halves of the head, cos / sin = cos_sin_cache[pos]
//        (rotary_embedding.py:7-15, 41-51)
//   k_cache[slot] = rotated k, v_cache[slot] = v   (attention.py:69-85; slots
//        outside [0, num_slots) are skipped)
// Queries and keys are written to their output rows (which may alias the
// inputs); V is only copied into the cache.
//
// Sixteen lanes per (token, head) row of q, k or v; each lane owns four
// elements of each half of the 128-wide head, so the pairs the rotation mixes
// sit in one lane and the norm's sum of squares is the only cross-lane step.
#include "mva_capi.h"
#include "mva_common.h"

#include <algorithm>

namespace mva {
namespace {

constexpr int kRopeDim = 128;

struct PrologueArgs {
  const void* q_in;
  void* q_out;
  int64_t q_tok_stride, q_head_stride;  // shared by q_in and q_out
  const void* k_in;
  void* k_out;
  int64_t k_tok_stride, k_head_stride;
  const void* v;
  int64_t v_tok_stride, v_head_stride;
  int num_q_heads, num_kv_heads;
  const int64_t* positions;
  const float* cos_sin;  // [max_position, 128]: cos(64) | sin(64)
  int64_t max_position;
  const void* q_norm_w;  // nullptr: no q/k norm
  const void* k_norm_w;
  float eps;
  void* k_cache;  // nullptr: no store
  void* v_cache;
  int64_t num_slots;
  const void* slots;
  int slot_is_int64;
  int64_t num_tokens;
};

typedef float f32x4v __attribute__((ext_vector_type(4)));

template <typename T>
struct Vec4;
template <>
struct Vec4<__bf16> {
  typedef __bf16 type __attribute__((ext_vector_type(4)));
};
template <>
struct Vec4<_Float16> {
  typedef _Float16 type __attribute__((ext_vector_type(4)));
};

template <typename W>
__device__ inline f32x4v load_w4(const void* w, int i) {
  if constexpr (sizeof(W) == 4) {
    return *reinterpret_cast<const f32x4v*>((const float*)w + i);
  } else {
    const typename Vec4<W>::type v = *reinterpret_cast<const typename Vec4<W>::type*>((const W*)w + i);
    return f32x4v{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
  }
}

// Rows r of a token: [0, Hq) queries, [Hq, Hq + Hkv) keys, then (with a
// store) [Hq + Hkv, Hq + 2 Hkv) values; a quad is four consecutive rows.
// Within a quad the 16 lanes of group g = lane / 16 own row 4q + g; lane
// c = lane % 16 holds elements 4c .. 4c+3 of the first half of the head and
// 64 + 4c .. 64 + 4c + 3 of the second (the pairs the rotation mixes),
// loaded and stored 8 bytes at a time.
//
// A wavefront takes one item at a time: up to kChunk quads of one token.
// The token is uniform over the wavefront, so its position and slot are
// two loads, and the item issues them, then every row load, then (once the
// position is in) the one cos / sin row all its rows share: two memory
// round trips per item.  Written row by row, each row would wait on the
// position, then the cos / sin row, then the data, and the compiler cannot
// hoist the next row's loads above this row's stores, since the outputs
// may alias the inputs.  Distinct rows never overlap, so reading an item's
// rows before writing any of them is exact even in place.
constexpr int kChunk = 6;

template <typename T, typename W, typename SlotT>
__global__ __launch_bounds__(256) void qk_norm_rope_store_kernel(PrologueArgs a) {
  // Separate fp32 multiplies and adds, as torch evaluates the rotation (no
  // fused multiply-add contraction).
#pragma clang fp contract(off)
  typedef typename Vec4<T>::type V4;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4;
  const int c4 = 4 * (lane & 15);
  const int hqk = a.num_q_heads + a.num_kv_heads;
  const bool store = a.k_cache != nullptr;
  const int R = hqk + (store ? a.num_kv_heads : 0);
  const int nq = (R + 3) / 4;
  const int S = (nq + kChunk - 1) / kChunk;  // items per token
  const int64_t waves = (int64_t)gridDim.x * 4;
  const bool norm = a.q_norm_w != nullptr;
  f32x4v wq1{}, wq2{}, wk1{}, wk2{};
  if (norm) {
    wq1 = load_w4<W>(a.q_norm_w, c4);
    wq2 = load_w4<W>(a.q_norm_w, 64 + c4);
    wk1 = load_w4<W>(a.k_norm_w, c4);
    wk2 = load_w4<W>(a.k_norm_w, 64 + c4);
  }
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  for (int64_t it = (int64_t)blockIdx.x * 4 + wave; it < a.num_tokens * S; it += waves) {
    const int64_t t = it / S;
    const int j0 = (int)(it - t * S) * kChunk;  // this item's quads [j0, j0 + kChunk) within [0, nq)
    // Without a store the slot pointer is the positions (a valid int64
    // array of the same length) and the value goes unused.
    const int64_t pos_in = a.positions[t];
    const int64_t slot_in = (int64_t)((const SlotT*)a.slots)[t];
    V4 lo[kChunk], hi[kChunk];
#pragma unroll
    for (int k = 0; k < kChunk; ++k) {
      int r = 4 * (j0 + k) + g;
      r = r < R ? r : 0;  // rows past the token read row 0 and are not written
      const T* src;
      if (r >= hqk)
        src = (const T*)a.v + t * a.v_tok_stride + (r - hqk) * a.v_head_stride;
      else if (r < a.num_q_heads)
        src = (const T*)a.q_in + t * a.q_tok_stride + r * a.q_head_stride;
      else
        src = (const T*)a.k_in + t * a.k_tok_stride + (r - a.num_q_heads) * a.k_head_stride;
      lo[k] = *reinterpret_cast<const V4*>(src + c4);
      hi[k] = *reinterpret_cast<const V4*>(src + 64 + c4);
    }
    const int64_t pos = pos_in < 0 ? 0 : (pos_in >= a.max_position ? a.max_position - 1 : pos_in);  // stay in bounds
    const f32x4v cs = *reinterpret_cast<const f32x4v*>(a.cos_sin + pos * kRopeDim + c4);
    const f32x4v sn = *reinterpret_cast<const f32x4v*>(a.cos_sin + pos * kRopeDim + 64 + c4);
    const int64_t slot = (store && slot_in < a.num_slots) ? slot_in : -1;  // negative: skipped
    const int64_t cache_row = (slot >= 0) ? slot * a.num_kv_heads : 0;  // rows of [slots * Hkv, 128]
#pragma unroll
    for (int k = 0; k < kChunk; ++k) {
      const int r = 4 * (j0 + k) + g;
      if (r >= R) continue;  // a whole 16-lane group: no shuffle partner is lost
      if (r >= hqk) {  // V: copy into the cache
        if (slot >= 0) {
          T* dst = (T*)a.v_cache + (cache_row + r - hqk) * kRopeDim;
          *reinterpret_cast<V4*>(dst + c4) = lo[k];
          *reinterpret_cast<V4*>(dst + 64 + c4) = hi[k];
        }
        continue;
      }
      const bool is_q = r < a.num_q_heads;
      const int h = is_q ? r : r - a.num_q_heads;
      float x1[4], x2[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x1[e] = (float)lo[k][e];
        x2[e] = (float)hi[k][e];
      }
      if (norm) {
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) ss += x1[e] * x1[e] + x2[e] * x2[e];
#pragma unroll
        for (int off = 8; off > 0; off >>= 1) ss += __shfl_xor(ss, off);  // within the 16-lane group
        const float rs = 1.0f / __builtin_sqrtf(ss / (float)kRopeDim + a.eps);
        const f32x4v w1 = is_q ? wq1 : wk1;
        const f32x4v w2 = is_q ? wq2 : wk2;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x1[e] = (float)(T)((float)(T)(x1[e] * rs) * w1[e]);
          x2[e] = (float)(T)((float)(T)(x2[e] * rs) * w2[e]);
        }
      }
      V4 y1, y2;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        y1[e] = (T)(x1[e] * cs[e] - x2[e] * sn[e]);
        y2[e] = (T)(x2[e] * cs[e] + x1[e] * sn[e]);
      }
      T* dst = is_q ? (T*)a.q_out + t * a.q_tok_stride + h * a.q_head_stride
                    : (T*)a.k_out + t * a.k_tok_stride + h * a.k_head_stride;
      *reinterpret_cast<V4*>(dst + c4) = y1;
      *reinterpret_cast<V4*>(dst + 64 + c4) = y2;
      if (!is_q && slot >= 0) {
        T* kd = (T*)a.k_cache + (cache_row + h) * kRopeDim;
        *reinterpret_cast<V4*>(kd + c4) = y1;
        *reinterpret_cast<V4*>(kd + 64 + c4) = y2;
      }
    }
  }
}

template <typename T, typename W>
void launch_prologue_kernel(PrologueArgs a, int64_t blocks, hipStream_t s) {
  if (a.k_cache == nullptr) {
    a.slots = a.positions;
    hipLaunchKernelGGL((qk_norm_rope_store_kernel<T, W, int64_t>), dim3((uint32_t)blocks), dim3(256), 0, s, a);
  } else if (a.slot_is_int64) {
    hipLaunchKernelGGL((qk_norm_rope_store_kernel<T, W, int64_t>), dim3((uint32_t)blocks), dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL((qk_norm_rope_store_kernel<T, W, int32_t>), dim3((uint32_t)blocks), dim3(256), 0, s, a);
  }
}

template <typename T>
int launch_prologue(const PrologueArgs& a, int weight_dtype, hipStream_t s) {
  const int rows = a.num_q_heads + a.num_kv_heads + (a.k_cache != nullptr ? a.num_kv_heads : 0);
  const int64_t items = a.num_tokens * (((rows + 3) / 4 + kChunk - 1) / kChunk);
  // Four wavefronts per workgroup; at most 16 workgroups per CU's worth,
  // beyond which the wavefronts loop.
  const int64_t blocks = std::min<int64_t>((items + 3) / 4, 256 * 16);
  if (weight_dtype == kF32)
    launch_prologue_kernel<T, float>(a, blocks, s);
  else
    launch_prologue_kernel<T, T>(a, blocks, s);
  return check_launch("qk_norm_rope_store");
}

}  // namespace
}  // namespace mva

extern "C" int mva_qk_norm_rope_store(const void* q_in, void* q_out, int64_t q_token_stride, int64_t q_head_stride,
                                      int num_q_heads, const void* k_in, void* k_out, int64_t k_token_stride,
                                      int64_t k_head_stride, const void* v, int64_t v_token_stride,
                                      int64_t v_head_stride, int num_kv_heads, const int64_t* positions,
                                      const float* cos_sin_cache, int64_t max_position, int rotary_dim,
                                      const void* q_norm_weight, const void* k_norm_weight, int weight_dtype,
                                      float eps, void* k_cache, void* v_cache, int64_t num_slots,
                                      const void* slot_mapping, int slot_is_int64, int64_t num_tokens, int head_dim,
                                      int dtype, void* stream) {
  using namespace mva;
  if (head_dim != kRopeDim || rotary_dim != kRopeDim)
    return set_error("qk_norm_rope: head_dim and rotary_dim must be 128");
  if (num_q_heads < 0 || num_kv_heads < 0 || num_tokens < 0) return set_error("qk_norm_rope: invalid shape");
  if (num_tokens == 0 || num_q_heads + num_kv_heads == 0) return 0;
  if (positions == nullptr || cos_sin_cache == nullptr || max_position <= 0)
    return set_error("qk_norm_rope: positions and cos_sin_cache are required");
  if ((q_norm_weight == nullptr) != (k_norm_weight == nullptr))
    return set_error("qk_norm_rope: give both norm weights or neither");
  if (k_cache != nullptr && (v_cache == nullptr || slot_mapping == nullptr || v == nullptr))
    return set_error("qk_norm_rope: the store needs v, v_cache and slot_mapping");
  if (q_norm_weight != nullptr && weight_dtype != kF32 && weight_dtype != dtype)
    return set_error("qk_norm_rope: norm weights must be fp32 or the input dtype");
  const uint64_t align = (uint64_t)(uintptr_t)q_in | (uint64_t)(uintptr_t)q_out | (uint64_t)(uintptr_t)k_in |
                         (uint64_t)(uintptr_t)k_out | (uint64_t)(uintptr_t)v | (uint64_t)(uintptr_t)k_cache |
                         (uint64_t)(uintptr_t)v_cache | (uint64_t)(q_token_stride | q_head_stride | k_token_stride |
                                                                k_head_stride | v_token_stride | v_head_stride) * 2 |
                         (uint64_t)(uintptr_t)cos_sin_cache | (uint64_t)(uintptr_t)q_norm_weight |
                         (uint64_t)(uintptr_t)k_norm_weight;
  if (align % 8 != 0)
    return set_error("qk_norm_rope: buffers and strides must be 8-byte aligned");
  if (((uint64_t)(uintptr_t)cos_sin_cache | (uint64_t)(uintptr_t)q_norm_weight | (uint64_t)(uintptr_t)k_norm_weight) % 16)
    return set_error("qk_norm_rope: cos_sin_cache and norm weights must be 16-byte aligned");
  PrologueArgs a{q_in, q_out, q_token_stride, q_head_stride, k_in, k_out, k_token_stride, k_head_stride,
                 v, v_token_stride, v_head_stride, num_q_heads, num_kv_heads, positions, cos_sin_cache,
                 max_position, q_norm_weight, k_norm_weight, eps, k_cache, v_cache, num_slots, slot_mapping,
                 slot_is_int64, num_tokens};
  hipStream_t s = (hipStream_t)stream;
  if (dtype == kBF16) return launch_prologue<__bf16>(a, weight_dtype, s);
  if (dtype == kF16) return launch_prologue<_Float16>(a, weight_dtype, s);
  return set_error("qk_norm_rope: dtype must be bf16 or fp16");
}
