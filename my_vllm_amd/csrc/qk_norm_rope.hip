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
// One wavefront per (token, head) row of q, k or v; lane j owns elements j
// and j + 64 of the 128-wide head, exactly the pair the rotation mixes, so
// the norm's sum of squares is the only cross-lane step.
#include "mva_capi.h"
#include "mva_common.h"

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

template <typename W>
__device__ inline float wget(const void* w, int i) {
  return (float)((const W*)w)[i];
}

template <typename T, typename W>
__global__ __launch_bounds__(256) void qk_norm_rope_store_kernel(PrologueArgs a) {
  // Separate fp32 multiplies and adds, as torch evaluates the rotation (no
  // fused multiply-add contraction).
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int rows_per_tok = a.num_q_heads + a.num_kv_heads + (a.k_cache != nullptr ? a.num_kv_heads : 0);
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.num_tokens * rows_per_tok) return;
  const int64_t t = row / rows_per_tok;
  const int r = (int)(row - t * rows_per_tok);
  int64_t slot = -1;
  if (a.k_cache != nullptr) {
    slot = a.slot_is_int64 ? ((const int64_t*)a.slots)[t] : (int64_t)((const int32_t*)a.slots)[t];
    if (slot >= a.num_slots) slot = -1;
  }
  const int64_t cache_row = (slot >= 0) ? slot * a.num_kv_heads : 0;  // rows of [slots * Hkv, 128]

  if (r >= a.num_q_heads + a.num_kv_heads) {  // V: copy into the cache
    if (slot < 0) return;
    const int h = r - a.num_q_heads - a.num_kv_heads;
    const T* src = (const T*)a.v + t * a.v_tok_stride + h * a.v_head_stride;
    T* dst = (T*)a.v_cache + (cache_row + h) * kRopeDim;
    dst[lane] = src[lane];
    dst[lane + 64] = src[lane + 64];
    return;
  }
  const bool is_q = r < a.num_q_heads;
  const int h = is_q ? r : r - a.num_q_heads;
  const T* src = is_q ? (const T*)a.q_in + t * a.q_tok_stride + h * a.q_head_stride
                      : (const T*)a.k_in + t * a.k_tok_stride + h * a.k_head_stride;
  float x1 = (float)src[lane];
  float x2 = (float)src[lane + 64];
  const void* w = is_q ? a.q_norm_w : a.k_norm_w;
  if (w != nullptr) {
    float ss = x1 * x1 + x2 * x2;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    const float rr = 1.0f / __builtin_sqrtf(ss / (float)kRopeDim + a.eps);
    x1 = (float)(T)((float)(T)(x1 * rr) * wget<W>(w, lane));
    x2 = (float)(T)((float)(T)(x2 * rr) * wget<W>(w, lane + 64));
  }
  int64_t pos = a.positions[t];
  pos = pos < 0 ? 0 : (pos >= a.max_position ? a.max_position - 1 : pos);  // stay in bounds
  const float c = a.cos_sin[pos * kRopeDim + lane];
  const float s = a.cos_sin[pos * kRopeDim + 64 + lane];
  const T y1 = (T)(x1 * c - x2 * s);
  const T y2 = (T)(x2 * c + x1 * s);
  T* dst = is_q ? (T*)a.q_out + t * a.q_tok_stride + h * a.q_head_stride
                : (T*)a.k_out + t * a.k_tok_stride + h * a.k_head_stride;
  dst[lane] = y1;
  dst[lane + 64] = y2;
  if (!is_q && slot >= 0) {
    T* kd = (T*)a.k_cache + (cache_row + h) * kRopeDim;
    kd[lane] = y1;
    kd[lane + 64] = y2;
  }
}

template <typename T>
int launch_prologue(const PrologueArgs& a, int weight_dtype, hipStream_t s) {
  const int64_t rows = a.num_tokens * (a.num_q_heads + a.num_kv_heads + (a.k_cache != nullptr ? a.num_kv_heads : 0));
  const int64_t blocks = (rows + 3) / 4;
  if (blocks > 0x7fffffffLL) return set_error("qk_norm_rope: too many rows");
  if (weight_dtype == kF32)
    hipLaunchKernelGGL((qk_norm_rope_store_kernel<T, float>), dim3((uint32_t)blocks), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((qk_norm_rope_store_kernel<T, T>), dim3((uint32_t)blocks), dim3(256), 0, s, a);
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
  PrologueArgs a{q_in, q_out, q_token_stride, q_head_stride, k_in, k_out, k_token_stride, k_head_stride,
                 v, v_token_stride, v_head_stride, num_q_heads, num_kv_heads, positions, cos_sin_cache,
                 max_position, q_norm_weight, k_norm_weight, eps, k_cache, v_cache, num_slots, slot_mapping,
                 slot_is_int64, num_tokens};
  hipStream_t s = (hipStream_t)stream;
  if (dtype == kBF16) return launch_prologue<__bf16>(a, weight_dtype, s);
  if (dtype == kF16) return launch_prologue<_Float16>(a, weight_dtype, s);
  return set_error("qk_norm_rope: dtype must be bf16 or fp16");
}
