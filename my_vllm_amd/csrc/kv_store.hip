// slot_mapping KV-cache store for gfx950.
//
// For every token t with slot_mapping[t] >= 0, copies the token's K and V rows
// (num_kv_heads * head_dim contiguous elements each, arbitrary row stride) to
// row slot_mapping[t] of the flat [num_pages * page_size, num_kv_heads *
// head_dim] view of k_cache / v_cache.  Negative slots are skipped, matching
// the reference's native path (nanovllm/layers/attention.py:69-85: `slot >= 0`
// mask) and its Triton kernel's `-1` early exit (:11-31).  Slots at or beyond
// the cache end are skipped as well instead of writing out of bounds.
//
// It is a byte copy, so the kernel is dtype-agnostic: each workgroup handles
// one token; its first half copies K, its second half V, in the widest access
// (16, 8, 4 or 2 bytes) that the row strides and base pointers allow.
#include "mva_capi.h"
#include "mva_common.h"

namespace mva {
namespace {

template <typename SlotT, typename W>
__global__ __launch_bounds__(256) void kv_store_kernel(
    const uint8_t* __restrict__ key, int64_t key_stride_b, const uint8_t* __restrict__ value,
    int64_t value_stride_b, uint8_t* __restrict__ k_cache, uint8_t* __restrict__ v_cache,
    int64_t num_slots, const SlotT* __restrict__ slots, int64_t row_bytes) {
  const int64_t t = blockIdx.x;
  const int64_t slot = (int64_t)slots[t];
  if (slot < 0 || slot >= num_slots) return;
  const int nw = (int)(row_bytes / (int64_t)sizeof(W));
  const W* ks = reinterpret_cast<const W*>(key + t * key_stride_b);
  const W* vs = reinterpret_cast<const W*>(value + t * value_stride_b);
  W* kd = reinterpret_cast<W*>(k_cache + slot * row_bytes);
  W* vd = reinterpret_cast<W*>(v_cache + slot * row_bytes);
  for (int i = threadIdx.x; i < 2 * nw; i += 256) {
    if (i < nw) kd[i] = ks[i];
    else vd[i - nw] = vs[i - nw];
  }
}

template <typename SlotT, typename W>
int launch(const void* key, int64_t ks, const void* value, int64_t vs, void* kc, void* vc,
           int64_t num_slots, const void* slots, int64_t num_tokens, int64_t row_bytes,
           hipStream_t stream) {
  hipLaunchKernelGGL((kv_store_kernel<SlotT, W>), dim3((uint32_t)num_tokens), dim3(256), 0, stream,
                     (const uint8_t*)key, ks, (const uint8_t*)value, vs, (uint8_t*)kc, (uint8_t*)vc,
                     num_slots, (const SlotT*)slots, row_bytes);
  return check_launch("kv_store");
}

template <typename SlotT>
int dispatch_width(const void* key, int64_t ks, const void* value, int64_t vs, void* kc, void* vc,
                   int64_t num_slots, const void* slots, int64_t num_tokens, int64_t row_bytes,
                   hipStream_t stream) {
  uint64_t bits = (uint64_t)(uintptr_t)key | (uint64_t)(uintptr_t)value | (uint64_t)(uintptr_t)kc |
                  (uint64_t)(uintptr_t)vc | (uint64_t)ks | (uint64_t)vs | (uint64_t)row_bytes;
  if (bits % 16 == 0) return launch<SlotT, uint4>(key, ks, value, vs, kc, vc, num_slots, slots, num_tokens, row_bytes, stream);
  if (bits % 8 == 0) return launch<SlotT, uint2>(key, ks, value, vs, kc, vc, num_slots, slots, num_tokens, row_bytes, stream);
  if (bits % 4 == 0) return launch<SlotT, uint32_t>(key, ks, value, vs, kc, vc, num_slots, slots, num_tokens, row_bytes, stream);
  return launch<SlotT, uint16_t>(key, ks, value, vs, kc, vc, num_slots, slots, num_tokens, row_bytes, stream);
}

}  // namespace
}  // namespace mva

extern "C" int mva_kv_store(const void* key, int64_t key_row_stride, const void* value,
                            int64_t value_row_stride, void* k_cache, void* v_cache, int64_t num_slots,
                            const void* slot_mapping, int slot_is_int64, int64_t num_tokens,
                            int64_t row_elems, int dtype, void* stream) {
  using namespace mva;
  if (num_tokens < 0 || row_elems <= 0 || num_slots < 0) return set_error("kv_store: invalid sizes");
  if (num_tokens == 0 || num_slots == 0) return 0;
  if (num_tokens > 0x7fffffffLL) return set_error("kv_store: too many tokens for one launch");
  if (!key || !value || !k_cache || !v_cache || !slot_mapping) return set_error("kv_store: null buffer");
  if (dtype != kBF16 && dtype != kF16) return set_error("kv_store: dtype must be bf16 or fp16");
  const int64_t esz = 2;
  const int64_t row_bytes = row_elems * esz;
  hipStream_t s = (hipStream_t)stream;
  if (slot_is_int64)
    return dispatch_width<int64_t>(key, key_row_stride * esz, value, value_row_stride * esz, k_cache,
                                   v_cache, num_slots, slot_mapping, num_tokens, row_bytes, s);
  return dispatch_width<int32_t>(key, key_row_stride * esz, value, value_row_stride * esz, k_cache,
                                 v_cache, num_slots, slot_mapping, num_tokens, row_bytes, s);
}
