// C-ABI entry point of the paged GQA decode kernel (kernel body in
// paged_decode.h, shared with the single-launch MIXED kernel).
#include "mva_capi.h"
#include "paged_decode.h"

#include <mutex>

namespace mva {
namespace {

// kWaves wavefronts per workgroup, each with private LDS buffers; wavefront
// w of workgroup b is decode wavefront b * kWaves + w.
template <typename T, int kWaves>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(2))) void paged_decode_kernel(
    DecodeParams p) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kWaves * kDecodeWaveLdsBytes];
  // Page counts of the wavefronts (8-wavefront groups pair w with w ^ 4 on a
  // SIMD); a wavefront without work reads as far ahead.
  __shared__ int progress[8];
  const int w = kWaves == 1 ? 0 : __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int wave = (int)blockIdx.x * kWaves + w;
  if (kWaves == 8 && (threadIdx.x & 63) == 0) progress[w] = 0x3fffffff;
  if (wave >= p.num_waves) return;
  decode_wave<T>(p, wave, (lds_u8*)lds + w * kDecodeWaveLdsBytes, kWaves == 8 ? progress : nullptr);
}

template <typename T>
int launch_paged_decode(const DecodeParams& p, int waves_per_group, hipStream_t s) {
  const uint32_t blocks = (uint32_t)((p.num_waves + waves_per_group - 1) / waves_per_group);
  switch (waves_per_group) {
    case 1: hipLaunchKernelGGL((paged_decode_kernel<T, 1>), dim3(blocks), dim3(64), 0, s, p); break;
    case 2: hipLaunchKernelGGL((paged_decode_kernel<T, 2>), dim3(blocks), dim3(128), 0, s, p); break;
    case 4: hipLaunchKernelGGL((paged_decode_kernel<T, 4>), dim3(blocks), dim3(256), 0, s, p); break;
    case 8: hipLaunchKernelGGL((paged_decode_kernel<T, 8>), dim3(blocks), dim3(512), 0, s, p); break;
    default: return set_error("paged attention: waves_per_group must be 1, 2, 4 or 8");
  }
  return check_launch("paged_decode");
}

// Split-K merges: four wavefronts per workgroup, one per (merge entry,
// query head), in the first merge_blocks workgroups.  Graph launches size the
// grid for the merge capacity and read this step's merge count from
// p.counts[2].  After a fused-store launch the workgroups past merge_blocks
// write the late rows, one wavefront per new token.
template <typename T>
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeParams p, const int32_t* __restrict__ merges,
                                                           int64_t num_waves, int64_t merge_blocks) {
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if ((int64_t)blockIdx.x >= merge_blocks) {
    const int64_t row = ((int64_t)blockIdx.x - merge_blocks) * 4 + w;
    if (row < p.num_new) decode_late_store_wave<T>(p, row);
    return;
  }
  const int64_t v = (int64_t)blockIdx.x * 4 + w;
  if (v >= num_waves) return;
  if (p.counts != nullptr && v >= (int64_t)max(sload(p.counts, 2), 0) * p.group) return;
  decode_merge_wave<T>(p, merges, v);
}

}  // namespace

// Launches the split-K merge kernel after a decode (or MIXED) launch on the
// same stream; `merges` lists the split segments (piece descriptors).  After
// a fused-store launch (p.k_new set) it always runs: its late-store
// workgroups write the new rows the decode launch left.
int launch_decode_merge(const DecodeParams& p, const int32_t* merges, int64_t num_merges, int dtype,
                        hipStream_t stream) {
  const int64_t late_rows = p.k_new != nullptr ? p.num_new : 0;
  if (num_merges == 0 && late_rows == 0) return 0;
  const int64_t waves = num_merges * p.group;
  const int64_t merge_blocks = (waves + 3) / 4;
  const int64_t blocks = merge_blocks + (late_rows + 3) / 4;
  if (blocks > 0x7fffffffLL) return set_error("paged attention: too many split-K merges");
  if (dtype == kBF16)
    hipLaunchKernelGGL(decode_merge_kernel<__bf16>, dim3((uint32_t)blocks), dim3(256), 0, stream, p, merges, waves,
                       merge_blocks);
  else
    hipLaunchKernelGGL(decode_merge_kernel<_Float16>, dim3((uint32_t)blocks), dim3(256), 0, stream, p, merges,
                       waves, merge_blocks);
  return check_launch("decode_merge");
}

static int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

// Workspace layout: [scheduler (kDecodeSchedBytes)][arrival counters
// (kArrivalBytes, MIXED launches)][fused-store row flags (kStoreFlagBytes)]
// [lse f32 slots*Hkv*G][o f32 slots*Hkv*G*D].
int64_t decode_workspace_bytes(int64_t slots, int hkv, int group) {
  return kDecodeSchedBytes + kArrivalBytes + kStoreFlagBytes + align256(slots * hkv * group * 4) +
         align256(slots * hkv * group * kHeadDim * 4);
}

// The arrival counters of a workspace laid out as above.
int32_t* decode_arrival_counters(void* workspace) { return (int32_t*)((uint8_t*)workspace + kDecodeSchedBytes); }

int fill_decode_params(DecodeParams& p, const void* q, int64_t q_token_stride, int64_t q_head_stride,
                       const void* k_cache, const void* v_cache, int64_t num_pages, int64_t page_stride,
                       int64_t token_stride, const int32_t* block_tables, int64_t block_table_stride,
                       const int32_t* seq_lens, const int32_t* items, int64_t num_items, int64_t num_waves,
                       const int32_t* wave_extra, const int32_t* merges, int64_t num_merges, int64_t num_part_slots, void* out,
                       int64_t out_token_stride,
                       int64_t out_head_stride, void* workspace, int64_t workspace_bytes,
                       int num_q_heads, int num_kv_heads, int head_dim, int page_size,
                       float softmax_scale) {
  if (head_dim != kHeadDim) return set_error("paged attention: head_dim must be 128");
  if (page_size != kPageSize) return set_error("paged attention: page_size must be 16");
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads)
    return set_error("paged attention: num_q_heads must be a positive multiple of num_kv_heads");
  const int group = num_q_heads / num_kv_heads;
  if (group > 16) return set_error("paged attention: at most 16 query heads per KV head");
  if (num_items < 0 || num_items > 0x7fffffffLL) return set_error("paged attention: invalid item count");
  if (num_waves < 0 || num_waves > 0x7fffffffLL) return set_error("paged attention: invalid wave count");
  if (num_items > 0 && (num_waves <= 0 || num_waves > num_items))
    return set_error("paged attention: num_waves must be in [1, num_items]");
  if (num_merges < 0 || num_merges > num_items) return set_error("paged attention: invalid merge count");
  if (num_merges > 0 && merges == nullptr) return set_error("paged attention: missing merge list");
  if (num_pages <= 0) return set_error("paged attention: empty KV cache");
  const uint64_t align_bits = (uint64_t)(uintptr_t)q | (uint64_t)(uintptr_t)k_cache |
                              (uint64_t)(uintptr_t)v_cache | (uint64_t)(q_token_stride * 2) |
                              (uint64_t)(q_head_stride * 2) | (uint64_t)(page_stride * 2) |
                              (uint64_t)(token_stride * 2);
  if (align_bits % 16) return set_error("paged attention: q / cache buffers and strides must be 16-byte aligned");
  if (((uint64_t)(uintptr_t)out | (uint64_t)(out_token_stride * 2) | (uint64_t)(out_head_stride * 2)) % 8)
    return set_error("paged attention: output buffer and strides must be 8-byte aligned");
  if (num_part_slots < 0) return set_error("paged attention: invalid partial slot count");
  if (workspace_bytes < decode_workspace_bytes(num_part_slots, num_kv_heads, group))
    return set_error("paged attention: workspace too small");
  if (num_items > 0 && workspace == nullptr) return set_error("paged attention: missing workspace");
  p.q = q;
  p.q_tok_stride = q_token_stride;
  p.q_head_stride = q_head_stride;
  p.k_cache = k_cache;
  p.v_cache = v_cache;
  p.num_pages = num_pages;
  p.page_stride = page_stride;
  p.tok_stride = token_stride;
  p.block_tables = block_tables;
  p.bt_stride = block_table_stride;
  p.seq_lens = seq_lens;
  p.items = items;
  p.num_items = (int)num_items;
  p.num_waves = (int)num_waves;
  p.wave_extra = wave_extra;
  p.counts = nullptr;
  p.out = out;
  p.out_tok_stride = out_token_stride;
  p.out_head_stride = out_head_stride;
  uint8_t* ws = (uint8_t*)workspace;
  p.k_new = nullptr;
  p.v_new = nullptr;
  p.slots = nullptr;
  p.num_new = 0;
  p.sched = (int32_t*)ws;
  ws += kDecodeSchedBytes + kArrivalBytes;
  p.store_flags = (int32_t*)ws;
  ws += kStoreFlagBytes;
  p.part_lse = (float*)ws;
  ws += align256(num_part_slots * num_kv_heads * group * 4);
  p.part_o = (float*)ws;
  p.arrive = nullptr;  // merges by the merge kernel
  p.num_kv_heads = num_kv_heads;
  p.group = group;
  p.scale_log2 = softmax_scale * 1.4426950408889634f;
  return 0;
}

}  // namespace mva

extern "C" int64_t mva_decode_workspace_bytes(int64_t num_part_slots, int num_kv_heads, int group) {
  if (num_part_slots < 0 || num_kv_heads <= 0 || group <= 0) return -1;
  return mva::decode_workspace_bytes(num_part_slots, num_kv_heads, group);
}

extern "C" int mva_paged_decode(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                                const void* k_cache, const void* v_cache, int64_t num_pages,
                                int64_t page_stride, int64_t token_stride, const int32_t* block_tables,
                                int64_t block_table_stride, const int32_t* seq_lens,
                                const int32_t* items, int64_t num_items, int64_t num_waves,
                                const int32_t* wave_extra, int waves_per_group,
                                const int32_t* merges, int64_t num_merges,
                                int64_t num_part_slots, void* out, int64_t out_token_stride,
                                int64_t out_head_stride, void* workspace, int64_t workspace_bytes,
                                int num_q_heads, int num_kv_heads, int head_dim, int page_size,
                                float softmax_scale, int dtype, void* stream) {
  using namespace mva;
  DecodeParams p;
  int rc = fill_decode_params(p, q, q_token_stride, q_head_stride, k_cache, v_cache, num_pages,
                              page_stride, token_stride, block_tables, block_table_stride, seq_lens,
                              items, num_items, num_waves, wave_extra, merges, num_merges, num_part_slots, out,
                              out_token_stride,
                              out_head_stride, workspace, workspace_bytes, num_q_heads, num_kv_heads,
                              head_dim, page_size, softmax_scale);
  if (rc) return rc;
  if (wave_extra == nullptr && waves_per_group != 1)
    return set_error("paged attention: the claim schedule runs one wavefront per workgroup");
  if (num_items == 0) return 0;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == kBF16) rc = launch_paged_decode<__bf16>(p, waves_per_group, s);
  else if (dtype == kF16) rc = launch_paged_decode<_Float16>(p, waves_per_group, s);
  else return set_error("paged attention: dtype must be bf16 or fp16");
  if (rc) return rc;
  return launch_decode_merge(p, merges, num_merges, dtype, s);
}

extern "C" int mva_paged_decode_store(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                                      const void* k_cache, const void* v_cache, int64_t num_pages,
                                      int64_t page_stride, int64_t token_stride, const int32_t* block_tables,
                                      int64_t block_table_stride, const int32_t* seq_lens,
                                      const int32_t* items, int64_t num_items, int64_t num_waves,
                                      const int32_t* wave_extra, int waves_per_group,
                                      const int32_t* merges, int64_t num_merges,
                                      int64_t num_part_slots, void* out, int64_t out_token_stride,
                                      int64_t out_head_stride, void* workspace, int64_t workspace_bytes,
                                      const void* k_new, int64_t k_token_stride, int64_t k_head_stride,
                                      const void* v_new, int64_t v_token_stride, int64_t v_head_stride,
                                      const void* slot_mapping, int slot_is_int64, int64_t num_new_tokens,
                                      int num_q_heads, int num_kv_heads, int head_dim, int page_size,
                                      float softmax_scale, int dtype, void* stream) {
  using namespace mva;
  if (wave_extra == nullptr) return set_error("paged attention: the fused store needs piece lists (wave_extra)");
  if (k_new == nullptr || v_new == nullptr || slot_mapping == nullptr)
    return set_error("paged attention: the fused store needs k, v and slot_mapping");
  if (num_new_tokens < 0 || num_new_tokens > 0x7fffffffLL) return set_error("paged attention: invalid token count");
  if (num_kv_heads > 0 && num_new_tokens * num_kv_heads > kStoreFlagInts)
    return set_error("paged attention: the fused store takes at most 65536 (token, KV head) rows");
  if (((uint64_t)(uintptr_t)k_new | (uint64_t)(uintptr_t)v_new | (uint64_t)(k_token_stride * 2) |
       (uint64_t)(k_head_stride * 2) | (uint64_t)(v_token_stride * 2) | (uint64_t)(v_head_stride * 2)) % 4)
    return set_error("paged attention: k / v rows must be 4-byte aligned");
  DecodeParams p;
  int rc = fill_decode_params(p, q, q_token_stride, q_head_stride, k_cache, v_cache, num_pages,
                              page_stride, token_stride, block_tables, block_table_stride, seq_lens,
                              items, num_items, num_waves, wave_extra, merges, num_merges, num_part_slots, out,
                              out_token_stride, out_head_stride, workspace, workspace_bytes, num_q_heads,
                              num_kv_heads, head_dim, page_size, softmax_scale);
  if (rc) return rc;
  p.k_new = k_new;
  p.kn_tok_stride = k_token_stride;
  p.kn_head_stride = k_head_stride;
  p.v_new = v_new;
  p.vn_tok_stride = v_token_stride;
  p.vn_head_stride = v_head_stride;
  p.slots = slot_mapping;
  p.slots_int64 = slot_is_int64 ? 1 : 0;
  p.num_new = (int)num_new_tokens;
  hipStream_t s = (hipStream_t)stream;
  if (dtype != kBF16 && dtype != kF16) return set_error("paged attention: dtype must be bf16 or fp16");
  // With no pieces every new row is a late row of the merge kernel.
  if (num_items > 0) {
    rc = dtype == kBF16 ? launch_paged_decode<__bf16>(p, waves_per_group, s)
                        : launch_paged_decode<_Float16>(p, waves_per_group, s);
    if (rc) return rc;
  }
  return launch_decode_merge(p, merges, num_merges, dtype, s);
}

extern "C" int mva_paged_decode_graph(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                                      const void* k_cache, const void* v_cache, int64_t num_pages,
                                      int64_t page_stride, int64_t token_stride, const int32_t* block_tables,
                                      int64_t block_table_stride, const int32_t* seq_lens, const int32_t* counts,
                                      const int32_t* items, int64_t item_capacity, const int32_t* wave_extra,
                                      int64_t wave_capacity, int waves_per_group, const int32_t* merges,
                                      int64_t merge_capacity, int64_t num_part_slots, void* out,
                                      int64_t out_token_stride, int64_t out_head_stride, void* workspace,
                                      int64_t workspace_bytes, int num_q_heads, int num_kv_heads, int head_dim,
                                      int page_size, float softmax_scale, int dtype, void* stream) {
  using namespace mva;
  if (counts == nullptr || items == nullptr || wave_extra == nullptr)
    return set_error("paged attention: graph launch needs counts, items and wave_extra");
  if (wave_capacity <= 0 || wave_capacity > item_capacity)
    return set_error("paged attention: graph launch needs 0 < wave_capacity <= item_capacity");
  if (merge_capacity < 0 || (merge_capacity > 0 && merges == nullptr))
    return set_error("paged attention: invalid merge capacity");
  DecodeParams p;
  int rc = fill_decode_params(p, q, q_token_stride, q_head_stride, k_cache, v_cache, num_pages, page_stride,
                              token_stride, block_tables, block_table_stride, seq_lens, items, item_capacity,
                              wave_capacity, wave_extra, merges, merge_capacity, num_part_slots, out,
                              out_token_stride, out_head_stride, workspace, workspace_bytes, num_q_heads,
                              num_kv_heads, head_dim, page_size, softmax_scale);
  if (rc) return rc;
  p.counts = counts;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == kBF16) rc = launch_paged_decode<__bf16>(p, waves_per_group, s);
  else if (dtype == kF16) rc = launch_paged_decode<_Float16>(p, waves_per_group, s);
  else return set_error("paged attention: dtype must be bf16 or fp16");
  if (rc) return rc;
  return launch_decode_merge(p, merges, merge_capacity, dtype, s);
}

// ---- decode with no allocation: static device scratch ---------------------
//
// mva_paged_decode_noalloc runs mva_paged_decode's kernels with the decode
// workspace (scheduler counters + split-K partials) placed in `scratch`, a
// file-scope device array, so a call allocates nothing.  Each GPU holds its
// own copy for the life of the process.  In host code `scratch` names a
// host-side stand-in: its device address on the current GPU comes from
// hipGetSymbolAddress, looked up once per device and kept in
// g_scratch_addr; only that address is ever handed to a kernel.

namespace mva {
namespace {

constexpr int64_t kStaticScratchBytes = int64_t(64) << 20;  // MVA_DECODE_STATIC_SCRATCH_BYTES
constexpr int kMaxScratchDevices = 64;

static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

std::mutex g_scratch_mutex;
void* g_scratch_addr[kMaxScratchDevices] = {};

// Zeroes `words` 32-bit words with vector stores (graph-capturable, unlike
// a memset node).
__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t* p, int words) {
  for (int i = threadIdx.x; i < words; i += 256) p[i] = 0u;
}

// The current device's scratch address.  The first call on a device looks it
// up and clears the scheduler area with one kernel on `stream`; the decode
// kernels leave it cleared again on exit, so later calls clear nothing.
int static_scratch(hipStream_t stream, void** addr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices)
    return set_error("paged attention (no-alloc): no usable current HIP device");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_addr[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || ptr == nullptr)
      return set_error("paged attention (no-alloc): hipGetSymbolAddress of the static scratch failed");
    hipLaunchKernelGGL(zero_words_kernel, dim3(1), dim3(256), 0, stream, (uint32_t*)ptr, kDecodeSchedBytes / 4);
    if (const int rc = check_launch("paged attention (no-alloc) scratch clear")) return rc;
    g_scratch_addr[dev] = ptr;
  }
  *addr = g_scratch_addr[dev];
  return 0;
}

}  // namespace
}  // namespace mva

extern "C" int mva_paged_decode_noalloc(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                                        const void* k_cache, const void* v_cache, int64_t num_pages,
                                        int64_t page_stride, int64_t token_stride, const int32_t* block_tables,
                                        int64_t block_table_stride, const int32_t* seq_lens,
                                        const int32_t* items, int64_t num_items, int64_t num_waves,
                                        const int32_t* wave_extra, int waves_per_group,
                                        const int32_t* merges, int64_t num_merges,
                                        int64_t num_part_slots, void* out, int64_t out_token_stride,
                                        int64_t out_head_stride, int num_q_heads, int num_kv_heads,
                                        int head_dim, int page_size, float softmax_scale, int dtype,
                                        void* stream) {
  using namespace mva;
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads || num_part_slots < 0)
    return set_error("paged attention (no-alloc): invalid head counts or partial slot count");
  const int64_t need = decode_workspace_bytes(num_part_slots, num_kv_heads, num_q_heads / num_kv_heads);
  if (need > kStaticScratchBytes)
    return set_error("paged attention (no-alloc): the plan's split-K partials exceed the 64 MiB static "
                     "scratch; use mva_paged_decode with a workspace");
  hipStream_t s = (hipStream_t)stream;
  void* ws = nullptr;
  if (const int rc = static_scratch(s, &ws)) return rc;
  return mva_paged_decode(q, q_token_stride, q_head_stride, k_cache, v_cache, num_pages, page_stride,
                          token_stride, block_tables, block_table_stride, seq_lens, items, num_items, num_waves,
                          wave_extra, waves_per_group, merges, num_merges, num_part_slots, out,
                          out_token_stride, out_head_stride, ws, kStaticScratchBytes, num_q_heads,
                          num_kv_heads, head_dim, page_size, softmax_scale, dtype, stream);
}
