// C-ABI entry points of the ragged causal prefill kernel and of the
// single-launch MIXED kernel (prefill tiles + decode items in one grid).
#include "mva_capi.h"
#include "paged_prefill.h"

namespace mva {

int fill_decode_params(DecodeParams& p, const void* q, int64_t q_token_stride, int64_t q_head_stride,
                       const void* k_cache, const void* v_cache, int64_t num_pages, int64_t page_stride,
                       int64_t token_stride, const int32_t* block_tables, int64_t block_table_stride,
                       const int32_t* seq_lens, const int32_t* items, int64_t num_items, int64_t num_waves,
                       const int32_t* wave_extra, const int32_t* merges, int64_t num_merges, int64_t num_part_slots, void* out,
                       int64_t out_token_stride,
                       int64_t out_head_stride, void* workspace, int64_t workspace_bytes,
                       int num_q_heads, int num_kv_heads, int head_dim, int page_size,
                       float softmax_scale);
int launch_decode_merge(const DecodeParams& p, const int32_t* merges, int64_t num_merges, int dtype,
                        hipStream_t stream);

namespace {

template <typename T>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void paged_prefill_kernel(
    PrefillParams p) {
  __shared__ __attribute__((aligned(16))) uint8_t k0[kPrefillTileBytes];
  __shared__ __attribute__((aligned(16))) uint8_t k1[kPrefillTileBytes];
  __shared__ __attribute__((aligned(16))) uint8_t v0[kPrefillTileBytes];
  __shared__ __attribute__((aligned(16))) uint8_t v1[kPrefillTileBytes];
  const int h = (int)(blockIdx.x % (uint32_t)p.num_kv_heads);
  const int item = (int)(blockIdx.x / (uint32_t)p.num_kv_heads);
  prefill_item<T>(p, p.items + (int64_t)item * kPrefillItemInts, h, (lds_u8*)k0, (lds_u8*)k1, (lds_u8*)v0,
                  (lds_u8*)v1);
}

// Workgroup roles of the MIXED launch: the decode workgroups come first, in
// chunks of 8 blocks (blocks are dealt to the 8 XCDs round-robin), then the
// prefill workgroups.  The host sizes the decode part below the GPU's
// resident capacity, so every decode wavefront starts at once and prefill
// tiles fill the remaining slots (and the slots decode frees): HBM-bound
// decode streaming overlaps MFMA-bound prefill on the same CUs.  Prefill
// blocks keep index % 8 == block % 8, so a prefill work item's KV head
// (index % num_kv_heads) stays on the same XCD as in the prefill-only launch.
struct MixedRole {
  bool prefill;
  uint32_t index;  // prefill workgroup or decode workgroup number
};
__host__ __device__ inline uint32_t mixed_chunks(uint32_t n) { return (n + 7u) >> 3; }
__device__ inline MixedRole mixed_role(uint32_t block, uint32_t n_decode_wgs) {
  const uint32_t c = block >> 3, r = block & 7u;
  const uint32_t cd = mixed_chunks(n_decode_wgs);
  if (c < cd) return {false, c * 8u + r};
  return {true, (c - cd) * 8u + r};
}

// Prefill workgroups run prefill tiles; decode workgroups run four decode
// wavefronts each, with private LDS buffers.
template <typename T>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void paged_mixed_kernel(
    PrefillParams pp, DecodeParams dp, uint32_t n_prefill_wgs, uint32_t n_decode_wgs) {
  __shared__ __attribute__((aligned(16))) uint8_t k0[kPrefillTileBytes];
  __shared__ __attribute__((aligned(16))) uint8_t k1[kPrefillTileBytes];
  __shared__ __attribute__((aligned(16))) uint8_t v0[kPrefillTileBytes];
  __shared__ __attribute__((aligned(16))) uint8_t v1[kPrefillTileBytes];
  const MixedRole role = mixed_role(blockIdx.x, n_decode_wgs);
  if (role.prefill) {
    if (role.index >= n_prefill_wgs) return;
    const int h = (int)(role.index % (uint32_t)pp.num_kv_heads);
    const int item = (int)(role.index / (uint32_t)pp.num_kv_heads);
    prefill_item<T>(pp, pp.items + (int64_t)item * kPrefillItemInts, h, (lds_u8*)k0, (lds_u8*)k1,
                    (lds_u8*)v0, (lds_u8*)v1);
    return;
  }
  const int w = threadIdx.x >> 6;
  const int64_t wave = (int64_t)role.index * 4 + w;
  if (wave >= dp.num_waves) return;
  // Each decode wavefront gets one of the four prefill buffers.
  lds_u8* mine = (lds_u8*)(w == 0 ? k0 : w == 1 ? k1 : w == 2 ? v0 : v1);
  decode_wave<T>(dp, (int)wave, mine);
}

static_assert(kDecodeWaveLdsBytes <= kPrefillTileBytes, "a decode wave's buffers must fit one prefill buffer");

}  // namespace

int fill_prefill_params(PrefillParams& p, const void* q, int64_t q_token_stride, int64_t q_head_stride,
                        const void* k_cache, const void* v_cache, int64_t num_pages, int64_t page_stride,
                        int64_t token_stride, const int32_t* block_tables, int64_t block_table_stride,
                        const int32_t* seq_lens, const int32_t* query_start_loc, const int32_t* items,
                        int64_t num_items, void* out, int64_t out_token_stride, int64_t out_head_stride,
                        int num_q_heads, int num_kv_heads, int head_dim, int page_size, float softmax_scale) {
  if (head_dim != kHeadDim) return set_error("paged attention: head_dim must be 128");
  if (page_size != kPageSize) return set_error("paged attention: page_size must be 16");
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads)
    return set_error("paged attention: num_q_heads must be a positive multiple of num_kv_heads");
  const int group = num_q_heads / num_kv_heads;
  if (group > 16) return set_error("paged attention: at most 16 query heads per KV head");
  if (num_items < 0 || num_items * num_kv_heads > 0x7fffffffLL) return set_error("paged attention: invalid item count");
  if (num_pages <= 0) return set_error("paged attention: empty KV cache");
  const uint64_t align_bits = (uint64_t)(uintptr_t)q | (uint64_t)(uintptr_t)k_cache |
                              (uint64_t)(uintptr_t)v_cache | (uint64_t)(q_token_stride * 2) |
                              (uint64_t)(q_head_stride * 2) | (uint64_t)(page_stride * 2) |
                              (uint64_t)(token_stride * 2);
  if (align_bits % 16) return set_error("paged attention: q / cache buffers and strides must be 16-byte aligned");
  if (((uint64_t)(uintptr_t)out | (uint64_t)(out_token_stride * 2) | (uint64_t)(out_head_stride * 2)) % 8)
    return set_error("paged attention: output buffer and strides must be 8-byte aligned");
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
  p.query_start_loc = query_start_loc;
  p.items = items;
  p.num_items = (int)num_items;
  p.out = out;
  p.out_tok_stride = out_token_stride;
  p.out_head_stride = out_head_stride;
  p.num_kv_heads = num_kv_heads;
  p.group = group;
  p.tile_tokens = kPrefillRows / group;
  p.scale_log2 = softmax_scale * 1.4426950408889634f;
  return 0;
}

}  // namespace mva

extern "C" int mva_prefill_tile_tokens(int num_q_heads, int num_kv_heads) {
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads) return -1;
  return mva::kPrefillRows / (num_q_heads / num_kv_heads);
}

extern "C" int mva_paged_prefill(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                                 const void* k_cache, const void* v_cache, int64_t num_pages,
                                 int64_t page_stride, int64_t token_stride, const int32_t* block_tables,
                                 int64_t block_table_stride, const int32_t* seq_lens,
                                 const int32_t* query_start_loc, const int32_t* items, int64_t num_items,
                                 void* out, int64_t out_token_stride, int64_t out_head_stride,
                                 int num_q_heads, int num_kv_heads, int head_dim, int page_size,
                                 float softmax_scale, int dtype, void* stream) {
  using namespace mva;
  PrefillParams p;
  int rc = fill_prefill_params(p, q, q_token_stride, q_head_stride, k_cache, v_cache, num_pages, page_stride,
                               token_stride, block_tables, block_table_stride, seq_lens, query_start_loc,
                               items, num_items, out, out_token_stride, out_head_stride, num_q_heads,
                               num_kv_heads, head_dim, page_size, softmax_scale);
  if (rc) return rc;
  if (num_items == 0) return 0;
  const dim3 grid((uint32_t)(num_items * num_kv_heads));
  hipStream_t s = (hipStream_t)stream;
  if (dtype == kBF16) hipLaunchKernelGGL(paged_prefill_kernel<__bf16>, grid, dim3(256), 0, s, p);
  else if (dtype == kF16) hipLaunchKernelGGL(paged_prefill_kernel<_Float16>, grid, dim3(256), 0, s, p);
  else return set_error("paged attention: dtype must be bf16 or fp16");
  return check_launch("paged_prefill");
}

extern "C" int mva_paged_mixed(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                               const void* k_cache, const void* v_cache, int64_t num_pages,
                               int64_t page_stride, int64_t token_stride, const int32_t* block_tables,
                               int64_t block_table_stride, const int32_t* seq_lens,
                               const int32_t* query_start_loc, const int32_t* prefill_items,
                               int64_t num_prefill_items, const int32_t* decode_items,
                               int64_t num_decode_items, int64_t num_decode_waves,
                               const int32_t* decode_merges, int64_t num_decode_merges, int64_t num_part_slots,
                               void* out, int64_t out_token_stride, int64_t out_head_stride,
                               void* workspace, int64_t workspace_bytes, int num_q_heads,
                               int num_kv_heads, int head_dim, int page_size, float softmax_scale,
                               int dtype, void* stream) {
  using namespace mva;
  PrefillParams pp;
  int rc = fill_prefill_params(pp, q, q_token_stride, q_head_stride, k_cache, v_cache, num_pages, page_stride,
                               token_stride, block_tables, block_table_stride, seq_lens, query_start_loc,
                               prefill_items, num_prefill_items, out, out_token_stride, out_head_stride,
                               num_q_heads, num_kv_heads, head_dim, page_size, softmax_scale);
  if (rc) return rc;
  DecodeParams dp;
  rc = fill_decode_params(dp, q, q_token_stride, q_head_stride, k_cache, v_cache, num_pages, page_stride,
                          token_stride, block_tables, block_table_stride, seq_lens, decode_items,
                          num_decode_items, num_decode_waves, nullptr, decode_merges, num_decode_merges, num_part_slots,
                          out,
                          out_token_stride, out_head_stride,
                          workspace, workspace_bytes, num_q_heads, num_kv_heads, head_dim, page_size,
                          softmax_scale);
  if (rc) return rc;
  const int64_t n_prefill_wgs = num_prefill_items * num_kv_heads;
  const int64_t n_decode_wgs = num_decode_items > 0 ? (num_decode_waves + 3) / 4 : 0;
  if (n_prefill_wgs + n_decode_wgs > 0x7fffff00LL) return set_error("paged attention: too many work items");
  if (n_prefill_wgs + n_decode_wgs == 0) return 0;
  const uint32_t np = (uint32_t)n_prefill_wgs, nd = (uint32_t)n_decode_wgs;
  const dim3 grid(8u * (mixed_chunks(np) + mixed_chunks(nd)));
  hipStream_t s = (hipStream_t)stream;
  if (dtype == kBF16)
    hipLaunchKernelGGL(paged_mixed_kernel<__bf16>, grid, dim3(256), 0, s, pp, dp, np, nd);
  else if (dtype == kF16)
    hipLaunchKernelGGL(paged_mixed_kernel<_Float16>, grid, dim3(256), 0, s, pp, dp, np, nd);
  else return set_error("paged attention: dtype must be bf16 or fp16");
  rc = check_launch("paged_mixed");
  if (rc) return rc;
  return launch_decode_merge(dp, decode_merges, num_decode_merges, dtype, s);
}
