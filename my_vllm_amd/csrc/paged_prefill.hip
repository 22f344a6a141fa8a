// C-ABI entry points of the ragged causal prefill kernel and of the
// single-launch MIXED kernel (prefill tiles + decode items in one grid).
#include "mva_capi.h"
#include "paged_prefill.h"
#include "paged_prefill_pingpong.h"

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
int32_t* decode_arrival_counters(void* workspace);

namespace {

// Exact tile list of a prefill batch, built on the device from
// query_start_loc / seq_lens (one workgroup; see kPrefillPlanHeaderInts for
// the format).  Sequences are ordered longest context first (batches of up
// to kPrefillPlanSortMax sequences; larger batches keep batch order), and a
// sequence's tiles largest key count first, so the tiles that read one
// sequence's pages run together and long work starts early.  The last
// `tail` tiles (at most 1024) are then reordered by key count, largest
// first (ties keep their order): they are the work the persistent grid
// drains last, and without it a long tile of the last sequences could start
// after the workgroups of its head had run out of work.  A sequence with no
// queries, or with more queries than keys, gets no tile.  At most
// `capacity` tiles are written; word 0 receives their number and word 1
// the number left out.
__global__ __launch_bounds__(1024) void prefill_plan_kernel(const int32_t* __restrict__ qsl,
                                                            const int32_t* __restrict__ seq_lens,
                                                            const int32_t* __restrict__ block_tables,
                                                            int64_t bt_stride, int64_t num_pages, int num_seqs,
                                                            int tile_tokens, int num_kv_heads,
                                                            int32_t* __restrict__ plan, int capacity, int tail,
                                                            int grid) {
  // Sequences in plan order (rank -> sequence) and the first tile of each
  // rank; beyond kPrefillPlanSortMax sequences, all keep batch order and are
  // planned in passes of kPrefillPlanSortMax.
  __shared__ int kv_of[kPrefillPlanSortMax];
  __shared__ int order[kPrefillPlanSortMax];
  __shared__ int first_tile[kPrefillPlanSortMax + 1];
  __shared__ int scan[1024];
  __shared__ int carry;
  const int tid = threadIdx.x;
  const bool sorted = num_seqs <= kPrefillPlanSortMax;
  if (tid == 0) carry = 0;
  if (sorted) {
    for (int s = tid; s < num_seqs; s += 1024) kv_of[s] = seq_lens[s];
    __syncthreads();
    for (int s = tid; s < num_seqs; s += 1024) {
      const int mine = kv_of[s];
      int rank = 0;
      for (int o = 0; o < num_seqs; ++o) {
        const int v = kv_of[o];
        rank += (v > mine) || (v == mine && o < s);
      }
      order[rank] = s;
    }
  }
  __syncthreads();
  int32_t* out = plan + kPrefillPlanHeaderInts;
  for (int c = 0; c < num_seqs; c += kPrefillPlanSortMax) {
    const int span = min(kPrefillPlanSortMax, num_seqs - c);
    // Tiles per rank in this pass over the sequences, then their exclusive
    // prefix sum.
    for (int r0 = 0; r0 < span; r0 += 1024) {
      const int r = r0 + tid;
      int nt = 0;
      if (r < span) {
        const int s = sorted ? order[r] : c + r;
        const int q_len = qsl[s + 1] - qsl[s];
        const int kv = seq_lens[s];
        if (q_len > 0 && kv >= q_len) nt = (q_len + tile_tokens - 1) / tile_tokens;
      }
      scan[tid] = nt;
      __syncthreads();
      for (int off = 1; off < 1024; off <<= 1) {
        const int add = tid >= off ? scan[tid - off] : 0;
        __syncthreads();
        scan[tid] += add;
        __syncthreads();
      }
      if (r < span) first_tile[r] = carry + scan[tid] - nt;
      __syncthreads();
      if (tid == 0) carry += scan[1023];
      __syncthreads();
    }
    if (tid == 0) first_tile[span] = carry;
    __syncthreads();
    // One tile per thread: find its rank by binary search, write its record.
    const int lo_tile = first_tile[0], hi_tile = first_tile[span];
    for (int i = lo_tile + tid; i < hi_tile && i < capacity; i += 1024) {
      int lo = 0, hi = span - 1;  // last rank whose first tile is <= i
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (first_tile[mid] <= i) lo = mid;
        else hi = mid - 1;
      }
      const int s = sorted ? order[lo] : c + lo;
      const int q0 = qsl[s];
      const int q_len = qsl[s + 1] - q0;
      const int kv = seq_lens[s];
      const int nt = (q_len + tile_tokens - 1) / tile_tokens;
      const int jt = i - first_tile[lo];
      const int t0 = (nt - 1 - jt) * tile_tokens;  // largest key count first
      const int bpos = kv - q_len;
      const int kv_end = bpos + min(t0 + tile_tokens, q_len);
      const int ntiles = (kv_end + kPrefillKeys - 1) / kPrefillKeys;
      const int full = min((bpos + t0 + 1) / kPrefillKeys, ntiles);
      const int npages = (kv_end + kPageSize - 1) / kPageSize;
      const int32_t* bt = block_tables + (int64_t)s * bt_stride;
      int pg[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int v = bt[min(k, npages - 1)];
        pg[k] = (v >= 0 && v < num_pages) ? v : 0;
      }
      int32_t* d = out + (int64_t)i * kPrefillPlanItemInts;
      *reinterpret_cast<int4*>(d) = int4{s, t0, q0, q_len};
      *reinterpret_cast<int4*>(d + 4) = int4{kv, ntiles, full, npages};
      *reinterpret_cast<int4*>(d + 8) = int4{pg[0], pg[1], pg[2], pg[3]};
      *reinterpret_cast<int4*>(d + 12) = int4{pg[4], pg[5], pg[6], pg[7]};
    }
    __syncthreads();
  }
  {
    // The tail: thread i holds tile base + i, ranks it among the tail by key
    // count (stable) and writes it to its rank.  Every thread has read its
    // record (the barrier waits for the loads) before any is written.
    const int n = min(carry, capacity);
    const int K = min(min(n, tail), 1024);
    if (K > 1) {
      const int base = n - K;
      int4 r0, r1, r2, r3;
      int key = -1;
      if (tid < K) {
        const int4* src = reinterpret_cast<const int4*>(out + (int64_t)(base + tid) * kPrefillPlanItemInts);
        r0 = src[0];
        r1 = src[1];
        r2 = src[2];
        r3 = src[3];
        key = r1.y;  // ntiles
      }
      scan[tid] = key;
      __syncthreads();
      if (tid < K) {
        int rank = 0;
        for (int o = 0; o < K; ++o) {
          const int v = scan[o];
          rank += (v > key) || (v == key && o < tid);
        }
        int4* dst = reinterpret_cast<int4*>(out + (int64_t)(base + rank) * kPrefillPlanItemInts);
        dst[0] = r0;
        dst[1] = r1;
        dst[2] = r2;
        dst[3] = r3;
      }
    }
  }
  if (tid == 0) {
    plan[0] = min(carry, capacity);
    plan[kPrefillPlanDroppedInt] = max(carry - capacity, 0);
    plan[kPrefillPlanExitInt] = 0;
    plan[kPrefillPlanGridInt] = grid;
  }
  if (tid < num_kv_heads) plan[kPrefillPlanLineInts * (1 + tid)] = 0;  // claim counters
}

// Persistent prefill: workgroup b serves KV head b % num_kv_heads (so head
// h stays on XCD h when the head count divides 8).  The workgroups of a head
// take tiles of the plan in order from that head's claim counter, one claim
// ahead (prefill_items_pingpong), so the grid never waits on dispatch and
// faster CUs simply run more tiles; once their head's queue is exhausted
// they take the remaining tiles of the other heads.
template <typename T>
__global__ __launch_bounds__(kPrefillPPThreads) void paged_prefill_stream_kernel(PrefillParams p,
                                                                                 int32_t* __restrict__ plan) {
  __shared__ __attribute__((aligned(16))) uint8_t tiles[kPrefillPPLdsBytes];
  __shared__ int nextq[4];
  const int h = (int)(blockIdx.x % (uint32_t)p.num_kv_heads);
  if (__builtin_amdgcn_readfirstlane((int)threadIdx.x >> 8) == 0)
    prefill_items_pingpong<T, 0>(p, plan, h, (lds_u8*)tiles, (lds_i32*)nextq);
  else
    prefill_items_pingpong<T, 1>(p, plan, h, (lds_u8*)tiles, (lds_i32*)nextq);
  // The last workgroup out zeroes the claim counters and the exit count, so
  // the plan serves the next launch as it is.  Every claim and counter read
  // of a workgroup has returned (its result decided the exit) before thread 0
  // counts the workgroup out, and workgroups of any head claim from every
  // head's counter, so only the grid's last exit may clear them.
  // (The grid size comes from the plan header, which keeps the dispatch
  // packet's registers out of the tile loop.)
  __syncthreads();
  if (threadIdx.x < 64) {
    int gone = 0;
    if (threadIdx.x == 0)
      gone = __hip_atomic_fetch_add(plan + kPrefillPlanExitInt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    gone = __builtin_amdgcn_readfirstlane(gone);
    if (gone == plan[kPrefillPlanGridInt] - 1) {
      for (int hh = threadIdx.x; hh < kPrefillPlanMaxHeads; hh += 64)
        __hip_atomic_store(plan + kPrefillPlanLineInts * (1 + hh), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (threadIdx.x == 0) __hip_atomic_store(plan + kPrefillPlanExitInt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

int device_cu_count() {
  static int counts[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (counts[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    counts[dev] = cus;
  }
  return counts[dev];
}

// Workgroup roles of the MIXED launch: the decode workgroups come first, in
// chunks of 8 blocks (blocks are dealt to the 8 XCDs round-robin), then the
// prefill workgroups.  The host sizes the decode part below the GPU's
// resident capacity, so every decode wavefront starts at once and prefill
// workgroups fill the remaining slots (and the slots decode frees): HBM-bound
// decode streaming overlaps MFMA-bound prefill on the same CUs.  Prefill
// blocks keep index % 8 == block % 8, so prefill workgroup i, which serves
// KV head i % num_kv_heads, runs on the XCD that serves that head in the
// prefill-only launch.
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

// Prefill sequences a MIXED launch orders in LDS.
constexpr int kMixedPrefillSeqsMax = 1024;

// The prefill workgroups of a MIXED launch are a persistent pool of
// `per_head` workgroups per KV head.  Each builds the launch's query-tile
// order in LDS from query_start_loc / seq_lens of the leading p.num_seqs
// sequences -- sequences longest context first (ties by index), a
// sequence's 128-row tiles largest key count first, as the PREFILL planner
// orders them -- then takes tiles from its head's claim counter until none
// are left.  So every tile run is a real tile, and no query count is needed
// on the host.  A workgroup claims its next tile when its current one ends:
// with about two tiles per workgroup, claiming one ahead would reserve
// nearly every tile at the start and undo the balancing (measured 11%
// slower on the prefill half of a budget-8192 batch).  A sequence with no queries, or more
// queries than keys, has no tile.  The last workgroup of a head to leave
// clears that head's counters for the next launch.
template <typename T>
__device__ void mixed_prefill_pool(const PrefillParams& p, int32_t* sched, uint32_t index, uint32_t per_head,
                                   int* order, int* first_tile, int* claimed, lds_u8* k0, lds_u8* k1, lds_u8* v0,
                                   lds_u8* v1) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int S = p.num_seqs;
  const int BMT = p.tile_tokens;
  const int h = (int)(index % (uint32_t)p.num_kv_heads);
  int* const ctr = sched + kMixedPrefillCtrInt + h * kDecodeSchedLineInts;
  if (tid == 0) *claimed = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // Tile order.  The K/V tile buffers are free until the first tile: k0
  // holds the context lengths, k1 the tile counts by rank.
  int* const kv_of = (int*)k0;
  int* const tiles_of = (int*)k1;
  for (int s = tid; s < S; s += 256) kv_of[s] = p.seq_lens[s];
  __syncthreads();
  for (int s = tid; s < S; s += 256) {
    const int mine = kv_of[s];
    int rank = 0;
    for (int o = 0; o < S; ++o) {
      const int v = kv_of[o];
      rank += (v > mine) || (v == mine && o < s);
    }
    order[rank] = s;
  }
  __syncthreads();
  for (int r = tid; r < S; r += 256) {
    const int s = order[r];
    const int q_len = p.query_start_loc[s + 1] - p.query_start_loc[s];
    const int kv = kv_of[s];
    tiles_of[r] = (q_len > 0 && kv >= q_len) ? (q_len + BMT - 1) / BMT : 0;
  }
  __syncthreads();
  if (tid < 64) {
    // Exclusive prefix sum over ranks, 64 at a time, by wave 0.
    int carry = 0;
    for (int c = 0; c < S; c += 64) {
      const int v = c + lane < S ? tiles_of[c + lane] : 0;
      int incl = v;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int up = __shfl_up(incl, off);
        if (lane >= off) incl += up;
      }
      if (c + lane < S) first_tile[c + lane] = carry + incl - v;
      carry += __shfl(incl, 63);
    }
    if (lane == 0) first_tile[S] = carry;
  }
  __syncthreads();
  const int total = __builtin_amdgcn_readfirstlane(first_tile[S]);

  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  int idx = __builtin_amdgcn_readfirstlane(*claimed);
  while (idx < total) {
    // Rank of tile idx: the last rank whose first tile is <= idx.
    int lo = 0, hi = S - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (first_tile[mid] <= idx) lo = mid;
      else hi = mid - 1;
    }
    lo = __builtin_amdgcn_readfirstlane(lo);
    PrefillWork wk;
    wk.s = __builtin_amdgcn_readfirstlane(order[lo]);
    wk.q0 = sload(p.query_start_loc, wk.s);
    wk.q_len = sload(p.query_start_loc, wk.s + 1) - wk.q0;
    wk.kv = sload(p.seq_lens, wk.s);
    const int nt = (wk.q_len + BMT - 1) / BMT;
    wk.t0 = (nt - 1 - (idx - __builtin_amdgcn_readfirstlane(first_tile[lo]))) * BMT;  // largest key count first
    const int base_pos = wk.kv - wk.q_len;
    const int kv_end = base_pos + min(wk.t0 + BMT, wk.q_len);  // keys [0, kv_end) are needed
    wk.ntiles = (kv_end + kPrefillKeys - 1) / kPrefillKeys;
    wk.full_tiles = min((base_pos + wk.t0 + 1) / kPrefillKeys, wk.ntiles);
    wk.npages = (kv_end + kPageSize - 1) / kPageSize;
    const int32_t* bt = p.block_tables + (int64_t)wk.s * p.bt_stride;
    auto page = [&](int i) {
      const int pg = sload(bt, min(i, wk.npages - 1));
      return (pg >= 0 && pg < p.num_pages) ? pg : 0;
    };
    wk.pg0 = page(w);
    wk.pg1 = page(kPrefillKeys / kPageSize + w);
    prefill_core<T>(p, wk, h, k0, k1, v0, v1);
    __syncthreads();  // every wave is done with this tile's LDS before `claimed` changes
    if (tid == 0) *claimed = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    idx = __builtin_amdgcn_readfirstlane(*claimed);
  }
  if (tid == 0) {
    // Every claim of this workgroup has returned (the last one ended the
    // loop), so all claims on the counter precede the clear.
    const int gone =
        __hip_atomic_fetch_add(ctr + kMixedPrefillExitOffset, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (gone == (int)per_head - 1) {
      __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(ctr + kMixedPrefillExitOffset, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// Prefill workgroups run the prefill pool; decode workgroups run four
// decode wavefronts each, with private LDS buffers.
template <typename T>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void paged_mixed_kernel(
    PrefillParams pp, DecodeParams dp, uint32_t n_prefill_wgs, uint32_t n_decode_wgs) {
  __shared__ __attribute__((aligned(16))) uint8_t k0[kPrefillTileBytes];
  __shared__ __attribute__((aligned(16))) uint8_t k1[kPrefillTileBytes];
  __shared__ __attribute__((aligned(16))) uint8_t v0[kPrefillTileBytes];
  __shared__ __attribute__((aligned(16))) uint8_t v1[kPrefillTileBytes];
  __shared__ int order[kMixedPrefillSeqsMax];
  __shared__ int first_tile[kMixedPrefillSeqsMax + 1];
  __shared__ int claimed;
  const MixedRole role = mixed_role(blockIdx.x, n_decode_wgs);
  if (role.prefill) {
    if (role.index >= n_prefill_wgs) return;
    mixed_prefill_pool<T>(pp, dp.sched, role.index, n_prefill_wgs / (uint32_t)pp.num_kv_heads, order, first_tile,
                          &claimed, (lds_u8*)k0, (lds_u8*)k1, (lds_u8*)v0, (lds_u8*)v1);
    return;
  }
  const int w = threadIdx.x >> 6;
  const int64_t wave = (int64_t)role.index * 4 + w;
  if (wave >= dp.num_waves) return;
  // Each decode wavefront gets one of the four prefill buffers.
  lds_u8* mine = (lds_u8*)(w == 0 ? k0 : w == 1 ? k1 : w == 2 ? v0 : v1);
  decode_wave<T, true>(dp, (int)wave, mine);
}

static_assert(kMixedPrefillSeqsMax * 4 <= kPrefillTileBytes, "context lengths fit one K/V tile buffer");
static_assert(kDecodeWaveLdsBytes <= kPrefillTileBytes, "a decode wave's buffers must fit one prefill buffer");

}  // namespace

int fill_prefill_params(PrefillParams& p, const void* q, int64_t q_token_stride, int64_t q_head_stride,
                        const void* k_cache, const void* v_cache, int64_t num_pages, int64_t page_stride,
                        int64_t token_stride, const int32_t* block_tables, int64_t block_table_stride,
                        const int32_t* seq_lens, const int32_t* query_start_loc, int64_t num_seqs,
                        void* out, int64_t out_token_stride, int64_t out_head_stride,
                        int num_q_heads, int num_kv_heads, int head_dim, int page_size, float softmax_scale) {
  if (head_dim != kHeadDim) return set_error("paged attention: head_dim must be 128");
  if (page_size != kPageSize) return set_error("paged attention: page_size must be 16");
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads)
    return set_error("paged attention: num_q_heads must be a positive multiple of num_kv_heads");
  const int group = num_q_heads / num_kv_heads;
  if (group > 16) return set_error("paged attention: at most 16 query heads per KV head");
  if (num_seqs < 0 || num_seqs > 0x7fffffffLL) return set_error("paged attention: invalid sequence count");
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
  p.num_seqs = (int)num_seqs;
  p.out = out;
  p.out_tok_stride = out_token_stride;
  p.out_head_stride = out_head_stride;
  p.num_kv_heads = num_kv_heads;
  p.group = group;
  p.tile_tokens = kPrefillRows / group;
  p.scale_log2 = softmax_scale * 1.4426950408889634f;
  p.out16 = ((uint64_t)(uintptr_t)out | (uint64_t)(out_token_stride * 2) | (uint64_t)(out_head_stride * 2)) % 16 == 0;
  return 0;
}

}  // namespace mva

extern "C" int mva_prefill_tile_tokens(int num_q_heads, int num_kv_heads) {
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads) return -1;
  return mva::kPrefillRows / (num_q_heads / num_kv_heads);
}

extern "C" int64_t mva_prefill_workspace_bytes(int64_t max_tiles) {
  if (max_tiles < 0 || max_tiles > 0x7fffffffLL / mva::kPrefillPlanItemInts) return -1;
  return (mva::kPrefillPlanHeaderInts + max_tiles * mva::kPrefillPlanItemInts) * 4;
}

namespace {

// Plans (plan_it) and/or streams (run_it) a prefill batch: the shared body
// of mva_paged_prefill, mva_paged_prefill_plan and mva_paged_prefill_run.
int prefill_launch(const void* q, int64_t q_token_stride, int64_t q_head_stride, const void* k_cache,
                   const void* v_cache, int64_t num_pages, int64_t page_stride, int64_t token_stride,
                   const int32_t* block_tables, int64_t block_table_stride, const int32_t* seq_lens,
                   const int32_t* query_start_loc, int64_t num_seqs, int64_t max_tiles, void* workspace,
                   int64_t workspace_bytes, void* out, int64_t out_token_stride, int64_t out_head_stride,
                   int num_q_heads, int num_kv_heads, int head_dim, int page_size, float softmax_scale, int dtype,
                   void* stream, bool plan_it, bool run_it) {
  using namespace mva;
  PrefillParams p;
  int rc = fill_prefill_params(p, q, q_token_stride, q_head_stride, k_cache, v_cache, num_pages, page_stride,
                               token_stride, block_tables, block_table_stride, seq_lens, query_start_loc,
                               num_seqs, out, out_token_stride, out_head_stride, num_q_heads,
                               num_kv_heads, head_dim, page_size, softmax_scale);
  if (rc) return rc;
  if (dtype != kBF16 && dtype != kF16) return set_error("paged attention: dtype must be bf16 or fp16");
  const int64_t need = mva_prefill_workspace_bytes(max_tiles);
  if (need < 0) return set_error("paged attention: invalid tile capacity");
  if (num_seqs == 0 || max_tiles == 0) return 0;
  if (workspace == nullptr || workspace_bytes < need)
    return set_error("paged attention: prefill workspace too small for max_tiles");
  if (((uintptr_t)workspace) % 16) return set_error("paged attention: prefill workspace must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  int32_t* plan = (int32_t*)workspace;
  if (num_kv_heads > kPrefillPlanMaxHeads) return set_error("paged attention: at most 127 KV heads");
  p.tile_tokens = kPrefillPPRows / p.group;
  // Persistent grid: one workgroup per CU (96 KB of LDS and two waves per
  // SIMD each), a whole number per KV head, never more than the tiles can use.
  int64_t per_head = (int64_t)device_cu_count() / num_kv_heads;
  per_head = per_head < 1 ? 1 : (per_head > max_tiles ? max_tiles : per_head);
  if (plan_it) {
    // The last three tiles per workgroup of a head go largest first.
    const int tail = (int)(3 * per_head < 1024 ? 3 * per_head : 1024);
    hipLaunchKernelGGL(prefill_plan_kernel, dim3(1), dim3(1024), 0, s, query_start_loc, seq_lens, block_tables,
                       block_table_stride, num_pages, (int)num_seqs, p.tile_tokens, num_kv_heads, plan,
                       (int)max_tiles, tail, (int)(per_head * num_kv_heads));
    rc = check_launch("paged_prefill plan");
    if (rc) return rc;
  }
  if (!run_it) return 0;
  const dim3 grid((uint32_t)(per_head * num_kv_heads));
  if (dtype == kBF16)
    hipLaunchKernelGGL(paged_prefill_stream_kernel<__bf16>, grid, dim3(kPrefillPPThreads), 0, s, p, plan);
  else
    hipLaunchKernelGGL(paged_prefill_stream_kernel<_Float16>, grid, dim3(kPrefillPPThreads), 0, s, p, plan);
  return check_launch("paged_prefill");
}

// Stand-ins for the buffers a plan-only launch does not touch: they pass the
// alignment checks and are never dereferenced.
alignas(16) const uint8_t kPlanOnlyDummy[16] = {};

}  // namespace

extern "C" int mva_paged_prefill(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                                 const void* k_cache, const void* v_cache, int64_t num_pages,
                                 int64_t page_stride, int64_t token_stride, const int32_t* block_tables,
                                 int64_t block_table_stride, const int32_t* seq_lens,
                                 const int32_t* query_start_loc, int64_t num_seqs, int64_t max_tiles,
                                 void* workspace, int64_t workspace_bytes, void* out, int64_t out_token_stride,
                                 int64_t out_head_stride, int num_q_heads, int num_kv_heads, int head_dim,
                                 int page_size, float softmax_scale, int dtype, void* stream) {
  return prefill_launch(q, q_token_stride, q_head_stride, k_cache, v_cache, num_pages, page_stride, token_stride,
                        block_tables, block_table_stride, seq_lens, query_start_loc, num_seqs, max_tiles, workspace,
                        workspace_bytes, out, out_token_stride, out_head_stride, num_q_heads, num_kv_heads, head_dim,
                        page_size, softmax_scale, dtype, stream, true, true);
}

extern "C" int mva_paged_prefill_plan(const int32_t* block_tables, int64_t block_table_stride, int64_t num_pages,
                                      const int32_t* seq_lens, const int32_t* query_start_loc, int64_t num_seqs,
                                      int64_t max_tiles, void* workspace, int64_t workspace_bytes,
                                      int num_q_heads, int num_kv_heads, void* stream) {
  const void* d = kPlanOnlyDummy;
  return prefill_launch(d, 0, 0, d, d, num_pages, 0, 0, block_tables, block_table_stride, seq_lens,
                        query_start_loc, num_seqs, max_tiles, workspace, workspace_bytes, (void*)d, 0, 0,
                        num_q_heads, num_kv_heads, mva::kHeadDim, mva::kPageSize, 1.0f, mva::kBF16, stream, true,
                        false);
}

extern "C" int mva_paged_prefill_run(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                                     const void* k_cache, const void* v_cache, int64_t num_pages,
                                     int64_t page_stride, int64_t token_stride, const int32_t* block_tables,
                                     int64_t block_table_stride, const int32_t* seq_lens,
                                     const int32_t* query_start_loc, int64_t num_seqs, int64_t max_tiles,
                                     void* workspace, int64_t workspace_bytes, void* out,
                                     int64_t out_token_stride, int64_t out_head_stride, int num_q_heads,
                                     int num_kv_heads, int head_dim, int page_size, float softmax_scale, int dtype,
                                     void* stream) {
  return prefill_launch(q, q_token_stride, q_head_stride, k_cache, v_cache, num_pages, page_stride, token_stride,
                        block_tables, block_table_stride, seq_lens, query_start_loc, num_seqs, max_tiles, workspace,
                        workspace_bytes, out, out_token_stride, out_head_stride, num_q_heads, num_kv_heads, head_dim,
                        page_size, softmax_scale, dtype, stream, false, true);
}

extern "C" int mva_paged_mixed(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                               const void* k_cache, const void* v_cache, int64_t num_pages,
                               int64_t page_stride, int64_t token_stride, const int32_t* block_tables,
                               int64_t block_table_stride, const int32_t* seq_lens,
                               const int32_t* query_start_loc, int64_t num_prefill_seqs, int64_t max_prefill_tiles,
                               const int32_t* decode_items, int64_t num_decode_items, int64_t num_decode_waves,
                               int64_t num_part_slots, void* out, int64_t out_token_stride, int64_t out_head_stride,
                               void* workspace, int64_t workspace_bytes, int num_q_heads,
                               int num_kv_heads, int head_dim, int page_size, float softmax_scale,
                               int dtype, void* stream) {
  using namespace mva;
  PrefillParams pp;
  int rc = fill_prefill_params(pp, q, q_token_stride, q_head_stride, k_cache, v_cache, num_pages, page_stride,
                               token_stride, block_tables, block_table_stride, seq_lens, query_start_loc,
                               num_prefill_seqs, out, out_token_stride, out_head_stride,
                               num_q_heads, num_kv_heads, head_dim, page_size, softmax_scale);
  if (rc) return rc;
  if (num_prefill_seqs > kMixedPrefillSeqsMax)
    return set_error("paged attention: a MIXED launch takes at most 1024 prefill sequences");
  if (max_prefill_tiles < 0 || max_prefill_tiles > 0x7fffffffLL)
    return set_error("paged attention: invalid prefill tile capacity");
  DecodeParams dp;
  rc = fill_decode_params(dp, q, q_token_stride, q_head_stride, k_cache, v_cache, num_pages, page_stride,
                          token_stride, block_tables, block_table_stride, seq_lens, decode_items,
                          num_decode_items, num_decode_waves, nullptr, nullptr, 0, num_part_slots, out,
                          out_token_stride, out_head_stride,
                          workspace, workspace_bytes, num_q_heads, num_kv_heads, head_dim, page_size,
                          softmax_scale);
  if (rc) return rc;
  // Split-K segments are merged inside the launch by their last piece.
  if (num_part_slots * num_kv_heads > kArrivalCounters)
    return set_error("paged attention: a MIXED launch takes at most 65536 split-K (partial slot, KV head) pairs");
  dp.arrive = decode_arrival_counters(workspace);
  // Prefill pool: two workgroups per CU (the CU's eight wave slots), a whole
  // number per KV head, never more than the tiles can use.
  int64_t per_head = 0;
  if (num_prefill_seqs > 0 && max_prefill_tiles > 0) {
    if (num_kv_heads > kMixedPrefillMaxHeads) return set_error("paged attention: a MIXED launch takes at most 64 KV heads");
    if (workspace == nullptr) return set_error("paged attention: MIXED launches need the decode workspace");
    per_head = 2 * (int64_t)device_cu_count() / num_kv_heads;
    per_head = per_head < 1 ? 1 : (per_head > max_prefill_tiles ? max_prefill_tiles : per_head);
  }
  const int64_t n_prefill_wgs = per_head * num_kv_heads;
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
  return check_launch("paged_mixed");
}
