// Paged GQA decode on gfx950: a persistent grid of wavefronts, each streaming
// an equal share of the batch's (sequence, KV head, page) units.
//
// Replaces FlashInfer's BatchDecodeWithPagedKVCacheWrapper.run on the DECODE
// route of the reference backend (nanovllm/layers/attention_backend.py:995-997)
// and the decode slice of MIXED_SPLIT (:1020-1025).  Math per query head:
//   o = sum_j softmax_j(scale * q . K[j]) V[j]   over j < seq_len,
// with K/V gathered from NHD pages [P, 16, Hkv, D] through block_tables.
//
// Work distribution, two host-chosen schedules over the same pieces
// (sequence, KV head, page range):
//  * piece lists: the host gives every wavefront an equal share of the
//    batch's pages as an ordered list of pieces (its first piece at index
//    `wave`, the rest in a per-wave range of the item array).  Launched as
//    workgroups of Hkv wavefronts, wavefront h of a workgroup streams KV head
//    h of the workgroup's page range, so one CU reads all heads of a page at
//    about the same time and no wavefront waits on a shared counter;
//  * claims: the host cuts every (sequence, KV head) into pieces of a few
//    pages (longest first); about one wavefront per resident wave slot is
//    launched.  Wavefront w starts on piece w and then takes pieces from a
//    device-scope counter, so CUs that get more HBM bandwidth simply process
//    more pieces (per-CU bandwidth on a multi-XCD part is uneven enough that
//    an equal static split of a multi-GB batch waits for the slowest CU).
//    The last wavefront to exit resets the counters for the next launch.
// Either way the next piece is known one piece ahead and its page table and
// queries are loaded while the current piece streams, so its first page is
// in flight before the current piece's epilogue runs.
//
// Inside a wavefront:
//  * The G query heads that share a KV head form the N=16 side of the MFMAs
//    (columns >= G are zero), so every K/V byte read from HBM serves all G
//    heads: S^T[token, g] = K[token, :] . Q[g, :].
//  * A tile is one 16-token page of one KV head (4 KB of K, 4 KB of V).  Both
//    go from HBM straight into LDS with global_load_lds (16 bytes per lane,
//    8 tokens x 128 contiguous bytes per instruction, no registers),
//    double-buffered, so a wavefront never carries pending loads in
//    registers.
//  * S^T (16x16x32 MFMA): A = K fragments read from the swizzled LDS page
//    (lane = token), B = Q held in registers.  PV (16x16x16 MFMA):
//    O^T[d, g] += V^T[d, t] P^T[t, g], A = V^T read with ds_read_b64_tr_b16
//    from the swizzled LDS page; B = P^T is exactly the C layout of S^T, so
//    no shuffle is needed.
//  * Online softmax in the log2 domain, fp32 accumulators, P rounded to the
//    storage type for the PV MFMA; the O rescale is skipped unless the
//    running max grows by more than 8 (log2 units).
//  * A (sequence, KV head) split into several pieces (split-K) gets one fp32
//    partial per piece (o / l, log2-sum-exp); a second, small kernel on the
//    same stream merges the partials of every split (sequence, KV head), one
//    wavefront per query head, so the page stream never waits on a merge.
#pragma once

#include "mva_common.h"

#include <type_traits>

namespace mva {

constexpr int kHeadDim = 128;
constexpr int kPageSize = 16;
// One page of one KV head (K or V) in LDS, and the LDS a decode wavefront
// uses: two buffers of (K page, V page).
constexpr int kDecodePageBytes = kPageSize * kHeadDim * 2;
constexpr int kDecodeWaveLdsBytes = 2 * 2 * kDecodePageBytes;
// int32 fields per decode work item (piece), see make_decode_plan on the host:
// {seq, page_begin, page_end, chunk, n_chunks, part_base, q_row, kv_head}.
constexpr int kDecodeItemInts = 8;

// s_waitcnt immediates (gfx9 encoding: vmcnt bits [3:0] and [15:14], expcnt
// [6:4], lgkmcnt [11:8]); only vmcnt is constrained.
constexpr int waitcnt_vm(int n) { return (n & 0xf) | ((n >> 4) << 14) | (0x7 << 4) | (0xf << 8); }
constexpr int kVmcnt0 = waitcnt_vm(0);

struct DecodeParams {
  const void* q;
  int64_t q_tok_stride;   // elements
  int64_t q_head_stride;  // elements
  const void* k_cache;
  const void* v_cache;
  int64_t num_pages;
  int64_t page_stride;  // elements between pages
  int64_t tok_stride;   // elements between tokens of a page
  const int32_t* block_tables;
  int64_t bt_stride;
  const int32_t* seq_lens;
  const int32_t* items;  // [num_items][8], see kDecodeItemInts
  int num_items;
  int num_waves;  // wavefronts in the launch
  // Piece lists: wavefront w runs piece w, then pieces
  // [wave_extra[w], wave_extra[w + 1]).  nullptr: the claim schedule.
  const int32_t* wave_extra;
  // Fixed-shape (graph) launches: {num_items, num_waves, num_merges} read on
  // the device, each clamped to the launch's capacity (num_items, num_waves
  // and the merge grid then hold capacities).  nullptr: the scalars above.
  const int32_t* counts;
  int32_t* sched;  // claim counters and exit counter, see kDecodeClaimCounters
  // Fused slot_mapping store (piece lists), or k_new == nullptr: before its
  // first page, a wavefront writes the new K/V row of (token q_row, KV head)
  // to cache slot slots[q_row] for every piece of its list that holds the
  // sequence's last page (that piece is the only reader of the row), when
  // the slot is the sequence's last position, and sets
  // store_flags[q_row * Hkv + kv_head].  The launch after it (the merge
  // kernel) writes every row of [0, num_new) with a slot >= 0 whose flag is
  // clear, and clears the flags.
  const void* k_new;
  int64_t kn_tok_stride;
  int64_t kn_head_stride;
  const void* v_new;
  int64_t vn_tok_stride;
  int64_t vn_head_stride;
  const void* slots;
  int slots_int64;
  int num_new;  // rows of k_new / v_new / slots
  int32_t* store_flags;  // [kStoreFlagInts], zero between launches
  void* out;
  int64_t out_tok_stride;
  int64_t out_head_stride;
  float* part_lse;    // [slots][Hkv][G]
  float* part_o;      // [slots][Hkv][G][D]
  // Split-K merges inside the launch (MIXED), or nullptr for the merge
  // kernel: the arrival counter of segment (part_base, KV head) at
  // arrive[part_base * Hkv + kv_head]; the last piece to arrive merges.
  int32_t* arrive;
  int num_kv_heads;
  int group;  // query heads per KV head, 1..16
  float scale_log2;
};

__device__ inline float wave_max16(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}
__device__ inline float wave_sum16(float x) {
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}

// Scalar (SMEM) loads of data that is read-only for the whole launch (work
// lists, page tables, lengths).  The constant address space tells the
// compiler the memory is invariant, so a wave-uniform index becomes an
// s_load whose completion is tracked by lgkmcnt, independent of the page
// DMAs counted by vmcnt.
typedef int32_t i32x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(4))) const int32_t const_i32;
typedef __attribute__((address_space(4))) const i32x8 const_i32x8;

__device__ inline int sload(const int32_t* base, int64_t idx) { return ((const_i32*)base)[idx]; }

// ---- vector-memory operations the compiler does not track -----------------
// Once a store or a returning atomic is outstanding, the compiler's wait
// insertion assumes vector-memory operations may complete out of order and
// waits for all of them (vmcnt(0)) before any later load result is used,
// which would drain the page stream at every piece boundary.  On this GPU
// vector-memory operations report completion in issue order, so the decode
// loop issues its atomics, stores and per-piece loads as inline asm (not
// counted by the compiler) and orders their completion itself.  Every
// operation whose result is read is issued in the same asm statement as the
// wait that retires it (decode_step), so no compiler-generated instruction
// can touch a destination register while the operation is in flight.

// Per-iteration memory work of a decode wavefront, issued as one asm
// statement, in this order:
//   * lane 0: claim = atomic_add(claim_ptr, 1) if `claiming`;
//   * all lanes, if `loading`: the next piece's page-table words
//     (bt0 -> bt_lo, bt1 -> bt_hi) and query fragments (q .. q + 63 -> qv);
//   * if kDma: the 8 DMAs of one page of one KV head (4 to lds_v, 4 to
//     lds_k, 1 KB each), then s_waitcnt vmcnt(8), which retires everything
//     above and the previous page; otherwise s_waitcnt vmcnt(0).
// Page layout in LDS (K at lds_k, V at lds_v, 4 KB each): 16-byte chunk ch
// (of 16 per token) of token t at byte
//   (2 * (ch / 8) + t / 8) * 1024 + (t % 8) * 128 + ((ch % 8) ^ swz(t)) * 16,
// swz(t) = 2 * ((t / 2) % 4) + (t / 8) % 2: each 1 KB block holds 8 tokens x
// 128 contiguous cache bytes, so every DMA reads whole 128-byte lines.  The
// caller's lane addresses src0 (tokens 0-7) and src1 (tokens 8-15) point at
// token lane/8 (+8), chunk (lane%8) ^ swz; DMA i reads src{i%2} + 128*(i/2)
// and fills block i.  The swizzle keeps the K A-operand reads (16 tokens at
// one chunk per 16 lanes) and the V transposed reads (8 tokens x 2 chunks per
// 32 lanes) free of bank conflicts.
// `loading` and `claiming` are wave-uniform.  Outputs not issued keep their previous
// contents (claim: unspecified).
struct DecodeStepIo {
  int claim;
  int bt_lo;
  int bt_hi;
  u32x4 qv[4];
};

template <bool kDma>
__device__ inline void decode_step(DecodeStepIo& io, int loading, int claiming, int* claim_ptr, const int32_t* bt0,
                                   const int32_t* bt1, const void* q, const void* v_src0, const void* v_src1,
                                   const void* k_src0, const void* k_src1, uint32_t lds_v, uint32_t lds_k) {
  uint64_t saved;
  uint32_t m0_saved;
  const int on_c = __builtin_amdgcn_readfirstlane(claiming != 0 ? 1 : 0);
  const int on_y = __builtin_amdgcn_readfirstlane(loading != 0 ? 1 : 0);
  lds_v = __builtin_amdgcn_readfirstlane(lds_v);
  lds_k = __builtin_amdgcn_readfirstlane(lds_k);
  const char* v0 = (const char*)v_src0;
  const char* v1 = (const char*)v_src1;
  const char* k0 = (const char*)k_src0;
  const char* k1 = (const char*)k_src1;
  if constexpr (kDma) {
    asm volatile(
        "s_mov_b64 %[sv], exec\n\t"
        "s_mov_b32 exec_lo, %[onc]\n\t"
        "s_mov_b32 exec_hi, 0\n\t"
        "global_atomic_add %[cl], %[cp], %[one], off sc0\n\t"
        "s_cmp_eq_u32 %[ony], 0\n\t"
        "s_cselect_b64 exec, 0, %[sv]\n\t"
        "global_load_dword %[blo], %[b0], off\n\t"
        "global_load_dword %[bhi], %[b1], off\n\t"
        "global_load_dwordx4 %[q0], %[qp], off\n\t"
        "global_load_dwordx4 %[q1], %[qp], off offset:16\n\t"
        "global_load_dwordx4 %[q2], %[qp], off offset:32\n\t"
        "global_load_dwordx4 %[q3], %[qp], off offset:48\n\t"
        "s_mov_b64 exec, %[sv]\n\t"
        "s_mov_b32 %[m0s], m0\n\t"
        "s_mov_b32 m0, %[lv]\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %[v0], off\n\t"
        "s_add_u32 m0, %[lv], 0x400\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %[v1], off\n\t"
        "s_add_u32 m0, %[lv], 0x800\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %[v2], off\n\t"
        "s_add_u32 m0, %[lv], 0xc00\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %[v3], off\n\t"
        "s_mov_b32 m0, %[lk]\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %[k0], off\n\t"
        "s_add_u32 m0, %[lk], 0x400\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %[k1], off\n\t"
        "s_add_u32 m0, %[lk], 0x800\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %[k2], off\n\t"
        "s_add_u32 m0, %[lk], 0xc00\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %[k3], off\n\t"
        "s_mov_b32 m0, %[m0s]\n\t"
        "s_waitcnt vmcnt(8)"
        : [cl] "=&v"(io.claim), [blo] "+v"(io.bt_lo), [bhi] "+v"(io.bt_hi),
          [q0] "+v"(io.qv[0]), [q1] "+v"(io.qv[1]), [q2] "+v"(io.qv[2]), [q3] "+v"(io.qv[3]), [sv] "=&s"(saved),
          [m0s] "=&s"(m0_saved)
        : [onc] "s"(on_c), [ony] "s"(on_y), [cp] "v"(claim_ptr), [one] "v"(1),
          [b0] "v"(bt0), [b1] "v"(bt1), [qp] "v"(q), [lv] "s"(lds_v), [lk] "s"(lds_k), [v0] "v"(v0),
          [v1] "v"(v1), [v2] "v"(v0 + 128), [v3] "v"(v1 + 128), [k0] "v"(k0), [k1] "v"(k1),
          [k2] "v"(k0 + 128), [k3] "v"(k1 + 128)
        : "memory", "scc");
  } else {
    asm volatile(
        "s_mov_b64 %[sv], exec\n\t"
        "s_mov_b32 exec_lo, %[onc]\n\t"
        "s_mov_b32 exec_hi, 0\n\t"
        "global_atomic_add %[cl], %[cp], %[one], off sc0\n\t"
        "s_cmp_eq_u32 %[ony], 0\n\t"
        "s_cselect_b64 exec, 0, %[sv]\n\t"
        "global_load_dword %[blo], %[b0], off\n\t"
        "global_load_dword %[bhi], %[b1], off\n\t"
        "global_load_dwordx4 %[q0], %[qp], off\n\t"
        "global_load_dwordx4 %[q1], %[qp], off offset:16\n\t"
        "global_load_dwordx4 %[q2], %[qp], off offset:32\n\t"
        "global_load_dwordx4 %[q3], %[qp], off offset:48\n\t"
        "s_mov_b64 exec, %[sv]\n\t"
        "s_waitcnt vmcnt(0)"
        : [cl] "=&v"(io.claim), [blo] "+v"(io.bt_lo), [bhi] "+v"(io.bt_hi),
          [q0] "+v"(io.qv[0]), [q1] "+v"(io.qv[1]), [q2] "+v"(io.qv[2]), [q3] "+v"(io.qv[3]), [sv] "=&s"(saved)
        : [onc] "s"(on_c), [ony] "s"(on_y), [cp] "v"(claim_ptr), [one] "v"(1),
          [b0] "v"(bt0), [b1] "v"(bt1), [qp] "v"(q)
        : "memory", "scc");
  }
}

// Device-scope (write-through) stores, and a plain 8-byte store.  The
// trailing s_nop covers the store-data hazard for multi-dword stores.
__device__ inline void store16_device_untracked(void* addr, u32x4 v) {
  asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1" ::"v"(addr), "v"(v) : "memory");
}
__device__ inline void store4_device_untracked(void* addr, float v) {
  asm volatile("global_store_dword %0, %1, off sc1" ::"v"(addr), "v"(v) : "memory");
}
__device__ inline void store8_untracked(void* addr, u32x2 v) {
  asm volatile("global_store_dwordx2 %0, %1, off\n\ts_nop 1" ::"v"(addr), "v"(v) : "memory");
}

// Piece claim counters: kDecodeClaimCounters counters, each on its own
// 128-byte line (atomics to one line serialize), then the exit counter.
constexpr int kDecodeClaimCounters = 32;
constexpr int kDecodeSchedLineInts = 32;
// (32 + 2 + kMixedPrefillMaxHeads) lines of 128 bytes, rounded up to 256.
constexpr int kMixedPrefillMaxHeads = 64;
constexpr int kDecodeSchedBytes = 12544;
static_assert((kDecodeClaimCounters + 1) * kDecodeSchedLineInts * 4 <= kDecodeSchedBytes, "sched area");
// Word set to 1 by a fused-store launch that found a new row whose slot is
// not in its sequence's last page (the row is not written); on its own line
// after the exit counter.  Only the host clears it.
constexpr int kDecodeStoreErrorInt = (kDecodeClaimCounters + 1) * kDecodeSchedLineInts;
static_assert((kDecodeStoreErrorInt + 1) * 4 <= kDecodeSchedBytes, "store error word");
// MIXED launches: the prefill claim counter of KV head h at word
// kMixedPrefillCtrInt + h * kDecodeSchedLineInts and that head's exit
// counter kMixedPrefillExitOffset words after it; the last prefill
// workgroup of the head to exit clears both.
constexpr int kMixedPrefillCtrInt = (kDecodeClaimCounters + 2) * kDecodeSchedLineInts;
constexpr int kMixedPrefillExitOffset = 16;
static_assert((kMixedPrefillCtrInt + kMixedPrefillMaxHeads * kDecodeSchedLineInts) * 4 <= kDecodeSchedBytes,
              "MIXED prefill counters");
// MIXED launches merge split-K segments themselves: one arrival counter per
// (partial slot, KV head), in a fixed region right after the scheduler area.
// No other kernel writes there, and the last arrival of a segment clears its
// counter, so the counters are zero at every MIXED launch whatever plans
// (and partial layouts) used the workspace in between.
constexpr int kArrivalCounters = 65536;
constexpr int64_t kArrivalBytes = (int64_t)kArrivalCounters * 4;
// Fused-store row flags: one int per (new row, KV head), in a fixed region
// after the arrival counters; a fused launch takes at most this many pairs.
constexpr int kStoreFlagInts = 65536;
constexpr int64_t kStoreFlagBytes = (int64_t)kStoreFlagInts * 4;

template <typename T, bool kAgent>
__device__ void merge_segment(const DecodeParams& p, const i32x8& d, int g);

// One wavefront of a decode launch (`wave` in [0, num_waves)); `lds` is its
// kDecodeWaveLdsBytes of LDS.
//
// Piece order with piece lists: piece w, then wave_extra[w] .. wave_extra[w+1]-1.
// Piece order with claims: wavefront w takes piece w, then piece W + w (W =
// num_waves), then pieces 2W + C*k + j for k drawn from claim counter
// j = (w / 8) mod C, C = min(32, max(1, W / 8)).  Blocks are dealt to the 8 XCDs round-robin,
// so wavefronts of every XCD share each counter and no counter's share of
// the queue waits on one slower XCD.  Three pieces are tracked: X (being computed), Y (its
// successor: descriptor and length known, page table and queries loaded
// during X's first page) and Z (Y's successor, claimed at X's first page;
// its descriptor is fetched right after that page).  The page stream runs
// one page ahead across piece boundaries, so the first page of Y (or of Z,
// when Y is a single page) is in flight while X's last page is computed,
// and a piece boundary costs no wait of its own.  Page ids come from the
// page-table registers (readlane); the loop issues no memory access per
// page other than the page itself.
//
// A split piece stores its partial when it ends; decode_merge_wave combines
// the partials in the kernel that follows on the same stream.
//
// `progress` (LDS, one int per wavefront of an 8-wavefront workgroup, or
// nullptr): wavefronts w and w ^ 4 share a SIMD and stream the same pages for
// two KV heads.  The older of the two wins issue arbitration and would finish
// first; each wavefront publishes its page count and keeps priority 2 unless
// it is ahead of its partner, so the pair stays level.
template <typename T, bool kMergeInLaunch = false>
__device__ void decode_wave(const DecodeParams& p, int wave, lds_u8* lds, int* progress = nullptr) {
  typedef typename Elem<T>::v8 V8;
  typedef typename Elem<T>::v4 V4;
  const int lane = threadIdx.x & 63;
  const int q4 = lane >> 4;
  const int c = lane & 15;
  const int G = p.group;
  const int Hkv = p.num_kv_heads;
  // Graph launches read this step's counts; wavefronts past them have no work.
  const int W = p.counts ? min(sload(p.counts, 1), p.num_waves) : p.num_waves;
  const int N = p.counts ? min(sload(p.counts, 0), p.num_items) : p.num_items;
  if (wave >= W || wave >= N) return;
  const int C = min(kDecodeClaimCounters, max(1, W >> 3));
  const int jc = (wave >> 3) % C;
  const bool q_lane = c < G;
  int* const claim_ctr = p.sched + jc * kDecodeSchedLineInts;

  // Descriptor fields: {seq, page_begin, page_end, chunk, n_chunks, part_base, q_row, kv_head}.
  auto desc_at = [&](int idx) -> i32x8 { return ((const_i32x8*)p.items)[idx]; };
  // Page table of piece d (at most 128 pages): lane L of lo/hi holds page L
  // and 64 + L; bt_word gives the clamped address of word k.
  auto bt_word = [&](const i32x8& d, int k) -> const int32_t* {
    return p.block_tables + (int64_t)d[0] * p.bt_stride + d[1] + min(k, d[2] - d[1] - 1);
  };
  auto page_of = [&](int lo, int hi, int k) -> int {
    const int a = __builtin_amdgcn_readlane(lo, k & 63);
    const int b = __builtin_amdgcn_readlane(hi, k & 63);
    const int pg = k < 64 ? a : b;
    return (pg >= 0 && pg < p.num_pages) ? pg : 0;
  };
  // Query fragments of piece d, the B operand of S^T = K Q^T: lane (q4, c)
  // holds Q[g = c][32*q4 + 8*j .. +8].  Lanes c >= G read head 0 of the
  // group (in bounds) and are zeroed where the fragments are used.
  auto q_addr = [&](const i32x8& d) -> const T* {
    const int g = q_lane ? c : 0;
    return (const T*)p.q + (int64_t)d[6] * p.q_tok_stride + (int64_t)(d[7] * G + g) * p.q_head_stride + 32 * q4;
  };

  // ---- piece state --------------------------------------------------------
  i32x8 X = desc_at(wave);
  int xi = wave;  // X's index in the piece array
  // Piece lists: nx is the next unassigned entry of this wavefront's range
  // [nx, nx_end).
  const bool listed = p.wave_extra != nullptr;
  int nx = N, nx_end = N;
  int yi = wave + W;  // >= N: none
  if (listed) {
    // Clamped to the item array, so a malformed list cannot index past it.
    nx = max(sload(p.wave_extra, wave), 0);
    nx_end = min(sload(p.wave_extra, wave + 1), N);
    yi = nx < nx_end ? nx : N;
    ++nx;
  }
  int zi = N;
  i32x8 Y = X, Z = X;
  if (yi < N) Y = desc_at(yi);
  int seq_len = sload(p.seq_lens, X[0]);
  int y_len = sload(p.seq_lens, Y[0]);
  int z_len = 0;
  int np = X[2] - X[1];
  // X's page table and queries; the first DMA needs the table, so this is
  // the one wait of the wavefront outside the page loop.
  int bt_lo = *bt_word(X, lane), bt_hi = *bt_word(X, 64 + lane);
  u32x4 qf[4];
  {
    const T* qp = q_addr(X);
#pragma unroll
    for (int j = 0; j < 4; ++j) qf[j] = ld16<u32x4>(qp + 8 * j);
  }
  // Fused store: the new token's K and V rows (256 bytes each, 4 per lane)
  // of every listed piece that reads its sequence's last page, loaded while
  // the page table and queries are in flight and written before any page
  // is read (the wait below also retires the stores).
  if (listed && p.k_new) {
    const int first = max(sload(p.wave_extra, wave), 0);
    const int count = min(sload(p.wave_extra, wave + 1), N) - first;
    for (int k = -1; k < count; ++k) {
      const i32x8 d = k < 0 ? X : desc_at(first + k);
      const int len = sload(p.seq_lens, d[0]);
      if (d[6] < 0 || d[6] >= p.num_new || len <= 0 || d[1] * kPageSize >= len || d[2] * kPageSize < len) continue;
      const int64_t slot = p.slots_int64 ? ((const int64_t*)p.slots)[d[6]] : ((const int32_t*)p.slots)[d[6]];
      if (slot < 0) continue;  // -1: nothing to store
      // The row must be the sequence's last position, in the last page,
      // which this piece alone reads; a slot anywhere else could be in a
      // page another wavefront is streaming.  Such a row is left to the
      // merge kernel that follows (it writes every unflagged row), and the
      // launch records it in the workspace's store-error word.
      const int last_page = sload(p.block_tables, (int64_t)d[0] * p.bt_stride + (len - 1) / kPageSize);
      if (slot != (int64_t)last_page * kPageSize + (len - 1) % kPageSize || last_page < 0 ||
          last_page >= p.num_pages) {
        if (lane == 0) *(volatile int32_t*)(p.sched + kDecodeStoreErrorInt) = 1;
        continue;
      }
      const int64_t dst = (slot / kPageSize) * p.page_stride + (slot % kPageSize) * p.tok_stride +
                          (int64_t)d[7] * kHeadDim + 2 * lane;
      const uint32_t kv = *(const uint32_t*)((const T*)p.k_new + (int64_t)d[6] * p.kn_tok_stride +
                                            (int64_t)d[7] * p.kn_head_stride + 2 * lane);
      const uint32_t vv = *(const uint32_t*)((const T*)p.v_new + (int64_t)d[6] * p.vn_tok_stride +
                                            (int64_t)d[7] * p.vn_head_stride + 2 * lane);
      *(uint32_t*)((T*)const_cast<void*>(p.k_cache) + dst) = kv;
      *(uint32_t*)((T*)const_cast<void*>(p.v_cache) + dst) = vv;
      if (lane == 0) p.store_flags[(int64_t)d[6] * p.num_kv_heads + d[7]] = 1;
    }
  }
  __builtin_amdgcn_s_waitcnt(kVmcnt0);
  DecodeStepIo io;
  io.bt_lo = io.bt_hi = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) io.qv[j] = u32x4{0u, 0u, 0u, 0u};


  f32x4 o[8];  // o[mt][r] = O^T[d = 16*mt + 4*q4 + r][g = c]
#pragma unroll
  for (int mt = 0; mt < 8; ++mt) o[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY;  // reference max of scaled scores (log2 domain), per g = c
  float l = 0.f;        // this lane's share of the running denominator

  // Per-lane addresses in the page layout of decode_step: the DMA sources
  // (token lane/8, and 8 + lane/8, at chunk (lane%8) ^ swz), the K fragment
  // of step j (token c, chunk 4*q4 + j) and the transposed V read: lane c of
  // group q4 supplies token 4*q4 + c/4 at d 16*mt + 4*(c%4) (chunk
  // 2*mt + (c%4)/2, byte 8*(c%2) inside it) and receives V[4*q4 + e][16*mt + c],
  // e = 0..3; d-tiles mt and mt + 4 differ by 2 KB.
  auto swz = [](int t) { return (2 * ((t >> 1) & 3)) | ((t >> 3) & 1); };
  const int64_t src0_off = (int64_t)(lane >> 3) * p.tok_stride + 8 * ((lane & 7) ^ swz(lane >> 3));
  const int64_t src1_off = (int64_t)(8 + (lane >> 3)) * p.tok_stride + 8 * ((lane & 7) ^ swz(8 + (lane >> 3)));
  int koff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    koff[j] = (2 * (q4 >> 1) + (c >> 3)) * 1024 + (c & 7) * 128 + (((4 * (q4 & 1) + j) ^ swz(c)) * 16);
  const int vtok = 4 * q4 + (c >> 2);
  int voff[4];
#pragma unroll
  for (int m = 0; m < 4; ++m)
    voff[m] = kDecodePageBytes + (vtok >> 3) * 1024 + (vtok & 7) * 128 +
              (((2 * m + ((c >> 1) & 1)) ^ swz(vtok)) * 16) + (c & 1) * 8;

  // `edge` pages contain tokens past seq_len; the choice is wave-uniform.
  auto compute = [&](int pg, const lds_u8* buf, auto edge_tag) __attribute__((always_inline)) {
    constexpr bool edge = decltype(edge_tag)::value;
    f32x4 sc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j)
      sc = Elem<T>::mfma16(lds_ld16<V8>(buf + koff[j]), q_lane ? __builtin_bit_cast(V8, qf[j]) : V8{}, sc);
    // sc[r] = S[token 4*q4 + r][g = c]
    float tmax = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if constexpr (edge) {
        if (pg * kPageSize + 4 * q4 + r >= seq_len) sc[r] = -INFINITY;
      }
      tmax = fmaxf(tmax, sc[r]);
    }
    tmax = wave_max16(tmax) * p.scale_log2;  // scale > 0 commutes with max
    // Move the reference max only when it grows by > 8 (p stays <= 2^8).
    const bool grow = tmax > m + 8.0f;
    if (__any(grow)) {
      const float m_new = grow ? tmax : m;
      const float alpha = grow ? fast_exp2(m - m_new) : 1.0f;  // m = -inf -> 0
      m = m_new;
      l *= alpha;
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) o[mt] *= alpha;
    }
    const float m_use = (m == -INFINITY) ? 0.f : m;
    V4 pf;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float pr = fast_exp2(sc[r] * p.scale_log2 - m_use);
      l += pr;
      pf[r] = (T)pr;
    }
    s16x4 vt[8];
    lds_ld_tr16_x8_4base(buf + voff[0], buf + voff[1], buf + voff[2], buf + voff[3], vt);
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) {
      s16x4 v = vt[mt];
      if constexpr (edge) {
        // Zero V of tokens past seq_len: stale (possibly NaN) cache rows
        // must not leak through 0 * NaN in the PV product.
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (pg * kPageSize + 4 * q4 + e >= seq_len) v[e] = 0;
      }
      o[mt] = Elem<T>::mfma16k16(__builtin_bit_cast(V4, v), pf, o[mt]);
    }
  };

  // In-launch merges (kMergeInLaunch, p.arrive): the split pieces this wavefront finished
  // wait in the lanes of split_list (piece indices) until it leaves.  It
  // then waits for its partial stores (written through to memory), counts
  // each piece in at its segment's arrival counter, and the piece that
  // arrives last merges the segment with agent-scope loads and clears the
  // counter.  Arrivals at exit keep atomics out of the page stream; a
  // 65th split piece flushes the list first.
  //
  // Visibility rests on the ISA, not on release/acquire atomics: every
  // partial store is an agent-scope write-through store (sc1, inline asm,
  // so the compiler cannot move or merge it), s_waitcnt vmcnt(0) retires
  // them -- written to memory -- before the arrival atomic issues, and the
  // last arrival reads the partials with agent-scope loads, which do not
  // hit in a non-coherent cache.  The memory model's agent-scope release
  // and acquire would add an L2 write-back and an L2 invalidate per
  // arrival, which measured 1.05 -> 1.16 ms on the budget-8192 MIXED batch
  // (the invalidates evict the prefill tiles' K/V lines).
  int split_list = 0;
  int nsplit = 0;
  auto settle = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(kVmcnt0);
    for (int j = 0; j < nsplit; ++j) {
      const i32x8 d = desc_at(__builtin_amdgcn_readlane(split_list, j));
      int* const ctr = p.arrive + (int64_t)d[5] * Hkv + d[7];
      int old = 0;
      if (lane == 0) old = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (__builtin_amdgcn_readfirstlane(old) == d[4] - 1) {
        for (int g = 0; g < G; ++g) merge_segment<T, true>(p, d, g);
        if (lane == 0) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    nsplit = 0;
  };

  // End of piece X: the final output, or its split-K partial (normalised o
  // and log2-sum-exp, device-scope stores that go past this XCD's L2).
  auto finish_piece = [&]() __attribute__((always_inline)) {
    const float l_tot = wave_sum16(l);
    const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
    const int h = X[7];
    if (X[4] == 1) {
      if (q_lane) {
        T* op = (T*)p.out + (int64_t)X[6] * p.out_tok_stride + (int64_t)(h * G + c) * p.out_head_stride + 4 * q4;
#pragma unroll
        for (int mt = 0; mt < 8; ++mt) {
          V4 w;
#pragma unroll
          for (int r = 0; r < 4; ++r) w[r] = (T)(o[mt][r] * inv);
          store8_untracked(op + 16 * mt, __builtin_bit_cast(u32x2, w));
        }
      }
      return;
    }
    const int64_t slot = (int64_t)(X[5] + X[3]) * Hkv + h;
    if (q_lane) {
      float* po = p.part_o + (slot * G + c) * kHeadDim + 4 * q4;
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) store16_device_untracked(po + 16 * mt, __builtin_bit_cast(u32x4, o[mt] * inv));
      if (q4 == 0)
        store4_device_untracked(&p.part_lse[slot * G + c], l_tot > 0.f ? m + fast_log2(l_tot) : -INFINITY);
    }
    if constexpr (kMergeInLaunch) {
      if (nsplit == 64) settle();
      split_list = lane == nsplit ? xi : split_list;
      ++nsplit;
    }
  };

  // ---- page stream --------------------------------------------------------
  // (fh, fpg) is the page the next iteration DMAs; fvalid == 0 when nothing
  // follows.
  {
    // X's first page, through the same asm path as every later page (the
    // compiler then tracks no LDS DMA at all in the loop).
    const int64_t base = (int64_t)page_of(bt_lo, bt_hi, 0) * p.page_stride + X[7] * kHeadDim;
    const T* vp = (const T*)p.v_cache + base;
    const T* kp = (const T*)p.k_cache + base;
    const uint32_t lds_k = (uint32_t)(uintptr_t)lds;
    decode_step<true>(io, 0, 0, claim_ctr, bt_word(X, lane), bt_word(X, 64 + lane), q_addr(X), vp + src0_off,
                      vp + src1_off, kp + src0_off, kp + src1_off, lds_k + kDecodePageBytes, lds_k);
  }
  int fvalid = 1;
  int fh = X[7], fpg = 0;
  if (np > 1) {
    fpg = page_of(bt_lo, bt_hi, 1);
  } else if (yi < N) {
    fh = Y[7];
    fpg = sload(p.block_tables, (int64_t)Y[0] * p.bt_stride + Y[1]);
    fpg = (fpg >= 0 && fpg < p.num_pages) ? fpg : 0;
  } else {
    fvalid = 0;
  }

  int i = 0;  // page of X being computed
  int buf = 0;
  const int slot = (int)(threadIdx.x >> 6) & 7;
  int steps = 0;
  for (;;) {
    if (progress) {
      if (lane == 0) progress[slot] = steps;
      ++steps;
      const int partner = __builtin_amdgcn_readfirstlane(*(volatile int*)&progress[slot ^ 4]);
      if (partner >= steps) __builtin_amdgcn_s_setprio(2);
      else __builtin_amdgcn_s_setprio(0);
    }
    // Loop state is wave-uniform; re-assert it so that the lane-dependent
    // code in the loop does not make the compiler keep it in VGPRs.
    i = __builtin_amdgcn_readfirstlane(i);
    np = __builtin_amdgcn_readfirstlane(np);
    buf = __builtin_amdgcn_readfirstlane(buf);
    seq_len = __builtin_amdgcn_readfirstlane(seq_len);
    y_len = __builtin_amdgcn_readfirstlane(y_len);
    z_len = __builtin_amdgcn_readfirstlane(z_len);
    fh = __builtin_amdgcn_readfirstlane(fh);
    fpg = __builtin_amdgcn_readfirstlane(fpg);
    fvalid = __builtin_amdgcn_readfirstlane(fvalid);
    yi = __builtin_amdgcn_readfirstlane(yi);
    zi = __builtin_amdgcn_readfirstlane(zi);
    nx = __builtin_amdgcn_readfirstlane(nx);
    nx_end = __builtin_amdgcn_readfirstlane(nx_end);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      X[k] = __builtin_amdgcn_readfirstlane(X[k]);
      Y[k] = __builtin_amdgcn_readfirstlane(Y[k]);
      Z[k] = __builtin_amdgcn_readfirstlane(Z[k]);
    }
    lds_u8* cur = lds + buf * (2 * kDecodePageBytes);
    lds_u8* nxt = lds + (buf ^ 1) * (2 * kDecodePageBytes);

    // One asm statement issues Y's page table and queries and the claim for
    // Z (first page of X) and the next page's DMAs, then waits for all of it
    // but those DMAs (see decode_step).  When the two static rounds cover
    // every piece (N <= 2W) there is nothing to claim.
    const int loading = (i == 0 && yi < N) ? 1 : 0;
    const int claiming = (!listed && loading && 2 * W < N) ? 1 : 0;
    // Z is assigned now: claimed, or the next entry of this wavefront's list.
    const int taking = listed ? loading : claiming;
    if (fvalid) {
      const int64_t base = (int64_t)fpg * p.page_stride + fh * kHeadDim;
      const T* vp = (const T*)p.v_cache + base;
      const T* kp = (const T*)p.k_cache + base;
      const uint32_t lds_k = (uint32_t)(uintptr_t)nxt;
      decode_step<true>(io, loading, claiming, claim_ctr, bt_word(Y, lane), bt_word(Y, 64 + lane), q_addr(Y),
                        vp + src0_off, vp + src1_off, kp + src0_off, kp + src1_off, lds_k + kDecodePageBytes,
                        lds_k);
    } else {
      decode_step<false>(io, loading, claiming, claim_ctr, bt_word(Y, lane), bt_word(Y, 64 + lane), q_addr(Y), nullptr,
                         nullptr, nullptr, nullptr, 0, 0);
    }
    wave_lds_fence();
    const int craw = io.claim;
    const int nbt_lo = io.bt_lo;
    const int nbt_hi = io.bt_hi;

    if (claiming) zi = 2 * W + C * __builtin_amdgcn_readfirstlane(craw) + jc;
    if (listed && taking) {
      zi = nx < nx_end ? nx : N;
      ++nx;
    }
    // Z's descriptor is needed now only when this is X's last page and Y is
    // a single page (Z's first page is then the next DMA); otherwise it is
    // fetched after the compute below.
    const bool z_now = taking && zi < N && i + 1 == np && Y[2] - Y[1] == 1;
    if (z_now) {
      Z = desc_at(zi);
      z_len = sload(p.seq_lens, Z[0]);
    }

    // The page after the one just issued (for X's last page: Y's second,
    // or Z's first when Y is a single page).
    if (i + 2 < np) {
      fpg = page_of(bt_lo, bt_hi, i + 2);
    } else if (i + 2 == np) {
      fvalid = yi < N;
      fh = Y[7];
      fpg = page_of(nbt_lo, nbt_hi, 0);
    } else if (yi < N) {
      if (Y[2] - Y[1] > 1) {
        fh = Y[7];
        fpg = page_of(nbt_lo, nbt_hi, 1);
      } else {
        fvalid = zi < N;
        if (fvalid) {
          fh = Z[7];
          fpg = sload(p.block_tables, (int64_t)Z[0] * p.bt_stride + Z[1]);
          fpg = (fpg >= 0 && fpg < p.num_pages) ? fpg : 0;
        }
      }
    }

    const int pg = X[1] + i;
    if ((pg + 1) * kPageSize > seq_len) compute(pg, cur, std::true_type{});
    else compute(pg, cur, std::false_type{});
    wave_lds_fence();
    // Z's descriptor and length, fetched after this page's LDS reads so the
    // scalar loads overlap the next page's wait.
    __builtin_amdgcn_sched_barrier(0);
    if (taking && zi < N && !z_now) {
      Z = desc_at(zi);
      z_len = sload(p.seq_lens, Z[0]);
    }
    buf ^= 1;
    if (++i < np) continue;

    // ---- piece boundary ----
    finish_piece();
    if (yi >= N) break;
    X = Y;
    xi = yi;
    seq_len = y_len;
    bt_lo = io.bt_lo;
    bt_hi = io.bt_hi;
    yi = zi;
    Y = Z;
    y_len = z_len;
    zi = N;
#pragma unroll
    for (int j = 0; j < 4; ++j) qf[j] = io.qv[j];
    np = X[2] - X[1];
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) o[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    m = -INFINITY;
    l = 0.f;
    i = 0;
  }

  if constexpr (kMergeInLaunch) {
    if (nsplit > 0) settle();
  }

  // Count this wavefront out; the last one resets the scheduler for the next
  // launch.  Every claim this wavefront made has returned by now (each was
  // retired by the wait of the iteration that issued it), so all claims
  // precede the reset.  Piece lists touch no counter.
  __builtin_amdgcn_s_waitcnt(kVmcnt0);
  if (listed) return;
  int* const exit_ctr = p.sched + kDecodeClaimCounters * kDecodeSchedLineInts;
  int gone = 0;
  if (lane == 0) gone = __hip_atomic_fetch_add(exit_ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (__builtin_amdgcn_readfirstlane(gone) == W - 1) {
    // Lane k < C clears claim counter k; lane C clears the exit counter.
    if (lane <= C) {
      int* const ctr = lane < C ? p.sched + lane * kDecodeSchedLineInts : exit_ctr;
      __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// Partial rows and log-sum-exps, read normally (after the launch that wrote
// them) or with agent-scope loads (inside it: the lines come from memory,
// where the writers' stores went through their own XCD's L2).
template <bool kAgent>
__device__ inline float part_load(const float* a) {
  if constexpr (kAgent) return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else return *a;
}
template <bool kAgent>
__device__ inline f32x2 part_load2(const float* a) {
  if constexpr (kAgent) return f32x2{part_load<true>(a), part_load<true>(a + 1)};
  else return *reinterpret_cast<const f32x2*>(a);
}

// Split-K merge of one (split segment, query head g): d is a piece
// descriptor {seq, -, -, -, n_chunks, part_base, q_row, kv_head} of a
// segment cut into n_chunks > 1 pieces; writes
//   o = sum_k w_k o_k / sum_k w_k,  w_k = 2^(lse_k - max_k lse_k)
// over the segment's chunks k.  Lane L owns chunks L, L+64, ... of the
// log-sum-exp pass and output columns d = 2L, 2L+1 of the weighted sum.
// Runs in the kernel after the decode kernel (kAgent false: the kernel
// boundary makes every partial visible) or inside the launch after the
// segment's last arrival (kAgent true).
template <typename T, bool kAgent>
__device__ void merge_segment(const DecodeParams& p, const i32x8& d, int g) {
  const int lane = threadIdx.x & 63;
  const int G = p.group;
  const int Hkv = p.num_kv_heads;
  const int n = d[4];
  const int pbase = d[5];
  const int64_t qrow = d[6];
  const int h = d[7];
  // Partial slot of chunk k (lse index; o row = slot * D).
  auto slot = [&](int k) -> int64_t { return ((int64_t)(pbase + k) * Hkv + h) * G + g; };
  // The first 16 chunks' rows are requested together with the log-sum-exps
  // (they do not depend on the weights), so a merge of up to 16 chunks costs
  // one memory round trip.  Chunk indices past n are clamped (weight 0).
  constexpr int kBatch = 16;
  f32x2 rows[kBatch];
#pragma unroll
  for (int j = 0; j < kBatch; ++j)
    rows[j] = part_load2<kAgent>(p.part_o + slot(min(j, n - 1)) * kHeadDim + 2 * lane);
  float lse0 = lane < n ? part_load<kAgent>(&p.part_lse[slot(lane)]) : -INFINITY;  // chunks 0..63, kept for the weights
  float mx = lse0;
  for (int k0 = 64; k0 < n; k0 += 64)
    if (k0 + lane < n) mx = fmaxf(mx, part_load<kAgent>(&p.part_lse[slot(k0 + lane)]));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  float a0 = 0.f, a1 = 0.f, wsum = 0.f;
  for (int k0 = 0; k0 < n; k0 += 64) {
    const int k = k0 + lane;
    const float lse = k0 == 0 ? lse0 : (k < n ? part_load<kAgent>(&p.part_lse[slot(k)]) : -INFINITY);
    const float w = (k < n && mx != -INFINITY) ? fast_exp2(lse - mx) : 0.f;
    wsum += w;
    const int cnt = min(64, n - k0);
    for (int j0 = 0; j0 < cnt; j0 += kBatch) {
      if (k0 + j0 > 0) {
#pragma unroll
        for (int j = 0; j < kBatch; ++j)
          rows[j] = part_load2<kAgent>(p.part_o + slot(min(k0 + j0 + j, n - 1)) * kHeadDim + 2 * lane);
      }
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        // Lanes past the chunk count hold weight 0; the clamped rows they
        // pair with are finite partials.
        const float wj =
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), min(j0 + j, 63)));
        const float wk = j0 + j < cnt ? wj : 0.f;
        a0 += wk * rows[j].x;
        a1 += wk * rows[j].y;
      }
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) wsum += __shfl_xor(wsum, off);
  const float winv = wsum > 0.f ? 1.0f / wsum : 0.f;
  T* op = (T*)p.out + qrow * p.out_tok_stride + (int64_t)(h * G + g) * p.out_head_stride + 2 * lane;
  op[0] = (T)(a0 * winv);
  op[1] = (T)(a1 * winv);
}

// Late rows of a fused-store launch: wavefront `row` writes the K/V rows of
// new token `row` (every KV head) that the decode launch did not write (flag
// clear) to slot slots[row] -- as the separate store would, a slot < 0 or
// past the cache is skipped -- and clears the row's flags.
template <typename T>
__device__ void decode_late_store_wave(const DecodeParams& p, int64_t row) {
  const int lane = threadIdx.x & 63;
  const int64_t slot = p.slots_int64 ? ((const int64_t*)p.slots)[row] : ((const int32_t*)p.slots)[row];
  const bool ok = slot >= 0 && slot / kPageSize < p.num_pages;
  for (int h = 0; h < p.num_kv_heads; ++h) {
    int32_t* flag = p.store_flags + row * p.num_kv_heads + h;
    const int32_t written = *flag;
    if (written) {
      if (lane == 0) *flag = 0;
      continue;
    }
    if (!ok) continue;
    const int64_t dst = (slot / kPageSize) * p.page_stride + (slot % kPageSize) * p.tok_stride +
                        (int64_t)h * kHeadDim + 2 * lane;
    const uint32_t kv = *(const uint32_t*)((const T*)p.k_new + row * p.kn_tok_stride +
                                          (int64_t)h * p.kn_head_stride + 2 * lane);
    const uint32_t vv = *(const uint32_t*)((const T*)p.v_new + row * p.vn_tok_stride +
                                          (int64_t)h * p.vn_head_stride + 2 * lane);
    *(uint32_t*)((T*)const_cast<void*>(p.k_cache) + dst) = kv;
    *(uint32_t*)((T*)const_cast<void*>(p.v_cache) + dst) = vv;
  }
}

// Split-K merge of one (split segment, query head g) of the merge list:
// wavefront v takes merge entry v / G and g = v % G.
template <typename T>
__device__ void decode_merge_wave(const DecodeParams& p, const int32_t* __restrict__ merges, int64_t v) {
  // v is wave-uniform: the descriptor comes in through scalar loads.
  const i32x8 d = ((const_i32x8*)merges)[v / p.group];
  merge_segment<T, false>(p, d, (int)(v % p.group));
}

}  // namespace mva
