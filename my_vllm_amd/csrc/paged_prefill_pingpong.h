// Ragged causal chunked prefill, ping-pong form: the kernel behind
// mva_paged_prefill (the PREFILL route).  Same mathematics, LDS tile layouts
// and MFMA fragment layouts as prefill_core (paged_prefill.h).
//
// A workgroup of 8 wavefronts (two per SIMD) holds a 256-row query tile (the
// G query heads of a KV head x 256 / G tokens, head-major); wave w owns rows
// 32w .. 32w + 31.  Every wave alternates two kinds of phase per 64-key tile:
//   M(t): P(t-1) V(t-1) and S(t) = K(t) Q^T on the matrix cores (32 MFMAs and
//         their LDS fragment reads, almost no vector work);
//   S(t): the softmax of S(t) on the vector ALU (mask, row max, reference-max
//         update, O rescale, P(t) = exp2(S * scale - m) packed for the next
//         M phase, row sums; no MFMA).
// Waves 0-3 (group 0) run M(0) S(0) M(1) S(1) ... M(n); waves 4-7 (group 1)
// run the same sequence one phase later, and a workgroup barrier closes
// every phase.  So each SIMD always holds one wave in an M phase and one in
// an S phase: the matrix cores of a SIMD overlap the vector work of the
// other wave, which they do well, instead of that of their own wave, which
// they do poorly.
//
// K and V tiles are triple-buffered in LDS (96 KB).  At even phase 2t the
// waves of group 0 issue the copies of K(t+2) and those of group 1 the
// copies of V(t+1), one 16-key page each (4 global_load_lds of 1 KB): the
// copies have two phase pairs to arrive, which the K/V stream (shared by all
// workgroups of a head through L2, but larger than L2 for long contexts)
// needs.
#pragma once

#include "paged_prefill.h"

namespace mva {

constexpr int kPrefillPPRows = 256;     // query rows per workgroup
constexpr int kPrefillPPThreads = 512;  // 8 wavefronts
constexpr int kPrefillPPBufs = 3;       // LDS buffers per K and V
constexpr int kPrefillPPLdsBytes = 2 * kPrefillPPBufs * kPrefillTileBytes;

// The plan record of tile `idx` with the page ids of page slot `slot` (0..3)
// of 64-key tiles 0 and 1.
__device__ inline PrefillWork plan_work_slot(const int32_t* plan, int idx, int slot) {
  const i32x16 d = ((const_i32x16*)(plan + kPrefillPlanHeaderInts))[idx];
  PrefillWork wk;
  wk.s = d[0];
  wk.t0 = d[1];
  wk.q0 = d[2];
  wk.q_len = d[3];
  wk.kv = d[4];
  wk.ntiles = d[5];
  wk.full_tiles = d[6];
  wk.npages = d[7];
  wk.pg0 = slot == 0 ? d[8] : slot == 1 ? d[9] : slot == 2 ? d[10] : d[11];
  wk.pg1 = slot == 0 ? d[12] : slot == 1 ? d[13] : slot == 2 ? d[14] : d[15];
  return wk;
}

typedef __attribute__((address_space(3))) int32_t lds_i32;

// The items one workgroup claims, run back to back by one wave group (kGrp:
// 0 = waves 0-3, 1 = waves 4-7; a compile-time constant, so that the K and
// V cache pointers are not a run-time choice, which the compiler would serve
// by copying the kernel argument block to scratch).  `tiles` holds
// kPrefillPPBufs K tile buffers then as many V tile buffers
// (kPrefillTileBytes each); `nextq` holds four LDS words through which
// thread 0 publishes claimed items: words 0 / 3 the first item's plan
// index and KV head, words 1 / 2 those of the successor of the item that
// starts next.
//
// Claims: a workgroup of KV head h0 claims from h0's counter.  Once that
// queue is exhausted it reads every head's counter (one per lane of wave 0)
// and claims from the head with the most items left (those items then run
// here, with their own K/V and output columns), so that the workgroups of a
// head served by a faster XCD take over the last items of slower heads
// instead of idling.
//
// Tiles are numbered across items: the tiles of an item that starts at
// global tile G0 are G0 .. G0 + n - 1, and global tile x uses buffer
// x % kPrefillPPBufs, so the copy stream runs on from one item into the
// next.  While item A runs, its successor B is already claimed (its index
// is read at A's start) and A's phases prepare B:
//   * each wave loads B's plan record at the end of its group's first M
//     phase (phase 0 for group 0, 1 for group 1), after its LDS reads, where
//     the group would wait for the other at the barrier anyway, and B's
//     tile-2 page in A's last phases;
//   * group 0 copies K(B, 0) at phase 2 max(n - 2, 1) and K(B, 1) at phase
//     2 max(n - 1, 1), group 1 copies V(B, 0) at phase 2 max(n - 1, 2) when
//     that phase exists (n >= 2); each is the earliest even phase at which
//     the buffer's previous tile has been read for the last time and B's
//     record is loaded;
//   * every wave loads B's query fragments after its last QK of A (phase
//     2n, or 3 for group 1 when n = 1), and thread 0 claims the item after B
//     at phase 2n;
//   * at the end of A's last phase every wave waits for all of these, thread
//     0 publishes the new claim, and one barrier separates A from B.
// So B starts with its queries and first tiles resident and its successor
// known: no plan read, query load, copy wait or claim sits between items.
// Only when A has a single tile does group 1 copy V(B, 0) at B's start
// (it is first read at B's phase 2, after the wait that ends phase 1).
template <typename T, int kGrp>
__device__ __attribute__((always_inline)) inline void prefill_items_pingpong(const PrefillParams& p, int32_t* plan,
                                                                             int h0, lds_u8* tiles, lds_i32* nextq) {
  typedef typename Elem<T>::v8 V8;
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // 0..7
  const int slot = w & 3;  // page slot this wave copies
  const int lane = tid & 63;
  const int ln = lane & 31;
  const int hi = lane >> 5;
  const int G = p.group;
  const int BMT = p.tile_tokens;  // 256 / G
  const int n_items = sload(plan, 0);
  const int H = p.num_kv_heads;
  auto claim = [&](int head) {
    return __hip_atomic_fetch_add(plan + kPrefillPlanLineInts * (1 + head), 1, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
  };
  // Wave 0 (all lanes): given r, lane 0's claim from `head`, and while r
  // shows an exhausted queue, reads every head's counter at once (one head
  // per lane) and claims from the head with the most items left; `head`
  // ends at the head whose queue yielded the returned index (>= n_items:
  // nothing left, or four claims lost to other workgroups).
  auto claim_on = [&](int r0, int& head) {
    int r = __builtin_amdgcn_readfirstlane(r0);
    for (int round = 0; r >= n_items && round < 4; ++round) {
      int best_left = 0, best_h = 0;
      for (int base = 0; base < H; base += 64) {
        const int hh = base + lane;
        int left = 0;
        if (hh < H)
          left = n_items - __hip_atomic_load(plan + kPrefillPlanLineInts * (1 + hh), __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
        int mx = left;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) mx = max(mx, __shfl_xor(mx, off));
        mx = __builtin_amdgcn_readfirstlane(mx);
        if (mx > best_left) {
          best_left = mx;
          best_h = base + (int)__builtin_ctzll(__builtin_amdgcn_ballot_w64(left == mx));
        }
      }
      if (best_left <= 0) break;
      head = best_h;
      int rr = 0;
      if (lane == 0) rr = claim(head);
      r = __builtin_amdgcn_readfirstlane(rr);
    }
    return r;
  };

  // This lane's query row of every item: head g of the KV head, token rr of
  // the item's 256 / G tokens.
  const int R = 32 * w + ln;
  const int g = R / BMT;
  const int rr = R % BMT;

  // Copies: group 0 fills K tiles, group 1 V tiles, wave w page slot w % 4.
  const uint32_t koff = (uint32_t)(((lane & 15) * p.tok_stride + 8 * (lane >> 4)) * (int64_t)sizeof(T));
  const uint32_t voff = (uint32_t)(((lane >> 2) * p.tok_stride + 8 * (lane & 3)) * (int64_t)sizeof(T));
  auto kbuf = [&](int x) { return tiles + (x % kPrefillPPBufs) * kPrefillTileBytes; };
  auto vbuf = [&](int x) { return tiles + (kPrefillPPBufs + x % kPrefillPPBufs) * kPrefillTileBytes; };
  // This wave's page of K (group 0) or V (group 1) of KV head `head`, global
  // tile x.
  auto copy_page = [&](int x, int page, int head) __attribute__((always_inline)) {
    const T* src = (const T*)(kGrp == 0 ? p.k_cache : p.v_cache) + head * kHeadDim;
    lds_u8* buf = kGrp == 0 ? kbuf(x) : vbuf(x);
    dma16_x4_saddr(src + (int64_t)__builtin_amdgcn_readfirstlane(page) * p.page_stride, kGrp == 0 ? koff : voff,
                   (uint32_t)(uintptr_t)(buf + 4096 * slot));
  };

  // Fragment reads (layouts as in prefill_core).
  auto kread = [&](const lds_u8* kb, int j) {  // QK step j: chain j % 2, k-step j / 2
    return lds_ld16<V8>(kb + klds_off(32 * (j & 1) + ln, 2 * (j >> 1) + hi));
  };
  const int ti = lane & 15;
  const int dgrp = (lane >> 4) & 1;
  const int vlane_off = (4 * hi + (ti >> 2)) * 64 + (2 * dgrp + ((ti >> 1) & 1)) * 16 + (ti & 1) * 8;
  auto vread = [&](const lds_u8* vb, int j) {  // PV step j: k-step j / 4, d-tile j % 4
    const lds_u8* a = vb + vlane_off + (j >> 2) * 4096 + (j & 3) * 1024;
    return __builtin_bit_cast(V8, __builtin_shufflevector(lds_ld_tr16(a), lds_ld_tr16(a + 512), 0, 1, 2, 3, 4, 5, 6,
                                                          7));
  };

  V8 qf[8];
  // Query fragments of item `it` of KV head `kvh` (rows past the sequence or
  // the heads read zeros).
  auto load_q = [&](const PrefillWork& it, int kvh) __attribute__((always_inline)) {
    const int tq = it.t0 + rr;
    const bool ok = g < G && tq < it.q_len;
    const int row_tok = it.q0 + (ok ? tq : 0);
    const int head = kvh * G + (g < G ? g : 0);
    const T* qp = (const T*)p.q + (int64_t)row_tok * p.q_tok_stride + (int64_t)head * p.q_head_stride;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) qf[kk] = ok ? ld16<V8>(qp + 8 * (2 * kk + hi)) : V8{};
  };

  f32x16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = f32x16{};
  f32x16 st[2];  // S(t): st[mt][i] = S[query ln][key 32*mt + 8*(i/4) + 4*hi + i%4]
  u32x4 pw[4];   // P(t) for PV k-step kk: four packed pairs
  float m = -INFINITY;  // reference max (log2 units) of the item's tiles so far
  float l = 0.f;        // row sum of P relative to m

  // Phase fences for the compiler.  A barrier orders memory only: without
  // these, passes before instruction scheduling move register-only work (a
  // row max, the exponentials) across it into the other phase.  An empty
  // asm statement that "rewrites" a phase's inputs at its start and its
  // outputs at its end ties that work to its phase.
  auto pin_s = [&]() __attribute__((always_inline)) { asm volatile("" : "+v"(st[0]), "+v"(st[1])); };
  auto pin_p = [&]() __attribute__((always_inline)) {
    asm volatile("" : "+v"(pw[0]), "+v"(pw[1]), "+v"(pw[2]), "+v"(pw[3]));
  };
  auto pin_o = [&]() __attribute__((always_inline)) {
    asm volatile("" : "+v"(o[0]), "+v"(o[1]), "+v"(o[2]), "+v"(o[3]));
  };
  // A workgroup barrier that also closes the phase for the instruction
  // scheduler (s_barrier alone lets register-only work move across it).
  auto phase_barrier = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
  };
  // Waits until at most the last c page copies (4 loads each) are in flight.
  auto wait_copies = [&](int c) __attribute__((always_inline)) {
    if (c >= 2) __builtin_amdgcn_s_waitcnt(waitcnt_vm(8));
    else if (c == 1) __builtin_amdgcn_s_waitcnt(waitcnt_vm(4));
    else __builtin_amdgcn_s_waitcnt(kVmcnt0);
  };

  // Page id of tile `tile` of item `it` at this wave's page slot.
  auto page_of_item = [&](const PrefillWork& it, int tile) {
    const int32_t* btp = p.block_tables + (int64_t)it.s * p.bt_stride;
    const int pg = sload(btp, min(tile * (kPrefillKeys / kPageSize) + slot, it.npages - 1));
    return (pg >= 0 && pg < p.num_pages) ? pg : 0;
  };

  // ---- the first item ---------------------------------------------------------
  int claim_head = h0;  // wave 0: the head claimed from last
  int claim_ret = 0;    // thread 0: the latest claim
  if (w == 0) {
    int r = 0;
    if (lane == 0) r = claim(h0);
    r = claim_on(r, claim_head);
    if (lane == 0) {
      nextq[0] = r;
      nextq[3] = claim_head;
    }
  }
  __syncthreads();
  int idx = __builtin_amdgcn_readfirstlane(nextq[0]);
  if (idx >= n_items) return;  // uniform: nothing for this workgroup
  int cur_h = __builtin_amdgcn_readfirstlane(nextq[3]);
  PrefillWork cur = plan_work_slot(plan, idx, slot);
  // The page of the item's tile 2, which the item's first copies need; for
  // later items it is loaded during the item before (see below).
  int pg2_next = page_of_item(cur, 2);
  if (tid == 0) claim_ret = claim(claim_head);
  load_q(cur, cur_h);
  if constexpr (kGrp == 0) {
    copy_page(0, cur.pg0, cur_h);
    if (1 < cur.ntiles) copy_page(1, cur.pg1, cur_h);
  } else {
    copy_page(0, cur.pg0, cur_h);
  }
  __builtin_amdgcn_s_waitcnt(kVmcnt0);
  if (w == 0) {
    const int r = claim_on(claim_ret, claim_head);
    if (lane == 0) {
      nextq[1] = r;
      nextq[2] = claim_head;
    }
  }
  phase_barrier();
  int G0 = 0;            // global index of the item's tile 0
  bool v0_done = true;   // V of the item's tile 0 is copied (group 1)

  const std::true_type yes;
  const std::false_type no;
  while (true) {
    const int nidx = __builtin_amdgcn_readfirstlane(nextq[1]);
    const int nh = __builtin_amdgcn_readfirstlane(nextq[2]);  // B's KV head
    const bool has_next = nidx < n_items;
    const int n = cur.ntiles;
    const int full_tiles = cur.full_tiles;
    const int kv = cur.kv;
    const int tq = cur.t0 + rr;
    const bool row_ok = g < G && tq < cur.q_len;
    const int pos = row_ok ? kv - cur.q_len + tq : -1;  // keys j <= pos are visible
    auto page_of = [&](int tile) { return page_of_item(cur, tile); };
    PrefillWork nx;  // B's record, loaded at this item's first S phase
    nx.ntiles = 0;
    auto load_next = [&]() __attribute__((always_inline)) {
      if (has_next) nx = plan_work_slot(plan, nidx, slot);
    };
    if constexpr (kGrp == 1) {
      if (!v0_done) copy_page(G0, cur.pg0, cur_h);
    }
    m = -INFINITY;
    l = 0.f;

    // M phase t: PV(t-1) and QK(t), alternating, fragment reads one step ahead.
    auto phase_m = [&](int t, auto with_qk_tag, auto with_pv_tag) __attribute__((always_inline)) {
      constexpr bool with_qk = decltype(with_qk_tag)::value;
      constexpr bool with_pv = decltype(with_pv_tag)::value;
      if constexpr (with_pv) pin_p();
      const lds_u8* kb = kbuf(G0 + t);
      const lds_u8* vb = vbuf(G0 + t + kPrefillPPBufs - 1);  // V(t-1)
      V8 kf[2], vf[2];
      if constexpr (with_qk) {
        kf[0] = kread(kb, 0);
        st[0] = f32x16{};
        st[1] = f32x16{};
      }
      if constexpr (with_pv) vf[0] = vread(vb, 0);
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        if constexpr (with_qk) {
          if (j + 1 < 16) kf[(j + 1) & 1] = kread(kb, j + 1);
          st[j & 1] = Elem<T>::mfma32(kf[j & 1], qf[j >> 1], st[j & 1]);
        }
        if constexpr (with_pv) {
          if (j + 1 < 16) vf[(j + 1) & 1] = vread(vb, j + 1);
          o[j & 3] = Elem<T>::mfma32(vf[j & 1], __builtin_bit_cast(V8, pw[j >> 2]), o[j & 3]);
        }
        // Keeps the fragment reads one step ahead instead of all at the top,
        // which would hold 48 fragments in registers at once.
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (with_qk) pin_s();
      if constexpr (with_pv) pin_o();
    };

    // S phase t: softmax of S(t) into P(t).
    //
    // Fast path (tiles after the first): P = exp2(S * scale - m) with the
    // reference max as it stands, no row max.  It stands for this tile exactly
    // when no element exceeds it by more than 8, and a row sum below 128 shows
    // that for every element of the lane (each P is >= 0, and P < 128 means
    // S * scale - m < 7.01, short of m + 8 by more than the rounding of
    // S * scale and m + 8 while |m| < 2^20).  A row whose max is still -inf
    // qualifies only when the tile masks all its keys (pos < 64 t): then P is
    // 0 either way.  When every lane of the wave qualifies, P, l and m are
    // bit for bit those of the full path below; otherwise the full path runs
    // (row max, reference-max update, O rescale) and overwrites P.
    auto phase_s = [&](int t) __attribute__((always_inline)) {
      pin_s();
      bool fast = false;
      if (t >= full_tiles) {
        // Key t*64 + 32*mt + 8*(i/4) + 4*hi + i%4 is visible when
        // 32*mt + 8*(i/4) + i%4 <= lim.  lim and S pass through an empty asm
        // statement so that the masking stays inside this branch.  Bit k of
        // vis[mt] says whether offset 32*mt + k is visible; each element is
        // then a bit extract and a bit select on vector registers.  (Written
        // as compares and selects, the compiler computes all 32 compare masks
        // first and keeps them in scalar registers, which pushed the loop's
        // other scalar state out to VGPR lanes: about 20 v_readlane restores
        // per tile in every phase that issues a copy.)
        int lim = pos - t * kPrefillKeys - 4 * hi;
        asm volatile("" : "+v"(lim), "+v"(st[0]), "+v"(st[1]));
        uint32_t vis[2];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const int bl = lim - 32 * mt;
          vis[mt] = bl < 0 ? 0u : bl >= 31 ? ~0u : (2u << bl) - 1u;
        }
        const uint32_t ninf = 0xff800000u;  // -inf
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            int sel;  // all ones when the key is visible
            uint32_t x = __float_as_uint(st[mt][i]);
            asm volatile("v_bfe_i32 %0, %1, %2, 1" : "=v"(sel) : "v"(vis[mt]), "i"(8 * (i >> 2) + (i & 3)));
            asm volatile("v_bfi_b32 %0, %1, %2, %3" : "=v"(x) : "v"(sel), "v"(x), "s"(ninf));
            st[mt][i] = __uint_as_float(x);
          }
      }
      if (t > 0) {
        const float m_fast = (m == -INFINITY) ? 0.f : m;
        float la = 0.f, lb = 0.f;
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          const int mt = q >> 3, i = 2 * (q & 7);
          const float e0 = fast_exp2(st[mt][i] * p.scale_log2 - m_fast);
          const float e1 = fast_exp2(st[mt][i + 1] * p.scale_log2 - m_fast);
          pw[2 * mt + (q & 7) / 4][((i >> 2) & 1) * 2 + ((i & 3) >> 1)] = PackedPair<T>::pack(e0, e1);
          la += e0;
          lb += e1;
        }
        const float lt = la + lb;
        const bool ok = __builtin_fabsf(m) < 0x1p20f ? lt < 128.f : (m == -INFINITY && pos < t * kPrefillKeys);
        fast = !__builtin_amdgcn_ballot_w64(!ok);
        if (fast) l += lt;
      }
      if (!fast) {
        // Row max with the IEEE maximum (v_maximum3_f32), which needs no
        // quieting of MFMA-produced inputs, unlike fmaxf.
        float tmax = -INFINITY;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int i = 0; i < 16; i += 2)
            tmax = __builtin_elementwise_maximum(__builtin_elementwise_maximum(tmax, st[mt][i]), st[mt][i + 1]);
        // The reference max moves only when it grows by more than 8 (log2
        // units): P stays <= 2^8 and most tiles skip the O rescale.
        const float tmax_s = pair_max(tmax) * p.scale_log2;  // scale > 0 commutes with max
        const bool grow = tmax_s > m + 8.0f;
        const float m_new = grow ? tmax_s : m;
        const float alpha = grow ? fast_exp2(m - m_new) : 1.0f;  // m = -inf -> 0
        m = m_new;
        const float m_use = (m == -INFINITY) ? 0.f : m;
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
          l *= alpha;
#pragma unroll
          for (int dt = 0; dt < 4; ++dt) o[dt] *= alpha;
        }
        float la = 0.f, lb = 0.f;
#pragma unroll
        for (int q = 0; q < 16; ++q) {  // element pair q: elements 2q, 2q + 1
          const int mt = q >> 3, i = 2 * (q & 7);
          const float e0 = fast_exp2(st[mt][i] * p.scale_log2 - m_use);
          const float e1 = fast_exp2(st[mt][i + 1] * p.scale_log2 - m_use);
          pw[2 * mt + (q & 7) / 4][((i >> 2) & 1) * 2 + ((i & 3) >> 1)] = PackedPair<T>::pack(e0, e1);
          la += e0;
          lb += e1;
        }
        l += la + lb;
      }
      pin_p();
    };

    // Zero V rows of keys >= kv in the item's last tile (stale rows may hold
    // NaN and 0 * NaN would leak through P = 0).
    auto zero_tail = [&]() __attribute__((always_inline)) {
      lds_u8* vb = vbuf(G0 + n - 1);
      const int first_bad = kv - (n - 1) * kPrefillKeys;  // rows >= first_bad are past the sequence
      for (int i = tid; i < (kPrefillKeys - first_bad) * 16; i += kPrefillPPThreads) {
        const int key = first_bad + (i >> 4);
        lds_st16<u32x4>(vb + vlds_blk_off(key, i & 15), u32x4{0, 0, 0, 0});
      }
    };

    // Copies this wave issues at phase 2t, and their number: this item's
    // K(t+2) (group 0) or V(t+1) (group 1), and B's first tiles at the
    // phases given above.
    int pg_next = 0;  // page id of this wave's next copy of this item
    auto issue = [&](int t) __attribute__((always_inline)) {
      int c = 0;
      if constexpr (kGrp == 0) {
        if (t + 2 < n) {
          copy_page(G0 + t + 2, pg_next, cur_h);
          ++c;
        }
        if (has_next && t == max(n - 2, 1)) {
          copy_page(G0 + n, nx.pg0, nh);
          ++c;
        }
        if (has_next && t == max(n - 1, 1) && 1 < nx.ntiles) {
          copy_page(G0 + n + 1, nx.pg1, nh);
          ++c;
        }
      } else {
        if (t + 1 < n) {
          copy_page(G0 + t + 1, pg_next, cur_h);
          ++c;
        }
        if (has_next && n >= 2 && t == max(n - 1, 2)) {
          copy_page(G0 + n, nx.pg0, nh);
          ++c;
        }
      }
      return c;
    };

    // Phases 0 .. 2n+1.  At phase 2t group 0 copies K(t+2) and group 1 V(t+1)
    // (three buffers each: the buffer written was last read in phase 2t-1),
    // and every wave waits for its copies of phase 2t-2 at the end of phase
    // 2t+1, before the barrier that opens their first reader's phase 2t+2; so
    // a copy has two phase pairs to land.  pg_next is loaded at the start of
    // an S phase (no LDS reads there to wait behind the scalar load) and used
    // at the next even phase.  V(n-1) lands by the end of phase 2n-1 and is
    // first read in phase 2n (group 0's M(n)): its stale tail rows are
    // cleared between them.  Both groups pass the same barriers.  M(0) (no
    // PV) and M(n) (no QK) are peeled off the loop so the loop body holds one
    // copy of each phase.
    const bool tail = n * kPrefillKeys > kv;
    auto end_odd_phase = [&](int t, int c) __attribute__((always_inline)) {
      wait_copies(c);
      phase_barrier();
      if (t == n - 1 && tail) {
        zero_tail();
        phase_barrier();
      }
    };
    // Phases 0 and 1.
    pg_next = kGrp == 0 ? pg2_next : __builtin_amdgcn_readfirstlane(cur.pg1);
    int c = issue(0);
    // B's record (and group 0's tile-3 page) are loaded at the end of the
    // group's phase-0 / phase-1 M phase, where it waits for the other group
    // anyway (its LDS reads are done, so nothing waits behind the loads).
    if constexpr (kGrp == 0) {
      phase_m(0, yes, no);
      load_next();
      pg_next = page_of(3);
      phase_barrier();
      phase_s(0);
    } else {
      pg_next = pg2_next;
      phase_barrier();
      phase_m(0, yes, no);
      load_next();
    }
    end_odd_phase(0, c);
    // Phases 2t and 2t+1, t = 1 .. n-1.
    for (int t = 1; t < n; ++t) {
      c = issue(t);
      if constexpr (kGrp == 0) {
        phase_m(t, yes, yes);
        phase_barrier();
        pg_next = page_of(t + 3);
        phase_s(t);
      } else {
        pg_next = page_of(t + 2);
        phase_s(t - 1);
        phase_barrier();
        phase_m(t, yes, yes);
      }
      end_odd_phase(t, c);
    }
    // Phases 2n and 2n+1; then every copy, query load and claim of this item
    // has landed, and thread 0 publishes the claim.
    if constexpr (kGrp == 0) {
      if (has_next) {
        load_q(nx, nh);
        if (tid == 0) claim_ret = claim(claim_head);
      }
      issue(n);
      phase_m(n, no, yes);
      phase_barrier();
      // B's tile-2 page, loaded while this group waits for group 1's M(n).
      if (has_next) pg2_next = page_of_item(nx, 2);
      __builtin_amdgcn_s_waitcnt(kVmcnt0);
      if (w == 0 && has_next) {
        const int r = claim_on(claim_ret, claim_head);
        if (lane == 0) {
          nextq[1] = r;
          nextq[2] = claim_head;
        }
      }
    } else {
      issue(n);
      if (has_next && n >= 2) load_q(nx, nh);
      // B's tile-2 page, in an S phase (no LDS read waits behind the load).
      if (has_next) pg2_next = page_of_item(nx, 2);
      phase_s(n - 1);
      phase_barrier();
      if (has_next && n == 1) load_q(nx, nh);
      phase_m(n, no, yes);
      __builtin_amdgcn_s_waitcnt(kVmcnt0);
    }
    phase_barrier();

    // Epilogue: O^T / l -> out[token][head][d].
    const float l_tot = pair_sum(l);
    const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
    if (p.out16) {
      // Staged in this wave's page slot of the K buffer (group 0) or V
      // buffer (group 1) of the item's last tile: the K buffer is next
      // written by this wave's own copy at the next item's phase 0, the V
      // buffer at its phase 2.
      lds_u8* stage = (kGrp == 0 ? kbuf(G0 + n - 1) : vbuf(G0 + n - 1)) + 4096 * slot;
      // Row 8j + lane / 8 of the wave: head g0 + (0..2), token rr0 + ...
      // (256 / G >= 16 tokens per head, so 32 rows span at most 3 heads).
      const int g0 = (32 * w) / BMT, rr0 = (32 * w) % BMT;
      T* rowp[4];
      bool rok[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        int rj = rr0 + 8 * j + (lane >> 3), gj = g0;
        if (rj >= BMT) rj -= BMT, ++gj;
        if (rj >= BMT) rj -= BMT, ++gj;
        const int tj = cur.t0 + rj;
        rok[j] = gj < G && tj < cur.q_len;
        rowp[j] = (T*)p.out + (int64_t)(cur.q0 + (rok[j] ? tj : 0)) * p.out_tok_stride +
                  (int64_t)(cur_h * G + (rok[j] ? gj : 0)) * p.out_head_stride + 8 * (lane & 7);
      }
      store_rows_staged<T>(stage, o, inv, rowp, rok);
    } else {
      T* op = (T*)p.out + (int64_t)(cur.q0 + tq) * p.out_tok_stride + (int64_t)(cur_h * G + g) * p.out_head_stride;
      store_rows<T>(p, op, o, inv, row_ok);
    }
    if (!has_next) return;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[dt] = f32x16{};
    G0 += n;
    v0_done = n >= 2;
    cur = nx;
    cur_h = nh;
  }
}

}  // namespace mva
