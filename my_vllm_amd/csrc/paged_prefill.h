// Ragged causal chunked prefill over prefix-cached pages, bf16/fp16 MFMA.
//
// Replaces FlashInfer's BatchPrefillWithPagedKVCacheWrapper.run on the
// reference's PREFILL route (nanovllm/layers/attention_backend.py:992-994) and
// the prefill half of MIXED_SPLIT (:1015-1019).  For query i of sequence s
// (q_s new tokens, kv_s = seq_lens[s] keys including them) the absolute
// position is kv_s - q_s + i and the query sees keys j <= kv_s - q_s + i
// (bottom-right causal alignment).  The new tokens' K/V are read from the
// cache: the slot_mapping store runs before this kernel.
//
// Work: one 256-thread workgroup (4 wavefronts) per (sequence, KV head,
// query tile).  A tile holds 128 query rows = the G query heads of the KV head
// x BMT = 128 / G tokens (head-major: row R -> head R / BMT, token R % BMT),
// so every K/V byte staged in LDS serves all G heads.  Wave w owns rows
// 32w .. 32w + 31.
//
// Per 64-key tile (double-buffered in LDS, filled by global_load_lds):
//   S^T[key, q] = K[key, :] . Q[q, :]       v_mfma_f32_32x32x16 (A = K from LDS,
//                                            B = Q held in registers)
//   online softmax per query (each lane owns one query row: the C layout of
//   S^T puts a query's 32 keys in lanes l and l^32)
//   O^T[d, q] += V^T[d, key] P^T[key, q]    (A = V^T via ds_read_b64_tr_b16,
//                                            B = P^T straight from S^T's C layout)
// The running max is only moved when it grows by more than 8 (log2 units), so
// the O rescale is skipped on most tiles.
#pragma once

#include "mva_common.h"
#include "paged_decode.h"

namespace mva {

constexpr int kPrefillRows = 128;  // query rows per workgroup
constexpr int kPrefillKeys = 64;   // keys per LDS tile
constexpr int kPrefillTileBytes = kPrefillKeys * kHeadDim * 2;  // one K (or V) tile
constexpr int kPrefillPtabEntries = 2048;                       // page ids staged per segment
constexpr int kPrefillLdsBytes = 4 * kPrefillTileBytes + kPrefillPtabEntries * 4;
constexpr int kPrefillItemInts = 4;  // {seq, first token of the tile, 0, 0}

struct PrefillParams {
  const void* q;
  int64_t q_tok_stride;
  int64_t q_head_stride;
  const void* k_cache;
  const void* v_cache;
  int64_t num_pages;
  int64_t page_stride;
  int64_t tok_stride;
  const int32_t* block_tables;
  int64_t bt_stride;
  const int32_t* seq_lens;
  const int32_t* query_start_loc;
  const int32_t* items;
  int num_items;
  void* out;
  int64_t out_tok_stride;
  int64_t out_head_stride;
  int num_kv_heads;
  int group;
  int tile_tokens;  // BMT = 128 / group (rounded down)
  float scale_log2;
};

// LDS tile layouts.  A 64-key x 128-d tile is 16 blocks of 1 KB, block
// (key/16, chunk/4) holding 16 keys x 4 16-byte d-chunks:
//   K: chunk-major inside a block, so the A-operand read of 16 consecutive
//      keys at one chunk is 256 contiguous bytes;
//   V: key-major inside a block, so a transposed read of 4 keys x 32 bytes by
//      each 16-lane group covers 512 contiguous bytes per wave.
// Both make every fragment address "lane base + immediate", and each
// global_load_lds instruction (64 lanes x 16 bytes) fills exactly one block.
__device__ inline int klds_off(int key, int ch) {
  return (((key >> 4) << 2) + (ch >> 2)) * 1024 + (ch & 3) * 256 + (key & 15) * 16;
}
__device__ inline int vlds_blk_off(int key, int ch) {
  return (((key >> 4) << 2) + (ch >> 2)) * 1024 + (key & 15) * 64 + (ch & 3) * 16;
}

template <typename T>
__device__ void prefill_item(const PrefillParams& p, const int32_t* __restrict__ it, int h, lds_u8* lds) {
  typedef typename Elem<T>::v8 V8;
  const int tid = threadIdx.x;
  const int w = tid >> 6;
  const int lane = tid & 63;
  const int ln = lane & 31;
  const int hi = lane >> 5;

  const int s = it[0];
  const int t0 = it[1];
  const int q0 = p.query_start_loc[s];
  const int q_len = p.query_start_loc[s + 1] - q0;
  if (t0 >= q_len) return;  // tile past this sequence's queries (host sizes conservatively)
  const int kv = p.seq_lens[s];
  const int G = p.group;
  const int BMT = p.tile_tokens;
  const int base_pos = kv - q_len;  // absolute position of query token 0

  // This lane's query row.
  const int R = 32 * w + ln;
  const int g = R / BMT;
  const int tq = t0 + R % BMT;
  const bool row_ok = g < G && tq < q_len;
  const int pos = row_ok ? base_pos + tq : -1;  // keys j <= pos are visible

  const int t_end = min(t0 + BMT, q_len);
  const int kv_end = base_pos + t_end;  // keys [0, kv_end) are needed by some row
  const int ntiles = (kv_end + kPrefillKeys - 1) / kPrefillKeys;
  const int full_tiles = (base_pos + t0 + 1) / kPrefillKeys;  // tiles no row masks

  // LDS: K buffers at [0, 32K), V buffers at [32K, 64K), page ids after.
  auto kbuf = [&](int b) { return lds + b * kPrefillTileBytes; };
  auto vbuf = [&](int b) { return lds + (2 + b) * kPrefillTileBytes; };
  __attribute__((address_space(3))) int32_t* ptab =
      reinterpret_cast<__attribute__((address_space(3))) int32_t*>(lds + 4 * kPrefillTileBytes);

  // Q fragments (B operand of S^T = K Q^T): k-step kk covers d-chunk 2*kk + hi.
  V8 qf[8];
  {
    const int row_tok = q0 + (row_ok ? tq : 0);
    const int head = h * G + (g < G ? g : 0);
    const T* qp = (const T*)p.q + (int64_t)row_tok * p.q_tok_stride + (int64_t)head * p.q_head_stride;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) qf[kk] = row_ok ? ld16<V8>(qp + 8 * (2 * kk + hi)) : V8{};
  }

  const T* kc = (const T*)p.k_cache + h * kHeadDim;
  const T* vc = (const T*)p.v_cache + h * kHeadDim;
  const int32_t* bt = p.block_tables + (int64_t)s * p.bt_stride;
  const int npages = (kv_end + kPageSize - 1) / kPageSize;

  // Stage page ids [seg0, seg0 + 2048) of this sequence in LDS.
  auto load_ptab = [&](int seg0) {
    for (int i = tid; i < kPrefillPtabEntries && seg0 + i < npages; i += 256) {
      int pg = bt[seg0 + i];
      ptab[i] = (pg >= 0 && pg < p.num_pages) ? pg : 0;
    }
  };
  int seg0 = 0;
  load_ptab(0);
  __syncthreads();

  // DMA of tile `tile` into buffer `b`: wave w loads page w of the tile (16
  // keys): 4 K blocks and 4 V blocks of 1 KB.  Keys past the needed range
  // clamp to the last needed page and are masked later.
  auto load_tile = [&](int tile, int b) {
    const int pg_abs = min(tile * (kPrefillKeys / kPageSize) + w, npages - 1);
    const int page = ptab[pg_abs - seg0];  // tiles never straddle a segment
    const T* kp = kc + (int64_t)page * p.page_stride;
    const T* vp = vc + (int64_t)page * p.page_stride;
#pragma unroll
    for (int cg = 0; cg < 4; ++cg) {
      const int blk = 4 * w + cg;
      // K block: lane -> token lane%16, chunk 4*cg + lane/16.
      dma16(kp + (lane & 15) * p.tok_stride + 8 * (4 * cg + (lane >> 4)), kbuf(b) + blk * 1024);
      // V block: lane -> token lane/4, chunk 4*cg + lane%4.
      dma16(vp + (lane >> 2) * p.tok_stride + 8 * (4 * cg + (lane & 3)), vbuf(b) + blk * 1024);
    }
  };

  f32x16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = f32x16{};
  float m = -INFINITY;
  float l = 0.f;

  auto compute = [&](int tile, int b, auto masked_tag) {
    constexpr bool masked = decltype(masked_tag)::value;
    const lds_u8* kb = kbuf(b);
    const lds_u8* vb = vbuf(b);
    const int j0 = tile * kPrefillKeys;
    f32x16 st[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      st[mt] = f32x16{};
      const int key = 32 * mt + ln;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const V8 a = lds_ld16<V8>(kb + klds_off(key, 2 * kk + hi));
        st[mt] = Elem<T>::mfma32(a, qf[kk], st[mt]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // st[mt][i] = S[query ln][key j0 + 32*mt + 8*(i/4) + 4*hi + i%4]
    float tmax = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if constexpr (masked) {
          const int key = j0 + 32 * mt + 8 * (i >> 2) + 4 * hi + (i & 3);
          if (key > pos) st[mt][i] = -INFINITY;
        }
        tmax = fmaxf(tmax, st[mt][i]);
      }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
    const float tmax_s = tmax * p.scale_log2;  // scale > 0 commutes with max
    // Move the reference max only when it grows by > 8 (p stays <= 2^8).
    const bool grow = tmax_s > m + 8.0f;
    if (__any(grow)) {
      const float m_new = grow ? tmax_s : m;
      const float alpha = grow ? fast_exp2(m - m_new) : 1.0f;  // m = -inf -> 0
      m = m_new;
      l *= alpha;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) o[dt] *= alpha;
    }
    const float m_use = (m == -INFINITY) ? 0.f : m;
    V8 pf[4];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float pr = fast_exp2(st[mt][i] * p.scale_log2 - m_use);
        l += pr;
        // PV k-step kk = 2*mt + (i/4)/2 takes blocks b0 = 2*(kk%2), b0+1:
        // slot (i/4 % 2)*4 + i%4.
        pf[2 * mt + ((i >> 2) >> 1)][((i >> 2) & 1) * 4 + (i & 3)] = (T)pr;
      }
    // PV: A = V^T via transposed LDS reads.  16-lane group a = lane/16 covers
    // d offset 16*(a&1) of the 32-d tile and keys 4*hi.. of each 8-key block;
    // supplier lane ti gives row 4*hi + ti/4 at d offset 4*(ti%4).
    const int ti = lane & 15;
    const int dgrp = (lane >> 4) & 1;
    const lds_u8* vlane = vb + (4 * hi + (ti >> 2)) * 64 + (2 * dgrp + ((ti >> 1) & 1)) * 16 + (ti & 1) * 8;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      // Reads for (dt, j) sit at byte dt*1024 + j*512 past block 4*kk.
      s16x4 vt[8];
      lds_ld_tr16_x8_stride512(vlane + 4 * kk * 1024, vt);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const s16x8 both = __builtin_shufflevector(vt[2 * dt], vt[2 * dt + 1], 0, 1, 2, 3, 4, 5, 6, 7);
        o[dt] = Elem<T>::mfma32(__builtin_bit_cast(V8, both), pf[kk], o[dt]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Zero V rows of keys >= kv in the last tile (stale rows may hold NaN and
  // 0 * NaN would leak through P = 0).
  auto zero_tail = [&](int tile, int b) {
    const int first_bad = kv - tile * kPrefillKeys;  // rows >= first_bad are past the sequence
    if (first_bad >= kPrefillKeys) return;
    for (int i = tid; i < (kPrefillKeys - first_bad) * 16; i += 256) {
      const int key = first_bad + (i >> 4);
      lds_st16<u32x4>(vbuf(b) + vlds_blk_off(key, i & 15), u32x4{0, 0, 0, 0});
    }
  };

  load_tile(0, 0);
  for (int tile = 0; tile < ntiles; ++tile) {
    const int b = tile & 1;
    __builtin_amdgcn_s_waitcnt(kVmcnt0);
    __syncthreads();  // tile landed for all waves; the other buffer is free
    if ((tile + 1) * kPrefillKeys / kPageSize - seg0 >= kPrefillPtabEntries && tile + 1 < ntiles) {
      // Next tile starts past the staged page ids: restage (rare, > 32K keys).
      seg0 = (tile + 1) * kPrefillKeys / kPageSize;
      load_ptab(seg0);
      __syncthreads();
    }
    if (tile + 1 < ntiles) load_tile(tile + 1, b ^ 1);
    if (tile == ntiles - 1 && (tile + 1) * kPrefillKeys > kv) {
      zero_tail(tile, b);
      __syncthreads();
    }
    if (tile < full_tiles) compute(tile, b, std::false_type{});
    else compute(tile, b, std::true_type{});
  }

  // Epilogue: O^T / l -> out[token][head][d].
  const float l_tot = l + __shfl_xor(l, 32);
  if (!row_ok) return;
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  T* op = (T*)p.out + (int64_t)(q0 + tq) * p.out_tok_stride + (int64_t)(h * G + g) * p.out_head_stride;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int bk = 0; bk < 4; ++bk) {
      typename Elem<T>::v4 wv;
#pragma unroll
      for (int e = 0; e < 4; ++e) wv[e] = (T)(o[dt][4 * bk + e] * inv);
      *reinterpret_cast<typename Elem<T>::v4*>(op + 32 * dt + 8 * bk + 4 * hi) = wv;
    }
}

}  // namespace mva
