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
// Per 64-key tile t, the K and V tiles sit in separate double-buffered LDS
// arrays, filled by global_load_lds:
//   S^T[key, q] = K[key, :] . Q[q, :]       v_mfma_f32_32x32x16 (A = K from LDS,
//                                            B = Q held in registers)
//   online softmax per query (each lane owns one query row: the C layout of
//   S^T puts a query's 32 keys in lanes l and l^32)
//   O^T[d, q] += V^T[d, key] P^T[key, q]    (A = V^T via ds_read_b64_tr_b16,
//                                            B = P^T straight from S^T's C layout)
// Software pipeline: iteration t computes S(t+1) on the matrix cores while
// the vector ALUs run the softmax of S(t), then accumulates P(t) V(t).  K runs
// one tile ahead of V, so iteration t needs K(t+1) and V(t) resident while
// K(t+2) and V(t+1) stream in.  The running max is only moved when it grows
// by more than 8 (log2 units), so P stays <= 2^8 and the O rescale is skipped
// on most tiles.
#pragma once

#include "mva_common.h"
#include "paged_decode.h"

namespace mva {

constexpr int kPrefillRows = 128;  // query rows per workgroup
constexpr int kPrefillKeys = 64;   // keys per LDS tile
constexpr int kPrefillTileBytes = kPrefillKeys * kHeadDim * 2;  // one K (or V) tile

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
  int num_seqs;  // prefill sequences (the leading rows of the batch)
  void* out;
  int64_t out_tok_stride;
  int64_t out_head_stride;
  int num_kv_heads;
  int group;
  int tile_tokens;  // BMT = 128 / group (rounded down)
  float scale_log2;
  int out16;  // out and its strides are 16-byte aligned (16-byte output stores)
};

// LDS tile layouts of the ping-pong kernel.  A 64-key x 128-d tile is 16
// blocks of 1 KB, block (key/16, chunk/4) holding 16 keys x 4 16-byte
// d-chunks:
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

// Whole-line tile layouts (the MIXED kernel's prefill core).  A page slot
// (16 keys, 4 KB) is 4 blocks of 1 KB, block 2 * (chunk / 8) + (key % 16) / 8
// holding 8 keys x 128 contiguous bytes (chunks 8 * (chunk / 8) ..), so each
// global_load_lds instruction reads whole cache lines.  The 16-byte chunk
// order inside a key's 128 bytes is XOR-swizzled by key: for K so that 16
// consecutive keys at one chunk cover all 64 banks (the A-operand read), for
// V so that each 32-lane half of a transposed read (4 keys x 4 chunks x 2
// halves) does.
__device__ inline int line_kswz(int t) { return ((t >> 1) & 3) | ((t >> 3) << 2); }
__device__ inline int line_vswz(int t) { return 4 * ((t >> 1) & 1); }
__device__ inline int line_klds_off(int key, int ch) {
  const int t = key & 15;
  return (key >> 4) * 4096 + (2 * (ch >> 3) + (t >> 3)) * 1024 + (t & 7) * 128 + ((ch & 7) ^ line_kswz(t)) * 16;
}
__device__ inline int line_vlds_off(int key, int ch) {
  return (key >> 4) * 4096 + (2 * (ch >> 3) + ((key >> 3) & 1)) * 1024 + (key & 7) * 128 +
         ((ch & 7) ^ line_vswz(key & 7)) * 16;
}

// Max / sum of a value over the lane pair (l, l ^ 32): v_permlane32_swap
// exchanges the two 32-lane halves without going through LDS.
__device__ inline float pair_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float pair_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// O^T / l of a lane's query row to out (op: the row's first column).  Lane
// (row, hi) holds d = 32 dt + 8 bk + 4 hi + 0..3 in o[dt][4 bk ..].  With a
// 16-byte aligned output (p.out16) one v_permlane32_swap per word pair gives
// lane hi = 0 d = 32 dt + 16 b + 0..7 and lane hi = 1 d = 32 dt + 16 b +
// 8..15 (both lanes of a pair hold the same row): 16 contiguous bytes per
// lane, half the store instructions and half the partial cache-line writes
// of 8-byte stores.  Every lane of the wave calls it.
template <typename T>
__device__ inline void store_rows(const PrefillParams& p, T* op, const f32x16 (&o)[4], float inv, bool row_ok) {
  const int hi = (int)(threadIdx.x & 63) >> 5;
  if (p.out16) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        typename Elem<T>::v4 lo, up;  // d chunks bk = 2b and 2b + 1
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          lo[e] = (T)(o[dt][8 * b + e] * inv);
          up[e] = (T)(o[dt][8 * b + 4 + e] * inv);
        }
        const u32x2 lw = __builtin_bit_cast(u32x2, lo), uw = __builtin_bit_cast(u32x2, up);
        u32x4 wv;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const auto r = __builtin_amdgcn_permlane32_swap(lw[k], uw[k], false, false);
          wv[k] = r[0];
          wv[2 + k] = r[1];
        }
        if (row_ok) *reinterpret_cast<u32x4*>(op + 32 * dt + 16 * b + 8 * hi) = wv;
      }
  } else if (row_ok) {
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
}

// The same rows written as whole cache lines: the wavefront's 32 rows go
// through a 4 KB LDS area `stage`, 64 columns at a time, and come back so
// that each 16-byte store instruction covers 8 rows x 128 contiguous bytes.
// The stores are non-temporal: the output is not read again by the launch,
// and written as ordinary stores its lines displace K/V lines that other
// workgroups still read from L2.  rowp[j] and rok[j] are the output address
// (column 8 * (lane % 8)) and validity of wavefront row 8j + lane / 8.  The
// stage rows are 128 bytes, their 16-byte chunks XOR-swizzled by row / 2, so
// that the row-per-lane writes and the chunk-per-lane reads both cover all
// banks.  Requires 16-byte aligned output rows (PrefillParams::out16).
template <typename T>
__device__ inline void store_rows_staged(lds_u8* stage, const f32x16 (&o)[4], float inv, T* const (&rowp)[4],
                                         const bool (&rok)[4]) {
  const int lane = (int)(threadIdx.x & 63);
  const int ln = lane & 31, hi = lane >> 5;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
#pragma unroll
    for (int dd = 0; dd < 2; ++dd)
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const int dt = 2 * half + dd;
        typename Elem<T>::v4 lo, up;  // this lane's columns 32dt + 16b + 4hi + (0..3) and + 8
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          lo[e] = (T)(o[dt][8 * b + e] * inv);
          up[e] = (T)(o[dt][8 * b + 4 + e] * inv);
        }
        const u32x2 lw = __builtin_bit_cast(u32x2, lo), uw = __builtin_bit_cast(u32x2, up);
        u32x4 wv;  // columns 32dt + 16b + 8hi .. + 7
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const auto r = __builtin_amdgcn_permlane32_swap(lw[k], uw[k], false, false);
          wv[k] = r[0];
          wv[2 + k] = r[1];
        }
        const int c = 4 * dd + 2 * b + hi;  // 16-byte chunk of the 64 columns
        lds_st16<u32x4>(stage + ln * 128 + ((c ^ ((ln >> 1) & 7)) << 4), wv);
      }
    wave_lds_fence();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = 8 * j + (lane >> 3), c = lane & 7;
      const u32x4 v = lds_ld16<u32x4>(stage + row * 128 + ((c ^ ((row >> 1) & 7)) << 4));
      if (rok[j]) __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(rowp[j] + 64 * half));
    }
    wave_lds_fence();
  }
}

// Two probabilities rounded to the storage type and packed into one word.
template <typename T>
struct PackedPair;
template <>
struct PackedPair<__bf16> {
  typedef __bf16 x2 __attribute__((ext_vector_type(2)));
  __device__ static inline uint32_t pack(float a, float b) { return __builtin_bit_cast(uint32_t, x2{(__bf16)a, (__bf16)b}); }
};
template <>
struct PackedPair<_Float16> {
  typedef _Float16 x2 __attribute__((ext_vector_type(2)));
  __device__ static inline uint32_t pack(float a, float b) {
    return __builtin_bit_cast(uint32_t, x2{(_Float16)a, (_Float16)b});
  }
};

// One query tile of one prefill sequence, as the kernel needs it.  pg0 /
// pg1 are the calling wave's pages of 64-key tiles 0 and 1 (wave w reads page
// w of the 4 in a tile).
struct PrefillWork {
  int s, t0, q0, q_len, kv, ntiles, full_tiles, npages, pg0, pg1;
};

// Runs one prefill work item.  k0/k1 and v0/v1 must be four distinct
// __shared__ arrays of kPrefillTileBytes (distinct objects keep the compiler
// from treating reads of one buffer as dependent on DMAs into another).
template <typename T>
__device__ __attribute__((always_inline)) inline void prefill_core(const PrefillParams& p, const PrefillWork& wk,
                                                                   int h, lds_u8* k0, lds_u8* k1, lds_u8* v0,
                                                                   lds_u8* v1) {
  typedef typename Elem<T>::v8 V8;
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int ln = lane & 31;
  const int hi = lane >> 5;

  const int s = wk.s;
  const int t0 = wk.t0;
  const int q0 = wk.q0;
  const int q_len = wk.q_len;
  const int kv = wk.kv;
  const int G = p.group;
  const int BMT = p.tile_tokens;
  const int base_pos = kv - q_len;  // absolute position of query token 0

  // This lane's query row.
  const int R = 32 * w + ln;
  const int g = R / BMT;
  const int tq = t0 + R % BMT;
  const bool row_ok = g < G && tq < q_len;
  const int pos = row_ok ? base_pos + tq : -1;  // keys j <= pos are visible

  const int ntiles = wk.ntiles;
  const int full_tiles = wk.full_tiles;  // tiles no row masks

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
  const int npages = wk.npages;

  // Page id of this wave's page (page w of the 4 in a tile) of `tile`; pages
  // past the needed range clamp to the last needed page (masked later).
  auto page_of = [&](int tile) {
    const int pg = sload(bt, min(tile * (kPrefillKeys / kPageSize) + w, npages - 1));
    return (pg >= 0 && pg < p.num_pages) ? pg : 0;
  };
  // DMA of this wave's page of a K (or V) tile in the whole-line layouts:
  // lane -> token lane/8 (offset a) or 8 + lane/8 (offset b), chunk
  // (lane % 8) ^ swizzle(token) of the 128-byte half the copy reads.
  const uint32_t ts = (uint32_t)(p.tok_stride * (int64_t)sizeof(T));
  const int lt = lane >> 3;
  const uint32_t koff_a = (uint32_t)lt * ts + 16u * (uint32_t)((lane & 7) ^ line_kswz(lt));
  const uint32_t koff_b = (uint32_t)(8 + lt) * ts + 16u * (uint32_t)((lane & 7) ^ line_kswz(8 + lt));
  const uint32_t voff_a = (uint32_t)lt * ts + 16u * (uint32_t)((lane & 7) ^ line_vswz(lt));
  const uint32_t voff_b = (uint32_t)(8 + lt) * ts + 16u * (uint32_t)((lane & 7) ^ line_vswz(lt));
  auto dma_k = [&](int page, lds_u8* buf) {
    dma16_x4_lines(kc + (int64_t)page * p.page_stride, koff_a, koff_b, (uint32_t)(uintptr_t)(buf + 4096 * w));
  };
  auto dma_v = [&](int page, lds_u8* buf) {
    dma16_x4_lines(vc + (int64_t)page * p.page_stride, voff_a, voff_b, (uint32_t)(uintptr_t)(buf + 4096 * w));
  };

  // The pipeline is written in issue order as steps of one MFMA each, its
  // LDS operand read one step ahead, a few vector instructions of the
  // softmax beside it, and a scheduling barrier after it.  The matrix cores
  // and the vector ALU of a SIMD overlap only a few vector instructions per
  // MFMA; spreading the softmax evenly over the MFMAs of both phases keeps
  // it in the MFMA shadow instead of in a block of its own.
  //
  // Element i of S block mt: st[mt][i] = S[query ln][key 32*mt + 8*(i/4) +
  // 4*hi + i%4] (the C layout of S^T = K Q^T).  Its probability goes to PV
  // k-step kk = 2*mt + (i/4)/2, word ((i/4) % 2)*2 + (i%4)/2 of pw[kk] (two
  // packed values per word: the B layout of P^T).
  // QK step j: key 32*(j%2) + ln, chunk 2*(j/2) + hi; the swizzle makes the
  // address a per-lane base (one per (j/2) % 4) plus an immediate.
  int kbase[4];
#pragma unroll
  for (int c4 = 0; c4 < 4; ++c4) kbase[c4] = line_klds_off(ln, 2 * c4 + hi);
  auto kread = [&](const lds_u8* kb, int j) {  // QK step j: chain j % 2, k-step j / 2
    return lds_ld16<V8>(kb + kbase[(j >> 1) & 3] + 8192 * (j & 1) + 2048 * (j >> 3));
  };
  // PV step j: k-step j / 4, d-tile j % 4.  16-lane group a = lane/16 covers
  // d offset 16*(a&1) of the 32-d tile and keys 4*hi.. of each 8-key block;
  // supplier lane ti gives row 4*hi + ti/4 at d offset 4*(ti%4), chunk
  // 4*(j%4) + 2*(a&1) + (ti/2)%2 (two per-lane bases, by j % 2), and the
  // same lanes give rows 8.. from the next block.
  const int ti = lane & 15;
  const int dgrp = (lane >> 4) & 1;
  const int vkey = 4 * hi + (ti >> 2);
  const int vch = (2 * dgrp + ((ti >> 1) & 1)) ^ line_vswz(vkey);
  const int vbase0 = vkey * 128 + vch * 16 + (ti & 1) * 8;
  const int vbase1 = vkey * 128 + (vch ^ 4) * 16 + (ti & 1) * 8;
  auto vread = [&](const lds_u8* vb, int j) {
    const lds_u8* a = vb + ((j & 1) ? vbase1 : vbase0) + (j >> 2) * 4096 + ((j >> 1) & 1) * 2048;
    return __builtin_bit_cast(V8, __builtin_shufflevector(lds_ld_tr16(a), lds_ld_tr16(a + 1024), 0, 1, 2, 3, 4, 5, 6,
                                                          7));
  };

  f32x16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = f32x16{};
  float m = -INFINITY;  // reference max (log2 units) of the tiles so far
  float l = 0.f;        // row sum of P, relative to m
  float m_use = 0.f;    // m, or 0 while no key is visible
  float alpha = 1.0f;   // O rescale factor of the tile whose P is computed next
  float tmax = -INFINITY;

  // Probabilities of element pair q (elements 2q, 2q + 1 of the 32 a lane
  // holds), in three stages one step apart so that no stage waits on the
  // latency of the previous one: (A) the exponents S * scale - m, (B) their
  // exp2, (C) the packed pair into pw and the row sums.  (Two v_add cost less
  // than a v_dot2 of the packed pair beside the MFMAs.)
  // la / lb: this tile's sums of the even / odd elements, added to l once
  // the tile's last pair is done (the same order as the ping-pong kernel, so
  // the two kernels agree bit for bit).
  float px[16][2], pe[16][2], la = 0.f, lb = 0.f;
  auto pair_a = [&](const f32x16 (&st)[2], int q) {
    const int mt = q >> 3, i = 2 * (q & 7);
    px[q][0] = st[mt][i] * p.scale_log2 - m_use;
    px[q][1] = st[mt][i + 1] * p.scale_log2 - m_use;
  };
  auto pair_b = [&](int q) {
    pe[q][0] = fast_exp2(px[q][0]);
    pe[q][1] = fast_exp2(px[q][1]);
  };
  auto pair_c = [&](u32x4 (&pw)[4], int q) {
    const int mt = q >> 3, i = 2 * (q & 7);
    pw[2 * mt + (q & 7) / 4][((i >> 2) & 1) * 2 + ((i & 3) >> 1)] = PackedPair<T>::pack(pe[q][0], pe[q][1]);
    la += pe[q][0];
    lb += pe[q][1];
    if (q == 15) {
      l += la + lb;
      la = 0.f;
      lb = 0.f;
    }
  };
  // Mask and running max of four elements (4c .. 4c + 3) of the next tile's S.
  auto max4 = [&](f32x16 (&st)[2], int c, int tile, auto masked_tag) {
    const int mt = c >> 2, i0 = 4 * (c & 3);
    if constexpr (decltype(masked_tag)::value) {
      // Key tile*64 + 32*mt + 8*(i/4) + 4*hi + i%4 is visible when
      // 32*mt + 8*(i/4) + i%4 <= lim.
      const int lim = pos - tile * kPrefillKeys - 4 * hi;
#pragma unroll
      for (int i = i0; i < i0 + 4; ++i)
        if (32 * mt + 8 * (i >> 2) + (i & 3) > lim) st[mt][i] = -INFINITY;
    }
    // IEEE maximum (NaN-propagating, v_maximum3_f32) needs no quieting of
    // its MFMA-produced inputs, unlike fmaxf.
    const float m3 = __builtin_elementwise_maximum(__builtin_elementwise_maximum(st[mt][i0], st[mt][i0 + 1]),
                                                   st[mt][i0 + 2]);
    tmax = __builtin_elementwise_maximum(__builtin_elementwise_maximum(tmax, m3), st[mt][i0 + 3]);
    asm volatile("" : "+v"(tmax));  // keeps this part of the max at its step
  };
  // Reference-max update from tmax: the max is only moved when it grows by
  // more than 8 (log2 units), so P stays <= 2^8 and most tiles skip the O
  // rescale (alpha exactly 1).
  auto max_update = [&]() {
    const float tmax_s = pair_max(tmax) * p.scale_log2;  // scale > 0 commutes with max
    tmax = -INFINITY;
    const bool grow = tmax_s > m + 8.0f;
    const float m_new = grow ? tmax_s : m;
    alpha = grow ? fast_exp2(m - m_new) : 1.0f;  // m = -inf -> 0
    m = m_new;
    l *= alpha;
    m_use = (m == -INFINITY) ? 0.f : m;
  };
  auto rescale = [&]() {
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) o[dt] *= alpha;
    }
  };

  // Zero V rows of keys >= kv in the last tile (stale rows may hold NaN and
  // 0 * NaN would leak through P = 0).
  auto zero_tail = [&](int tile, lds_u8* vb) {
    const int first_bad = kv - tile * kPrefillKeys;  // rows >= first_bad are past the sequence
    for (int i = tid; i < (kPrefillKeys - first_bad) * 16; i += 256) {
      const int key = first_bad + (i >> 4);
      lds_st16<u32x4>(vb + line_vlds_off(key, i & 15), u32x4{0, 0, 0, 0});
    }
  };

  // Prologue: K(0), K(1), V(0) in flight, then S(0) and its max.
  int pg_v = __builtin_amdgcn_readfirstlane(wk.pg1);  // page of V(t+1) at iteration t (= page of K(t+1))
  {
    const int pg0 = __builtin_amdgcn_readfirstlane(wk.pg0);
    dma_k(pg0, k0);
    if (ntiles > 1) dma_k(pg_v, k1);
    dma_v(pg0, v0);
  }
  int pg_k = page_of(2);  // page of K(t+2) at iteration t
  __builtin_amdgcn_s_waitcnt(kVmcnt0);
  __syncthreads();
  f32x16 st_a[2], st_b[2];  // S(t) lives in st_a for even t, st_b for odd t
  {
    st_a[0] = f32x16{};
    st_a[1] = f32x16{};
#pragma unroll
    for (int j = 0; j < 16; ++j) st_a[j & 1] = Elem<T>::mfma32(kread(k0, j), qf[j >> 1], st_a[j & 1]);
    const bool masked0 = full_tiles == 0;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      if (masked0) max4(st_a, c, 0, std::true_type{});
      else max4(st_a, c, 0, std::false_type{});
    }
    max_update();
  }

  // Iteration t.  kb_cur holds K(t) (free: S(t) is done) and receives
  // K(t+2); kb_next holds K(t+1); vb_cur holds V(t); vb_next receives V(t+1);
  // st_cur holds S(t), already masked with its max taken, and st_next
  // receives S(t+1).  Without a next tile (has_next false) the S(t+1) MFMAs
  // and its max are left out.
  auto iteration = [&](int t, lds_u8* kb_cur, lds_u8* kb_next, lds_u8* vb_cur, lds_u8* vb_next,
                       f32x16 (&st_cur)[2], f32x16 (&st_next)[2], auto masked_next_tag, auto has_next_tag) {
    constexpr bool has_next = decltype(has_next_tag)::value;
    __builtin_amdgcn_s_waitcnt(kVmcnt0);
    __syncthreads();  // K(t+1), V(t) landed for all waves; S(t) and PV(t-1) done everywhere
    if (t == ntiles - 1 && (t + 1) * kPrefillKeys > kv) {
      zero_tail(t, vb_cur);
      __syncthreads();
    }
    if (t + 2 < ntiles) dma_k(pg_k, kb_cur);
    if (t + 1 < ntiles) dma_v(pg_v, vb_next);
    pg_v = pg_k;
    pg_k = page_of(t + 3);
    rescale();  // O *= alpha(t) before P(t) V(t) accumulates
    __builtin_amdgcn_sched_barrier(0);

    // 32 steps: 0..15 the S(t+1) MFMAs (kread one step ahead), 16..31 the
    // P(t)V(t) MFMAs (vread one step ahead; k-step kk from step 16 + 4kk).
    // Pair q of P(t) runs stage A at step (3q)/2, B and C on the two steps
    // after it, so k-step kk's pairs are packed before step 16 + 4kk; the
    // mask and max of S(t+1) run on steps 24..31, and its reference-max
    // update after them.
    u32x4 pw[4];
    V8 kf[2], vf[2];
    if constexpr (has_next) {
      kf[0] = kread(kb_next, 0);
      st_next[0] = f32x16{};
      st_next[1] = f32x16{};
    }
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      if (j < 16) {
        if constexpr (has_next) {
          if (j + 1 < 16) kf[(j + 1) & 1] = kread(kb_next, j + 1);
          st_next[j & 1] = Elem<T>::mfma32(kf[j & 1], qf[j >> 1], st_next[j & 1]);
        }
        if (j == 15) vf[0] = vread(vb_cur, 0);
      } else {
        const int v = j - 16;
        if (v + 1 < 16) vf[(v + 1) & 1] = vread(vb_cur, v + 1);
        o[v & 3] = Elem<T>::mfma32(vf[v & 1], __builtin_bit_cast(V8, pw[v >> 2]), o[v & 3]);
      }
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int sa = (3 * q) >> 1;
        if (j == sa) pair_a(st_cur, q);
        if (j == sa + 1) pair_b(q);
        if (j == sa + 2) pair_c(pw, q);
      }
      if constexpr (has_next) {
        if (j >= 24) max4(st_next, j - 24, t + 1, masked_next_tag);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (has_next) max_update();
  };

  // Iterations [t, t_stop), each with a next tile, its S masked iff the tag
  // says so.  Unrolled by two so each iteration body names its LDS buffers
  // and S registers statically.
  const std::true_type yes;
  const std::false_type no;
  auto run = [&](int t, int t_stop, auto masked_next_tag) {
    if (t < t_stop && (t & 1)) iteration(t++, k1, k0, v1, v0, st_b, st_a, masked_next_tag, yes);
    for (; t + 1 < t_stop; t += 2) {
      iteration(t, k0, k1, v0, v1, st_a, st_b, masked_next_tag, yes);
      iteration(t + 1, k1, k0, v1, v0, st_b, st_a, masked_next_tag, yes);
    }
    if (t < t_stop) iteration(t, k0, k1, v0, v1, st_a, st_b, masked_next_tag, yes);
  };
  // Tile t + 1 is below every row's causal bound iff t + 1 < full_tiles.
  const int t_split = max(min(full_tiles - 1, ntiles - 1), 0);
  run(0, t_split, no);
  run(t_split, ntiles - 1, yes);
  if ((ntiles - 1) & 1) iteration(ntiles - 1, k1, k0, v1, v0, st_b, st_a, no, no);
  else iteration(ntiles - 1, k0, k1, v0, v1, st_a, st_b, no, no);

  // Epilogue: O^T / l -> out[token][head][d].
  const float l_tot = pair_sum(l);
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  T* op = (T*)p.out + (int64_t)(q0 + tq) * p.out_tok_stride + (int64_t)(h * G + g) * p.out_head_stride;
  store_rows<T>(p, op, o, inv, row_ok);
}


// ---- exact, device-built tile list and the persistent prefill launch -------
//
// Plan buffer (int32): a header (tile count and per-head claim counters),
// then the tiles from word kPrefillPlanHeaderInts, kPrefillPlanItemInts words
// each:
//   {seq, t0, q0, q_len, kv, ntiles, full_tiles, npages,
//    page ids of 64-key tile 0 (4 pages), of tile 1 (4 pages)}
// for the BMT-token query tile [t0, t0 + BMT) of prefill sequence `seq`
// (query rows q0 .. q0 + q_len - 1, kv keys), which needs `ntiles` 64-key
// tiles (`npages` pages), the first `full_tiles` of them below every row's
// causal bound.  Page ids past npages repeat the last page; ids outside the
// cache read as page 0.
constexpr int kPrefillPlanItemInts = 16;
// Header: word 0 = tile count (at most the capacity); word 1 = tiles of the
// batch beyond the capacity, which are not run (0 when the capacity bounds
// the batch); word 16 = workgroups of the running launch that have finished;
// word 17 = workgroups of the launches that stream the plan; the claim
// counter of KV head h at word kPrefillPlanLineInts * (1 + h), each on its
// own 128-byte line.  The planner zeroes the counters and the last
// workgroup of every launch zeroes them again, so one plan serves any number
// of launches in stream order.
constexpr int kPrefillPlanDroppedInt = 1;
constexpr int kPrefillPlanExitInt = 16;
constexpr int kPrefillPlanGridInt = 17;
constexpr int kPrefillPlanLineInts = 32;
constexpr int kPrefillPlanMaxHeads = 127;
constexpr int kPrefillPlanHeaderInts = kPrefillPlanLineInts * (1 + kPrefillPlanMaxHeads);
// Largest batch the planner sorts longest-context first (a larger batch is
// planned in batch order).
constexpr int kPrefillPlanSortMax = 2048;

// The tile list mva_paged_prefill builds on the device: the record of tile
// i at word kPrefillPlanHeaderInts + i * kPrefillPlanItemInts (see
// kPrefillPlanHeaderInts), read with one scalar load.
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(4))) const i32x16 const_i32x16;

}  // namespace mva
