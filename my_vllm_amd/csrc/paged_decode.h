// Paged GQA decode: one wavefront per (sequence chunk, KV head) work item.
//
// Replaces FlashInfer's BatchDecodeWithPagedKVCacheWrapper.run on the DECODE
// route of the reference backend (nanovllm/layers/attention_backend.py:995-997)
// and the decode slice of MIXED_SPLIT (:1020-1025).  Math per query head:
//   o = sum_j softmax_j(scale * q . K[j]) V[j]   over j < seq_len,
// with K/V gathered from NHD pages [P, 16, Hkv, D] through block_tables.
//
// Layout of the work (one 64-lane wavefront per item):
//  * The G query heads that share a KV head form the N=16 side of the
//    16x16x32 MFMA (rows >= G are zero), so every K/V byte read from HBM serves
//    all G heads: S^T[token, g] = K[token, :] . Q[g, :].
//  * A tile is 2 pages (32 tokens).  K goes straight from HBM into MFMA
//    A-operand registers (lane = token, 16-byte d-chunks).  V goes from HBM
//    straight into LDS (global_load_lds, row-major, XOR-swizzled 16-byte
//    chunks, double-buffered) and is read back transposed with
//    ds_read_b64_tr_b16 as the A operand of O^T[d, g] += V^T[d, t] P^T[t, g];
//    the C layout of S^T is already the B-operand layout of P^T.
//  * Online softmax in the log2 domain, fp32 accumulators, P rounded to the
//    storage type for the PV MFMA.
//  * Long contexts are split into chunks (split-K).  Each chunk writes an fp32
//    partial (o / l, log2-sum-exp); the last chunk of a (sequence, KV head) to
//    finish, detected with a device-scope counter, merges the partials, so one
//    launch produces the final output.  Counters are reset by the merger, so
//    the workspace only has to be zeroed when first allocated.
#pragma once

#include "mva_common.h"

#include <type_traits>

namespace mva {

constexpr int kHeadDim = 128;
constexpr int kPageSize = 16;
// Bytes of one LDS V buffer of decode_item (two 16-token pages); decode_item
// takes two such buffers (double buffering), which should be distinct
// __shared__ arrays so the compiler can tell their LDS-DMA writes apart.
constexpr int kDecodeVBufBytes = 2 * kPageSize * kHeadDim * 2;
// Longest chunk (pages) one decode work item may cover.
constexpr int kMaxChunkPages = 128;
// int32 fields per decode work item (see make_decode_items on the host).
constexpr int kDecodeItemInts = 8;

// s_waitcnt immediates (gfx9 encoding: vmcnt bits [3:0] and [15:14], expcnt
// [6:4], lgkmcnt [11:8]); only vmcnt is constrained.
constexpr int waitcnt_vm(int n) { return (n & 0xf) | ((n >> 4) << 14) | (0x7 << 4) | (0xf << 8); }
// One tile issues 16 vector-memory instructions (8 K loads, 8 V LDS loads).
constexpr int kVmcntTile = waitcnt_vm(16);
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
  const int32_t* items;  // [num_items][8]: seq, page_begin, page_end, chunk, n_chunks, part_base, q_row, 0
  int num_items;
  void* out;
  int64_t out_tok_stride;
  int64_t out_head_stride;
  int32_t* counters;  // [num_seqs][Hkv]
  float* part_lse;    // [slots][Hkv][G]
  float* part_o;      // [slots][Hkv][G][D]
  int num_kv_heads;
  int group;  // query heads per KV head, 1..16
  float scale_log2;
};

template <typename T>
struct DecodeTile {
  typedef typename Elem<T>::v8 V8;
  V8 k[2][4];  // k[pp][j] = K[page pp][token c][32*q4 + 8*j .. +8]
};

__device__ inline float wave_max16(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}
__device__ inline float wave_sum16(float x) {
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}

// Swizzled byte offset of 16-byte chunk `ch` of token row `t` in a V page
// staged in LDS: rows are 256 bytes, chunks are XOR-ed with 2*(t & 7) so that
// the transposed reads of 16 token rows hit distinct banks.
__device__ inline int vlds_off(int t, int ch) { return t * 256 + ((ch ^ ((t & 7) << 1)) << 4); }

// Issues the loads of one tile (pages `page0`, `page1`): K into MFMA A-operand
// registers and V straight from HBM into LDS (gfx950 global_load_lds, 16 bytes
// per lane, no registers), laid out by vlds_off.  Instruction i of page pp
// fills LDS bytes [pp*4096 + 1024*i, +1024): token row 4*i + lane/16, physical
// chunk lane%16.  16 vector-memory instructions per tile.
template <typename T>
__device__ inline void decode_load_tile(const DecodeParams& p, const T* kc, const T* vc, int page0,
                                        int page1, int lane, DecodeTile<T>& tile, lds_u8* vlds) {
  typedef typename Elem<T>::v8 V8;
  const int q4 = lane >> 4;
  const int c = lane & 15;
#pragma unroll
  for (int pp = 0; pp < 2; ++pp) {
    const int page = pp ? page1 : page0;
    const T* kp = kc + (int64_t)page * p.page_stride;
    const T* vp = vc + (int64_t)page * p.page_stride;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 4 * i + q4;
      const int ch = c ^ ((t & 7) << 1);
      dma16(vp + t * p.tok_stride + 8 * ch, vlds + pp * 4096 + 1024 * i);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) tile.k[pp][j] = ld16<V8>(kp + c * p.tok_stride + 32 * q4 + 8 * j);
  }
}

template <typename T>
__device__ void decode_item(const DecodeParams& p, const int32_t* __restrict__ it, int h,
                            lds_u8* vbuf0, lds_u8* vbuf1) {
  typedef typename Elem<T>::v8 V8;
  const int lane = threadIdx.x & 63;
  const int q4 = lane >> 4;
  const int c = lane & 15;
  const int s = it[0], pb = it[1], pe = it[2], chunk = it[3], nchunks = it[4], pbase = it[5];
  const int64_t qrow = it[6];
  const int G = p.group;
  const int seq_len = p.seq_lens[s];
  const T* kc = (const T*)p.k_cache + h * kHeadDim;
  const T* vc = (const T*)p.v_cache + h * kHeadDim;
  const int32_t* bt = p.block_tables + (int64_t)s * p.bt_stride;

  // Q as the B operand of S^T = K Q^T: lane (q4, c) holds Q[g = c][32*q4 + 8*j .. +8].
  V8 qf[4];
  if (c < G) {
    const T* qp = (const T*)p.q + qrow * p.q_tok_stride + (int64_t)(h * G + c) * p.q_head_stride + 32 * q4;
#pragma unroll
    for (int j = 0; j < 4; ++j) qf[j] = ld16<V8>(qp + 8 * j);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) qf[j] = V8{};
  }

  f32x4 o[8];  // o[mt][r] = O^T[d = 16*mt + 4*q4 + r][g = c]
#pragma unroll
  for (int mt = 0; mt < 8; ++mt) o[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY;  // running max of scaled scores (log2 domain), per g = c
  float l = 0.f;        // this lane's share of the running denominator

  const int ntiles = (pe - pb + 1) >> 1;
  // Transposed V^T reads: lane c of group q4 supplies token row 4*q4 + c/4 at
  // d offset 4*(c%4) of each 16-wide d block and receives V[4*q4 + e][16*mt + c].
  const int tt = 4 * q4 + (c >> 2);
  const int dsub = (c & 3) * 4;

  // `edge` tiles contain masked tokens (sequence end, or an odd page past the
  // chunk end); the choice is wave-uniform and made per tile by `run`.
  auto compute = [&](int t, const DecodeTile<T>& tile, const lds_u8* vbuf, auto edge_tag) {
    constexpr bool edge = decltype(edge_tag)::value;
    const int pg0 = pb + 2 * t;
    f32x4 sc[2];
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
      sc[pp] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) sc[pp] = Elem<T>::mfma16(tile.k[pp][j], qf[j], sc[pp]);
    }
    float x[2][4];
    float tmax = -INFINITY;
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        x[pp][r] = sc[pp][r] * p.scale_log2;
        if constexpr (edge) {
          const int pos = (pg0 + pp) * kPageSize + 4 * q4 + r;
          if ((pg0 + pp) >= pe || pos >= seq_len) x[pp][r] = -INFINITY;
        }
        tmax = fmaxf(tmax, x[pp][r]);
      }
    }
    tmax = wave_max16(tmax);
    const float m_new = fmaxf(m, tmax);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = fast_exp2(m - m_use);
    m = m_new;
    V8 pf;
    float psum = 0.f;
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float pr = fast_exp2(x[pp][r] - m_use);
        psum += pr;
        pf[pp * 4 + r] = (T)pr;
      }
    }
    l = l * alpha + psum;
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) o[mt] *= alpha;

    // Element e of the page-pp half of a V^T fragment is token 4*q4 + e.
    unsigned vmask = 0xffu;  // bit pp*4+e set = token valid
    if constexpr (edge) {
      vmask = 0;
#pragma unroll
      for (int pp = 0; pp < 2; ++pp)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int pos = (pg0 + pp) * kPageSize + 4 * q4 + e;
          if ((pg0 + pp) < pe && pos < seq_len) vmask |= 1u << (pp * 4 + e);
        }
    }
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) {
      const int d = 16 * mt + dsub;
      const int off = vlds_off(tt, d >> 3) + (d & 7) * 2;
      const s16x4 lo = lds_ld_tr16(vbuf + off);
      const s16x4 hi = lds_ld_tr16(vbuf + 4096 + off);
      s16x8 both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      if constexpr (edge) {
        // Zero V of masked tokens so stale (possibly NaN) cache rows cannot
        // leak through 0 * NaN in the PV product.
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (!((vmask >> e) & 1u)) both[e] = 0;
      }
      o[mt] = Elem<T>::mfma16(__builtin_bit_cast(V8, both), pf, o[mt]);
    }
  };

  // The chunk's page table lives in two VGPRs (lane i: pages i and 64 + i of
  // the chunk; chunks are at most kMaxChunkPages long) and is read with
  // v_readlane, so the tile loop issues no dependent memory reads.
  const int np = pe - pb;
  const int bt_lo = lane < np ? bt[pb + lane] : 0;
  const int bt_hi = lane + 64 < np ? bt[pb + 64 + lane] : 0;
  auto page_at = [&](int k) -> int {
    const int a = __builtin_amdgcn_readlane(bt_lo, k & 63);
    const int b = __builtin_amdgcn_readlane(bt_hi, k & 63);
    const int pg = k < 64 ? a : b;
    return (pg >= 0 && pg < p.num_pages) ? pg : 0;
  };
  // Tile t covers chunk pages 2t and 2t+1; a missing odd page and the
  // prefetch past the last tile re-read pages already in flight (cache hits)
  // and are masked or ignored, so every iteration issues the same loads.
  auto load = [&](int t, DecodeTile<T>& tile, lds_u8* vbuf) {
    t = t < ntiles ? t : ntiles - 1;
    const int k0 = 2 * t;
    const int k1 = (2 * t + 1 < np) ? 2 * t + 1 : 2 * t;
    decode_load_tile<T>(p, kc, vc, page_at(k0), page_at(k1), lane, tile, vbuf);
  };
  auto run = [&](int t, const DecodeTile<T>& tile, const lds_u8* vbuf) {
    const int pg0 = pb + 2 * t;
    if ((pg0 + 2 > pe) || ((pg0 + 2) * kPageSize > seq_len)) compute(t, tile, vbuf, std::true_type{});
    else compute(t, tile, vbuf, std::false_type{});
  };

  if (ntiles > 0) {
    DecodeTile<T> ta, tb;
    load(0, ta, vbuf0);
    for (int t = 0; t < ntiles; t += 2) {
      load(t + 1, tb, vbuf1);
      __builtin_amdgcn_s_waitcnt(kVmcntTile);
      wave_lds_fence();
      run(t, ta, vbuf0);
      wave_lds_fence();
      load(t + 2, ta, vbuf0);
      __builtin_amdgcn_s_waitcnt(kVmcntTile);
      wave_lds_fence();
      if (t + 1 < ntiles) run(t + 1, tb, vbuf1);
      wave_lds_fence();
    }
    // Drain the final prefetch: LDS writes must land before the wave exits.
    __builtin_amdgcn_s_waitcnt(kVmcnt0);
  }

  const float l_tot = wave_sum16(l);
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  const int Hkv = p.num_kv_heads;
  if (nchunks == 1) {
    if (c < G) {
      T* op = (T*)p.out + qrow * p.out_tok_stride + (int64_t)(h * G + c) * p.out_head_stride + 4 * q4;
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) {
        typename Elem<T>::v4 w;
#pragma unroll
        for (int r = 0; r < 4; ++r) w[r] = (T)(o[mt][r] * inv);
        *reinterpret_cast<typename Elem<T>::v4*>(op + 16 * mt) = w;
      }
    }
    return;
  }

  // Split-K: publish this chunk's normalised partial and log2-sum-exp with
  // device-scope stores (written through past this XCD's L2), drain them,
  // then count the chunk in.  This avoids a full L2 write-back/invalidate
  // (what a device-scope fence costs on a multi-XCD part) per chunk.
  const int64_t slot = (int64_t)(pbase + chunk) * Hkv + h;
  if (c < G) {
    float* po = p.part_o + (slot * G + c) * kHeadDim + 4 * q4;
#pragma unroll
    for (int mt = 0; mt < 8; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        __hip_atomic_store(po + 16 * mt + r, o[mt][r] * inv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (q4 == 0)
      __hip_atomic_store(&p.part_lse[slot * G + c], l_tot > 0.f ? m + fast_log2(l_tot) : -INFINITY,
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  int prev = 0;
  if (lane == 0)
    prev = __hip_atomic_fetch_add(&p.counters[(int64_t)s * Hkv + h], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  prev = __shfl(prev, 0);
  if (prev != nchunks - 1) return;

  // Last chunk to arrive: merge all partials of this (sequence, KV head);
  // device-scope loads read them from past the (per-XCD) L2.
  const int d = 2 * lane;
  for (int g = 0; g < G; ++g) {
    float mx = -INFINITY;
    for (int k = 0; k < nchunks; ++k) {
      const float lse = __hip_atomic_load(&p.part_lse[((int64_t)(pbase + k) * Hkv + h) * G + g],
                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      mx = fmaxf(mx, lse);
    }
    float a0 = 0.f, a1 = 0.f, wsum = 0.f;
    if (mx != -INFINITY) {
      for (int k = 0; k < nchunks; ++k) {
        const int64_t sl = ((int64_t)(pbase + k) * Hkv + h) * G + g;
        const float lse = __hip_atomic_load(&p.part_lse[sl], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const float w = fast_exp2(lse - mx);
        const float* po = p.part_o + sl * kHeadDim + d;
        a0 += w * __hip_atomic_load(po, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        a1 += w * __hip_atomic_load(po + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        wsum += w;
      }
    }
    const float winv = wsum > 0.f ? 1.0f / wsum : 0.f;
    T* op = (T*)p.out + qrow * p.out_tok_stride + (int64_t)(h * G + g) * p.out_head_stride + d;
    op[0] = (T)(a0 * winv);
    op[1] = (T)(a1 * winv);
  }
  if (lane == 0)
    __hip_atomic_store(&p.counters[(int64_t)s * Hkv + h], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace mva
