// Shared device helpers for the gfx950 (MI355X, CDNA4) kernels of this library.
//
// Everything here is written for one target: 64-lane wavefronts, bf16/fp16
// MFMA through the gfx950 builtins, and 16-byte global/LDS accesses.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace mva {

// Element codes shared with the host side (include/my_vllm_amd.h).
enum DType : int { kBF16 = 0, kF16 = 1, kF32 = 2 };

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Per-element-type traits: the 8-wide vector used as an MFMA operand and the
// matching gfx950 MFMA instructions (fp32 accumulate).
template <typename T>
struct Elem;

typedef short s16x4_t __attribute__((ext_vector_type(4)));

template <>
struct Elem<__bf16> {
  typedef bf16x8 v8;
  typedef bf16x4 v4;
  // 16x16x16 (K = 16): A/B hold 4 elements per lane (k = 4*(lane/16) + s).
  __device__ static inline f32x4 mfma16k16(v4 a, v4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, a),
                                                     __builtin_bit_cast(s16x4_t, b), c, 0, 0, 0);
  }
  __device__ static inline f32x4 mfma16(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static inline f32x16 mfma32(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Elem<_Float16> {
  typedef f16x8 v8;
  typedef f16x4 v4;
  __device__ static inline f32x4 mfma16k16(v4 a, v4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
  }
  __device__ static inline f32x4 mfma16(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  __device__ static inline f32x16 mfma32(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// 16-byte load/store of an 8-element vector; callers guarantee alignment.
template <typename V>
__device__ inline V ld16(const void* p) {
  return *reinterpret_cast<const V*>(p);
}
template <typename V>
__device__ inline void st16(void* p, V v) {
  *reinterpret_cast<V*>(p) = v;
}

// LDS (address space 3) byte pointer.  Kernels pass LDS buffers around with
// this type so every access compiles to ds_* instructions (a generic pointer
// would compile to flat_* loads with 64-bit addresses).
typedef __attribute__((address_space(3))) uint8_t lds_u8;

template <typename V>
__device__ inline V lds_ld16(const lds_u8* p) {
  return *reinterpret_cast<const __attribute__((address_space(3))) V*>(p);
}
template <typename V>
__device__ inline void lds_st16(lds_u8* p, V v) {
  *reinterpret_cast<__attribute__((address_space(3))) V*>(p) = v;
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));

// ds_read_b64_tr_b16: within each 16-lane group, lane j receives element j%4
// of the 8-byte rows supplied by lanes 4e + j/4 (e = 0..3); i.e. if lane i
// points at row i/4, columns 4*(i%4)..+3 of a 4 x 16 block of 16-bit values,
// lane j gets column j of the block.
__device__ inline s16x4 lds_ld_tr16(const lds_u8* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)p);
}

// Eight ds_read_b64_tr_b16: i = 0..3 at b[i], i = 4..7 at b[i - 4] + 2048,
// then lgkmcnt(0).  Issued as one asm block: the compiler cannot see that
// these reads do not alias in-flight global_load_lds writes to another LDS
// buffer and would otherwise wait for every outstanding DMA before each
// read.  Callers order the block after the waits that make the bases valid.
__device__ inline void lds_ld_tr16_x8_4base(const lds_u8* b0, const lds_u8* b1, const lds_u8* b2, const lds_u8* b3,
                                             s16x4 (&out)[8]) {
  asm volatile(
      "ds_read_b64_tr_b16 %0, %8\n"
      "ds_read_b64_tr_b16 %1, %9\n"
      "ds_read_b64_tr_b16 %2, %10\n"
      "ds_read_b64_tr_b16 %3, %11\n"
      "ds_read_b64_tr_b16 %4, %8 offset:2048\n"
      "ds_read_b64_tr_b16 %5, %9 offset:2048\n"
      "ds_read_b64_tr_b16 %6, %10 offset:2048\n"
      "ds_read_b64_tr_b16 %7, %11 offset:2048\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(out[0]), "=&v"(out[1]), "=&v"(out[2]), "=&v"(out[3]), "=&v"(out[4]), "=&v"(out[5]),
        "=&v"(out[6]), "=&v"(out[7])
      : "v"((uint32_t)(uintptr_t)b0), "v"((uint32_t)(uintptr_t)b1), "v"((uint32_t)(uintptr_t)b2),
        "v"((uint32_t)(uintptr_t)b3)
      : "memory");
}

// Four 1 KB global -> LDS copies from a uniform base: copy c moves 16 bytes
// per lane from base + 64*c + voff to LDS byte address lds + 1024*c + 16*lane.
// Written as one asm block so the scalar base + 32-bit lane offset form is
// used (no 64-bit per-lane addresses) and M0 is restored afterwards.  The
// instruction's immediate offset would also move the LDS destination, so each
// copy gets its own scalar base instead.  The s_nop after each M0 write is
// the wait state an LDS DMA needs after an SALU write of M0.  The compiler
// does not track these loads: callers wait for them (vmcnt) and synchronize
// before reading the LDS they fill.
__device__ inline void dma16_x4_saddr(const void* base, uint32_t voff, uint32_t lds) {
  uint32_t m0_saved;
  const char* b = (const char*)base;
  lds = __builtin_amdgcn_readfirstlane(lds);
  asm volatile(
      "s_mov_b32 %[m0s], m0\n\t"
      "s_mov_b32 m0, %[l]\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %[vo], %[b0]\n\t"
      "s_add_u32 m0, %[l], 0x400\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %[vo], %[b1]\n\t"
      "s_add_u32 m0, %[l], 0x800\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %[vo], %[b2]\n\t"
      "s_add_u32 m0, %[l], 0xc00\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %[vo], %[b3]\n\t"
      "s_mov_b32 m0, %[m0s]"
      : [m0s] "=&s"(m0_saved)
      : [l] "s"(lds), [vo] "v"(voff), [b0] "s"(b), [b1] "s"(b + 64), [b2] "s"(b + 128), [b3] "s"(b + 192)
      : "memory", "scc");
}

// The same four copies for a page read as whole 128-byte lines: copy c moves
// 16 bytes per lane from base + 128*(c/2) + (c%2 ? voff_b : voff_a) to LDS
// byte address lds + 1024*c + 16*lane (voff_a addressing tokens 0-7 of a
// page, voff_b tokens 8-15, 8 lanes per 128-byte line).
__device__ inline void dma16_x4_lines(const void* base, uint32_t voff_a, uint32_t voff_b, uint32_t lds) {
  uint32_t m0_saved;
  const char* b = (const char*)base;
  lds = __builtin_amdgcn_readfirstlane(lds);
  asm volatile(
      "s_mov_b32 %[m0s], m0\n\t"
      "s_mov_b32 m0, %[l]\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %[va], %[b0]\n\t"
      "s_add_u32 m0, %[l], 0x400\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %[vb], %[b0]\n\t"
      "s_add_u32 m0, %[l], 0x800\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %[va], %[b1]\n\t"
      "s_add_u32 m0, %[l], 0xc00\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %[vb], %[b1]\n\t"
      "s_mov_b32 m0, %[m0s]"
      : [m0s] "=&s"(m0_saved)
      : [l] "s"(lds), [va] "v"(voff_a), [vb] "v"(voff_b), [b0] "s"(b), [b1] "s"(b + 128)
      : "memory", "scc");
}

// 16-byte global -> LDS copy; lane i's bytes land at lds_base + 16*i.
__device__ inline void dma16(const void* g, lds_u8* lds_base) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds_base, 16, 0, 0);
}

// As dma16, with cache-policy bits `Policy` (e.g. device-scope coherence).
template <int Policy>
__device__ inline void dma16_policy(const void* g, lds_u8* lds_base) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds_base, 16, 0, Policy);
}

template <typename V>
__device__ inline V lds_ld8(const lds_u8* p) {
  return *reinterpret_cast<const __attribute__((address_space(3))) V*>(p);
}

// Compiler-level ordering point for LDS traffic that is shared between lanes
// of one wavefront.  LDS instructions of a wavefront execute in issue order,
// so only the compiler has to be kept from reordering them.
__device__ inline void wave_lds_fence() {
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ inline float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

__device__ inline float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

}  // namespace mva
