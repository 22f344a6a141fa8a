// RMSNorm and fused residual-add RMSNorm for gfx950.
//
// Semantics follow the reference's native path (nanovllm/layers/layernorm.py:
// 31-52, the compiled torch restatement its CUDA providers must match):
//   rms_norm:      x32 = float(x); y = T(T(x32 * rsqrt(mean(x32^2) + eps)) * w)
//   add_rms_norm:  s32 = float(x) + float(residual); residual_out = T(s32);
//                  y = T(T(s32 * rsqrt(mean(s32^2) + eps)) * w)
// i.e. the statistics use the fp32 sum (not the rounded residual), the scaled
// row is rounded to the storage type T before the weight multiply, and the
// product is rounded again (torch multiplies two T tensors in fp32 and rounds
// once).  `w` is T or fp32.
//
// HBM-bound: one wavefront per row (four rows per 256-thread workgroup); each
// lane keeps its 16-byte chunks of the row in registers between the sum of
// squares and the output, so a row is read once and written once, and an
// in-place call (out == x, residual_out == residual) is safe: every element is
// read before any element of its row is written.
#include "mva_capi.h"
#include "mva_common.h"

namespace mva {
namespace {

// Row r of a call is row (r % rows_per_group) of group (r / rows_per_group):
// x + (r / rows_per_group) * x_group_stride + (r % rows_per_group) * x_stride
// (likewise for out; the fused form uses one group per row).
struct RmsArgs {
  const void* x;
  int64_t x_stride;  // elements between rows of a group
  const void* residual;  // nullptr: plain RMSNorm
  int64_t res_stride;
  const void* weight;
  void* out;
  int64_t out_stride;
  void* residual_out;
  int64_t res_out_stride;
  int64_t rows;
  int hidden;
  float eps;
  int64_t rows_per_group;
  int64_t x_group_stride;
  int64_t out_group_stride;
};

__device__ inline int64_t row_offset(int64_t r, int64_t per_group, int64_t group_stride, int64_t stride) {
  const int64_t g = r / per_group;
  return g * group_stride + (r - g * per_group) * stride;
}

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

template <typename W>
__device__ inline void load_w8(const W* w, float (&f)[8]);
template <>
__device__ inline void load_w8<float>(const float* w, float (&f)[8]) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(w);
  const f32x4 b = *reinterpret_cast<const f32x4*>(w + 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[i] = a[i];
    f[4 + i] = b[i];
  }
}
template <>
__device__ inline void load_w8<__bf16>(const __bf16* w, float (&f)[8]) {
  const bf16x8 a = *reinterpret_cast<const bf16x8*>(w);
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = (float)a[i];
}
template <>
__device__ inline void load_w8<_Float16>(const _Float16* w, float (&f)[8]) {
  const f16x8 a = *reinterpret_cast<const f16x8*>(w);
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = (float)a[i];
}

// Vector path: hidden % 8 == 0, 16-byte aligned rows, hidden <= 512 * kChunks
// (at most 8192: larger rows take the scalar path).
template <typename T, typename W, int kChunks, bool kAdd>
__global__ __launch_bounds__(256) void rms_norm_vec_kernel(RmsArgs a) {
  typedef typename Elem<T>::v8 V;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const int nvec = a.hidden >> 3;
  const T* xr = (const T*)a.x + row_offset(row, a.rows_per_group, a.x_group_stride, a.x_stride);
  const T* rr = kAdd ? (const T*)a.residual + row * a.res_stride : nullptr;
  float v[kChunks][8];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int j = lane + 64 * c;
    if (j < nvec) {
      const V xv = *reinterpret_cast<const V*>(xr + 8 * j);
      V rv;
      if constexpr (kAdd) rv = *reinterpret_cast<const V*>(rr + 8 * j);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float f = (float)xv[i];
        if constexpr (kAdd) f += (float)rv[i];
        v[c][i] = f;
        ss += f * f;
      }
    }
  }
  ss = wave_sum(ss);
  const float r = 1.0f / __builtin_sqrtf(ss / (float)a.hidden + a.eps);
  T* orow = (T*)a.out + row_offset(row, a.rows_per_group, a.out_group_stride, a.out_stride);
  T* ro = kAdd ? (T*)a.residual_out + row * a.res_out_stride : nullptr;
  const W* w = (const W*)a.weight;
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int j = lane + 64 * c;
    if (j < nvec) {
      float wf[8];
      load_w8<W>(w + 8 * j, wf);
      V o;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = (T)((float)(T)(v[c][i] * r) * wf[i]);
      if constexpr (kAdd) {
        V s;
#pragma unroll
        for (int i = 0; i < 8; ++i) s[i] = (T)v[c][i];
        *reinterpret_cast<V*>(ro + 8 * j) = s;
      }
      *reinterpret_cast<V*>(orow + 8 * j) = o;
    }
  }
}

// Any width and alignment: two passes over the row per wavefront (the first
// only reads), so in-place calls stay correct.
template <typename T, typename W, bool kAdd>
__global__ __launch_bounds__(256) void rms_norm_scalar_kernel(RmsArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const T* xr = (const T*)a.x + row_offset(row, a.rows_per_group, a.x_group_stride, a.x_stride);
  const T* rr = kAdd ? (const T*)a.residual + row * a.res_stride : nullptr;
  float ss = 0.f;
  for (int i = lane; i < a.hidden; i += 64) {
    float f = (float)xr[i];
    if constexpr (kAdd) f += (float)rr[i];
    ss += f * f;
  }
  ss = wave_sum(ss);
  const float r = 1.0f / __builtin_sqrtf(ss / (float)a.hidden + a.eps);
  T* orow = (T*)a.out + row_offset(row, a.rows_per_group, a.out_group_stride, a.out_stride);
  T* ro = kAdd ? (T*)a.residual_out + row * a.res_out_stride : nullptr;
  const W* w = (const W*)a.weight;
  for (int i = lane; i < a.hidden; i += 64) {
    float f = (float)xr[i];
    if constexpr (kAdd) f += (float)rr[i];
    const T y = (T)((float)(T)(f * r) * (float)w[i]);
    if constexpr (kAdd) ro[i] = (T)f;
    orow[i] = y;
  }
}

template <typename T, typename W, bool kAdd>
int launch_rms(const RmsArgs& a, hipStream_t s) {
  const int64_t blocks = (a.rows + 3) / 4;
  if (blocks > 0x7fffffffLL) return set_error("rms_norm: too many rows");
  const dim3 grid((uint32_t)blocks), block(256);
  uint64_t bits = (uint64_t)(uintptr_t)a.x | (uint64_t)(uintptr_t)a.out | (uint64_t)(uintptr_t)a.weight |
                  (uint64_t)(a.x_stride * (int64_t)sizeof(T)) | (uint64_t)(a.out_stride * (int64_t)sizeof(T)) |
                  (uint64_t)(a.x_group_stride * (int64_t)sizeof(T)) |
                  (uint64_t)(a.out_group_stride * (int64_t)sizeof(T));
  if (kAdd)
    bits |= (uint64_t)(uintptr_t)a.residual | (uint64_t)(uintptr_t)a.residual_out |
            (uint64_t)(a.res_stride * (int64_t)sizeof(T)) | (uint64_t)(a.res_out_stride * (int64_t)sizeof(T));
  const int nvec = a.hidden / 8;
  if (a.hidden % 8 == 0 && bits % 16 == 0 && nvec <= 64 * 16) {
    const int chunks = (nvec + 63) / 64;
    if (chunks <= 1) hipLaunchKernelGGL((rms_norm_vec_kernel<T, W, 1, kAdd>), grid, block, 0, s, a);
    else if (chunks <= 2) hipLaunchKernelGGL((rms_norm_vec_kernel<T, W, 2, kAdd>), grid, block, 0, s, a);
    else if (chunks <= 4) hipLaunchKernelGGL((rms_norm_vec_kernel<T, W, 4, kAdd>), grid, block, 0, s, a);
    else if (chunks <= 8) hipLaunchKernelGGL((rms_norm_vec_kernel<T, W, 8, kAdd>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((rms_norm_vec_kernel<T, W, 16, kAdd>), grid, block, 0, s, a);
  } else {
    hipLaunchKernelGGL((rms_norm_scalar_kernel<T, W, kAdd>), grid, block, 0, s, a);
  }
  return check_launch("rms_norm");
}

template <bool kAdd>
int dispatch(const RmsArgs& a, int dtype, int weight_dtype, hipStream_t s) {
  if (a.rows < 0 || a.hidden <= 0) return set_error("rms_norm: invalid shape");
  if (a.rows == 0) return 0;
  const bool wf32 = weight_dtype == kF32;
  if (!wf32 && weight_dtype != dtype) return set_error("rms_norm: weight must be fp32 or the input dtype");
  if (dtype == kBF16) return wf32 ? launch_rms<__bf16, float, kAdd>(a, s) : launch_rms<__bf16, __bf16, kAdd>(a, s);
  if (dtype == kF16)
    return wf32 ? launch_rms<_Float16, float, kAdd>(a, s) : launch_rms<_Float16, _Float16, kAdd>(a, s);
  return set_error("rms_norm: dtype must be bf16 or fp16");
}

}  // namespace
}  // namespace mva

extern "C" int mva_rms_norm(const void* x, int64_t x_group_stride, int64_t x_row_stride, const void* weight,
                            void* out, int64_t out_group_stride, int64_t out_row_stride, int64_t rows,
                            int64_t rows_per_group, int64_t hidden, float eps, int dtype, int weight_dtype,
                            void* stream) {
  using namespace mva;
  if (hidden > 0x7fffffffLL) return set_error("rms_norm: hidden too large");
  if (rows_per_group <= 0) return set_error("rms_norm: rows_per_group must be positive");
  RmsArgs a{x, x_row_stride, nullptr, 0, weight, out, out_row_stride, nullptr, 0, rows, (int)hidden, eps,
            rows_per_group, x_group_stride, out_group_stride};
  return dispatch<false>(a, dtype, weight_dtype, (hipStream_t)stream);
}

extern "C" int mva_fused_add_rms_norm(const void* x, int64_t x_row_stride, const void* residual,
                                      int64_t residual_row_stride, const void* weight, void* out,
                                      int64_t out_row_stride, void* residual_out,
                                      int64_t residual_out_row_stride, int64_t rows, int64_t hidden, float eps,
                                      int dtype, int weight_dtype, void* stream) {
  using namespace mva;
  if (hidden > 0x7fffffffLL) return set_error("rms_norm: hidden too large");
  if (residual == nullptr || residual_out == nullptr) return set_error("rms_norm: missing residual buffers");
  RmsArgs a{x, x_row_stride, residual, residual_row_stride, weight, out, out_row_stride,
            residual_out, residual_out_row_stride, rows, (int)hidden, eps, 1, x_row_stride, out_row_stride};
  return dispatch<true>(a, dtype, weight_dtype, (hipStream_t)stream);
}
