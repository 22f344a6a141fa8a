// SiLU-and-mul for gfx950: out[r, c] = silu(x[r, c]) * x[r, c + I], I = hidden.
//
// Semantics follow the reference's fused op (csrc/silu_and_mul_kernel.cu:11-31
// and the compiled native path nanovllm/layers/activation.py:34-37): both
// halves are widened to fp32, silu(g) = g / (1 + e^-g) is evaluated in fp32,
// multiplied by the up value in fp32 and rounded to the storage type once.
//
// The op is a pure HBM stream (3 bytes moved per 2 input elements per output
// element), so the fast path moves 16 bytes per access: each thread reads 8
// gate and 8 up elements and writes 8 outputs.  Rows whose width is not a
// multiple of 8 (or unaligned buffers) take the one-element-per-thread path.
#include "mva_capi.h"
#include "mva_common.h"

namespace mva {
namespace {

__device__ inline float silu_mul(float g, float u) {
  // g * 1/(1+2^(-g*log2 e)); v_exp_f32 and v_rcp_f32 are accurate to about
  // 1 fp32 ulp, far below the 2^-8 relative step of bf16.
  const float e = fast_exp2(-g * 1.4426950408889634f);
  return g * fast_rcp(1.0f + e) * u;
}

template <typename T>
__global__ __launch_bounds__(256) void silu_and_mul_vec8_kernel(
    const T* __restrict__ in, T* __restrict__ out, uint32_t vecs_per_row,
    uint32_t total_vecs) {
  typedef typename Elem<T>::v8 V;
  const uint32_t v = blockIdx.x * 256u + threadIdx.x;
  if (v >= total_vecs) return;
  const uint32_t row = v / vecs_per_row;
  const uint32_t col = v - row * vecs_per_row;
  const uint64_t hidden = (uint64_t)vecs_per_row * 8u;
  const T* gp = in + (uint64_t)row * (2u * hidden) + (uint64_t)col * 8u;
  const V g = __builtin_nontemporal_load(reinterpret_cast<const V*>(gp));
  const V u = __builtin_nontemporal_load(reinterpret_cast<const V*>(gp + hidden));
  V o;
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = (T)silu_mul((float)g[i], (float)u[i]);
  __builtin_nontemporal_store(o, reinterpret_cast<V*>(out + (uint64_t)row * hidden + (uint64_t)col * 8u));
}

template <typename T>
__global__ __launch_bounds__(256) void silu_and_mul_scalar_kernel(
    const T* __restrict__ in, T* __restrict__ out, uint64_t hidden,
    uint64_t total) {
  const uint64_t stride = (uint64_t)gridDim.x * 256u;
  for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < total; i += stride) {
    const uint64_t row = i / hidden;
    const uint64_t col = i - row * hidden;
    const T* gp = in + row * 2u * hidden + col;
    out[i] = (T)silu_mul((float)gp[0], (float)gp[hidden]);
  }
}

template <typename T>
int launch(const void* input, void* output, int64_t rows, int64_t hidden, hipStream_t stream) {
  const uint64_t total = (uint64_t)rows * (uint64_t)hidden;
  const bool aligned = ((uintptr_t)input % 16 == 0) && ((uintptr_t)output % 16 == 0);
  if (aligned && hidden % 8 == 0 && total / 8 < (1ull << 31)) {
    const uint32_t vecs_per_row = (uint32_t)(hidden / 8);
    const uint32_t total_vecs = (uint32_t)(total / 8);
    const uint32_t blocks = (total_vecs + 255u) / 256u;
    hipLaunchKernelGGL(silu_and_mul_vec8_kernel<T>, dim3(blocks), dim3(256), 0, stream,
                       (const T*)input, (T*)output, vecs_per_row, total_vecs);
  } else {
    uint64_t blocks = (total + 255u) / 256u;
    if (blocks > 65535u * 8u) blocks = 65535u * 8u;
    hipLaunchKernelGGL(silu_and_mul_scalar_kernel<T>, dim3((uint32_t)blocks), dim3(256), 0, stream,
                       (const T*)input, (T*)output, (uint64_t)hidden, total);
  }
  return check_launch("silu_and_mul");
}

}  // namespace
}  // namespace mva

extern "C" int mva_silu_and_mul(const void* input, void* output, int64_t rows, int64_t hidden,
                                int dtype, void* stream) {
  using namespace mva;
  if (rows < 0 || hidden <= 0) return set_error("silu_and_mul: rows must be >= 0 and hidden > 0");
  if (rows == 0) return 0;
  if (input == nullptr || output == nullptr) return set_error("silu_and_mul: null buffer");
  hipStream_t s = (hipStream_t)stream;
  if (dtype == kBF16) return launch<__bf16>(input, output, rows, hidden, s);
  if (dtype == kF16) return launch<_Float16>(input, output, rows, hidden, s);
  return set_error("silu_and_mul: dtype must be bf16 or fp16");
}
