// RMS normalisation of q / k rows over the head dim (qk-norm), forward and
// VJP, one pass each.
//
// Same math as the reference's qk_rms_norm (src/nitrix/nn/attention/
// _reference.py:52-77, eps 1e-6 at :32), which the fused path applies in the
// I/O dtype before the attention kernel (nn/attention/__init__.py:196-197):
// upcast to fp32, y = x * rsqrt(mean(x^2) + eps), cast back.  The VJP is the
// closed form dx = r (dy - y mean(dy y)) with r = rsqrt(mean(x^2) + eps) and
// y = x r in fp32 (autodiff through the cast passes the cotangent unchanged).
//
// 16 lanes per row, 16-byte loads, fp32 accumulation; the forward keeps r per
// row for the VJP.  HBM-bound: one read of x (and dy) and one write per pass.
#include "nxa_common.h"
#include "nxa_launch.h"

namespace nxa {

// Sum over the 16 lanes of a row group (lanes 16k .. 16k + 15).
__device__ __forceinline__ float sum16(float x) {
  x += __shfl_xor(x, 8, 16);
  x += __shfl_xor(x, 4, 16);
  x += __shfl_xor(x, 2, 16);
  x += __shfl_xor(x, 1, 16);
  return x;
}

template <typename T>
__global__ __launch_bounds__(256) void rms_norm_fwd_kernel(const NormParams p) {
  using Frag = typename Mma<T>::Frag;
  constexpr int EPC = Mma<T>::EPC;
  const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int sub = threadIdx.x & 15;
  if (row >= p.rows) return;  // whole 16-lane groups leave together
  const T* x = (const T*)p.x + row * p.x_stride;
  T* y = (T*)p.y + row * p.D;
  float ss = 0.f;
  for (int c = sub * EPC; c < p.D; c += 16 * EPC) {
    const Frag v = ld16(x + c);
#pragma unroll
    for (int j = 0; j < EPC; ++j) ss = __builtin_fmaf(to_f32(v[j]), to_f32(v[j]), ss);
  }
  ss = sum16(ss);
  const float r = 1.0f / __builtin_sqrtf(ss / (float)p.D + p.eps);
  for (int c = sub * EPC; c < p.D; c += 16 * EPC) {
    const Frag v = ld16(x + c);
    Frag o;
#pragma unroll
    for (int j = 0; j < EPC; ++j) o[j] = (T)(to_f32(v[j]) * r);
    *reinterpret_cast<Frag*>(y + c) = o;
  }
  if (sub == 0 && p.rstd) p.rstd[row] = r;
}

template <typename T>
__global__ __launch_bounds__(256) void rms_norm_bwd_kernel(const NormParams p) {
  using Frag = typename Mma<T>::Frag;
  constexpr int EPC = Mma<T>::EPC;
  const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int sub = threadIdx.x & 15;
  if (row >= p.rows) return;
  const T* x = (const T*)p.x + row * p.x_stride;
  const T* dy = (const T*)p.dy + row * p.D;
  T* dx = (T*)p.dx + row * p.D;
  const float r = p.rstd[row];
  float s = 0.f;  // sum dy * y
  for (int c = sub * EPC; c < p.D; c += 16 * EPC) {
    const Frag v = ld16(x + c), g = ld16(dy + c);
#pragma unroll
    for (int j = 0; j < EPC; ++j) s = __builtin_fmaf(to_f32(g[j]), to_f32(v[j]) * r, s);
  }
  const float m = sum16(s) / (float)p.D;
  for (int c = sub * EPC; c < p.D; c += 16 * EPC) {
    const Frag v = ld16(x + c), g = ld16(dy + c);
    Frag o;
#pragma unroll
    for (int j = 0; j < EPC; ++j)
      o[j] = (T)(r * (to_f32(g[j]) - to_f32(v[j]) * r * m));
    *reinterpret_cast<Frag*>(dx + c) = o;
  }
}

template <typename T>
static void launch_norm_t(const NormParams& p, bool bwd, hipStream_t stream) {
  const int64_t blocks = (p.rows + 15) / 16;
  if (bwd)
    hipLaunchKernelGGL(rms_norm_bwd_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(rms_norm_fwd_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, stream, p);
}

void launch_rms_norm(const NormParams& p, int dtype, bool bwd, hipStream_t stream) {
  if (dtype == kBF16) launch_norm_t<bf16>(p, bwd, stream);
  else if (dtype == kF16) launch_norm_t<f16>(p, bwd, stream);
  else launch_norm_t<float>(p, bwd, stream);
}

}  // namespace nxa
