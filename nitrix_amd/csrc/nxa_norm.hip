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
// 16 lanes per row, 16-byte loads, the whole row held in registers (the
// head dim is at most 256: two 16-byte chunks per lane for 16-bit types, four
// for fp32), fp32 accumulation; the forward keeps r per row for the VJP.  A
// grid of a few blocks per CU strides over the rows, two rows per 16-lane
// group and step, so each lane has several loads in flight: HBM-bound, one
// read of x (and dy) and one write per pass.
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

constexpr int kNormRowsPerStep = 2;  // rows per 16-lane group and loop step

template <typename T>
struct NormRow {
  using Frag = typename Mma<T>::Frag;
  static constexpr int EPC = Mma<T>::EPC;
  static constexpr int NCH = 256 / (16 * EPC);  // chunks per lane at the largest D
  Frag v[NCH];
  __device__ __forceinline__ void load(const T* row, int sub, int D) {
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      const int c = (k * 16 + sub) * EPC;
      if (c < D) v[k] = ld16(row + c);
      else v[k] = zero_frag<T>();
    }
  }
};

template <typename T>
__global__ __launch_bounds__(256) void rms_norm_fwd_kernel(const NormParams p) {
  using R = NormRow<T>;
  using Frag = typename R::Frag;
  constexpr int EPC = R::EPC, NCH = R::NCH, RS = kNormRowsPerStep;
  const int sub = threadIdx.x & 15;
  const int64_t groups = (int64_t)gridDim.x * 16;
  for (int64_t r0 = ((int64_t)blockIdx.x * 16 + (threadIdx.x >> 4)) * RS; r0 < p.rows;
       r0 += groups * RS) {
    R x[RS];
#pragma unroll
    for (int u = 0; u < RS; ++u)
      if (r0 + u < p.rows) x[u].load((const T*)p.x + (r0 + u) * p.x_stride, sub, p.D);
#pragma unroll
    for (int u = 0; u < RS; ++u) {
      const int64_t row = r0 + u;
      if (row >= p.rows) break;  // uniform over the 16-lane group
      float ss = 0.f;
#pragma unroll
      for (int k = 0; k < NCH; ++k)
#pragma unroll
        for (int j = 0; j < EPC; ++j)
          ss = __builtin_fmaf(to_f32(x[u].v[k][j]), to_f32(x[u].v[k][j]), ss);
      ss = sum16(ss);
      const float r = 1.0f / __builtin_sqrtf(ss / (float)p.D + p.eps);
      T* y = (T*)p.y + row * p.D;
#pragma unroll
      for (int k = 0; k < NCH; ++k) {
        const int c = (k * 16 + sub) * EPC;
        if (c < p.D) {
          Frag o;
#pragma unroll
          for (int j = 0; j < EPC; ++j) o[j] = (T)(to_f32(x[u].v[k][j]) * r);
          *reinterpret_cast<Frag*>(y + c) = o;
        }
      }
      if (sub == 0 && p.rstd) p.rstd[row] = r;
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void rms_norm_bwd_kernel(const NormParams p) {
  using R = NormRow<T>;
  using Frag = typename R::Frag;
  constexpr int EPC = R::EPC, NCH = R::NCH, RS = kNormRowsPerStep;
  const int sub = threadIdx.x & 15;
  const int64_t groups = (int64_t)gridDim.x * 16;
  for (int64_t r0 = ((int64_t)blockIdx.x * 16 + (threadIdx.x >> 4)) * RS; r0 < p.rows;
       r0 += groups * RS) {
    R x[RS], gy[RS];
    float r[RS];
#pragma unroll
    for (int u = 0; u < RS; ++u)
      if (r0 + u < p.rows) {
        x[u].load((const T*)p.x + (r0 + u) * p.x_stride, sub, p.D);
        gy[u].load((const T*)p.dy + (r0 + u) * p.D, sub, p.D);
        r[u] = p.rstd[r0 + u];
      }
#pragma unroll
    for (int u = 0; u < RS; ++u) {
      const int64_t row = r0 + u;
      if (row >= p.rows) break;
      float s = 0.f;  // sum dy * y
#pragma unroll
      for (int k = 0; k < NCH; ++k)
#pragma unroll
        for (int j = 0; j < EPC; ++j)
          s = __builtin_fmaf(to_f32(gy[u].v[k][j]), to_f32(x[u].v[k][j]) * r[u], s);
      const float m = sum16(s) / (float)p.D;
      T* dx = (T*)p.dx + row * p.D;
#pragma unroll
      for (int k = 0; k < NCH; ++k) {
        const int c = (k * 16 + sub) * EPC;
        if (c < p.D) {
          Frag o;
#pragma unroll
          for (int j = 0; j < EPC; ++j)
            o[j] = (T)(r[u] * (to_f32(gy[u].v[k][j]) - to_f32(x[u].v[k][j]) * r[u] * m));
          *reinterpret_cast<Frag*>(dx + c) = o;
        }
      }
    }
  }
}

template <typename T>
static void launch_norm_t(const NormParams& p, bool bwd, hipStream_t stream) {
  // Enough 256-thread blocks for eight per CU, fewer for small problems.
  const int64_t need = (p.rows + 16 * kNormRowsPerStep - 1) / (16 * kNormRowsPerStep);
  const unsigned blocks = (unsigned)(need < 2048 ? need : 2048);
  if (blocks == 0) return;
  if (bwd)
    hipLaunchKernelGGL(rms_norm_bwd_kernel<T>, dim3(blocks), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(rms_norm_fwd_kernel<T>, dim3(blocks), dim3(256), 0, stream, p);
}

void launch_rms_norm(const NormParams& p, int dtype, bool bwd, hipStream_t stream) {
  if (dtype == kBF16) launch_norm_t<bf16>(p, bwd, stream);
  else if (dtype == kF16) launch_norm_t<f16>(p, bwd, stream);
  else launch_norm_t<float>(p, bwd, stream);
}

}  // namespace nxa
