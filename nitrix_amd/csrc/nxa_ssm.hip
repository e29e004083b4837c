// Selective state-space scan (Mamba / S6), forward and backward, fp32.
//
// Same math as the reference (src/nitrix/nn/ssm/_reference.py:59-97): per
// batch b, channel d and state n, h_t = exp(delta_t A) h_{t-1} + delta_t B_t x_t
// from h = 0, y_t = sum_n C_t h_t (+ D x_t).  The backward is the reverse-mode
// adjoint of that recurrence, recomputing the states instead of storing the
// (l, d, n) trajectory (the fused path's recompute adjoint,
// src/nitrix/_kernels/cuda/selective_scan.py:239-419).  With a_t =
// exp(delta_t A) and the state adjoint g_t = C_t dy_t + a_{t+1} g_{t+1}:
//   dx_t = D dy_t + sum_n g_t delta_t B_t        dA = sum_t g_t delta_t a_t h_{t-1}
//   ddelta_t = sum_n g_t (B_t x_t + A a_t h_{t-1})   dB_t = sum_d g_t delta_t x_t
//   dC_t = sum_d dy_t h_t                          dD = sum_t dy_t x_t
//
// Layout: x, delta, y, dy, dx, ddelta [nb, L, Dm]; B, C, dB, dC [nb, L, N];
// A, dA [Dm, N]; D, dD [Dm]; all fp32, contiguous.  One lane per channel d
// with the N states in registers (padded to NP in {4, 8, 16, 32}: padded
// states have A = B = C = 0 and stay zero).  B_t and C_t are the same for
// every lane of a block (scalar loads).
//
// The sequence is cut into chunks of 32 steps so nb * Dm * L / 32 lanes work
// at once; a chunk's state (or adjoint) depends on the others only through
// the value entering it, which a short carry pass over the chunks supplies:
//  forward  1. each chunk from h = 0: end state and sum(delta);
//           2. carry over chunks per (b, n, d): the state entering each
//              chunk (prod_t a_t over a chunk = exp(A sum(delta)));
//           3. each chunk again from its entering state: y, and (for the
//              backward) the state entering every sub-chunk of 8 steps.
//  backward 4. each chunk in reverse from adjoint 0: its first-step adjoint
//              (times a) and sum(delta);
//           5. carry over chunks from the last: the adjoint entering each
//              chunk from the right;
//           6. each chunk again, sub-chunk by sub-chunk from the last: the
//              forward states from the saved sub-chunk state (registers), then
//              the reverse walk: dx, ddelta, and per-chunk partial sums of
//              dA, dD (per lane) and dB, dC (over the block's channels:
//              butterfly reduce-scatter across the wave, then LDS);
//           7. fixed-order sums of the partials (deterministic results).
#include "nxa_common.h"
#include "nxa_launch.h"

namespace nxa {

namespace {

constexpr int kWaves = kSsmBlock / 64;

__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }

struct SsmBlock {
  int dblk, c, b, d, t0, t1;
};

__device__ __forceinline__ SsmBlock ssm_block(const SsmParams& p) {
  SsmBlock k;
  const int bid = blockIdx.x;
  k.dblk = bid % p.ndblk;
  const int rest = bid / p.ndblk;
  k.c = rest % p.nc;
  k.b = rest / p.nc;
  k.d = k.dblk * kSsmBlock + threadIdx.x;
  k.t0 = k.c * kSsmChunk;
  k.t1 = min(p.L, k.t0 + kSsmChunk);
  return k;
}

// A * log2(e) for the lane's channel (0 for padded states and idle lanes).
template <int NP>
__device__ __forceinline__ void load_al(const SsmParams& p, int d, bool ok, float (&al)[NP]) {
#pragma unroll
  for (int n = 0; n < NP; ++n) al[n] = (ok && n < p.N) ? p.A[(int64_t)d * p.N + n] * kLog2e : 0.f;
}

__device__ __forceinline__ float row_val(const float* row, int n, int N) {
  return n < N ? row[n] : 0.f;
}

// (1) Local forward scan of a chunk from zero: end state and sum(delta).
template <int NP>
__global__ __launch_bounds__(kSsmBlock) void ssm_fwd_local_kernel(const SsmParams p) {
  const SsmBlock k = ssm_block(p);
  if (k.d >= p.Dm) return;
  float al[NP], h[NP];
  load_al<NP>(p, k.d, true, al);
#pragma unroll
  for (int n = 0; n < NP; ++n) h[n] = 0.f;
  float sdt = 0.f;
  for (int t = k.t0; t < k.t1; ++t) {
    const int64_t xi = ((int64_t)k.b * p.L + t) * p.Dm + k.d;
    const float dt = p.delta[xi], dx = dt * p.x[xi];
    const float* Bt = p.B + ((int64_t)k.b * p.L + t) * p.N;
#pragma unroll
    for (int n = 0; n < NP; ++n)
      h[n] = __builtin_fmaf(fexp2(dt * al[n]), h[n], dx * row_val(Bt, n, p.N));
    sdt += dt;
  }
  const int64_t cb = ((int64_t)k.b * p.nc + k.c) * NP;
#pragma unroll
  for (int n = 0; n < NP; ++n) p.hc[(cb + n) * p.Dm + k.d] = h[n];
  p.sdt[((int64_t)k.b * p.nc + k.c) * p.Dm + k.d] = sdt;
}

// (2) / (5) Carry over the chunks of each (b, n, d), in place on buf: the
// chunk-local value loc[c] becomes the value entering chunk c, H, walking
// forward (REV = false) or from the last chunk (REV = true), with
// H <- exp2(al sdt[c]) H + loc[c].
template <bool REV>
__global__ __launch_bounds__(kSsmBlock) void ssm_carry_kernel(const SsmParams p, int NP,
                                                             float* buf) {
  const int64_t i = (int64_t)blockIdx.x * kSsmBlock + threadIdx.x;  // (b, n, d)
  const int64_t per_b = (int64_t)NP * p.Dm;
  if (i >= p.nb * per_b) return;
  const int64_t b = i / per_b, nd = i % per_b;
  const int n = (int)(nd / p.Dm), d = (int)(nd % p.Dm);
  const float al = n < p.N ? p.A[(int64_t)d * p.N + n] * kLog2e : 0.f;
  float H = 0.f;
  for (int k = 0; k < p.nc; ++k) {
    const int c = REV ? p.nc - 1 - k : k;
    const int64_t ci = (b * p.nc + c) * per_b + nd;
    const float loc = buf[ci];
    buf[ci] = H;
    H = __builtin_fmaf(fexp2(al * p.sdt[(b * p.nc + c) * p.Dm + d]), H, loc);
  }
}

// (3) Output pass: each chunk from its entering state; y, and the state
// entering each SC-step sub-chunk when p.hs is set.
template <int NP>
__global__ __launch_bounds__(kSsmBlock) void ssm_fwd_out_kernel(const SsmParams p) {
  const SsmBlock k = ssm_block(p);
  if (k.d >= p.Dm) return;
  float al[NP], h[NP];
  load_al<NP>(p, k.d, true, al);
  const int64_t cb = ((int64_t)k.b * p.nc + k.c) * NP;
#pragma unroll
  for (int n = 0; n < NP; ++n) h[n] = p.hc[(cb + n) * p.Dm + k.d];
  const float Dd = p.D ? p.D[k.d] : 0.f;
  constexpr int SC = kSsmSub;
  for (int ts = k.t0; ts < k.t1; ts += SC) {
    if (p.hs) {
      const int64_t sb = ((int64_t)k.b * p.ns + ts / SC) * NP;
#pragma unroll
      for (int n = 0; n < NP; ++n) p.hs[(sb + n) * p.Dm + k.d] = h[n];
    }
#pragma unroll
    for (int j = 0; j < SC; ++j) {
      const int t = ts + j;
      if (t < k.t1) {
        const int64_t xi = ((int64_t)k.b * p.L + t) * p.Dm + k.d;
        const float dt = p.delta[xi], xv = p.x[xi], dx = dt * xv;
        const float* Bt = p.B + ((int64_t)k.b * p.L + t) * p.N;
        const float* Ct = p.C + ((int64_t)k.b * p.L + t) * p.N;
        float y = 0.f;
#pragma unroll
        for (int n = 0; n < NP; ++n) {
          h[n] = __builtin_fmaf(fexp2(dt * al[n]), h[n], dx * row_val(Bt, n, p.N));
          y = __builtin_fmaf(row_val(Ct, n, p.N), h[n], y);
        }
        p.y[xi] = __builtin_fmaf(Dd, xv, y);
      }
    }
  }
}

// (4) Local reverse scan of a chunk from adjoint 0: a_{t0} g_{t0} and
// sum(delta).
template <int NP>
__global__ __launch_bounds__(kSsmBlock) void ssm_bwd_local_kernel(const SsmParams p) {
  const SsmBlock k = ssm_block(p);
  if (k.d >= p.Dm) return;
  float al[NP], gh[NP];
  load_al<NP>(p, k.d, true, al);
#pragma unroll
  for (int n = 0; n < NP; ++n) gh[n] = 0.f;
  float sdt = 0.f;
  for (int t = k.t1 - 1; t >= k.t0; --t) {
    const int64_t xi = ((int64_t)k.b * p.L + t) * p.Dm + k.d;
    const float dt = p.delta[xi], dyv = p.dy[xi];
    const float* Ct = p.C + ((int64_t)k.b * p.L + t) * p.N;
#pragma unroll
    for (int n = 0; n < NP; ++n)
      gh[n] = fexp2(dt * al[n]) * __builtin_fmaf(row_val(Ct, n, p.N), dyv, gh[n]);
    sdt += dt;
  }
  const int64_t cb = ((int64_t)k.b * p.nc + k.c) * NP;
#pragma unroll
  for (int n = 0; n < NP; ++n) p.gc[(cb + n) * p.Dm + k.d] = gh[n];
  p.sdt[((int64_t)k.b * p.nc + k.c) * p.Dm + k.d] = sdt;
}

// Sums v[0..V) over the 64 lanes of a wave.  log2(V) halving exchanges
// leave each lane one value index, lane >> (6 - log2(V)), summed over the
// lanes that share the lane's top log2(V) bits; the remaining exchanges
// complete the 64-lane sum.  V - 1 + 6 - log2(V) shuffles in all.
template <int V>
__device__ __forceinline__ float wave_sum_scatter(float (&v)[V], int lane) {
  static_assert(V >= 1 && V <= 64 && (V & (V - 1)) == 0, "V: power of two <= 64");
#pragma unroll
  for (int half = V / 2, m = 32; half >= 1; half /= 2, m /= 2) {
    const bool up = lane & m;
#pragma unroll
    for (int i = 0; i < half; ++i) {
      // Select values, not addresses (an address select becomes a dynamic
      // register index).
      const float lo = v[i], hi = v[i + half];
      const float keep = up ? hi : lo;
      const float send = up ? lo : hi;
      v[i] = keep + __shfl_xor(send, m, 64);
    }
  }
  float s = v[0];
#pragma unroll
  for (int m = 32 / V; m >= 1; m /= 2) s += __shfl_xor(s, m, 64);
  return s;
}

// (6) Backward pass over one chunk, sub-chunk by sub-chunk from the last.
// A sub-chunk's SC states are rebuilt from its saved entering state in parts
// of HS steps (registers hold HS + 1 states of NP), the last part first; a
// part q first advances the saved state over the q * HS steps before it.
template <int NP, int HS>
__global__ __launch_bounds__(kSsmBlock) void ssm_bwd_chunk_kernel(const SsmParams p) {
  constexpr int SC = kSsmSub;
  constexpr int SH = 6 - __builtin_ctz(NP);
  static_assert(SC % HS == 0, "HS must divide the sub-chunk");
  __shared__ float red[kSsmChunk][kWaves][2 * NP];
  __shared__ float sB[kSsmChunk][NP], sC[kSsmChunk][NP];  // the chunk's B, C rows
  const SsmBlock k = ssm_block(p);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool ok = k.d < p.Dm;  // idle lanes still take part in the sums, with zeros
  const int d = ok ? k.d : p.Dm - 1;
  for (int e = tid; e < kSsmChunk * NP; e += kSsmBlock) {
    const int j = e / NP, n = e % NP, t = k.t0 + j;
    const bool in = t < k.t1 && n < p.N;
    const int64_t bi = ((int64_t)k.b * p.L + t) * p.N + n;
    sB[j][n] = in ? p.B[bi] : 0.f;
    sC[j][n] = in ? p.C[bi] : 0.f;
  }
  __syncthreads();
  float al[NP], gh[NP], dA[NP];
  load_al<NP>(p, d, ok, al);
  const int64_t cb = ((int64_t)k.b * p.nc + k.c) * NP;
#pragma unroll
  for (int n = 0; n < NP; ++n) {
    gh[n] = ok ? p.gc[(cb + n) * p.Dm + d] : 0.f;
    dA[n] = 0.f;
  }
  const float Dd = (ok && p.D) ? p.D[d] : 0.f;
  float dD = 0.f;
  const int nsub = (k.t1 - k.t0 + SC - 1) / SC;
  for (int s = nsub - 1; s >= 0; --s) {
    const int ts = k.t0 + s * SC;
    const int64_t sb = ((int64_t)k.b * p.ns + ts / SC) * NP;
    for (int q = SC / HS - 1; q >= 0; --q) {
      const int tq = ts + q * HS;
      if (tq >= k.t1) continue;  // uniform over the block
      // hist[j]: the state entering step tq + j (hist[HS]: after the last).
      float hist[HS + 1][NP];
#pragma unroll
      for (int n = 0; n < NP; ++n) hist[0][n] = ok ? p.hs[(sb + n) * p.Dm + d] : 0.f;
      for (int t = ts; t < tq; ++t) {
        const int64_t xi = ((int64_t)k.b * p.L + t) * p.Dm + d;
        const float dt = p.delta[xi], dx = dt * p.x[xi];
        const float* Bt = sB[t - k.t0];
#pragma unroll
        for (int n = 0; n < NP; ++n)
          hist[0][n] = __builtin_fmaf(fexp2(dt * al[n]), hist[0][n], dx * Bt[n]);
      }
#pragma unroll
      for (int j = 0; j < HS; ++j) {
        const int t = min(tq + j, k.t1 - 1);  // states past the end are never read
        const int64_t xi = ((int64_t)k.b * p.L + t) * p.Dm + d;
        const float dt = p.delta[xi], dx = dt * p.x[xi];
        const float* Bt = sB[t - k.t0];
#pragma unroll
        for (int n = 0; n < NP; ++n)
          hist[j + 1][n] = __builtin_fmaf(fexp2(dt * al[n]), hist[j][n], dx * Bt[n]);
      }
#pragma unroll
      for (int j = HS - 1; j >= 0; --j) {
        const int t = tq + j;
        if (t < k.t1) {  // uniform over the block
          const int64_t xi = ((int64_t)k.b * p.L + t) * p.Dm + d;
          const float dt = p.delta[xi], xv = p.x[xi], dyv = ok ? p.dy[xi] : 0.f;
          const float dtx = dt * xv;
          const float* Bt = sB[t - k.t0];
          const float* Ct = sC[t - k.t0];
          float dx = Dd * dyv, ddt = 0.f;
          float v[NP];
          // Recompute a here rather than keep the rebuild's HS x NP values live.
          float dto = dt;
          asm volatile("" : "+v"(dto));
#pragma unroll
          for (int n = 0; n < NP; ++n) {
            const float bn = Bt[n], cn = Ct[n];
            const float a = fexp2(dto * al[n]);
            const float ah = a * hist[j][n];
            const float g = __builtin_fmaf(cn, dyv, gh[n]);
            dx = __builtin_fmaf(g * dt, bn, dx);
            ddt = __builtin_fmaf(g, __builtin_fmaf(bn, xv, al[n] * kLn2 * ah), ddt);
            dA[n] = __builtin_fmaf(g * dt, ah, dA[n]);
            v[n] = g * dtx;  // dB_t
            gh[n] = a * g;
          }
          dD = __builtin_fmaf(dyv, xv, dD);
          if (ok) {
            p.dx[xi] = dx;
            p.ddelta[xi] = ddt;
          }
          const bool head = (lane & ((1 << SH) - 1)) == 0;
          float r = wave_sum_scatter<NP>(v, lane);
          if (head) red[t - k.t0][wave][lane >> SH] = r;
#pragma unroll
          for (int n = 0; n < NP; ++n) v[n] = dyv * hist[j + 1][n];  // dC_t
          r = wave_sum_scatter<NP>(v, lane);
          if (head) red[t - k.t0][wave][NP + (lane >> SH)] = r;
        }
      }
    }
  }
  if (ok) {
    // The chunk's adjoint slot is this lane's own: reuse it for the dA partials.
#pragma unroll
    for (int n = 0; n < NP; ++n) p.gc[(cb + n) * p.Dm + d] = dA[n];
    p.dDpart[((int64_t)k.b * p.nc + k.c) * p.Dm + d] = dD;
  }
  __syncthreads();
  constexpr int V = 2 * NP;
  for (int e = tid; e < kSsmChunk * V; e += kSsmBlock) {
    const int j = e / V, q = e % V;
    if (k.t0 + j < k.t1) {
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) s += red[j][w][q];
      p.dBCpart[(((int64_t)k.dblk * p.nb + k.b) * p.L + k.t0 + j) * V + q] = s;
    }
  }
}

// (7a) dA [Dm, N] and dD [Dm]: sums over the nb * nc chunk partials, 64
// columns per block, four row groups combined through LDS in a fixed order.
__global__ __launch_bounds__(kSsmBlock) void ssm_reduce_dad_kernel(const SsmParams p, int NP) {
  __shared__ float part[kWaves][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t col = (int64_t)blockIdx.x * 64 + lane;
  const int64_t na = (int64_t)NP * p.Dm, ncol = na + p.Dm;
  const int64_t rows = p.nb * p.nc;
  float s = 0.f;
  if (col < ncol) {
    if (col < na) {
      for (int64_t r = w; r < rows; r += kWaves) s += p.gc[r * na + col];
    } else {
      for (int64_t r = w; r < rows; r += kWaves) s += p.dDpart[r * p.Dm + (col - na)];
    }
  }
  part[w][lane] = s;
  __syncthreads();
  if (w == 0 && col < ncol) {
    s = (part[0][lane] + part[1][lane]) + (part[2][lane] + part[3][lane]);
    if (col < na) {
      const int n = (int)(col / p.Dm), d = (int)(col % p.Dm);
      if (n < p.N) p.dA[(int64_t)d * p.N + n] = s;
    } else if (p.dD) {
      p.dD[col - na] = s;
    }
  }
}

// (7b) dB / dC [nb, L, N]: sums over the channel blocks.
__global__ __launch_bounds__(kSsmBlock) void ssm_reduce_dbc_kernel(const SsmParams p, int NP) {
  const int V = 2 * NP;
  const int64_t i = (int64_t)blockIdx.x * kSsmBlock + threadIdx.x;  // (b, t, q)
  const int64_t per_blk = p.nb * p.L * V;
  if (i >= per_blk) return;
  float s = 0.f;
  for (int blk = 0; blk < p.ndblk; ++blk) s += p.dBCpart[(int64_t)blk * per_blk + i];
  const int q = (int)(i % V), n = q % NP;
  if (n < p.N) (q < NP ? p.dB : p.dC)[(i / V) * p.N + n] = s;
}

unsigned blocks_for(int64_t n) { return (unsigned)((n + kSsmBlock - 1) / kSsmBlock); }

template <int NP>
void launch_ssm_t(const SsmParams& p, bool bwd, hipStream_t stream) {
  constexpr int HS = NP > 8 ? 2 : 8;  // register budget: 2 waves per SIMD at NP = 16
  const dim3 grid((unsigned)(p.ndblk * p.nc * p.nb)), block(kSsmBlock);
  const dim3 cgrid(blocks_for(p.nb * NP * p.Dm));
  if (!bwd) {
    hipLaunchKernelGGL((ssm_fwd_local_kernel<NP>), grid, block, 0, stream, p);
    hipLaunchKernelGGL((ssm_carry_kernel<false>), cgrid, block, 0, stream, p, NP, p.hc);
    hipLaunchKernelGGL((ssm_fwd_out_kernel<NP>), grid, block, 0, stream, p);
  } else {
    hipLaunchKernelGGL((ssm_bwd_local_kernel<NP>), grid, block, 0, stream, p);
    hipLaunchKernelGGL((ssm_carry_kernel<true>), cgrid, block, 0, stream, p, NP, p.gc);
    hipLaunchKernelGGL((ssm_bwd_chunk_kernel<NP, HS>), grid, block, 0, stream, p);
    const int64_t ncol = (int64_t)(NP + 1) * p.Dm;
    hipLaunchKernelGGL(ssm_reduce_dad_kernel, dim3((unsigned)((ncol + 63) / 64)), block, 0,
                       stream, p, NP);
    hipLaunchKernelGGL(ssm_reduce_dbc_kernel, dim3(blocks_for(p.nb * p.L * 2 * NP)), block, 0,
                       stream, p, NP);
  }
}

}  // namespace

int ssm_padded_states(int N) { return N <= 4 ? 4 : N <= 8 ? 8 : N <= 16 ? 16 : 32; }

void launch_ssm(const SsmParams& p, bool bwd, hipStream_t stream) {
  switch (ssm_padded_states(p.N)) {
    case 4: launch_ssm_t<4>(p, bwd, stream); break;
    case 8: launch_ssm_t<8>(p, bwd, stream); break;
    case 16: launch_ssm_t<16>(p, bwd, stream); break;
    default: launch_ssm_t<32>(p, bwd, stream); break;
  }
}

}  // namespace nxa
