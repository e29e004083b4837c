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
//              forward states from the saved sub-chunk state (registers; 16
//              or 32 states are split over 2 or 4 lanes of a channel), then
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

// Block -> (channel block, chunk, batch); `lpc` lanes per channel.
__device__ __forceinline__ SsmBlock ssm_block(const SsmParams& p, int ndblk = 0, int lpc = 1) {
  SsmBlock k;
  if (ndblk == 0) ndblk = p.ndblk;
  const int bid = blockIdx.x;
  k.dblk = bid % ndblk;
  const int rest = bid / ndblk;
  k.c = rest % p.nc;
  k.b = rest / p.nc;
  k.d = k.dblk * (kSsmBlock / lpc) + threadIdx.x / lpc;
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

// The chunk's rows of a [nb, L, N] matrix (B or C) into LDS, zero-padded to
// NP states and past the end of the sequence.  Every thread of the block
// takes part; the caller synchronises.
template <int NP>
__device__ __forceinline__ void stage_rows(const SsmParams& p, const SsmBlock& k,
                                           const float* src, float (*dst)[NP]) {
  for (int e = threadIdx.x; e < kSsmChunk * NP; e += kSsmBlock) {
    const int j = e / NP, n = e % NP, t = k.t0 + j;
    dst[j][n] = (t < k.t1 && n < p.N) ? src[((int64_t)k.b * p.L + t) * p.N + n] : 0.f;
  }
}

// The lane's values of a [nb, L, Dm] tensor over KP steps of the chunk from
// step j0, all loads issued at once (steps past the end are left unset and
// never read).
constexpr int kSsmPart = 16;

template <int KP>
__device__ __forceinline__ void load_part(const SsmParams& p, const SsmBlock& k, int d, int j0,
                                          const float* src, float (&r)[KP]) {
  const float* base = src + ((int64_t)k.b * p.L + k.t0 + j0) * p.Dm + d;
#pragma unroll
  for (int j = 0; j < KP; ++j)
    if (k.t0 + j0 + j < k.t1) r[j] = base[(int64_t)j * p.Dm];
}

// (1) Local forward scan of a chunk from zero: end state and sum(delta).
template <int NP>
__global__ __launch_bounds__(kSsmBlock) void ssm_fwd_local_kernel(const SsmParams p) {
  __shared__ float sB[kSsmChunk][NP];
  const SsmBlock k = ssm_block(p);
  stage_rows<NP>(p, k, p.B, sB);
  __syncthreads();
  if (k.d >= p.Dm) return;
  float al[NP], h[NP];
  load_al<NP>(p, k.d, true, al);
#pragma unroll
  for (int n = 0; n < NP; ++n) h[n] = 0.f;
  float sdt = 0.f;
#pragma unroll 1
  for (int j0 = 0; j0 < kSsmChunk; j0 += kSsmPart) {
    float dr[kSsmPart], xr[kSsmPart];
    load_part(p, k, k.d, j0, p.delta, dr);
    load_part(p, k, k.d, j0, p.x, xr);
#pragma unroll
    for (int j = 0; j < kSsmPart; ++j) {
      if (k.t0 + j0 + j < k.t1) {
        const float dt = dr[j], dx = dt * xr[j];
#pragma unroll
        for (int n = 0; n < NP; ++n)
          h[n] = __builtin_fmaf(fexp2(dt * al[n]), h[n], dx * sB[j0 + j][n]);
        sdt += dt;
      }
    }
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
#pragma unroll 8
  for (int k = 0; k < p.nc; ++k) {
    const int c = REV ? p.nc - 1 - k : k;
    const int64_t ci = (b * p.nc + c) * per_b + nd;
    const float loc = buf[ci];
    buf[ci] = H;
    H = __builtin_fmaf(fexp2(al * p.sdt[(b * p.nc + c) * p.Dm + d]), H, loc);
  }
}

// (3) Output pass: each chunk from its entering state; y, and the state
// entering each 8-step sub-chunk when p.hs is set.
template <int NP>
__global__ __launch_bounds__(kSsmBlock) void ssm_fwd_out_kernel(const SsmParams p) {
  __shared__ float sB[kSsmChunk][NP], sC[kSsmChunk][NP];
  const SsmBlock k = ssm_block(p);
  stage_rows<NP>(p, k, p.B, sB);
  stage_rows<NP>(p, k, p.C, sC);
  __syncthreads();
  if (k.d >= p.Dm) return;
  float al[NP], h[NP];
  load_al<NP>(p, k.d, true, al);
  const int64_t cb = ((int64_t)k.b * p.nc + k.c) * NP;
#pragma unroll
  for (int n = 0; n < NP; ++n) h[n] = p.hc[(cb + n) * p.Dm + k.d];
  const float Dd = p.D ? p.D[k.d] : 0.f;
  float* yb = p.y + ((int64_t)k.b * p.L + k.t0) * p.Dm + k.d;
#pragma unroll 1
  for (int j0 = 0; j0 < kSsmChunk; j0 += kSsmPart) {
    float dr[kSsmPart], xr[kSsmPart];
    load_part(p, k, k.d, j0, p.delta, dr);
    load_part(p, k, k.d, j0, p.x, xr);
#pragma unroll
    for (int jj = 0; jj < kSsmPart; ++jj) {
      const int j = j0 + jj, t = k.t0 + j;
      if (t < k.t1) {
        if (jj % kSsmSub == 0 && p.hs) {
          const int64_t sb = ((int64_t)k.b * p.ns + t / kSsmSub) * NP;
#pragma unroll
          for (int n = 0; n < NP; ++n) p.hs[(sb + n) * p.Dm + k.d] = h[n];
        }
        const float dt = dr[jj], dx = dt * xr[jj];
        float y = 0.f;
#pragma unroll
        for (int n = 0; n < NP; ++n) {
          h[n] = __builtin_fmaf(fexp2(dt * al[n]), h[n], dx * sB[j][n]);
          y = __builtin_fmaf(sC[j][n], h[n], y);
        }
        yb[(int64_t)j * p.Dm] = __builtin_fmaf(Dd, xr[jj], y);
      }
    }
  }
}

// (4) Local reverse scan of a chunk from adjoint 0: a_{t0} g_{t0} and
// sum(delta).
template <int NP>
__global__ __launch_bounds__(kSsmBlock) void ssm_bwd_local_kernel(const SsmParams p) {
  __shared__ float sC[kSsmChunk][NP];
  const SsmBlock k = ssm_block(p);
  stage_rows<NP>(p, k, p.C, sC);
  __syncthreads();
  if (k.d >= p.Dm) return;
  float al[NP], gh[NP];
  load_al<NP>(p, k.d, true, al);
#pragma unroll
  for (int n = 0; n < NP; ++n) gh[n] = 0.f;
  float sdt = 0.f;
#pragma unroll 1
  for (int j0 = kSsmChunk - kSsmPart; j0 >= 0; j0 -= kSsmPart) {
    float dr[kSsmPart], gr[kSsmPart];
    load_part(p, k, k.d, j0, p.delta, dr);
    load_part(p, k, k.d, j0, p.dy, gr);
#pragma unroll
    for (int jj = kSsmPart - 1; jj >= 0; --jj) {
      if (k.t0 + j0 + jj < k.t1) {
        const float dt = dr[jj], dyv = gr[jj];
#pragma unroll
        for (int n = 0; n < NP; ++n)
          gh[n] = fexp2(dt * al[n]) * __builtin_fmaf(sC[j0 + jj][n], dyv, gh[n]);
        sdt += dt;
      }
    }
  }
  const int64_t cb = ((int64_t)k.b * p.nc + k.c) * NP;
#pragma unroll
  for (int n = 0; n < NP; ++n) p.gc[(cb + n) * p.Dm + k.d] = gh[n];
  p.sdt[((int64_t)k.b * p.nc + k.c) * p.Dm + k.d] = sdt;
}

// x of lane ^ m, for a lane mask m that is a compile-time constant once the
// callers' loops are unrolled, with every lane of the wave active.  Masks 1
// and 2 are DPP quad permutes (the following add takes the operand straight
// from the permute), 4 to 16 ds_swizzle xor patterns (within 32 lanes); both
// need no address arithmetic, unlike ds_bpermute.  Mask 32 falls back to
// the generic shuffle.
__device__ __forceinline__ float lane_xor(float x, int m) {
  const int xi = __float_as_int(x);
  if (m == 1)
    return __int_as_float(__builtin_amdgcn_mov_dpp(xi, 0xB1, 0xF, 0xF, false));  // [1,0,3,2]
  if (m == 2)
    return __int_as_float(__builtin_amdgcn_mov_dpp(xi, 0x4E, 0xF, 0xF, false));  // [2,3,0,1]
  if (m == 4) return __int_as_float(__builtin_amdgcn_ds_swizzle(xi, 0x1F | (4 << 10)));
  if (m == 8) return __int_as_float(__builtin_amdgcn_ds_swizzle(xi, 0x1F | (8 << 10)));
  if (m == 16) return __int_as_float(__builtin_amdgcn_ds_swizzle(xi, 0x1F | (16 << 10)));
  return __shfl_xor(x, m, 64);
}

// Sums v[0..V) over the lanes of a wave that share lane % LPC (the lanes
// of one state group, one per channel).  log2(V) halving exchanges (masks
// 32 down to 2^SH, SH = 6 - log2(V)) leave each lane one value index,
// lane >> SH, summed over the lanes that share the lane's top log2(V) bits;
// exchanges over the remaining channel bits (masks 2^(SH-1) down to LPC)
// complete the sum.  The result is in the lanes whose bits between LPC and
// 2^SH are zero.
template <int V, int LPC>
__device__ __forceinline__ float wave_sum_scatter(float (&v)[V], int lane) {
  static_assert(V >= 1 && V <= 32 && (V & (V - 1)) == 0, "V: power of two <= 32");
  static_assert(V * LPC < 64, "state groups must leave channel bits to reduce");
#pragma unroll
  for (int half = V / 2, m = 32; half >= 1; half /= 2, m /= 2) {
    const bool up = lane & m;
#pragma unroll
    for (int i = 0; i < half; ++i) {
      if (m >= 16) {
        // v_permlane{32,16}_swap exchanges the upper lanes of v[i] with the
        // lower lanes of v[i + half] (partners lane ^ m): afterwards the
        // lower lane holds both lower values of index i, the upper lane both
        // values of index i + half, with no select.
        const uint32_t lo = __float_as_uint(v[i]), hi = __float_as_uint(v[i + half]);
        const auto r = m == 32 ? __builtin_amdgcn_permlane32_swap(lo, hi, false, false)
                               : __builtin_amdgcn_permlane16_swap(lo, hi, false, false);
        v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
      } else {
        // Select values, not addresses (an address select becomes a dynamic
        // register index).
        const float lo = v[i], hi = v[i + half];
        const float keep = up ? hi : lo;
        const float send = up ? lo : hi;
        v[i] = keep + lane_xor(send, m);
      }
    }
  }
  float s = v[0];
#pragma unroll
  for (int m = 32 / V; m >= LPC; m /= 2) s += lane_xor(s, m);
  return s;
}

// (6) Backward pass over one chunk, sub-chunk by sub-chunk from the last:
// the sub-chunk's 8 states are rebuilt in registers from its saved entering
// state, then walked in reverse.  LPC lanes share a channel, each with NPL
// of its states (NP = NPL * LPC), which keeps the 9 x NPL history in
// registers; dx and ddelta are summed over the LPC lanes.
template <int NPL, int LPC>
__global__ __launch_bounds__(kSsmBlock) void ssm_bwd_chunk_kernel(const SsmParams p) {
  constexpr int NP = NPL * LPC;
  constexpr int SC = kSsmSub;
  constexpr int SH = 6 - __builtin_ctz(NPL);
  __shared__ float red[kSsmChunk][kWaves][2 * NP];
  __shared__ float sB[kSsmChunk][NP], sC[kSsmChunk][NP];  // the chunk's B, C rows
  const SsmBlock k = ssm_block(p, p.ndblk_b, LPC);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int sub = tid & (LPC - 1), n0 = sub * NPL;
  const bool ok = k.d < p.Dm;  // idle lanes still take part in the sums, with zeros
  const int d = ok ? k.d : p.Dm - 1;
  const bool head = (lane & ((1 << SH) - 1) & ~(LPC - 1)) == 0;
  stage_rows<NP>(p, k, p.B, sB);
  stage_rows<NP>(p, k, p.C, sC);
  __syncthreads();
  float al[NPL], gh[NPL], dA[NPL];
#pragma unroll
  for (int i = 0; i < NPL; ++i)
    al[i] = (ok && n0 + i < p.N) ? p.A[(int64_t)d * p.N + n0 + i] * kLog2e : 0.f;
  const int64_t cb = ((int64_t)k.b * p.nc + k.c) * NP + n0;
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    gh[i] = ok ? p.gc[(cb + i) * p.Dm + d] : 0.f;
    dA[i] = 0.f;
  }
  const float Dd = (ok && p.D && sub == 0) ? p.D[d] : 0.f;  // skip term once per channel
  float dD = 0.f;
  const int nsub = (k.t1 - k.t0 + SC - 1) / SC;
  for (int s = nsub - 1; s >= 0; --s) {
    const int ts = k.t0 + s * SC;
    // hist[j]: the state entering step ts + j (hist[SC]: after the last).
    float hist[SC + 1][NPL];
    const int64_t sb = ((int64_t)k.b * p.ns + ts / SC) * NP + n0;
#pragma unroll
    for (int i = 0; i < NPL; ++i) hist[0][i] = ok ? p.hs[(sb + i) * p.Dm + d] : 0.f;
#pragma unroll
    for (int j = 0; j < SC; ++j) {
      const int t = min(ts + j, k.t1 - 1);  // states past the end are never read
      const int64_t xi = ((int64_t)k.b * p.L + t) * p.Dm + d;
      const float dt = p.delta[xi], dx = dt * p.x[xi];
      const float* Bt = sB[t - k.t0] + n0;
#pragma unroll
      for (int i = 0; i < NPL; ++i)
        hist[j + 1][i] = __builtin_fmaf(fexp2(dt * al[i]), hist[j][i], dx * Bt[i]);
    }
#pragma unroll
    for (int j = SC - 1; j >= 0; --j) {
      const int t = ts + j;
      if (t < k.t1) {  // uniform over the block
        const int64_t xi = ((int64_t)k.b * p.L + t) * p.Dm + d;
        const float dt = p.delta[xi], xv = p.x[xi], dyv = ok ? p.dy[xi] : 0.f;
        const float dtx = dt * xv;
        const float* Bt = sB[t - k.t0] + n0;
        const float* Ct = sC[t - k.t0] + n0;
        // dx = D dy + delta sum g B and ddelta = x sum g B + ln2 sum g al a h,
        // from the two sums sgb = sum g B and sga = sum g al a h.
        float sgb = 0.f, sga = 0.f;
        float v[NPL];
        // Recompute a here rather than keep the rebuild's values live.
        float dto = dt;
        asm volatile("" : "+v"(dto));
#pragma unroll
        for (int i = 0; i < NPL; ++i) {
          const float bn = Bt[i], cn = Ct[i];
          const float a = fexp2(dto * al[i]);
          const float ah = a * hist[j][i];
          const float g = __builtin_fmaf(cn, dyv, gh[i]);
          sgb = __builtin_fmaf(g, bn, sgb);
          sga = __builtin_fmaf(g * al[i], ah, sga);
          dA[i] = __builtin_fmaf(g * dt, ah, dA[i]);
          v[i] = g * dtx;  // dB_t
          gh[i] = a * g;
        }
#pragma unroll
        for (int m = 1; m < LPC; m *= 2) {
          sgb += lane_xor(sgb, m);
          sga += lane_xor(sga, m);
        }
        const float dx = __builtin_fmaf(dt, sgb, Dd * dyv);
        const float ddt = __builtin_fmaf(xv, sgb, kLn2 * sga);
        dD = __builtin_fmaf(dyv, xv, dD);
        if (ok && sub == 0) {
          p.dx[xi] = dx;
          p.ddelta[xi] = ddt;
        }
        float r = wave_sum_scatter<NPL, LPC>(v, lane);
        if (head) red[t - k.t0][wave][n0 + (lane >> SH)] = r;
#pragma unroll
        for (int i = 0; i < NPL; ++i) v[i] = dyv * hist[j + 1][i];  // dC_t
        r = wave_sum_scatter<NPL, LPC>(v, lane);
        if (head) red[t - k.t0][wave][NP + n0 + (lane >> SH)] = r;
      }
    }
  }
  if (ok) {
    // The chunk's adjoint slots are this lane's own: reuse them for the dA partials.
#pragma unroll
    for (int i = 0; i < NPL; ++i) p.gc[(cb + i) * p.Dm + d] = dA[i];
    if (sub == 0) p.dDpart[((int64_t)k.b * p.nc + k.c) * p.Dm + d] = dD;
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

// (7a) dA [Dm, N] and dD [Dm]: sums over the nb * nc chunk partials in two
// fixed-order levels.  Level 1: block (x, y) sums rows y, y + G, ... (G =
// gridDim.y) of 64 columns, four row groups combined through LDS, into
// part[y][col]; level 2 sums the G partials of each column.
__global__ __launch_bounds__(kSsmBlock) void ssm_reduce_dad_kernel(const SsmParams p, int NP) {
  __shared__ float part[kWaves][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t col = (int64_t)blockIdx.x * 64 + lane;
  const int64_t na = (int64_t)NP * p.Dm, ncol = na + p.Dm;
  const int64_t rows = p.nb * p.nc, step = (int64_t)gridDim.y * kWaves;
  float s = 0.f;
  if (col < ncol) {
    const int64_t r0 = (int64_t)blockIdx.y * kWaves + w;
    if (col < na) {
      for (int64_t r = r0; r < rows; r += step) s += p.gc[r * na + col];
    } else {
      for (int64_t r = r0; r < rows; r += step) s += p.dDpart[r * p.Dm + (col - na)];
    }
  }
  part[w][lane] = s;
  __syncthreads();
  if (w == 0 && col < ncol)
    p.dadpart[blockIdx.y * ncol + col] =
        (part[0][lane] + part[1][lane]) + (part[2][lane] + part[3][lane]);
}

__global__ __launch_bounds__(kSsmBlock) void ssm_reduce_dad2_kernel(const SsmParams p, int NP,
                                                                   int groups) {
  const int64_t col = (int64_t)blockIdx.x * kSsmBlock + threadIdx.x;
  const int64_t na = (int64_t)NP * p.Dm, ncol = na + p.Dm;
  if (col >= ncol) return;
  float s = 0.f;
  for (int g = 0; g < groups; ++g) s += p.dadpart[g * ncol + col];
  if (col < na) {
    const int n = (int)(col / p.Dm), d = (int)(col % p.Dm);
    if (n < p.N) p.dA[(int64_t)d * p.N + n] = s;
  } else if (p.dD) {
    p.dD[col - na] = s;
  }
}

// (7b) dB / dC [nb, L, N]: sums over the channel blocks.
__global__ __launch_bounds__(kSsmBlock) void ssm_reduce_dbc_kernel(const SsmParams p, int NP) {
  const int V = 2 * NP;
  const int64_t i = (int64_t)blockIdx.x * kSsmBlock + threadIdx.x;  // (b, t, q)
  const int64_t per_blk = p.nb * p.L * V;
  if (i >= per_blk) return;
  float s = 0.f;
  for (int blk = 0; blk < p.ndblk_b; ++blk) s += p.dBCpart[(int64_t)blk * per_blk + i];
  const int q = (int)(i % V), n = q % NP;
  if (n < p.N) (q < NP ? p.dB : p.dC)[(i / V) * p.N + n] = s;
}

unsigned blocks_for(int64_t n) { return (unsigned)((n + kSsmBlock - 1) / kSsmBlock); }

template <int NP>
void launch_ssm_t(const SsmParams& p, bool bwd, hipStream_t stream) {
  constexpr int NPL = NP > 8 ? 8 : NP, LPC = NP / NPL;
  const dim3 grid((unsigned)(p.ndblk * p.nc * p.nb)), block(kSsmBlock);
  const dim3 grid_b((unsigned)(p.ndblk_b * p.nc * p.nb));
  const dim3 cgrid(blocks_for(p.nb * NP * p.Dm));
  if (!bwd) {
    hipLaunchKernelGGL((ssm_fwd_local_kernel<NP>), grid, block, 0, stream, p);
    hipLaunchKernelGGL((ssm_carry_kernel<false>), cgrid, block, 0, stream, p, NP, p.hc);
    hipLaunchKernelGGL((ssm_fwd_out_kernel<NP>), grid, block, 0, stream, p);
  } else {
    hipLaunchKernelGGL((ssm_bwd_local_kernel<NP>), grid, block, 0, stream, p);
    hipLaunchKernelGGL((ssm_carry_kernel<true>), cgrid, block, 0, stream, p, NP, p.gc);
    hipLaunchKernelGGL((ssm_bwd_chunk_kernel<NPL, LPC>), grid_b, block, 0, stream, p);
    const int64_t ncol = (int64_t)(NP + 1) * p.Dm;
    hipLaunchKernelGGL(ssm_reduce_dad_kernel, dim3((unsigned)((ncol + 63) / 64), kSsmDadGroups),
                       block, 0, stream, p, NP);
    hipLaunchKernelGGL(ssm_reduce_dad2_kernel, dim3(blocks_for(ncol)), block, 0, stream, p, NP,
                       kSsmDadGroups);
    hipLaunchKernelGGL(ssm_reduce_dbc_kernel, dim3(blocks_for(p.nb * p.L * 2 * NP)), block, 0,
                       stream, p, NP);
  }
}

}  // namespace

int ssm_padded_states(int N) { return N <= 4 ? 4 : N <= 8 ? 8 : N <= 16 ? 16 : 32; }

int ssm_lanes_per_channel(int NP) { return NP > 8 ? NP / 8 : 1; }

void launch_ssm(const SsmParams& p, bool bwd, hipStream_t stream) {
  switch (ssm_padded_states(p.N)) {
    case 4: launch_ssm_t<4>(p, bwd, stream); break;
    case 8: launch_ssm_t<8>(p, bwd, stream); break;
    case 16: launch_ssm_t<16>(p, bwd, stream); break;
    default: launch_ssm_t<32>(p, bwd, stream); break;
  }
}

}  // namespace nxa
