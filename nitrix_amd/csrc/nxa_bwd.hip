// Backward pass: delta = rowsum(O * dO), the dK/dV and dQ kernels for fp32
// I/O (the 16-bit ones live in nxa_bwd16.h), the dbias reduction and the
// launchers.
// Two deterministic kernels
// (no atomics): dK/dV (+ dbias) with a grid over key tiles, and dQ with a
// grid over query tiles.  Both recompute P from the forward's LSE.
//
// Replaces the reference's backward glue and Pallas launches:
// src/nitrix/_kernels/cuda/attention.py:600-653 (delta, broadcast,
// unbroadcast), :390-499 (launches), :272-332 (dK/dV kernel), :335-387
// (dQ kernel), :517-544 (unbroadcast of dbias; folded in here as an
// in-kernel column sum or a reduction kernel).
#include "nxa_common.h"
#include "nxa_launch.h"

namespace nxa {

// ---------------------------------------------------------------------------
// ndelta[b, h, q] = -sum_d O[q, d] * dO[q, d]  (fp32) and nlse2 = -lse * log2(e),
// so the backward kernels stream both per-row values straight from memory
// (negated: the 16-bit kernels start their MFMA accumulators at them).  The
// fp32 kernels need it; with 16-bit I/O the dQ kernel computes both for its
// own rows instead, and runs first.
// 16 lanes per row.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void delta_kernel(const Params p) {
  using Frag = typename Mma<T>::Frag;
  constexpr int EPC = Mma<T>::EPC;
  const int rows = p.B * p.H * p.Lq;
  const int row = blockIdx.x * 16 + (threadIdx.x >> 4);
  const int sub = threadIdx.x & 15;
  float acc = 0.f;
  if (row < rows) {
    const int q = row % p.Lq;
    const int bh = row / p.Lq;
    const int b = bh / p.H, h = bh % p.H;
    const int64_t off = b * p.o_str[0] + h * p.o_str[1] + (int64_t)q * p.o_str[2];
    const T* o = (const T*)p.o + off;
    const T* d = (const T*)p.dout + off;
    for (int c = sub * EPC; c < p.Dv; c += 16 * EPC) {
      const Frag x = ld16(o + c), y = ld16(d + c);
#pragma unroll
      for (int j = 0; j < EPC; ++j) acc += to_f32(x[j]) * to_f32(y[j]);
    }
  }
  acc += __shfl_xor(acc, 8, 16);
  acc += __shfl_xor(acc, 4, 16);
  acc += __shfl_xor(acc, 2, 16);
  acc += __shfl_xor(acc, 1, 16);
  if (row < rows && sub == 0) {
    p.ndelta[row] = -acc;
    p.nlse2[row] = -p.lse[row] * kLog2e;
  }
}

// Loads a [ROWS x DP] tile (rows r0.., unit-stride head dim) into a row-major
// LDS tile `dst` (row stride SK) and, when TRANS, also into a transposed LDS
// tile `dstT` (row stride STT, row index = head dim).
template <typename T, int DP, int ROWS, int SK, int STT, bool TRANS>
__device__ __forceinline__ void load_tile(const T* src, int64_t rs, int r0,
                                          int nrows, int D, T* dst, T* dstT,
                                          int tid) {
  using Frag = typename Mma<T>::Frag;
  constexpr int EPC = Mma<T>::EPC;
  constexpr int CPR = DP / EPC;
#pragma unroll
  for (int i = tid; i < ROWS * CPR; i += 256) {
    const int r = i / CPR, cc = i % CPR;
    const int d = cc * EPC;
    Frag x = zero_frag<T>();
    if (r0 + r < nrows && d < D) x = ld16(src + (int64_t)(r0 + r) * rs + d);
    *reinterpret_cast<Frag*>(&dst[r * SK + d]) = x;
    if constexpr (TRANS) {
#pragma unroll
      for (int j = 0; j < EPC; ++j) dstT[(d + j) * STT + r] = x[j];
    }
  }
}

__device__ __forceinline__ void store_dbias(const Params& p, int64_t off,
                                            float x) {
  store_elem(p.dbias_f32 ? kF32 : p.bias_dtype, p.dbias, off, x);
}

// ---------------------------------------------------------------------------
// dK / dV (and dbias), fp32 I/O.  Block = 4 waves x 32 keys; loops over query tiles
// (64 queries; 32 at DP = 256, to fit LDS).  Each wave computes S = Q K^T and
// dP = dO V^T with the key as the lane's column, so P and dS feed
// dV^T = dO^T P and dK^T = Q^T dS as reduction operands straight from
// registers.  OUT selects the outputs (kOutDv, kOutDk = dK and dbias, or
// both) and CW the head-dim columns accumulated (kColAll, or one half:
// kColLo / kColHi).  At DP = 256 dV and dK take passes of their own (dK
// two, one per half), so that the stationary K and V and one set of
// accumulators fit a wave's 512 registers; dbias comes with the first dK
// pass.
// ---------------------------------------------------------------------------
enum : int { kOutDv = 1, kOutDk = 2, kOutBoth = 3 };
enum : int { kColAll = 0, kColLo = 1, kColHi = 2 };

template <typename T, int DP, int OUT, int CW = kColAll>
__global__ __launch_bounds__(256) void dkdv_kernel(const Params p) {
  using M = Mma<T>;
  using Frag = typename M::Frag;
  constexpr int EPC = M::EPC, KC = M::KC;
  constexpr int BNK = 128, BQ = DP > 128 ? 32 : 64;
  constexpr int NQB = BQ / 32;  // 32-query blocks per tile
  constexpr bool DV = OUT & kOutDv, DK = OUT & kOutDk;
  constexpr bool DBIAS = DK && CW != kColHi;  // dbias in this pass
  constexpr int SK = DP + EPC;
  constexpr int ST = BQ + 4;
  constexpr int NC = DP / KC;
  constexpr int NDB = DP / 32;
  constexpr int NDW = CW == kColAll ? NDB : NDB / 2;  // 32-column blocks accumulated
  constexpr int DB0 = CW == kColHi ? NDB / 2 : 0;     // the first of them
  constexpr int FPB = M::FRAGS_PER_BLOCK;
  __shared__ __attribute__((aligned(16))) T Qs[BQ * SK];
  __shared__ __attribute__((aligned(16))) T Qt[DP * ST];
  __shared__ __attribute__((aligned(16))) T Ds[BQ * SK];
  __shared__ __attribute__((aligned(16))) T Dt[DP * ST];
  __shared__ float lse_s[BQ], dlt_s[BQ];

  const int vid = xcd_remap(blockIdx.x, p.nbh, p.nkt);
  const int bh = p.bh0 + vid / p.nkt;
  const int kt = vid % p.nkt;
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, c32 = lane & 31;
  const int kblk0 = kt * BNK;
  const int kw0 = kblk0 + wave * 32;
  const int key = kw0 + c32;
  const bool kok = key < p.Lk;
  const int kclamp = kok ? key : p.Lk - 1;

  const T* qp = (const T*)p.q + b * p.q_str[0] + h * p.q_str[1];
  const T* kp = (const T*)p.k + b * p.k_str[0] + h * p.k_str[1];
  const T* vp = (const T*)p.v + b * p.v_str[0] + h * p.v_str[1];
  const T* dop = (const T*)p.dout + b * p.o_str[0] + h * p.o_str[1];
  const float* lsep = p.lse + ((int64_t)b * p.H + h) * p.Lq;
  const float* ndltp = p.ndelta + ((int64_t)b * p.H + h) * p.Lq;

  Frag kf[NC], vf[DK ? NC : 1];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int d = c * KC + g * EPC;
    kf[c] = kok && d < p.D ? ld16(kp + (int64_t)key * p.k_str[2] + d) : zero_frag<T>();
    if constexpr (DK)
      vf[c] = kok && d < p.Dv ? ld16(vp + (int64_t)key * p.v_str[2] + d) : zero_frag<T>();
  }
  f32x16 dk[DK ? NDW : 1], dv[DV ? NDW : 1];
#pragma unroll
  for (int w = 0; w < NDW; ++w)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      if constexpr (DK) dk[w][r] = 0.f;
      if constexpr (DV) dv[w][r] = 0.f;
    }
  float colsum = 0.f;

  const int64_t bbase =
      p.has_bias ? b * p.bias_str[0] + h * p.bias_str[1] + kclamp : 0;
  const uint8_t* mbase =
      p.has_mask ? p.mask + b * p.mask_str[0] + h * p.mask_str[1] + kclamp
                 : nullptr;
  const int64_t dbbase = b * p.dbias_str[0] + h * p.dbias_str[1] + key - p.dbias_off;
  const bool full_db = DBIAS && p.dbias_mode == kDbiasFull;

  const int nq = (p.Lq + BQ - 1) / BQ;
  for (int qt = 0; qt < nq; ++qt) {
    const int q0 = qt * BQ;
    bool active = !p.causal || (q0 + BQ - 1 >= kblk0);
    int cls = 3;
    if (active && p.has_tilemap)
      cls = tile_class(p, b, h, q0, q0 + BQ, kblk0, kblk0 + BNK);
    active = active && (cls & 1);
    if (!active) {
      if (full_db && kok) {
        for (int i = 0; i < BQ; ++i)
          if (q0 + i < p.Lq) store_dbias(p, dbbase + (int64_t)(q0 + i) * p.dbias_str[2], 0.f);
      }
      continue;
    }
    __syncthreads();
    load_tile<T, DP, BQ, SK, ST, true>(qp, p.q_str[2], q0, p.Lq, p.D, Qs, Qt, tid);
    load_tile<T, DP, BQ, SK, ST, true>(dop, p.o_str[2], q0, p.Lq, p.Dv, Ds, Dt, tid);
    if (tid < BQ) {
      const int q = q0 + tid;
      lse_s[tid] = q < p.Lq ? lsep[q] * kLog2e : 0.f;
      dlt_s[tid] = q < p.Lq ? -ndltp[q] : 0.f;
    }
    __syncthreads();

    f32x16 s[NQB], dp[NQB];
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[qb][r] = 0.f;
        dp[qb][r] = 0.f;
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int off = (qb * 32 + c32) * SK + c * KC + g * EPC;
        M::run(s[qb], ld16(&Qs[off]), kf[c]);
        if constexpr (DK) M::run(dp[qb], ld16(&Ds[off]), vf[c]);
      }
    }

    const bool need_mask = p.has_mask && !(cls & 2);
    const bool diag = p.causal && (kw0 + 31 > q0);
    const bool tail = (q0 + BQ > p.Lq) || (kw0 + 32 > p.Lk);
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int ql = qb * 32 + 8 * (r / 4) + 4 * g + (r % 4);
        const int q = q0 + ql;
        const int qc = q < p.Lq ? q : p.Lq - 1;
        float x = s[qb][r] * p.scale_log2;
        if (p.has_bias) {
          const int64_t off = bbase + (int64_t)qc * p.bias_str[2];
          const float bv = load_elem(p.bias_dtype, p.bias, off);
          x = __builtin_fmaf(bv, kLog2e, x);
        }
        bool keep = true;
        if (need_mask) keep = mbase[(int64_t)qc * p.mask_str[2]] != 0;
        if (tail) keep = keep && q < p.Lq && kok;
        if (diag) keep = keep && key <= q;
        const float pr = keep ? fast_exp2(x - lse_s[ql]) : 0.f;
        const float ds = pr * (dp[qb][r] - dlt_s[ql]);
        s[qb][r] = pr;
        dp[qb][r] = ds;
        if (full_db && kok && q < p.Lq)
          store_dbias(p, dbbase + (int64_t)q * p.dbias_str[2], ds);
        if constexpr (DBIAS) colsum += ds;
      }

#pragma unroll
    for (int w = 0; w < NDW; ++w) {
      const int db = DB0 + w;
      const T* rowd = &Dt[(db * 32 + c32) * ST];
      const T* rowq = &Qt[(db * 32 + c32) * ST];
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb)
#pragma unroll
        for (int f = 0; f < FPB; ++f) {
          if constexpr (DV)
            M::run(dv[w], lds_frag_t<T>(rowd + qb * 32, g, f), M::pack(s[qb], f));
          if constexpr (DK)
            M::run(dk[w], lds_frag_t<T>(rowq + qb * 32, g, f), M::pack(dp[qb], f));
        }
    }
  }

  if (kok) {
    T* dkp = (T*)p.dk + b * p.k_str[0] + h * p.k_str[1] + (int64_t)key * p.k_str[2];
    T* dvp = (T*)p.dv + b * p.v_str[0] + h * p.v_str[1] + (int64_t)key * p.v_str[2];
#pragma unroll
    for (int w = 0; w < NDW; ++w)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d0 = (DB0 + w) * 32 + 8 * c + 4 * g;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if constexpr (DK)
            if (d0 < p.D) dkp[d0 + j] = from_f32<T>(dk[w][4 * c + j] * p.scale);
          if constexpr (DV)
            if (d0 < p.Dv) dvp[d0 + j] = from_f32<T>(dv[w][4 * c + j]);
        }
      }
  }
  if (DBIAS && p.dbias_mode == kDbiasColsum) {
    const float tot = colsum + shfl_xor32(colsum);
    if (kok && g == 0) store_dbias(p, dbbase, tot);
  }
}

// ---------------------------------------------------------------------------
// dQ.  Block = 4 waves x 32 queries; loops over 64-key tiles.  Each wave
// computes S^T = K Q^T and dP^T = V dO^T (query = lane column) so dS^T feeds
// dQ^T = K^T dS^T from registers.
// ---------------------------------------------------------------------------
// CW as in dkdv_kernel: at DP = 256 fp32 dQ takes two passes, one per half of
// its columns (the stationary Q and dO fill half of a wave's registers).
template <typename T, int DP, int CW = kColAll>
__global__ __launch_bounds__(256) void dq_kernel(const Params p) {
  using M = Mma<T>;
  using Frag = typename M::Frag;
  constexpr int EPC = M::EPC, KC = M::KC;
  constexpr int BM = 128, BN = DP > 128 ? 32 : 64;
  constexpr int NKB = BN / 32;  // 32-key blocks per tile
  constexpr int SK = DP + EPC;
  constexpr int ST = BN + 4;
  constexpr int NC = DP / KC;
  constexpr int NDB = DP / 32;
  constexpr int NDW = CW == kColAll ? NDB : NDB / 2;
  constexpr int DB0 = CW == kColHi ? NDB / 2 : 0;
  constexpr int FPB = M::FRAGS_PER_BLOCK;
  __shared__ __attribute__((aligned(16))) T Ks[BN * SK];
  __shared__ __attribute__((aligned(16))) T Vs[BN * SK];
  __shared__ __attribute__((aligned(16))) T Kt[DP * ST];

  const int vid = xcd_remap(blockIdx.x, p.B * p.H, p.nqt);
  const int bh = vid / p.nqt;
  const int qt = p.nqt - 1 - (vid % p.nqt);
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, c32 = lane & 31;
  const int q0 = qt * BM;
  const int qw0 = q0 + wave * 32;
  const int qrow = qw0 + c32;
  const bool qok = qrow < p.Lq;
  const int qclamp = qok ? qrow : p.Lq - 1;

  const T* qp = (const T*)p.q + b * p.q_str[0] + h * p.q_str[1];
  const T* kp = (const T*)p.k + b * p.k_str[0] + h * p.k_str[1];
  const T* vp = (const T*)p.v + b * p.v_str[0] + h * p.v_str[1];
  const T* dop = (const T*)p.dout + b * p.o_str[0] + h * p.o_str[1];

  Frag qf[NC], df[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int d = c * KC + g * EPC;
    qf[c] = qok && d < p.D ? ld16(qp + (int64_t)qrow * p.q_str[2] + d) : zero_frag<T>();
    df[c] = qok && d < p.Dv ? ld16(dop + (int64_t)qrow * p.o_str[2] + d) : zero_frag<T>();
  }
  const int64_t rowid = ((int64_t)b * p.H + h) * p.Lq + qclamp;
  const float lse2 = p.lse[rowid] * kLog2e;
  const float dlt = -p.ndelta[rowid];

  f32x16 dq[NDW];
#pragma unroll
  for (int w = 0; w < NDW; ++w)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[w][r] = 0.f;

  int k_end = p.Lk;
  if (p.causal) k_end = min(k_end, q0 + BM);
  const int nkt = (k_end + BN - 1) / BN;
  const int64_t brow =
      p.has_bias ? b * p.bias_str[0] + h * p.bias_str[1] +
                       (int64_t)qclamp * p.bias_str[2]
                 : 0;
  const uint8_t* mrow =
      p.has_mask ? p.mask + b * p.mask_str[0] + h * p.mask_str[1] +
                       (int64_t)qclamp * p.mask_str[2]
                 : nullptr;

  for (int kt = 0; kt < nkt; ++kt) {
    const int k0 = kt * BN;
    int cls = 3;
    if (p.has_tilemap) cls = tile_class(p, b, h, q0, q0 + BM, k0, k0 + BN);
    if (!(cls & 1)) continue;
    __syncthreads();
    load_tile<T, DP, BN, SK, ST, true>(kp, p.k_str[2], k0, p.Lk, p.D, Ks, Kt, tid);
    load_tile<T, DP, BN, SK, ST, false>(vp, p.v_str[2], k0, p.Lk, p.Dv, Vs, nullptr, tid);
    __syncthreads();

    f32x16 s[NKB], dp[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[kb][r] = 0.f;
        dp[kb][r] = 0.f;
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int off = (kb * 32 + c32) * SK + c * KC + g * EPC;
        M::run(s[kb], ld16(&Ks[off]), qf[c]);
        M::run(dp[kb], ld16(&Vs[off]), df[c]);
      }
    }

    const bool need_mask = p.has_mask && !(cls & 2);
    const bool diag = p.causal && (k0 + BN - 1 > qw0);
    const bool tail = k0 + BN > p.Lk;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int key0 = k0 + kb * 32 + 8 * c + 4 * g;
        f32x4 bv = {0.f, 0.f, 0.f, 0.f};
        if (p.has_bias) bv = load_bias4(p, p.bias, brow + key0, p.Lk - key0);
        uint32_t mw = 0x01010101u;
        if (need_mask) mw = load_mask4(p, mrow + key0, p.Lk - key0);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int kk = key0 + j;
          float x = s[kb][4 * c + j] * p.scale_log2;
          x = __builtin_fmaf(bv[j], kLog2e, x);
          bool keep = mask_bit(mw, j) && qok;
          if (tail) keep = keep && kk < p.Lk;
          if (diag) keep = keep && kk <= qrow;
          const float pr = keep ? fast_exp2(x - lse2) : 0.f;
          dp[kb][4 * c + j] = pr * (dp[kb][4 * c + j] - dlt);
        }
      }

#pragma unroll
    for (int w = 0; w < NDW; ++w) {
      const T* row = &Kt[((DB0 + w) * 32 + c32) * ST];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int f = 0; f < FPB; ++f)
          M::run(dq[w], lds_frag_t<T>(row + kb * 32, g, f), M::pack(dp[kb], f));
    }
  }

  if (qok) {
    T* dqp = (T*)p.dq + b * p.q_str[0] + h * p.q_str[1] + (int64_t)qrow * p.q_str[2];
#pragma unroll
    for (int w = 0; w < NDW; ++w)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d0 = (DB0 + w) * 32 + 8 * c + 4 * g;
        if (d0 < p.D) {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            dqp[d0 + j] = from_f32<T>(dq[w][4 * c + j] * p.scale);
        }
      }
  }
}

// ---------------------------------------------------------------------------
// dbias reduction over broadcast batch / head axes, one chunk of (batch, head)
// pairs at a time.  The dK/dV launch of a chunk writes the fp32 partials of
// its pairs bh0 .. bh0 + nbh - 1 as [nbh, LQ, Lk] (slot = pair - bh0); this
// kernel adds them into the fp32 accumulator acc [OB, OH, LQ, Lk] (starting
// from zero for the first chunk) and, for the last chunk, writes the sums to
// `out` in the bias dtype.  Each output element adds its pairs in increasing
// pair order whatever the chunk size, so the result is deterministic and
// does not depend on the chunking.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void dbias_reduce_kernel(DbiasReduce r) {
  const int64_t n = (int64_t)r.OB * r.OH * r.LQ * r.Lk;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int k = i % r.Lk;
  int64_t t = i / r.Lk;
  const int q = t % r.LQ;
  t /= r.LQ;
  const int oh = t % r.OH;
  const int ob = t / r.OH;
  const int bh1 = r.bh0 + r.nbh;
  // Pairs (b, h) of this output: every b when the bias is shared over the
  // batch (OB == 1), else b = ob; likewise for h.  Restricted to the chunk.
  const int b_lo = max(r.OB == 1 ? 0 : ob, r.bh0 / r.H);
  const int b_hi = min(r.OB == 1 ? r.B - 1 : ob, (bh1 - 1) / r.H);
  float sum = r.first ? 0.f : r.acc[i];
  const int64_t slot = (int64_t)r.LQ * r.Lk;
  for (int b = b_lo; b <= b_hi; ++b) {
    const int h_lo = max(r.OH == 1 ? 0 : oh, r.bh0 - b * r.H);
    const int h_hi = min(r.OH == 1 ? r.H - 1 : oh, bh1 - 1 - b * r.H);
    for (int h = h_lo; h <= h_hi; ++h)
      sum += r.part[(int64_t)(b * r.H + h - r.bh0) * slot + (int64_t)q * r.Lk + k];
  }
  if (r.last)
    store_elem(r.dtype, r.out, ob * r.s[0] + oh * r.s[1] + q * r.s[2] + k, sum);
  else
    r.acc[i] = sum;
}

// ---------------------------------------------------------------------------
// Host launchers.
// ---------------------------------------------------------------------------
void launch_delta(const Params& p, int io_dtype, hipStream_t stream) {
  (void)io_dtype;  // fp32 only: 16-bit backward passes compute it in dQ
  const int rows = p.B * p.H * p.Lq;
  const int n = (rows + 15) / 16;
  hipLaunchKernelGGL(delta_kernel<float>, dim3(n), dim3(256), 0, stream, p);
}

template <typename T, int DP, int OUT, int CW = kColAll>
static void launch_dkdv_t(Params p, hipStream_t stream) {
  p.nkt = (p.Lk + 127) / 128;
  const int n = p.nbh * p.nkt;
  hipLaunchKernelGGL((dkdv_kernel<T, DP, OUT, CW>), dim3(n), dim3(256), 0, stream, p);
}

void launch_dkdv(const Params& p, int io_dtype, int dp, hipStream_t stream) {
  if (io_dtype == kBF16 || io_dtype == kF16) {
    launch_dkdv16(p, io_dtype, dp, stream);
  } else if (!launch_dkdv32(p, dp, stream)) {
    if (dp == 256) {
      // fp32 at DP = 256: dV, then dK in two column halves.
      launch_dkdv_t<float, 256, kOutDv>(p, stream);
      launch_dkdv_t<float, 256, kOutDk, kColLo>(p, stream);
      launch_dkdv_t<float, 256, kOutDk, kColHi>(p, stream);
    } else if (dp == 64) {
      launch_dkdv_t<float, 64, kOutBoth>(p, stream);
    } else {
      launch_dkdv_t<float, 128, kOutBoth>(p, stream);
    }
  }
}

template <typename T, int DP, int CW = kColAll>
static void launch_dq_t(Params p, hipStream_t stream) {
  p.nqt = (p.Lq + 127) / 128;
  const int n = p.B * p.H * p.nqt;
  hipLaunchKernelGGL((dq_kernel<T, DP, CW>), dim3(n), dim3(256), 0, stream, p);
}

void launch_dq(const Params& p, int io_dtype, int dp, hipStream_t stream) {
  if (io_dtype == kBF16 || io_dtype == kF16) {
    launch_dq16(p, io_dtype, dp, stream);
  } else if (!launch_dq32(p, dp, stream)) {
    if (dp == 256) {
      // fp32 dQ at DP = 256: one pass per half of its columns.
      launch_dq_t<float, 256, kColLo>(p, stream);
      launch_dq_t<float, 256, kColHi>(p, stream);
    } else if (dp == 64) {
      launch_dq_t<float, 64>(p, stream);
    } else {
      launch_dq_t<float, 128>(p, stream);
    }
  }
}

void launch_dbias_reduce(const DbiasReduce& r, hipStream_t stream) {
  const int64_t n = (int64_t)r.OB * r.OH * r.LQ * r.Lk;
  const int nb = (int)((n + 255) / 256);
  hipLaunchKernelGGL(dbias_reduce_kernel, dim3(nb), dim3(256), 0, stream, r);
}

}  // namespace nxa
