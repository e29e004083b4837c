// fp32 attention kernels (forward, dK / dV and dQ) at padded head dims 64,
// 128 and 256.
//
// Same math as the 16-bit kernels and the reference's Pallas kernels
// (src/nitrix/_kernels/cuda/attention.py:85-156 forward, :272-332 dK/dV,
// :335-387 dQ, :159-264 and :390-499 launches): online base-2 softmax with
// an fp32 log-sum-exp in the forward; in the backward P = exp2(S scale
// log2(e) - lse log2(e)) recomputed from it, dS = P (dP - delta),
// dV = P^T dO, dK = scale dS^T Q, dQ = scale dS K; fp32 throughout
// (v_mfma_f32_32x32x2_f32).
//
// fp32 MFMAs take 64 cycles for 4,096 flops, so these kernels are bound by
// the matrix core, not by LDS or VALU issue: a block of 4 waves (one per
// SIMD, up to 512 registers each) holds its 128 queries (forward, dQ) or
// keys (dK/dV) stationary and streams the other side's [64 x DP] fp32 tiles
// ([32 x DP] at head dim 256) through a double-buffered LDS ring, filled by
// direct global -> LDS copies one tile ahead while the current one is
// consumed.  No transposed copies
// are made: the products that contract over the streamed rows (O^T = V^T
// P^T, dV^T = dO^T P, dK^T = Q^T dS, dQ^T = K^T dS^T) read their A operand
// as four ds_read_b32 per fragment from the row-major tile -- bandwidth the
// 64-cycle MFMAs leave to spare.  The tiles' 16-byte chunks are XOR-swizzled by row (chunk c of
// row r at c ^ swz32(r)), which keeps both access patterns free of bank
// conflicts: 16 consecutive rows of 16-byte reads, and 32 consecutive
// columns of rows r and r + 4 (r % 8 < 4) of 4-byte reads.
#include "nxa_common.h"
#include "nxa_launch.h"

namespace nxa {

namespace {

constexpr int kF32MaxTiles = 1024;  // streamed tiles listed per block

// Swizzle of fp32 tiles: bit 3 also takes bit 2 of the row, so rows r and
// r + 4 (r % 8 < 4) use different halves of the banks.
__device__ __forceinline__ int swz32(int r) {
  const int t = r & 15;
  return t ^ ((t & 4) << 1);
}

// [ROWS x DP] fp32 tiles of one [rows, D] matrix (row stride rs floats),
// 1 KB direct copies: a tile is ROWS * DP / 256 copies, CNT per wave of the
// NW; slot s of the tile holds row s / SPR, physical chunk s % SPR, i.e.
// logical chunk (s % SPR) ^ swz32(row).  Head-dim chunks past D read chunk
// 0 (finite filler multiplied by the zero padding of the stationary side or
// never stored); rows past the range's end read zero.  COMPACT keeps one
// swizzle period (16 rows) of lane offsets and adds the uniform 16-row step
// at the copy, for kernels short of registers.
template <int DP, int NW = 4, int ROWS = 64, bool COMPACT = false>
struct F32Stream {
  static constexpr int SPR = DP / 4;                  // 16-byte slots per row
  static constexpr int CNT = ROWS * SPR / (64 * NW);  // copies per wave per tile (NW waves copy it)
  static_assert(ROWS * SPR % (64 * NW) == 0, "tile copies split evenly over the waves");
  static constexpr int PER = 16 * SPR / (64 * NW);    // copies per 16 rows
  static constexpr int NOFF = COMPACT && PER >= 1 && CNT % PER == 0 ? PER : CNT;
  uint32_t off[NOFF];
  uint32_t step16 = 0;  // bytes of 16 rows
  __device__ __forceinline__ void init(int64_t rs, int D, int wave, int lane) {
#pragma unroll
    for (int m = 0; m < NOFF; ++m) {
      const int s = (m * NW + wave) * 64 + lane;
      const int row = s / SPR;
      const int col = ((s % SPR) ^ swz32(row)) * 4;
      off[m] = 4u * (uint32_t)(row * rs + (col < D ? col : 0));
    }
    step16 = 64u * (uint32_t)rs;
  }
  __device__ __forceinline__ void issue(i32x4 rsrc, uint32_t lds, int m, int wave) const {
    const uint32_t o = NOFF == CNT ? off[m] : off[m % NOFF] + (uint32_t)(m / NOFF) * step16;
    dma16_buf(rsrc, o, lds + (m * NW + wave) * 1024);
  }
};

// Buffer resource of tile rows r0 .. r0 + ROWS - 1 of a [n, D] matrix (row
// stride rs floats): only the rows that exist (an empty range past the end).
template <int ROWS = 64>
__device__ __forceinline__ i32x4 tile_rsrc(const float* base, int64_t rs, int r0, int n, int D) {
  const int rows = min(ROWS, n - r0);
  return make_rsrc(base + (int64_t)max(r0, 0) * rs,
                   rows > 0 ? (uint32_t)(((int64_t)(rows - 1) * rs + D) * 4) : 0u);
}

// Active tiles of a block, in order, as index | class << 16 (tile-map class
// bit0 = some entry kept, bit1 = all kept); built by wave 0 with ballots.
template <typename F>
__device__ __forceinline__ int list_tiles(uint32_t* lst, int nt, int wave, int lane, F cls) {
  __shared__ int n_s;
  if (wave == 0) {
    int base = 0;
    for (int t0 = 0; t0 < nt; t0 += 64) {
      const int t = t0 + lane;
      const int c = t < nt ? cls(t) : 0;
      const uint64_t m = __ballot(c & 1);
      if (c & 1) lst[base + __popcll(m & ((1ull << lane) - 1))] = (uint32_t)t | (uint32_t)c << 16;
      base += __popcll(m);
    }
    if (lane == 0) n_s = base;
  }
  __syncthreads();
  return n_s;
}

// Per-lane LDS offsets of the two read patterns of a swizzled fp32 tile
// (bytes from the tile's base).
//  * Row fragments: lane (g, c32) reads row j*32 + c32, head-dim elements
//    8c + 4g .. +3, logical chunk 2c + g, physical (2c + g) ^ s with
//    s = swz32(c32): 2 (c ^ (s >> 1)) + (g ^ (s & 1)).  c ^ (s >> 1) is
//    (c & ~7) + ((c & 7) ^ (s >> 1)), so eight per-lane offsets rowoff[c & 7]
//    plus an immediate (c & ~7) * 32 (+ j * 32 rows) cover every c.
//  * Transposed fragments: reduction rows q = j*32 + 8f + 4g + i (i = 0..3,
//    the row groups the accumulator layout gives fragment f), column
//    d = db*32 + c32: row q, chunk (d / 4) ^ swz32(q), element d % 4.  With
//    swz32(q) = 8 ((f & 1) ^ g) + 4g + i the chunk is
//    8 ((db & 1) ^ (f & 1) ^ g) + ((c32 / 4) ^ (4g + i)) plus the part of
//    db above bit 0, so troff[x][i] (x = (db ^ f) & 1) plus (j*32 + 8f + i)
//    rows and (db & ~1) * 128 bytes, both immediates, cover every read.
template <int DP>
struct F32Offsets {
  static constexpr int ROWB = DP * 4;
  uint32_t rowoff[8];
  uint32_t troff[2][4];
  __device__ __forceinline__ void init(int g, int c32) {
    const int s = swz32(c32);
#pragma unroll
    for (int k = 0; k < 8; ++k)
      rowoff[k] = (uint32_t)(c32 * ROWB + 32 * (k ^ (s >> 1)) + 16 * (g ^ (s & 1)));
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        troff[x][i] = (uint32_t)(4 * g * ROWB + 128 * (x ^ g) + 16 * ((c32 >> 2) ^ (4 * g + i)) +
                                 4 * (c32 & 3));
  }
  // Row fragment c of 32-row block j.
  __device__ __forceinline__ f32x4 row(uint32_t tile, int j, int c) const {
    typedef __attribute__((address_space(3))) f32x4 lds_f4;
    return *(const lds_f4*)(uintptr_t)(tile + rowoff[c & 7] + (c & ~7) * 32 + j * 32 * ROWB);
  }
  // Transposed fragment: rows j*32 + 8f + 4g + i (i = 0..3), column
  // db*32 + c32.
  __device__ __forceinline__ f32x4 tr(uint32_t tile, int j, int f, int db) const {
    typedef __attribute__((address_space(3))) float lds_f;
    f32x4 a;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      a[i] = *(const lds_f*)(uintptr_t)(tile + troff[(db ^ f) & 1][i] +
                                        (j * 32 + 8 * f + i) * ROWB + (db & ~1) * 128);
    return a;
  }
};

// Products of N independent accumulators over one 4-element reduction step,
// interleaved element by element so that consecutive MFMAs never depend on
// each other.
template <int N>
__device__ __forceinline__ void mma4n(f32x16* c, const f32x4* a, const f32x4* b) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < N; ++n) c[n] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[n][i], b[n][i], c[n], 0, 0, 0);
}

__device__ __forceinline__ f32x4 pack4(const f32x16& acc, int f) {
  return f32x4{acc[4 * f], acc[4 * f + 1], acc[4 * f + 2], acc[4 * f + 3]};
}

__device__ __forceinline__ void store_db32(const Params& p, int64_t off, float x) {
  store_elem(p.dbias_f32 ? kF32 : p.bias_dtype, p.dbias, off, x);
}

}  // namespace

// Lazy reference raise threshold of the fp32 forward (log2 units).
constexpr float kF32Slack = 8.0f;

// One key tile (BN = 64, or 32 at head dim 256) of the fp32 forward for a
// wave's 32 queries: S^T = K Q^T (K rows at `ak`), the online softmax
// against the wave's running reference, O^T += V^T P^T (V rows at `av`).
template <int DP, bool HAS_BIAS, bool CAUSAL, int BN = 64>
__device__ __forceinline__ void fwd32_tile(const Params& p, const F32Offsets<DP>& lo, uint32_t ak,
                                           uint32_t av, int k0, int cls,
                                           const f32x4 (&qf)[DP / 8], f32x16 (&oacc)[DP / 32],
                                           float& m_ref, float& l_i, int64_t brow,
                                           const uint8_t* mrow, int qrow, int qw0, int g) {
  constexpr int NKB = BN / 32, NA = 2 * NKB, NC = DP / 8, NDB = DP / 32;
  const uint32_t at = ak;
    // S^T = K Q^T: each 32-key block over two halves of the head dim
    // (independent accumulators, summed after), fragments read a step
    // ahead.
    f32x16 sacc[NA];
#pragma unroll
    for (int u = 0; u < NA; ++u)
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[u][r] = 0.f;
    {
      constexpr int NH = NC / 2;
      f32x4 a[2][NA], bq[NA];
      auto rd = [&](f32x4* x, int c) NXA_INLINE {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) x[kb] = lo.row(at, kb, c);
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) x[NKB + kb] = lo.row(at, kb, c + NH);
      };
      rd(a[0], 0);
#pragma unroll
      for (int c = 0; c < NH; ++c) {
        if (c + 1 < NH) rd(a[(c + 1) & 1], c + 1);
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) bq[kb] = qf[c];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) bq[NKB + kb] = qf[c + NH];
        mma4n<NA>(sacc, a[c & 1], bq);
      }
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2 * NA, 0);
#pragma unroll
      for (int c = 0; c + 2 < NH; ++c) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 4 * NA, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, NA, 0);
      }
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 8 * NA, 0);
    }
    f32x16 sv[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) sv[kb][r] = sacc[kb][r] + sacc[NKB + kb][r];

    // Logits.  Fast path (no bias, nothing masked in the tile): the scale
    // is folded into the exponent's FMA and the max is taken on raw scores.
    const bool need_mask = p.has_mask && !(cls & 2);
    const bool tail = k0 + BN > p.Lk;
    const bool diag = CAUSAL && (k0 + BN - 1 > qw0);
    const bool general = HAS_BIAS || need_mask || tail || diag || !(p.scale_log2 > 0.f);
    float cc = p.scale_log2;
    if (general) {
      cc = 1.0f;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int key0 = k0 + kb * 32 + 8 * c + 4 * g;
          f32x4 bv = {0.f, 0.f, 0.f, 0.f};
          if constexpr (HAS_BIAS) bv = load_bias4(p, p.bias, brow + key0, p.Lk - key0);
          uint32_t mw = 0x01010101u;
          if (need_mask) mw = load_mask4(p, mrow + key0, p.Lk - key0);
          // Every element written exactly once, masked entries a select.
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int key = key0 + e;
            float x = sv[kb][4 * c + e] * p.scale_log2;
            if constexpr (HAS_BIAS) x = __builtin_fmaf(bv[e], kLog2e, x);
            bool keep = mask_bit(mw, e) && key < p.Lk;
            if (CAUSAL) keep = keep && key <= qrow;
            sv[kb][4 * c + e] = keep ? x : -INFINITY;
          }
        }
    }
    float mt = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mt = fmaxf(mt, sv[kb][r]);
    mt = fmaxf(mt, shfl_xor32(mt)) * cc;
    const bool raise = mt > m_ref + kF32Slack;
    if (__any(raise)) {
      const float alpha = raise ? fast_exp2(m_ref - mt) : 1.f;
      m_ref = raise ? mt : m_ref;
      l_i *= alpha;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;
    }
    const float neg_m = (m_ref == -INFINITY) ? 0.f : -m_ref;
    float rs = 0.f;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float e = fast_exp2(__builtin_fmaf(sv[kb][r], cc, neg_m));
        sv[kb][r] = e;
        rs += e;
      }
    l_i += rs;

    // O^T += V^T P^T, the accumulators of NDH column blocks interleaved
    // (all NDB, or at head dim 256 one half and then the other), fragments
    // read a step ahead.
    {
      constexpr int NH = NDB > 4 ? 2 : 1, NDH = NDB / NH, NS = 4 * NKB, NU = NH * NS;
      f32x4 a[2][NDH], bb[NDH];
      auto rd = [&](f32x4* x, int u) NXA_INLINE {
        const int step = u % NS, d0 = (u / NS) * NDH;
#pragma unroll
        for (int k = 0; k < NDH; ++k) x[k] = lo.tr(av, step >> 2, step & 3, d0 + k);
      };
      rd(a[0], 0);
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        if (u + 1 < NU) rd(a[(u + 1) & 1], u + 1);
        const int step = u % NS;
#pragma unroll
        for (int k = 0; k < NDH; ++k) bb[k] = pack4(sv[step >> 2], step & 3);
        mma4n<NDH>(oacc + (u / NS) * NDH, a[u & 1], bb);
      }
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 8 * NDH, 0);
#pragma unroll
      for (int u = 0; u + 2 < NU; ++u) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 4 * NDH, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 4 * NDH, 0);
      }
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 8 * NDH, 0);
    }

}

// ---------------------------------------------------------------------------
// Forward.  Block = 4 waves x 32 queries; key tiles of 64 rows (32 at head
// dim 256, so that two stages of K and V fit the LDS).  A wave holds
// its queries' Q stationary and forms S^T = K Q^T with the query on the
// lane's column, so the row max and sum take one lane ^ 32 exchange and P^T
// feeds O^T += V^T P^T from registers.  The running max is raised only when
// a row's maximum exceeds it by more than kF32Slack (log2 units), so the
// rescale of O is rare; O and l always accumulate against the same
// reference, so the result is exact.
// ---------------------------------------------------------------------------
template <int DP, bool HAS_BIAS, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void fwd32_kernel(const Params p) {
  constexpr int BM = 128, BN = DP > 128 ? 32 : 64, NC = DP / 8, NDB = DP / 32;
  constexpr int TILE = BN * DP * 4;
  constexpr int STAGE = 2 * TILE;  // K, V
  using S = F32Stream<DP, 4, BN, (DP > 128)>;
  __shared__ __attribute__((aligned(16))) char smem[2 * STAGE];
  __shared__ uint32_t lst[kF32MaxTiles];

  const int vid = xcd_remap(blockIdx.x, p.B * p.H, p.nqt);
  const int bh = vid / p.nqt;
  const int qt = p.nqt - 1 - (vid % p.nqt);  // longest (causal) blocks first
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, c32 = lane & 31;
  const int q0 = qt * BM;
  const int qw0 = q0 + wave * 32;
  const int qrow = qw0 + c32;
  const bool qok = qrow < p.Lq;
  const int qc = qok ? qrow : p.Lq - 1;

  const float* kp = (const float*)p.k + b * p.k_str[0] + h * p.k_str[1];
  const float* vp = (const float*)p.v + b * p.v_str[0] + h * p.v_str[1];

  const int k_end = CAUSAL ? min(p.Lk, q0 + BM) : p.Lk;
  const int nk = (k_end + BN - 1) / BN;
  const int n = list_tiles(lst, nk, wave, lane, [&](int t) -> int {
    return p.has_tilemap ? tile_class(p, b, h, q0, q0 + BM, t * BN, t * BN + BN) : 3;
  });

  f32x4 qf[NC];
  {
    const float* qr = (const float*)p.q + b * p.q_str[0] + h * p.q_str[1] + (int64_t)qc * p.q_str[2];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d = 8 * c + 4 * g;
      qf[c] = qok && d < p.D ? *reinterpret_cast<const f32x4*>(qr + d) : f32x4{0, 0, 0, 0};
    }
  }
  const int64_t brow = HAS_BIAS ? b * p.bias_str[0] + h * p.bias_str[1] + (int64_t)qc * p.bias_str[2] : 0;
  const uint8_t* mrow = p.has_mask ? p.mask + b * p.mask_str[0] + h * p.mask_str[1] + (int64_t)qc * p.mask_str[2] : nullptr;

  f32x16 oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[db][r] = 0.f;
  float m_ref = -INFINITY, l_i = 0.f;

  S ks, vs_;
  ks.init(p.k_str[2], p.D, wave, lane);
  vs_.init(p.v_str[2], p.Dv, wave, lane);
  F32Offsets<DP> lo;
  lo.init(g, c32);
  const uint32_t lds0 = lds_offset(smem);
  auto issue = [&](int i, int st) NXA_INLINE {
    const int t = i < n ? (int)(lst[i] & 0xffff) : nk;
    const uint32_t at = lds0 + st * STAGE;
    const i32x4 rk = tile_rsrc<BN>(kp, p.k_str[2], t * BN, p.Lk, p.D);
    const i32x4 rv = tile_rsrc<BN>(vp, p.v_str[2], t * BN, p.Lk, p.Dv);
#pragma unroll
    for (int m = 0; m < S::CNT; ++m) {
      ks.issue(rk, at, m, wave);
      vs_.issue(rv, at + TILE, m, wave);
    }
  };

  if (n > 0) issue(0, 0);
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  __syncthreads();
  for (int i = 0; i < n; ++i) {
    const int st = i & 1;
    const uint32_t at = lds0 + st * STAGE;
    const int t = (int)(lst[i] & 0xffff), cls = (int)(lst[i] >> 16);
    const int k0 = t * BN;
    issue(i + 1, st ^ 1);

    fwd32_tile<DP, HAS_BIAS, CAUSAL, BN>(p, lo, at, at + TILE, k0, cls, qf, oacc, m_ref, l_i,
                                          brow, mrow, qrow, qw0, g);

    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __syncthreads();
  }

  // O = O / l (a fully masked row gives 0/0 = NaN, as the reference's
  // softmax over all -inf logits does), lse = ln sum exp.
  const float l = l_i + shfl_xor32(l_i);
  const float inv = 1.0f / l;
  if (qok) {
    float* op = (float*)p.o + b * p.o_str[0] + h * p.o_str[1] + (int64_t)qrow * p.o_str[2];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d0 = db * 32 + 8 * c + 4 * g;
        if (d0 < p.Dv) store4(op + d0, oacc[db], 4 * c, inv);
      }
    if (g == 0 && p.lse) p.lse[((int64_t)b * p.H + h) * p.Lq + qrow] = (m_ref + __log2f(l)) * kLn2;
  }
}

// ---------------------------------------------------------------------------
// Forward of small problems at head dim 64 (few query blocks for 256 CUs):
// the four waves of a block share 32 queries and split the key tiles
// between them (wave w takes active tiles w, w + 4, ...), each with K / V
// stages of its own; at the end the block merges the four partial results
// in LDS, O = sum_w 2^(m_w - M) O_w and l likewise with M = max_w m_w.
// Four times the blocks of the 32-query grid, the same arithmetic per tile.
// ---------------------------------------------------------------------------
template <bool HAS_BIAS, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void fwd32s_kernel(const Params p) {
  constexpr int DP = 64, BM = 32, BN = 64, NC = DP / 8, NDB = DP / 32, NW = 4;
  constexpr int TILE = BN * DP * 4;
  using S = F32Stream<DP, 1>;
  __shared__ __attribute__((aligned(16))) char smem[NW * 2 * TILE];
  __shared__ uint32_t lst[kF32MaxTiles];
  static_assert(NW * 64 * (NDB * 16 + 2) * 4 <= NW * 2 * TILE, "the merge fits the stages");

  const int vid = xcd_remap(blockIdx.x, p.B * p.H, p.nqt);
  const int bh = vid / p.nqt;
  const int qt = p.nqt - 1 - (vid % p.nqt);
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, c32 = lane & 31;
  const int q0 = qt * BM;
  const int qrow = q0 + c32;
  const bool qok = qrow < p.Lq;
  const int qc = qok ? qrow : p.Lq - 1;

  const float* kp = (const float*)p.k + b * p.k_str[0] + h * p.k_str[1];
  const float* vp = (const float*)p.v + b * p.v_str[0] + h * p.v_str[1];
  const int k_end = CAUSAL ? min(p.Lk, q0 + BM) : p.Lk;
  const int nk = (k_end + BN - 1) / BN;
  const int n = list_tiles(lst, nk, wave, lane, [&](int t) -> int {
    return p.has_tilemap ? tile_class(p, b, h, q0, q0 + BM, t * BN, t * BN + BN) : 3;
  });

  f32x4 qf[NC];
  {
    const float* qr = (const float*)p.q + b * p.q_str[0] + h * p.q_str[1] + (int64_t)qc * p.q_str[2];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d = 8 * c + 4 * g;
      qf[c] = qok && d < p.D ? *reinterpret_cast<const f32x4*>(qr + d) : f32x4{0, 0, 0, 0};
    }
  }
  const int64_t brow = HAS_BIAS ? b * p.bias_str[0] + h * p.bias_str[1] + (int64_t)qc * p.bias_str[2] : 0;
  const uint8_t* mrow = p.has_mask ? p.mask + b * p.mask_str[0] + h * p.mask_str[1] + (int64_t)qc * p.mask_str[2] : nullptr;

  f32x16 oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[db][r] = 0.f;
  float m_ref = -INFINITY, l_i = 0.f;

  S ks, vs_;
  ks.init(p.k_str[2], p.D, 0, lane);
  vs_.init(p.v_str[2], p.Dv, 0, lane);
  F32Offsets<DP> lo;
  lo.init(g, c32);
  const uint32_t at = lds_offset(smem) + wave * 2 * TILE;  // this wave's K, V
  for (int i = wave; i < n; i += NW) {
    const int t = (int)(lst[i] & 0xffff), cls = (int)(lst[i] >> 16);
    const i32x4 rk = tile_rsrc(kp, p.k_str[2], t * BN, p.Lk, p.D);
    const i32x4 rv = tile_rsrc(vp, p.v_str[2], t * BN, p.Lk, p.Dv);
#pragma unroll
    for (int m = 0; m < S::CNT; ++m) {
      ks.issue(rk, at, m, 0);
      vs_.issue(rv, at + TILE, m, 0);
    }
    // Only this wave reads its stages: its own wait publishes the copies.
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    fwd32_tile<DP, HAS_BIAS, CAUSAL>(p, lo, at, at + TILE, t * BN, cls, qf, oacc, m_ref, l_i,
                                     brow, mrow, qrow, q0, g);
    // The next copies overwrite the stages the products just read.
    __builtin_amdgcn_s_waitcnt(lgkmcnt_imm(0));
  }

  // Merge: [field][wave][lane] floats, fields O (NDB x 16), m, l.
  __syncthreads();
  float* ms = reinterpret_cast<float*>(smem);
  constexpr int F = NDB * 16 + 2;
  auto slot = [&](int f, int w) -> float& { return ms[(f * NW + w) * 64 + lane]; };
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) slot(db * 16 + r, wave) = oacc[db][r];
  slot(F - 2, wave) = m_ref;
  slot(F - 1, wave) = l_i;
  __syncthreads();
  if (wave != 0) return;
  float mw[NW], M = -INFINITY;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    mw[w] = slot(F - 2, w);
    M = fmaxf(M, mw[w]);
  }
  float sc[NW], l = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    sc[w] = mw[w] == -INFINITY ? 0.f : fast_exp2(mw[w] - M);
    l = __builtin_fmaf(slot(F - 1, w), sc[w], l);
  }
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float o = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) o = __builtin_fmaf(slot(db * 16 + r, w), sc[w], o);
      oacc[db][r] = o;
    }
  l += shfl_xor32(l);
  const float inv = 1.0f / l;
  if (qok) {
    float* op = (float*)p.o + b * p.o_str[0] + h * p.o_str[1] + (int64_t)qrow * p.o_str[2];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d0 = db * 32 + 8 * c + 4 * g;
        if (d0 < p.Dv) store4(op + d0, oacc[db], 4 * c, inv);
      }
    if (g == 0 && p.lse) p.lse[((int64_t)b * p.H + h) * p.Lq + qrow] = (M + __log2f(l)) * kLn2;
  }
}

// Outputs of one dK / dV launch.
enum : int { kF32Dv = 1, kF32Dk = 2, kF32Both = 3 };

// ---------------------------------------------------------------------------
// dK / dV (+ dbias).  Block = 4 waves x 32 keys; query tiles of 64 rows.
// A wave holds its keys' K and V stationary and forms S = Q K^T and
// dP = dO V^T with the key on the lane's column, so P and dS feed
// dV^T += dO^T P and dK^T += Q^T dS from registers.  At head dim 256 the
// stationary rows and both accumulator sets do not fit one wave's
// registers: two launches, OUT = kF32Dv (K stationary; S, P, dV) and then
// kF32Dk (K, V stationary; S, dP, dS, dK, dbias), over 32-query tiles.
// ---------------------------------------------------------------------------
template <int DP, bool CAUSAL, int OUT = kF32Both>
__global__ __launch_bounds__(256, 1) void dkdv32_kernel(const Params p) {
  constexpr bool DV = OUT & kF32Dv, DK = OUT & kF32Dk;
  static_assert(OUT == kF32Both || DP > 128, "split launches are for head dim 256");
  constexpr int BNK = 128, BQ = OUT == kF32Both ? 64 : 32, NQB = BQ / 32;
  constexpr int NC = DP / 8, NDB = DP / 32;
  constexpr int TILE = BQ * DP * 4;
  constexpr int STAGE = 2 * TILE + 2 * BQ * 4;  // Q, dO, -lse log2(e), -delta
  using S = F32Stream<DP, 4, BQ, (DP > 128)>;
  __shared__ __attribute__((aligned(16))) char smem[2 * STAGE];
  __shared__ uint32_t lst[kF32MaxTiles];

  const int vid = xcd_remap(blockIdx.x, p.nbh, p.nkt);
  const int bh = p.bh0 + vid / p.nkt;
  const int kt = vid % p.nkt;
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, c32 = lane & 31;
  const int kblk0 = kt * BNK;
  const int kw0 = kblk0 + wave * 32;
  const int key = kw0 + c32;
  const bool kok = key < p.Lk;
  const int kc = kok ? key : p.Lk - 1;

  const float* qp = (const float*)p.q + b * p.q_str[0] + h * p.q_str[1];
  const float* dop = (const float*)p.dout + b * p.o_str[0] + h * p.o_str[1];
  const float* nlp = p.nlse2 + ((int64_t)b * p.H + h) * p.Lq;
  const float* ndp = p.ndelta + ((int64_t)b * p.H + h) * p.Lq;

  const int nq = (p.Lq + BQ - 1) / BQ;
  const int n = list_tiles(lst, nq, wave, lane, [&](int t) -> int {
    const int q0 = t * BQ;
    if (CAUSAL && q0 + BQ - 1 < kblk0) return 0;
    return p.has_tilemap ? tile_class(p, b, h, q0, q0 + BQ, kblk0, kblk0 + BNK) : 3;
  });

  // Stationary K and V rows of the lane's key (B operands; V only where dP
  // is formed).
  f32x4 kf[NC], vf[NC];
  {
    const float* kr = (const float*)p.k + b * p.k_str[0] + h * p.k_str[1] + (int64_t)kc * p.k_str[2];
    const float* vr = (const float*)p.v + b * p.v_str[0] + h * p.v_str[1] + (int64_t)kc * p.v_str[2];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d = 8 * c + 4 * g;
      kf[c] = kok && d < p.D ? *reinterpret_cast<const f32x4*>(kr + d) : f32x4{0, 0, 0, 0};
      if constexpr (DK)
        vf[c] = kok && d < p.Dv ? *reinterpret_cast<const f32x4*>(vr + d) : f32x4{0, 0, 0, 0};
    }
  }
  f32x16 dk[NDB], dv[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) dk[db][r] = dv[db][r] = 0.f;
  float colsum = 0.f;

  S qs, ds_;
  qs.init(p.q_str[2], p.D, wave, lane);
  ds_.init(p.o_str[2], p.Dv, wave, lane);
  F32Offsets<DP> lo;
  lo.init(g, c32);
  const uint32_t lds0 = lds_offset(smem);

  // Copies of active tile i (empty ranges past the list) into stage st:
  // CNT Q and CNT dO copies, and BQ / 4 rows of -lse log2(e) and -delta per
  // wave (lanes 0 .. BQ / 4 - 1).
  auto issue = [&](int i, int st) NXA_INLINE {
    const int t = i < n ? (int)(lst[i] & 0xffff) : nq;
    const int q0 = t * BQ;
    const uint32_t at = lds0 + st * STAGE;
    const i32x4 rq = tile_rsrc<BQ>(qp, p.q_str[2], q0, p.Lq, p.D);
    const i32x4 ro = tile_rsrc<BQ>(dop, p.o_str[2], q0, p.Lq, p.Dv);
#pragma unroll
    for (int m = 0; m < S::CNT; ++m) {
      qs.issue(rq, at, m, wave);
      ds_.issue(ro, at + TILE, m, wave);
    }
    const int rows = max(min(BQ, p.Lq - q0), 0);
    constexpr int RW = BQ / 4;  // row values per wave
    if (lane < RW) {
      dma4_buf(make_rsrc(nlp + min(q0, p.Lq), (uint32_t)rows * 4u), 4u * (RW * wave + lane),
               at + 2 * TILE + 4 * RW * wave);
      dma4_buf(make_rsrc(ndp + min(q0, p.Lq), (uint32_t)rows * 4u), 4u * (RW * wave + lane),
               at + 2 * TILE + BQ * 4 + 4 * RW * wave);
    }
  };
  constexpr int CPT = 2 * S::CNT + 2;  // copies per wave per tile

  const int64_t bbase = p.has_bias ? b * p.bias_str[0] + h * p.bias_str[1] + kc : 0;
  const uint8_t* mbase = p.has_mask ? p.mask + b * p.mask_str[0] + h * p.mask_str[1] + kc : nullptr;
  const int64_t dbbase = b * p.dbias_str[0] + h * p.dbias_str[1] + key - p.dbias_off;
  const bool full_db = p.dbias_mode == kDbiasFull;

  if (n > 0) issue(0, 0);
  if (DK && full_db && kok) {
    // A full dbias gets zeros where no query of a tile keeps this key block.
    int li = 0;
    for (int t = 0; t < nq; ++t) {
      if (li < n && (int)(lst[li] & 0xffff) == t) {
        ++li;
        continue;
      }
      for (int q = t * BQ; q < min(t * BQ + BQ, p.Lq); ++q)
        store_db32(p, dbbase + (int64_t)q * p.dbias_str[2], 0.f);
    }
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  __syncthreads();
  for (int i = 0; i < n; ++i) {
    const int st = i & 1;
    const uint32_t at = lds0 + st * STAGE;
    const int t = (int)(lst[i] & 0xffff), cls = (int)(lst[i] >> 16);
    const int q0 = t * BQ;
    issue(i + 1, st ^ 1);

    // S = Q K^T and dP = dO V^T.  Both outputs: acc[0..1] = S of query
    // blocks 0, 1, acc[2..3] = dP.  dK: acc[0] = S, acc[1] = dP of the one
    // 32-query block.  dV: S over the low and the high half of the head
    // dim, summed after.  The A fragments of step c + 1 are read while the
    // MFMAs of step c run.
    constexpr int NA = OUT == kF32Both ? 4 : 2;
    constexpr int NSTEP = OUT == kF32Dv ? NC / 2 : NC;
    f32x16 acc[NA];
#pragma unroll
    for (int n = 0; n < NA; ++n)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[n][r] = 0.f;
    {
      f32x4 a[2][NA], bq[NA];
      auto rd = [&](f32x4* x, int c) NXA_INLINE {
        if constexpr (OUT == kF32Both) {
          x[0] = lo.row(at, 0, c);
          x[1] = lo.row(at, 1, c);
          x[2] = lo.row(at + TILE, 0, c);
          x[3] = lo.row(at + TILE, 1, c);
        } else if constexpr (OUT == kF32Dk) {
          x[0] = lo.row(at, 0, c);
          x[1] = lo.row(at + TILE, 0, c);
        } else {
          x[0] = lo.row(at, 0, c);
          x[1] = lo.row(at, 0, c + NC / 2);
        }
      };
      rd(a[0], 0);
#pragma unroll
      for (int c = 0; c < NSTEP; ++c) {
        if (c + 1 < NSTEP) rd(a[(c + 1) & 1], c + 1);
        if constexpr (OUT == kF32Both) {
          bq[0] = bq[1] = kf[c];
          bq[2] = bq[3] = vf[c];
        } else if constexpr (OUT == kF32Dk) {
          bq[0] = kf[c];
          bq[1] = vf[c];
        } else {
          bq[0] = kf[c];
          bq[1] = kf[c + NC / 2];
        }
        mma4n<NA>(acc, a[c & 1], bq);
      }
      // The next step's fragments ahead of this step's products.
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2 * NA, 0);
#pragma unroll
      for (int c = 0; c + 2 < NSTEP; ++c) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 4 * NA, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, NA, 0);
      }
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 8 * NA, 0);
    }
    if constexpr (OUT == kF32Dv) {
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[0][r] += acc[1][r];
    }
    f32x16* s = acc;
    f32x16* dp = acc + NQB;

    // P and dS, element by element (the query is the accumulator row).
    typedef __attribute__((address_space(3))) f32x4 lds_f4;
    const bool need_mask = p.has_mask && !(cls & 2);
    const bool diag = CAUSAL && (kw0 + 31 > q0);
    const bool tail = (q0 + BQ > p.Lq) || (kw0 + 32 > p.Lk);
#pragma unroll
    for (int j = 0; j < NQB; ++j)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int ql0 = j * 32 + 8 * c + 4 * g;
        const f32x4 nl = *(const lds_f4*)(uintptr_t)(at + 2 * TILE + ql0 * 4);
        const f32x4 nd = *(const lds_f4*)(uintptr_t)(at + 2 * TILE + BQ * 4 + ql0 * 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * c + e;
          const int q = q0 + ql0 + e;
          const int qc = q < p.Lq ? q : p.Lq - 1;
          float x = __builtin_fmaf(s[j][r], p.scale_log2, nl[e]);
          if (p.has_bias)
            x = __builtin_fmaf(load_elem(p.bias_dtype, p.bias, bbase + (int64_t)qc * p.bias_str[2]),
                               kLog2e, x);
          bool keep = true;
          if (need_mask) keep = mbase[(int64_t)qc * p.mask_str[2]] != 0;
          if (tail) keep = keep && q < p.Lq && kok;
          if (diag) keep = keep && key <= q;
          const float pr = keep ? fast_exp2(x) : 0.f;
          if constexpr (DV) s[j][r] = pr;
          if constexpr (DK) {
            const float dsv = pr * (dp[j][r] + nd[e]);
            dp[j][r] = dsv;
            if (full_db && kok && q < p.Lq) store_db32(p, dbbase + (int64_t)q * p.dbias_str[2], dsv);
            colsum += dsv;
          }
        }
      }

    // dV^T += dO^T P and dK^T += Q^T dS (A operands read transposed), in
    // halves of the head dim: four accumulators (dV and dK of two 32-column
    // blocks) interleaved, the fragments of the next step read during this
    // one.  A launch with one output: groups of four of its column blocks,
    // read ahead across the groups.
    if constexpr (OUT != kF32Both) {
      constexpr int NDH = 4, NS = 4 * NQB, NU = (NDB / NDH) * NS;
      f32x16* o = DV ? dv : dk;
      f32x16* pb = DV ? s : dp;
      const uint32_t src = DV ? at + TILE : at;  // dO or Q
      f32x4 a[2][NDH], bb[NDH];
      auto rd = [&](f32x4* x, int u) NXA_INLINE {
        const int step = u % NS, d0 = (u / NS) * NDH;
#pragma unroll
        for (int k = 0; k < NDH; ++k) x[k] = lo.tr(src, step >> 2, step & 3, d0 + k);
      };
      rd(a[0], 0);
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        if (u + 1 < NU) rd(a[(u + 1) & 1], u + 1);
        const int step = u % NS;
#pragma unroll
        for (int k = 0; k < NDH; ++k) bb[k] = pack4(pb[step >> 2], step & 3);
        mma4n<NDH>(o + (u / NS) * NDH, a[u & 1], bb);
      }
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 8 * NDH, 0);
#pragma unroll
      for (int u = 0; u + 2 < NU; ++u) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 4 * NDH, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 4 * NDH, 0);
      }
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 8 * NDH, 0);
    }
#pragma unroll
    for (int hb = 0; hb < (OUT == kF32Both ? NDB : 0); hb += 2) {
      constexpr int NA = NDB >= 2 ? 4 : 2;
      f32x16 o[NA];
#pragma unroll
      for (int u = 0; u < NA / 2; ++u) {
        o[u] = dv[hb + u];
        o[NA / 2 + u] = dk[hb + u];
      }
      f32x4 a[2][NA], bb[NA];
      auto rd = [&](f32x4* x, int step) NXA_INLINE {
        const int j = step >> 2, f = step & 3;
#pragma unroll
        for (int u = 0; u < NA / 2; ++u) {
          x[u] = lo.tr(at + TILE, j, f, hb + u);
          x[NA / 2 + u] = lo.tr(at, j, f, hb + u);
        }
      };
      rd(a[0], 0);
#pragma unroll
      for (int step = 0; step < 8; ++step) {
        if (step + 1 < 8) rd(a[(step + 1) & 1], step + 1);
        const int j = step >> 2, f = step & 3;
#pragma unroll
        for (int u = 0; u < NA / 2; ++u) {
          bb[u] = pack4(s[j], f);
          bb[NA / 2 + u] = pack4(dp[j], f);
        }
        mma4n<NA>(o, a[step & 1], bb);
      }
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 8 * NA, 0);
#pragma unroll
      for (int step = 0; step < 6; ++step) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 4 * NA, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 4 * NA, 0);
      }
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 8 * NA, 0);
#pragma unroll
      for (int u = 0; u < NA / 2; ++u) {
        dv[hb + u] = o[u];
        dk[hb + u] = o[NA / 2 + u];
      }
    }

    // Tile i + 1 is resident, and every wave is done with stage st, before
    // the next iteration.
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __syncthreads();
  }
  static_assert(CPT <= 63, "copies per tile fit the vmcnt counter");

  if (kok) {
    float* dkp = (float*)p.dk + b * p.k_str[0] + h * p.k_str[1] + (int64_t)key * p.k_str[2];
    float* dvp = (float*)p.dv + b * p.v_str[0] + h * p.v_str[1] + (int64_t)key * p.v_str[2];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d0 = db * 32 + 8 * c + 4 * g;
        if (DK && d0 < p.D) store4(dkp + d0, dk[db], 4 * c, p.scale);
        if (DV && d0 < p.Dv) store4(dvp + d0, dv[db], 4 * c, 1.0f);
      }
  }
  if (DK && p.dbias_mode == kDbiasColsum) {
    const float tot = colsum + shfl_xor32(colsum);
    if (kok && g == 0) store_db32(p, dbbase, tot);
  }
}

// ---------------------------------------------------------------------------
// dQ.  Block = 4 waves x 32 queries; key tiles of 64 rows (32 at head dim
// 256, so that two stages of K and V fit the LDS).  A wave holds its
// queries' Q and dO stationary and forms S^T = K Q^T and dP^T = V dO^T with
// the query on the lane's column, so dS^T feeds dQ^T += K^T dS^T.
// ---------------------------------------------------------------------------
template <int DP, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void dq32_kernel(const Params p) {
  constexpr int BM = 128, BN = DP > 128 ? 32 : 64, NKB = BN / 32, NC = DP / 8, NDB = DP / 32;
  constexpr int TILE = BN * DP * 4;
  constexpr int STAGE = 2 * TILE;  // K, V
  using S = F32Stream<DP, 4, BN, (DP > 128)>;
  __shared__ __attribute__((aligned(16))) char smem[2 * STAGE];
  __shared__ uint32_t lst[kF32MaxTiles];

  const int vid = xcd_remap(blockIdx.x, p.B * p.H, p.nqt);
  const int bh = vid / p.nqt;
  const int qt = p.nqt - 1 - (vid % p.nqt);  // longest (causal) blocks first
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, c32 = lane & 31;
  const int q0 = qt * BM;
  const int qw0 = q0 + wave * 32;
  const int qrow = qw0 + c32;
  const bool qok = qrow < p.Lq;
  const int qc = qok ? qrow : p.Lq - 1;

  const float* kp = (const float*)p.k + b * p.k_str[0] + h * p.k_str[1];
  const float* vp = (const float*)p.v + b * p.v_str[0] + h * p.v_str[1];

  const int k_end = CAUSAL ? min(p.Lk, q0 + BM) : p.Lk;
  const int nk = (k_end + BN - 1) / BN;
  const int n = list_tiles(lst, nk, wave, lane, [&](int t) -> int {
    return p.has_tilemap ? tile_class(p, b, h, q0, q0 + BM, t * BN, t * BN + BN) : 3;
  });

  f32x4 qf[NC], df[NC];
  {
    const float* qr = (const float*)p.q + b * p.q_str[0] + h * p.q_str[1] + (int64_t)qc * p.q_str[2];
    const float* dr = (const float*)p.dout + b * p.o_str[0] + h * p.o_str[1] + (int64_t)qc * p.o_str[2];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d = 8 * c + 4 * g;
      qf[c] = qok && d < p.D ? *reinterpret_cast<const f32x4*>(qr + d) : f32x4{0, 0, 0, 0};
      df[c] = qok && d < p.Dv ? *reinterpret_cast<const f32x4*>(dr + d) : f32x4{0, 0, 0, 0};
    }
  }
  const int64_t rowid = ((int64_t)b * p.H + h) * p.Lq + qc;
  const float nl2 = p.nlse2[rowid];
  const float ndl = p.ndelta[rowid];
  f32x16 dq[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[db][r] = 0.f;

  S ks, vs_;
  ks.init(p.k_str[2], p.D, wave, lane);
  vs_.init(p.v_str[2], p.Dv, wave, lane);
  F32Offsets<DP> lo;
  lo.init(g, c32);
  const uint32_t lds0 = lds_offset(smem);
  auto issue = [&](int i, int st) NXA_INLINE {
    const int t = i < n ? (int)(lst[i] & 0xffff) : nk;
    const uint32_t at = lds0 + st * STAGE;
    const i32x4 rk = tile_rsrc<BN>(kp, p.k_str[2], t * BN, p.Lk, p.D);
    const i32x4 rv = tile_rsrc<BN>(vp, p.v_str[2], t * BN, p.Lk, p.Dv);
#pragma unroll
    for (int m = 0; m < S::CNT; ++m) {
      ks.issue(rk, at, m, wave);
      vs_.issue(rv, at + TILE, m, wave);
    }
  };

  const int64_t brow = p.has_bias ? b * p.bias_str[0] + h * p.bias_str[1] + (int64_t)qc * p.bias_str[2] : 0;
  const uint8_t* mrow = p.has_mask ? p.mask + b * p.mask_str[0] + h * p.mask_str[1] + (int64_t)qc * p.mask_str[2] : nullptr;

  if (n > 0) issue(0, 0);
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  __syncthreads();
  for (int i = 0; i < n; ++i) {
    const int st = i & 1;
    const uint32_t at = lds0 + st * STAGE;
    const int t = (int)(lst[i] & 0xffff), cls = (int)(lst[i] >> 16);
    const int k0 = t * BN;
    issue(i + 1, st ^ 1);

    constexpr int NA = 2 * NKB;  // S^T of each 32-key block, then dP^T
    f32x16 acc[NA];
#pragma unroll
    for (int n = 0; n < NA; ++n)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[n][r] = 0.f;
    {
      f32x4 a[2][NA], bq[NA];
      auto rd = [&](f32x4* x, int c) NXA_INLINE {
#pragma unroll
        for (int j = 0; j < NKB; ++j) {
          x[j] = lo.row(at, j, c);
          x[NKB + j] = lo.row(at + TILE, j, c);
        }
      };
      rd(a[0], 0);
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        if (c + 1 < NC) rd(a[(c + 1) & 1], c + 1);
#pragma unroll
        for (int j = 0; j < NKB; ++j) {
          bq[j] = qf[c];
          bq[NKB + j] = df[c];
        }
        mma4n<NA>(acc, a[c & 1], bq);
      }
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2 * NA, 0);
#pragma unroll
      for (int c = 0; c + 2 < NC; ++c) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 4 * NA, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, NA, 0);
      }
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 8 * NA, 0);
    }
    f32x16* s = acc;
    f32x16* dp = acc + NKB;

    const bool need_mask = p.has_mask && !(cls & 2);
    const bool diag = CAUSAL && (k0 + BN - 1 > qw0);
    const bool tail = k0 + BN > p.Lk;
#pragma unroll
    for (int j = 0; j < NKB; ++j)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int key0 = k0 + j * 32 + 8 * c + 4 * g;
        f32x4 bv = {0.f, 0.f, 0.f, 0.f};
        if (p.has_bias) bv = load_bias4(p, p.bias, brow + key0, p.Lk - key0);
        uint32_t mw = 0x01010101u;
        if (need_mask) mw = load_mask4(p, mrow + key0, p.Lk - key0);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * c + e;
          const int kk = key0 + e;
          float x = __builtin_fmaf(s[j][r], p.scale_log2, nl2);
          x = __builtin_fmaf(bv[e], kLog2e, x);
          bool keep = mask_bit(mw, e) && qok;
          if (tail) keep = keep && kk < p.Lk;
          if (diag) keep = keep && kk <= qrow;
          const float pr = keep ? fast_exp2(x) : 0.f;
          dp[j][r] = pr * (dp[j][r] + ndl);
        }
      }

    // dQ^T += K^T dS^T, the accumulators of a group of NDH column blocks
    // interleaved (all NDB at once, or, at head dim 256, one half and then
    // the other, which halves the read-ahead registers), fragments read a
    // step ahead.
    {
      constexpr int NH = NDB > 4 ? 2 : 1, NDH = NDB / NH, NS = 4 * NKB, NU = NH * NS;
      f32x4 a[2][NDH], bb[NDH];
      auto rd = [&](f32x4* x, int u) NXA_INLINE {
        const int step = u % NS, d0 = (u / NS) * NDH;
#pragma unroll
        for (int k = 0; k < NDH; ++k) x[k] = lo.tr(at, step >> 2, step & 3, d0 + k);
      };
      rd(a[0], 0);
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        if (u + 1 < NU) rd(a[(u + 1) & 1], u + 1);
        const int step = u % NS;
#pragma unroll
        for (int k = 0; k < NDH; ++k) bb[k] = pack4(dp[step >> 2], step & 3);
        mma4n<NDH>(dq + (u / NS) * NDH, a[u & 1], bb);
      }
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 8 * NDH, 0);
#pragma unroll
      for (int u = 0; u + 2 < NU; ++u) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 4 * NDH, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 4 * NDH, 0);
      }
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 8 * NDH, 0);
    }

    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __syncthreads();
  }

  if (qok) {
    float* dqp = (float*)p.dq + b * p.q_str[0] + h * p.q_str[1] + (int64_t)qrow * p.q_str[2];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d0 = db * 32 + 8 * c + 4 * g;
        if (d0 < p.D) store4(dqp + d0, dq[db], 4 * c, p.scale);
      }
  }
}

// Launchers: false when the problem is outside what these kernels take
// (more streamed tiles than a block lists).
bool launch_fwd32(Params p, int dp, hipStream_t stream) {
  const int bn = dp > 128 ? 32 : 64;
  if (dp > 256 || (p.Lk + bn - 1) / bn > kF32MaxTiles) return false;
  p.nqt = (p.Lq + 127) / 128;
  // Fewer 128-query blocks than a quarter of the CUs, at head dim 64 and
  // with at least two key tiles: the key-split kernel, four blocks per
  // 128 queries.
  if (dp == 64 && p.B * p.H * p.nqt < 64 && p.Lk > 64) {
    p.nqt = (p.Lq + 31) / 32;
    const dim3 grid(p.B * p.H * p.nqt);
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, dim3(256), 0, stream, p); };
    if (p.has_bias) {
      if (p.causal) go(fwd32s_kernel<true, true>);
      else go(fwd32s_kernel<true, false>);
    } else {
      if (p.causal) go(fwd32s_kernel<false, true>);
      else go(fwd32s_kernel<false, false>);
    }
    return true;
  }
  const dim3 grid(p.B * p.H * p.nqt);
  auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, dim3(256), 0, stream, p); };
  if (dp == 64) {
    if (p.has_bias) {
      if (p.causal) go(fwd32_kernel<64, true, true>);
      else go(fwd32_kernel<64, true, false>);
    } else {
      if (p.causal) go(fwd32_kernel<64, false, true>);
      else go(fwd32_kernel<64, false, false>);
    }
  } else if (dp == 256) {
    if (p.has_bias) {
      if (p.causal) go(fwd32_kernel<256, true, true>);
      else go(fwd32_kernel<256, true, false>);
    } else {
      if (p.causal) go(fwd32_kernel<256, false, true>);
      else go(fwd32_kernel<256, false, false>);
    }
  } else {
    if (p.has_bias) {
      if (p.causal) go(fwd32_kernel<128, true, true>);
      else go(fwd32_kernel<128, true, false>);
    } else {
      if (p.causal) go(fwd32_kernel<128, false, true>);
      else go(fwd32_kernel<128, false, false>);
    }
  }
  return true;
}

bool launch_dkdv32(Params p, int dp, hipStream_t stream) {
  const int bq = dp > 128 ? 32 : 64;
  if (dp > 256 || (p.Lq + bq - 1) / bq > kF32MaxTiles) return false;
  p.nkt = (p.Lk + 127) / 128;
  const dim3 grid(p.nbh * p.nkt);
  if (dp == 256) {
    // dV, then dK and dbias.
    if (p.causal) {
      hipLaunchKernelGGL((dkdv32_kernel<256, true, kF32Dv>), grid, dim3(256), 0, stream, p);
      hipLaunchKernelGGL((dkdv32_kernel<256, true, kF32Dk>), grid, dim3(256), 0, stream, p);
    } else {
      hipLaunchKernelGGL((dkdv32_kernel<256, false, kF32Dv>), grid, dim3(256), 0, stream, p);
      hipLaunchKernelGGL((dkdv32_kernel<256, false, kF32Dk>), grid, dim3(256), 0, stream, p);
    }
  } else if (dp == 64) {
    if (p.causal) hipLaunchKernelGGL((dkdv32_kernel<64, true>), grid, dim3(256), 0, stream, p);
    else hipLaunchKernelGGL((dkdv32_kernel<64, false>), grid, dim3(256), 0, stream, p);
  } else {
    if (p.causal) hipLaunchKernelGGL((dkdv32_kernel<128, true>), grid, dim3(256), 0, stream, p);
    else hipLaunchKernelGGL((dkdv32_kernel<128, false>), grid, dim3(256), 0, stream, p);
  }
  return true;
}

bool launch_dq32(Params p, int dp, hipStream_t stream) {
  const int bn = dp > 128 ? 32 : 64;
  if (dp > 256 || (p.Lk + bn - 1) / bn > kF32MaxTiles) return false;
  p.nqt = (p.Lq + 127) / 128;
  const dim3 grid(p.B * p.H * p.nqt);
  if (dp == 64) {
    if (p.causal) hipLaunchKernelGGL((dq32_kernel<64, true>), grid, dim3(256), 0, stream, p);
    else hipLaunchKernelGGL((dq32_kernel<64, false>), grid, dim3(256), 0, stream, p);
  } else if (dp == 256) {
    if (p.causal) hipLaunchKernelGGL((dq32_kernel<256, true>), grid, dim3(256), 0, stream, p);
    else hipLaunchKernelGGL((dq32_kernel<256, false>), grid, dim3(256), 0, stream, p);
  } else {
    if (p.causal) hipLaunchKernelGGL((dq32_kernel<128, true>), grid, dim3(256), 0, stream, p);
    else hipLaunchKernelGGL((dq32_kernel<128, false>), grid, dim3(256), 0, stream, p);
  }
  return true;
}

}  // namespace nxa
