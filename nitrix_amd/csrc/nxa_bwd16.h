// 16-bit (bf16 / fp16 I/O) backward kernels for gfx950: dK/dV (+ dbias) and
// dQ, templated on the element type T (the MFMA and conversions follow it).
//
// Same math as the reference's two backward Pallas kernels
// (src/nitrix/_kernels/cuda/attention.py:272-332 dK/dV, :335-387 dQ):
// P = exp2(S * scale * log2e + bias * log2e - lse2), dS = P (dP - delta),
// dV = P^T dO, dK = scale dS^T Q, dQ = scale dS K.  Deterministic (no
// atomics): dK/dV own key tiles and stream query tiles, dQ owns query tiles
// and streams key tiles.
//
// Layout choices for CDNA4:
// * streamed tiles are row-major [64 x DP] 16-bit tiles in LDS whose 16-byte
//   chunks are XOR-swizzled by row, conflict-free both for the 16-byte row
//   reads of the S / dP products and for the ds_read_b64_tr_b16 reads that
//   give the transposed operands (dO^T, Q^T for dV / dK, K^T for dQ), so no
//   transposed copies are written;
// * tiles move from HBM into an LDS ring by direct copies through buffer
//   resources bounded at the last row, spread between the MFMAs;
// * -delta enters the dP accumulators as their initial value; the logits
//   come out of one FMA per element, S * scale * log2(e) - lse * log2(e), on
//   the exact fp32 products (scaling Q or K before the 16-bit rounding would
//   perturb every logit by 2^-9 of its size in bf16).
//
// Kernel and launcher templates; instantiated by nxa_bwd16.hip (head dims
// 64 and 128) and nxa_bwd16_wide.hip (256, compiled with flags of its own).
#pragma once

#include "nxa_common.h"
#include "nxa_launch.h"

#include <type_traits>

namespace nxa {

constexpr int kMaxBwdTiles = 1024;
// dQ's packed tile entries: key-tile index in the low 30 bits (and the
// index past the last active tile), class in the top 2.
constexpr int kTileEnd = 0x3fffffff;

// Active query tiles of one key block (tile class & 1: something kept).
// Wave 0 compacts them, in order, into an LDS list, so the tile loop finds
// the k-th active tile with one LDS read (issued an iteration ahead) instead
// of a scan over the classes; a contiguous run (no mask, key padding,
// causal) needs no read at all.  Above kMaxBwdTiles query tiles no list is
// kept and the loop scans the tile map itself.
struct QTiles {
  int nq, first, cnt, ucls;
  bool listed, dense;
  const uint16_t* act;   // active tiles, in order (listed)
  const uint8_t* acls;   // their classes
  const uint8_t* cls;    // class of every tile (listed)
  // Active tile k, given active tile k - 1 = prev (-1 for k = 0); nq past
  // the last.
  template <typename F>
  __device__ __forceinline__ int tile(int k, int prev, F&& cg) const {
    if (dense) return k < cnt ? first + k : nq;
    if (listed) return k < cnt ? __builtin_amdgcn_readfirstlane((int)act[k]) : nq;
    int t = prev + 1;
    while (t < nq && !(cg(t) & 1)) ++t;
    return t;
  }
  // Class of active tile k (= t): uniform over the block's tiles when ucls >= 0.
  template <typename F>
  __device__ __forceinline__ int klass(int k, int t, F&& cg) const {
    if (ucls >= 0) return ucls;
    return listed ? __builtin_amdgcn_readfirstlane((int)acls[k]) : cg(t);
  }
  template <typename F>
  __device__ __forceinline__ bool active(int t, F&& cg) const {
    return ((listed ? (int)cls[t] : cg(t)) & 1) != 0;
  }
};

// Builds the list (every thread of the block calls it; two block barriers).
// cg(t) is the class of query tile t for this key block.
template <typename F>
__device__ QTiles build_qtiles(uint16_t* act, uint8_t* acls, uint8_t* cls, int* hdr,
                               int nq, int tid, int nthreads, F&& cg) {
  const bool listed = nq <= kMaxBwdTiles;
  if (listed)
    for (int t = tid; t < nq; t += nthreads) cls[t] = (uint8_t)cg(t);
  __syncthreads();
  if (tid < 64) {
    const int lane = tid;
    int first = nq, last = -1, cnt = 0;
    bool all_full = true, all_part = true;
    for (int t0 = 0; t0 < nq; t0 += 64) {
      const int t = t0 + lane;
      const int c = t < nq ? (listed ? (int)cls[t] : cg(t)) : 0;
      const uint64_t m = __ballot(c & 1);
      if (listed && (c & 1)) {
        const int pos = cnt + __popcll(m & ((1ull << lane) - 1));
        act[pos] = (uint16_t)t;
        acls[pos] = (uint8_t)c;
      }
      if (m) {
        first = min(first, t0 + (int)__builtin_ctzll(m));
        last = t0 + 63 - (int)__builtin_clzll(m);
        cnt += __popcll(m);
      }
      all_full = all_full && __ballot((c & 1) && !(c & 2)) == 0;
      all_part = all_part && __ballot((c & 3) == 3) == 0;
    }
    if (lane == 0) {
      hdr[0] = first;
      hdr[1] = cnt;
      hdr[2] = all_full ? 3 : all_part ? 1 : -1;
      hdr[3] = cnt > 0 && last - first + 1 == cnt;
    }
  }
  __syncthreads();
  QTiles r;
  r.nq = nq;
  r.first = __builtin_amdgcn_readfirstlane(hdr[0]);
  r.cnt = __builtin_amdgcn_readfirstlane(hdr[1]);
  r.ucls = __builtin_amdgcn_readfirstlane(hdr[2]);
  r.dense = __builtin_amdgcn_readfirstlane(hdr[3]) != 0;
  r.listed = listed;
  r.act = act;
  r.acls = acls;
  r.cls = cls;
  return r;
}
// Build-time tuning knob (-D on the compiler line): the wave priority
// (s_setprio) of the dK/dV waves' critical chains.
#ifndef DKDV_PRIO
#define DKDV_PRIO 1
#endif
// Transposed fragments the dK/dV products read ahead of their use.
#ifndef TRPD
#define TRPD 4
#endif

// dbias handling compiled into dK/dV.
enum : int { kDbNone = 0, kDbFull = 1, kDbColsum = 2 };

__device__ __forceinline__ void store_db(const Params& p, int64_t off, float x) {
  store_elem(p.dbias_f32 ? kF32 : p.bias_dtype, p.dbias, off, x);
}

__device__ __forceinline__ float load_bias1(const Params& p, int64_t off) {
  return load_elem(p.bias_dtype, p.bias, off);
}

// ---------------------------------------------------------------------------
// dK / dV.  Block = 8 waves over 128 keys.  Waves w and w + 4 own the same
// 32 keys (the key is the lane's column, so P and dS feed the dV / dK
// products from registers) and share SIMD w:
//   * the P wave (w < 4) holds K stationary, forms P = exp2(S c - lse2)
//     (c = scale * log2(e), one FMA per element on the fp32 scores), publishes
//     P (in fp16, register order) through LDS and accumulates dV^T += dO^T P;
//   * the dS wave (w >= 4) holds V stationary and starts at -delta, so its
//     product is dP - delta; dS = P (dP - delta) with P read back from LDS,
//     dK^T += Q^T dS (and dbias).
// S is computed once per tile, and one barrier separates iterations.  In
// iteration i the P wave runs dV of tile i - 1 (its P kept in registers)
// and S of tile i, then the exponentials of tile i (publishing P(i)); the
// dS wave runs dS of tile i - 1 (from the dP - delta it formed in iteration
// i - 1 and the published P(i - 1)), then dK of tile i - 1 and dP - delta
// of tile i.  So each wave's VALU phase meets the other's products: the dS
// pass beside the P wave's dV and S, the exponentials beside dK and dP.
// Query tiles (Q, dO as swizzled [64 x DP] tiles, -lse2, -delta) move from
// HBM into a 3-stage LDS ring by direct copies, which the dS waves issue
// during their dS pass, one tile ahead.
//
// ---------------------------------------------------------------------------
template <typename T, int DP, bool HAS_BIAS, bool CAUSAL, int DBM>
__global__ __launch_bounds__(512, 1) void dkdv16_kernel(const Params p) {
  using M = Mma<T>;
  using Frag = typename M::Frag;
  constexpr int EPC = 8, KC = 16;
  constexpr int BNK = 128, BQ = 64, NW = 8, NST = 3;
  constexpr int NC = DP / KC, NDB = DP / 32, FPB = M::FRAGS_PER_BLOCK;
  using QS = SwzStream<DP, 4>;  // copied by the 4 dS waves
  constexpr int NCPY = 2 * QS::CNT;  // Q and dO copies per dS wave per tile
  constexpr int TILE_BYTES = BQ * DP * 2;
  constexpr int ROWS_OFF = 2 * TILE_BYTES;             // -lse2[64], then -delta[64]
  constexpr int STAGE_BYTES = ROWS_OFF + 2 * BQ * 4;
  constexpr int PB_BYTES = 4 * 2 * 2 * 1024;           // [P wave][query block][frag][lane]
  constexpr int PBUF_BYTES = 2 * PB_BYTES;             // two P buffers (alternating tiles)
  __shared__ __attribute__((aligned(16))) char smem[NST * STAGE_BYTES + PBUF_BYTES];
  __shared__ uint16_t act[kMaxBwdTiles];
  __shared__ uint8_t acls[kMaxBwdTiles], tcls[kMaxBwdTiles];
  __shared__ int sched_s[4];

  const int vid = xcd_remap(blockIdx.x, p.nbh, p.nkt);
  const int bh = p.bh0 + vid / p.nkt;
  const int b = bh / p.H, h = bh % p.H;
  // Longest blocks first by the mask's block order (causal: the first key
  // blocks are the longest and come first in index order).
  const int kt = p.order ? ordered_tile(p, b, h, p.ord_k128, vid % p.nkt, p.nkt)
                         : vid % p.nkt;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform
  const bool pw = wave < 4;                                   // role (uniform)
  const int g = lane >> 5, c32 = lane & 31;
  const int kblk0 = kt * BNK;
  const int kw0 = kblk0 + (wave & 3) * 32;
  const int key = kw0 + c32;
  const bool kok = key < p.Lk;
  const int kc = kok ? key : p.Lk - 1;

  const T* qp = (const T*)p.q + b * p.q_str[0] + h * p.q_str[1];
  const T* dop = (const T*)p.dout + b * p.o_str[0] + h * p.o_str[1];
  const float* nlp = p.nlse2 + ((int64_t)b * p.H + h) * p.Lq;
  const float* ndp = p.ndelta + ((int64_t)b * p.H + h) * p.Lq;
  const int64_t qs = p.q_str[2], os = p.o_str[2];

  // Query-tile classes (0 = nothing kept for this key block).
  const int nq = (p.Lq + BQ - 1) / BQ;
  auto tclass_g = [&](int t) -> int {
    const int q0 = t * BQ;
    if (CAUSAL && q0 + BQ - 1 < kblk0) return 0;
    if (!p.has_tilemap) return 3;
    return tile_class(p, b, h, q0, q0 + BQ, kblk0, kblk0 + BNK);
  };
  const QTiles tl = build_qtiles(act, acls, tcls, sched_s, nq, tid, NW * 64, tclass_g);

  // Stationary B operands for this lane's key: K (P wave) or V (dS wave).
  Frag bfr[NC];
  {
    const T* src = pw ? (const T*)p.k + b * p.k_str[0] + h * p.k_str[1] +
                            (int64_t)kc * p.k_str[2]
                      : (const T*)p.v + b * p.v_str[0] + h * p.v_str[1] +
                            (int64_t)kc * p.v_str[2];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d = c * KC + g * EPC;
      bfr[c] = (kok && d < (pw ? p.D : p.Dv)) ? ld16(src + d) : zero_frag<T>();
    }
  }
  f32x16 acc[NDB];  // dV^T (P wave) or dK^T (dS wave)
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;
  // Column sums of dS (dbias of a query-broadcast bias) on the matrix core:
  // an all-ones A operand times the packed dS of each fragment adds the
  // fragment's 16 queries into every row of csacc.
  f32x16 csacc;
  Frag ones;
  if constexpr (DBM == kDbColsum) {
#pragma unroll
    for (int r = 0; r < 16; ++r) csacc[r] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ones[e] = (T)1.0f;
  }

  // Bias: a per-key constant when it broadcasts over queries, else per row.
  const bool bias_rows = HAS_BIAS && p.bias_str[2] != 0;
  const int64_t bbase =
      HAS_BIAS ? b * p.bias_str[0] + h * p.bias_str[1] + kc : 0;
  const float bkey = (HAS_BIAS && !bias_rows) ? load_bias1(p, bbase) * kLog2e : 0.f;
  const uint8_t* mbase =
      p.has_mask ? p.mask + b * p.mask_str[0] + h * p.mask_str[1] + kc : nullptr;
  const int64_t dbbase = b * p.dbias_str[0] + h * p.dbias_str[1] + key - p.dbias_off;
  // Everything that depends on the key alone folds into one additive term
  // of the P wave's logits: the query-broadcast bias, -inf for a key past
  // Lk, and -inf for a key that a query-broadcast mask (key padding)
  // removes.  Only a mask that varies over queries needs the element pass.
  const bool mask_rows = p.has_mask && p.mask_str[2] != 0;
  const bool kmasked = !kok || (p.has_mask && !mask_rows && mbase[0] == 0);
  const float kadd = kmasked ? -INFINITY : bkey;
  // Without a bias, only waves with a nonzero key term for some lane add it
  // (with key padding, just the block that straddles the valid length).
  const bool use_kadd = HAS_BIAS || __any(kadd != 0.f);  // uniform

  // Full dbias: entries of skipped tiles are zero.
  if constexpr (DBM == kDbFull) {
    if (!pw && kok)
      for (int t = 0; t < nq; ++t)
        if (!tl.active(t, tclass_g))
          for (int i = 0; i < BQ && t * BQ + i < p.Lq; ++i)
            store_db(p, dbbase + (int64_t)(t * BQ + i) * p.dbias_str[2], 0.f);
  }
  // The stationary loads complete here, so no wait inside the tile loop has
  // to cover them (vmcnt there only tracks the tile copies).
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

  // --- copies --------------------------------------------------------------------
  // The dS waves copy the query tiles, spread over their phase-A products
  // (a burst of copies from every wave at the tile barrier would hold all
  // of them in the memory pipeline's issue queue at once).  Copies go
  // through buffer resources bounded at the last row: rows past Lq read as
  // zero (those queries are masked), and a tile index past the last active
  // tile gives an empty range, so every tile issues the same copies.
  const int cw = wave & 3;
  QS qsm, dsm;
  qsm.init(qs, p.D, cw, lane);
  dsm.init(os, p.Dv, cw, lane);
  const uint32_t lds0 = lds_offset(smem);
  const uint32_t pbuf = lds0 + NST * STAGE_BYTES;
  struct TileSrc {
    i32x4 q, d, r;  // Q rows, dO rows, per-row values (-lse2 or -delta)
  };
  auto tile_src = [&](int t) NXA_INLINE -> TileSrc {
    const int q0 = t < nq ? t * BQ : p.Lq;
    // Rows of this tile that exist (0: empty ranges).  Each range covers
    // only the tile's own rows, so its byte size stays below 64 row strides,
    // which the host bounds below 2^32 bytes.
    const int rows = min(p.Lq - q0, BQ);
    TileSrc s;
    s.q = make_rsrc(qp + (int64_t)q0 * qs,
                    rows > 0 ? (uint32_t)(((int64_t)(rows - 1) * qs + p.D) * 2) : 0u);
    s.d = make_rsrc(dop + (int64_t)q0 * os,
                    rows > 0 ? (uint32_t)(((int64_t)(rows - 1) * os + p.Dv) * 2) : 0u);
    s.r = make_rsrc((cw == 0 ? nlp : ndp) + q0, (uint32_t)max(rows, 0) * 4u);
    return s;
  };
  // Copy j of a tile into stage st: j < NCPY the wave's share of Q, then of
  // dO; j == NCPY the 64 per-row values of -lse2 (wave 4) or -delta (wave 5).
  auto copy = [&](const TileSrc& s, int st, int j) NXA_INLINE {
    const uint32_t at = lds0 + st * STAGE_BYTES;
    if (j < QS::CNT)
      dma16_buf(s.q, qsm.off[j], at + (j * 4 + cw) * 1024);
    else if (j < NCPY)
      dma16_buf(s.d, dsm.off[j - QS::CNT], at + TILE_BYTES + ((j - QS::CNT) * 4 + cw) * 1024);
    else if (cw < 2)
      dma4_buf(s.r, 4u * lane, at + ROWS_OFF + cw * (BQ * 4));
  };
  // --- per-lane LDS read offsets (bytes) --------------------------------------------
  // Row reads (A of S and dP): row c32 of a 32-row block, chunk 2m + g.  The
  // swizzle depends on the row's low 4 bits only, so other blocks and
  // fragments are compile-time row offsets.
  uint32_t roff[NC];
#pragma unroll
  for (int m = 0; m < NC; ++m) roff[m] = 2 * swz_off<DP>(c32, 2 * m + g);
  // Transposed reads (A of dV^T = dO^T P and dK^T = Q^T dS).
  const int tr_row = 4 * ((lane >> 4) >> 1) + ((lane & 15) >> 2);
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  uint32_t toff[NDB][2];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int col = db * 32 + tr_col;
      toff[db][hh] = 2 * (swz_off<DP>(tr_row + 8 * hh, col >> 3) + (col & 7));
    }
  // Per-row values: rows 8c + 4g .. +3 of each 32-row block.
  const uint32_t rvoff = ROWS_OFF + (pw ? 0 : BQ * 4) + 16 * g;
  // P exchange: the lane's two fp16 fragments per query block, 1 KB apart.
  const uint32_t poff = pbuf + (wave & 3) * (2 * 2 * 1024) + 16 * lane;

  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  typedef __attribute__((address_space(3))) Frag lds_frag;
  typedef __attribute__((address_space(3))) f16x8 lds_pfrag;
  typedef __attribute__((address_space(3))) f32x4 lds_f32x4;
  typedef short i16x8 __attribute__((ext_vector_type(8)));
  auto tr_frag = [&](uint32_t a0, uint32_t a1) NXA_INLINE -> Frag {
    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(uintptr_t)a0);
    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(uintptr_t)a1);
    const i16x8 r = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(Frag, r);
  };
  auto vadd = [](uint32_t sb, uint32_t v) NXA_INLINE -> uint32_t {
    uint32_t r;
    asm("v_add_u32 %0, %1, %2" : "=v"(r) : "s"(sb), "v"(v));
    return r;
  };

  // Row products of one tile, two 32-query blocks: A B^T with A = Q (P
  // wave) or dO (dS wave) of the tile in stage `at`.  The dS wave's
  // accumulators start at the per-row values (x = dP - delta); the P wave's
  // start at zero and its per-row values (-lse2) land in `rows`.
  // `between(j)` runs after product j (the dS wave's tile copies).
  auto row_products = [&](uint32_t at, f32x16 (&x)[2], f32x16 (&rows)[2],
                          auto&& between) NXA_INLINE {
    const uint32_t rt = at + (pw ? 0 : TILE_BYTES);
    uint32_t ra[NC];
#pragma unroll
    for (int m = 0; m < NC; ++m) ra[m] = vadd(rt, roff[m]);
    const uint32_t rv = vadd(at, rvoff);
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const f32x4 v4 = *(const lds_f32x4*)(uintptr_t)(rv + (qb * 32 + 8 * c) * 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (pw) {
            rows[qb][4 * c + j] = v4[j];
            x[qb][4 * c + j] = 0.f;
          } else {
            x[qb][4 * c + j] = v4[j];
          }
        }
      }
    // Product j: query block j & 1, head-dim chunk pair j >> 1.  The A
    // fragments are read PD products ahead (a rotating register buffer) so
    // the LDS latency is covered.
    constexpr int NPA = 2 * NC, PD = NPA < 8 ? NPA : 8;
    auto afrag = [&](int j) NXA_INLINE -> Frag {
      return *(const lds_frag*)(uintptr_t)(ra[j >> 1] + (j & 1) * (32 * DP * 2));
    };
    Frag abuf[PD];
#pragma unroll
    for (int j = 0; j < PD; ++j) abuf[j] = afrag(j);
#pragma unroll
    for (int j = 0; j < NPA; ++j) {
      M::run(x[j & 1], abuf[j % PD], bfr[j >> 1]);
      if (j + PD < NPA) abuf[j % PD] = afrag(j + PD);
      between(j);
    }
    // Keep that order: the row values, PD reads, then one product and one
    // read at a time.
    __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 8 + PD, 0);
#pragma unroll
    for (int j = 0; j < NPA; ++j) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      if (j + PD < NPA) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
    }
  };
  // Transposed products: acc += A^T F[qb] for both query blocks, A = dO (P
  // wave) or Q (dS wave) of the tile in stage `at`.
  auto tr_products = [&](uint32_t at, const Frag (&pf)[2][FPB]) NXA_INLINE {
    const uint32_t tt = at + (pw ? TILE_BYTES : 0);
    uint32_t ta[NDB][2];
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      ta[db][0] = vadd(tt, toff[db][0]);
      ta[db][1] = vadd(tt, toff[db][1]);
    }
    // Product j: query fragment qf = j / NDB (block qf / FPB, fragment
    // qf % FPB), head-dim block db = j % NDB.  The A fragments (two
    // transposed reads each) are read TRPD products ahead of their use, so
    // the reads of later products are in flight while one runs.
    constexpr int NTR = 2 * FPB * NDB, PT = NTR < TRPD ? NTR : TRPD;
    auto afrag = [&](int j) NXA_INLINE -> Frag {
      const int qf = j / NDB, db = j % NDB;
      const uint32_t ro = (32 * (qf / FPB) + 16 * (qf % FPB)) * (DP * 2);
      return tr_frag(ta[db][0] + ro, ta[db][1] + ro);
    };
    Frag tbuf[PT];
#pragma unroll
    for (int j = 0; j < PT; ++j) tbuf[j] = afrag(j);
#pragma unroll
    for (int j = 0; j < NTR; ++j) {
      const int qf = j / NDB;
      M::run(acc[j % NDB], tbuf[j % PT], pf[qf / FPB][qf % FPB]);
      if (j + PT < NTR) tbuf[j % PT] = afrag(j + PT);
      if constexpr (DBM == kDbColsum)
        if (!pw && j % NDB == NDB - 1) M::run(csacc, ones, pf[qf / FPB][qf % FPB]);
    }
    if constexpr (DBM != kDbColsum) {
      // Keep that order: PT fragment reads, then one product and one read
      // at a time.
#pragma unroll
      for (int j = 0; j < PT; ++j) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
#pragma unroll
      for (int j = 0; j < NTR; ++j) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
        if (j + PT < NTR) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
      }
    }
  };

  // P wave, tile t in stage st: P = exp2(S'), published (in fp16) in P buffer
  // `par`, then dV^T += dO^T P.
  auto p_tile = [&](int t, int cls, int st, int par, Frag (&pf)[2][FPB]) NXA_INLINE {
    const uint32_t at = lds0 + st * STAGE_BYTES;
    const int q0 = t * BQ;
    __builtin_amdgcn_s_setprio(DKDV_PRIO);  // the exp pass depends on these
    f32x16 x[2], rows[2];
    row_products(at, x, rows, [](int) {});
    __builtin_amdgcn_s_setprio(0);
    const bool need_mask = mask_rows && !(cls & 2);
    const bool tail = q0 + BQ > p.Lq;
    const bool diag = CAUSAL && (kw0 + 31 > q0);
    const bool general = need_mask || tail || diag || bias_rows;
    // Logits of query block qb in place; GEN selects the element-wise pass
    // (per-row mask, query tail, causal diagonal, per-row bias) and ADD the
    // per-key term, so interior tiles run straight-line.
    auto p_logits = [&](int qb, auto gen_tag, auto add_tag) NXA_INLINE {
      constexpr bool GEN = decltype(gen_tag)::value;
      constexpr bool ADD = decltype(add_tag)::value;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float xv = __builtin_fmaf(x[qb][r], p.scale_log2, rows[qb][r]);
        if constexpr (ADD) xv += kadd;
        if constexpr (GEN) {
          const int q = q0 + qb * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
          const int qcl = q < p.Lq ? q : p.Lq - 1;
          if constexpr (HAS_BIAS)
            if (bias_rows)
              xv = __builtin_fmaf(load_bias1(p, bbase + (int64_t)qcl * p.bias_str[2]),
                                  kLog2e, xv);
          bool keep = q < p.Lq;
          if (need_mask) keep = keep && mbase[(int64_t)qcl * p.mask_str[2]] != 0;
          if (CAUSAL) keep = keep && key <= q;
          xv = keep ? xv : -INFINITY;
        }
        x[qb][r] = xv;
      }
    };
    auto exp_pack = [&](int qb) NXA_INLINE {
#pragma unroll
      for (int r = 0; r < 16; ++r) x[qb][r] = fast_exp2(x[qb][r]);
#pragma unroll
      for (int f = 0; f < FPB; ++f) {
        pf[qb][f] = M::pack(x[qb], f);
        // The exchange carries P in fp16 whatever T is: P <= 1 here, fp16
        // holds it with more mantissa than bf16, and the dS wave multiplies
        // it in one mixed-precision FMA.
        *(lds_pfrag*)(uintptr_t)(poff + par * PB_BYTES + (qb * FPB + f) * 1024) =
            std::is_same<T, f16>::value ? __builtin_bit_cast(f16x8, pf[qb][f])
                                        : Mma<f16>::pack(x[qb], f);
      }
    };
    auto p_blocks = [&](auto gen_tag, auto add_tag) NXA_INLINE {
      if constexpr (DP <= 64) {
        // All 32 logits before their exponentials: left to itself the
        // compiler chains FMA -> exp element by element through one
        // temporary, and at D = 64 that chain's latency, not the issue
        // rate, sets the pace of the phase (at D = 128 the registers it
        // would take cost more than the chain).
        p_logits(0, gen_tag, add_tag);
        p_logits(1, gen_tag, add_tag);
        __builtin_amdgcn_sched_barrier(0);
        exp_pack(0);
        exp_pack(1);
      } else {
        p_logits(0, gen_tag, add_tag);
        exp_pack(0);
        p_logits(1, gen_tag, add_tag);
        exp_pack(1);
      }
    };
    if (general)
      p_blocks(std::true_type{}, std::true_type{});
    else if (use_kadd)
      p_blocks(std::false_type{}, std::true_type{});
    else
      p_blocks(std::false_type{}, std::false_type{});
  };

  // dS wave, first half of an iteration: dS and dK^T += Q^T dS (and dbias)
  // of tile t (stage st, P from buffer `par`) from x = dP - delta, which the
  // previous iteration formed; the copies of the next tile (sources s,
  // stage stn) ride along with the dS pass.
  auto ds_lag = [&](int t, int st, int par, f32x16 (&x)[2], const TileSrc& s,
                    int stn) NXA_INLINE {
    const uint32_t at = lds0 + st * STAGE_BYTES;
    const int q0 = t * BQ;
    Frag pf[2][FPB];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
#pragma unroll
      for (int f = 0; f < FPB; ++f) {
        const f16x8 pb = *(const lds_pfrag*)(uintptr_t)(poff + par * PB_BYTES + (qb * FPB + f) * 1024);
        constexpr int CPS = NCPY / (2 * FPB);  // copies per fragment step
        const int step = qb * FPB + f;
#pragma unroll
        for (int j = 0; j < CPS; ++j) copy(s, stn, step * CPS + j);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int r = 8 * f + e;
          // fp16 P times fp32: an FMA with a zero addend on the converted
          // half, which the compiler emits as one mixed-precision
          // v_fma_mix_f32 (exact conversion, one rounding).
          const float ds = __builtin_fmaf((float)pb[e], x[qb][r], 0.0f);
          x[qb][r] = ds;
          if constexpr (DBM == kDbFull) {
            const int q = q0 + qb * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
            if (kok && q < p.Lq) store_db(p, dbbase + (int64_t)q * p.dbias_str[2], ds);
          }
        }
        pf[qb][f] = M::pack(x[qb], f);
      }
    }
    __builtin_amdgcn_s_setprio(DKDV_PRIO);
    tr_products(at, pf);
  };
  // dS wave, second half: x = dP - delta of tile t (stage st), for the next
  // iteration.
  auto dp_lag = [&](int st, f32x16 (&x)[2]) NXA_INLINE {
    f32x16 rows[2];
    row_products(lds0 + st * STAGE_BYTES, x, rows, [](int) {});
    __builtin_amdgcn_s_setprio(0);
  };

  // The tile loop is instantiated per role with the same barrier sequence.
  // Iteration i (active tiles): the P wave forms dV of tile i - 1 and S, P of
  // tile i; the dS wave dS, dK of tile i - 1 (whose P the barrier between
  // them published) and dP of tile i; the dS waves copy tile i + 1 into the
  // stage that tile i - 2 left (no wave reads it in iteration i).  Tile
  // i + 2 is looked up one iteration ahead of its use.
  // qk-norm: in the last iteration the P waves have no new tile; they stage the
  // raw rows of their keys (and the rows' rsqrt) into the stage that no one
  // reads then, for the dS waves' norm VJP after the loop, so that no global
  // load waits at the end of the block.  Rows at [wave % 4][key][DP], the
  // rsqrt after them.
  constexpr int KROWS_BYTES = 4 * 32 * DP * 2;
  static_assert(KROWS_BYTES + 4 * 32 * 4 <= STAGE_BYTES, "staged rows fit one stage");
  auto stage_krows = [&](int st) NXA_INLINE {
    // Direct copies (no registers): 1 KB blocks of RPB whole rows; rows past
    // Lk are outside the range and land as zeros (never read).
    constexpr int SPR = DP * 2 / 16, RPB = 64 / SPR;
    const int rows = min(32, p.Lk - kw0);
    const uint32_t reg = lds0 + st * STAGE_BYTES + (wave & 3) * 32 * DP * 2;
    const i32x4 rs = make_rsrc((const T*)p.kraw + b * p.k_str[0] + h * p.k_str[1] +
                                   (int64_t)kw0 * p.k_str[2],
                               (uint32_t)(max(rows, 0) * p.k_str[2] * 2));
#pragma unroll
    for (int m = 0; m < 32 / RPB; ++m) {
      const int row = m * RPB + lane / SPR;
      dma16_buf(rs, 2u * (uint32_t)(row * p.k_str[2] + (lane % SPR) * 8), reg + m * 1024);
    }
    // The rsqrt of the wave's 32 keys: 4 bytes per lane from lanes 0-31 only
    // (each wave's 128 bytes sit next to the others').
    if (lane < 32)
      dma4_buf(make_rsrc(p.krstd + ((int64_t)b * p.H + h) * p.Lk + kw0,
                         (uint32_t)(max(rows, 0) * 4)),
               4u * lane, lds0 + st * STAGE_BYTES + KROWS_BYTES + (wave & 3) * 128);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  };
  // Returns the stage of the last iteration (-1 when the block had no tile).
  auto run = [&](auto role_tag) -> int {
    constexpr bool PW = decltype(role_tag)::value;
    int last = -1;
    int cur = tl.tile(0, -1, tclass_g), prv = nq;
    int nxt = cur < nq ? tl.tile(1, cur, tclass_g) : nq;
    int k = 0;
    int stc = 0, stp = 2, par = 0;
    f32x16 xs[2];      // dS wave: dP - delta of the tile it forms dS of next
    Frag pfs[2][FPB];  // P wave: P of the tile whose dV the next iteration forms
    if constexpr (!PW) {
      const TileSrc s0 = tile_src(cur);
#pragma unroll
      for (int j = 0; j <= NCPY; ++j) copy(s0, 0, j);
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    }
    barrier_nofence();
    while (cur < nq || prv < nq) {
      const int nn = nxt < nq ? tl.tile(k + 2, nxt, tclass_g) : nq;
      const int stn = stc == 2 ? 0 : stc + 1;
      if constexpr (PW) {
        // Lagged dV: the products of the previous tile open the iteration,
        // so that the exponentials of this one end it (against the dS
        // wave's products).
        if (prv < nq) tr_products(lds0 + stp * STAGE_BYTES, pfs);
        if (cur < nq) p_tile(cur, tl.klass(k, cur, tclass_g), stc, par, pfs);
        else if (p.qk_norm) stage_krows(stc);
        // P (or the staged rows) is in LDS before the barrier.
        __builtin_amdgcn_s_waitcnt(lgkmcnt_imm(0));
      } else {
        const TileSrc s = tile_src(nxt);
        copy(s, stn, NCPY);
        if (prv < nq) {
          ds_lag(prv, stp, par ^ 1, xs, s, stn);
        } else {
#pragma unroll
          for (int j = 0; j < NCPY; ++j) copy(s, stn, j);
        }
        if (cur < nq) dp_lag(stc, xs);
        // Tile nxt is resident before the barrier.
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
      }
      barrier_nofence();
      last = stc;
      prv = cur;
      stp = stc;
      cur = nxt;
      nxt = nn;
      ++k;
      stc = stn;
      par ^= 1;
    }
    return last;
  };
  const int last = pw ? run(std::true_type{}) : run(std::false_type{});
  // No copy may still be writing LDS when the block ends.
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

  if (!pw && p.qk_norm) {
    // dK of the raw (pre-norm) keys: the norm's VJP on the finished rows,
    // whose raw values the P waves staged in the last iteration.
    float gy[NDB][16];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) gy[db][e] = acc[db][e] * p.scale;
    // A block without an active tile has dK-hat = 0, whose VJP is 0.
    if (last >= 0) {
      const T* xl = (const T*)(smem + last * STAGE_BYTES + ((wave & 3) * 32 + c32) * DP * 2);
      const float r = *reinterpret_cast<const float*>(smem + last * STAGE_BYTES + KROWS_BYTES +
                                                      ((wave & 3) * 32 + c32) * 4);
      rms_norm_vjp_rows<T, NDB>(gy, xl, r, p.D, g);
    }
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[db][e] = gy[db][e];
  }
  if (kok) {
    if (!pw) {
      T* dkp = (T*)p.dk + b * p.k_str[0] + h * p.k_str[1] + (int64_t)key * p.k_str[2];
      const float sc = p.qk_norm ? 1.0f : p.scale;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int d0 = db * 32 + 8 * c + 4 * g;
          if (d0 < p.D) store4(dkp + d0, acc[db], 4 * c, sc);
        }
    } else {
      T* dvp = (T*)p.dv + b * p.v_str[0] + h * p.v_str[1] + (int64_t)key * p.v_str[2];
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int d0 = db * 32 + 8 * c + 4 * g;
          if (d0 < p.Dv) store4(dvp + d0, acc[db], 4 * c, 1.0f);
        }
    }
  }
  if constexpr (DBM == kDbColsum) {
    const float tot = csacc[0];  // every row holds the column sum
    if (!pw && kok && g == 0) store_db(p, dbbase, tot);
  }
}

// ---------------------------------------------------------------------------
// dK / dV at head dim 256.  Block = 4 waves x 32 keys (128), one block per
// CU, one wave per SIMD.  A wave holds its keys' K and V stationary (128
// registers) and accumulates dK^T and dV^T (256 registers), so it runs every
// product of its keys itself: S = Q K^T and dP - delta = dO V^T - delta (row
// products on the Q / dO tile, the key on the lane's column),
// P = exp2(S c - lse2) and dS = P (dP - delta) in fp32, then
// dV^T += dO^T P and dK^T += Q^T dS (transposed products, ds_read_b64_tr_b16
// reads of the same tiles).  The products are ordered so that the matrix
// core runs dP while the VALU forms P, and dV while it forms dS.  Query
// tiles of 32 rows (Q, dO, -lse2, -delta) stream through a 3-stage LDS ring
// by direct copies two tiles ahead, every wave copying a quarter of each
// tile between its row products.
// ---------------------------------------------------------------------------
template <typename T, bool HAS_BIAS, bool CAUSAL, int DBM>
__global__ __launch_bounds__(256, 1) void dkdv256_kernel(const Params p) {
  using M = Mma<T>;
  using Frag = typename M::Frag;
  constexpr int DP = 256, EPC = 8, KC = 16;
  constexpr int BNK = 128, BQ = 32, NW = 4, NST = 3;
  constexpr int NC = DP / KC, NDB = DP / 32, FPB = M::FRAGS_PER_BLOCK;
  using QS = SwzStream<DP, NW, BQ>;
  constexpr int NCPY = 2 * QS::CNT;                 // Q and dO copies per wave per tile
  constexpr int TILE_BYTES = BQ * DP * 2;           // 16 KB
  constexpr int ROWS_OFF = 2 * TILE_BYTES;          // -lse2[64], then -delta[64]
  constexpr int STAGE_BYTES = ROWS_OFF + 2 * 64 * 4;
  __shared__ __attribute__((aligned(16))) char smem[NST * STAGE_BYTES];
  __shared__ uint16_t act[kMaxBwdTiles];
  __shared__ uint8_t acls[kMaxBwdTiles], tcls[kMaxBwdTiles];
  __shared__ int sched_s[4];

  const int vid = xcd_remap(blockIdx.x, p.nbh, p.nkt);
  const int bh = p.bh0 + vid / p.nkt;
  const int b = bh / p.H, h = bh % p.H;
  // Longest blocks first by the mask's block order (causal: the first key
  // blocks are the longest and come first in index order).
  const int kt = p.order ? ordered_tile(p, b, h, p.ord_k128, vid % p.nkt, p.nkt)
                         : vid % p.nkt;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform
  const int g = lane >> 5, c32 = lane & 31;
  const int kblk0 = kt * BNK;
  const int kw0 = kblk0 + wave * 32;
  const int key = kw0 + c32;
  const bool kok = key < p.Lk;
  const int kc = kok ? key : p.Lk - 1;

  const T* qp = (const T*)p.q + b * p.q_str[0] + h * p.q_str[1];
  const T* dop = (const T*)p.dout + b * p.o_str[0] + h * p.o_str[1];
  const float* nlp = p.nlse2 + ((int64_t)b * p.H + h) * p.Lq;
  const float* ndp = p.ndelta + ((int64_t)b * p.H + h) * p.Lq;
  const int64_t qs = p.q_str[2], os = p.o_str[2];

  // Query-tile classes (0 = nothing kept for this key block), as in dkdv16.
  const int nq = (p.Lq + BQ - 1) / BQ;
  auto tclass_g = [&](int t) -> int {
    const int q0 = t * BQ;
    if (CAUSAL && q0 + BQ - 1 < kblk0) return 0;
    if (!p.has_tilemap) return 3;
    return tile_class(p, b, h, q0, q0 + BQ, kblk0, kblk0 + BNK);
  };
  const QTiles tl = build_qtiles(act, acls, tcls, sched_s, nq, tid, NW * 64, tclass_g);

  // Stationary B operands of this lane's key: K (for S) and V (for dP).
  Frag kf[NC], vf[NC];
  {
    const T* ks = (const T*)p.k + b * p.k_str[0] + h * p.k_str[1] + (int64_t)kc * p.k_str[2];
    const T* vs = (const T*)p.v + b * p.v_str[0] + h * p.v_str[1] + (int64_t)kc * p.v_str[2];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d = c * KC + g * EPC;
      kf[c] = (kok && d < p.D) ? ld16(ks + d) : zero_frag<T>();
      vf[c] = (kok && d < p.Dv) ? ld16(vs + d) : zero_frag<T>();
    }
  }
  f32x16 dk[NDB], dv[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) dk[db][r] = dv[db][r] = 0.f;
  float colsum = 0.f;

  const bool bias_rows = HAS_BIAS && p.bias_str[2] != 0;
  const int64_t bbase = HAS_BIAS ? b * p.bias_str[0] + h * p.bias_str[1] + kc : 0;
  const float bkey = (HAS_BIAS && !bias_rows) ? load_bias1(p, bbase) * kLog2e : 0.f;
  const uint8_t* mbase =
      p.has_mask ? p.mask + b * p.mask_str[0] + h * p.mask_str[1] + kc : nullptr;
  const int64_t dbbase = b * p.dbias_str[0] + h * p.dbias_str[1] + key - p.dbias_off;
  // Key-only terms of the logits (query-broadcast bias, key past Lk, key
  // padding) fold into one additive term; per-row masks and biases take the
  // element pass.
  const bool mask_rows = p.has_mask && p.mask_str[2] != 0;
  const bool kmasked = !kok || (p.has_mask && !mask_rows && mbase[0] == 0);
  const float kadd = kmasked ? -INFINITY : bkey;
  // Without a bias, only waves with a nonzero key term for some lane add it
  // (with key padding, just the block that straddles the valid length).
  const bool use_kadd = HAS_BIAS || __any(kadd != 0.f);  // uniform

  if constexpr (DBM == kDbFull) {
    if (kok)
      for (int t = 0; t < nq; ++t)
        if (!tl.active(t, tclass_g))
          for (int i = 0; i < BQ && t * BQ + i < p.Lq; ++i)
            store_db(p, dbbase + (int64_t)(t * BQ + i) * p.dbias_str[2], 0.f);
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

  // --- copies --------------------------------------------------------------------
  QS qsm, dsm;
  qsm.init(qs, p.D, wave, lane);
  dsm.init(os, p.Dv, wave, lane);
  const uint32_t lds0 = lds_offset(smem);
  struct TileSrc {
    i32x4 q, d, r;
  };
  auto tile_src = [&](int t) NXA_INLINE -> TileSrc {
    const int q0 = t < nq ? t * BQ : p.Lq;
    const int rows = min(p.Lq - q0, BQ);  // 0: empty ranges
    TileSrc s;
    s.q = make_rsrc(qp + (int64_t)q0 * qs,
                    rows > 0 ? (uint32_t)(((int64_t)(rows - 1) * qs + p.D) * 2) : 0u);
    s.d = make_rsrc(dop + (int64_t)q0 * os,
                    rows > 0 ? (uint32_t)(((int64_t)(rows - 1) * os + p.Dv) * 2) : 0u);
    s.r = make_rsrc((wave == 0 ? nlp : ndp) + q0, (uint32_t)max(rows, 0) * 4u);
    return s;
  };
  // Copy j of a tile into stage st: j < NCPY the wave's share of Q, then of
  // dO; j == NCPY the per-row values (-lse2 by wave 0, -delta by wave 1).
  auto copy = [&](const TileSrc& s, int st, int j) NXA_INLINE {
    const uint32_t at = lds0 + st * STAGE_BYTES;
    if (j < QS::CNT)
      dma16_buf(s.q, qsm.off[j], at + (j * NW + wave) * 1024);
    else if (j < NCPY)
      dma16_buf(s.d, dsm.off[j - QS::CNT], at + TILE_BYTES + ((j - QS::CNT) * NW + wave) * 1024);
    else if (wave < 2)
      dma4_buf(s.r, 4u * lane, at + ROWS_OFF + wave * 256);
  };

  // --- per-lane LDS read offsets (bytes) --------------------------------------------
  // Row reads: row c32, chunk 2m + g.  The swizzle touches the low 4 chunk
  // bits only, so chunk pairs m and m + 8 are 256 bytes apart.
  uint32_t roff[NC / 2];
#pragma unroll
  for (int m = 0; m < NC / 2; ++m) roff[m] = 2 * swz_off<DP>(c32, 2 * m + g);
  // Transposed reads; 32-column blocks db and db + 4 are 256 bytes apart.
  const int tr_row = 4 * ((lane >> 4) >> 1) + ((lane & 15) >> 2);
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  uint32_t toff[NDB / 2][2];
#pragma unroll
  for (int db = 0; db < NDB / 2; ++db)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int col = db * 32 + tr_col;
      toff[db][hh] = 2 * (swz_off<DP>(tr_row + 8 * hh, col >> 3) + (col & 7));
    }

  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  typedef __attribute__((address_space(3))) Frag lds_frag;
  typedef __attribute__((address_space(3))) f32x4 lds_f32x4;
  typedef short i16x8 __attribute__((ext_vector_type(8)));
  auto tr_frag = [&](uint32_t a0, uint32_t a1) NXA_INLINE -> Frag {
    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(uintptr_t)a0);
    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(uintptr_t)a1);
    const i16x8 r = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(Frag, r);
  };
  auto vadd = [](uint32_t sb, uint32_t v) NXA_INLINE -> uint32_t {
    uint32_t r;
    asm("v_add_u32 %0, %1, %2" : "=v"(r) : "s"(sb), "v"(v));
    return r;
  };

  // --- one query tile ------------------------------------------------------------------
  // Tile t in stage st; the copies of a later tile (sources s, stage stn)
  // ride along with the row products.
  auto tile = [&](int t, int cls, int st, const TileSrc& s, int stn) NXA_INLINE {
    const uint32_t at = lds0 + st * STAGE_BYTES;
    const int q0 = t * BQ;
    copy(s, stn, NCPY);
    // Per-row values of rows 8c + 4g .. +3: -delta seeds dP, -lse2 the logits.
    f32x16 xs, xp, rl;
    {
      const uint32_t rv = vadd(at, ROWS_OFF + 16 * g);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const f32x4 l4 = *(const lds_f32x4*)(uintptr_t)(rv + 32 * c);
        const f32x4 d4 = *(const lds_f32x4*)(uintptr_t)(rv + 256 + 32 * c);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          rl[4 * c + j] = l4[j];
          xp[4 * c + j] = d4[j];
        }
      }
    }
    // Row products: j < NC is S (Q tile, K), j >= NC is dP (dO tile, V);
    // chunk pair m = j % NC.  A fragments are read PD products ahead.
    uint32_t ra[NC / 2], rd[NC / 2];
#pragma unroll
    for (int m = 0; m < NC / 2; ++m) {
      ra[m] = vadd(at, roff[m]);
      rd[m] = vadd(at + TILE_BYTES, roff[m]);
    }
    constexpr int NPA = 2 * NC, PD = 6;
    auto afrag = [&](int j) NXA_INLINE -> Frag {
      const int m = j % NC;
      const uint32_t a = j < NC ? ra[m % (NC / 2)] : rd[m % (NC / 2)];
      return *(const lds_frag*)(uintptr_t)(a + (m / (NC / 2)) * 256);
    };
    Frag abuf[PD];
#pragma unroll
    for (int j = 0; j < PD; ++j) abuf[j] = afrag(j);
#pragma unroll
    for (int j = 0; j < NPA; ++j) {
      if (j == 0)
        xs = M::first(abuf[0], kf[0]);
      else if (j < NC)
        M::run(xs, abuf[j % PD], kf[j]);
      else
        M::run(xp, abuf[j % PD], vf[j - NC]);
      if (j + PD < NPA) abuf[j % PD] = afrag(j + PD);
      static_assert(NPA == 4 * NCPY, "one tile copy per four row products");
      if ((j & 3) == 3) copy(s, stn, j >> 2);
    }

    // P = exp2(S c - lse2 [+ key term]) in fp32, packed to T for dV.
    const bool need_mask = mask_rows && !(cls & 2);
    const bool tail = q0 + BQ > p.Lq;
    const bool diag = CAUSAL && (kw0 + 31 > q0);
    const bool general = need_mask || tail || diag || bias_rows;
    auto p_pass = [&](auto gen_tag, auto add_tag) NXA_INLINE {
      constexpr bool GEN = decltype(gen_tag)::value;
      constexpr bool ADD = decltype(add_tag)::value;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float xv = __builtin_fmaf(xs[r], p.scale_log2, rl[r]);
        if constexpr (ADD) xv += kadd;
        if constexpr (GEN) {
          const int q = q0 + 8 * (r >> 2) + 4 * g + (r & 3);
          const int qcl = q < p.Lq ? q : p.Lq - 1;
          if constexpr (HAS_BIAS)
            if (bias_rows)
              xv = __builtin_fmaf(load_bias1(p, bbase + (int64_t)qcl * p.bias_str[2]),
                                  kLog2e, xv);
          bool keep = q < p.Lq;
          if (need_mask) keep = keep && mbase[(int64_t)qcl * p.mask_str[2]] != 0;
          if (CAUSAL) keep = keep && key <= q;
          xv = keep ? xv : -INFINITY;
        }
        xs[r] = fast_exp2(xv);
      }
    };
    if (general)
      p_pass(std::true_type{}, std::true_type{});
    else if (use_kadd)
      p_pass(std::false_type{}, std::true_type{});
    else
      p_pass(std::false_type{}, std::false_type{});
    Frag pf[FPB];
#pragma unroll
    for (int f = 0; f < FPB; ++f) pf[f] = M::pack(xs, f);

    // dV^T += dO^T P while the VALU forms dS = P (dP - delta).
    const uint32_t tq = at, td = at + TILE_BYTES;
    uint32_t ta[NDB / 2][2];
#pragma unroll
    for (int db = 0; db < NDB / 2; ++db) {
      ta[db][0] = vadd(td, toff[db][0]);
      ta[db][1] = vadd(td, toff[db][1]);
    }
#pragma unroll
    for (int f = 0; f < FPB; ++f)
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const uint32_t o = (16 * f) * (DP * 2) + (db / (NDB / 2)) * 256;
        M::run(dv[db], tr_frag(ta[db % (NDB / 2)][0] + o, ta[db % (NDB / 2)][1] + o), pf[f]);
      }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float ds = xs[r] * xp[r];
      xp[r] = ds;
      if constexpr (DBM == kDbFull) {
        const int q = q0 + 8 * (r >> 2) + 4 * g + (r & 3);
        if (kok && q < p.Lq) store_db(p, dbbase + (int64_t)q * p.dbias_str[2], ds);
      }
      if constexpr (DBM == kDbColsum) colsum += ds;
    }
#pragma unroll
    for (int f = 0; f < FPB; ++f) pf[f] = M::pack(xp, f);
    // dK^T += Q^T dS.
#pragma unroll
    for (int db = 0; db < NDB / 2; ++db) {
      ta[db][0] = vadd(tq, toff[db][0]);
      ta[db][1] = vadd(tq, toff[db][1]);
    }
#pragma unroll
    for (int f = 0; f < FPB; ++f)
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const uint32_t o = (16 * f) * (DP * 2) + (db / (NDB / 2)) * 256;
        M::run(dk[db], tr_frag(ta[db % (NDB / 2)][0] + o, ta[db % (NDB / 2)][1] + o), pf[f]);
      }
  };

  // --- tile loop -----------------------------------------------------------------
  // Iteration i handles active tile cur (stage stc) and copies the active
  // tile after next into the stage that the previous tile left; before the
  // barrier that ends it, each wave waits for its own copies of the next
  // tile.  Every wave issues the same copies per tile (empty ranges past the
  // last active tile), so the waits are compile-time.
  int cur = tl.tile(0, -1, tclass_g);
  int nxt = cur < nq ? tl.tile(1, cur, tclass_g) : nq;
  int k = 0;
  {
    const TileSrc s0 = tile_src(cur), s1 = tile_src(nxt);
#pragma unroll
    for (int j = 0; j <= NCPY; ++j) copy(s0, 0, j);
#pragma unroll
    for (int j = 0; j <= NCPY; ++j) copy(s1, 1, j);
    // Tile cur is resident (the copies of nxt may still fly).
    if (wave < 2)
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(NCPY + 1));
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(NCPY));
  }
  barrier_nofence();
  int stc = 0;
  while (cur < nq) {
    const int nn = nxt < nq ? tl.tile(k + 2, nxt, tclass_g) : nq;
    const int stn = stc == 0 ? 2 : stc - 1;  // (stc + 2) % 3
    tile(cur, tl.klass(k, cur, tclass_g), stc, tile_src(nn), stn);
    // Tile nxt resident: only the copies of nn may be in flight.
    if (wave < 2)
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(NCPY + 1));
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(NCPY));
    barrier_nofence();
    cur = nxt;
    nxt = nn;
    ++k;
    stc = stc == 2 ? 0 : stc + 1;
  }
  // No copy may still be writing LDS when the block ends.
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

  if (p.qk_norm) {
    // dK of the raw (pre-norm) keys: the norm's VJP on the finished rows.
    float gy[NDB][16];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) gy[db][e] = dk[db][e] * p.scale;
    const int64_t xoff = b * p.k_str[0] + h * p.k_str[1] + (int64_t)kc * p.k_str[2];
    const float r = p.krstd[((int64_t)b * p.H + h) * p.Lk + kc];
    rms_norm_vjp_rows<T, NDB>(gy, (const T*)p.kraw + xoff, r, p.D, g);
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) dk[db][e] = gy[db][e];
  }
  if (kok) {
    T* dkp = (T*)p.dk + b * p.k_str[0] + h * p.k_str[1] + (int64_t)key * p.k_str[2];
    T* dvp = (T*)p.dv + b * p.v_str[0] + h * p.v_str[1] + (int64_t)key * p.v_str[2];
    const float sc = p.qk_norm ? 1.0f : p.scale;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d0 = db * 32 + 8 * c + 4 * g;
        if (d0 < p.D) store4(dkp + d0, dk[db], 4 * c, sc);
        if (d0 < p.Dv) store4(dvp + d0, dv[db], 4 * c, 1.0f);
      }
  }
  if constexpr (DBM == kDbColsum) {
    const float tot = colsum + shfl_xor32(colsum);
    if (kok && g == 0) store_db(p, dbbase, tot);
  }
}

// ---------------------------------------------------------------------------
// dQ.  Block = 4 waves x 32 queries (128); two blocks share a CU (one at
// head dim 256, where the stationary Q and dO and the dQ accumulators need
// a wave's 512 registers).  Each wave
// holds its queries' Q and dO rows stationary and streams 64-key tiles:
// S^T = K Q^T and dP^T = V dO^T put the query on the lane's column, so dS^T
// feeds dQ^T += K^T dS^T from registers; K^T comes from ds_read_b64_tr_b16
// reads of the row-major (swizzled) K tile.  K / V tiles reach an LDS ring
// by direct copies through buffer resources bounded at Lk (keys past it
// read as zero and are masked), one tile ahead at D >= 128 and two at D = 64,
// each wave copying its share between its S / dP products.  A bias that
// broadcasts over queries (BMODE kFbRow) enters S^T through one more MFMA
// per 32-key block, as in the forward; other biases take the element pass.
// ---------------------------------------------------------------------------
template <typename T, int DP, int BMODE, bool CAUSAL>
__global__ __launch_bounds__(256, DP > 128 ? 1 : 2) void dq16_kernel(const Params p) {
  using M = Mma<T>;
  using Frag = typename M::Frag;
  using MB = Mma<bf16>;  // the ones-column product of -delta
  constexpr int EPC = 8, KC = 16;
  constexpr int NW = 4, BM = NW * 32, BN = 64;
  constexpr int NC = DP / KC, NDB = DP / 32, FPB = M::FRAGS_PER_BLOCK;
  constexpr bool ROW_BIAS = BMODE == kFbRow;
  constexpr bool VALU_BIAS = BMODE == kFbValu;
  using KS = SwzStream<DP, NW>;
  constexpr int TILE_BYTES = BN * DP * 2;
  constexpr int ROWB_BYTES = ROW_BIAS ? NW * 256 : 0;  // each wave's copy of the bias row
  constexpr int STAGE_BYTES = 2 * TILE_BYTES + ROWB_BYTES;
  constexpr int NST = DP == 64 ? 3 : 2;                // K / V stages (two blocks per CU)
  constexpr int CPT = 2 * KS::CNT + (ROW_BIAS ? 1 : 0);  // copies per wave per tile
  // At D = 128 (two stages, so the next tile must land within the tile)
  // the copies ride with the first key block's products, one per two, for
  // the most time in flight; elsewhere one per four over both blocks.
  constexpr bool COPY_EARLY = DP == 128;
  __shared__ __attribute__((aligned(16))) char smem[NST * STAGE_BYTES];
  __shared__ uint32_t ainfo[kMaxBwdTiles];  // active key tiles, in order: index | class << 30
  __shared__ int nact_s;

  const int vid = xcd_remap(blockIdx.x, p.B * p.H, p.nqt);
  const int bh = vid / p.nqt;
  const int b = bh / p.H, h = bh % p.H;
  // Longest blocks first: by the mask's block order, else (causal) the last
  // query blocks, which see the most keys.
  const int qt = p.order ? ordered_tile(p, b, h, p.ord_q128, vid % p.nqt, p.nqt)
                         : p.nqt - 1 - (vid % p.nqt);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform
  const int g = lane >> 5, c32 = lane & 31;
  const int q0 = qt * BM;
  const int qw0 = q0 + wave * 32;
  const int qrow = qw0 + c32;
  const bool qok = qrow < p.Lq;
  const int qc = qok ? qrow : p.Lq - 1;

  const T* kp = (const T*)p.k + b * p.k_str[0] + h * p.k_str[1];
  const T* vp = (const T*)p.v + b * p.v_str[0] + h * p.v_str[1];
  const int64_t ks = p.k_str[2], vs = p.v_str[2];

  // --- active key tiles of this block (tile-map classes) --------------------
  const int k_end = CAUSAL ? min(p.Lk, q0 + BM) : p.Lk;
  const int nkt = (k_end + BN - 1) / BN;
  const bool listed = p.has_tilemap && nkt <= kMaxBwdTiles;
  auto class_g = [&](int t) -> int {
    return p.has_tilemap ? tile_class(p, b, h, q0, q0 + BM, t * BN, t * BN + BN) : 3;
  };
  if (listed && wave == 0) {
    int base = 0;
    for (int t0 = 0; t0 < nkt; t0 += 64) {
      const int t = t0 + lane;
      const int c = t < nkt ? class_g(t) : 0;
      const uint64_t m = __ballot(c & 1);
      if (c & 1) {
        const int pos = base + __popcll(m & ((1ull << lane) - 1));
        ainfo[pos] = (uint32_t)t | (uint32_t)c << 30;
      }
      base += __popcll(m);
    }
    if (lane == 0) nact_s = base;
  }
  __syncthreads();
  const int n = listed ? __builtin_amdgcn_readfirstlane(nact_s) : nkt;
  // Active tile i as index | class << 30 (index kTileEnd past the last
  // one; a length below 2^31 has fewer than 2^25 key tiles, so any index
  // fits the 30 bits).
  // Listed tiles take one LDS read, which the tile loop issues NST
  // iterations before the tile's use; unlisted ones are contiguous.
  auto info_raw = [&](int i) NXA_INLINE -> int {
    if (i >= n) return kTileEnd;
    if (listed) return (int)ainfo[i];
    return (int)((uint32_t)i | (uint32_t)class_g(i) << 30);
  };

  // --- stationary Q^T, dO^T fragments and per-row values ------------------------
  Frag qf[NC], df[NC];
  {
    const T* qp = (const T*)p.q + b * p.q_str[0] + h * p.q_str[1] +
                  (int64_t)qc * p.q_str[2];
    const T* dop = (const T*)p.dout + b * p.o_str[0] + h * p.o_str[1] +
                   (int64_t)qc * p.o_str[2];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d = c * KC + g * EPC;
      qf[c] = qok && d < p.D ? ld16(qp + d) : zero_frag<T>();
      df[c] = qok && d < p.Dv ? ld16(dop + d) : zero_frag<T>();
    }
  }
  // Per-row values of the backward, computed here for this block's rows
  // (the dK/dV kernel that runs next reads them from the workspace):
  // delta = sum_d O dO over the row (each lane of the pair l, l ^ 32 holds
  // half of it) and lse * log2(e), both negated.
  const int64_t rowid = ((int64_t)b * p.H + h) * p.Lq + qc;
  float dacc = 0.f;
  {
    const T* op = (const T*)p.o + b * p.o_str[0] + h * p.o_str[1] +
                  (int64_t)qc * p.o_str[2];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d = c * KC + g * EPC;
      const Frag of = (qok && d < p.Dv) ? ld16(op + d) : zero_frag<T>();
#pragma unroll
      for (int e = 0; e < EPC; ++e) dacc = __builtin_fmaf((float)of[e], (float)df[c][e], dacc);
    }
  }
  const float ndlt = -(dacc + shfl_xor32(dacc));
  const float neg_lse2 = -p.lse[rowid] * kLog2e;
  if (qok && g == 0) {
    p.ndelta[rowid] = ndlt;
    p.nlse2[rowid] = neg_lse2;
  }
  // -delta enters dP^T through one more MFMA per 32-key block: a column of
  // ones times the per-query value split into two bf16 terms (hi + lo, exact
  // to 2^-16 relative; bf16 for either T, whose range covers any finite fp32
  // value).  The logits are one FMA per element on the exact fp32 scores,
  // S c - lse2 (c = scale * log2(e)), and dS^T = exp2(.) (dP - delta).
  auto split_hi = [](float v) -> float { return (float)(bf16)v; };
  auto split_lo = [](float v, float hi) -> float {
    return __builtin_isfinite(v) ? (float)(bf16)(v - hi) : 0.f;
  };
  typename MB::Frag ones = zero_frag<bf16>(), bdlt = zero_frag<bf16>();
  if (g == 0) {
    ones[0] = ones[1] = (bf16)1.0f;
    const float dh = split_hi(ndlt);
    bdlt[0] = (bf16)dh;
    bdlt[1] = (bf16)split_lo(ndlt, dh);
  }
  const int64_t brow = VALU_BIAS ? b * p.bias_str[0] + h * p.bias_str[1] +
                                       (int64_t)qc * p.bias_str[2]
                                 : 0;
  const uint8_t* mrow = p.has_mask ? p.mask + b * p.mask_str[0] +
                                         h * p.mask_str[1] +
                                         (int64_t)qc * p.mask_str[2]
                                   : nullptr;
  // Row bias (of dtype T, as in the forward's row mode): B[0][q] = 1/scale
  // split into the T terms h + l for every query, reduction row 0 only, so
  // S^T accumulates bias / scale + K Q^T.
  Frag bdh = zero_frag<T>(), bdl = zero_frag<T>();
  if constexpr (ROW_BIAS) {
    bdh[0] = (T)(g == 0 ? p.bias_h : 0.f);
    bdl[0] = (T)(g == 0 ? p.bias_l : 0.f);
  }
  constexpr bool bias_l = ROW_BIAS;
  // The stationary loads complete here, so the waits in the tile loop only
  // count tile copies.
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

  f32x16 dq[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[db][r] = 0.f;

  // --- copies --------------------------------------------------------------------
  KS ksm, vsm;
  ksm.init(ks, p.D, wave, lane);
  vsm.init(vs, p.Dv, wave, lane);
  const uint32_t lds0 = lds_offset(smem);
  const T* bp = ROW_BIAS ? (const T*)p.bias + b * p.bias_str[0] + h * p.bias_str[1]
                         : nullptr;
  struct TileSrc {
    i32x4 k, v, r;  // K rows, V rows, bias row
  };
  // Sources of key tile kt (an empty range past the last one, so every
  // tile issues the same copies).
  auto tile_src = [&](int kt) NXA_INLINE -> TileSrc {
    const int k0 = (int)min((int64_t)kt * BN, (int64_t)p.Lk);
    // Keys of this tile that exist (0: empty ranges); each range covers only
    // the tile's own rows (below 64 row strides, bounded by the host).
    const int rows = min(p.Lk - k0, BN);
    TileSrc s;
    s.k = make_rsrc(kp + (int64_t)k0 * ks,
                    rows > 0 ? (uint32_t)(((int64_t)(rows - 1) * ks + p.D) * 2) : 0u);
    s.v = make_rsrc(vp + (int64_t)k0 * vs,
                    rows > 0 ? (uint32_t)(((int64_t)(rows - 1) * vs + p.Dv) * 2) : 0u);
    if constexpr (ROW_BIAS)
      s.r = make_rsrc(bp + k0, (uint32_t)max(rows, 0) * 2u);
    return s;
  };
  // Copy j of a tile into stage st: K share, V share, then the bias row
  // (lane l: keys 2(l % 32), 2(l % 32) + 1, so the row lands twice).
  auto copy = [&](const TileSrc& s, int st, int j) NXA_INLINE {
    const uint32_t at = lds0 + st * STAGE_BYTES;
    if (j < KS::CNT)
      dma16_buf(s.k, ksm.off[j], at + (j * NW + wave) * 1024);
    else if (j < 2 * KS::CNT)
      dma16_buf(s.v, vsm.off[j - KS::CNT], at + TILE_BYTES + ((j - KS::CNT) * NW + wave) * 1024);
    else if (ROW_BIAS)
      dma4_buf(s.r, 4u * c32, at + 2 * TILE_BYTES + wave * 256);
  };

  // --- per-lane LDS read offsets (bytes) ----------------------------------------
  uint32_t koff[NC];  // row reads: row c32 of a 32-key block, chunk 2m + g
#pragma unroll
  for (int m = 0; m < NC; ++m) koff[m] = 2 * swz_off<DP>(c32, 2 * m + g);
  const int tr_row = 4 * ((lane >> 4) >> 1) + ((lane & 15) >> 2);
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  uint32_t toff[NDB][2];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int col = db * 32 + tr_col;
      toff[db][hh] = 2 * (swz_off<DP>(tr_row + 8 * hh, col >> 3) + (col & 7));
    }
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  typedef __attribute__((address_space(3))) Frag lds_frag;
  typedef __attribute__((address_space(3))) T lds_t;
  typedef short i16x8 __attribute__((ext_vector_type(8)));
  auto tr_frag = [&](uint32_t a0, uint32_t a1) NXA_INLINE -> Frag {
    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(uintptr_t)a0);
    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(uintptr_t)a1);
    const i16x8 r = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(Frag, r);
  };
  auto vadd = [](uint32_t sb, uint32_t v) NXA_INLINE -> uint32_t {
    uint32_t r;
    asm("v_add_u32 %0, %1, %2" : "=v"(r) : "s"(sb), "v"(v));
    return r;
  };

  // --- tile loop ----------------------------------------------------------------
  // Tile i lives in stage i % NST; after the barrier that starts tile i the
  // stage of tile i - 1 is free and receives tile i + NST - 1.
  // win[j]: active tile i + j (info_raw, made uniform).
  int win[NST];
#pragma unroll
  for (int j = 0; j < NST; ++j) win[j] = __builtin_amdgcn_readfirstlane(info_raw(j));
  {
    TileSrc s0 = tile_src(win[0] & kTileEnd);
#pragma unroll
    for (int j = 0; j < CPT; ++j) copy(s0, 0, j);
    if constexpr (NST > 2) {
      TileSrc s1 = tile_src(win[1] & kTileEnd);
#pragma unroll
      for (int j = 0; j < CPT; ++j) copy(s1, 1, j);
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(CPT));
    } else {
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    }
  }
  barrier_nofence();

  for (int i = 0; i < n; ++i) {
    const int st = i % NST;
    const int stn = (i + NST - 1) % NST;
    const int ahead = info_raw(i + NST);  // uniform after the barrier below
    const TileSrc sn = tile_src(win[NST - 1] & kTileEnd);
    auto copy_next = [&](int j) NXA_INLINE { copy(sn, stn, j); };
    const uint32_t at = lds0 + st * STAGE_BYTES;
    const int k0 = (win[0] & kTileEnd) * BN;

    const int cls = (int)((uint32_t)win[0] >> 30);
    const bool need_mask = p.has_mask && !(cls & 2);
    const bool tail = k0 + BN > p.Lk;
    const bool diag = CAUSAL && (k0 + BN - 1 > qw0);
    const bool general = VALU_BIAS || need_mask || tail || diag;
    // A tile with nothing but mask bytes to apply: the mask loads read zero
    // past Lk (the key tail), and query rows past Lq are not stored, as in
    // the tiles without an element pass.
    const bool mask_only = !VALU_BIAS && !CAUSAL && need_mask;
    uint32_t ka[NC];
#pragma unroll
    for (int m = 0; m < NC; ++m) ka[m] = vadd(at, koff[m]);
    uint32_t ta[NDB][2];
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      ta[db][0] = vadd(at, toff[db][0]);
      ta[db][1] = vadd(at, toff[db][1]);
    }

    // Two 32-key blocks, one after the other.
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      // S^T (+ row bias) and dP^T: product j is S chunk j / 2 (j even) or
      // dP chunk j / 2 (j odd); A fragments are read PD products ahead, and
      // this wave's copies of tile i + NST - 1 ride along (COPY_EARLY).
      f32x16 s;
      f32x16 dp = MB::first(ones, bdlt);
      if constexpr (ROW_BIAS) {
        const uint32_t rb = at + 2 * TILE_BYTES + wave * 256;
        Frag a = zero_frag<T>();
        const T bv = *(const lds_t*)(uintptr_t)(rb + 2 * (kb * 32 + c32));
        a[0] = g == 0 ? bv : (T)0.f;
        s = M::first(a, bdh);
        if (bias_l) M::run(s, a, bdl);
      }
      constexpr int NP = 2 * NC, PD = DP == 128 ? (ROW_BIAS ? 3 : 4) : 8;
      auto afrag = [&](int j) NXA_INLINE -> Frag {
        const uint32_t base = ka[j >> 1] + ((j & 1) ? TILE_BYTES : 0);
        return *(const lds_frag*)(uintptr_t)(base + kb * (32 * DP * 2));
      };
      Frag abuf[PD];
#pragma unroll
      for (int j = 0; j < PD; ++j) abuf[j] = afrag(j);
#pragma unroll
      for (int j = 0; j < NP; ++j) {
        const int m = j >> 1;
        if (j & 1)
          M::run(dp, abuf[j % PD], df[m]);
        else if (!ROW_BIAS && j == 0)
          s = M::first(abuf[0], qf[0]);
        else
          M::run(s, abuf[j % PD], qf[m]);
        if (j + PD < NP) abuf[j % PD] = afrag(j + PD);
        const int pc = kb * NP + j;  // product count in this tile
        if constexpr (COPY_EARLY) {
          if ((pc & 1) == 1 && (pc >> 1) < CPT) copy_next(pc >> 1);
        } else {
          if ((pc & 3) == 3 && (pc >> 2) < CPT) copy_next(pc >> 2);
        }
      }
      if (kb == 1) {
#pragma unroll
        for (int jc = COPY_EARLY ? NP : NP / 2; jc < CPT; ++jc) copy_next(jc);
      }
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, PD, 0);
#pragma unroll
      for (int j = 0; j < NP; ++j) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
        if (j + PD < NP) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
      }

      // dS^T = P (dP - delta), P = exp2(S c - lse2) (+ element pass: GEN 1
      // mask bytes only, GEN 2 everything).
      Frag pd[FPB];
      auto ds_block = [&](auto gen_tag) NXA_INLINE {
        constexpr int GEN = decltype(gen_tag)::value;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int key0 = k0 + kb * 32 + 8 * c + 4 * g;
          f32x4 bv = {0.f, 0.f, 0.f, 0.f};
          uint32_t mw = 0x01010101u;
          if constexpr (GEN == 1) mw = load_mask4(p, mrow + key0, p.Lk - key0);
          if constexpr (GEN == 2) {
            if constexpr (VALU_BIAS) bv = load_bias4(p, p.bias, brow + key0, p.Lk - key0);
            if (need_mask) mw = load_mask4(p, mrow + key0, p.Lk - key0);
          }
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int r = 4 * c + j;
            float x = __builtin_fmaf(s[r], p.scale_log2, neg_lse2);
            if constexpr (GEN == 1) x = mask_bit(mw, j) ? x : -INFINITY;
            if constexpr (GEN == 2) {
              const int kk = key0 + j;
              if constexpr (VALU_BIAS) x = __builtin_fmaf(bv[j], kLog2e, x);
              bool keep = mask_bit(mw, j) && kk < p.Lk && qok;
              if (CAUSAL) keep = keep && kk <= qrow;
              x = keep ? x : -INFINITY;
            }
            dp[r] = fast_exp2(x) * dp[r];
          }
        }
#pragma unroll
        for (int f = 0; f < FPB; ++f) pd[f] = M::pack(dp, f);
      };
      if (!general)
        ds_block(std::integral_constant<int, 0>{});
      else if (mask_only)
        ds_block(std::integral_constant<int, 1>{});
      else
        ds_block(std::integral_constant<int, 2>{});

      // dQ^T += K^T dS^T.
      constexpr int NQ = FPB * NDB, PQ = NQ < 4 ? NQ : 4;
      auto kfrag = [&](int j) NXA_INLINE -> Frag {
        const int f = j / NDB, db = j % NDB;
        const uint32_t ro = (kb * 32 + 16 * f) * (DP * 2);
        return tr_frag(ta[db][0] + ro, ta[db][1] + ro);
      };
      Frag kbuf[PQ];
#pragma unroll
      for (int j = 0; j < PQ; ++j) kbuf[j] = kfrag(j);
#pragma unroll
      for (int j = 0; j < NQ; ++j) {
        M::run(dq[j % NDB], kbuf[j % PQ], pd[j / NDB]);
        if (j + PQ < NQ) kbuf[j % PQ] = kfrag(j + PQ);
      }
      // Keep that order: PQ fragment reads, then one product and one read
      // at a time (left to itself the compiler keeps one or two fragments
      // in flight, and the products wait on their reads).
#pragma unroll
      for (int j = 0; j < PQ; ++j) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
#pragma unroll
      for (int j = 0; j < NQ; ++j) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
        if (j + PQ < NQ) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
      }
    }

    // Tile i + 1 is resident before the barrier (later tiles may stay in
    // flight).
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(CPT * (NST - 2)));
    barrier_nofence();
#pragma unroll
    for (int j = 0; j + 1 < NST; ++j) win[j] = win[j + 1];
    win[NST - 1] = __builtin_amdgcn_readfirstlane(ahead);
  }
  // No copy may still be writing LDS when the block ends.
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

  if (p.qk_norm) {
    // dQ of the raw (pre-norm) queries: the norm's VJP on the finished rows
    // (both halves of a row take part in the row sum).  The raw rows are
    // read here, after the loop: dQ runs two blocks per CU, so the other
    // block's work covers the wait (staging them in the last iteration
    // measured no faster and costs the D = 128 kernel registers it has not
    // got).
    float gy[NDB][16];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) gy[db][e] = dq[db][e] * p.scale;
    const int64_t roff = b * p.q_str[0] + h * p.q_str[1] + (int64_t)qc * p.q_str[2];
    const float r = p.qrstd[((int64_t)b * p.H + h) * p.Lq + qc];
    rms_norm_vjp_rows<T, NDB>(gy, (const T*)p.qraw + roff, r, p.D, g);
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) dq[db][e] = gy[db][e];
  }
  if (qok) {
    T* dqp = (T*)p.dq + b * p.q_str[0] + h * p.q_str[1] + (int64_t)qrow * p.q_str[2];
    const float sc = p.qk_norm ? 1.0f : p.scale;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d0 = db * 32 + 8 * c + 4 * g;
        if (d0 < p.D) store4(dqp + d0, dq[db], 4 * c, sc);
      }
  }
}

// ---------------------------------------------------------------------------
// Launchers.
// ---------------------------------------------------------------------------
template <typename T, int DP, bool HB, bool CA, int DBM>
static void launch_dkdv16_t(Params p, hipStream_t stream) {
  p.nkt = (p.Lk + 127) / 128;
  const int n = p.nbh * p.nkt;
  hipLaunchKernelGGL((dkdv16_kernel<T, DP, HB, CA, DBM>), dim3(n), dim3(512), 0,
                     stream, p);
}

template <typename T, int DP, bool CA>
static void launch_dkdv16_db(const Params& p, hipStream_t stream) {
  if (!p.has_bias) {
    launch_dkdv16_t<T, DP, false, CA, kDbNone>(p, stream);
  } else if (p.dbias_mode == kDbiasFull) {
    launch_dkdv16_t<T, DP, true, CA, kDbFull>(p, stream);
  } else if (p.dbias_mode == kDbiasColsum) {
    launch_dkdv16_t<T, DP, true, CA, kDbColsum>(p, stream);
  } else {
    launch_dkdv16_t<T, DP, true, CA, kDbNone>(p, stream);
  }
}

template <typename T, bool HB, bool CA, int DBM>
static void launch_dkdv256_t(Params p, hipStream_t stream) {
  p.nkt = (p.Lk + 127) / 128;
  const int n = p.nbh * p.nkt;
  hipLaunchKernelGGL((dkdv256_kernel<T, HB, CA, DBM>), dim3(n), dim3(256), 0, stream, p);
}

template <typename T, bool CA>
static void launch_dkdv256_db(const Params& p, hipStream_t stream) {
  if (!p.has_bias)
    launch_dkdv256_t<T, false, CA, kDbNone>(p, stream);
  else if (p.dbias_mode == kDbiasFull)
    launch_dkdv256_t<T, true, CA, kDbFull>(p, stream);
  else if (p.dbias_mode == kDbiasColsum)
    launch_dkdv256_t<T, true, CA, kDbColsum>(p, stream);
  else
    launch_dkdv256_t<T, true, CA, kDbNone>(p, stream);
}

template <typename T>
static void launch_dkdv256(const Params& p, hipStream_t stream) {
  if (p.causal) launch_dkdv256_db<T, true>(p, stream);
  else launch_dkdv256_db<T, false>(p, stream);
}

template <typename T, int DP, int BMODE, bool CA>
static void launch_dq16_t(Params p, hipStream_t stream) {
  p.nqt = (p.Lq + 127) / 128;
  const int n = p.B * p.H * p.nqt;
  hipLaunchKernelGGL((dq16_kernel<T, DP, BMODE, CA>), dim3(n), dim3(256), 0, stream, p);
}

template <typename T, int DP, int BMODE>
static void launch_dq16_c(const Params& p, hipStream_t stream) {
  if (p.causal) launch_dq16_t<T, DP, BMODE, true>(p, stream);
  else launch_dq16_t<T, DP, BMODE, false>(p, stream);
}

// Bias: through an MFMA when it broadcasts over queries (the forward's row
// mode), else the element pass.
template <typename T, int DP>
static void launch_dq16_flags(const Params& p, hipStream_t stream) {
  if (!p.has_bias) launch_dq16_c<T, DP, kFbNone>(p, stream);
  else if (p.fwd_bias == kFbRow) launch_dq16_c<T, DP, kFbRow>(p, stream);
  else launch_dq16_c<T, DP, kFbValu>(p, stream);
}

}  // namespace nxa
