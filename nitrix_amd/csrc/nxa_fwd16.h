// 16-bit (bf16 / fp16 I/O) forward kernel for gfx950: fused flash-attention
// forward with an online softmax in base 2 and an fp32 log-sum-exp per query
// row.  Both element types share the code: the MFMA (bf16 or f16 32x32x16)
// and the conversions follow the template type T.
//
// Same math as the reference's forward Pallas kernel
// (src/nitrix/_kernels/cuda/attention.py:85-156): logits = scale * Q K^T +
// bias, masked entries -inf, softmax over keys, O = P V, lse = ln sum exp.
//
// Block = 8 waves x 32 queries (256 rows), one block per CU, two waves per
// SIMD.  Each wave computes S^T = K Q^T (the lane owns one query, so the row
// max needs one cross-half exchange and P feeds O^T += V^T P^T from
// registers); V^T comes from ds_read_b64_tr_b16 on the row-major V tile.
//
// K / V tiles (64 keys) travel from HBM straight into an LDS ring by direct
// global->LDS copies, issued tiles ahead of use.  Tiles are XOR-swizzled
// (swz_off), conflict-free for the K row reads and the V transposed reads;
// every wave issues the same number of copies per tile, so the waits are
// compile-time vmcnt immediates, and each lane's LDS read offsets are
// computed once per block.
//
// Schedule: the two waves of a SIMD ping-pong.  Every tile takes two phases
// (one block barrier per tile, two with full bias tiles); in one phase wave
// w runs its matrix products
// (O += P(t-1) V(t-1), S(t) = K(t) Q^T) while wave w + 4 runs the softmax of
// tile t-1 (VALU, v_exp), in the next they swap, so one wave of each SIMD
// pair keeps the matrix core busy while the other works on the VALU.
//
// Bias.  Rather than adding bias element by element on the VALU, the bias
// enters the score accumulator as MFMA products before Q K^T accumulates on
// top: S^T += bias^T x diag(1/scale), so S^T = K Q^T + bias / scale and the
// exponent's FMA by scale*log2(e) yields the logits of the reference.  1/scale
// is split into two terms h + l of the bias dtype, which these modes require
// to be T (l = 0 when 1/scale is a power of two, e.g. D = 64), so the bias
// contributes bias * (h + l) * scale = bias to within 2^-16 relative (bf16;
// 2^-22 for fp16).
//  * Full bias tiles (kFbTile, [query, key] rows of 64 keys): a ring of its
//    own holds the block's [256 x 64] bias tiles (XOR-swizzled, filled by
//    direct copies, 8 contiguous 128-byte rows per copy, each wave its own
//    32 rows); bias^T fragments are ds_read_b64_tr_b16 reads of it.  The
//    bias stream is the HBM-bound part of the kernel: at D = 64 it runs two
//    tiles ahead (K / V one), at D = 128 LDS allows one tile ahead and the
//    waves run in step (S, softmax, P V of tile t between barriers).
//  * Bias broadcast over queries (kFbRow): each wave copies the 64-key row
//    of the tile next to its K / V stage, one MFMA per 32-key block with the
//    bias in reduction row 0.
//
// Kernel and launcher templates; instantiated by nxa_fwd16.hip (head dims
// 64 and 128) and nxa_fwd16_wide.hip (256, compiled with flags of its own).
#pragma once

#include "nxa_common.h"
#include "nxa_launch.h"

#include <type_traits>

// Build-time tuning knobs (-D on the compiler line): the wave priority
// (s_setprio) of the matrix phase, and how many MFMA operand fragments the
// products read ahead of their use.
#ifndef FWD_PRIO
#define FWD_PRIO 1
#endif
#ifndef PD_FWD
#define PD_FWD 4
#endif
// In-step schedule (4-wave blocks): the next tiles' K / V copies ride along
// with the S products (1) or are issued before them (0).
#ifndef FWD_COPY_IN_S
#define FWD_COPY_IN_S 1
#endif

namespace nxa {

constexpr int kFwdMaxTiles = 1024;       // key tiles listed in LDS per block
constexpr float kFwdRescaleSlack = 8.0f;  // lazy max raise threshold (log2)
// Half-row tile sum of P accepted without a row max: every P is then below
// 2^15, inside the fp16 range of the packed P V operand.
constexpr float kFwdSumLimit = 32768.0f;

// max over the two 32-lane halves (lanes l and l ^ 32).
__device__ __forceinline__ float half_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x),
                                                  __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// s_waitcnt vmcnt(min(n, C)) for a wave-uniform n (the immediate must be a
// compile-time constant).
template <int C>
__device__ __forceinline__ void vm_wait_le(int n) {
  if constexpr (C == 0) {
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  } else {
    if (n >= C)
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(C));
    else
      vm_wait_le<C - 1>(n);
  }
}

// Ring geometry per (head-dim width, waves per block, bias mode).
// Ping-pong (LAG, 8 waves) schedule: after barrier t the waves read V(t-1)
// and K(t) (and bias tile t), so the K / V stage of tile t-2 and the bias
// stage of tile t-1 are free there.  With 4 K / V stages tile t+2 is issued
// after barrier t; with full bias tiles LDS holds 3 K / V stages (tile t+1
// issued, one ahead: K and V mostly come from L2) and 3 bias stages (tile
// t+2, two ahead: the bias streams from HBM).  In-step schedule (4-wave
// blocks, and D = 128 with full bias tiles): tile t is read only between
// barriers t and t+1, so the stage of tile t-1 receives tile t + NST - 1.
// Head dim 256 (4-wave blocks, one per CU): two 64 KB K / V stages, one tile
// ahead; no bias-tile ring (LDS is full).
template <int DP, int NW, int BMODE>
struct FwdRing {
  static constexpr bool TILE_BIAS = BMODE == kFbTile;
  static_assert(DP <= 128 || (NW == 4 && !TILE_BIAS), "head dim 256: 4 waves, no bias tiles");
  static constexpr bool LAG = NW == 8 && !(TILE_BIAS && DP == 128);
  static constexpr int NST = DP > 128 ? 2 : TILE_BIAS ? (LAG ? 3 : 2) : 4;  // K/V stages
  static constexpr int AHEAD = LAG ? NST - 2 : NST - 1;      // K/V tiles ahead
  static constexpr int NSTB = TILE_BIAS ? (LAG ? 3 : 2) : 1;  // bias stages
  static constexpr int AHEADB = TILE_BIAS ? NSTB - 1 : 0;     // bias tiles ahead
};

// NW waves of 32 queries per block: 8 (ping-pong pairs on each SIMD, one
// block per CU) or 4 (two blocks per CU; for masks that vary over queries, so
// that a block's key-tile list is that of its own 128 rows).  Head dim 256:
// 4 waves and one block per CU, so that each wave has the 512 registers that
// its stationary Q (64) and O (128) need.
template <typename T, int DP, int NW, int BMODE, bool CAUSAL>
__global__ __launch_bounds__(NW * 64, DP > 128 ? 1 : 2) void fwd16_kernel(const Params p) {
  using M = Mma<T>;
  using Frag = typename M::Frag;
  constexpr int EPC = 8, KC = 16;
  constexpr int BM = NW * 32, BN = 64;
  using R = FwdRing<DP, NW, BMODE>;
  constexpr int NST = R::NST, AHEAD = R::AHEAD, NSTB = R::NSTB, AHEADB = R::AHEADB;
  constexpr bool VALU_BIAS = BMODE == kFbValu;
  constexpr bool MFMA_BIAS = BMODE == kFbRow || BMODE == kFbTile;
  using KS = SwzStream<DP, NW>;
  constexpr int NC = DP / KC, NDB = DP / 32, FPB = M::FRAGS_PER_BLOCK;
  constexpr int TILE_ELEMS = BN * DP;
  constexpr int TILE_BYTES = TILE_ELEMS * 2;
  // Row bias: 256 bytes per wave (the 64-key row, twice) after K and V.
  constexpr int ROWB_ELEMS = BMODE == kFbRow ? NW * 128 : 0;
  constexpr int STAGE_ELEMS = 2 * TILE_ELEMS + ROWB_ELEMS;
  constexpr int STAGE_BYTES = STAGE_ELEMS * 2;
  // Tile bias: [BM queries x 64 keys] per stage, 4 KB (4 copies) per wave.
  constexpr int BT_ELEMS = BMODE == kFbTile ? BM * BN : 8;
  constexpr int BT_BYTES = BT_ELEMS * 2;
  constexpr int BT_COPIES = BMODE == kFbTile ? 4 : 0;
  // Copies each wave issues per tile into the K / V ring.
  constexpr int KV_COPIES = 2 * KS::CNT + (BMODE == kFbRow ? 1 : 0);
  __shared__ __attribute__((aligned(16))) T ring[NST * STAGE_ELEMS];
  __shared__ __attribute__((aligned(16))) T bring[NSTB * BT_ELEMS];
  __shared__ uint32_t ainfo[kFwdMaxTiles];  // active key tiles, in order: index | class << 16
  __shared__ int nact_s;
  // Mask bytes of the first partial key tiles of a query-broadcast mask
  // (mstage below): tile index per slot (-1: empty) and 64 bytes per slot.
  constexpr int kMaskSlots = 4;
  __shared__ int mslot_kt[kMaskSlots];
  __shared__ uint32_t mslot_w[kMaskSlots * 16];

  const int vid = xcd_remap(blockIdx.x, p.B * p.H, p.nqt);
  const int bh = vid / p.nqt;
  const int b = bh / p.H, h = bh % p.H;
  // Longest blocks first: by the mask's block order, else (causal) the last
  // query tiles, which see the most keys.
  const int qt = p.order ? ordered_tile(p, b, h, BM == 128 ? p.ord_q128 : p.ord_q256,
                                        vid % p.nqt, p.nqt)
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
  const bool listed = p.has_tilemap && nkt <= kFwdMaxTiles;
  auto class_g = [&](int t) -> int {
    return p.has_tilemap ? tile_class(p, b, h, q0, q0 + BM, t * BN, t * BN + BN) : 3;
  };
  // A mask shared by every query row (key padding) has the same bytes for
  // the whole block: wave 0 copies those of the first kMaskSlots partial
  // tiles into LDS before the first K / V copies, so the element pass of
  // such a tile reads LDS instead of waiting on a global load (whose wait
  // would also drain the K / V prefetch).  The copy is complete once wave
  // 0 passes the vmcnt(0) that follows its Q loads (below), and the first
  // tile barrier publishes it to the other waves.
  const bool mstage = listed && p.has_mask && p.tm_rows == 1 && p.mask_vec && !VALU_BIAS &&
                      !CAUSAL && p.scale_log2 > 0.f;
  const uint8_t* mrow0 = p.has_mask ? p.mask + b * p.mask_str[0] + h * p.mask_str[1] : nullptr;
  if (listed && wave == 0) {
    int base = 0, nsl = 0;
    for (int t0 = 0; t0 < nkt; t0 += 64) {
      const int t = t0 + lane;
      const int c = t < nkt ? class_g(t) : 0;
      const uint64_t m = __ballot(c & 1);
      if (c & 1) {
        const int pos = base + __popcll(m & ((1ull << lane) - 1));
        ainfo[pos] = (uint32_t)t | (uint32_t)c << 16;
      }
      base += __popcll(m);
      if (mstage) {
        const bool part = (c & 3) == 1;
        const uint64_t pm = __ballot(part);
        if (part) {
          const int s = nsl + __popcll(pm & ((1ull << lane) - 1));
          if (s < kMaskSlots) mslot_kt[s] = t;
        }
        nsl += __popcll(pm);
      }
    }
    if (lane == 0) nact_s = base;
    if (mstage) {
      if (lane >= nsl && lane < kMaskSlots) mslot_kt[lane] = -1;
      // Lane l: word l % 16 of slot l / 16; bytes past Lk (and empty slots,
      // addressed past the range) read as zero.  A block without a partial
      // tile never reads the slots, so it skips the copy.
      if (nsl > 0) {
        const int skt = mslot_kt[lane >> 4];
        const uint32_t voff =
            skt >= 0 ? (uint32_t)skt * (uint32_t)BN + 4u * (lane & 15) : 0xfffffff0u;
        dma4_buf(make_rsrc(mrow0, (uint32_t)p.Lk), voff, lds_offset(mslot_w));
      }
    }
  }
  __syncthreads();
  const int n = listed ? nact_s : nkt;
  // Active tile i as index | class << 16.  A listed tile takes one LDS
  // read: the tile loop issues the reads of the next iteration's tiles one
  // iteration early and makes them wave-uniform (the tile index feeds
  // scalar addresses) only then, so no lookup waits at a tile's start.
  // Unlisted tiles are contiguous and computed in place; the tile loop is
  // instantiated for both (LIST).
  auto info_raw = [&](int i) NXA_INLINE -> int { return i < n ? (int)ainfo[i] : 0; };
  auto uni = [](int x) NXA_INLINE -> int { return __builtin_amdgcn_readfirstlane(x); };
  auto tile_at = [&](auto list_tag, int i, int pre) NXA_INLINE -> int {
    if constexpr (decltype(list_tag)::value) return pre & 0xffff;
    else return i;
  };
  auto class_at = [&](auto list_tag, int i, int pre) NXA_INLINE -> int {
    if constexpr (decltype(list_tag)::value) return pre >> 16;
    else return class_g(i);
  };

  // --- stationary Q^T fragments ----------------------------------------------
  Frag qf[NC];
  {
    const T* qp = (const T*)p.q + b * p.q_str[0] + h * p.q_str[1] +
                     (int64_t)qrow * p.q_str[2];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d = c * KC + g * EPC;
      qf[c] = (qok && d < p.D) ? ld16(qp + d) : zero_frag<T>();
    }
  }
  const int64_t brow = VALU_BIAS ? b * p.bias_str[0] + h * p.bias_str[1] +
                                       (int64_t)qc * p.bias_str[2]
                                 : 0;
  const uint8_t* mrow = p.has_mask ? p.mask + b * p.mask_str[0] +
                                         h * p.mask_str[1] +
                                         (int64_t)qc * p.mask_str[2]
                                   : nullptr;

  // --- bias operands (MFMA bias modes) ---------------------------------------
  // diag(1/scale) as the B operand.  Tile mode: B[r][q] = h (or l) iff r == q,
  // with the reduction index r(f, g, e) = 16f + 8(e/4) + 4g + e%4 of the
  // transposed bias reads.  Row mode: reduction row 0 only, B[0][q] = h.
  const bool bias_l = MFMA_BIAS && p.bias_l != 0.f;  // uniform
  Frag bdh[2], bdl[2];
  if constexpr (BMODE == kFbTile) {
#pragma unroll
    for (int f = 0; f < 2; ++f)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const bool on = 16 * f + 8 * (e >> 2) + 4 * g + (e & 3) == c32;
        bdh[f][e] = (T)(on ? p.bias_h : 0.f);
        bdl[f][e] = (T)(on ? p.bias_l : 0.f);
      }
  } else if constexpr (BMODE == kFbRow) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const bool on = g == 0 && e == 0;
      bdh[0][e] = (T)(on ? p.bias_h : 0.f);
      bdl[0][e] = (T)(on ? p.bias_l : 0.f);
      bdh[1][e] = bdl[1][e] = (T)0.f;
    }
  }

  // The Q loads complete here, so the waits in the tile loop only count
  // tile copies (and the normalised rows below, which are older than every
  // copy: loads complete in order, so waiting for a copy never passes an
  // older one).
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

  // qk-norm of the raw q row the lane shares with lane ^ 32 (each holds
  // half of every 16-element chunk; padding past D is zero), in fp32 as the
  // reference's qk_rms_norm.  The normalised rows the backward streams are
  // stored here, before the first copies, so that no store is left to
  // drain when the block ends.
  if (p.qn_on) {
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int j = 0; j < EPC; ++j) ss = __builtin_fmaf(to_f32(qf[c][j]), to_f32(qf[c][j]), ss);
    ss += shfl_xor32(ss);
    const float qn_r = 1.0f / __builtin_sqrtf(ss / (float)p.D + p.qn_eps);
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int j = 0; j < EPC; ++j) qf[c][j] = (T)(to_f32(qf[c][j]) * qn_r);
    if (qok) {
      if (p.qn_out) {
        T* qo = (T*)p.qn_out + b * p.q_str[0] + h * p.q_str[1] + (int64_t)qrow * p.q_str[2];
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const int d = c * KC + g * EPC;
          if (d < p.D) *reinterpret_cast<Frag*>(qo + d) = qf[c];
        }
      }
      if (p.qn_rstd && g == 0) p.qn_rstd[((int64_t)b * p.H + h) * p.Lq + qrow] = qn_r;
    }
  }

  f32x16 oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[db][r] = 0.f;
  float m_ref = -INFINITY, l_i = 0.f;

  // --- copies ------------------------------------------------------------------
  KS ksm, vsm;
  ksm.init(ks, p.D, wave, lane);
  vsm.init(vs, p.Dv, wave, lane);
  const uint32_t lds0 = lds_offset(ring);
  const uint32_t ldsb = lds_offset(bring);

  // Tile bias: wave w fills rows 32w..32w+31 of the stage's [BM x 64] tile,
  // 8 rows (8 x 128 contiguous bytes) per 1 KB copy; 16-byte slot s of the
  // wave holds row s/8, key chunk (s%8) ^ swz<64>(row).  Rows past Lq are
  // clamped to the last row; in the tail tile key chunks past Lk read the
  // last chunk (Lk % 8 == 0 in this mode; those keys are masked).
  // Row bias: lane l copies keys 2(l%32), 2(l%32)+1 of the row.
  // Offsets are relative to the wave's first row (32 rows times the row
  // stride fit in 32 bits: the host bounds the stride).
  const T* bp = (const T*)p.bias;  // MFMA bias modes: bias dtype is T
  uint32_t boff[BT_COPIES > 0 ? BT_COPIES : 1];
  if constexpr (MFMA_BIAS) bp += b * p.bias_str[0] + h * p.bias_str[1];
  auto bias_chunk = [&](int m) NXA_INLINE -> int {
    const int sl = m * 64 + lane;
    return (sl & 7) ^ swz<64>(sl >> 3);
  };
  if constexpr (BMODE == kFbTile) {
    const int qlast = p.Lq - 1 - min(qw0, p.Lq - 1);  // rows of the wave in range - 1
    bp += (int64_t)min(qw0, p.Lq - 1) * p.bias_str[2];
#pragma unroll
    for (int m = 0; m < BT_COPIES; ++m) {
      const int r = min((m * 64 + lane) >> 3, qlast);
      boff[m] = 2u * (uint32_t)(r * p.bias_str[2] + 8 * bias_chunk(m));
    }
  }

  auto issue_kv = [&](int i, int kt) NXA_INLINE {
    const int k0 = kt * BN;
    const uint32_t at = lds0 + (i % NST) * STAGE_BYTES;
    ksm.issue(kp, ks, k0, p.Lk, p.D, at, wave, lane);
    vsm.issue(vp, vs, k0, p.Lk, p.Dv, at + TILE_BYTES, wave, lane);
    if constexpr (BMODE == kFbRow) {
      const int kk = min(k0 + 2 * c32, p.Lk - 2);
      dma4_sv(bp, 2u * (uint32_t)kk, at + 2 * TILE_BYTES + wave * 256);
    }
  };
  auto issue_bias = [&](int i, int kt) NXA_INLINE {
    if constexpr (BMODE == kFbTile) {
      const int k0 = kt * BN;
      const uint32_t bt = ldsb + (i % NSTB) * BT_BYTES + wave * (32 * BN * 2);
      if (k0 + BN <= p.Lk) {
#pragma unroll
        for (int m = 0; m < BT_COPIES; ++m) dma16_sv_nt(bp + k0, boff[m], bt + m * 1024);
      } else {
#pragma unroll
        for (int m = 0; m < BT_COPIES; ++m) {
          const int ch = bias_chunk(m);
          const int kk = min(k0 + 8 * ch, p.Lk - 8);
          dma16_sv_nt(bp, boff[m] + 2u * (uint32_t)(kk - 8 * ch), bt + m * 1024);
        }
      }
    }
  };
  // Tile i needs K/V(i) and bias(i).  Issued after K/V(i): bias(i+1) (LAG
  // with full bias tiles: K / V one ahead, bias two) or the K / V tiles
  // i+1 .. i+AHEAD-1 that exist.
  auto wait_tile = [&](int i) NXA_INLINE {
    if constexpr (R::LAG && BMODE == kFbTile) {
      if (i + 1 < n)
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(BT_COPIES));
      else
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    } else {
      const int later = min(AHEAD - 1, n - 1 - i);
      if (AHEAD > 2 && later >= 2)
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * KV_COPIES));
      else if (AHEAD > 1 && later >= 1)
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(KV_COPIES));
      else
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    }
  };

  // --- per-lane LDS read offsets (bytes) ----------------------------------------
  // K row reads: row (j&1)*32 + c32, chunk 2m + g (m = j/2).
  uint32_t koff[NC];
#pragma unroll
  for (int m = 0; m < NC; ++m) koff[m] = 2 * swz_off<DP>(c32, 2 * m + g);
  // Transposed reads (see lds_tr_frag): lane (grp, i) reads row
  // r0 + 16f + 4(grp/2) + i/4 [+8] at column col0 + 16(grp%2) + 4(i%4); the
  // swizzle depends only on the row's low 4 bits, so for each 32-column block
  // the offset is a per-lane constant plus a compile-time row offset.
  const int tr_row = 4 * ((lane >> 4) >> 1) + ((lane & 15) >> 2);
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  uint32_t voff[NDB][2];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int col = db * 32 + tr_col;
      voff[db][hh] = 2 * (swz_off<DP>(tr_row + 8 * hh, col >> 3) + (col & 7));
    }
  uint32_t btoff[2][2];
  if constexpr (BMODE == kFbTile) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int col = kb * 32 + tr_col;
        btoff[kb][hh] = 2 * (swz_off<64>(wave * 32 + tr_row + 8 * hh, col >> 3) + (col & 7));
      }
  }
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  typedef short i16x8 __attribute__((ext_vector_type(8)));
  auto tr_frag = [&](uint32_t a0, uint32_t a1) NXA_INLINE -> Frag {
    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(uintptr_t)a0);
    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(uintptr_t)a1);
    const i16x8 r = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(Frag, r);
  };
  typedef __attribute__((address_space(3))) Frag lds_frag;

  // LDS addresses: a per-lane offset plus the stage base, added once per
  // tile (as an opaque VGPR add, so every read of that offset folds its row
  // offset into the instruction's immediate).
  auto vadd = [](uint32_t sb, uint32_t v) NXA_INLINE -> uint32_t {
    uint32_t r;
    asm("v_add_u32 %0, %1, %2" : "=v"(r) : "s"(sb), "v"(v));
    return r;
  };

  // S = K Q^T (+ bias / scale) of tile i, two 32-key blocks.  The K
  // fragments are read PD products ahead of their use (a rotating register
  // buffer) to cover the LDS latency.
  constexpr int PD = PD_FWD < 2 * NC ? PD_FWD : 2 * NC;
  f32x16 S[2];  // scores of one tile, two 32-key blocks
  auto qk = [&](int i, auto&& between) NXA_INLINE {
    const uint32_t kt = lds0 + (i % NST) * STAGE_BYTES;
    uint32_t ka[NC];
#pragma unroll
    for (int m = 0; m < NC; ++m) ka[m] = vadd(kt, koff[m]);
    // Product j: key block j & 1, head-dim chunk pair m = j >> 1.
    auto kfrag = [&](int j) NXA_INLINE -> Frag {
      return *(const lds_frag*)(uintptr_t)(ka[j >> 1] + (j & 1) * (32 * DP * 2));
    };
    // The products of one tile.  LB: the bias products include the 1/scale
    // remainder l (a wave-uniform choice made once per tile, outside the
    // straight-line sequence, so that its reads and products schedule as
    // one block).
    auto products = [&](auto lb_tag) NXA_INLINE {
      constexpr bool LB = decltype(lb_tag)::value;
      // Bias operands, all read before the first product: the bias^T
      // fragments of the tile (tile mode; rows = this wave's queries,
      // columns = keys) or the two 32-key row segments (row mode).
      Frag bfr[2][2];
      if constexpr (BMODE == kFbTile) {
        const uint32_t bt = ldsb + (i % NSTB) * BT_BYTES;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          const uint32_t b0 = vadd(bt, btoff[kb][0]), b1 = vadd(bt, btoff[kb][1]);
#pragma unroll
          for (int f = 0; f < 2; ++f) bfr[kb][f] = tr_frag(b0 + f * (16 * 128), b1 + f * (16 * 128));
        }
      } else if constexpr (BMODE == kFbRow) {
        const T* Bs = ring + (i % NST) * STAGE_ELEMS + 2 * TILE_ELEMS + wave * 128;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          bfr[kb][0] = zero_frag<T>();
          const T bv = Bs[kb * 32 + c32];
          bfr[kb][0][0] = g == 0 ? bv : (T)0.f;
        }
      }
      Frag kbuf[PD];
#pragma unroll
      for (int j = 0; j < PD; ++j) kbuf[j] = kfrag(j);
      constexpr int NBF = BMODE == kFbTile ? 2 : 1;  // bias fragments per key block
      if constexpr (MFMA_BIAS) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int f = 0; f < NBF; ++f) {
            if (f == 0)
              S[kb] = M::first(bfr[kb][f], bdh[f]);
            else
              M::run(S[kb], bfr[kb][f], bdh[f]);
            if constexpr (LB) M::run(S[kb], bfr[kb][f], bdl[f]);
          }
      }
#pragma unroll
      for (int j = 0; j < 2 * NC; ++j) {
        if (!MFMA_BIAS && j < 2)
          S[j & 1] = M::first(kbuf[j % PD], qf[j >> 1]);
        else
          M::run(S[j & 1], kbuf[j % PD], qf[j >> 1]);
        if (j + PD < 2 * NC) kbuf[j % PD] = kfrag(j + PD);
        between(j);
      }
      // Keep that order: the bias reads, PD K reads, the bias products,
      // then one product and one read at a time.
      if constexpr (BMODE == kFbTile)
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 8, 0);
      else if constexpr (BMODE == kFbRow)
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
#pragma unroll
      for (int j = 0; j < PD; ++j) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
      if constexpr (MFMA_BIAS)
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2 * NBF * (LB ? 2 : 1), 0);
#pragma unroll
      for (int j = 0; j < 2 * NC; ++j) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
        if (j + PD < 2 * NC) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
      }
    };
    if (MFMA_BIAS && bias_l)
      products(std::true_type{});
    else
      products(std::false_type{});
  };

  // Whether tile i needs the element-wise pass (mask bytes, key tail, causal
  // diagonal, VALU bias, non-positive scale).  Otherwise the scale is folded
  // into the exponent's FMA and the max is taken on raw scores.
  auto tile_general = [&](int kt, int cls) NXA_INLINE -> bool {
    const int k0 = kt * BN;
    const bool need_mask = p.has_mask && !(cls & 2);
    const bool tail = k0 + BN > p.Lk;
    const bool diag = CAUSAL && (k0 + BN - 1 > qw0);
    return VALU_BIAS || need_mask || tail || diag || !(p.scale_log2 > 0.f);
  };
  // Whether a general tile needs nothing but its mask bytes (no VALU bias,
  // not causal, positive scale): its scores then stay raw, masked entries
  // -inf, and the exponent's FMA applies the scale as on full tiles.  The
  // mask loads read zero past Lk, so the mask also covers a key tail.
  auto mask_only = [&](int cls) NXA_INLINE -> bool {
    return !VALU_BIAS && !CAUSAL && p.has_mask && !(cls & 2) && p.scale_log2 > 0.f;
  };
  // Element-wise pass of a general tile: logits in log2 units (raw scores
  // for mask_only tiles), masked entries -inf.  Every element is written
  // exactly once, unconditionally: masked entries are a select, never a
  // divergent partial write.
  auto mask_tile = [&](int kt, int cls) NXA_INLINE {
    const int k0 = kt * BN;
    const bool need_mask = p.has_mask && !(cls & 2);
    if (mask_only(cls)) {
      int slot = -1;
      if (mstage) {
#pragma unroll
        for (int s = 0; s < kMaskSlots; ++s)
          if (mslot_kt[s] == kt) slot = s;
        slot = __builtin_amdgcn_readfirstlane(slot);
      }
      if (slot >= 0) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const uint32_t mw = mslot_w[slot * 16 + kb * 8 + 2 * c + g];
#pragma unroll
            for (int j = 0; j < 4; ++j)
              S[kb][4 * c + j] = mask_bit(mw, j) ? S[kb][4 * c + j] : -INFINITY;
          }
        return;
      }
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int key0 = k0 + kb * 32 + 8 * c + 4 * g;
          const uint32_t mw = load_mask4(p, mrow + key0, p.Lk - key0);
#pragma unroll
          for (int j = 0; j < 4; ++j)
            S[kb][4 * c + j] = mask_bit(mw, j) ? S[kb][4 * c + j] : -INFINITY;
        }
      return;
    }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int key0 = k0 + kb * 32 + 8 * c + 4 * g;
        f32x4 bv = {0.f, 0.f, 0.f, 0.f};
        if constexpr (VALU_BIAS) bv = load_bias4(p, p.bias, brow + key0, p.Lk - key0);
        uint32_t mw = 0x01010101u;
        if (need_mask) mw = load_mask4(p, mrow + key0, p.Lk - key0);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int key = key0 + j;
          float x = S[kb][4 * c + j] * p.scale_log2;
          if constexpr (VALU_BIAS) x = __builtin_fmaf(bv[j], kLog2e, x);
          bool keep = mask_bit(mw, j) && key < p.Lk;
          if (CAUSAL) keep = keep && key <= qrow;
          S[kb][4 * c + j] = keep ? x : -INFINITY;
        }
      }
  };
  // Row max of the tile (in log2 units: raw scores times cc): two chains of
  // three-input maxima.  Written as v_max3_f32 directly: the compiler's
  // IEEE-mode fmaxf would first quiet each MFMA output separately (scores
  // are never NaN here; masked entries are -inf).
  auto max3 = [](float a, float b, float c) NXA_INLINE -> float {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
  };
  auto row_max = [&](float cc) NXA_INLINE -> float {
    // The max3 below is inline assembly, which the compiler's hazard
    // checks do not see: on the first tile of a block it can follow the S
    // products directly, so 16 wait states cover the MFMA result latency
    // (the rare redo path only).
    asm volatile("s_nop 7\n\ts_nop 7");
    float mx[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      mx[kb] = max3(S[kb][0], S[kb][1], S[kb][2]);
#pragma unroll
      for (int r = 3; r + 1 < 16; r += 2) mx[kb] = max3(mx[kb], S[kb][r], S[kb][r + 1]);
    }
    const float m = max3(mx[0], mx[1], max3(S[0][15], S[1][15], -INFINITY));
    return half_max(m) * cc;
  };
  // Lazily raised reference max: only a row max more than kFwdRescaleSlack
  // above the reference moves it.  O and l always accumulate against the
  // same reference, so the result is exact; l is rescaled here, O by the
  // caller (after the products of the previous reference have landed).
  auto raise_ref = [&](float mt, float& alpha) NXA_INLINE -> bool {
    const bool raise = mt > m_ref + kFwdRescaleSlack;
    alpha = raise ? fast_exp2(m_ref - mt) : 1.f;
    m_ref = raise ? mt : m_ref;
    l_i *= alpha;
    return __any(raise);
  };
  auto rescale_o = [&](float alpha) NXA_INLINE {
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;
  };
  // P = exp2(S cc - m_ref) of the tile, packed to the T reduction fragments
  // of P V; returns this lane's half-row sum of P (four chains per block).
  // S is left intact, so a tile can be redone against another reference.
  Frag pf[2][FPB];
  auto exp_tile = [&](float cc) NXA_INLINE -> float {
    const float neg_m = (m_ref == -INFINITY) ? 0.f : -m_ref;
    float ts = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      f32x16 pt;
      float rs[4];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        pt[r] = fast_exp2(__builtin_fmaf(S[kb][r], cc, neg_m));
        rs[r & 3] = r < 4 ? pt[r] : rs[r & 3] + pt[r];
      }
      ts += (rs[0] + rs[1]) + (rs[2] + rs[3]);
#pragma unroll
      for (int f = 0; f < FPB; ++f) pf[kb][f] = M::pack(pt, f);
    }
    return ts;
  };

  // O^T += V^T P^T for tile i (P^T from exp_tile).
  constexpr int NPV = 2 * FPB * NDB;
  auto pv = [&](int i) NXA_INLINE {
    const uint32_t vt = lds0 + (i % NST) * STAGE_BYTES + TILE_BYTES;
    uint32_t va[NDB][2];
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      va[db][0] = vadd(vt, voff[db][0]);
      va[db][1] = vadd(vt, voff[db][1]);
    }
    // Product j: key block kb = j / (FPB NDB), fragment f, head-dim block db.
    auto vfrag = [&](int j) NXA_INLINE -> Frag {
      const int kb = j / (FPB * NDB), f = (j / NDB) % FPB, db = j % NDB;
      const uint32_t ro = (kb * 32 + 16 * f) * (DP * 2);
      return tr_frag(va[db][0] + ro, va[db][1] + ro);
    };
    Frag vbuf[PD];
#pragma unroll
    for (int j = 0; j < PD; ++j) vbuf[j] = vfrag(j);
#pragma unroll
    for (int j = 0; j < NPV; ++j) {
      M::run(oacc[j % NDB], vbuf[j % PD], pf[j / (FPB * NDB)][(j / NDB) % FPB]);
      if (j + PD < NPV) vbuf[j % PD] = vfrag(j + PD);
    }
    // Each V fragment is two transposed reads.
#pragma unroll
    for (int j = 0; j < PD; ++j) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
#pragma unroll
    for (int j = 0; j < NPV; ++j) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      if (j + PD < NPV) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
    }
  };

  // --- schedule -------------------------------------------------------------------
  // Infos an iteration uses, read during the iteration before: the K / V
  // tile it issues (i + AHEAD), the bias tile (i + AHEADB) and the tile of
  // its softmax (i, or i - 1 in the lagging waves).
  struct Infos {
    int kv, bias, sm;
  };
  auto issue_ahead = [&](auto lt, int i, const Infos& f) NXA_INLINE {
    if (i + AHEAD < n) issue_kv(i + AHEAD, tile_at(lt, i + AHEAD, f.kv));
    if constexpr (BMODE == kFbTile)
      if (i + AHEADB < n) issue_bias(i + AHEADB, tile_at(lt, i + AHEADB, f.bias));
  };
  auto prologue = [&](auto lt) NXA_INLINE {
    constexpr int NA = AHEAD > AHEADB ? AHEAD : AHEADB;
    constexpr bool LIST = decltype(lt)::value;
#pragma unroll
    for (int a = 0; a < NA; ++a) {
      const int inf = LIST ? uni(info_raw(a)) : 0;
      if (a < AHEAD && a < n) issue_kv(a, tile_at(lt, a, inf));
      if (BMODE == kFbTile && a < AHEADB && a < n) issue_bias(a, tile_at(lt, a, inf));
    }
  };
  // Infos of iteration i (sm: tile j), as raw LDS values.
  auto infos_raw = [&](int i, int j) NXA_INLINE -> Infos {
    return {info_raw(i + AHEAD), BMODE == kFbTile ? info_raw(i + AHEADB) : 0,
            info_raw(j < 0 ? 0 : j)};
  };
  auto infos_uni = [&](const Infos& r) NXA_INLINE -> Infos {
    return {uni(r.kv), uni(r.bias), uni(r.sm)};
  };
  // Matrix work of tile i: O += P(i-1) V(i-1), then S = K(i) Q^T, with
  // `between` after each S product.
  auto mfma_phase = [&](int i, auto&& between) NXA_INLINE {
    // The wave feeding the matrix core issues first whenever it can; the
    // softmax wave of the pair fills the remaining issue slots.
    __builtin_amdgcn_s_setprio(FWD_PRIO);
    if (i > 0) pv(i - 1);
    if (i < n) qk(i, between);
    __builtin_amdgcn_s_setprio(0);
  };
  auto no_copy = [](int) {};
  // The wave's K / V copies of tile i + AHEAD spread over the S products of
  // tile i, one every SPC products (the row bias copy goes first), instead
  // of holding the wave at the copy path before its first product: `body`
  // receives the callback that qk runs after each product.
  auto with_copies = [&](auto lt, int i, const Infos& f, auto&& body) NXA_INLINE {
    const bool nx = i + AHEAD < n;
    const int k0n = nx ? tile_at(lt, i + AHEAD, f.kv) * BN : 0;
    const uint32_t atn = lds0 + ((i + AHEAD) % NST) * STAGE_BYTES;
    if constexpr (BMODE == kFbRow) {
      if (nx) {
        const int kk = min(k0n + 2 * c32, p.Lk - 2);
        dma4_sv(bp, 2u * (uint32_t)kk, atn + 2 * TILE_BYTES + wave * 256);
      }
    }
    const T* kb = kp + (int64_t)k0n * ks;
    const T* vb = vp + (int64_t)k0n * vs;
    uint32_t ok[KS::CNT], ov[KS::CNT];
#pragma unroll
    for (int m = 0; m < KS::CNT; ++m) {
      ok[m] = ksm.off[m];
      ov[m] = vsm.off[m];
    }
    if (nx && k0n + BN > p.Lk) {
      // Tail tile: rows past Lk read the last row.
#pragma unroll
      for (int m = 0; m < KS::CNT; ++m) {
        const int r = min(KS::row_of(m, wave, lane), p.Lk - 1 - k0n);
        ok[m] = 2u * (uint32_t)(r * ks + KS::col_of(m, wave, lane, p.D));
        ov[m] = 2u * (uint32_t)(r * vs + KS::col_of(m, wave, lane, p.Dv));
      }
    }
    constexpr int SPC = NC / KS::CNT;  // S products per copy (2 NC products, 2 CNT copies)
    static_assert(NC % KS::CNT == 0, "copies spread evenly over the S products");
    body([&](int j) NXA_INLINE {
      if (nx && j % SPC == SPC - 1) {
        const int c = j / SPC;
        if (c < KS::CNT)
          dma16_sv(kb, ok[c], atn + (c * NW + wave) * 1024);
        else
          dma16_sv(vb, ov[c - KS::CNT], atn + TILE_BYTES + ((c - KS::CNT) * NW + wave) * 1024);
      }
    });
  };
  // VALU work of tile i: element-wise pass (general tiles), P = exp(...)
  // and, when needed, the row max and a lazy reference update (O is
  // complete up to tile i-1 here).
  auto valu_phase = [&](auto lt, int i, int pre) NXA_INLINE {
    if (i < 0 || i >= n) return;
    const int kt = tile_at(lt, i, pre), cls = class_at(lt, i, pre);
    const bool gen = tile_general(kt, cls);
    if (gen) mask_tile(kt, cls);
    const float cc = gen && !mask_only(cls) ? 1.0f : p.scale_log2;
    float alpha;
    // Optimistic pass against the current reference, no row max: kept
    // when every half-row sum of the tile's P (32 keys) is at most 2^15
    // (then no P exceeds 2^15); otherwise, or before a row has a
    // reference, the tile takes the row max, raises the reference (a sum
    // above 2^15 means a P above 2^10, so the max exceeds the reference by
    // more than the slack) and is redone.  O and l always accumulate
    // against the reference in force, so the result is exact either way.
    float ts = 0.f;
    bool redo = __any(m_ref == -INFINITY);
    if (!redo) {
      ts = exp_tile(cc);
      redo = __any(!(ts <= kFwdSumLimit));
    }
    if (redo) {
      if (raise_ref(row_max(cc), alpha)) rescale_o(alpha);
      ts = exp_tile(cc);
    }
    l_i += ts;
  };
  if constexpr (R::LAG) {
    // Ping-pong: every tile takes two phases.  In phase a of tile t the
    // leading wave (w < 4) runs its matrix work while the lagging wave
    // (w + 4, same SIMD) runs the softmax of tile t-1; in phase b they swap.
    // One block barrier per tile orders the LDS ring (tile t resident, the
    // stage of tile t-2 free for the copies issued after it); a second one
    // between the phases keeps the pairs in step only with full bias tiles,
    // whose HBM stream it paces (without bias tiles it costs 1-2.5 %).
    // Without bias tiles each wave's copies of tile t+2 ride along with its
    // own S products, which keeps the copy path from holding both waves of
    // a SIMD after the barrier (tile t+2 has more than a tile to land).
    constexpr bool MID_BARRIER = BMODE == kFbTile;
    constexpr bool COPY_IN_MFMA = BMODE != kFbTile && AHEAD >= 2;
    auto run = [&](auto lag_tag, auto lt) {
      constexpr bool LAG = decltype(lag_tag)::value;
      constexpr bool LIST = decltype(lt)::value;
      prologue(lt);
      Infos f = {0, 0, 0};
      if constexpr (LIST) f = infos_uni(infos_raw(0, LAG ? -1 : 0));
      for (int i = 0; i < n; ++i) {
        Infos r = {0, 0, 0};
        if constexpr (LIST) r = infos_raw(i + 1, LAG ? i : i + 1);
        wait_tile(i);
        barrier_nofence();
        auto matrix = [&]() NXA_INLINE {
          if constexpr (COPY_IN_MFMA)
            with_copies(lt, i, f, [&](auto&& between) NXA_INLINE { mfma_phase(i, between); });
          else
            mfma_phase(i, no_copy);
        };
        if constexpr (!COPY_IN_MFMA) issue_ahead(lt, i, f);
        if (LAG) valu_phase(lt, i - 1, f.sm);
        else matrix();
        if constexpr (MID_BARRIER) barrier_nofence();
        if (LAG) matrix();
        else valu_phase(lt, i, f.sm);
        if constexpr (LIST) f = infos_uni(r);
      }
      if (n > 0) {
        barrier_nofence();
        if (LAG) valu_phase(lt, n - 1, f.sm);
        else mfma_phase(n, no_copy);
        barrier_nofence();
        if (LAG) mfma_phase(n, no_copy);
      }
    };
    if (wave >= NW / 2) {
      if (listed) run(std::true_type{}, std::true_type{});
      else run(std::true_type{}, std::false_type{});
    } else {
      if (listed) run(std::false_type{}, std::true_type{});
      else run(std::false_type{}, std::false_type{});
    }
  } else {
    // In-step: every wave runs S, softmax, O += P V of tile t between
    // barriers t and t+1.
    constexpr bool COPY_IN_S = FWD_COPY_IN_S && (DP > 128 || BMODE != kFbTile);
    auto run = [&](auto lt) {
      constexpr bool LIST = decltype(lt)::value;
      prologue(lt);
      Infos f = {0, 0, 0};
      if constexpr (LIST) f = infos_uni(infos_raw(0, 0));
      for (int i = 0; i < n; ++i) {
        Infos r = {0, 0, 0};
        if constexpr (LIST) r = infos_raw(i + 1, i + 1);
        wait_tile(i);
        barrier_nofence();
        if constexpr (COPY_IN_S) {
          // The K / V copies of tile i + AHEAD ride along with the S
          // products (one per two).
          with_copies(lt, i, f, [&](auto&& between) NXA_INLINE { qk(i, between); });
        } else {
          issue_ahead(lt, i, f);
          qk(i, [](int) {});
        }
        valu_phase(lt, i, f.sm);
        pv(i);
        if constexpr (LIST) f = infos_uni(r);
      }
    };
    if (listed)
      run(std::true_type{});
    else
      run(std::false_type{});
  }

  // Finalise: O = O / l (a fully masked row gives 0/0 = NaN, as the
  // reference's softmax over all -inf logits does), lse = ln sum exp.
  const float l = l_i + shfl_xor32(l_i);
  const float inv = 1.0f / l;
  if (qok) {
    T* op = (T*)p.o + b * p.o_str[0] + h * p.o_str[1] + (int64_t)qrow * p.o_str[2];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d0 = db * 32 + 8 * c + 4 * g;
        if (d0 < p.Dv) store4(op + d0, oacc[db], 4 * c, inv);
      }
    if (g == 0 && p.lse)
      p.lse[((int64_t)b * p.H + h) * p.Lq + qrow] = (m_ref + __log2f(l)) * kLn2;
  }
}

template <typename T, int DP, int NW, int BMODE, bool CA>
static void launch_fwd16_t(Params p, hipStream_t stream) {
  constexpr int BM = NW * 32;
  p.nqt = (p.Lq + BM - 1) / BM;
  const int n = p.B * p.H * p.nqt;
  hipLaunchKernelGGL((fwd16_kernel<T, DP, NW, BMODE, CA>), dim3(n), dim3(NW * 64), 0, stream,
                     p);
}

template <typename T, int DP, int NW, int BMODE>
static void launch_fwd16_c(const Params& p, hipStream_t stream) {
  if (p.causal) launch_fwd16_t<T, DP, NW, BMODE, true>(p, stream);
  else launch_fwd16_t<T, DP, NW, BMODE, false>(p, stream);
}

// 4-wave blocks when the mask varies over queries (its tile map has rows) at
// D <= 64, where two such blocks (4 K / V stages each) share a CU's LDS;
// full bias tiles keep the 8-wave block, whose bias ring they need.
template <typename T, int DP, int BMODE>
static void launch_fwd16_nw(const Params& p, hipStream_t stream) {
  if constexpr (DP > 128) {
    launch_fwd16_c<T, DP, 4, BMODE>(p, stream);
  } else {
    if constexpr (DP == 64 && BMODE != kFbTile) {
      if (p.has_tilemap && p.tm_rows > 1) {
        launch_fwd16_c<T, DP, 4, BMODE>(p, stream);
        return;
      }
    }
    launch_fwd16_c<T, DP, 8, BMODE>(p, stream);
  }
}

template <typename T, int DP>
static void launch_fwd16_flags(const Params& p, hipStream_t stream) {
  switch (p.has_bias ? p.fwd_bias : kFbNone) {
    case kFbRow: launch_fwd16_nw<T, DP, kFbRow>(p, stream); break;
    case kFbTile:
      // The host maps full bias tiles to the element pass above DP = 128.
      if constexpr (DP <= 128) launch_fwd16_nw<T, DP, kFbTile>(p, stream);
      else launch_fwd16_nw<T, DP, kFbValu>(p, stream);
      break;
    case kFbValu: launch_fwd16_nw<T, DP, kFbValu>(p, stream); break;
    default: launch_fwd16_nw<T, DP, kFbNone>(p, stream); break;
  }
}

}  // namespace nxa
