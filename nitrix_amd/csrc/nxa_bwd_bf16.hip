// bf16 backward kernels for gfx950: dK/dV (+ dbias) and dQ.
//
// Same math as the reference's two backward Pallas kernels
// (src/nitrix/_kernels/cuda/attention.py:272-332 dK/dV, :335-387 dQ):
// P = exp2(S * scale * log2e + bias * log2e - lse2), dS = P (dP - delta),
// dV = P^T dO, dK = scale dS^T Q, dQ = scale dS K.  Deterministic (no
// atomics): dK/dV own key tiles and stream query tiles, dQ owns query tiles
// and streams key tiles.
//
// Layout choices for CDNA4:
// * streamed tiles stay row-major in LDS; the transposed operands
//   (dO^T, Q^T for dV/dK, K^T for dQ) come from ds_read_b64_tr_b16, so no
//   transposed copies are written;
// * tiles read both ways (Q, dO in dK/dV; K in dQ) are XOR-swizzled by
//   16-byte chunk, conflict-free for the 16-byte row reads of the S / dP
//   products and for the transposed reads; row-read-only tiles are padded;
// * the next tile is fetched into registers while the current one is
//   consumed (double-buffered LDS, one barrier per tile);
// * per-row LSE / delta are read as float4 for the four consecutive rows a
//   lane's accumulator group covers.
#include "nxa_common.h"
#include "nxa_launch.h"

#include <type_traits>

namespace nxa {

constexpr int kMaxBwdTiles = 1024;

// dbias handling compiled into dK/dV.
enum : int { kDbNone = 0, kDbFull = 1, kDbColsum = 2 };

__device__ __forceinline__ void store_db(const Params& p, int64_t off, float x) {
  if (p.dbias_f32 || p.bias_dtype == kF32)
    reinterpret_cast<float*>(p.dbias)[off] = x;
  else
    reinterpret_cast<bf16*>(p.dbias)[off] = (bf16)x;
}

__device__ __forceinline__ float load_bias1(const Params& p, int64_t off) {
  return p.bias_dtype == kBF16 ? (float)reinterpret_cast<const bf16*>(p.bias)[off]
                               : reinterpret_cast<const float*>(p.bias)[off];
}

// ---------------------------------------------------------------------------
// dK / dV.  Block = 8 waves over 128 keys: waves 0-3 accumulate dV, waves 4-7
// accumulate dK (and dbias) for the same 32-key column each; a dV wave and a
// dK wave share a SIMD, so one's softmax VALU overlaps the other's MFMAs.
// Splitting the roles keeps each wave under 256 registers (two waves per
// SIMD) at the price of computing S = Q K^T in both roles.
//
// Each wave computes S = Q K^T (and dP = dO V^T for dK) with the key as the
// lane's column, so P and dS feed dV^T = dO^T P and dK^T = Q^T dS from
// registers.  Query tiles (Q, dO, lse2, delta) move straight from HBM into a
// 3-stage LDS ring with direct global->LDS copies, two tiles ahead; each wave
// waits only for its own copies of the next tile before the per-tile barrier.
// ---------------------------------------------------------------------------
template <int DP, bool HAS_BIAS, bool CAUSAL, int DBM>
__global__ __launch_bounds__(512, 1) void dkdv_bf16_kernel(const Params p) {
  using M = Mma<bf16>;
  using Frag = bf16x8;
  constexpr int EPC = 8, KC = 16;
  constexpr int BNK = 128, BQ = 64, NW = 8;
  using PT = PTile<DP>;
  // Only the dV waves (0-3) copy query tiles: their MFMA chain is shorter,
  // so the copy issue (limited by the CU's address unit) fills their slack
  // while the dK waves keep computing.
  constexpr int NCW = 4;
  using PC = PTileCopy<DP, NCW>;
  constexpr int NC = DP / KC, NDB = DP / 32;
  constexpr int FPB = M::FRAGS_PER_BLOCK;
  // copies per wave per query tile (Q, dO, lse2, delta)
  constexpr int LPT_HI = 2 * PC::CNT_HI + 2, LPT_LO = 2 * PC::CNT_LO + 2;
  static_assert(PT::ROWS == BQ, "tile / block mismatch");
  __shared__ __attribute__((aligned(16))) bf16 tiles[3][2][PT::ELEMS];
  __shared__ __attribute__((aligned(16))) float rowv[3][NCW][2][BQ];
  __shared__ uint8_t tcls[kMaxBwdTiles];

  const int vid = xcd_remap(blockIdx.x, p.B * p.H, p.nkt);
  const int bh = vid / p.nkt;
  const int kt = vid % p.nkt;
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool is_dk = wave >= 4;  // wave-uniform role
  const int g = lane >> 5, c32 = lane & 31;
  const int kblk0 = kt * BNK;
  const int kw0 = kblk0 + (wave & 3) * 32;
  const int key = kw0 + c32;
  const bool kok = key < p.Lk;
  const int kc = kok ? key : p.Lk - 1;

  const bf16* qp = (const bf16*)p.q + b * p.q_str[0] + h * p.q_str[1];
  const bf16* dop = (const bf16*)p.dout + b * p.o_str[0] + h * p.o_str[1];
  const float* lse2p = p.lse2 + ((int64_t)b * p.H + h) * p.Lq;
  const float* dltp = p.delta + ((int64_t)b * p.H + h) * p.Lq;
  const int64_t qs = p.q_str[2], os = p.o_str[2];

  // Query-tile classes (0 = nothing kept for this key block).
  const int nq = (p.Lq + BQ - 1) / BQ;
  const bool cls_lds = nq <= kMaxBwdTiles;
  auto tclass_g = [&](int t) -> int {
    const int q0 = t * BQ;
    if (CAUSAL && q0 + BQ - 1 < kblk0) return 0;
    if (!p.has_tilemap) return 3;
    return tile_class(p, b, h, q0, q0 + BQ, kblk0, kblk0 + BNK);
  };
  if (cls_lds)
    for (int t = tid; t < nq; t += NW * 64) tcls[t] = (uint8_t)tclass_g(t);
  __syncthreads();
  auto tclass = [&](int t) -> int { return cls_lds ? tcls[t] : tclass_g(t); };
  auto next_active = [&](int t) {
    while (t < nq && !(tclass(t) & 1)) ++t;
    return t;
  };

  // Stationary B operands: K (both roles), V (dK role) for this lane's key.
  Frag kf[NC], vf[NC];
  {
    const bf16* kp = (const bf16*)p.k + b * p.k_str[0] + h * p.k_str[1] +
                     (int64_t)kc * p.k_str[2];
    const bf16* vp = (const bf16*)p.v + b * p.v_str[0] + h * p.v_str[1] +
                     (int64_t)kc * p.v_str[2];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d = c * KC + g * EPC;
      const bool ok = kok && d < p.D;
      kf[c] = ok ? ld16(kp + d) : zero_frag<bf16>();
      vf[c] = (ok && is_dk) ? ld16(vp + d) : zero_frag<bf16>();
    }
  }
  f32x16 acc[NDB];  // dV^T (dV role) or dK^T (dK role)
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;
  float colsum = 0.f;

  // Bias: a per-key constant when it broadcasts over queries, else per row.
  const bool bias_rows = HAS_BIAS && p.bias_str[2] != 0;
  const int64_t bbase =
      HAS_BIAS ? b * p.bias_str[0] + h * p.bias_str[1] + kc : 0;
  const float bkey = (HAS_BIAS && !bias_rows) ? load_bias1(p, bbase) * kLog2e : 0.f;
  const uint8_t* mbase =
      p.has_mask ? p.mask + b * p.mask_str[0] + h * p.mask_str[1] + kc : nullptr;
  const int64_t dbbase = b * p.dbias_str[0] + h * p.dbias_str[1] + key;

  // Full dbias: entries of skipped tiles are zero.
  if constexpr (DBM == kDbFull) {
    if (is_dk && kok)
      for (int t = 0; t < nq; ++t)
        if (!(tclass(t) & 1))
          for (int i = 0; i < BQ && t * BQ + i < p.Lq; ++i)
            store_db(p, dbbase + (int64_t)(t * BQ + i) * p.dbias_str[2], 0.f);
  }
  // The stationary loads complete here, so no wait inside the tile loop has
  // to cover them (vmcnt there only tracks the tile copies).
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

  // Copies of query tile t into ring stage st (dV waves only).  Rows past Lq
  // are clamped to the last row and head-dim chunks past D to chunk 0 (finite
  // values that the keep-mask or the zero K / V columns cancel).
  auto issue = [&](int t, int st) {
    const int q0 = t * BQ;
    PC::issue(qp, qs, q0, p.Lq, p.D, &tiles[st][0][0], wave, lane);
    PC::issue(dop, os, q0, p.Lq, p.D, &tiles[st][1][0], wave, lane);
    const int q = min(q0 + lane, p.Lq - 1);
    dma4(lse2p + q, &rowv[st][wave][0][0]);
    dma4(dltp + q, &rowv[st][wave][1][0]);
  };
  // Waits until the tile issued before the most recent one is resident
  // (more = a later tile is still in flight) or until everything is.
  auto wait_tiles = [&](bool more) {
    if (!more)
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    else if (wave < PC::N_HI)
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(LPT_HI));
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(LPT_LO));
  };

  // The tile loop is instantiated per role (dV / dK): identical barrier
  // sequence, role-specific straight-line bodies.
  auto run = [&](auto role_tag) {
    constexpr bool DK = decltype(role_tag)::value;
    int cur = next_active(0);
    int nxt = cur < nq ? next_active(cur + 1) : nq;
    if constexpr (!DK) {
      if (cur < nq) issue(cur, 0);
      if (nxt < nq) issue(nxt, 1);
      wait_tiles(nxt < nq);
    }
    barrier_nofence();
    int st = 0;

    while (cur < nq) {
      const int nxt2 = nxt < nq ? next_active(nxt + 1) : nq;
      if constexpr (!DK)
        if (nxt2 < nq) issue(nxt2, st == 0 ? 2 : st - 1);

      const int cls = tclass(cur);
      const bf16* Qs = tiles[st][0];
      const bf16* Ds = tiles[st][1];
      const float* lse2s = rowv[st][wave & 3][0];
      const float* dlts = rowv[st][wave & 3][1];
      const int q0 = cur * BQ;
      const bool need_mask = p.has_mask && !(cls & 2);
      const bool tail = (q0 + BQ > p.Lq) || (kw0 + 32 > p.Lk);
      const bool diag = CAUSAL && (kw0 + 31 > q0);
      const bool general = need_mask || tail || diag || bias_rows;

      // One 32-query block; GEN selects the masked / per-row-bias body so the
      // interior-tile body is straight-line code.
      auto block = [&](int qb, auto gen_tag) {
        constexpr bool GEN = decltype(gen_tag)::value;
        // S = Q K^T (both roles); dP = dO V^T (dK role).
        f32x16 s, dp;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          s[r] = 0.f;
          dp[r] = 0.f;
        }
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const int off = PT::row_off(qb * 32 + c32, c * KC + g * EPC);
          M::run(s, ld16(&Qs[off]), kf[c]);
          if constexpr (DK) M::run(dp, ld16(&Ds[off]), vf[c]);
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int ql0 = qb * 32 + 8 * c + 4 * g;
          const f32x4 l4 = *reinterpret_cast<const f32x4*>(&lse2s[ql0]);
          f32x4 d4 = {0.f, 0.f, 0.f, 0.f};
          if constexpr (DK) d4 = *reinterpret_cast<const f32x4*>(&dlts[ql0]);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int r = 4 * c + j;
            float x = __builtin_fmaf(s[r], p.scale_log2, -l4[j]);
            if constexpr (HAS_BIAS) x += bkey;
            if constexpr (GEN) {
              const int q = q0 + ql0 + j;
              const int qcl = q < p.Lq ? q : p.Lq - 1;
              if constexpr (HAS_BIAS)
                if (bias_rows)
                  x = __builtin_fmaf(
                      load_bias1(p, bbase + (int64_t)qcl * p.bias_str[2]), kLog2e, x);
              bool keep = q < p.Lq && kok;
              if (need_mask) keep = keep && mbase[(int64_t)qcl * p.mask_str[2]] != 0;
              if (CAUSAL) keep = keep && key <= q;
              x = keep ? x : -INFINITY;
            }
            const float pr = fast_exp2(x);
            if constexpr (DK) {
              const float ds = pr * (dp[r] - d4[j]);
              s[r] = ds;
              if constexpr (DBM == kDbFull) {
                const int q = q0 + ql0 + j;
                if (kok && q < p.Lq)
                  store_db(p, dbbase + (int64_t)q * p.dbias_str[2], ds);
              }
              if constexpr (DBM == kDbColsum) colsum += ds;
            } else {
              s[r] = pr;
            }
          }
        }
        // dV^T += dO^T P (dV role) or dK^T += Q^T dS (dK role).
        const bf16* At = DK ? Qs : Ds;
#pragma unroll
        for (int f = 0; f < FPB; ++f) {
          const Frag pf = M::pack(s, f);
#pragma unroll
          for (int db = 0; db < NDB; ++db)
            M::run(acc[db], ptile_tr_frag<DP>(At, qb * 32, db * 32, lane, f), pf);
        }
      };
      // The scheduling barrier keeps block 1's loads from being hoisted into
      // block 0, which would exceed the two-waves-per-SIMD register budget.
      if (general) {
        block(0, std::true_type{});
        __builtin_amdgcn_sched_barrier(0);
        block(1, std::true_type{});
      } else {
        block(0, std::false_type{});
        __builtin_amdgcn_sched_barrier(0);
        block(1, std::false_type{});
      }

      // Tile nxt must be resident before the barrier; nxt2 may stay in flight.
      if constexpr (!DK) wait_tiles(nxt2 < nq);
      barrier_nofence();
      st = st == 2 ? 0 : st + 1;
      cur = nxt;
      nxt = nxt2;
    }
  };
  if (is_dk)
    run(std::true_type{});
  else
    run(std::false_type{});

  if (kok) {
    if (is_dk) {
      bf16* dkp = (bf16*)p.dk + b * p.k_str[0] + h * p.k_str[1] + (int64_t)key * p.k_str[2];
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int d0 = db * 32 + 8 * c + 4 * g;
          if (d0 < p.D) store4(dkp + d0, acc[db], 4 * c, p.scale);
        }
    } else {
      bf16* dvp = (bf16*)p.dv + b * p.v_str[0] + h * p.v_str[1] + (int64_t)key * p.v_str[2];
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int d0 = db * 32 + 8 * c + 4 * g;
          if (d0 < p.D) store4(dvp + d0, acc[db], 4 * c, 1.0f);
        }
    }
  }
  if constexpr (DBM == kDbColsum) {
    const float tot = colsum + shfl_xor32(colsum);
    if (is_dk && kok && g == 0) store_db(p, dbbase, tot);
  }
}

// ---------------------------------------------------------------------------
// dQ.  Block = 4 waves x 32 queries (128); streams 64-key tiles in two
// 32-key halves.  S^T = K Q^T and dP^T = V dO^T put the query on the lane's
// column, so dS^T feeds dQ^T = K^T dS^T from registers; K^T is read
// transposed from the row-major K tile.  K / V tiles arrive by direct
// global->LDS copies into a double-buffered ring (no staging registers), one
// tile ahead; two blocks share a CU.
// ---------------------------------------------------------------------------
template <int DP, bool HAS_BIAS, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void dq_bf16_kernel(const Params p) {
  using M = Mma<bf16>;
  using Frag = bf16x8;
  constexpr int EPC = 8, KC = 16;
  constexpr int BM = 128, BN = 64;
  constexpr int TSZ = BN * DP;         // swizzled, unpadded tile (elements)
  constexpr int NC = DP / KC, NDB = DP / 32;
  constexpr int FPB = M::FRAGS_PER_BLOCK;
  constexpr int CPRW = DP / 8;
  constexpr int RPB = 64 / CPRW;
  constexpr int BPW = TSZ / 512 / 4;
  __shared__ __attribute__((aligned(16))) bf16 tiles[2][2][TSZ];  // [stage][K|V]
  __shared__ uint8_t tcls[kMaxBwdTiles];

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
  const int qc = qok ? qrow : p.Lq - 1;

  const bf16* kp = (const bf16*)p.k + b * p.k_str[0] + h * p.k_str[1];
  const bf16* vp = (const bf16*)p.v + b * p.v_str[0] + h * p.v_str[1];
  const int64_t ks = p.k_str[2], vs = p.v_str[2];

  const int k_end = CAUSAL ? min(p.Lk, q0 + BM) : p.Lk;
  const int nkt = (k_end + BN - 1) / BN;
  const bool cls_lds = p.has_tilemap && nkt <= kMaxBwdTiles;
  if (cls_lds)
    for (int t = tid; t < nkt; t += 256)
      tcls[t] = (uint8_t)tile_class(p, b, h, q0, q0 + BM, t * BN, t * BN + BN);
  __syncthreads();
  auto tclass = [&](int t) -> int {
    if (!p.has_tilemap) return 3;
    if (cls_lds) return tcls[t];
    return tile_class(p, b, h, q0, q0 + BM, t * BN, t * BN + BN);
  };
  auto next_active = [&](int t) {
    while (t < nkt && !(tclass(t) & 1)) ++t;
    return t;
  };

  Frag qf[NC], df[NC];
  {
    const bf16* qp = (const bf16*)p.q + b * p.q_str[0] + h * p.q_str[1] +
                     (int64_t)qc * p.q_str[2];
    const bf16* dop = (const bf16*)p.dout + b * p.o_str[0] + h * p.o_str[1] +
                      (int64_t)qc * p.o_str[2];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d = c * KC + g * EPC;
      const bool ok = qok && d < p.D;
      qf[c] = ok ? ld16(qp + d) : zero_frag<bf16>();
      df[c] = ok ? ld16(dop + d) : zero_frag<bf16>();
    }
  }
  const int64_t rowid = ((int64_t)b * p.H + h) * p.Lq + qc;
  const float neg_lse2 = -p.lse2[rowid];
  const float dlt = p.delta[rowid];
  const int64_t brow = HAS_BIAS ? b * p.bias_str[0] + h * p.bias_str[1] +
                                      (int64_t)qc * p.bias_str[2]
                                : 0;
  const uint8_t* mrow = p.has_mask ? p.mask + b * p.mask_str[0] +
                                         h * p.mask_str[1] +
                                         (int64_t)qc * p.mask_str[2]
                                   : nullptr;
  // Stationary loads complete before the copies start (vmcnt in the loop
  // then only tracks tile copies).
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

  f32x16 dq[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[db][r] = 0.f;

  // Copies of key tile t into ring stage st (rows past Lk clamped to the last
  // key, head-dim chunks past D to chunk 0; both are masked or cancelled).
  auto issue = [&](int t, int st) {
    const int k0 = t * BN;
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
      const int blk = wave * BPW + i;
      const int row = blk * RPB + lane / CPRW;
      const int lc = (lane % CPRW) ^ swz<DP>(row);
      const int key = min(k0 + row, p.Lk - 1);
      const int col = lc * 8 < p.D ? lc * 8 : 0;
      dma16(kp + (int64_t)key * ks + col, &tiles[st][0][blk * 512]);
      dma16(vp + (int64_t)key * vs + col, &tiles[st][1][blk * 512]);
    }
  };

  int kt = next_active(0);
  if (kt < nkt) issue(kt, 0);
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  barrier_nofence();
  int st = 0;

  while (kt < nkt) {
    const int cls = tclass(kt);
    const int kn = next_active(kt + 1);
    if (kn < nkt) issue(kn, st ^ 1);

    const bf16* Ks = tiles[st][0];
    const bf16* Vs = tiles[st][1];
    const int k0 = kt * BN;
    const bool need_mask = p.has_mask && !(cls & 2);
    const bool tail = k0 + BN > p.Lk;
    const bool diag = CAUSAL && (k0 + BN - 1 > qw0);

    const bool general = HAS_BIAS || need_mask || tail || diag;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      f32x16 s, dpt;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[r] = 0.f;
        dpt[r] = 0.f;
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int off = swz_off<DP>(kb * 32 + c32, 2 * c + g);
        M::run(s, ld16(&Ks[off]), qf[c]);
        M::run(dpt, ld16(&Vs[off]), df[c]);
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int key0 = k0 + kb * 32 + 8 * c + 4 * g;
        f32x4 bv = {0.f, 0.f, 0.f, 0.f};
        uint32_t mw = 0x01010101u;
        if (general) {
          if constexpr (HAS_BIAS) bv = load_bias4(p, p.bias, brow + key0, p.Lk - key0);
          if (need_mask) mw = load_mask4(p, mrow + key0, p.Lk - key0);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 4 * c + j;
          float x = __builtin_fmaf(s[r], p.scale_log2, neg_lse2);
          if (general) {
            const int kk = key0 + j;
            if constexpr (HAS_BIAS) x = __builtin_fmaf(bv[j], kLog2e, x);
            bool keep = mask_bit(mw, j) && kk < p.Lk && qok;
            if (CAUSAL) keep = keep && kk <= qrow;
            x = keep ? x : -INFINITY;
          }
          const float pr = fast_exp2(x);
          dpt[r] = pr * (dpt[r] - dlt);
        }
      }
#pragma unroll
      for (int f = 0; f < FPB; ++f) {
        const Frag pd = M::pack(dpt, f);
#pragma unroll
        for (int db = 0; db < NDB; ++db)
          M::run(dq[db], lds_tr_frag_swz<DP>(Ks, kb * 32, db * 32, lane, f), pd);
      }
    }

    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // tile kn resident
    barrier_nofence();
    st ^= 1;
    kt = kn;
  }

  if (qok) {
    bf16* dqp = (bf16*)p.dq + b * p.q_str[0] + h * p.q_str[1] + (int64_t)qrow * p.q_str[2];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d0 = db * 32 + 8 * c + 4 * g;
        if (d0 < p.D) store4(dqp + d0, dq[db], 4 * c, p.scale);
      }
  }
}

// ---------------------------------------------------------------------------
// Launchers.
// ---------------------------------------------------------------------------
template <int DP, bool HB, bool CA, int DBM>
static void launch_dkdv_bf16_t(Params p, hipStream_t stream) {
  p.nkt = (p.Lk + 127) / 128;
  const int n = p.B * p.H * p.nkt;
  hipLaunchKernelGGL((dkdv_bf16_kernel<DP, HB, CA, DBM>), dim3(n), dim3(512), 0,
                     stream, p);
}

template <int DP, bool CA>
static void launch_dkdv_bf16_db(const Params& p, hipStream_t stream) {
  if (!p.has_bias) {
    launch_dkdv_bf16_t<DP, false, CA, kDbNone>(p, stream);
  } else if (p.dbias_mode == kDbiasFull) {
    launch_dkdv_bf16_t<DP, true, CA, kDbFull>(p, stream);
  } else if (p.dbias_mode == kDbiasColsum) {
    launch_dkdv_bf16_t<DP, true, CA, kDbColsum>(p, stream);
  } else {
    launch_dkdv_bf16_t<DP, true, CA, kDbNone>(p, stream);
  }
}

void launch_dkdv_bf16(const Params& p, int dp, hipStream_t stream) {
  if (dp == 64) {
    if (p.causal) launch_dkdv_bf16_db<64, true>(p, stream);
    else launch_dkdv_bf16_db<64, false>(p, stream);
  } else {
    if (p.causal) launch_dkdv_bf16_db<128, true>(p, stream);
    else launch_dkdv_bf16_db<128, false>(p, stream);
  }
}

template <int DP, bool HB, bool CA>
static void launch_dq_bf16_t(Params p, hipStream_t stream) {
  p.nqt = (p.Lq + 127) / 128;
  const int n = p.B * p.H * p.nqt;
  hipLaunchKernelGGL((dq_bf16_kernel<DP, HB, CA>), dim3(n), dim3(256), 0, stream, p);
}

template <int DP>
static void launch_dq_bf16_flags(const Params& p, hipStream_t stream) {
  if (p.has_bias) {
    if (p.causal) launch_dq_bf16_t<DP, true, true>(p, stream);
    else launch_dq_bf16_t<DP, true, false>(p, stream);
  } else {
    if (p.causal) launch_dq_bf16_t<DP, false, true>(p, stream);
    else launch_dq_bf16_t<DP, false, false>(p, stream);
  }
}

void launch_dq_bf16(const Params& p, int dp, hipStream_t stream) {
  if (dp == 64) launch_dq_bf16_flags<64>(p, stream);
  else launch_dq_bf16_flags<128>(p, stream);
}

}  // namespace nxa
