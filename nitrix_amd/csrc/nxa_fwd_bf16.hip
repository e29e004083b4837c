// bf16 forward kernel for gfx950: fused flash-attention forward with an
// online softmax in base 2 and an fp32 log-sum-exp per query row.
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
// K / V tiles (64 keys) travel from HBM straight into a 4-stage LDS ring by
// direct global->LDS copies, two tiles ahead of use; both tiles are
// row-permuted, padded P-tiles, conflict-free for the K row reads and the V
// transposed reads.  No staging registers, one barrier per tile.
//
// The two waves of a SIMD run half a tile apart: waves 0-3 compute
// S(t), softmax(t), O += P(t) V(t) between barriers t and t+1, while waves
// 4-7 compute softmax(t-1), O += P(t-1) V(t-1), S(t).  So while one wave of
// the pair runs its softmax (VALU, v_exp) the other keeps the matrix core
// busy.  The lagging waves still read V(t-1) after barrier t, which is why the
// ring holds four tiles: after barrier t the stage of tile t-2 is free and
// receives tile t+2.
#include "nxa_common.h"
#include "nxa_launch.h"

#include <type_traits>

namespace nxa {

constexpr int kFwdMaxTiles = 1024;       // key tiles listed in LDS per block
constexpr float kFwdRescaleSlack = 8.0f;  // lazy max raise threshold (log2)
// Instruction classes of __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedMfma = 0x008, kSchedDsRead = 0x100;

// max / sum over the two 32-lane halves (lanes l and l ^ 32).
__device__ __forceinline__ float half_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x),
                                                  __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

template <int DP, bool HAS_BIAS, bool CAUSAL>
__global__ __launch_bounds__(512, 1) void fwd_bf16_kernel(const Params p) {
  using M = Mma<bf16>;
  using Frag = bf16x8;
  constexpr int EPC = 8, KC = 16;
  constexpr int NW = 8, BM = NW * 32, BN = 64, NST = 4;
  using PT = PTile<DP>;
  using PS = PTileStream<DP, NW>;
  constexpr int NC = DP / KC, NDB = DP / 32, FPB = M::FRAGS_PER_BLOCK;
  static_assert(PT::ROWS == BN, "tile / block mismatch");
  __shared__ __attribute__((aligned(16))) bf16 tiles[NST][2][PT::ELEMS];
  __shared__ uint16_t act[kFwdMaxTiles];  // active key tiles, in order
  __shared__ uint8_t acls[kFwdMaxTiles];  // their classes
  __shared__ int nact_s;

  const int vid = xcd_remap(blockIdx.x, p.B * p.H, p.nqt);
  const int bh = vid / p.nqt;
  const int qt = p.nqt - 1 - (vid % p.nqt);  // longest (causal) tiles first
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform
  const int g = lane >> 5, c32 = lane & 31;
  const int q0 = qt * BM;
  const int qw0 = q0 + wave * 32;
  const int qrow = qw0 + c32;
  const bool qok = qrow < p.Lq;
  const int qc = qok ? qrow : p.Lq - 1;

  const bf16* kp = (const bf16*)p.k + b * p.k_str[0] + h * p.k_str[1];
  const bf16* vp = (const bf16*)p.v + b * p.v_str[0] + h * p.v_str[1];
  const int64_t ks = p.k_str[2], vs = p.v_str[2];

  // --- active key tiles of this block (tile-map classes) --------------------
  const int k_end = CAUSAL ? min(p.Lk, q0 + BM) : p.Lk;
  const int nkt = (k_end + BN - 1) / BN;
  const bool listed = nkt <= kFwdMaxTiles;
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
        act[pos] = (uint16_t)t;
        acls[pos] = (uint8_t)c;
      }
      base += __popcll(m);
    }
    if (lane == 0) nact_s = base;
  }
  __syncthreads();
  const int n = listed ? nact_s : nkt;
  // Contiguous active tiles (no mask, key padding, causal) need no lookup.
  const bool dense = !listed || n == 0 || act[n - 1] == n - 1;
  auto tile_of = [&](int i) NXA_INLINE -> int { return dense ? i : (int)act[i]; };
  auto class_of = [&](int i) NXA_INLINE -> int { return listed ? (int)acls[i] : class_g(i); };

  // --- stationary Q^T fragments ----------------------------------------------
  Frag qf[NC];
  {
    const bf16* qp = (const bf16*)p.q + b * p.q_str[0] + h * p.q_str[1] +
                     (int64_t)qrow * p.q_str[2];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d = c * KC + g * EPC;
      qf[c] = (qok && d < p.D) ? ld16(qp + d) : zero_frag<bf16>();
    }
  }
  const int64_t brow = HAS_BIAS ? b * p.bias_str[0] + h * p.bias_str[1] +
                                      (int64_t)qc * p.bias_str[2]
                                : 0;
  const uint8_t* mrow = p.has_mask ? p.mask + b * p.mask_str[0] +
                                         h * p.mask_str[1] +
                                         (int64_t)qc * p.mask_str[2]
                                   : nullptr;
  // The Q loads complete here, so the waits in the tile loop only count
  // tile copies.
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

  f32x16 oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[db][r] = 0.f;
  float m_ref = -INFINITY, l_i = 0.f;
  f32x16 s[2];

  // Copies of the i-th active tile into ring stage st.  Keys past Lk are
  // clamped to the last key (masked below) and head-dim chunks past D read
  // chunk 0 (multiplied by Q's zero columns, or landing in unstored O rows).
  // K copy j is issued by wave j % 8 and V copy j by wave (j + 4) % 8, so the
  // odd copy of each (17 per tile at D = 128) lands on different waves.
  PS ksm, vsm;
  ksm.init(ks, p.D, wave, 0, lane);
  vsm.init(vs, p.D, wave, NW / 2, lane);
  const int my_copies = ksm.count() + vsm.count();  // wave-uniform
  const uint32_t lds0 = lds_offset(&tiles[0][0][0]);
  constexpr uint32_t kTileBytes = PT::ELEMS * 2;
  auto issue = [&](int i, int st) NXA_INLINE {
    const int k0 = tile_of(i) * BN;
    const uint32_t at = lds0 + st * 2 * kTileBytes;
    ksm.issue(kp, ks, k0, p.Lk, at);
    vsm.issue(vp, vs, k0, p.Lk, at + kTileBytes);
  };
  // Waits for this wave's copies of the oldest tile in flight (more = a
  // later tile is in flight too).
  auto wait_tile = [&](bool more) NXA_INLINE {
    if (!more)
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    else if (my_copies == 2 * PS::CNT)
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * PS::CNT));
    else if (my_copies == 2 * PS::CNT - 1)
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * PS::CNT - 1));
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * PS::CNT - 2));
  };
  // A tile holds nothing for this wave when all its keys are past the
  // wave's last query (causal) or the wave has no query rows.
  auto skip = [&](int i) NXA_INLINE -> bool {
    if (qw0 >= p.Lq) return true;
    return CAUSAL && tile_of(i) * BN > qw0 + 31;
  };

  // S^T = K Q^T for the tile in stage st: 64 keys (two 32-key blocks).
  // The K fragments are read PD products ahead of their use (a rotating
  // register buffer) to cover the LDS latency.
  constexpr int PD = 4;
  auto qk = [&](int st) NXA_INLINE {
    const bf16* Ks = tiles[st][0];
    auto kfrag = [&](int j) NXA_INLINE {
      return ld16(&Ks[PT::row_off((j & 1) * 32 + c32, (j >> 1) * KC + g * EPC)]);
    };
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kb][r] = 0.f;
    Frag kbuf[PD];
#pragma unroll
    for (int j = 0; j < PD; ++j) kbuf[j] = kfrag(j);
#pragma unroll
    for (int j = 0; j < 2 * NC; ++j) {
      M::run(s[j & 1], kbuf[j % PD], qf[j >> 1]);
      if (j + PD < 2 * NC) kbuf[j % PD] = kfrag(j + PD);
    }
    // Keep that order: PD reads, then one product and one read at a time.
#pragma unroll
    for (int j = 0; j < PD; ++j) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
#pragma unroll
    for (int j = 0; j < 2 * NC; ++j) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      if (j + PD < 2 * NC) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
    }
  };

  // Softmax of the i-th active tile (scores in s) and O^T += V^T P^T.
  auto sm_pv = [&](int i, int st) NXA_INLINE {
    const int k0 = tile_of(i) * BN;
    const int cls = class_of(i);
    const bool need_mask = p.has_mask && !(cls & 2);
    const bool tail = k0 + BN > p.Lk;
    const bool diag = CAUSAL && (k0 + BN - 1 > qw0);
    const bool general = HAS_BIAS || need_mask || tail || diag || !(p.scale_log2 > 0.f);
    // Fast path (nothing masked, no bias): the scale is folded into the
    // exponent's FMA and the max is taken on raw scores.
    float cc = p.scale_log2;
    if (general) {
      cc = 1.0f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int key0 = k0 + kb * 32 + 8 * c + 4 * g;
          f32x4 bv = {0.f, 0.f, 0.f, 0.f};
          if constexpr (HAS_BIAS) bv = load_bias4(p, p.bias, brow + key0, p.Lk - key0);
          uint32_t mw = 0x01010101u;
          if (need_mask) mw = load_mask4(p, mrow + key0, p.Lk - key0);
          // Every element is written exactly once, unconditionally: masked
          // entries are a select, never a divergent partial write.
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int key = key0 + j;
            float x = s[kb][4 * c + j] * p.scale_log2;
            if constexpr (HAS_BIAS) x = __builtin_fmaf(bv[j], kLog2e, x);
            bool keep = mask_bit(mw, j) && key < p.Lk;
            if (CAUSAL) keep = keep && key <= qrow;
            s[kb][4 * c + j] = keep ? x : -INFINITY;
          }
        }
    }

    // Online softmax against a lazily raised reference max.
    float mt = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[kb][r]);
    mt = half_max(mt) * cc;
    const bool raise = mt > m_ref + kFwdRescaleSlack;
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
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float e = fast_exp2(__builtin_fmaf(s[kb][r], cc, neg_m));
        s[kb][r] = e;
        rs += e;
      }
    l_i += rs;

    const bf16* Vs = tiles[st][1];
    // Product j: key block kb = j / (FPB NDB), fragment f, head-dim block db.
    constexpr int NPV = 2 * FPB * NDB;
    auto vfrag = [&](int j) NXA_INLINE {
      return ptile_tr_frag<DP>(Vs, (j / (FPB * NDB)) * 32, (j % NDB) * 32, lane,
                               (j / NDB) % FPB);
    };
    Frag vbuf[PD];
#pragma unroll
    for (int j = 0; j < PD; ++j) vbuf[j] = vfrag(j);
    Frag pf;
#pragma unroll
    for (int j = 0; j < NPV; ++j) {
      if (j % NDB == 0) pf = M::pack(s[j / (FPB * NDB)], (j / NDB) % FPB);
      M::run(oacc[j % NDB], vbuf[j % PD], pf);
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

  auto run = [&](auto lag_tag) {
    constexpr bool LAG = decltype(lag_tag)::value;
    if (n > 0) issue(0, 0);
    if (n > 1) issue(1, 1);
    for (int i = 0; i < n; ++i) {
      wait_tile(i + 1 < n);
      barrier_nofence();
      if (i + 2 < n) issue(i + 2, (i + 2) % NST);
      const int st = i % NST;
      if constexpr (LAG) {
        if (i > 0 && !skip(i - 1)) sm_pv(i - 1, (i + NST - 1) % NST);
        __builtin_amdgcn_sched_barrier(0);
        if (!skip(i)) qk(st);
      } else {
        if (!skip(i)) {
          qk(st);
          sm_pv(i, st);
        }
      }
    }
    if constexpr (LAG)
      if (n > 0 && !skip(n - 1)) sm_pv(n - 1, (n - 1) % NST);
  };
  if (wave >= NW / 2)
    run(std::true_type{});
  else
    run(std::false_type{});

  // Finalise: O = O / l (a fully masked row gives 0/0 = NaN, as the
  // reference's softmax over all -inf logits does), lse = ln sum exp.
  const float l = l_i + shfl_xor32(l_i);
  const float inv = 1.0f / l;
  if (qok) {
    bf16* op = (bf16*)p.o + b * p.o_str[0] + h * p.o_str[1] + (int64_t)qrow * p.o_str[2];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d0 = db * 32 + 8 * c + 4 * g;
        if (d0 < p.D) store4(op + d0, oacc[db], 4 * c, inv);
      }
    if (g == 0 && p.lse)
      p.lse[((int64_t)b * p.H + h) * p.Lq + qrow] = (m_ref + __log2f(l)) * kLn2;
  }
}

template <int DP, bool HB, bool CA>
static void launch_fwd_bf16_t(Params p, hipStream_t stream) {
  constexpr int BM = 256;
  p.nqt = (p.Lq + BM - 1) / BM;
  const int n = p.B * p.H * p.nqt;
  hipLaunchKernelGGL((fwd_bf16_kernel<DP, HB, CA>), dim3(n), dim3(512), 0, stream, p);
}

template <int DP>
static void launch_fwd_bf16_flags(const Params& p, hipStream_t stream) {
  if (p.has_bias) {
    if (p.causal) launch_fwd_bf16_t<DP, true, true>(p, stream);
    else launch_fwd_bf16_t<DP, true, false>(p, stream);
  } else {
    if (p.causal) launch_fwd_bf16_t<DP, false, true>(p, stream);
    else launch_fwd_bf16_t<DP, false, false>(p, stream);
  }
}

void launch_fwd_bf16(const Params& p, int dp, hipStream_t stream) {
  if (dp == 64) launch_fwd_bf16_flags<64>(p, stream);
  else launch_fwd_bf16_flags<128>(p, stream);
}

}  // namespace nxa
