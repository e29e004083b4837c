// Forward pass: tile-map pre-pass over the keep-mask and the fused
// flash-attention forward kernel (online softmax in base 2, fp32 LSE).
//
// Replaces the reference's `nitrix_mha_forward` Pallas launch and its XLA
// glue: src/nitrix/_kernels/cuda/attention.py:85-156 (kernel body),
// :159-264 (launch), :547-584 (broadcast / layout adapter, which this
// library replaces with zero-stride descriptors instead of copies).
#include "nxa_common.h"
#include "nxa_launch.h"

namespace nxa {

// ---------------------------------------------------------------------------
// Tile map.  One block per 64x64 tile of the mask's own (un-broadcast)
// extent; writes bit0 = some entry kept, bit1 = every in-range entry kept.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void tilemap_kernel(const Params p, int MB,
                                                      int MH, int MQ, int MK,
                                                      int vec16) {
  int id = blockIdx.x;
  const int mk = id % MK;
  id /= MK;
  const int mq = id % MQ;
  id /= MQ;
  const int mh = id % MH;
  const int mb = id / MH;
  const int t = threadIdx.x;
  const int r = t >> 2, seg = t & 3;
  const int r0 = mq * kTile, c0 = mk * kTile;
  const int nrows = min(kTile, p.tm_rows - r0);
  const int ncols = min(kTile, p.Lk - c0);
  int any = 0, all = 1;
  if (r < nrows) {
    const uint8_t* m = p.mask + mb * p.mask_str[0] + mh * p.mask_str[1] +
                       (int64_t)(r0 + r) * p.mask_str[2] + c0 + 16 * seg;
    const int nc = ncols - 16 * seg;
    if (vec16 && nc >= 16) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(m);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t x = w[i];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int on = ((x >> (8 * j)) & 0xffu) != 0;
          any |= on;
          all &= on;
        }
      }
    } else {
      for (int j = 0; j < 16; ++j)
        if (j < nc) {
          const int on = m[j] != 0;
          any |= on;
          all &= on;
        }
    }
  }
  any = __syncthreads_or(any);
  all = __syncthreads_and(all);
  if (t == 0) p.tilemap_out[blockIdx.x] = (uint8_t)(any | (all << 1));
}

// ---------------------------------------------------------------------------
// Forward kernel.  Block = 4 waves, each owning QB blocks of 32 queries;
// streams 64-key tiles through double-buffered LDS (the next tile is fetched
// into registers while the current one is consumed).
//
// Each wave computes S^T = K Q^T so that a lane owns one query row: the row
// max / sum need one cross-lane exchange (lane l <-> l^32) and P feeds the
// P.V product straight from registers as its reduction operand.  Every K and
// V fragment read from LDS is used by QB MFMAs.
//
// The running max is only raised when a row's new maximum exceeds it by more
// than kRescaleSlack (in log2 units): P is then bounded by 2^kRescaleSlack and
// the O / l rescale, a full pass over the accumulators, becomes rare.  The
// result is exact: O and l are accumulated against the same reference max.
// ---------------------------------------------------------------------------
constexpr float kRescaleSlack = 8.0f;

template <typename T, int DP, int QB, bool HAS_BIAS, bool CAUSAL>
__global__ __launch_bounds__(256) void fwd_kernel(const Params p) {
  using M = Mma<T>;
  using Frag = typename M::Frag;
  constexpr int EPC = M::EPC, KC = M::KC;
  constexpr int BM = 128 * QB, BN = 64;
  constexpr int SK = DP + EPC;  // K tile row stride (elements)
  constexpr int ST = BN + 4;    // transposed V tile row stride
  constexpr int NC = DP / KC;
  constexpr int NDB = DP / 32;
  constexpr int CPR = DP / EPC;  // 16-byte chunks per row
  constexpr int FPB = M::FRAGS_PER_BLOCK;
  constexpr int KSZ = BN * SK, VSZ = DP * ST;
  constexpr int NCH = BN * CPR / 256;  // 16-byte chunks per thread per tile
  static_assert(NCH >= 2 && NCH % 2 == 0, "tile / block mismatch");
  __shared__ __attribute__((aligned(16))) T smem[2 * (KSZ + VSZ)];

  const int nblk = p.B * p.H * p.nqt;
  const int vid = xcd_remap(blockIdx.x, nblk);
  const int bh = vid / p.nqt;
  const int qt = p.nqt - 1 - (vid % p.nqt);  // longest (causal) tiles first
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, c32 = lane & 31;
  const int q0 = qt * BM;
  const int qw0 = q0 + wave * 32 * QB;

  const T* qp = (const T*)p.q + b * p.q_str[0] + h * p.q_str[1];
  const T* kp = (const T*)p.k + b * p.k_str[0] + h * p.k_str[1];
  const T* vp = (const T*)p.v + b * p.v_str[0] + h * p.v_str[1];
  const int64_t ks = p.k_str[2], vs = p.v_str[2];

  Frag qf[QB][NC];
  int qrow[QB];
  int64_t brow[QB];
  const uint8_t* mrow[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    qrow[qb] = qw0 + qb * 32 + c32;
    const bool qok = qrow[qb] < p.Lq;
    const int qc = qok ? qrow[qb] : p.Lq - 1;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d = c * KC + g * EPC;
      qf[qb][c] = (qok && d < p.D) ? ld16(qp + (int64_t)qrow[qb] * p.q_str[2] + d)
                                   : zero_frag<T>();
    }
    brow[qb] = HAS_BIAS ? b * p.bias_str[0] + h * p.bias_str[1] +
                              (int64_t)qc * p.bias_str[2]
                        : 0;
    mrow[qb] = p.has_mask ? p.mask + b * p.mask_str[0] + h * p.mask_str[1] +
                                (int64_t)qc * p.mask_str[2]
                          : nullptr;
  }

  f32x16 oacc[QB][NDB];
  float m_ref[QB], l_i[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m_ref[qb] = -INFINITY;
    l_i[qb] = 0.f;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[qb][db][r] = 0.f;
  }

  // --- K / V tile staging (global -> registers -> LDS) ----------------------
  Frag kst[NCH], vst[NCH];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int idx = tid + i * 256;
      const int r = idx / CPR, d = (idx % CPR) * EPC;
      const int key = k0 + r;
      kst[i] = (key < p.Lk && d < p.D) ? ld16(kp + (int64_t)key * ks + d)
                                       : zero_frag<T>();
    }
    if constexpr (sizeof(T) == 2) {
      // V in row pairs so the transposed LDS writes are 32-bit.
#pragma unroll
      for (int i = 0; i < NCH / 2; ++i) {
        const int idx = tid + i * 256;
        const int rp = idx / CPR, d = (idx % CPR) * EPC;
        const int key = k0 + 2 * rp;
        vst[2 * i] = (key < p.Lk && d < p.D) ? ld16(vp + (int64_t)key * vs + d)
                                             : zero_frag<T>();
        vst[2 * i + 1] = (key + 1 < p.Lk && d < p.D)
                             ? ld16(vp + (int64_t)(key + 1) * vs + d)
                             : zero_frag<T>();
      }
    } else {
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        const int idx = tid + i * 256;
        const int r = idx / CPR, d = (idx % CPR) * EPC;
        const int key = k0 + r;
        vst[i] = (key < p.Lk && d < p.D) ? ld16(vp + (int64_t)key * vs + d)
                                         : zero_frag<T>();
      }
    }
  };
  auto lstore = [&](int buf) {
    T* Ks = smem + buf * (KSZ + VSZ);
    T* Vt = Ks + KSZ;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int idx = tid + i * 256;
      const int r = idx / CPR, d = (idx % CPR) * EPC;
      *reinterpret_cast<Frag*>(&Ks[r * SK + d]) = kst[i];
    }
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int i = 0; i < NCH / 2; ++i) {
        const int idx = tid + i * 256;
        const int rp = idx / CPR, d = (idx % CPR) * EPC;
#pragma unroll
        for (int j = 0; j < EPC; ++j) {
          bf16 pair[2] = {vst[2 * i][j], vst[2 * i + 1][j]};
          *reinterpret_cast<uint32_t*>(&Vt[(d + j) * ST + 2 * rp]) =
              *reinterpret_cast<uint32_t*>(pair);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        const int idx = tid + i * 256;
        const int r = idx / CPR, d = (idx % CPR) * EPC;
#pragma unroll
        for (int j = 0; j < EPC; ++j) Vt[(d + j) * ST + r] = vst[i][j];
      }
    }
  };

  // --- key-tile schedule ------------------------------------------------------
  const int k_end = CAUSAL ? min(p.Lk, q0 + BM) : p.Lk;
  const int nkt = (k_end + BN - 1) / BN;
  auto tclass = [&](int kt) {
    return p.has_tilemap ? tile_class(p, b, h, q0, q0 + BM, kt * BN, kt * BN + BN)
                         : 3;
  };
  int kt = 0, cls = 0;
  for (; kt < nkt; ++kt) {
    cls = tclass(kt);
    if (cls & 1) break;
  }
  if (kt < nkt) {
    gload(kt * BN);
    lstore(0);
  }
  __syncthreads();
  int buf = 0;

  while (kt < nkt) {
    int kn = kt + 1, ncls = 0;
    for (; kn < nkt; ++kn) {
      ncls = tclass(kn);
      if (ncls & 1) break;
    }
    if (kn < nkt) gload(kn * BN);  // in flight while this tile is consumed

    const T* Ks = smem + buf * (KSZ + VSZ);
    const T* Vt = Ks + KSZ;
    const int k0 = kt * BN;

    const bool need_mask = p.has_mask && !(cls & 2);
    const bool tail = k0 + BN > p.Lk;
    const bool diag = CAUSAL && (k0 + BN - 1 > qw0);
    const bool edge = need_mask || tail || diag;

    // The tile is consumed in two 32-key halves: S, P live per half only.
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      // S^T = K Q^T: 32 keys x 32 queries per qb; K fragments shared by qb.
      f32x16 s[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[qb][r] = 0.f;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const Frag a = ld16(&Ks[(kb * 32 + c32) * SK + c * KC + g * EPC]);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) M::run(s[qb], a, qf[qb][c]);
      }

      typename M::Frag pk[QB][FPB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        // Logits in base-2 units (+ bias), then keep-mask / key tail / causal.
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int key0 = k0 + kb * 32 + 8 * c + 4 * g;
          f32x4 bv = {0.f, 0.f, 0.f, 0.f};
          if constexpr (HAS_BIAS)
            bv = load_bias4(p, p.bias, brow[qb] + key0, p.Lk - key0);
          // Masked entries are a select, and every element is written exactly
          // once, unconditionally (no divergent partial writes into the
          // accumulator vector).
          uint32_t mw = 0x01010101u;
          if (need_mask) mw = load_mask4(p, mrow[qb] + key0, p.Lk - key0);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float x = s[qb][4 * c + j] * p.scale_log2;
            if constexpr (HAS_BIAS) x = __builtin_fmaf(bv[j], kLog2e, x);
            if (edge) {
              const int key = key0 + j;
              bool keep = mask_bit(mw, j) && key < p.Lk;
              if (CAUSAL) keep = keep && key <= qrow[qb];
              x = keep ? x : -INFINITY;
            }
            s[qb][4 * c + j] = x;
          }
        }

        // Online softmax with a lazily raised reference max.
        float mt = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[qb][r]);
        mt = fmaxf(mt, shfl_xor32(mt));
        const bool raise = mt > m_ref[qb] + kRescaleSlack;
        if (__any(raise)) {
          const float alpha = raise ? fast_exp2(m_ref[qb] - mt) : 1.f;
          m_ref[qb] = raise ? mt : m_ref[qb];
          l_i[qb] *= alpha;
#pragma unroll
          for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) oacc[qb][db][r] *= alpha;
        }
        const float m_use = (m_ref[qb] == -INFINITY) ? 0.f : m_ref[qb];
        float rs = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float e = fast_exp2(s[qb][r] - m_use);
          s[qb][r] = e;
          rs += e;
        }
        l_i[qb] += rs;
#pragma unroll
        for (int f = 0; f < FPB; ++f) pk[qb][f] = M::pack(s[qb], f);
      }

      // O^T += V^T P^T over these 32 keys; each V fragment feeds QB MFMAs.
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const T* row = &Vt[(db * 32 + c32) * ST + kb * 32];
#pragma unroll
        for (int f = 0; f < FPB; ++f) {
          const Frag a = lds_frag_t<T>(row, g, f);
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) M::run(oacc[qb][db], a, pk[qb][f]);
        }
      }
    }

    if (kn < nkt) lstore(buf ^ 1);
    __syncthreads();
    buf ^= 1;
    kt = kn;
    cls = ncls;
  }

  // Finalise: O = O / l (a fully masked row gives 0/0 = NaN, as the
  // reference's softmax over all -inf logits does), lse = ln sum exp.
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const float l = l_i[qb] + shfl_xor32(l_i[qb]);
    const float inv = 1.0f / l;
    if (qrow[qb] < p.Lq) {
      T* op = (T*)p.o + b * p.o_str[0] + h * p.o_str[1] +
              (int64_t)qrow[qb] * p.o_str[2];
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int d0 = db * 32 + 8 * c + 4 * g;
          if (d0 < p.D) store4(op + d0, oacc[qb][db], 4 * c, inv);
        }
      if (g == 0 && p.lse)
        p.lse[((int64_t)b * p.H + h) * p.Lq + qrow[qb]] =
            (m_ref[qb] + __log2f(l)) * kLn2;
    }
  }
}

// ---------------------------------------------------------------------------
// Host launchers.
// ---------------------------------------------------------------------------
void launch_tilemap(const Params& p, int MB, int MH, int MQ, int MK, int vec16,
                    hipStream_t stream) {
  const int n = MB * MH * MQ * MK;
  hipLaunchKernelGGL(tilemap_kernel, dim3(n), dim3(256), 0, stream, p, MB, MH,
                     MQ, MK, vec16);
}

template <typename T, int DP, int QB, bool HB, bool CA>
static void launch_fwd_t(Params p, hipStream_t stream) {
  constexpr int BM = 128 * QB;
  p.nqt = (p.Lq + BM - 1) / BM;
  const int n = p.B * p.H * p.nqt;
  hipLaunchKernelGGL((fwd_kernel<T, DP, QB, HB, CA>), dim3(n), dim3(256), 0,
                     stream, p);
}

template <typename T, int DP, int QB>
static void launch_fwd_flags(const Params& p, hipStream_t stream) {
  if (p.has_bias) {
    if (p.causal) launch_fwd_t<T, DP, QB, true, true>(p, stream);
    else launch_fwd_t<T, DP, QB, true, false>(p, stream);
  } else {
    if (p.causal) launch_fwd_t<T, DP, QB, false, true>(p, stream);
    else launch_fwd_t<T, DP, QB, false, false>(p, stream);
  }
}

void launch_fwd(const Params& p, int io_dtype, int dp, hipStream_t stream) {
  if (io_dtype == kBF16) {
    if (dp == 64) launch_fwd_flags<bf16, 64, 2>(p, stream);
    else launch_fwd_flags<bf16, 128, 2>(p, stream);
  } else {
    if (dp == 64) launch_fwd_flags<float, 64, 1>(p, stream);
    else launch_fwd_flags<float, 128, 1>(p, stream);
  }
}

}  // namespace nxa
