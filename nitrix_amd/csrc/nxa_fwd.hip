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
// Forward kernel.  Block = 4 waves x 32 queries; streams 64-key tiles.
// Each wave computes S^T = K Q^T so that a lane owns one query row: the row
// max / sum need one cross-lane exchange (lane l <-> l^32) and P feeds the
// P.V product straight from registers as its reduction operand.
// ---------------------------------------------------------------------------
template <typename T, int DP>
__global__ __launch_bounds__(256) void fwd_kernel(const Params p) {
  using M = Mma<T>;
  using Frag = typename M::Frag;
  constexpr int EPC = M::EPC, KC = M::KC;
  constexpr int BM = 128, BN = 64;
  constexpr int SK = DP + EPC;  // K tile row stride (elements)
  constexpr int ST = BN + 4;    // transposed V tile row stride
  constexpr int NC = DP / KC;
  constexpr int NDB = DP / 32;
  constexpr int CPR = DP / EPC;  // 16-byte chunks per row
  constexpr int FPB = M::FRAGS_PER_BLOCK;
  __shared__ __attribute__((aligned(16))) T Ks[BN * SK];
  __shared__ __attribute__((aligned(16))) T Vt[DP * ST];

  const int nblk = p.B * p.H * p.nqt;
  const int vid = xcd_remap(blockIdx.x, nblk);
  const int bh = vid / p.nqt;
  const int qt = p.nqt - 1 - (vid % p.nqt);  // longest (causal) tiles first
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

  Frag qf[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int d = c * KC + g * EPC;
    qf[c] = (qok && d < p.D) ? ld16(qp + (int64_t)qrow * p.q_str[2] + d)
                             : zero_frag<T>();
  }

  f32x16 oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[db][r] = 0.f;
  float m_i = -INFINITY, l_i = 0.f;

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
    if (!(cls & 1)) continue;  // every entry masked: skip the tile

    __syncthreads();  // previous tile's LDS reads are complete
    // K tile -> Ks (row-major); V tile -> Vt (transposed, key contiguous).
#pragma unroll
    for (int i = tid; i < BN * CPR; i += 256) {
      const int r = i / CPR, cc = i % CPR;
      const int key = k0 + r, d = cc * EPC;
      Frag x = zero_frag<T>();
      if (key < p.Lk && d < p.D) x = ld16(kp + (int64_t)key * p.k_str[2] + d);
      *reinterpret_cast<Frag*>(&Ks[r * SK + d]) = x;
    }
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int i = tid; i < (BN / 2) * CPR; i += 256) {
        const int rp = i / CPR, cc = i % CPR;
        const int key = k0 + 2 * rp, d = cc * EPC;
        Frag x0 = zero_frag<T>(), x1 = zero_frag<T>();
        if (d < p.D) {
          if (key < p.Lk) x0 = ld16(vp + (int64_t)key * p.v_str[2] + d);
          if (key + 1 < p.Lk)
            x1 = ld16(vp + (int64_t)(key + 1) * p.v_str[2] + d);
        }
#pragma unroll
        for (int j = 0; j < EPC; ++j) {
          bf16 pair[2] = {x0[j], x1[j]};
          *reinterpret_cast<uint32_t*>(&Vt[(d + j) * ST + 2 * rp]) =
              *reinterpret_cast<uint32_t*>(pair);
        }
      }
    } else {
#pragma unroll
      for (int i = tid; i < BN * CPR; i += 256) {
        const int r = i / CPR, cc = i % CPR;
        const int key = k0 + r, d = cc * EPC;
        Frag x = zero_frag<T>();
        if (key < p.Lk && d < p.D) x = ld16(vp + (int64_t)key * p.v_str[2] + d);
#pragma unroll
        for (int j = 0; j < EPC; ++j) Vt[(d + j) * ST + r] = x[j];
      }
    }
    __syncthreads();

    // S^T = K Q^T for 64 keys x 32 queries (two 32-key blocks).
    f32x16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kb][r] = 0.f;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const Frag a = ld16(&Ks[(kb * 32 + c32) * SK + c * KC + g * EPC]);
        M::run(s[kb], a, qf[c]);
      }
    }

    // Logits in base-2 units, bias, keep-mask, causal and key-tail masking.
    const bool need_mask = p.has_mask && !(cls & 2);
    const bool diag = p.causal && (k0 + BN - 1 > qw0);
    const bool tail = k0 + BN > p.Lk;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int key0 = k0 + kb * 32 + 8 * c + 4 * g;
        f32x4 bv = {0.f, 0.f, 0.f, 0.f};
        if (p.has_bias) bv = load_bias4(p, p.bias, brow + key0, p.Lk - key0);
        uint32_t mw = 0x01010101u;
        if (need_mask) mw = load_mask4(p, mrow + key0, p.Lk - key0);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int key = key0 + j;
          float x = s[kb][4 * c + j] * p.scale_log2;
          x = __builtin_fmaf(bv[j], kLog2e, x);
          bool keep = mask_bit(mw, j);
          if (tail) keep = keep && key < p.Lk;
          if (diag) keep = keep && key <= qrow;
          s[kb][4 * c + j] = keep ? x : -INFINITY;
        }
      }

    // Online softmax (row state is per query; lanes l and l^32 share it).
    float mt = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[kb][r]);
    mt = fmaxf(mt, shfl_xor32(mt));
    const float m_new = fmaxf(m_i, mt);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = fast_exp2(m_i - m_use);
    float rs = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float e = fast_exp2(s[kb][r] - m_use);
        s[kb][r] = e;
        rs += e;
      }
    l_i = l_i * alpha + rs;
    m_i = m_new;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;

    // O^T += V^T P^T.
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const T* row = &Vt[(db * 32 + c32) * ST];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int f = 0; f < FPB; ++f) {
          const Frag a = lds_frag_t<T>(row + kb * 32, g, f);
          M::run(oacc[db], a, M::pack(s[kb], f));
        }
    }
  }

  // Finalise: O = O / l (a fully masked row gives 0/0 = NaN, as the
  // reference's softmax over all -inf logits does), lse = ln sum exp.
  const float l = l_i + shfl_xor32(l_i);
  const float inv = 1.0f / l;
  T* op = (T*)p.o + b * p.o_str[0] + h * p.o_str[1] + (int64_t)qclamp * p.o_str[2];
  if (qok) {
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d0 = db * 32 + 8 * c + 4 * g;
        if (d0 < p.D) {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            op[d0 + j] = from_f32<T>(oacc[db][4 * c + j] * inv);
        }
      }
    if (g == 0 && p.lse)
      p.lse[((int64_t)b * p.H + h) * p.Lq + qrow] = (m_i + __log2f(l)) * kLn2;
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

template <typename T, int DP>
static void launch_fwd_t(Params p, hipStream_t stream) {
  p.nqt = (p.Lq + 127) / 128;
  const int n = p.B * p.H * p.nqt;
  hipLaunchKernelGGL((fwd_kernel<T, DP>), dim3(n), dim3(256), 0, stream, p);
}

void launch_fwd(const Params& p, int io_dtype, int dp, hipStream_t stream) {
  if (io_dtype == kBF16) {
    if (dp == 64) launch_fwd_t<bf16, 64>(p, stream);
    else launch_fwd_t<bf16, 128>(p, stream);
  } else {
    if (dp == 64) launch_fwd_t<float, 64>(p, stream);
    else launch_fwd_t<float, 128>(p, stream);
  }
}

}  // namespace nxa
