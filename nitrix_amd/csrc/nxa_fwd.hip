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
// Tile map.  One wave per pair of horizontally adjacent 64x64 tiles of the
// mask's own (un-broadcast) extent, so every row read is one whole 128-byte
// line: lane l reads 16 bytes (column chunk l % 8) of rows l / 8 + 8 k.
// Writes bit0 = some entry kept, bit1 = every in-range entry kept; wave
// ballots do the reductions (no block barriers).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void tilemap_kernel(const Params p, int MB,
                                                      int MH, int MQ, int MK,
                                                      int vec16) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int MK2 = (MK + 1) / 2;  // tile pairs per tile row
  const int64_t pair = (int64_t)blockIdx.x * 4 + wave;
  if (pair >= (int64_t)MB * MH * MQ * MK2) return;  // wave-uniform
  int64_t id = pair;
  const int mk2 = (int)(id % MK2);
  id /= MK2;
  const int mq = (int)(id % MQ);
  id /= MQ;
  const int mh = (int)(id % MH);
  const int mb = (int)(id / MH);
  const int r0 = mq * kTile, c0 = mk2 * 2 * kTile;
  const int nrows = min(kTile, p.tm_rows - r0);
  const int sub = lane & 7, rr = lane >> 3;
  const int nc = min(2 * kTile, p.Lk - c0) - 16 * sub;  // in-range bytes of the chunk
  const uint8_t* m0 = p.mask + mb * p.mask_str[0] + mh * p.mask_str[1] +
                      (int64_t)r0 * p.mask_str[2] + c0 + 16 * sub;
  bool any = false, all = true;
  if (nc > 0) {
#pragma unroll
    for (int k = 0; k < kTile / 8; ++k) {
      const int r = 8 * k + rr;
      if (r < nrows) {
        const uint8_t* m = m0 + (int64_t)r * p.mask_str[2];
        if (vec16 && nc >= 16) {
          // (read once: non-temporal)
          const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(m));
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t x = w[i];
            // x has a zero byte iff (x - 0x01010101) & ~x & 0x80808080 != 0.
            any = any || x != 0;
            all = all && ((x - 0x01010101u) & ~x & 0x80808080u) == 0;
          }
        } else {
          for (int j = 0; j < 16 && j < nc; ++j) {
            const bool on = m[j] != 0;
            any = any || on;
            all = all && on;
          }
        }
      }
    }
  }
  const uint64_t anyb = __ballot(any), offb = __ballot(!all);
  constexpr uint64_t kLeft = 0x0f0f0f0f0f0f0f0full;  // lanes with sub < 4
  if (lane == 0) {
    const int64_t t = (((int64_t)mb * MH + mh) * MQ + mq) * MK + 2 * mk2;
    p.tilemap_out[t] = (uint8_t)(((anyb & kLeft) != 0) | (((offb & kLeft) == 0) << 1));
    if (2 * mk2 + 1 < MK)
      p.tilemap_out[t + 1] =
          (uint8_t)(((anyb & ~kLeft) != 0) | (((offb & ~kLeft) == 0) << 1));
  }
}

// ---------------------------------------------------------------------------
// Block order.  The hardware hands out blocks in index order, each CU taking
// the next one when it is free; when a mask that varies over queries gives
// the blocks of one head unequal work, the grid ends on whichever blocks
// come last.  Sorting each head's blocks by their work, most first (the
// longest-processing-time rule), lets the short ones fill the end.  One
// workgroup per tile-map slice:
//  1. work per block, in map tiles: a 128-row block (two map rows) runs one
//     key tile for every map column either row keeps, a 256-row block (four
//     rows) likewise, a 128-key block (two map columns) one query tile for
//     every map row that keeps either column.  Each thread keeps one
//     16-column chunk and walks row groups of four map rows, loading four
//     groups at a time; a map row stays four words with bit 0 of each byte
//     (popcounts of ORs give the row counts, packed 16-bit adds the column
//     counts).  Row counts are summed over the lanes that share the rows (a
//     segmented shuffle sum, then one LDS add per segment); column counts
//     stay in registers until one LDS add per column pair.
//  2. position of block i = #{j : c_j > c_i} + #{j < i : c_j = c_i}, a
//     permutation (ties keep index order): with key_i = c_i * 2048 +
//     (2047 - i) it is #{j : key_j > key_i}.  The three lists are ranked at
//     once, one thread per block, keys read four at a time (entries past a
//     list's end hold -1, below every key).
// Output per slice: [128-row blocks | 256-row blocks | 128-key blocks].
// ---------------------------------------------------------------------------
__device__ __forceinline__ int rank_of(const int* key, int n, int i) {
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  const int ki = key[i];
  int r = 0;
#pragma unroll 8
  for (int j = 0; j < n; j += 4) {
    const i32x4 v = *reinterpret_cast<const i32x4*>(key + j);
#pragma unroll
    for (int e = 0; e < 4; ++e) r += v[e] > ki;
  }
  return r;
}

__global__ __launch_bounds__(1024) void tile_order_kernel(const uint8_t* tm, int MQ, int MK,
                                                          int vec16, int* order) {
  __shared__ __attribute__((aligned(16))) int cq2[kOrderMax];
  __shared__ __attribute__((aligned(16))) int cq4[kOrderMax / 2];
  __shared__ __attribute__((aligned(16))) int ck2[kOrderMax];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nq2 = (MQ + 1) >> 1, nq4 = (MQ + 3) >> 2, nk2 = (MK + 1) >> 1;
  for (int i = tid; i < kOrderMax; i += 1024) {
    cq2[i] = i < nq2 ? 0 : -1;
    ck2[i] = i < nk2 ? 0 : -1;
    if (i < kOrderMax / 2) cq4[i] = i < nq4 ? 0 : -1;
  }
  __syncthreads();
  const uint8_t* s = tm + (int64_t)blockIdx.x * MQ * MK;
  // Thread t keeps 16-column chunk c = t % nch and walks the row groups
  // (four map rows) r0, r0 + tr, ...; lanes of one row group are contiguous.
  const int nch = (MK + 15) >> 4;  // at most 128 (nk2 <= kOrderMax)
  const int tr = 1024 / nch;
  const int c = tid % nch, r0 = tid / nch;
  const bool live = r0 < tr;
  const int iters = (nq4 + tr - 1) / tr;  // uniform
  // Row `row` of the chunk as four words, bit 0 of byte j = map column
  // 16c + j keeps something (the other bits cleared).
  auto row_words = [&](int row) -> u32x4 {
    const uint8_t* m = s + (int64_t)row * MK + 16 * c;
    u32x4 w = {0u, 0u, 0u, 0u};
    if (vec16) {
      w = *reinterpret_cast<const u32x4*>(m);
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if (16 * c + j < MK) w[j >> 2] |= (uint32_t)m[j] << (8 * (j & 3));
    }
    return w & 0x01010101u;
  };
  // Column-pair counts, two per word: pair 8c + 2i in the low half of
  // colacc[i], pair 8c + 2i + 1 in the high half (at most MQ each).
  uint32_t colacc[4] = {0u, 0u, 0u, 0u};
  constexpr int U = 4;  // row groups whose loads are issued together
  for (int k0 = 0; k0 < iters; k0 += U) {
    u32x4 x[U][4];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int g = r0 + (k0 + u) * tr;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        x[u][r] = u32x4{0u, 0u, 0u, 0u};
        if (live && k0 + u < iters && g < nq4 && 4 * g + r < MQ) x[u][r] = row_words(4 * g + r);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (k0 + u >= iters) break;  // uniform
      const int gv = r0 + (k0 + u) * tr;
      const bool ok = live && gv < nq4;
      const int g = ok ? gv : nq4 + r0;  // idle lanes: row groups past the end
      const u32x4 a01 = x[u][0] | x[u][1], a23 = x[u][2] | x[u][3], a4 = a01 | a23;
      int w01 = 0, w23 = 0, w4 = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        w01 += __popc(a01[i]);
        w23 += __popc(a23[i]);
        w4 += __popc(a4[i]);
      }
      // Segmented sums: after the doubling steps a lane holds the sum from
      // itself to the end of its row group's lanes in this wave.
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int gd = __shfl_down(g, d);
        const int a = __shfl_down(w01, d), b = __shfl_down(w23, d), q = __shfl_down(w4, d);
        if (lane + d < 64 && gd == g) {
          w01 += a;
          w23 += b;
          w4 += q;
        }
      }
      const int gu = __shfl_up(g, 1);
      if (ok && (lane == 0 || gu != g)) {
        atomicAdd(&cq2[2 * g], w01);
        if (2 * g + 1 < nq2) atomicAdd(&cq2[2 * g + 1], w23);
        atomicAdd(&cq4[g], w4);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) colacc[i] += (x[u][r][i] | (x[u][r][i] >> 8)) & 0x00010001u;
    }
  }
  if (live) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int kp = 8 * c + 2 * i + h;
        const int n = (int)((colacc[i] >> (16 * h)) & 0xffffu);
        if (n && kp < nk2) atomicAdd(&ck2[kp], n);
      }
  }
  // Counts -> sort keys count * 2048 + (2047 - index): a larger key sorts
  // first, equal counts in index order (indices < 2048); entries past the
  // ends keep -1.
  __syncthreads();
  for (int i = tid; i < kOrderMax; i += 1024) {
    if (i < nq2) cq2[i] = cq2[i] * 2048 + (2047 - i);
    if (i < nk2) ck2[i] = ck2[i] * 2048 + (2047 - i);
    if (i < nq4) cq4[i] = cq4[i] * 2048 + (2047 - i);
  }
  __syncthreads();
  int* out = order + (int64_t)blockIdx.x * (nq2 + nq4 + nk2);
  for (int u = tid; u < nq2 + nq4 + nk2; u += 1024) {
    if (u < nq2) {
      out[rank_of(cq2, nq2, u)] = u;
    } else if (u < nq2 + nq4) {
      const int i = u - nq2;
      out[nq2 + rank_of(cq4, nq4, i)] = i;
    } else {
      const int i = u - nq2 - nq4;
      out[nq2 + nq4 + rank_of(ck2, nk2, i)] = i;
    }
  }
}

// ---------------------------------------------------------------------------
// Forward kernel for fp32 I/O (16-bit I/O has its own kernel with direct
// global->LDS tile copies).  Block = 4 waves x 32 queries (128 rows).  Up to
// DP = 128 two blocks share a CU, so one block's softmax (VALU, v_exp)
// overlaps the other's MFMAs; at DP = 256 a block has the CU alone (one wave
// per SIMD, up to 512 registers for the stationary Q and the O
// accumulators).  K/V tiles (64 keys; 32 at DP = 256, to fit LDS) stream
// through double-buffered LDS: the next tile is fetched into registers while
// the current one is consumed.
//
// Each wave computes S^T = K Q^T so that a lane owns one query row: the row
// max / sum need one cross-lane exchange (lane l <-> l^32) and P feeds the
// P.V product straight from registers as its reduction operand; V is stored
// transposed in LDS.
//
// The running max is only raised when a row's new maximum exceeds it by more
// than kRescaleSlack (in log2 units): P is then bounded by 2^kRescaleSlack and
// the O / l rescale, a full pass over the accumulators, becomes rare.  The
// result is exact: O and l are accumulated against the same reference max.
// ---------------------------------------------------------------------------
constexpr float kRescaleSlack = 8.0f;
constexpr int kMaxTileClasses = 1024;  // per-block key-tile classes kept in LDS

template <typename T, int DP, bool HAS_BIAS, bool CAUSAL>
__global__ __launch_bounds__(256, DP > 128 ? 1 : 2) void fwd_kernel(const Params p) {
  using M = Mma<T>;
  using Frag = typename M::Frag;
  static_assert(sizeof(T) == 4, "fp32 I/O");
  constexpr int EPC = M::EPC, KC = M::KC;
  constexpr int BM = 128, BN = DP > 128 ? 32 : 64;
  constexpr int NKB = BN / 32;    // 32-key blocks per tile
  constexpr int SKK = DP + EPC;   // K row stride (16 B pad)
  constexpr int SKV = BN + 4;     // transposed V row stride
  constexpr int KSZ = BN * SKK;
  constexpr int VSZ = DP * SKV;
  constexpr int NC = DP / KC;
  constexpr int NDB = DP / 32;
  constexpr int CPR = DP / EPC;  // 16-byte chunks per row
  constexpr int FPB = M::FRAGS_PER_BLOCK;
  constexpr int NCH = BN * CPR / 256;  // 16-byte chunks per thread per tile
  __shared__ __attribute__((aligned(16))) T smem[2 * (KSZ + VSZ)];
  __shared__ uint8_t tcls[kMaxTileClasses];

  const int vid = xcd_remap(blockIdx.x, p.B * p.H, p.nqt);
  const int bh = vid / p.nqt;
  const int qt = p.nqt - 1 - (vid % p.nqt);  // longest (causal) tiles first
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, c32 = lane & 31;
  const int q0 = qt * BM;
  const int qw0 = q0 + wave * 32;
  const int qrow = qw0 + c32;
  const bool qok = qrow < p.Lq;
  const int qc = qok ? qrow : p.Lq - 1;

  const T* kp = (const T*)p.k + b * p.k_str[0] + h * p.k_str[1];
  const T* vp = (const T*)p.v + b * p.v_str[0] + h * p.v_str[1];
  const int64_t ks = p.k_str[2], vs = p.v_str[2];

  // --- key-tile schedule: classes of this block's tiles into LDS ------------
  const int k_end = CAUSAL ? min(p.Lk, q0 + BM) : p.Lk;
  const int nkt = (k_end + BN - 1) / BN;
  const bool cls_lds = p.has_tilemap && nkt <= kMaxTileClasses;
  if (cls_lds) {
    for (int t = tid; t < nkt; t += 256)
      tcls[t] = (uint8_t)tile_class(p, b, h, q0, q0 + BM, t * BN, t * BN + BN);
  }
  __syncthreads();
  auto tclass = [&](int t) -> int {
    if (!p.has_tilemap) return 3;
    if (cls_lds) return tcls[t];
    return tile_class(p, b, h, q0, q0 + BM, t * BN, t * BN + BN);
  };

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
  const int64_t brow = HAS_BIAS ? b * p.bias_str[0] + h * p.bias_str[1] +
                                      (int64_t)qc * p.bias_str[2]
                                : 0;
  const uint8_t* mrow = p.has_mask ? p.mask + b * p.mask_str[0] +
                                         h * p.mask_str[1] +
                                         (int64_t)qc * p.mask_str[2]
                                   : nullptr;

  f32x16 oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[db][r] = 0.f;
  float m_ref = -INFINITY, l_i = 0.f;

  // --- K / V tile staging (global -> registers -> LDS) ----------------------
  Frag kst[NCH], vst[NCH];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int idx = tid + i * 256;
      const int r = idx / CPR, d = (idx % CPR) * EPC;
      const int key = k0 + r;
      const bool ok = key < p.Lk;
      kst[i] = ok && d < p.D ? ld16(kp + (int64_t)key * ks + d) : zero_frag<T>();
      vst[i] = ok && d < p.Dv ? ld16(vp + (int64_t)key * vs + d) : zero_frag<T>();
    }
  };
  auto lstore = [&](int buf) {
    T* Ks = smem + buf * (KSZ + VSZ);
    T* Vs = Ks + KSZ;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int idx = tid + i * 256;
      const int r = idx / CPR, d = (idx % CPR) * EPC;
      *reinterpret_cast<Frag*>(&Ks[r * SKK + d]) = kst[i];
#pragma unroll
      for (int j = 0; j < EPC; ++j) Vs[(d + j) * SKV + r] = vst[i][j];
    }
  };

  int kt = 0;
  while (kt < nkt && !(tclass(kt) & 1)) ++kt;
  if (kt < nkt) {
    gload(kt * BN);
    lstore(0);
  }
  __syncthreads();
  int buf = 0;

  while (kt < nkt) {
    const int cls = tclass(kt);
    int kn = kt + 1;
    while (kn < nkt && !(tclass(kn) & 1)) ++kn;
    // In flight while this tile is consumed (at DP = 256 the staging
    // registers are not free during the tile: the load follows it).
    if (DP <= 128 && kn < nkt) gload(kn * BN);

    const T* Ks = smem + buf * (KSZ + VSZ);
    const T* Vs = Ks + KSZ;
    const int k0 = kt * BN;

    // S^T = K Q^T: BN keys (NKB 32-key blocks) x 32 queries.
    f32x16 s[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kb][r] = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
        M::run(s[kb], ld16(&Ks[(kb * 32 + c32) * SKK + c * KC + g * EPC]),
               qf[c]);

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
          if constexpr (HAS_BIAS)
            bv = load_bias4(p, p.bias, brow + key0, p.Lk - key0);
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

    // Online softmax with a lazily raised reference max.
    float mt = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[kb][r]);
    mt = fmaxf(mt, shfl_xor32(mt)) * cc;
    const bool raise = mt > m_ref + kRescaleSlack;
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
        const float e = fast_exp2(__builtin_fmaf(s[kb][r], cc, neg_m));
        s[kb][r] = e;
        rs += e;
      }
    l_i += rs;

    // O^T += V^T P^T.
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int f = 0; f < FPB; ++f) {
        const Frag pf = M::pack(s[kb], f);
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          M::run(oacc[db], lds_frag_t<T>(&Vs[(db * 32 + c32) * SKV + kb * 32], g, f), pf);
        }
      }

    if (DP > 128 && kn < nkt) gload(kn * BN);
    if (kn < nkt) lstore(buf ^ 1);
    __syncthreads();
    buf ^= 1;
    kt = kn;
  }

  // Finalise: O = O / l (a fully masked row gives 0/0 = NaN, as the
  // reference's softmax over all -inf logits does), lse = ln sum exp.
  const float l = l_i + shfl_xor32(l_i);
  const float inv = 1.0f / l;
  if (qok) {
    T* op = (T*)p.o + b * p.o_str[0] + h * p.o_str[1] +
            (int64_t)qrow * p.o_str[2];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d0 = db * 32 + 8 * c + 4 * g;
        if (d0 < p.Dv) store4(op + d0, oacc[db], 4 * c, inv);
      }
    if (g == 0 && p.lse)
      p.lse[((int64_t)b * p.H + h) * p.Lq + qrow] =
          (m_ref + __log2f(l)) * kLn2;
  }
}

// ---------------------------------------------------------------------------
// Host launchers.
// ---------------------------------------------------------------------------
void launch_tilemap(const Params& p, int MB, int MH, int MQ, int MK, int vec16,
                    hipStream_t stream) {
  const int64_t pairs = (int64_t)MB * MH * MQ * ((MK + 1) / 2);
  const int n = (int)((pairs + 3) / 4);
  hipLaunchKernelGGL(tilemap_kernel, dim3(n), dim3(256), 0, stream, p, MB, MH,
                     MQ, MK, vec16);
}

void launch_tile_order(const uint8_t* tilemap, int slices, int MQ, int MK, int vec16,
                       int* order, hipStream_t stream) {
  hipLaunchKernelGGL(tile_order_kernel, dim3(slices), dim3(1024), 0, stream, tilemap, MQ,
                     MK, vec16, order);
}

template <typename T, int DP, bool HB, bool CA>
static void launch_fwd_t(Params p, hipStream_t stream) {
  constexpr int BM = 128;
  p.nqt = (p.Lq + BM - 1) / BM;
  const int n = p.B * p.H * p.nqt;
  hipLaunchKernelGGL((fwd_kernel<T, DP, HB, CA>), dim3(n), dim3(256), 0,
                     stream, p);
}

template <typename T, int DP>
static void launch_fwd_flags(const Params& p, hipStream_t stream) {
  if (p.has_bias) {
    if (p.causal) launch_fwd_t<T, DP, true, true>(p, stream);
    else launch_fwd_t<T, DP, true, false>(p, stream);
  } else {
    if (p.causal) launch_fwd_t<T, DP, false, true>(p, stream);
    else launch_fwd_t<T, DP, false, false>(p, stream);
  }
}

void launch_fwd(const Params& p, int io_dtype, int dp, hipStream_t stream) {
  if (io_dtype == kBF16 || io_dtype == kF16) {
    launch_fwd16(p, io_dtype, dp, stream);
  } else if (!launch_fwd32(p, dp, stream)) {
    if (dp == 64) launch_fwd_flags<float, 64>(p, stream);
    else if (dp == 128) launch_fwd_flags<float, 128>(p, stream);
    else launch_fwd_flags<float, 256>(p, stream);
  }
}

}  // namespace nxa
