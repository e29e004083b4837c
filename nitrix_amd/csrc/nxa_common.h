// Shared device-side definitions for the gfx950 attention kernels.
//
// Conventions used by every kernel in this library
// ------------------------------------------------
// * Tensors are [B, H, L, D] with unit stride over D; the B/H/L strides come
//   from the descriptor (element units).  Bias and mask are [B, H, Lq, Lk]
//   with unit stride over Lk and zero strides on broadcast axes.
// * Matrix products run on 32x32 MFMA tiles (v_mfma_f32_32x32x16_bf16 /
//   _f16 for bf16 / fp16 I/O, v_mfma_f32_32x32x2_f32 for fp32 I/O), fp32
//   accumulation.
// * A lane's 16-byte operand chunk c covers head-dim elements
//   d = c*KC + g*EPC + [0, EPC) where g = lane / 32, EPC = elements per 16 B
//   and KC = 2*EPC.  A and B operands use the same mapping, so any fixed
//   permutation of the reduction index is harmless.
// * 32x32 accumulator layout: lane l holds column (l % 32) and rows
//   8*(r/4) + 4*(l/32) + (r%4) for register r in [0, 16).
// * When an accumulator feeds the next product as its reduction operand
//   (P into P.V, dS into dS.K, ...), register group c (registers 4c..4c+3)
//   maps to reduction rows 8c + 4g + [0, 4); the transposed LDS copy of the
//   other operand is read at exactly those rows.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// Lambdas used several times in a kernel body must still be inlined: an
// outlined call would spill the accumulators through the call ABI.
#define NXA_INLINE __attribute__((always_inline))

namespace nxa {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kTile = 64;  // tile-map granularity (queries x keys)

enum DType : int { kBF16 = 0, kF32 = 1, kF16 = 2 };

// dbias handling selected on the host.
enum DbiasMode : int {
  kDbiasNone = 0,
  kDbiasFull = 1,      // dbias has the full [Lq, Lk] extent per (b, h): store dS
  kDbiasColsum = 2,    // bias broadcast over Lq: store sum_q dS per key
};

// All kernels take one parameter block by value.
struct Params {
  const void* q;
  const void* k;
  const void* v;
  const void* bias;
  const uint8_t* mask;
  void* o;
  float* lse;
  const void* dout;
  void* dq;
  void* dk;
  void* dv;
  void* dbias;         // final dbias, or the fp32 partial buffer (dbias_f32=1)
  float* ndelta;       // [B, H, Lq] -rowsum(O * dO)       (backward workspace)
  float* nlse2;        // [B, H, Lq] -lse * log2(e)         (backward workspace)
  const uint8_t* tilemap;
  uint8_t* tilemap_out;

  int64_t q_str[3], k_str[3], v_str[3], o_str[3];  // B, H, L (D stride is 1)
  int64_t bias_str[3];                               // B, H, Lq (Lk stride 1)
  int64_t mask_str[3];
  int64_t dbias_str[3];
  int64_t tm_str[3];                                 // tile-map B, H, Q-tile

  int B, H, Lq, Lk, D;
  int Dv;              // head dim of v, o, dO, dv (D: q, k, dq, dk)
  int nqt;             // query tiles of the launching kernel (grid decode)
  int nkt;             // key tiles of the launching kernel
  int bh0, nbh;        // dK/dV launches cover (batch, head) pairs bh0 .. bh0+nbh-1
                       // (pair index b * H + h)
  int64_t dbias_off;   // subtracted from every dbias offset (chunked partials)
  float scale;
  float scale_log2;    // scale * log2(e)
  int causal;
  int has_bias, bias_dtype, bias_vec;
  int has_mask, mask_vec;
  int has_tilemap;
  int tm_nk;           // tile-map key tiles
  int tm_rows;         // mask rows covered by the tile map (Lq, or 1 if broadcast)
  int dbias_mode;
  int dbias_f32;       // 1: dbias points at fp32 partials, else bias dtype
  int fwd_bias;        // FwdBias mode of the 16-bit forward
  float bias_h, bias_l;  // 1/scale = bias_h + bias_l, both exact in the bias dtype
  // qk-norm VJP fused into the dQ and dK epilogues (16-bit backward): q and k
  // are the RMS-normalised inputs, qraw / kraw the inputs before the norm
  // (same strides), qrstd / krstd their per-row rsqrt(mean(x^2) + eps)
  // ([B, H, Lq] and [B, H, Lk]); dq / dk then receive the gradients with
  // respect to the raw inputs.
  int qk_norm;
  const void* qraw;
  const void* kraw;
  const float* qrstd;
  const float* krstd;
  // qk-norm of q fused into the 16-bit forward (qn_on): q holds the raw
  // rows, the kernel normalises its stationary Q fragments (y = x
  // rsqrt(mean(x^2) + eps), fp32, cast to the I/O dtype) and, where not
  // NULL, writes them to qn_out (q's strides) and the per-row rsqrt to
  // qn_rstd ([B, H, Lq]).
  int qn_on;
  void* qn_out;
  float* qn_rstd;
  float qn_eps;
  // Block order of a mask that varies over queries (non-causal, 16-bit
  // kernels): per tile-map slice, the 128-row query blocks, the 256-row
  // query blocks and the 128-key blocks, each sorted by kept map tiles, most
  // first (tile_order_kernel).  NULL: blocks in index order.
  const int* order;
  int64_t ord_str[2];  // per batch / per head of the slice (0 if broadcast)
  int ord_q128, ord_q256, ord_k128;  // offsets of the three lists in a slice
};

// Longest list tile_order_kernel sorts (blocks per list per slice).
constexpr int kOrderMax = 1024;

// Tile index of the i-th block (of n) of (b, h) under the block order, as a
// block-uniform value.  The lists are permutations of 0 .. n-1 by
// construction; the clamp keeps a block inside its head whatever the list
// holds.
__device__ __forceinline__ int ordered_tile(const Params& p, int b, int h, int off, int i,
                                            int n) {
  const int t = p.order[b * p.ord_str[0] + h * p.ord_str[1] + off + i];
  return __builtin_amdgcn_readfirstlane(min(max(t, 0), n - 1));
}

// Gradient of y = x * r (r = rsqrt(mean(x^2) + eps) over one row of n
// elements) for the row a lane shares with lane ^ 32: dx = r (dy - y
// mean(dy y)), with y = x r in fp32.  `gy` holds the lane's NDB x 16
// values of dy (accumulator layout: element 4c + j of block db is column
// db * 32 + 8c + 4g + j), `xrow` the row of x; the results overwrite gy.
// Two passes over x (the second re-reads the row, 2n bytes, from cache) so
// that y needs no registers of its own.
template <typename T, int NDB>
__device__ __forceinline__ void rms_norm_vjp_rows(float (&gy)[NDB][16], const T* xrow,
                                                  float r, int n, int g) {
  typedef T t4 __attribute__((ext_vector_type(4)));
  auto y4 = [&](int d0, int j, const t4& xv) -> float {
    return d0 < n ? (float)xv[j] * r : 0.f;
  };
  float dot = 0.f;
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int d0 = db * 32 + 8 * c + 4 * g;
      t4 xv;
      if (d0 < n) xv = *reinterpret_cast<const t4*>(xrow + d0);
#pragma unroll
      for (int j = 0; j < 4; ++j) dot = __builtin_fmaf(gy[db][4 * c + j], y4(d0, j, xv), dot);
    }
  dot += __shfl_xor(dot, 32, 64);
  const float mean = dot / (float)n;
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int d0 = db * 32 + 8 * c + 4 * g;
      t4 xv;
      if (d0 < n) xv = *reinterpret_cast<const t4*>(xrow + d0);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        gy[db][4 * c + j] = r * (gy[db][4 * c + j] - y4(d0, j, xv) * mean);
    }
}

// Parameter block of the qk-norm kernels.
struct NormParams {
  const void* x;        // rows of D elements, x_stride apart
  void* y;              // forward output [rows, D]
  float* rstd;          // per-row rsqrt(mean(x^2) + eps)
  const void* dy;       // backward: cotangent of y [rows, D]
  void* dx;             // backward output [rows, D]
  int64_t rows, x_stride;
  int D;
  float eps;
};

// Parameter block of the selective-scan kernels (fp32; layouts in nxa_ssm.hip).
struct SsmParams {
  const float *x, *delta, *A, *B, *C, *D;  // D may be null
  float* y;
  const float* dy;
  float *dx, *ddelta, *dA, *dB, *dC, *dD;  // dD may be null
  float* hc;      // [nb][nc][NP][Dm] chunk states: local end state, then entering state
  float* gc;      // [nb][nc][NP][Dm] chunk adjoints, then the dA partial sums
  float* sdt;     // [nb][nc][Dm] sum of delta over each chunk
  float* hs;      // [nb][ns][NP][Dm] state entering each sub-chunk (may be null in fwd)
  float* dDpart;  // [nb][nc][Dm]
  float* dBCpart; // [ndblk_b][nb][L][2 NP]
  float* dadpart; // [groups][(NP + 1) Dm] first-level sums of dA / dD
  int64_t nb;
  int L, Dm, N;
  int nc, ns;     // chunks, sub-chunks
  int ndblk;      // channel blocks (one lane per channel)
  int ndblk_b;    // channel blocks of the backward chunk pass (lanes per channel > 1)
};

// How the 16-bit forward adds the bias (chosen on the host).
//  * kFbRow  / kFbTile: the bias enters the score accumulator through MFMA
//    products bias^T x diag(1/scale) (1/scale split into two terms of the
//    bias dtype, which is then the I/O dtype), so
//    it costs no VALU work; kFbTile streams [query, key] bias tiles through
//    the LDS ring, kFbRow (bias broadcast over queries) one key row per tile.
//  * kFbValu: per-element loads and adds (fp32 bias, unaligned layouts).
enum FwdBias : int { kFbNone = 0, kFbRow = 1, kFbTile = 2, kFbValu = 3 };

// ---------------------------------------------------------------------------
// MFMA policy per I/O type.
// ---------------------------------------------------------------------------
template <typename T>
struct Mma;

template <>
struct Mma<bf16> {
  static constexpr int EPC = 8;   // elements per 16-byte chunk
  static constexpr int KC = 16;   // reduction elements per chunk (both lane groups)
  using Frag = bf16x8;
  static __device__ __forceinline__ void run(f32x16& c, const Frag& a,
                                             const Frag& b) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  // The product alone (accumulator input zero).
  static __device__ __forceinline__ f32x16 first(const Frag& a, const Frag& b) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, f32x16{}, 0, 0, 0);
  }
  // Reduction fragment f of a 32-row accumulator block: registers 8f..8f+7
  // (row groups c = 2f, 2f+1).
  static constexpr int FRAGS_PER_BLOCK = 2;
  static __device__ __forceinline__ Frag pack(const f32x16& acc, int f) {
    Frag r;
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = (bf16)acc[8 * f + j];
    return r;
  }
};

// fp16: the same operand layout as bf16 (8 elements per 16 bytes).
template <>
struct Mma<f16> {
  static constexpr int EPC = 8;
  static constexpr int KC = 16;
  using Frag = f16x8;
  static __device__ __forceinline__ void run(f32x16& c, const Frag& a,
                                             const Frag& b) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x16 first(const Frag& a, const Frag& b) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, f32x16{}, 0, 0, 0);
  }
  static constexpr int FRAGS_PER_BLOCK = 2;
  static __device__ __forceinline__ Frag pack(const f32x16& acc, int f) {
    Frag r;
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = (f16)acc[8 * f + j];
    return r;
  }
};

template <>
struct Mma<float> {
  static constexpr int EPC = 4;
  static constexpr int KC = 8;
  using Frag = f32x4;
  static __device__ __forceinline__ void run(f32x16& c, const Frag& a,
                                             const Frag& b) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[i], c, 0, 0, 0);
  }
  static constexpr int FRAGS_PER_BLOCK = 4;
  static __device__ __forceinline__ Frag pack(const f32x16& acc, int f) {
    Frag r;
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = acc[4 * f + j];
    return r;
  }
};

// ---------------------------------------------------------------------------
// Memory helpers.
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ typename Mma<T>::Frag ld16(const T* p) {
  return *reinterpret_cast<const typename Mma<T>::Frag*>(p);
}

template <typename T>
__device__ __forceinline__ typename Mma<T>::Frag zero_frag() {
  typename Mma<T>::Frag z;
#pragma unroll
  for (int j = 0; j < Mma<T>::EPC; ++j) z[j] = (T)0.0f;
  return z;
}

// Transposed-operand fragment f from an LDS row holding reduction index as
// the contiguous axis: row groups c = f*(EPC/4) + i read 4 elements at
// row[8c + 4g].
template <typename T>
__device__ __forceinline__ typename Mma<T>::Frag lds_frag_t(const T* row,
                                                            int g, int f) {
  using Frag = typename Mma<T>::Frag;
  if constexpr (sizeof(T) == 4) {
    return *reinterpret_cast<const Frag*>(row + 8 * f + 4 * g);
  } else {
    typedef T t4 __attribute__((ext_vector_type(4)));
    const t4 lo = *reinterpret_cast<const t4*>(row + 16 * f + 4 * g);
    const t4 hi = *reinterpret_cast<const t4*>(row + 16 * f + 8 + 4 * g);
    Frag r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      r[j] = lo[j];
      r[4 + j] = hi[j];
    }
    return r;
  }
}

// Reduction-operand fragment f of a 32x16 MFMA operand read *transposed*
// from a row-major 16-bit LDS tile whose rows are the reduction index:
// lane L receives tile[r0 + key(f, L/32, j)][col0 + L%32] for j = 0..7 with
// key(f, g, j) = 16f + 8(j/4) + 4g + j%4 -- the row groups the accumulator
// layout assigns to fragment f.
//
// ds_read_b64_tr_b16 works on 16-lane groups: output lane j, element e is
// element (j%4) of the 8 bytes addressed by lane 4e + j/4 of the group.  So
// lane i of a group addresses row (r0 + 16f + 4g + i/4 [+8]) at column
// (col0 + 16*(group%2) + 4*(i%4)).
typedef short i16x4 __attribute__((ext_vector_type(4)));
template <typename T>
__device__ __forceinline__ typename Mma<T>::Frag lds_tr_frag(const T* tile, int stride,
                                                             int r0, int col0, int lane,
                                                             int f) {
  static_assert(sizeof(T) == 2, "16-bit tiles");
  const int grp = lane >> 4, i = lane & 15;
  const int row = r0 + 16 * f + 4 * (grp >> 1) + (i >> 2);
  const int col = col0 + 16 * (grp & 1) + 4 * (i & 3);
  const T* p0 = tile + row * stride + col;
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)p0);
  const i16x4 hi =
      __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p0 + 8 * stride));
  typedef short i16x8 __attribute__((ext_vector_type(8)));
  const i16x8 r = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(typename Mma<T>::Frag, r);
}

// XOR-swizzled bf16 tiles with DP columns and no row padding.  The 16-byte
// chunk c of row r is stored at chunk c ^ swz(r).  The swizzle is
// conflict-free (64 banks x 4 bytes) both for 16-byte row reads of 16
// consecutive rows and for ds_read_b64_tr_b16 reads, whose 32 lanes cover
// 4 consecutive rows x 64 bytes; plain padding cannot serve both patterns.
template <int DP>
__device__ __forceinline__ int swz(int r);
template <>
__device__ __forceinline__ int swz<128>(int r) {
  return 4 * (r & 3) + ((r >> 2) & 3);
}
// 256 columns: the same pattern as 128 (the row stride is a multiple of
// the 64 banks either way, and the XOR touches only the low 4 chunk bits).
template <>
__device__ __forceinline__ int swz<256>(int r) {
  return 4 * (r & 3) + ((r >> 2) & 3);
}
template <>
__device__ __forceinline__ int swz<64>(int r) {
  return 4 * ((r >> 1) & 1) + ((r >> 2) & 3);
}
template <int DP>
__device__ __forceinline__ int swz_off(int row, int chunk) {
  return row * DP + 8 * (chunk ^ swz<DP>(row));
}

// ---------------------------------------------------------------------------
// Direct global -> LDS copies (no staging registers).  For one wave, lane l's
// `size` bytes land at lds + l * size; the LDS address must be wave-uniform.
// Completion is tracked by vmcnt like any vector load.
// ---------------------------------------------------------------------------
//
// The copies are written as inline assembly on purpose: the compiler treats
// its own LDS-DMA builtin as a store to all of LDS and waits for vmcnt(0)
// before the next LDS read, which would drain every prefetch in flight.
// Callers order the copies themselves: a vmcnt wait for their own copies,
// then a barrier, before anyone reads the destination.  M0 carries the LDS
// base; one wait state separates its write from the copy.
__device__ __forceinline__ uint32_t lds_offset(const void* lds) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds;
}
// Instruction classes of __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedValu = 0x002, kSchedMfma = 0x008, kSchedDsRead = 0x100,
              kSchedDsWrite = 0x200;

// s_waitcnt immediate that waits for vmcnt <= n and leaves expcnt / lgkmcnt
// unconstrained (gfx9 encoding: vmcnt bits [3:0] and [15:14]).
__device__ __forceinline__ constexpr int vmcnt_imm(int n) {
  return (n & 0xF) | (((n >> 4) & 3) << 14) | (0x7 << 4) | (0xF << 8);
}
// s_waitcnt immediate that waits for lgkmcnt <= n (LDS / scalar memory)
// and leaves vmcnt / expcnt unconstrained.
__device__ __forceinline__ constexpr int lgkmcnt_imm(int n) {
  return 0xF | (3 << 14) | (0x7 << 4) | ((n & 0xF) << 8);
}

// Workgroup barrier without a memory fence: LDS filled by direct copies is
// published by each wave's own vmcnt wait before the barrier (a fenced
// __syncthreads would wait for every copy still in flight, including the
// prefetch of later tiles).  The empty asm statements keep the compiler from
// moving memory accesses across the barrier.
__device__ __forceinline__ void barrier_nofence() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Direct copies addressed as a wave-uniform base (SGPR pair) plus a per-lane
// 32-bit byte offset (the global_load "saddr" form): no 64-bit per-lane
// address arithmetic and no 64-bit per-lane address registers.
__device__ __forceinline__ void dma16_sv(const void* base, uint32_t voff, uint32_t lds) {
  const uint32_t m = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(voff), "s"(base), "s"(m) : "m0");
}
// The same, marked non-temporal: for streams read exactly once (full bias
// tiles), so that they do not displace the reused K / V tiles in the caches.
__device__ __forceinline__ void dma16_sv_nt(const void* base, uint32_t voff, uint32_t lds) {
  const uint32_t m = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt"
               :: "v"(voff), "s"(base), "s"(m) : "m0");
}
__device__ __forceinline__ void dma4_sv(const void* base, uint32_t voff, uint32_t lds) {
  const uint32_t m = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1"
               :: "v"(voff), "s"(base), "s"(m) : "m0");
}

// Streams XOR-swizzled [ROWS x DP] bf16 tiles (64 rows unless stated; swz_off
// layout, no padding) of one [nrows, D] matrix (row stride rs elements) into
// LDS with 1 KB direct copies: a tile is ROWS*DP/512 copies, each covering
// 512/DP whole rows of global memory, and every one of the NW waves issues
// exactly CNT of them (so per-wave copy counts are compile-time).  The
// lane's source offset inside the tile is computed once.  Rows past nrows
// are clamped to the last row (only in the tail tile) and head-dim chunks
// past D read chunk 0 of the row: finite filler that callers mask or
// multiply by zero.
template <int DP, int NW, int ROWS = 64>
struct SwzStream {
  static constexpr int SPR = DP / 8;         // 16-byte slots per row
  static constexpr int NI = ROWS * SPR / 64;  // 1 KB copies per tile
  static constexpr int CNT = NI / NW;
  static_assert(NI % NW == 0, "tile copies must split evenly over the waves");
  // Byte offset of the lane's 16 bytes inside a full tile (64 rows times the
  // row stride fit in 32 bits: the host bounds the row stride).
  uint32_t off[CNT];

  __device__ __forceinline__ static int row_of(int m, int wave, int lane) {
    return ((m * NW + wave) * 64 + lane) / SPR;
  }
  __device__ __forceinline__ static int col_of(int m, int wave, int lane, int D) {
    const int s = (m * NW + wave) * 64 + lane;
    const int lc = (s % SPR) ^ swz<DP>(s / SPR);
    return lc * 8 < D ? lc * 8 : 0;
  }
  __device__ __forceinline__ void init(int64_t rs, int D, int wave, int lane) {
#pragma unroll
    for (int m = 0; m < CNT; ++m)
      off[m] = 2u * (uint32_t)(row_of(m, wave, lane) * rs + col_of(m, wave, lane, D));
  }
  // Copies rows r0.. of `src` (2-byte elements) into the tile at LDS byte
  // offset `lds`.
  template <typename E>
  __device__ __forceinline__ void issue(const E* src, int64_t rs, int r0,
                                        int nrows, int D, uint32_t lds, int wave,
                                        int lane) const {
#pragma unroll
    for (int m = 0; m < CNT; ++m) issue_one(src, rs, r0, nrows, D, lds, m, wave, lane);
  }
  // Copy m of the wave's CNT copies of that tile.
  template <typename E>
  __device__ __forceinline__ void issue_one(const E* src, int64_t rs, int r0,
                                            int nrows, int D, uint32_t lds, int m,
                                            int wave, int lane) const {
    static_assert(sizeof(E) == 2, "16-bit tiles");
    const E* base = src + (int64_t)r0 * rs;  // wave-uniform
    if (r0 + ROWS <= nrows) {
      dma16_sv(base, off[m], lds + (m * NW + wave) * 1024);
    } else {
      const int r = min(row_of(m, wave, lane), nrows - 1 - r0);
      dma16_sv(base, 2u * (uint32_t)(r * rs + col_of(m, wave, lane, D)),
               lds + (m * NW + wave) * 1024);
    }
  }
};

// Buffer resource (V#) of the raw byte range [base, base + bytes): buffer
// loads at offsets beyond it return zero instead of touching memory, so a
// tile that runs past the end of a matrix needs no clamping (and a range of
// zero bytes turns a copy into a no-op that still counts in vmcnt).
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4 make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)base;
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((int)((a >> 32) & 0xffff));  // stride 0
  r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
  r[3] = 0x00020000;
  return r;
}
// Direct copies through a buffer resource: 16 (or 4) bytes at byte offset
// voff of the range to LDS byte offset `lds` (wave-uniform) + 16 (4) * lane.
__device__ __forceinline__ void dma16_buf(i32x4 rsrc, uint32_t voff, uint32_t lds) {
  const uint32_t m = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :: "v"(voff), "s"(rsrc), "s"(m) : "m0");
}
__device__ __forceinline__ void dma4_buf(i32x4 rsrc, uint32_t voff, uint32_t lds) {
  const uint32_t m = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dword %0, %1, 0 offen lds"
               :: "v"(voff), "s"(rsrc), "s"(m) : "m0");
}

__device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(f16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(float x) { return x; }

template <typename T>
__device__ __forceinline__ T from_f32(float x) {
  return (T)x;
}

// Stores acc[off..off+3] * scale as four contiguous elements (8 or 16 bytes).
__device__ __forceinline__ void store4(bf16* dst, const f32x16& acc, int off,
                                       float scale) {
  bf16x4 v;
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = (bf16)(acc[off + j] * scale);
  *reinterpret_cast<bf16x4*>(dst) = v;
}
__device__ __forceinline__ void store4(f16* dst, const f32x16& acc, int off,
                                       float scale) {
  f16x4 v;
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = (f16)(acc[off + j] * scale);
  *reinterpret_cast<f16x4*>(dst) = v;
}

// One bias / dbias element of runtime dtype `dt` (kBF16, kF16 or kF32).
__device__ __forceinline__ float load_elem(int dt, const void* base, int64_t off) {
  if (dt == kBF16) return (float)reinterpret_cast<const bf16*>(base)[off];
  if (dt == kF16) return (float)reinterpret_cast<const f16*>(base)[off];
  return reinterpret_cast<const float*>(base)[off];
}
__device__ __forceinline__ void store_elem(int dt, void* base, int64_t off, float x) {
  if (dt == kBF16)
    reinterpret_cast<bf16*>(base)[off] = (bf16)x;
  else if (dt == kF16)
    reinterpret_cast<f16*>(base)[off] = (f16)x;
  else
    reinterpret_cast<float*>(base)[off] = x;
}
__device__ __forceinline__ void store4(float* dst, const f32x16& acc, int off,
                                       float scale) {
  f32x4 v;
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = acc[off + j] * scale;
  *reinterpret_cast<f32x4*>(dst) = v;
}

// Four contiguous bias values (as fp32), honouring the runtime dtype.
__device__ __forceinline__ f32x4 load_bias4(const Params& p, const void* base,
                                            int64_t off, int valid) {
  f32x4 r = {0.f, 0.f, 0.f, 0.f};
  if (p.bias_dtype == kBF16) {
    const bf16* b = reinterpret_cast<const bf16*>(base) + off;
    if (p.bias_vec && valid >= 4) {
      const bf16x4 v = *reinterpret_cast<const bf16x4*>(b);
#pragma unroll
      for (int j = 0; j < 4; ++j) r[j] = (float)v[j];
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (j < valid) r[j] = (float)b[j];
    }
  } else if (p.bias_dtype == kF16) {
    const f16* b = reinterpret_cast<const f16*>(base) + off;
    if (p.bias_vec && valid >= 4) {
      const f16x4 v = *reinterpret_cast<const f16x4*>(b);
#pragma unroll
      for (int j = 0; j < 4; ++j) r[j] = (float)v[j];
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (j < valid) r[j] = (float)b[j];
    }
  } else {
    const float* b = reinterpret_cast<const float*>(base) + off;
    if (p.bias_vec && valid >= 4) {
      r = *reinterpret_cast<const f32x4*>(b);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (j < valid) r[j] = b[j];
    }
  }
  return r;
}

// Four contiguous keep-mask bytes packed into the low bits of each byte
// (nonzero = keep); entries past `valid` read as masked.
__device__ __forceinline__ uint32_t load_mask4(const Params& p, const uint8_t* m,
                                               int valid) {
  if (p.mask_vec && valid >= 4) return *reinterpret_cast<const uint32_t*>(m);
  uint32_t r = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (j < valid) r |= (uint32_t)m[j] << (8 * j);
  return r;
}

__device__ __forceinline__ bool mask_bit(uint32_t w, int j) {
  return ((w >> (8 * j)) & 0xffu) != 0;
}

__device__ __forceinline__ float fast_exp2(float x) {
  return __builtin_amdgcn_exp2f(x);
}

__device__ __forceinline__ float shfl_xor32(float x) {
  return __shfl_xor(x, 32, 64);
}

// Tile-map lookup: bit0 = some entry kept, bit1 = every entry kept.
__device__ __forceinline__ int tile_class(const Params& p, int b, int h,
                                          int q_lo, int q_hi, int k_lo,
                                          int k_hi) {
  // [q_lo, q_hi) x [k_lo, k_hi) in element units; clipped to the mask extent.
  const uint8_t* tm = p.tilemap + b * p.tm_str[0] + h * p.tm_str[1];
  int any = 0, all = 1;
  const int qt0 = p.tm_rows == 1 ? 0 : q_lo / kTile;
  const int qt1 = p.tm_rows == 1 ? 0 : (min(q_hi, p.Lq) - 1) / kTile;
  const int kt0 = k_lo / kTile;
  const int kt1 = (min(k_hi, p.Lk) - 1) / kTile;
  for (int qt = qt0; qt <= qt1; ++qt)
    for (int kt = kt0; kt <= kt1; ++kt) {
      const int c = tm[qt * p.tm_str[2] + kt];
      any |= c & 1;
      all &= (c >> 1) & 1;
    }
  return any | (all << 1);
}

// Maps a linear block id to a virtual id head * ntiles + tile.  Blocks are
// dispatched round-robin over the 8 XCDs, so block b runs on XCD b % 8; this
// map gives XCD x the heads x, x + 8, x + 16, ... whole: the blocks of one
// (batch, head), which share K / V, share one L2, and every XCD gets the same
// mix of batches (sequence lengths differ between batches, so handing an XCD
// a contiguous range of heads -- a whole batch -- would unbalance them).
__device__ __forceinline__ int xcd_remap(int bid, int nheads, int ntiles) {
  constexpr int kXcd = 8;
  if (nheads % kXcd != 0) return bid;
  const int x = bid % kXcd, k = bid / kXcd;
  return (x + kXcd * (k / ntiles)) * ntiles + k % ntiles;
}

}  // namespace nxa
