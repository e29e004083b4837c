// C ABI of the attention library: descriptor validation, workspace layout,
// kernel dispatch and the thread-local error message.  Declarations and the
// reference interfaces each entry point replaces are in include/nxattn.h.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cmath>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/nxattn.h"
#include "nxa_launch.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

int esize(int dt) { return dt == NXA_F32 ? 4 : 2; }

bool known_dtype(int dt) { return dt == NXA_BF16 || dt == NXA_F32 || dt == NXA_F16; }

// Head dim of v / o (Dv = 0 means Dv = D).
int value_dim(const nxa_desc* d) { return d->Dv > 0 ? d->Dv : d->D; }

// Largest head dim (D or Dv) the kernels take.
constexpr int kMaxHeadDim = 256;

// Padded head-dim width the kernels are instantiated for.
int padded_dim(const nxa_desc* d) {
  const int m = d->D > value_dim(d) ? d->D : value_dim(d);
  return m <= 64 ? 64 : m <= 128 ? 128 : 256;
}

// ---------------------------------------------------------------------------
// Profiling: HIP events around each launch while enabled.
// ---------------------------------------------------------------------------
struct ProfRec {
  std::string name;
  hipEvent_t start, stop;
};
std::mutex g_prof_mu;
bool g_prof_on = false;
std::vector<ProfRec> g_prof;

template <typename F>
int launch(const char* name, hipStream_t stream, F&& f) {
  bool on;
  {
    std::lock_guard<std::mutex> lk(g_prof_mu);
    on = g_prof_on;
  }
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (on) {
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess)
      return fail(NXA_E_LAUNCH, "%s: hipEventCreate failed", name);
    hipEventRecord(e0, stream);
  }
  f();
  const hipError_t err = hipGetLastError();
  if (on) {
    hipEventRecord(e1, stream);
    std::lock_guard<std::mutex> lk(g_prof_mu);
    g_prof.push_back({name, e0, e1});
  }
  if (err != hipSuccess)
    return fail(NXA_E_LAUNCH, "%s: launch failed: %s", name,
                hipGetErrorString(err));
  return NXA_OK;
}

// ---------------------------------------------------------------------------
// Validation shared by every entry point.
// ---------------------------------------------------------------------------
// 64 rows of `stride` elements of `es` bytes, plus one more row of up to
// 256 elements, span less than 2^32 bytes.
bool row_stride_ok(int64_t stride, int es) {
  return stride >= 0 && (64 * stride + 256) * es < ((int64_t)1 << 32);
}

int check_desc(const nxa_desc* d, int has_bias, int has_mask) {
  if (!d) return fail(NXA_E_ARG, "descriptor is NULL");
  if (!known_dtype(d->io_dtype))
    return fail(NXA_E_DTYPE, "io_dtype %d is not NXA_BF16, NXA_F16 or NXA_F32",
                d->io_dtype);
  if (has_bias && !known_dtype(d->bias_dtype))
    return fail(NXA_E_DTYPE, "bias_dtype %d is not NXA_BF16, NXA_F16 or NXA_F32",
                d->bias_dtype);
  if (d->B <= 0 || d->H <= 0 || d->Lq <= 0 || d->Lk <= 0 || d->D <= 0)
    return fail(NXA_E_SHAPE, "extents must be positive (B=%d H=%d Lq=%d Lk=%d D=%d)",
                d->B, d->H, d->Lq, d->Lk, d->D);
  const int epc = 16 / esize(d->io_dtype);
  if (d->Dv < 0) return fail(NXA_E_SHAPE, "value head dim Dv=%d is negative", d->Dv);
  const int dims[2] = {d->D, value_dim(d)};
  const char* dnames[2] = {"D", "Dv"};
  for (int i = 0; i < 2; ++i) {
    if (dims[i] > kMaxHeadDim)
      return fail(NXA_E_UNSUPPORTED, "head dim %s=%d exceeds %d", dnames[i], dims[i],
                  kMaxHeadDim);
    if (dims[i] % epc != 0)
      return fail(NXA_E_UNSUPPORTED, "head dim %s=%d must be a multiple of %d",
                  dnames[i], dims[i], epc);
  }
  const int64_t rows = (int64_t)d->B * d->H * (int64_t)(d->Lq > d->Lk ? d->Lq : d->Lk);
  if (rows >= (int64_t)1 << 31)
    return fail(NXA_E_SHAPE, "B*H*L = %lld exceeds 2^31", (long long)rows);
  const int64_t* strs[4] = {d->q_str, d->k_str, d->v_str, d->o_str};
  const char* names[4] = {"q", "k", "v", "o"};
  for (int t = 0; t < 4; ++t)
    for (int i = 0; i < 3; ++i) {
      if (strs[t][i] < 0)
        return fail(NXA_E_LAYOUT, "%s stride %d is negative", names[t], i);
      if (strs[t][i] % epc != 0)
        return fail(NXA_E_LAYOUT,
                    "%s stride %d (%lld) must be a multiple of %d elements",
                    names[t], i, (long long)strs[t][i], epc);
    }
  // The kernels address a tile's rows (at most 64) with 32-bit byte offsets
  // from the tile's first row: 64 row strides (plus a row) must stay below
  // 2^32 bytes.
  const int io_es = esize(d->io_dtype);
  const int64_t* rows_str[4] = {&d->q_str[2], &d->k_str[2], &d->v_str[2], &d->o_str[2]};
  for (int t = 0; t < 4; ++t)
    if (!row_stride_ok(*rows_str[t], io_es))
      return fail(NXA_E_LAYOUT,
                  "%s row stride %lld elements is too large: 64 rows must span "
                  "less than 2^32 bytes",
                  names[t], (long long)*rows_str[t]);
  if (has_bias)
    for (int i = 0; i < 3; ++i)
      if (d->bias_str[i] < 0)
        return fail(NXA_E_LAYOUT, "bias stride %d is negative", i);
  if (has_bias && !row_stride_ok(d->bias_str[2], esize(d->bias_dtype)))
    return fail(NXA_E_LAYOUT,
                "bias row stride %lld elements is too large: 64 rows must span "
                "less than 2^32 bytes",
                (long long)d->bias_str[2]);
  if (has_mask)
    for (int i = 0; i < 3; ++i)
      if (d->mask_str[i] < 0)
        return fail(NXA_E_LAYOUT, "mask stride %d is negative", i);
  return NXA_OK;
}

bool aligned(const void* p, size_t a) {
  return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

struct MaskGeom {
  int MB, MH, MQ, MK, rows;
  size_t bytes;
  // Block order (nxa::Params::order): per slice nq2 128-row, nq4 256-row and
  // nk2 128-key blocks; `order` false leaves the blocks in index order.
  bool order;
  int nq2, nq4, nk2;
  size_t order_bytes;
};

MaskGeom mask_geom(const nxa_desc* d) {
  MaskGeom m;
  m.MB = (d->mask_str[0] == 0) ? 1 : d->B;
  m.MH = (d->mask_str[1] == 0) ? 1 : d->H;
  const bool qb = d->mask_str[2] == 0 || d->Lq == 1;
  m.rows = qb ? 1 : d->Lq;
  m.MQ = qb ? 1 : (d->Lq + nxa::kTile - 1) / nxa::kTile;
  m.MK = (d->Lk + nxa::kTile - 1) / nxa::kTile;
  m.bytes = (size_t)m.MB * m.MH * m.MQ * m.MK;
  m.nq2 = (m.MQ + 1) / 2;
  m.nq4 = (m.MQ + 3) / 4;
  m.nk2 = (m.MK + 1) / 2;
  // Only a mask that varies over queries gives one head's blocks unequal
  // work (a broadcast row only switches whole key blocks off); causal calls
  // keep their own longest-first order; the 16-bit kernels read the order.
  m.order = !qb && !d->causal && d->io_dtype != NXA_F32 && m.nq2 <= nxa::kOrderMax &&
            m.nk2 <= nxa::kOrderMax;
  m.order_bytes =
      m.order ? (size_t)m.MB * m.MH * (m.nq2 + m.nq4 + m.nk2) * sizeof(int) : 0;
  return m;
}

struct DbiasGeom {
  int mode;        // nxa::DbiasMode
  int LQ;          // rows of dbias: Lq (full) or 1 (column sum)
  bool reduce;     // batch / head axes broadcast: fp32 partials + reduction
  int OB, OH;
  int chunk;       // (batch, head) pairs per dK/dV launch when reducing
  size_t acc_bytes, partial_bytes;
};

// dbias over a bias shared across batch or heads is summed over those axes.
// The dK/dV kernel writes fp32 partials per (batch, head) pair; the pairs
// run in chunks, each followed by a reduction into an fp32 accumulator of the
// bias's own extent, so the workspace is that accumulator plus one chunk of
// partials -- not B * H * Lq * Lk.  A chunk holds as many pairs as the
// accumulator has slots (so the partials never exceed it), or more when that
// gives the dK/dV launch fewer than ~512 blocks (two per CU).
DbiasGeom dbias_geom(const nxa_desc* d) {
  DbiasGeom g;
  const bool colsum = d->Lq > 1 && d->bias_str[2] == 0;
  g.mode = colsum ? nxa::kDbiasColsum : nxa::kDbiasFull;
  g.LQ = colsum ? 1 : d->Lq;
  g.OB = d->bias_str[0] == 0 ? 1 : d->B;
  g.OH = d->bias_str[1] == 0 ? 1 : d->H;
  g.reduce = (d->B > 1 && g.OB == 1) || (d->H > 1 && g.OH == 1);
  const int64_t pairs = (int64_t)d->B * d->H;
  const int64_t nkt = (d->Lk + 127) / 128;
  int64_t chunk = (512 + nkt - 1) / nkt;
  if (chunk < (int64_t)g.OB * g.OH) chunk = (int64_t)g.OB * g.OH;
  if (chunk > pairs) chunk = pairs;
  g.chunk = (int)chunk;
  const size_t slot = (size_t)g.LQ * (size_t)d->Lk * sizeof(float);
  g.acc_bytes = g.reduce ? (size_t)g.OB * g.OH * slot : 0;
  g.partial_bytes = g.reduce ? (size_t)chunk * slot : 0;
  return g;
}

struct WsLayout {
  size_t tilemap, order, delta, acc, partial, total;
};

// flags: NXA_WS_BWD (bit 0) sizes the backward's per-row values, and
// NXA_WS_DBIAS (bit 1) its dbias reduction buffers.
WsLayout ws_layout(const nxa_desc* d, int has_bias, int has_mask, int flags) {
  WsLayout w{0, 0, 0, 0, 0, 0};
  size_t off = 0;
  if (has_mask) {
    const MaskGeom m = mask_geom(d);
    w.tilemap = off;
    off += align256(m.bytes);
    w.order = off;
    off += align256(m.order_bytes);
  }
  if (flags & NXA_WS_BWD) {
    w.delta = off;  // -delta[B*H*Lq], then -lse2[B*H*Lq]
    off += 2 * align256((size_t)d->B * d->H * d->Lq * sizeof(float));
    if (has_bias && (flags & NXA_WS_DBIAS)) {
      const DbiasGeom g = dbias_geom(d);
      w.acc = off;
      off += align256(g.acc_bytes);
      w.partial = off;
      off += align256(g.partial_bytes);
    }
  }
  w.total = off;
  return w;
}

// Round to the nearest bf16 (ties to even), returned as a float.
float round_bf16(float x) {
  uint32_t u;
  std::memcpy(&u, &x, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  u &= 0xffff0000u;
  float r;
  std::memcpy(&r, &u, 4);
  return r;
}

// Round to the nearest fp16 (ties to even), returned as a float: 10 fraction
// bits in the normal range, multiples of 2^-24 below 2^-14 (subnormals), inf
// from 65520 up.
float round_f16(float x) {
  if (!std::isfinite(x)) return x;
  if (std::fabs(x) >= 65520.f) return std::copysign(INFINITY, x);
  if (std::fabs(x) < 6.103515625e-05f)
    return std::nearbyint(x * 16777216.f) / 16777216.f;
  uint32_t u;
  std::memcpy(&u, &x, 4);
  u += 0xfffu + ((u >> 13) & 1u);
  u &= 0xffffe000u;
  float r;
  std::memcpy(&r, &u, 4);
  return r;
}

// Chooses how the 16-bit forward adds the bias (nxa::FwdBias).  The MFMA
// modes need a bias of the I/O dtype whose rows are 16-byte aligned whole
// 8-key chunks, and a positive scale whose reciprocal splits into two normal
// terms h + l of that dtype.
int fwd_bias_mode(const nxa_desc* d, const void* bias, float* h, float* l) {
  *h = *l = 0.f;
  if (d->io_dtype == NXA_F32 || d->bias_dtype != d->io_dtype) return nxa::kFbValu;
  if (!(d->scale > 0.f) || !std::isfinite(d->scale)) return nxa::kFbValu;
  const bool f16 = d->io_dtype == NXA_F16;
  // Smallest normal and largest finite value of the dtype.
  const float tiny = f16 ? 6.103515625e-05f : 1e-30f;
  const float huge = f16 ? 65504.f : 1e30f;
  const float inv = 1.0f / d->scale;
  const float hi = f16 ? round_f16(inv) : round_bf16(inv);
  const float lo = f16 ? round_f16(inv - hi) : round_bf16(inv - hi);
  if (!std::isfinite(hi) || !(std::fabs(hi) >= tiny) || !(std::fabs(hi) <= huge))
    return nxa::kFbValu;
  if (lo != 0.f && !(std::fabs(lo) >= tiny)) return nxa::kFbValu;
  if (d->Lk % 8 != 0 || !aligned(bias, 16) || d->bias_str[0] % 8 != 0 ||
      d->bias_str[1] % 8 != 0)
    return nxa::kFbValu;
  *h = hi;
  *l = lo;
  if (d->bias_str[2] == 0 || d->Lq == 1) return nxa::kFbRow;
  if (d->bias_str[2] % 8 != 0) return nxa::kFbValu;
  return nxa::kFbTile;
}

nxa::Params base_params(const nxa_desc* d, const void* q, const void* k,
                        const void* v, const void* bias, const uint8_t* mask) {
  nxa::Params p;
  std::memset(&p, 0, sizeof(p));
  p.q = q;
  p.k = k;
  p.v = v;
  p.bias = bias;
  p.mask = mask;
  for (int i = 0; i < 3; ++i) {
    p.q_str[i] = d->q_str[i];
    p.k_str[i] = d->k_str[i];
    p.v_str[i] = d->v_str[i];
    p.o_str[i] = d->o_str[i];
    p.bias_str[i] = bias ? d->bias_str[i] : 0;
    p.mask_str[i] = mask ? d->mask_str[i] : 0;
  }
  p.B = d->B;
  p.H = d->H;
  p.bh0 = 0;
  p.nbh = d->B * d->H;
  p.Lq = d->Lq;
  p.Lk = d->Lk;
  p.D = d->D;
  p.Dv = value_dim(d);
  p.scale = d->scale;
  p.scale_log2 = d->scale * nxa::kLog2e;
  p.causal = d->causal ? 1 : 0;
  p.has_bias = bias != nullptr;
  p.bias_dtype = d->bias_dtype;
  if (bias) {
    const int bes = esize(d->bias_dtype);
    bool vec = (d->Lk % 4 == 0) && aligned(bias, 4 * bes);
    for (int i = 0; i < 3; ++i) vec = vec && (d->bias_str[i] % 4 == 0);
    p.bias_vec = vec;
  }
  p.fwd_bias = bias ? fwd_bias_mode(d, bias, &p.bias_h, &p.bias_l) : nxa::kFbNone;
  p.has_mask = mask != nullptr;
  if (mask) {
    bool vec = (d->Lk % 4 == 0) && aligned(mask, 4);
    for (int i = 0; i < 3; ++i) vec = vec && (d->mask_str[i] % 4 == 0);
    p.mask_vec = vec;
  }
  return p;
}

// Writes (or just binds) the tile map for `mask`, and the block order when
// the mask takes one, into the workspace (`ws` its base).
int setup_tilemap(nxa::Params& p, const nxa_desc* d, uint8_t* ws, bool build,
                  hipStream_t stream) {
  const MaskGeom m = mask_geom(d);
  const WsLayout w = ws_layout(d, 0, 1, 0);
  uint8_t* tm = ws + w.tilemap;
  p.has_tilemap = 1;
  p.tilemap = tm;
  p.tilemap_out = tm;
  p.tm_rows = m.rows;
  p.tm_nk = m.MK;
  p.tm_str[0] = m.MB > 1 ? (int64_t)m.MH * m.MQ * m.MK : 0;
  p.tm_str[1] = m.MH > 1 ? (int64_t)m.MQ * m.MK : 0;
  p.tm_str[2] = m.MQ > 1 ? m.MK : 0;
  int* order = reinterpret_cast<int*>(ws + w.order);
  if (m.order) {
    const int64_t ps = (int64_t)m.nq2 + m.nq4 + m.nk2;
    p.order = order;
    p.ord_str[0] = m.MB > 1 ? m.MH * ps : 0;
    p.ord_str[1] = m.MH > 1 ? ps : 0;
    p.ord_q128 = 0;
    p.ord_q256 = m.nq2;
    p.ord_k128 = m.nq2 + m.nq4;
  }
  if (!build) return NXA_OK;
  bool vec16 = aligned(p.mask, 16);
  for (int i = 0; i < 3; ++i) vec16 = vec16 && (p.mask_str[i] % 16 == 0);
  if (m.bytes >= ((size_t)1 << 31))
    return fail(NXA_E_SHAPE, "mask tile map has %zu tiles (limit 2^31)", m.bytes);
  int rc = launch("tilemap", stream, [&] {
    nxa::launch_tilemap(p, m.MB, m.MH, m.MQ, m.MK, vec16 ? 1 : 0, stream);
  });
  if (rc || !m.order) return rc;
  const int tm16 = m.MK % 16 == 0 && aligned(tm, 16);
  return launch("tile_order", stream, [&] {
    nxa::launch_tile_order(tm, m.MB * m.MH, m.MQ, m.MK, tm16, order, stream);
  });
}

int check_io_ptrs(const nxa_desc* d, const void* const* ptrs, const char* const* names,
                  int n) {
  for (int i = 0; i < n; ++i) {
    if (!ptrs[i]) return fail(NXA_E_ARG, "%s is NULL", names[i]);
    if (!aligned(ptrs[i], 16))
      return fail(NXA_E_LAYOUT, "%s is not 16-byte aligned", names[i]);
  }
  (void)d;
  return NXA_OK;
}

// Validation of the qk-norm entry points.
int check_norm(int64_t rows, int32_t D, int32_t dtype, const void* x, int64_t x_stride,
               const void* const* ptrs, const char* const* names, int n) {
  if (!known_dtype(dtype))
    return fail(NXA_E_DTYPE, "dtype %d is not NXA_BF16, NXA_F16 or NXA_F32", dtype);
  if (rows <= 0 || D <= 0)
    return fail(NXA_E_SHAPE, "rms norm needs rows > 0 and D > 0 (rows=%lld D=%d)",
                (long long)rows, D);
  if (rows > ((int64_t)1 << 31) * 16)
    return fail(NXA_E_SHAPE, "rms norm: %lld rows exceed the grid", (long long)rows);
  const int epc = 16 / esize(dtype);
  if (D % epc != 0)
    return fail(NXA_E_UNSUPPORTED, "rms norm: D=%d must be a multiple of %d", D, epc);
  if (D > 256)
    return fail(NXA_E_UNSUPPORTED, "rms norm: D=%d exceeds 256 (rows are held in registers)", D);
  if (x_stride < D || x_stride % epc != 0)
    return fail(NXA_E_LAYOUT, "rms norm: row stride %lld must be >= D and a multiple of %d",
                (long long)x_stride, epc);
  if (!x) return fail(NXA_E_ARG, "x is NULL");
  if (!aligned(x, 16)) return fail(NXA_E_LAYOUT, "x is not 16-byte aligned");
  for (int i = 0; i < n; ++i) {
    if (!ptrs[i]) return fail(NXA_E_ARG, "%s is NULL", names[i]);
    if (!aligned(ptrs[i], 16)) return fail(NXA_E_LAYOUT, "%s is not 16-byte aligned", names[i]);
  }
  return NXA_OK;
}

// Selective scan: extents, limits and workspace layout.
constexpr int kSsmMaxStates = 32;

struct SsmLayout {
  int NP, nc, ns, ndblk, ndblk_b;
  size_t hc, sdt, gc, dD, dBC, dad;  // byte sizes of the workspace parts
  size_t state;                 // byte size of the saved sub-chunk states
};

SsmLayout ssm_layout(int64_t nb, int32_t L, int32_t Dm, int32_t N) {
  SsmLayout s;
  s.NP = nxa::ssm_padded_states(N);
  s.nc = (L + nxa::kSsmChunk - 1) / nxa::kSsmChunk;
  s.ns = (L + nxa::kSsmSub - 1) / nxa::kSsmSub;
  s.ndblk = (Dm + nxa::kSsmBlock - 1) / nxa::kSsmBlock;
  const int cpb = nxa::kSsmBlock / nxa::ssm_lanes_per_channel(s.NP);
  s.ndblk_b = (Dm + cpb - 1) / cpb;
  const size_t f = sizeof(float);
  s.hc = align256((size_t)nb * s.nc * s.NP * Dm * f);
  s.gc = s.hc;
  s.sdt = align256((size_t)nb * s.nc * Dm * f);
  s.dD = s.sdt;
  s.dBC = align256((size_t)s.ndblk_b * nb * L * 2 * s.NP * f);
  s.dad = align256((size_t)nxa::kSsmDadGroups * (s.NP + 1) * Dm * f);
  s.state = (size_t)nb * s.ns * s.NP * Dm * f;
  return s;
}

int check_ssm(int64_t nb, int32_t L, int32_t Dm, int32_t N) {
  if (nb <= 0 || L <= 0 || Dm <= 0 || N <= 0)
    return fail(NXA_E_SHAPE, "selective scan: extents must be positive (nb=%lld L=%d d=%d n=%d)",
                (long long)nb, L, Dm, N);
  if (N > kSsmMaxStates)
    return fail(NXA_E_UNSUPPORTED, "selective scan: state dim n=%d exceeds %d", N,
                kSsmMaxStates);
  const SsmLayout s = ssm_layout(nb, L, Dm, N);
  // Grids: chunk passes ndblk * nc * nb blocks, carry nb * NP * Dm / 256,
  // dB / dC reduction nb * L * 2 NP / 256; all below 2^31.
  if ((int64_t)s.ndblk_b * s.nc * nb >= ((int64_t)1 << 31) ||
      nb * s.NP * (int64_t)Dm >= ((int64_t)1 << 38) ||
      nb * (int64_t)L * 2 * s.NP >= ((int64_t)1 << 38))
    return fail(NXA_E_SHAPE, "selective scan: nb=%lld L=%d d=%d exceed the grid",
                (long long)nb, L, Dm);
  return NXA_OK;
}

int check_ptrs(const void* const* ptrs, const char* const* names, int n) {
  for (int i = 0; i < n; ++i) {
    if (!ptrs[i]) return fail(NXA_E_ARG, "selective scan: %s is NULL", names[i]);
    if (!aligned(ptrs[i], 4))
      return fail(NXA_E_LAYOUT, "selective scan: %s is not 4-byte aligned", names[i]);
  }
  return NXA_OK;
}

// Validation shared by the forward entry points.
int check_fwd(const nxa_desc* d, const void* q, const void* k, const void* v,
              const void* bias, const uint8_t* mask, const void* o) {
  int rc = check_desc(d, bias != nullptr, mask != nullptr);
  if (rc) return rc;
  const void* ptrs[4] = {q, k, v, o};
  const char* names[4] = {"q", "k", "v", "o"};
  return check_io_ptrs(d, ptrs, names, 4);
}

// qk-norm of q fused into the forward (nxa_fwd_normed).
struct FwdNorm {
  void* q_hat;
  float* q_rstd;
  float eps;
};

int run_fwd(const nxa_desc* d, const void* q, const void* k, const void* v,
            const void* bias, const uint8_t* mask, void* o, float* lse,
            void* workspace, void* stream_, const FwdNorm* fn = nullptr);

// ---------------------------------------------------------------------------
// Static scratch of nxa_fwd_noalloc: a device array that every GPU the
// library runs on holds for the life of the process.  In host code `scratch`
// names a host-side stand-in, not device memory: its device address is looked
// up once per device (hipGetSymbolAddress, with that device current) and only
// that address is handed to kernels.
// ---------------------------------------------------------------------------
constexpr size_t kScratchBytes = NXA_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;
__device__ __align__(256) uint8_t scratch[kScratchBytes];
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device.
int device_scratch(void** out) {
  int dev = -1;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return fail(NXA_E_LAUNCH, "nxa_fwd_noalloc: hipGetDevice failed: %s",
                hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(NXA_E_ARG, "nxa_fwd_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t r = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (r != hipSuccess || !p)
      return fail(NXA_E_LAUNCH, "nxa_fwd_noalloc: hipGetSymbolAddress(scratch) failed: %s",
                  hipGetErrorString(r));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return NXA_OK;
}

}  // namespace

extern "C" {

int nxa_version(void) { return NXA_VERSION; }

const char* nxa_last_error(void) { return g_err.c_str(); }

int nxa_check(const nxa_desc* desc, int has_bias, int has_mask) {
  return check_desc(desc, has_bias, has_mask);
}

size_t nxa_workspace_bytes(const nxa_desc* desc, int has_bias, int has_mask,
                           int flags) {
  if (check_desc(desc, has_bias, has_mask) != NXA_OK) return 0;
  if (flags & ~(NXA_WS_BWD | NXA_WS_DBIAS)) {
    fail(NXA_E_ARG, "workspace flags %d: only NXA_WS_BWD | NXA_WS_DBIAS", flags);
    return 0;
  }
  return ws_layout(desc, has_bias, has_mask, flags).total;
}

int nxa_fwd(const nxa_desc* d, const void* q, const void* k, const void* v,
            const void* bias, const uint8_t* mask, void* o, float* lse,
            void* workspace, size_t workspace_bytes, void* stream_) {
  int rc = check_fwd(d, q, k, v, bias, mask, o);
  if (rc) return rc;
  const WsLayout ws = ws_layout(d, bias != nullptr, mask != nullptr, 0);
  if (ws.total > 0 && (!workspace || workspace_bytes < ws.total))
    return fail(NXA_E_WORKSPACE, "forward needs %zu workspace bytes, got %zu",
                ws.total, workspace ? workspace_bytes : (size_t)0);
  return run_fwd(d, q, k, v, bias, mask, o, lse, workspace, stream_);
}

int nxa_fwd_normed(const nxa_desc* d, const void* q, const void* k_hat, const void* v,
                   const void* bias, const uint8_t* mask, void* o, float* lse,
                   void* q_hat, float* q_rstd, float eps, void* workspace,
                   size_t workspace_bytes, void* stream_) {
  int rc = check_fwd(d, q, k_hat, v, bias, mask, o);
  if (rc) return rc;
  if (d->io_dtype != NXA_BF16 && d->io_dtype != NXA_F16)
    return fail(NXA_E_UNSUPPORTED,
                "nxa_fwd_normed: bf16 / fp16 I/O only (fp32: nxa_rms_norm_fwd, then nxa_fwd)");
  if ((d->q_str[0] == 0 && d->B > 1) || (d->q_str[1] == 0 && d->H > 1))
    return fail(NXA_E_UNSUPPORTED,
                "nxa_fwd_normed: q broadcast over batch or heads (normalise it with "
                "nxa_rms_norm_fwd, then nxa_fwd)");
  if (q_hat && !aligned(q_hat, 16)) return fail(NXA_E_LAYOUT, "q_hat is not 16-byte aligned");
  if (!(eps >= 0.f)) return fail(NXA_E_ARG, "nxa_fwd_normed: eps must be >= 0");
  const WsLayout ws = ws_layout(d, bias != nullptr, mask != nullptr, 0);
  if (ws.total > 0 && (!workspace || workspace_bytes < ws.total))
    return fail(NXA_E_WORKSPACE, "forward needs %zu workspace bytes, got %zu",
                ws.total, workspace ? workspace_bytes : (size_t)0);
  const FwdNorm fn{q_hat, q_rstd, eps};
  return run_fwd(d, q, k_hat, v, bias, mask, o, lse, workspace, stream_, &fn);
}

int nxa_fwd_noalloc(const nxa_desc* d, const void* q, const void* k, const void* v,
                    const void* bias, const uint8_t* mask, void* o, float* lse,
                    void* stream_) {
  int rc = check_fwd(d, q, k, v, bias, mask, o);
  if (rc) return rc;
  const WsLayout ws = ws_layout(d, bias != nullptr, mask != nullptr, 0);
  if (ws.total > kScratchBytes)
    return fail(NXA_E_WORKSPACE,
                "nxa_fwd_noalloc: the mask's tile map needs %zu bytes, the static "
                "scratch holds %zu; use nxa_fwd with a workspace",
                ws.total, kScratchBytes);
  void* scratch_ptr = nullptr;
  if (ws.total > 0 && (rc = device_scratch(&scratch_ptr))) return rc;
  return run_fwd(d, q, k, v, bias, mask, o, lse, scratch_ptr, stream_);
}

}  // extern "C"

namespace {

// The forward after validation: tile map into `workspace` (when there is a
// mask), then the forward kernel.
int run_fwd(const nxa_desc* d, const void* q, const void* k, const void* v,
            const void* bias, const uint8_t* mask, void* o, float* lse,
            void* workspace, void* stream_, const FwdNorm* fn) {
  int rc;
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  nxa::Params p = base_params(d, q, k, v, bias, mask);
  p.o = o;
  p.lse = lse;
  if (fn) {
    p.qn_on = 1;
    p.qn_out = fn->q_hat;
    p.qn_rstd = fn->q_rstd;
    p.qn_eps = fn->eps;
  }
  if (mask) {
    rc = setup_tilemap(p, d, static_cast<uint8_t*>(workspace), true, stream);
    if (rc) return rc;
  }
  const int dp = padded_dim(d);
  return launch("fwd", stream, [&] { nxa::launch_fwd(p, d->io_dtype, dp, stream); });
}

}  // namespace

extern "C" {

}  // extern "C"

namespace {

// Raw (pre-norm) q / k and their per-row rsqrt for the fused qk-norm VJP.
struct NormArgs {
  const void* q;
  const void* k;
  const float* q_rstd;
  const float* k_rstd;
};

int run_bwd(const nxa_desc* d, const void* q, const void* k, const void* v,
            const void* bias, const uint8_t* mask, const void* o,
            const float* lse, const void* dout, void* dq, void* dk, void* dv,
            void* dbias, const int64_t* dbias_str, void* workspace,
            size_t workspace_bytes, int tilemap_ready, void* stream_,
            const NormArgs* na) {
  int rc = check_desc(d, bias != nullptr, mask != nullptr);
  if (rc) return rc;
  const void* ptrs[8] = {q, k, v, o, dout, dq, dk, dv};
  const char* names[8] = {"q", "k", "v", "o", "dout", "dq", "dk", "dv"};
  if ((rc = check_io_ptrs(d, ptrs, names, 8))) return rc;
  if (!lse) return fail(NXA_E_ARG, "lse is NULL");
  if (dbias && !bias) return fail(NXA_E_ARG, "dbias requested without a bias");
  if (dbias && !dbias_str) return fail(NXA_E_ARG, "dbias_str is NULL");
  // dK / dV are written once per (b, h): broadcast k / v cannot take them.
  for (int i = 0; i < 2; ++i) {
    const int ext = i == 0 ? d->B : d->H;
    if (ext > 1 && (d->k_str[i] == 0 || d->v_str[i] == 0))
      return fail(NXA_E_UNSUPPORTED,
                  "backward needs k / v materialised over axis %d (stride 0)", i);
    if (ext > 1 && d->q_str[i] == 0)
      return fail(NXA_E_UNSUPPORTED,
                  "backward needs q materialised over axis %d (stride 0)", i);
  }
  const WsLayout ws = ws_layout(d, bias != nullptr, mask != nullptr,
                                NXA_WS_BWD | (dbias ? NXA_WS_DBIAS : 0));
  if (!workspace || workspace_bytes < ws.total)
    return fail(NXA_E_WORKSPACE, "backward needs %zu workspace bytes, got %zu",
                ws.total, workspace ? workspace_bytes : (size_t)0);
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  uint8_t* wsb = static_cast<uint8_t*>(workspace);
  nxa::Params p = base_params(d, q, k, v, bias, mask);
  p.o = const_cast<void*>(o);
  p.lse = const_cast<float*>(lse);
  p.dout = dout;
  p.dq = dq;
  p.dk = dk;
  p.dv = dv;
  p.ndelta = reinterpret_cast<float*>(wsb + ws.delta);
  p.nlse2 = reinterpret_cast<float*>(
      wsb + ws.delta + align256((size_t)d->B * d->H * d->Lq * sizeof(float)));
  // 16-bit I/O: the dQ kernel computes -delta and -lse * log2(e) for its own
  // rows and runs first; the fp32 kernels have a pass of its own.
  const bool dq_first = d->io_dtype != NXA_F32;
  if (na) {
    if (!dq_first)
      return fail(NXA_E_UNSUPPORTED, "fused qk-norm backward needs bf16 / fp16 I/O");
    const void* nptrs[4] = {na->q, na->k, na->q_rstd, na->k_rstd};
    const char* nnames[4] = {"q (raw)", "k (raw)", "q_rstd", "k_rstd"};
    if ((rc = check_io_ptrs(d, nptrs, nnames, 2))) return rc;
    for (int i = 2; i < 4; ++i)
      if (!nptrs[i]) return fail(NXA_E_ARG, "%s is NULL", nnames[i]);
    for (int i = 0; i < 2; ++i)
      if (d->q_str[i] == 0 || d->k_str[i] == 0)
        return fail(NXA_E_UNSUPPORTED,
                    "fused qk-norm backward needs q and k materialised over axis %d", i);
    p.qk_norm = 1;
    p.qraw = na->q;
    p.kraw = na->k;
    p.qrstd = na->q_rstd;
    p.krstd = na->k_rstd;
  }
  if (!dq_first && (rc = launch("delta", stream,
                               [&] { nxa::launch_delta(p, d->io_dtype, stream); })))
    return rc;
  if (mask) {
    rc = setup_tilemap(p, d, wsb, !tilemap_ready, stream);
    if (rc) return rc;
  }
  DbiasGeom dg{};
  if (dbias) {
    dg = dbias_geom(d);
    p.dbias_mode = dg.mode;
    if (dg.reduce) {
      // Partials of one chunk of pairs, slot = pair - bh0 (dbias_off).
      p.dbias = wsb + ws.partial;
      p.dbias_f32 = 1;
      p.dbias_str[0] = (int64_t)d->H * dg.LQ * d->Lk;
      p.dbias_str[1] = (int64_t)dg.LQ * d->Lk;
      p.dbias_str[2] = dg.mode == nxa::kDbiasFull ? d->Lk : 0;
    } else {
      p.dbias = dbias;
      for (int i = 0; i < 3; ++i) p.dbias_str[i] = dbias_str[i];
    }
  }
  const int dp = padded_dim(d);
  if (dq_first &&
      (rc = launch("dq", stream, [&] { nxa::launch_dq(p, d->io_dtype, dp, stream); })))
    return rc;
  if (!(dbias && dg.reduce)) {
    if ((rc = launch("dkdv", stream,
                     [&] { nxa::launch_dkdv(p, d->io_dtype, dp, stream); })))
      return rc;
  } else {
    const int pairs = d->B * d->H;
    nxa::DbiasReduce r{};
    r.part = reinterpret_cast<const float*>(wsb + ws.partial);
    r.acc = reinterpret_cast<float*>(wsb + ws.acc);
    r.out = dbias;
    for (int i = 0; i < 3; ++i) r.s[i] = dbias_str[i];
    r.B = d->B;
    r.H = d->H;
    r.OB = dg.OB;
    r.OH = dg.OH;
    r.LQ = dg.LQ;
    r.Lk = d->Lk;
    r.dtype = d->bias_dtype;
    for (int bh0 = 0; bh0 < pairs; bh0 += dg.chunk) {
      p.bh0 = bh0;
      p.nbh = pairs - bh0 < dg.chunk ? pairs - bh0 : dg.chunk;
      p.dbias_off = (int64_t)bh0 * dg.LQ * d->Lk;
      if ((rc = launch("dkdv", stream,
                       [&] { nxa::launch_dkdv(p, d->io_dtype, dp, stream); })))
        return rc;
      r.bh0 = p.bh0;
      r.nbh = p.nbh;
      r.first = bh0 == 0;
      r.last = bh0 + p.nbh == pairs;
      if ((rc = launch("dbias_reduce", stream,
                       [&] { nxa::launch_dbias_reduce(r, stream); })))
        return rc;
    }
  }
  if (!dq_first &&
      (rc = launch("dq", stream, [&] { nxa::launch_dq(p, d->io_dtype, dp, stream); })))
    return rc;
  return NXA_OK;
}

}  // namespace

extern "C" {

int nxa_bwd(const nxa_desc* d, const void* q, const void* k, const void* v,
            const void* bias, const uint8_t* mask, const void* o,
            const float* lse, const void* dout, void* dq, void* dk, void* dv,
            void* dbias, const int64_t* dbias_str, void* workspace,
            size_t workspace_bytes, int tilemap_ready, void* stream) {
  return run_bwd(d, q, k, v, bias, mask, o, lse, dout, dq, dk, dv, dbias, dbias_str,
                 workspace, workspace_bytes, tilemap_ready, stream, nullptr);
}

int nxa_bwd_normed(const nxa_desc* d, const void* q_hat, const void* k_hat,
                   const void* v, const void* bias, const uint8_t* mask, const void* o,
                   const float* lse, const void* dout, const void* q, const void* k,
                   const float* q_rstd, const float* k_rstd, void* dq, void* dk, void* dv,
                   void* dbias, const int64_t* dbias_str, void* workspace,
                   size_t workspace_bytes, int tilemap_ready, void* stream) {
  const NormArgs na{q, k, q_rstd, k_rstd};
  return run_bwd(d, q_hat, k_hat, v, bias, mask, o, lse, dout, dq, dk, dv, dbias,
                 dbias_str, workspace, workspace_bytes, tilemap_ready, stream, &na);
}

int nxa_rms_norm_fwd(int64_t rows, int32_t D, int32_t dtype, const void* x,
                     int64_t x_stride, void* y, float* rstd, float eps, void* stream) {
  const void* ptrs[1] = {y};
  const char* names[1] = {"y"};
  int rc = check_norm(rows, D, dtype, x, x_stride, ptrs, names, 1);
  if (rc) return rc;
  if (!(eps >= 0.f)) return fail(NXA_E_ARG, "rms norm: eps must be >= 0");
  nxa::NormParams p{};
  p.x = x;
  p.y = y;
  p.rstd = rstd;
  p.rows = rows;
  p.x_stride = x_stride;
  p.D = D;
  p.eps = eps;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  return launch("rms_norm_fwd", s, [&] { nxa::launch_rms_norm(p, dtype, false, s); });
}

int nxa_rms_norm_bwd(int64_t rows, int32_t D, int32_t dtype, const void* x,
                     int64_t x_stride, const void* dy, const float* rstd, void* dx,
                     void* stream) {
  const void* ptrs[3] = {dy, rstd, dx};
  const char* names[3] = {"dy", "rstd", "dx"};
  int rc = check_norm(rows, D, dtype, x, x_stride, ptrs, names, 3);
  if (rc) return rc;
  nxa::NormParams p{};
  p.x = x;
  p.rstd = const_cast<float*>(rstd);
  p.dy = dy;
  p.dx = dx;
  p.rows = rows;
  p.x_stride = x_stride;
  p.D = D;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  return launch("rms_norm_bwd", s, [&] { nxa::launch_rms_norm(p, dtype, true, s); });
}

int nxa_ssm_check(int64_t nb, int32_t L, int32_t d, int32_t n) {
  return check_ssm(nb, L, d, n);
}

size_t nxa_ssm_state_bytes(int64_t nb, int32_t L, int32_t d, int32_t n) {
  if (check_ssm(nb, L, d, n)) return 0;
  return ssm_layout(nb, L, d, n).state;
}

size_t nxa_ssm_workspace_bytes(int64_t nb, int32_t L, int32_t d, int32_t n, int is_bwd) {
  if (check_ssm(nb, L, d, n)) return 0;
  const SsmLayout s = ssm_layout(nb, L, d, n);
  return is_bwd ? s.gc + s.sdt + s.dD + s.dBC + s.dad : s.hc + s.sdt;
}

int nxa_ssm_fwd(int64_t nb, int32_t L, int32_t d, int32_t n, const float* x,
                const float* delta, const float* A, const float* B, const float* C,
                const float* D, float* y, float* state, void* workspace,
                size_t workspace_bytes, void* stream) {
  int rc = check_ssm(nb, L, d, n);
  if (rc) return rc;
  const void* ptrs[7] = {x, delta, A, B, C, y, workspace};
  const char* names[7] = {"x", "delta", "A", "B", "C", "y", "workspace"};
  if ((rc = check_ptrs(ptrs, names, 7))) return rc;
  if ((D && !aligned(D, 4)) || (state && !aligned(state, 4)))
    return fail(NXA_E_LAYOUT, "selective scan: D / state not 4-byte aligned");
  const SsmLayout s = ssm_layout(nb, L, d, n);
  if (workspace_bytes < s.hc + s.sdt || !aligned(workspace, 256))
    return fail(NXA_E_WORKSPACE, "selective scan: workspace needs %zu bytes, 256-byte aligned",
                s.hc + s.sdt);
  nxa::SsmParams p{};
  p.x = x;
  p.delta = delta;
  p.A = A;
  p.B = B;
  p.C = C;
  p.D = D;
  p.y = y;
  p.hs = state;
  char* ws = static_cast<char*>(workspace);
  p.hc = reinterpret_cast<float*>(ws);
  p.sdt = reinterpret_cast<float*>(ws + s.hc);
  p.nb = nb;
  p.L = L;
  p.Dm = d;
  p.N = n;
  p.nc = s.nc;
  p.ns = s.ns;
  p.ndblk = s.ndblk;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  return launch("ssm_fwd", st, [&] { nxa::launch_ssm(p, false, st); });
}

int nxa_ssm_bwd(int64_t nb, int32_t L, int32_t d, int32_t n, const float* x,
                const float* delta, const float* A, const float* B, const float* C,
                const float* D, const float* state, const float* dy, float* dx,
                float* ddelta, float* dA, float* dB, float* dC, float* dD,
                void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_ssm(nb, L, d, n);
  if (rc) return rc;
  const void* ptrs[13] = {x, delta, A, B, C, state, dy, dx, ddelta, dA, dB, dC, workspace};
  const char* names[13] = {"x", "delta", "A", "B", "C", "state", "dy",
                           "dx", "ddelta", "dA", "dB", "dC", "workspace"};
  if ((rc = check_ptrs(ptrs, names, 13))) return rc;
  if ((D && !aligned(D, 4)) || (dD && !aligned(dD, 4)))
    return fail(NXA_E_LAYOUT, "selective scan: D / dD not 4-byte aligned");
  const SsmLayout s = ssm_layout(nb, L, d, n);
  const size_t need = s.gc + s.sdt + s.dD + s.dBC + s.dad;
  if (workspace_bytes < need || !aligned(workspace, 256))
    return fail(NXA_E_WORKSPACE, "selective scan: workspace needs %zu bytes, 256-byte aligned",
                need);
  nxa::SsmParams p{};
  p.x = x;
  p.delta = delta;
  p.A = A;
  p.B = B;
  p.C = C;
  p.D = D;
  p.hs = const_cast<float*>(state);
  p.dy = dy;
  p.dx = dx;
  p.ddelta = ddelta;
  p.dA = dA;
  p.dB = dB;
  p.dC = dC;
  p.dD = D ? dD : nullptr;
  char* ws = static_cast<char*>(workspace);
  p.gc = reinterpret_cast<float*>(ws);
  p.sdt = reinterpret_cast<float*>(ws + s.gc);
  p.dDpart = reinterpret_cast<float*>(ws + s.gc + s.sdt);
  p.dBCpart = reinterpret_cast<float*>(ws + s.gc + s.sdt + s.dD);
  p.dadpart = reinterpret_cast<float*>(ws + s.gc + s.sdt + s.dD + s.dBC);
  p.nb = nb;
  p.L = L;
  p.Dm = d;
  p.N = n;
  p.nc = s.nc;
  p.ns = s.ns;
  p.ndblk = s.ndblk;
  p.ndblk_b = s.ndblk_b;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  return launch("ssm_bwd", st, [&] { nxa::launch_ssm(p, true, st); });
}

int nxa_profile_enable(int on) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  g_prof_on = on != 0;
  return NXA_OK;
}

int nxa_profile_read(const char* kernel, double* total_ms, int64_t* launches) {
  if (!kernel || !total_ms || !launches)
    return fail(NXA_E_ARG, "nxa_profile_read: NULL argument");
  std::lock_guard<std::mutex> lk(g_prof_mu);
  double tot = 0.0;
  int64_t n = 0;
  const size_t kl = std::strlen(kernel);
  for (auto& r : g_prof) {
    if (r.name.compare(0, kl, kernel) != 0) continue;
    if (hipEventSynchronize(r.stop) != hipSuccess)
      return fail(NXA_E_LAUNCH, "nxa_profile_read: event wait failed");
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, r.start, r.stop) != hipSuccess)
      return fail(NXA_E_LAUNCH, "nxa_profile_read: elapsed time failed");
    tot += ms;
    ++n;
  }
  *total_ms = tot;
  *launches = n;
  return NXA_OK;
}

int nxa_profile_reset(void) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  for (auto& r : g_prof) {
    hipEventDestroy(r.start);
    hipEventDestroy(r.stop);
  }
  g_prof.clear();
  return NXA_OK;
}

}  // extern "C"
