/*
 * nxattn -- fused scaled-dot-product attention (additive bias, boolean
 * keep-mask, causal) for AMD Instinct MI355X (gfx950), C ABI.
 *
 * Drop-in boundary for nitrix's fused attention path.  The reference binds
 * its fused kernel at
 *   src/nitrix/nn/attention/__init__.py:63-123   (_attention_pallas, the
 *                                                 dispatcher's call site)
 *   src/nitrix/_kernels/cuda/attention.py:768-824 (scaled_dot_product_attention_pallas)
 * and the entry points below replace, one for one, the pieces behind it:
 *
 *   nxa_check            <- _check_tileable           attention.py:708-765
 *   nxa_fwd              <- _fused_forward_with_lse   attention.py:547-584
 *                           + _mha_forward / nitrix_mha_forward
 *                                                     attention.py:159-264, 85-156
 *   nxa_bwd              <- _fused_backward           attention.py:600-653
 *                           + _mha_backward / nitrix_mha_backward_kv, _q
 *                                                     attention.py:390-499, 272-387
 *                           + _unbroadcast (dbias)    attention.py:517-544
 *   nxa_workspace_bytes  <- (XLA temp buffers of the broadcast_to / transpose
 *                           glue at attention.py:560-569, 616-633; here a
 *                           small caller-owned workspace instead)
 *
 * Conventions
 *   - Every tensor is [B, H, L, D] (leading batch axes pre-flattened into B)
 *     with unit stride over D.  Strides are in elements; the D stride is not
 *     passed.  dO / dQ / dK / dV share the strides of O / Q / K / V.
 *   - bias and mask are [B, H, Lq, Lk] with unit stride over Lk; a zero
 *     stride broadcasts that axis (the reference's right-aligned
 *     broadcast_to, without materialising it).  mask is one byte per entry,
 *     nonzero = keep.  causal keeps key j for query i iff j <= i (indices
 *     aligned at 0, also when Lq != Lk).
 *   - lse is fp32 [B, H, Lq], natural log of sum_j exp(logit_ij).  A fully
 *     masked query row yields O = NaN and lse = -inf, as the reference's
 *     softmax over all -inf logits does.
 *   - The library never allocates or frees device memory and never
 *     synchronises the stream; the caller owns every buffer.  All work is
 *     enqueued on `stream` (a hipStream_t, or NULL for the default stream).
 *   - Return value 0 on success, a negative NXA_E_* code otherwise; the
 *     message of the last failure on the calling thread is nxa_last_error().
 */
#ifndef NXATTN_H
#define NXATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NXA_VERSION 5

/* Flags of nxa_workspace_bytes. */
#define NXA_WS_FWD 0   /* the forward                                        */
#define NXA_WS_BWD 1   /* the backward                                       */
#define NXA_WS_DBIAS 2 /* with NXA_WS_BWD: a backward that writes dbias      */

typedef enum { NXA_BF16 = 0, NXA_F32 = 1, NXA_F16 = 2 } nxa_dtype;

enum {
  NXA_OK = 0,
  NXA_E_ARG = -1,         /* null descriptor / pointer, bad enum value       */
  NXA_E_SHAPE = -2,       /* non-positive or unsupported extents             */
  NXA_E_DTYPE = -3,       /* dtype outside nxa_dtype                         */
  NXA_E_LAYOUT = -4,      /* misaligned pointer or stride                    */
  NXA_E_WORKSPACE = -5,   /* workspace smaller than nxa_workspace_bytes      */
  NXA_E_LAUNCH = -6,      /* the HIP runtime rejected a kernel launch        */
  NXA_E_UNSUPPORTED = -7  /* valid request this build does not tile          */
};

/* Row strides (q_str[2], k_str[2], v_str[2], o_str[2], bias_str[2]): 64 rows
 * plus 256 elements must span less than 2^32 bytes (NXA_E_LAYOUT otherwise);
 * the kernels address a tile's rows with 32-bit offsets. */
typedef struct {
  int32_t B, H, Lq, Lk, D;  /* head dim of q, k; D <= 256, D % 8 == 0 (bf16,
                               fp16) or % 4 (fp32)                            */
  int32_t io_dtype;         /* nxa_dtype of q, k, v, o, dO, dq, dk, dv       */
  int32_t bias_dtype;       /* nxa_dtype of bias and dbias                   */
  int32_t causal;           /* nonzero: keep key j for query i iff j <= i    */
  float scale;              /* softmax scale applied to q.k                  */
  int64_t q_str[3];         /* B, H, Lq strides of q (and dq)                */
  int64_t k_str[3];         /* B, H, Lk strides of k (and dk)                */
  int64_t v_str[3];         /* B, H, Lk strides of v (and dv)                */
  int64_t o_str[3];         /* B, H, Lq strides of o (and dO)                */
  int64_t bias_str[3];      /* B, H, Lq strides of bias; 0 = broadcast       */
  int64_t mask_str[3];      /* B, H, Lq strides of mask; 0 = broadcast       */
  int32_t Dv;               /* head dim of v, o (dO, dv); 0 = D; same limits  */
} nxa_desc;

/* Library version (NXA_VERSION of the build). */
int nxa_version(void);

/* Host-only validation of a descriptor (no GPU needed).  `has_bias` and
 * `has_mask` say whether the bias / mask strides are meaningful.
 * Replaces _check_tileable (attention.py:708-765). */
int nxa_check(const nxa_desc* desc, int has_bias, int has_mask);

/* Bytes of caller-provided device workspace that nxa_fwd (flags NXA_WS_FWD)
 * or nxa_bwd (NXA_WS_BWD, or NXA_WS_BWD | NXA_WS_DBIAS when dbias is
 * requested) needs for this descriptor: the mask's tile map (one byte per
 * 64 x 64 tile of the mask's own extent) and, for 16-bit I/O without causal
 * masking when the mask varies over queries, the blocks' longest-first
 * order (three int32 lists per 64 x 64-tile slice, at most 1024 blocks
 * each; nothing beyond that), two fp32 values per query row in
 * the backward, and for dbias of a bias shared across batch or heads an fp32
 * accumulator of the bias's own extent plus one chunk of per-(batch, head)
 * partials (at most the larger of that accumulator and 256 KiB per query
 * row).  A workspace sized for the backward also serves the forward.
 * Returns 0 for an invalid descriptor or flags. */
size_t nxa_workspace_bytes(const nxa_desc* desc, int has_bias, int has_mask,
                           int flags);

/* Forward: o = softmax(scale * q k^T + bias, masked) v and its lse.
 * bias / mask may be NULL; lse may be NULL.  When mask is given, the first
 * nxa_workspace_bytes(desc, .., 0) bytes of the workspace receive the
 * tile map (and block order) that nxa_bwd can reuse (tilemap_ready = 1). */
int nxa_fwd(const nxa_desc* desc, const void* q, const void* k, const void* v,
            const void* bias, const uint8_t* mask, void* o, float* lse,
            void* workspace, size_t workspace_bytes, void* stream);

/* Forward that allocates nothing and takes no workspace.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory at all
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The same kernels and results as nxa_fwd; the mask's tile map
 * (and block order) goes to a static device array of NXA_NOALLOC_SCRATCH_BYTES
 * that every GPU the library runs on holds until the process ends.  A tile
 * map larger than that (nxa_workspace_bytes(desc, .., NXA_WS_FWD)) is
 * NXA_E_WORKSPACE, before any launch.  The scratch keeps the last call's
 * contents and is shared by every call on one GPU: calls that overlap on one
 * GPU (other streams, other threads) race, so the caller serialises them.
 * Runs on the current device. */
#define NXA_NOALLOC_SCRATCH_BYTES ((size_t)8 << 20)
int nxa_fwd_noalloc(const nxa_desc* desc, const void* q, const void* k,
                    const void* v, const void* bias, const uint8_t* mask, void* o,
                    float* lse, void* stream);

/* Backward: dq, dk, dv (and dbias if non-NULL) of sum(dO * o).
 * dbias has the extent of bias (size 1 on the axes whose bias stride is 0)
 * with strides dbias_str (B, H, Lq; unit stride over Lk); broadcast axes are
 * summed, as the reference's _unbroadcast does, in a fixed order.
 * `workspace` must hold nxa_workspace_bytes(desc, .., NXA_WS_BWD, or
 * NXA_WS_BWD | NXA_WS_DBIAS when dbias is non-NULL) bytes; when
 * tilemap_ready is nonzero its leading nxa_workspace_bytes(desc, .., 0)
 * bytes hold the tile map (and block order) written by nxa_fwd for the same
 * descriptor and mask. */
int nxa_bwd(const nxa_desc* desc, const void* q, const void* k, const void* v,
            const void* bias, const uint8_t* mask, const void* o,
            const float* lse, const void* dout, void* dq, void* dk, void* dv,
            void* dbias, const int64_t* dbias_str, void* workspace,
            size_t workspace_bytes, int tilemap_ready, void* stream);

/* Forward of attention on RMS-normalised q and k (qk-norm) with q's norm
 * fused into the kernel.  Replaces, on the fused path, qk_rms_norm(q)
 * followed by the forward kernel (nn/attention/__init__.py:196-197 with
 * _reference.py:52-77 and _kernels/cuda/attention.py:768-824): q holds the
 * raw rows (the descriptor's q strides), k_hat the normalised keys
 * (nxa_rms_norm_fwd's y); each query block normalises its stationary rows
 * in registers (y = x * rsqrt(mean(x^2) + eps) in fp32, cast to the I/O
 * dtype) and, unless they are NULL (a forward without a backward), writes
 * them to q_hat (q's strides, for the backward) and the per-row rsqrt to
 * q_rstd ([B, H, Lq] fp32).  Everything else as nxa_fwd.  bf16 / fp16 I/O
 * with q not broadcast over B or H, else NXA_E_UNSUPPORTED. */
int nxa_fwd_normed(const nxa_desc* desc, const void* q, const void* k_hat,
                   const void* v, const void* bias, const uint8_t* mask, void* o,
                   float* lse, void* q_hat, float* q_rstd, float eps, void* workspace,
                   size_t workspace_bytes, void* stream);

/* Backward of attention on RMS-normalised q and k (qk-norm) with the norm's
 * VJP fused into the dQ and dK kernels.  Replaces, on the fused path, the
 * autodiff of qk_rms_norm that the reference composes around its kernel
 * (nn/attention/__init__.py:196-197 with _reference.py:52-77).
 * q_hat / k_hat are the normalised inputs the forward ran on
 * (nxa_rms_norm_fwd's y, in the I/O dtype), q / k the inputs before the
 * norm with the same strides, q_rstd / k_rstd the per-row rsqrt from
 * nxa_rms_norm_fwd ([B, H, Lq] / [B, H, Lk] fp32, rows in the order of the
 * descriptor's B, H, L).  dq / dk receive the gradients with respect to q
 * and k (dx = r (dy - y mean(dy y)), y = x r in fp32, on the un-rounded dQ /
 * dK rows); everything else as nxa_bwd.  bf16 / fp16 I/O with q, k
 * materialised over B and H, else NXA_E_UNSUPPORTED. */
int nxa_bwd_normed(const nxa_desc* desc, const void* q_hat, const void* k_hat,
                   const void* v, const void* bias, const uint8_t* mask,
                   const void* o, const float* lse, const void* dout,
                   const void* q, const void* k, const float* q_rstd,
                   const float* k_rstd, void* dq, void* dk, void* dv, void* dbias,
                   const int64_t* dbias_str, void* workspace,
                   size_t workspace_bytes, int tilemap_ready, void* stream);

/* qk-norm: y = x * rsqrt(mean(x^2) + eps) over each row of D elements, in
 * fp32, written in `dtype` (the reference's qk_rms_norm, _reference.py:52-77,
 * which the fused path applies in the I/O dtype before the kernel,
 * nn/attention/__init__.py:196-197), with the per-row rsqrt kept in `rstd`
 * (fp32, may be NULL).  Rows of x are x_stride elements apart (unit stride
 * over D); y is [rows, D] contiguous.  D must be at most 256 (the fused
 * attention's head-dim limit) and a multiple of 8 (bf16, fp16) or 4 (fp32),
 * and the pointers 16-byte aligned.  One pass, HBM-bound. */
int nxa_rms_norm_fwd(int64_t rows, int32_t D, int32_t dtype, const void* x,
                     int64_t x_stride, void* y, float* rstd, float eps,
                     void* stream);

/* VJP of nxa_rms_norm_fwd: dx = r * (dy - y * mean(dy * y)) with r = rstd
 * and y = x * r in fp32; dy and dx are [rows, D] contiguous. */
int nxa_rms_norm_bwd(int64_t rows, int32_t D, int32_t dtype, const void* x,
                     int64_t x_stride, const void* dy, const float* rstd,
                     void* dx, void* stream);

/* Selective state-space scan (Mamba / S6), fp32.  The counterpart of the
 * fused selective scan the reference dispatches to at
 *   src/nitrix/nn/ssm/__init__.py:81-124        (_selective_scan_pallas)
 *   src/nitrix/_kernels/cuda/selective_scan.py:497-549 (selective_scan_pallas)
 * one for one:
 *   nxa_ssm_check            <- _check_tileable / _resolve_chunk  :463-494
 *   nxa_ssm_fwd              <- _fused_forward + _mha_like_forward :119-233
 *                               (y and the saved chunk-start states, hstart)
 *   nxa_ssm_bwd              <- _fused_backward + _mha_like_backward :324-419
 *                               (dx, ddelta, dA, dB, dC, dD; dA / dD summed
 *                               over the batch as the reference's partials)
 *   nxa_ssm_state_bytes,
 *   nxa_ssm_workspace_bytes  <- (XLA buffers of the reference; caller-owned
 *                               here)
 * Layout: x, delta, y, dy, dx, ddelta [nb, L, d]; B, C, dB, dC [nb, L, n];
 * A, dA [d, n]; D, dD [d]; contiguous fp32, 4-byte aligned; leading batch
 * axes pre-flattened into nb.  h_t = exp(delta_t A) h_{t-1} + delta_t B_t x_t
 * from h = 0 and y_t = C_t . h_t (+ D x_t), per (batch, channel).  Any L >= 1,
 * 1 <= n <= 32 (else NXA_E_UNSUPPORTED).  D may be NULL (no skip term; dD is
 * then not written).  `state` (nxa_ssm_state_bytes) receives the state
 * entering every 8-step sub-chunk, which nxa_ssm_bwd reads; it may be NULL
 * in nxa_ssm_fwd when no backward follows.  The workspace (256-byte aligned,
 * nxa_ssm_workspace_bytes) is scratch for one call.  dA, dB, dC, dD are
 * overwritten (not accumulated), deterministically (fixed-order sums). */
int nxa_ssm_check(int64_t nb, int32_t L, int32_t d, int32_t n);
size_t nxa_ssm_state_bytes(int64_t nb, int32_t L, int32_t d, int32_t n);
size_t nxa_ssm_workspace_bytes(int64_t nb, int32_t L, int32_t d, int32_t n, int is_bwd);
int nxa_ssm_fwd(int64_t nb, int32_t L, int32_t d, int32_t n, const float* x,
                const float* delta, const float* A, const float* B, const float* C,
                const float* D, float* y, float* state, void* workspace,
                size_t workspace_bytes, void* stream);
int nxa_ssm_bwd(int64_t nb, int32_t L, int32_t d, int32_t n, const float* x,
                const float* delta, const float* A, const float* B, const float* C,
                const float* D, const float* state, const float* dy, float* dx,
                float* ddelta, float* dA, float* dB, float* dC, float* dD,
                void* workspace, size_t workspace_bytes, void* stream);

/* Message of the last failure on this thread ("" if none). */
const char* nxa_last_error(void);

/* Kernel timing for profiling harnesses.  While enabled, every kernel the
 * library launches is bracketed by HIP events on its stream; nxa_profile_read
 * waits for them and returns the summed milliseconds and launch count of the
 * kernels whose name starts with `kernel` ("fwd", "dkdv", "dq", "delta",
 * "tilemap", "dbias_reduce", "rms_norm_fwd", "rms_norm_bwd", "ssm_fwd",
 * "ssm_bwd"; the last two cover a whole scan pass, several kernels).  Not for concurrent use from several threads. */
int nxa_profile_enable(int on);
int nxa_profile_read(const char* kernel, double* total_ms, int64_t* launches);
int nxa_profile_reset(void);

#ifdef __cplusplus
}
#endif

#endif /* NXATTN_H */
