"""Scaled-dot-product attention with a fused gfx950 engine.

Host side of the drop-in for nitrix's attention path.  It keeps the
reference's public call signature and layering:

* :func:`scaled_dot_product_attention` -- the public dispatcher
  (``src/nitrix/nn/attention/__init__.py:126-230``): validation, default
  scale, backend resolution, qk-norm outside the fused core, loud fallback.
* :func:`scaled_dot_product_attention_hip` -- the fused entry point, the
  counterpart of ``scaled_dot_product_attention_pallas``
  (``src/nitrix/_kernels/cuda/attention.py:768-824``): a tileability gate
  (:func:`_check_tileable`, ``:708-765``) and a differentiable wrapper
  (:class:`_SdpaHip`, the ``custom_vjp`` of ``:661-700``) around the C ABI of
  ``libnxattn.so``.
* :func:`reference_scaled_dot_product_attention` -- the unfused reference
  engine (``backend='jax'``), the recipe of
  ``src/nitrix/nn/attention/_reference.py:80-181`` in stock tensor ops.

Tensors live on the device (PyTorch-ROCm provides memory and streams); the
fused path launches on the current stream of the tensors' device.
"""

from __future__ import annotations

import ctypes
import math
from typing import Optional, Sequence

import torch
from torch.autograd.function import once_differentiable

from . import _lib
from ._backend import (
    NitrixBackendError,
    fallback,
    resolve_backend,
)

__all__ = [
    'HipNotTileable',
    'default_scale',
    'qk_rms_norm',
    'reference_scaled_dot_product_attention',
    'scaled_dot_product_attention',
    'scaled_dot_product_attention_hip',
]

# RMS-norm epsilon for qk-norm (_reference.py:32).
_QK_RMS_EPS = 1e-6

_IO_DTYPES = {
    torch.bfloat16: _lib.NXA_BF16,
    torch.float16: _lib.NXA_F16,
    torch.float32: _lib.NXA_F32,
}
# Bias dtypes the kernels read natively (others are upcast to float32).
_BIAS_DTYPES = _IO_DTYPES
_MAX_HEAD_DIM = 256


class HipNotTileable(RuntimeError):
    """The fused kernel declines this shape / dtype (the counterpart of the
    reference's ``PallasNotTileable``, ``attention.py:71-77``); the dispatcher
    turns it into a loud fallback to the reference engine."""


def default_scale(head_dim: int) -> float:
    """``1 / sqrt(d)`` (``_reference.py:35-49``)."""
    return 1.0 / math.sqrt(float(head_dim))


def qk_rms_norm(z: torch.Tensor) -> torch.Tensor:
    """``z * rsqrt(mean(z^2, -1) + 1e-6)`` (``_reference.py:52-77``).

    Computed in at least float32 and returned in ``z``'s dtype.
    """
    acc = torch.promote_types(z.dtype, torch.float32)
    zf = z.to(acc)
    ms = zf.square().mean(dim=-1, keepdim=True)
    return (zf * torch.rsqrt(ms + _QK_RMS_EPS)).to(z.dtype)


def _rms_norm_rows(x: torch.Tensor):
    """``nxa_rms_norm_fwd`` over the rows of ``x``: returns ``(y, x2, rstd)``
    with ``y`` normalised in ``x.dtype`` (shape of ``x``, contiguous), ``x2``
    the rows of ``x`` as a contiguous ``[rows, d]`` tensor (a view of ``x``
    when ``x`` is already laid out so) and ``rstd`` the fp32 per-row
    ``rsqrt(mean(x^2) + eps)``."""
    d = x.shape[-1]
    epc = 4 if x.dtype == torch.float32 else 8
    x2 = x.reshape(-1, d)
    if not x2.is_contiguous() or x2.data_ptr() % 16 or d % epc:
        x2 = x2.contiguous()
    rows = x2.shape[0]
    y = torch.empty((rows, d), dtype=x.dtype, device=x.device)
    rstd = torch.empty((rows,), dtype=torch.float32, device=x.device)
    stream = torch.cuda.current_stream(x.device).cuda_stream
    _lib.check(
        _lib.lib().nxa_rms_norm_fwd(
            rows, d, _IO_DTYPES[x.dtype], x2.data_ptr(), x2.stride(0),
            y.data_ptr(), rstd.data_ptr(), _QK_RMS_EPS, stream,
        )
    )
    return y.reshape(x.shape), x2, rstd


class _RmsNormHip(torch.autograd.Function):
    """qk-norm in one HIP pass per direction (``nxa_rms_norm_fwd`` /
    ``nxa_rms_norm_bwd``): the same math as :func:`qk_rms_norm` (fp32, cast
    back to ``x.dtype``), without its fp32 temporaries."""

    @staticmethod
    def forward(ctx, x):
        y, x2, rstd = _rms_norm_rows(x)
        ctx.save_for_backward(x2, rstd)
        ctx.shape = x.shape
        return y

    @staticmethod
    @once_differentiable
    def backward(ctx, dy):
        x2, rstd = ctx.saved_tensors
        rows, d = x2.shape
        dy2 = dy.reshape(rows, d)
        if not dy2.is_contiguous() or dy2.data_ptr() % 16:
            dy2 = dy2.contiguous()
        dx = torch.empty((rows, d), dtype=x2.dtype, device=x2.device)
        stream = torch.cuda.current_stream(x2.device).cuda_stream
        _lib.check(
            _lib.lib().nxa_rms_norm_bwd(
                rows, d, _IO_DTYPES[x2.dtype], x2.data_ptr(), x2.stride(0),
                dy2.data_ptr(), rstd.data_ptr(), dx.data_ptr(), stream,
            )
        )
        return dx.reshape(ctx.shape)


def _qk_norm_fused(z: torch.Tensor) -> torch.Tensor:
    """qk-norm on the fused path: the one-pass HIP kernels for GPU tensors of
    a kernel dtype whose head dim fits their 16-byte loads, else
    :func:`qk_rms_norm`."""
    epc = 4 if z.dtype == torch.float32 else 8
    if z.is_cuda and z.dtype in _IO_DTYPES and z.numel() > 0 and z.shape[-1] % epc == 0:
        return _RmsNormHip.apply(z)
    return qk_rms_norm(z)


def _validate(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    """``__init__.py:40-60``: same checks, same exception type."""
    if q.ndim < 3 or k.ndim < 3 or v.ndim < 3:
        raise ValueError(
            'scaled_dot_product_attention: q, k, v must have at least 3 '
            'dims (..., h, s, d); got ndim '
            f'{q.ndim}, {k.ndim}, {v.ndim}.'
        )
    if q.shape[-1] != k.shape[-1]:
        raise ValueError(
            'scaled_dot_product_attention: q/k head-dim mismatch '
            f'(q d={q.shape[-1]}, k d={k.shape[-1]}).'
        )
    if k.shape[-2] != v.shape[-2]:
        raise ValueError(
            'scaled_dot_product_attention: k/v key-length mismatch '
            f'(k t={k.shape[-2]}, v t={v.shape[-2]}).'
        )


# ---------------------------------------------------------------------------
# Reference engine (backend='jax')
# ---------------------------------------------------------------------------


def reference_scaled_dot_product_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    bias: Optional[torch.Tensor] = None,
    mask: Optional[torch.Tensor] = None,
    scale: Optional[float] = None,
    causal: bool = False,
    qk_norm: bool = False,
    qk_upcast: Optional[bool] = None,
) -> torch.Tensor:
    """Unfused attention, op for op as ``_reference.py:80-181``.

    Upcast to ``promote(result_type(q, k, v), float32)``, optional qk-norm,
    ``q k^T``, ``* scale``, ``+ bias``, ``where(mask & causal, ., -inf)``,
    softmax, ``. v``, cast back.  A fully masked row yields NaN.

    ``qk_upcast`` (``docs/feature-requests/attention-no-upcast-knob.md``, the
    "nitrix determination": a reference-only knob) chooses the precision of
    the stages instead: ``None`` (default) the above; ``True`` q / k cast to
    float32, scores and softmax in float32, the probabilities cast back to
    the I/O dtype and the value product and output in the I/O dtype (the
    ``upcast_attention=True`` regime); ``False`` every stage in the I/O
    dtype (``upcast_attention=False``; the caller owns overflow).  For
    float32 or float64 inputs all three coincide.
    """
    if scale is None:
        scale = default_scale(q.shape[-1])
    out_dtype = torch.promote_types(torch.promote_types(q.dtype, k.dtype), v.dtype)
    acc = torch.promote_types(out_dtype, torch.float32)
    # Dtypes of the score stage (q k^T, scale, bias, mask, softmax) and of the
    # value stage (P v).
    sdt = acc if qk_upcast in (None, True) else out_dtype
    vdt = acc if qk_upcast is None else out_dtype
    q = q.to(sdt)
    k = k.to(sdt)
    # (the right operand of every 16-bit product is made contiguous: the
    # batched bf16 / fp16 products of this PyTorch-ROCm build are documented
    # to fault the GPU when that operand is a transposed view)
    v = v.to(vdt).contiguous()
    acc = sdt
    if qk_norm:
        q = qk_rms_norm(q)
        k = qk_rms_norm(k)
    logits = torch.matmul(q, k.transpose(-1, -2).contiguous()) * scale
    if bias is not None:
        logits = logits + bias.to(acc)
    keep = mask
    if causal:
        s, t = logits.shape[-2], logits.shape[-1]
        cm = (
            torch.arange(s, device=logits.device)[:, None]
            >= torch.arange(t, device=logits.device)[None, :]
        )
        keep = cm if keep is None else (keep.to(torch.bool) & cm)
    if keep is not None:
        logits = torch.where(
            keep.to(torch.bool), logits, torch.full((), -math.inf, dtype=acc, device=logits.device)
        )
    weights = torch.softmax(logits, dim=-1)
    out = torch.matmul(weights.to(vdt), v)
    return out.to(out_dtype)


# ---------------------------------------------------------------------------
# Fused HIP engine
# ---------------------------------------------------------------------------


def _check_tileable(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    """Reject shapes the gfx950 kernels cannot run (``attention.py:708-765``).

    Accepts bf16, fp16 or fp32 (q, k, v of one dtype), head dims ``d`` (q, k)
    and ``d_v`` (v) up to 256 each (multiples of 8 for the 16-bit types, of 4
    for fp32) and any positive query / key lengths (tails are predicated in
    the kernels).
    """
    if q.dtype not in _IO_DTYPES:
        raise HipNotTileable(
            f'fused attention supports bfloat16, float16 and float32; got {q.dtype}.'
        )
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise HipNotTileable(
            f'fused attention needs one dtype for q, k, v; got {q.dtype}, '
            f'{k.dtype}, {v.dtype}.'
        )
    d, d_v = q.shape[-1], v.shape[-1]
    epc = 4 if q.dtype == torch.float32 else 8
    for name, n in (('d', d), ('d_v', d_v)):
        if n > _MAX_HEAD_DIM or n % epc != 0:
            raise HipNotTileable(
                f'fused attention requires head dims <= {_MAX_HEAD_DIM} and '
                f'multiples of {epc}; got {name}={n}.'
            )
    if q.shape[-2] == 0 or k.shape[-2] == 0 or d == 0 or d_v == 0:
        raise HipNotTileable('fused attention needs non-empty q / k / v.')
    if not (q.device == k.device == v.device):
        raise HipNotTileable('q, k, v are on different devices.')


def _row_stride_ok(stride: int, esize: int) -> bool:
    """The kernels address up to 64 rows of a tile with 32-bit byte offsets
    (``nxa_check`` rejects larger row strides with ``NXA_E_LAYOUT``)."""
    return (64 * stride + 256) * esize < (1 << 32)


def _layout_ok(x: torch.Tensor, epc: int) -> bool:
    if x.stride(-1) != 1 and x.shape[-1] != 1:
        return False
    if x.data_ptr() % 16 != 0:
        return False
    if not _row_stride_ok(x.stride(-2), x.element_size()):
        return False
    return all(s % epc == 0 for s in x.stride()[:-1])


def _lead_shape(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> tuple:
    """The broadcast leading axes of q, k, v (``torch.broadcast_shapes``,
    whose tensor machinery costs more host time than a whole small launch,
    only when they differ)."""
    lq, lk, lv = tuple(q.shape[:-2]), tuple(k.shape[:-2]), tuple(v.shape[:-2])
    if lq == lk == lv:
        return lq
    return tuple(torch.broadcast_shapes(lq, lk, lv))


def _as_bhld(x: torch.Tensor, lead: Sequence[int], nb: int, epc: int) -> torch.Tensor:
    L, d = x.shape[-2], x.shape[-1]
    h = lead[-1]
    if len(lead) == 2 and tuple(x.shape[:-2]) == tuple(lead):
        y = x  # already [nb, h, L, d]
    else:
        y = x.expand(*lead, L, d).reshape(nb, h, L, d)
    if not _layout_ok(y, epc):
        y = y.contiguous()
    return y


def _as_bhst(
    x: torch.Tensor, lead: Sequence[int], nb: int, s: int, t: int
) -> torch.Tensor:
    h = lead[-1]
    if len(lead) == 2 and tuple(x.shape) == (*lead, s, t):
        y = x  # already [nb, h, s, t]
    else:
        y = x.expand(*lead, s, t).reshape(nb, h, s, t)
    if (y.stride(-1) != 1 and t != 1) or not _row_stride_ok(y.stride(-2), y.element_size()):
        y = y.contiguous()
    return y


def _unbroadcast(g: torch.Tensor, shape: Sequence[int]) -> torch.Tensor:
    """VJP of a broadcast (``attention.py:517-544``)."""
    while g.ndim > len(shape):
        g = g.sum(dim=0)
    axes = tuple(i for i, n in enumerate(shape) if n == 1 and g.shape[i] != 1)
    if axes:
        g = g.sum(dim=axes, keepdim=True)
    return g.reshape(tuple(shape))


def _ptr(x: Optional[torch.Tensor]) -> Optional[int]:
    return None if x is None else x.data_ptr()


class _Prepared:
    """Flattened [nb, h, L, d] views plus the C descriptor of one call."""

    def __init__(self, q, k, v, bias, mask, scale, causal):
        *_, s, d = q.shape
        t = k.shape[-2]
        lead = _lead_shape(q, k, v)
        self.lead = lead
        self.batch = lead[:-1]
        self.h = lead[-1]
        self.nb = int(math.prod(self.batch)) if self.batch else 1
        self.s, self.t, self.d = s, t, d
        self.dv = v.shape[-1]
        self.dtype = q.dtype
        self.device = q.device
        self.epc = 4 if q.dtype == torch.float32 else 8
        self.q = _as_bhld(q, lead, self.nb, self.epc)
        self.k = _as_bhld(k, lead, self.nb, self.epc)
        self.v = _as_bhld(v, lead, self.nb, self.epc)
        self.bias_shape = None if bias is None else tuple(bias.shape)
        self.bias_dtype = None if bias is None else bias.dtype
        self.bias = None
        if bias is not None:
            b = bias.to(self.device)
            if b.dtype not in _BIAS_DTYPES:
                b = b.to(torch.float32)
            self.bias = _as_bhst(b, lead, self.nb, s, t)
        self.mask = None
        if mask is not None:
            m = mask.to(self.device)
            if m.dtype not in (torch.bool, torch.uint8):
                m = m != 0
            self.mask = _as_bhst(m, lead, self.nb, s, t)

        desc = _lib.NxaDesc()
        desc.B, desc.H, desc.Lq, desc.Lk, desc.D = self.nb, self.h, s, t, d
        desc.Dv = self.dv
        desc.io_dtype = _IO_DTYPES[q.dtype]
        desc.bias_dtype = (
            _BIAS_DTYPES[self.bias.dtype] if self.bias is not None else _lib.NXA_F32
        )
        desc.causal = 1 if causal else 0
        desc.scale = float(scale)
        desc.q_str[:] = self.q.stride()[:3]
        desc.k_str[:] = self.k.stride()[:3]
        desc.v_str[:] = self.v.stride()[:3]
        # outputs are allocated contiguous
        dv = self.dv
        desc.o_str[:] = (self.h * s * dv, s * dv, dv)
        if self.bias is not None:
            desc.bias_str[:] = self.bias.stride()[:3]
        if self.mask is not None:
            desc.mask_str[:] = self.mask.stride()[:3]
        self.desc = desc

    @property
    def has_bias(self) -> int:
        return 1 if self.bias is not None else 0

    @property
    def has_mask(self) -> int:
        return 1 if self.mask is not None else 0

    def stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def workspace_bytes(self, flags: int) -> int:
        """``nxa_workspace_bytes`` for ``flags`` (``NXA_WS_*``)."""
        return _lib.lib().nxa_workspace_bytes(
            ctypes.byref(self.desc), self.has_bias, self.has_mask, flags
        )

    def workspace(self, flags: int) -> Optional[torch.Tensor]:
        nbytes = self.workspace_bytes(flags)
        if nbytes == 0:
            return None
        return torch.empty(nbytes, dtype=torch.uint8, device=self.device)


def _forward(prep: _Prepared, for_bwd: bool = False, qnorm=None):
    """Run ``nxa_fwd``; returns ``(o [nb,h,s,d], lse [nb,h,s], workspace)``.

    With ``for_bwd`` the workspace is sized for a backward without dbias (it
    starts with the forward's tile map, then the per-row values), so such a
    backward reuses it as is; a backward that wants dbias of a shared bias
    allocates its larger workspace itself.  With ``qnorm = (q_hat,
    q_rstd)`` (``prep.q`` then holds the raw rows) the kernel normalises q
    itself (``nxa_fwd_normed``) and writes q_hat and its per-row rsqrt."""
    lib = _lib.lib()
    o = torch.empty(
        (prep.nb, prep.h, prep.s, prep.dv), dtype=prep.dtype, device=prep.device
    )
    lse = torch.empty(
        (prep.nb, prep.h, prep.s), dtype=torch.float32, device=prep.device
    )
    ws = prep.workspace(_lib.NXA_WS_BWD if for_bwd else _lib.NXA_WS_FWD)
    args = (ctypes.byref(prep.desc), _ptr(prep.q), _ptr(prep.k), _ptr(prep.v),
            _ptr(prep.bias), _ptr(prep.mask), _ptr(o), _ptr(lse))
    tail = (_ptr(ws), 0 if ws is None else ws.numel(), prep.stream())
    if qnorm is None:
        _lib.check(lib.nxa_fwd(*args, *tail))
    else:
        q_hat, q_rstd = qnorm
        _lib.check(lib.nxa_fwd_normed(*args, _ptr(q_hat), _ptr(q_rstd), _QK_RMS_EPS, *tail))
    return o, lse, ws


def _dbias_geometry(prep: _Prepared):
    bs = prep.desc.bias_str
    ob = 1 if bs[0] == 0 else prep.nb
    oh = 1 if bs[1] == 0 else prep.h
    lq = 1 if (prep.s > 1 and bs[2] == 0) else prep.s
    return ob, oh, lq


def _backward(prep: _Prepared, o, lse, fwd_ws, dout, want_dbias: bool, norm=None):
    """Run ``nxa_bwd`` (or, with ``norm = (q_raw, k_raw, q_rstd, k_rstd)``,
    ``nxa_bwd_normed``: ``prep`` holds the normalised q / k and dq / dk are
    taken with respect to the raw ones); returns flattened
    ``(dq, dk, dv, dbias_kernel)``."""
    lib = _lib.lib()
    # dK / dV are written per (b, h): broadcast q / k / v are materialised.
    q = prep.q if all(x != 0 for x in prep.q.stride()[:2]) else prep.q.contiguous()
    k = prep.k if all(x != 0 for x in prep.k.stride()[:2]) else prep.k.contiguous()
    v = prep.v if all(x != 0 for x in prep.v.stride()[:2]) else prep.v.contiguous()
    if q is not prep.q or k is not prep.k or v is not prep.v:
        prep.desc.q_str[:] = q.stride()[:3]
        prep.desc.k_str[:] = k.stride()[:3]
        prep.desc.v_str[:] = v.stride()[:3]
    dout = dout.reshape(prep.nb, prep.h, prep.s, prep.dv)
    if not dout.is_contiguous() or dout.data_ptr() % 16 != 0:
        dout = dout.contiguous()
    dq = torch.empty_like(q, memory_format=torch.contiguous_format)
    dk = torch.empty_like(k, memory_format=torch.contiguous_format)
    dv = torch.empty_like(v, memory_format=torch.contiguous_format)
    if dq.stride() != q.stride() or dk.stride() != k.stride() or dv.stride() != v.stride():
        # gradients share the input strides in the C ABI
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        prep.desc.q_str[:] = q.stride()[:3]
        prep.desc.k_str[:] = k.stride()[:3]
        prep.desc.v_str[:] = v.stride()[:3]
    dbias = None
    dbias_str = None
    if want_dbias and prep.bias is not None:
        ob, oh, lq = _dbias_geometry(prep)
        dbias = torch.empty(
            (ob, oh, lq, prep.t), dtype=prep.bias.dtype, device=prep.device
        )
        dbias_str = (ctypes.c_int64 * 3)(oh * lq * prep.t, lq * prep.t, prep.t)
    # The workspace begins with the forward's tile map; a forward workspace
    # already sized for this backward is reused in place.
    flags = _lib.NXA_WS_BWD | (_lib.NXA_WS_DBIAS if dbias is not None else 0)
    need = prep.workspace_bytes(flags)
    ready = 0
    if fwd_ws is not None and fwd_ws.numel() >= need:
        ws = fwd_ws
        ready = 1 if prep.mask is not None else 0
    else:
        ws = prep.workspace(flags)
        if prep.mask is not None and fwd_ws is not None:
            tm = prep.workspace_bytes(_lib.NXA_WS_FWD)
            ws[:tm].copy_(fwd_ws[:tm])
            ready = 1
    if norm is None:
        rc = lib.nxa_bwd(
            ctypes.byref(prep.desc), _ptr(q), _ptr(k), _ptr(v), _ptr(prep.bias),
            _ptr(prep.mask), _ptr(o), _ptr(lse), _ptr(dout), _ptr(dq), _ptr(dk),
            _ptr(dv), _ptr(dbias), dbias_str, _ptr(ws), ws.numel(), ready,
            prep.stream(),
        )
    else:
        q_raw, k_raw, q_rstd, k_rstd = norm
        rc = lib.nxa_bwd_normed(
            ctypes.byref(prep.desc), _ptr(q), _ptr(k), _ptr(v), _ptr(prep.bias),
            _ptr(prep.mask), _ptr(o), _ptr(lse), _ptr(dout), _ptr(q_raw),
            _ptr(k_raw), _ptr(q_rstd), _ptr(k_rstd), _ptr(dq), _ptr(dk), _ptr(dv),
            _ptr(dbias), dbias_str, _ptr(ws), ws.numel(), ready, prep.stream(),
        )
    _lib.check(rc)
    return dq, dk, dv, dbias


class _SdpaHip(torch.autograd.Function):
    """Differentiable fused attention: ``(q, k, v, bias, mask) -> out``.

    ``scale`` and ``causal`` are non-differentiable; the mask gets no
    gradient -- the structure of the reference's ``custom_vjp``
    (``attention.py:661-700``), whose residuals are the inputs, the output
    and the log-sum-exp.  They are kept with ``save_for_backward``, so an
    in-place change of an input between forward and backward raises
    torch's version-counter error; the backward is not itself
    differentiable (``once_differentiable``)."""

    @staticmethod
    def forward(ctx, q, k, v, bias, mask, scale, causal):
        prep = _Prepared(q, k, v, bias, mask, scale, causal)
        o, lse, ws = _forward(prep, for_bwd=any(ctx.needs_input_grad[:4]))
        ctx.args = (scale, causal)
        ctx.save_for_backward(
            q, k, v, bias, mask, o, lse, ws if ws is not None else torch.empty(0)
        )
        return o.reshape(*prep.lead, prep.s, prep.dv)

    @staticmethod
    @once_differentiable
    def backward(ctx, dout):
        q, k, v, bias, mask, o, lse, ws = ctx.saved_tensors
        prep = _Prepared(q, k, v, bias, mask, *ctx.args)
        want_dbias = bool(ctx.needs_input_grad[3])
        grads = _backward(prep, o, lse, ws if ws.numel() else None, dout, want_dbias)
        return _input_grads(prep, (q.shape, k.shape, v.shape), grads)


def _input_grads(prep: _Prepared, shapes, grads):
    """Flattened kernel gradients -> gradients of the caller's q, k, v, bias
    (broadcast axes summed, as the reference's ``_unbroadcast``)."""
    dq, dk, dv, dbias_k = grads
    qs, ks, vs = (tuple(x) for x in shapes)
    lead = prep.lead
    dq = _unbroadcast(dq.reshape(*lead, prep.s, prep.d), qs)
    dk = _unbroadcast(dk.reshape(*lead, prep.t, prep.d), ks)
    dv = _unbroadcast(dv.reshape(*lead, prep.t, prep.dv), vs)
    dbias = None
    if dbias_k is not None:
        ob, oh, lq = dbias_k.shape[:3]
        bdims = list(prep.batch) if ob > 1 else [1] * len(prep.batch)
        g = dbias_k.reshape(*bdims, oh, lq, prep.t)
        dbias = _unbroadcast(g, prep.bias_shape).to(prep.bias_dtype)
    return dq, dk, dv, dbias, None, None, None


class _SdpaNormHip(torch.autograd.Function):
    """Fused attention on RMS-normalised q and k (``qk_norm=True``): the
    one-pass norm kernels, the attention forward on the normalised rows, and
    a backward (``nxa_bwd_normed``) whose dQ / dK kernels apply the norm's
    VJP to their finished rows, so no normalised gradient makes an extra
    round trip through memory.  The forward is the one of the composed path
    (the reference normalises in the I/O dtype before its kernel,
    ``nn/attention/__init__.py:196-197``)."""

    @staticmethod
    def forward(ctx, q, k, v, bias, mask, scale, causal):
        # q is normalised inside the forward kernel (its query blocks hold
        # the rows stationary), k by the one-pass norm kernel: every query
        # block streams all key tiles, so normalising them on load would
        # repeat the work once per query block.
        # Without a backward the normalised q is not written at all.
        d = q.shape[-1]
        q2 = q.reshape(-1, d)
        if not q2.is_contiguous() or q2.data_ptr() % 16:
            q2 = q2.contiguous()
        for_bwd = any(ctx.needs_input_grad[:4])
        qn = torch.empty_like(q2) if for_bwd else None
        rq = (torch.empty((q2.shape[0],), dtype=torch.float32, device=q.device)
              if for_bwd else None)
        kn, k2, rk = _rms_norm_rows(k)
        prep = _Prepared(q2.reshape(q.shape), kn, v, bias, mask, scale, causal)
        o, lse, ws = _forward(prep, for_bwd=for_bwd, qnorm=(qn, rq))
        if qn is not None:
            qn = qn.reshape(q.shape)
        ctx.args = (scale, causal)
        ctx.save_for_backward(
            q, k, v, bias, mask, qn, kn, q2, k2, rq, rk, o, lse,
            ws if ws is not None else torch.empty(0),
        )
        return o.reshape(*prep.lead, prep.s, prep.dv)

    @staticmethod
    @once_differentiable
    def backward(ctx, dout):
        q, k, v, bias, mask, qn, kn, q2, k2, rq, rk, o, lse, ws = ctx.saved_tensors
        prep = _Prepared(qn, kn, v, bias, mask, *ctx.args)
        want_dbias = bool(ctx.needs_input_grad[3])
        grads = _backward(prep, o, lse, ws if ws.numel() else None, dout, want_dbias,
                          norm=(q2, k2, rq, rk))
        return _input_grads(prep, (q.shape, k.shape, v.shape), grads)


def _norm_fusable(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> bool:
    """Whether ``nxa_bwd_normed`` takes this qk-norm call: 16-bit I/O, a
    tileable head dim, and q, k not broadcast against each other or v over
    the leading axes."""
    if q.dtype not in (torch.bfloat16, torch.float16) or not q.is_cuda:
        return False
    if max(q.shape[-1], v.shape[-1]) > _MAX_HEAD_DIM or q.shape[-1] % 8 or v.shape[-1] % 8:
        return False
    lead = _lead_shape(q, k, v)
    return tuple(q.shape[:-2]) == lead and tuple(k.shape[:-2]) == lead


def scaled_dot_product_attention_hip(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    scale: float,
    bias: Optional[torch.Tensor] = None,
    mask: Optional[torch.Tensor] = None,
    causal: bool = False,
) -> torch.Tensor:
    """Fused attention on gfx950 (``attention.py:768-824`` counterpart).

    Raises :class:`HipNotTileable` for shapes outside the supported set; the
    dispatcher turns that into a loud fallback.  Differentiable in q, k, v and
    bias.
    """
    _check_tileable(q, k, v)
    _lib.lib()  # a missing library is an error here, not a fallback
    if not (torch.is_grad_enabled() and any(
            t is not None and t.requires_grad for t in (q, k, v, bias))):
        # Nothing to differentiate: the forward alone, without the autograd
        # node (whose bookkeeping costs host time a small call notices).
        prep = _Prepared(q, k, v, bias, mask, float(scale), bool(causal))
        o, _, _ = _forward(prep)
        return o.reshape(*prep.lead, prep.s, prep.dv)
    return _SdpaHip.apply(q, k, v, bias, mask, float(scale), bool(causal))


def _io_dtype(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.dtype:
    return torch.promote_types(torch.promote_types(q.dtype, k.dtype), v.dtype)


def _below_fp32(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> bool:
    """Whether the I/O dtype is narrower than float32 (bf16 / fp16)."""
    return torch.promote_types(_io_dtype(q, k, v), torch.float32) != _io_dtype(q, k, v)


def scaled_dot_product_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    bias: Optional[torch.Tensor] = None,
    mask: Optional[torch.Tensor] = None,
    scale: Optional[float] = None,
    causal: bool = False,
    qk_norm: bool = False,
    qk_upcast: Optional[bool] = None,
    backend: str = 'auto',
) -> torch.Tensor:
    """Scaled-dot-product attention with backend dispatch
    (``src/nitrix/nn/attention/__init__.py:126-230``).

    ``softmax(scale * q k^T + bias [masked]) v`` over the key axis.  q/k/v are
    ``(..., h, s, d)`` / ``(..., h, t, d)`` / ``(..., h, t, d_v)``; bias and the
    boolean keep-mask broadcast to ``(..., h, s, t)``; ``causal`` keeps key
    ``j`` for query ``i`` iff ``j <= i``; ``scale`` defaults to ``1/sqrt(d)``;
    ``qk_norm`` RMS-normalises q and k over the head dim first.

    ``backend``: ``'hip'`` (fused gfx950 kernels), ``'jax'`` (the unfused
    reference engine) or ``'auto'`` (``'hip'`` on a gfx950 device, else
    ``'jax'``; ``NITRIX_BACKEND`` and reproducible mode as in the reference).

    ``qk_upcast`` (default ``None``) selects the reference engine's stage
    precisions (:func:`reference_scaled_dot_product_attention`).  With
    bf16 / fp16 inputs ``True`` or ``False`` asks for accumulation below
    float32, which the fused kernels (float32 online softmax) do not
    provide: ``backend='hip'`` then raises :class:`NitrixBackendError` and
    ``'auto'`` resolves to the reference engine (``SPEC.md`` tenet 11,
    corollary (a)).  With float32 / float64 inputs it changes nothing.
    """
    _validate(q, k, v)
    if qk_upcast is not None and _below_fp32(q, k, v):
        if backend in ('hip', 'pallas-cuda'):
            raise NitrixBackendError(
                f'scaled_dot_product_attention: qk_upcast={qk_upcast!r} with '
                f'{_io_dtype(q, k, v)} inputs asks for accumulation below float32, '
                f'which backend={backend!r} (float32 online softmax) does not provide. '
                "Use backend='jax' or backend='auto'."
            )
        return reference_scaled_dot_product_attention(
            q, k, v, bias=bias, mask=mask, scale=scale, causal=causal,
            qk_norm=qk_norm, qk_upcast=qk_upcast,
        )
    resolved_scale = default_scale(q.shape[-1]) if scale is None else scale
    resolved = resolve_backend(backend, q.device)
    if resolved == 'hip':
        try:
            if qk_norm and _norm_fusable(q, k, v):
                _check_tileable(q, k, v)
                _lib.lib()
                return _SdpaNormHip.apply(
                    q, k, v, bias, mask, float(resolved_scale), bool(causal)
                )
            q_in = _qk_norm_fused(q) if qk_norm else q
            k_in = _qk_norm_fused(k) if qk_norm else k
            return scaled_dot_product_attention_hip(
                q_in,
                k_in,
                v,
                bias=bias,
                mask=mask,
                scale=resolved_scale,
                causal=causal,
            )
        except HipNotTileable as exc:
            fallback(
                function='scaled_dot_product_attention',
                requested='hip',
                resolved='jax',
                reason=f'the fused attention kernel does not support this shape ({exc})',
                shapes=(tuple(q.shape), tuple(k.shape), tuple(v.shape)),
                dtype=q.dtype,
            )
        except _lib.HipLibraryMissing as exc:
            raise NitrixBackendError(str(exc)) from exc
    return reference_scaled_dot_product_attention(
        q,
        k,
        v,
        bias=bias,
        mask=mask,
        scale=resolved_scale,
        causal=causal,
        qk_norm=qk_norm,
    )
