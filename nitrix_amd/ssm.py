"""Selective state-space scan (Mamba / S6) with a fused gfx950 engine.

Host side of the drop-in for nitrix's ``nn.ssm.selective_scan``, with the
reference's public call signature and layering:

* :func:`selective_scan` -- the public dispatcher
  (``src/nitrix/nn/ssm/__init__.py:127-202``): validation (``:40-77``),
  ``driver`` / ``backend`` resolution, loud fallback.
* :func:`selective_scan_hip` -- the fused entry point, the counterpart of
  ``selective_scan_pallas`` (``src/nitrix/_kernels/cuda/selective_scan.py:497-549``):
  a tileability gate and a differentiable wrapper (:class:`_ScanHip`, the
  ``custom_vjp`` of ``:420-460``) around ``nxa_ssm_fwd`` / ``nxa_ssm_bwd``.
* :func:`reference_selective_scan` -- the reference engine
  (``backend='jax'``), the recipe of ``src/nitrix/nn/ssm/_reference.py:193-290``
  in stock tensor ops, with its ``'sequential'``, ``'associative'`` and
  ``'chunked'`` drivers.

The fused kernels compute in float32.  bfloat16 / float16 inputs are upcast
at the boundary and the output cast back, as the reference's float32
accumulation rule does (``_reference.py:255-281``); float64 is declined (a
loud fallback to the reference engine).
"""

from __future__ import annotations

import ctypes
import math
from typing import Optional

import torch
from torch.autograd.function import once_differentiable

from . import _lib
from ._backend import (
    NitrixBackendError,
    fallback,
    reproducible_enabled,
    resolve_backend,
)
from .attention import HipNotTileable

__all__ = [
    'reference_selective_scan',
    'selective_scan',
    'selective_scan_hip',
]

_DRIVERS = ('auto', 'sequential', 'associative', 'chunked')
_HIP_DTYPES = (torch.float32, torch.bfloat16, torch.float16)
_MAX_STATES = 32


def _validate(x, delta, A, B, C, D) -> None:
    """Shape checks of ``nn/ssm/__init__.py:40-77`` (same messages)."""
    if x.shape != delta.shape:
        raise ValueError(
            f'selective_scan: x and delta must match; got x.shape={tuple(x.shape)}, '
            f'delta.shape={tuple(delta.shape)}.'
        )
    if x.ndim < 2:
        raise ValueError(f'selective_scan: x must be at least (l, d); got ndim {x.ndim}.')
    d = x.shape[-1]
    length = x.shape[-2]
    if A.ndim != 2 or A.shape[0] != d:
        raise ValueError(
            f'selective_scan: A must be (d, n) with d={d}; got A.shape={tuple(A.shape)}.'
        )
    n = A.shape[1]
    if B.shape[-1] != n or C.shape[-1] != n:
        raise ValueError(
            f'selective_scan: B/C last dim must be n={n}; got B.shape={tuple(B.shape)}, '
            f'C.shape={tuple(C.shape)}.'
        )
    if B.shape[-2] != length or C.shape[-2] != length:
        raise ValueError(
            f'selective_scan: B/C sequence dim must be l={length}; got '
            f'B.shape={tuple(B.shape)}, C.shape={tuple(C.shape)}.'
        )
    if D is not None and tuple(D.shape) != (d,):
        raise ValueError(
            f'selective_scan: D must be (d,) with d={d}; got D.shape={tuple(D.shape)}.'
        )


def _io_dtype(x, delta, A, B, C, D) -> torch.dtype:
    dt = x.dtype
    for t in (delta, A, B, C) + (() if D is None else (D,)):
        dt = torch.promote_types(dt, t.dtype)
    return dt


# ---------------------------------------------------------------------------
# Reference engine (backend='jax')
# ---------------------------------------------------------------------------


def _scan_sequential(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    # h_t = a_t h_{t-1} + b_t over axis -3 of (..., l, d, n), h_0 = 0.
    h = torch.zeros_like(b[..., 0, :, :])
    out = torch.empty_like(b)
    for t in range(b.shape[-3]):
        h = a[..., t, :, :] * h + b[..., t, :, :]
        out[..., t, :, :] = h
    return out


def _scan_associative(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    # Inclusive prefix of (a1, b1) o (a2, b2) = (a1 a2, a2 b1 + b2) by recursive
    # doubling (log2(l) rounds).
    a = a.clone()
    b = b.clone()
    length = b.shape[-3]
    step = 1
    while step < length:
        a_prev = a[..., :-step, :, :]
        b_prev = b[..., :-step, :, :]
        b_new = a[..., step:, :, :] * b_prev + b[..., step:, :, :]
        a_new = a[..., step:, :, :] * a_prev
        b = torch.cat([b[..., :step, :, :], b_new], dim=-3)
        a = torch.cat([a[..., :step, :, :], a_new], dim=-3)
        step *= 2
    return b


def _scan_chunked(x, delta, A, B, C, D, chunk: int) -> torch.Tensor:
    # Chunks in sequence, the recurrence inside a chunk by _scan_associative,
    # the chunk-entry state propagated with the cumulative decay; the state
    # axis is collapsed per chunk (_reference.py:113-190).
    *batch, length, d = x.shape
    h = torch.zeros((*batch, d, A.shape[1]), dtype=x.dtype, device=x.device)
    ys = []
    for c0 in range(0, length, chunk):
        sl = slice(c0, c0 + chunk)
        dA = torch.exp(delta[..., sl, :, None] * A)
        dBx = delta[..., sl, :, None] * B[..., sl, None, :] * x[..., sl, :, None]
        cum_a = torch.cumprod(dA, dim=-3)
        h_loc = _scan_associative(dA, dBx)
        hh = h_loc + cum_a * h.unsqueeze(-3)
        y = (hh * C[..., sl, None, :]).sum(-1)
        if D is not None:
            y = y + D * x[..., sl, :]
        ys.append(y)
        h = hh[..., -1, :, :]
    return torch.cat(ys, dim=-2)


def reference_selective_scan(
    x: torch.Tensor,
    delta: torch.Tensor,
    A: torch.Tensor,
    B: torch.Tensor,
    C: torch.Tensor,
    D: Optional[torch.Tensor] = None,
    *,
    driver: str = 'auto',
    chunk_size: int = 64,
) -> torch.Tensor:
    """The reference engine, op for op as ``_reference.py:193-290``.

    Upcast to ``promote(io dtype, float32)``, discretise ``exp(delta A)`` and
    ``delta B x``, scan (``'sequential'``: one step at a time, the canonical
    variant; ``'associative'``: parallel prefix; ``'chunked'``: chunks of
    ``chunk_size`` in sequence), read out ``C . h (+ D x)``, cast back.
    ``'auto'`` is ``'sequential'`` on the CPU or under reproducible mode and
    ``'associative'`` on a GPU.
    """
    if driver not in _DRIVERS:
        raise ValueError(f'selective_scan: driver={driver!r} not in {_DRIVERS!r}')
    if driver == 'auto':
        on_gpu = x.device.type == 'cuda'
        driver = 'associative' if (on_gpu and not reproducible_enabled()) else 'sequential'
    io = _io_dtype(x, delta, A, B, C, D)
    acc = torch.promote_types(io, torch.float32)
    x, delta, A, B, C = (t.to(acc) for t in (x, delta, A, B, C))
    D = None if D is None else D.to(acc)
    if driver == 'chunked':
        chunk = min(chunk_size, x.shape[-2])
        if x.shape[-2] % chunk != 0:
            raise ValueError(
                f"driver='chunked' requires l % chunk_size == 0; got "
                f'l={x.shape[-2]}, chunk_size={chunk_size}.'
            )
        out = _scan_chunked(x, delta, A, B, C, D, chunk)
    else:
        a = torch.exp(delta[..., None] * A)
        b = delta[..., None] * B[..., :, None, :] * x[..., None]
        h = _scan_sequential(a, b) if driver == 'sequential' else _scan_associative(a, b)
        out = (h * C[..., :, None, :]).sum(-1)
        if D is not None:
            out = out + D * x
    return out.to(io)


# ---------------------------------------------------------------------------
# Fused HIP engine
# ---------------------------------------------------------------------------


def _check_tileable(x, delta, A, B, C, D) -> None:
    """Shapes and dtypes the gfx950 kernels decline (the counterpart of
    ``_check_tileable`` / ``_resolve_chunk``, ``selective_scan.py:463-494``;
    any length and any state dim up to 32 tile here)."""
    io = _io_dtype(x, delta, A, B, C, D)
    if io not in _HIP_DTYPES:
        raise HipNotTileable(
            f'fused selective scan supports float32 / bfloat16 / float16; got {io} '
            '(use backend="jax" for other dtypes).'
        )
    n = A.shape[1]
    if not 1 <= n <= _MAX_STATES:
        raise HipNotTileable(f'fused selective scan needs 1 <= n <= {_MAX_STATES}; got n={n}.')
    if x.numel() == 0 or B.numel() == 0:
        raise HipNotTileable('fused selective scan needs non-empty inputs.')
    devs = {t.device for t in (x, delta, A, B, C) + (() if D is None else (D,))}
    if len(devs) != 1:
        raise HipNotTileable('selective scan inputs are on different devices.')


def _unbroadcast(g: torch.Tensor, shape) -> torch.Tensor:
    """Sum g over the leading axes that ``shape`` broadcasts."""
    extra = g.ndim - len(shape)
    if extra > 0:
        g = g.sum(dim=tuple(range(extra)))
    axes = tuple(i for i, s in enumerate(shape) if s == 1 and g.shape[i] != 1)
    if axes:
        g = g.sum(dim=axes, keepdim=True)
    return g


class _ScanPrep:
    """float32 [nb, l, d] / [nb, l, n] views and the extents of one call."""

    def __init__(self, x, delta, A, B, C, D):
        f32 = torch.float32
        *batch, length, d = x.shape
        self.batch = tuple(batch)
        self.nb = int(math.prod(batch)) if batch else 1
        self.length, self.d, self.n = length, d, A.shape[1]
        self.device = x.device
        self.io = _io_dtype(x, delta, A, B, C, D)
        self.shapes = [tuple(t.shape) for t in (x, delta, A, B, C)]
        self.dtypes = [t.dtype for t in (x, delta, A, B, C)]
        self.D_dtype = None if D is None else D.dtype
        bn = self.batch + (length, self.n)

        def flat(t, shape, last):
            return t.to(f32).expand(shape).reshape(self.nb, length, last).contiguous()

        self.x = flat(x, self.batch + (length, d), d)
        self.delta = flat(delta, self.batch + (length, d), d)
        self.B = flat(B, bn, self.n)
        self.C = flat(C, bn, self.n)
        self.A = A.to(f32).contiguous()
        self.D = None if D is None else D.to(f32).contiguous()

    def dims(self):
        return (self.nb, self.length, self.d, self.n)

    def stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def workspace(self, is_bwd: int) -> torch.Tensor:
        nbytes = _lib.lib().nxa_ssm_workspace_bytes(*self.dims(), is_bwd)
        return torch.empty(nbytes, dtype=torch.uint8, device=self.device)


def _p(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _scan_forward(prep: _ScanPrep, keep_state: bool):
    lib = _lib.lib()
    y = torch.empty((prep.nb, prep.length, prep.d), dtype=torch.float32, device=prep.device)
    state = None
    if keep_state:
        nbytes = lib.nxa_ssm_state_bytes(*prep.dims())
        state = torch.empty(nbytes // 4, dtype=torch.float32, device=prep.device)
    ws = prep.workspace(0)
    _lib.check(
        lib.nxa_ssm_fwd(
            *prep.dims(),
            _p(prep.x), _p(prep.delta), _p(prep.A), _p(prep.B), _p(prep.C), _p(prep.D),
            _p(y), _p(state), _p(ws), ctypes.c_size_t(ws.numel()), prep.stream(),
        )
    )
    return y, state


def _scan_backward(prep: _ScanPrep, state: torch.Tensor, dy: torch.Tensor):
    lib = _lib.lib()
    f32 = torch.float32
    dy = dy.to(f32).reshape(prep.nb, prep.length, prep.d).contiguous()
    dx = torch.empty_like(prep.x)
    ddelta = torch.empty_like(prep.x)
    dA = torch.empty_like(prep.A)
    dB = torch.empty_like(prep.B)
    dC = torch.empty_like(prep.C)
    dD = None if prep.D is None else torch.empty_like(prep.D)
    ws = prep.workspace(1)
    _lib.check(
        lib.nxa_ssm_bwd(
            *prep.dims(),
            _p(prep.x), _p(prep.delta), _p(prep.A), _p(prep.B), _p(prep.C), _p(prep.D),
            _p(state), _p(dy), _p(dx), _p(ddelta), _p(dA), _p(dB), _p(dC), _p(dD),
            _p(ws), ctypes.c_size_t(ws.numel()), prep.stream(),
        )
    )
    return dx, ddelta, dA, dB, dC, dD


class _ScanHip(torch.autograd.Function):
    """Fused forward, recompute-adjoint fused backward.

    The fp32 views the kernels read (which alias the caller's tensors when
    those are already contiguous fp32) and the saved sub-chunk states are
    kept with ``save_for_backward``, so an in-place change of an input
    between forward and backward raises torch's version-counter error; the
    backward is not itself differentiable."""

    @staticmethod
    def forward(ctx, x, delta, A, B, C, D):
        prep = _ScanPrep(x, delta, A, B, C, D)
        keep = any(ctx.needs_input_grad)
        y, state = _scan_forward(prep, keep)
        if keep:
            ctx.save_for_backward(prep.x, prep.delta, prep.A, prep.B, prep.C, prep.D, state)
            for name in ('x', 'delta', 'A', 'B', 'C', 'D'):
                setattr(prep, name, None)
            ctx.prep = prep
        return y.reshape(*prep.batch, prep.length, prep.d).to(prep.io)

    @staticmethod
    @once_differentiable
    def backward(ctx, dy):
        prep = ctx.prep
        prep.x, prep.delta, prep.A, prep.B, prep.C, prep.D, state = ctx.saved_tensors
        dx, ddelta, dA, dB, dC, dD = _scan_backward(prep, state, dy)
        lead = prep.batch
        out = []
        grads = (dx, ddelta, dA, dB, dC)
        for i, (g, shape, dtype) in enumerate(zip(grads, prep.shapes, prep.dtypes)):
            if not ctx.needs_input_grad[i]:
                out.append(None)
                continue
            if i in (0, 1):
                g = g.reshape(*lead, prep.length, prep.d)
            elif i in (3, 4):
                g = _unbroadcast(g.reshape(*lead, prep.length, prep.n), shape)
            out.append(g.to(dtype))
        out.append(None if dD is None or not ctx.needs_input_grad[5] else dD.to(prep.D_dtype))
        return tuple(out)


def selective_scan_hip(
    x: torch.Tensor,
    delta: torch.Tensor,
    A: torch.Tensor,
    B: torch.Tensor,
    C: torch.Tensor,
    D: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Fused selective scan on gfx950 (``selective_scan.py:497-549``
    counterpart).  Raises :class:`HipNotTileable` for inputs outside the
    supported set; differentiable in every input."""
    _check_tileable(x, delta, A, B, C, D)
    _lib.lib()  # a missing library is an error here, not a fallback
    return _ScanHip.apply(x, delta, A, B, C, D)


def selective_scan(
    x: torch.Tensor,
    delta: torch.Tensor,
    A: torch.Tensor,
    B: torch.Tensor,
    C: torch.Tensor,
    D: Optional[torch.Tensor] = None,
    *,
    driver: str = 'auto',
    backend: str = 'auto',
) -> torch.Tensor:
    """Mamba / S6 selective scan with backend dispatch
    (``src/nitrix/nn/ssm/__init__.py:127-202``).

    ``h_t = exp(delta_t A) h_{t-1} + delta_t B_t x_t`` from ``h = 0`` and
    ``y_t = C_t . h_t (+ D x_t)`` per channel; x, delta ``(..., l, d)``, A
    ``(d, n)``, B, C ``(..., l, n)``, D ``(d,)`` or None.

    ``driver`` other than ``'auto'`` selects a reference variant and so the
    reference engine (with ``backend='hip'`` it is an error, as with
    ``'pallas-cuda'`` in the reference).  ``backend``: ``'hip'`` (fused
    gfx950 kernels), ``'jax'`` (reference engine) or ``'auto'``.
    """
    _validate(x, delta, A, B, C, D)
    if driver != 'auto':
        if backend in ('hip', 'pallas-cuda'):
            raise NitrixBackendError(
                f'selective_scan: driver={driver!r} selects a reference variant and '
                f'does not apply to backend={backend!r} (the fused kernel has no '
                "driver variants). Use backend='jax' or backend='auto'."
            )
        return reference_selective_scan(x, delta, A, B, C, D, driver=driver)
    resolved = resolve_backend(backend, x.device)
    if resolved == 'hip':
        try:
            return selective_scan_hip(x, delta, A, B, C, D)
        except HipNotTileable as exc:
            fallback(
                function='selective_scan',
                requested='hip',
                resolved='jax',
                reason=f'the fused selective-scan kernel does not support this input ({exc})',
                shapes=(tuple(x.shape), tuple(A.shape)),
                dtype=x.dtype,
            )
        except _lib.HipLibraryMissing as exc:
            raise NitrixBackendError(str(exc)) from exc
    return reference_selective_scan(x, delta, A, B, C, D, driver='auto')
