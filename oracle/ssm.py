"""CPU oracle for the selective state-space scan (numpy).

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports this
module: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker (or as
the timed CPU baseline), never as a code path of the product.

It restates nitrix's reference Mamba / S6 scan
(``src/nitrix/nn/ssm/_reference.py``) in numpy, in its canonical
``'sequential'`` variant: upcast to ``promote(result_type, float32)``
(``:268-281``), discretise ``dA = exp(delta A)``, ``dBx = delta B x``
(``:59-68``), scan ``h_t = dA_t h_{t-1} + dBx_t`` from ``h_0 = 0``
(``:84-97``), read out ``y_t = sum_n C_{t,n} h_{t,n} (+ D x_t)``
(``:71-81``), cast back (``:290``).

The backward is the closed-form reverse-mode adjoint of that recurrence, what
autodiff through the reference gives: with ``a_t = exp(delta_t A)`` and the
state cotangent ``g_t = C_t dy_t + a_{t+1} g_{t+1}`` (``g`` past the end = 0),

* ``dx_t     = D dy_t + sum_n g_{t,n} delta_t B_{t,n}``
* ``ddelta_t = sum_n g_{t,n} (B_{t,n} x_t + A_n a_{t,n} h_{t-1,n})``
* ``dA_n     = sum_t g_{t,n} delta_t a_{t,n} h_{t-1,n}``
* ``dB_{t,n} = sum_d g_{t,d,n} delta_{t,d} x_{t,d}``
* ``dC_{t,n} = sum_d dy_{t,d} h_{t,d,n}``
* ``dD       = sum_t dy_t x_t``

Pinning (``tests/test_oracle_ssm.py``): the reference's golden fixture
``tests/golden/selective_scan_float32.npz``, an independent per-step loop
(the reference's naive oracle form, ``tests/test_nn_ssm.py:89-103``), the
invariants of ``tests/test_nn_ssm.py:124-145`` (D-skip linearity, A -> 0 is a
cumulative sum), and central finite differences in float64 for every input
of the VJP.
"""

from __future__ import annotations

from typing import Optional

import numpy as np

__all__ = ['selective_scan', 'selective_scan_vjp']


def _acc(*arrays) -> np.dtype:
    return np.promote_types(np.result_type(*arrays), np.float32)


def selective_scan(x, delta, A, B, C, D=None, acc_dtype=None):
    """Forward scan; x, delta ``(..., l, d)``, A ``(d, n)``, B, C ``(..., l, n)``,
    D ``(d,)`` or None.  Returns ``y`` ``(..., l, d)`` in ``acc_dtype``
    (default ``promote(result_type, float32)``)."""
    acc = acc_dtype or _acc(x, delta, A, B, C, *([] if D is None else [D]))
    x, delta, A, B, C = (np.asarray(t, acc) for t in (x, delta, A, B, C))
    length = x.shape[-2]
    h = np.zeros(x.shape[:-2] + A.shape, acc)  # (..., d, n)
    y = np.empty_like(x)
    for t in range(length):
        dA = np.exp(delta[..., t, :, None] * A)
        dBx = delta[..., t, :, None] * B[..., t, None, :] * x[..., t, :, None]
        h = dA * h + dBx
        y[..., t, :] = np.sum(h * C[..., t, None, :], axis=-1)
    if D is not None:
        y = y + np.asarray(D, acc) * x
    return y


def selective_scan_vjp(x, delta, A, B, C, D, dy, acc_dtype=np.float64):
    """Cotangents ``(dx, ddelta, dA, dB, dC, dD)`` of ``sum(dy * y)``; dD is
    None when D is None.  Batch axes of B / C / x are summed into dA and dD
    only (A and D are shared)."""
    acc = acc_dtype
    x, delta, A, B, C, dy = (np.asarray(t, acc) for t in (x, delta, A, B, C, dy))
    length = x.shape[-2]
    batch = x.shape[:-2]
    # Forward states h_t (the (..., l, d, n) trajectory; fine at oracle sizes).
    a = np.exp(delta[..., :, :, None] * A)                    # (..., l, d, n)
    bx = delta[..., :, :, None] * B[..., :, None, :] * x[..., :, :, None]
    H = np.empty(batch + (length,) + A.shape, acc)
    h = np.zeros(batch + A.shape, acc)
    for t in range(length):
        h = a[..., t, :, :] * h + bx[..., t, :, :]
        H[..., t, :, :] = h
    Hprev = np.concatenate([np.zeros(batch + (1,) + A.shape, acc), H[..., :-1, :, :]], axis=-3)
    # Reverse adjoint of the state.
    G = np.empty_like(H)
    g = np.zeros(batch + A.shape, acc)
    for t in range(length - 1, -1, -1):
        nxt = a[..., t + 1, :, :] * g if t + 1 < length else 0.0
        g = C[..., t, None, :] * dy[..., t, :, None] + nxt
        G[..., t, :, :] = g
    dx = np.sum(G * delta[..., None] * B[..., :, None, :], axis=-1)
    ddelta = np.sum(G * (B[..., :, None, :] * x[..., None] + A * a * Hprev), axis=-1)
    dA = np.sum(G * delta[..., None] * a * Hprev, axis=tuple(range(len(batch) + 1)))
    dB = np.sum(G * (delta * x)[..., None], axis=-2)
    dC = np.sum(dy[..., None] * H, axis=-2)
    dD = None
    if D is not None:
        D = np.asarray(D, acc)
        dx = dx + D * dy
        dD = np.sum(dy * x, axis=tuple(range(len(batch) + 1)))
    return dx, ddelta, dA, dB, dC, dD
