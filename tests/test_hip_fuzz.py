"""Seeded random configurations of the fused attention on the GPU.

Each case draws, from its own seed, a head dim (8 .. 256, the 16-bit kernels'
multiples of 8, any multiple of 4 for fp32), a value head dim, ragged query
and key lengths, a dtype, a mask kind, a bias broadcast pattern, causality
and the default or an explicit scale, then checks the output and every
gradient (dbias included) against the float64 oracle at the dtype's budget,
through the same C ABI as the fixed cases of ``test_hip_parity.py``.  The
point is combinations the fixed cases do not list; the draws are fixed by
the seeds, so a failure names a reproducible case.

The gradients are checked against the oracle's backward fed the stored
forward output, from which the reference's fused backward forms
delta = rowsum(o * do) (``attention.py:600-622``), with the budget
``tol * max|ref| + u * M``: M bounds the terms whose difference forms dS
(``M = max scale * sum_j P_ij (sum|dO_i||v_j| + sum|o_i||dO_i|) |k_j|`` for
dQ, likewise for dK and dS itself for dbias) and u is the rounding of the
kernels' fp32 intermediates (2^-24; 2^-16 for the 16-bit kernels, whose dQ
kernel adds -delta to its dP products as a two-term bf16 split).  The term only
matters where dS cancels almost entirely: an explicit scale that makes the
softmax one-hot, or a single key (the exact gradient of q, k and the bias
is then zero).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _golden import relerr
from oracle import attention as O
from test_hip_parity import REL, _draw, _make_mask, _to

pytestmark = pytest.mark.gpu

DTYPES = (torch.bfloat16, torch.float16, torch.float32)
BIAS_SHAPES = ('none', 'full', 'batch', 'query', 'shared', 'head')
MASKS = (None, 'keypad', 'random', 'block', 'rowbcast')


def _dev():
    return torch.device('cuda:0')


def _case(seed):
    rng = np.random.default_rng(1000 + seed)
    dtype = DTYPES[seed % 3]
    step = 4 if dtype == torch.float32 else 8
    d = int(rng.choice([step, 24, 40, 64, 64, 72, 96, 128, 128, 136, 192, 248, 256]))
    d -= d % step
    dv = d if rng.random() < 0.7 else int(rng.choice([8, 32, 64, 128, 256]))
    B, H = int(rng.integers(1, 3)), int(rng.integers(1, 3))
    s, t = int(rng.integers(1, 260)), int(rng.integers(1, 300))
    causal = bool(rng.random() < 0.3)
    mask_kind = MASKS[int(rng.integers(len(MASKS)))]
    bias_kind = BIAS_SHAPES[int(rng.integers(len(BIAS_SHAPES)))]
    scale = None if rng.random() < 0.7 else float(rng.uniform(0.05, 0.5))
    return dict(dtype=dtype, d=d, dv=dv, B=B, H=H, s=s, t=t, causal=causal,
                mask_kind=mask_kind, bias_kind=bias_kind, scale=scale, rng=rng)


def _bias_shape(kind, B, H, s, t):
    return {'none': None, 'full': (B, H, s, t), 'batch': (H, s, t),
            'query': (B, H, 1, t), 'shared': (s, t), 'head': (B, 1, s, t)}[kind]


def _cancel_bounds(q, k, v, g, o, bias, mask, scale, causal, bias_shape):
    """M for dQ, dK and dbias (float64): the magnitudes of the terms that
    cancel in dS = P (dP - delta)."""
    logits, qa, ka = O._logits(q, k, bias, mask, scale, causal, False, np.dtype(np.float64))
    p = O._softmax(logits)
    ag, av, ao = np.abs(g.astype(np.float64)), np.abs(v.astype(np.float64)), np.abs(o)
    w = p * (np.matmul(ag, np.swapaxes(av, -1, -2)) + np.sum(ao * ag, axis=-1, keepdims=True))
    m_dq = scale * np.max(np.matmul(w, np.abs(ka)))
    m_dk = scale * np.max(np.matmul(np.swapaxes(w, -1, -2), np.abs(qa)))
    m_db = 0.0 if bias_shape is None else float(np.max(O.unbroadcast(w, bias_shape)))
    return {'dq': m_dq, 'dk': m_dk, 'dv': 0.0, 'dbias': m_db}


@pytest.mark.parametrize('seed', range(416))
def test_random_configuration(seed):
    c = _case(seed)
    dtype, d, dv, B, H, s, t = (c[k] for k in ('dtype', 'd', 'dv', 'B', 'H', 's', 't'))
    rng = c['rng']
    q, k = _draw(rng, (B, H, s, d), dtype), _draw(rng, (B, H, t, d), dtype)
    v, g = _draw(rng, (B, H, t, dv), dtype), _draw(rng, (B, H, s, dv), dtype)
    bshape = _bias_shape(c['bias_kind'], B, H, s, t)
    bias = None if bshape is None else _draw(rng, bshape, dtype)
    mask = _make_mask(rng, c['mask_kind'], B, H, s, t)
    if c['causal'] and mask is not None:
        # Every row keeps key 0 (the masks keep it too), so no row is empty.
        mask = np.broadcast_to(mask, (B, H, s, t)).copy()
        mask[..., 0] = True
    print(f'[case] seed {seed}: {dtype} B{B} H{H} s{s} t{t} d{d} dv{dv} '
          f'causal={c["causal"]} mask={c["mask_kind"]} bias={c["bias_kind"]} '
          f'scale={c["scale"]}', flush=True)
    from nitrix_amd import scaled_dot_product_attention

    tq, tk, tv = _to(q, dtype, True), _to(k, dtype, True), _to(v, dtype, True)
    tb = None if bias is None else _to(bias, dtype, True)
    tm = None if mask is None else torch.from_numpy(np.ascontiguousarray(mask)).to(_dev())
    out = scaled_dot_product_attention(tq, tk, tv, bias=tb, mask=tm, causal=c['causal'],
                                       scale=c['scale'], backend='hip')
    scale = c['scale'] if c['scale'] is not None else 1.0 / np.sqrt(d)
    ref = O.sdpa_forward(q, k, v, bias=bias, mask=mask, scale=scale, causal=c['causal'],
                         acc_dtype=np.float64)
    tol = REL[dtype]
    got = out.detach().float().cpu().numpy()
    # Fully masked rows are NaN in both (the reference's softmax of all -inf).
    nan_ref = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan_ref), 'NaN rows differ'
    e = relerr(np.where(nan_ref, 0, got), np.where(nan_ref, 0, ref))
    print(f'  out relerr {e:.2e}', flush=True)
    assert e <= tol, f'out relerr {e:.3e}'
    if nan_ref.any():
        return  # gradients through NaN rows are NaN by definition
    out.backward(_to(g, dtype))
    torch.cuda.synchronize()
    o = got.astype(np.float64)
    dq, dk, dvr, db = O.sdpa_backward(q, k, v, g, bias=bias, mask=mask, scale=scale,
                                      causal=c['causal'], acc_dtype=np.float64, out=o)
    u = 2.0 ** -24 if dtype == torch.float32 else 2.0 ** -16
    bound = _cancel_bounds(q, k, v, g, o, bias, mask, scale, c['causal'], bshape)
    checks = [('dq', tq.grad, dq), ('dk', tk.grad, dk), ('dv', tv.grad, dvr)]
    if bias is not None:
        checks.append(('dbias', tb.grad, db))
    for name, got_t, want in checks:
        a = got_t.float().cpu().numpy()
        assert a.shape == want.shape, (name, a.shape, want.shape)
        err = float(np.max(np.abs(a - want))) if a.size else 0.0
        budget = tol * float(np.max(np.abs(want))) + u * bound[name] if a.size else 0.0
        print(f'  {name} relerr {relerr(a, want):.2e} err {err:.2e} budget {budget:.2e}', flush=True)
        assert err <= budget, f'{name} error {err:.3e} > budget {budget:.3e}'
