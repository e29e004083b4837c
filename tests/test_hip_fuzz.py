"""Seeded random configurations of the fused attention on the GPU.

Each case draws, from its own seed, a head dim (8 .. 256, the 16-bit kernels'
multiples of 8, any multiple of 4 for fp32), a value head dim, ragged query
and key lengths, a dtype, a mask kind, a bias broadcast pattern, causality
and the default or an explicit scale, then checks the output and every
gradient (dbias included) against the float64 oracle at the dtype's budget,
through the same C ABI as the fixed cases of ``test_hip_parity.py``.  The
point is combinations the fixed cases do not list; the draws are fixed by
the seeds, so a failure names a reproducible case.
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


@pytest.mark.parametrize('seed', range(48))
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
    dq, dk, dvr, db = O.sdpa_backward(q, k, v, g, bias=bias, mask=mask, scale=scale,
                                      causal=c['causal'], acc_dtype=np.float64)
    checks = [('dq', tq.grad, dq), ('dk', tk.grad, dk), ('dv', tv.grad, dvr)]
    if bias is not None:
        checks.append(('dbias', tb.grad, db))
    for name, got_t, want in checks:
        a = got_t.float().cpu().numpy()
        assert a.shape == want.shape, (name, a.shape, want.shape)
        e = relerr(a, want)
        print(f'  {name} relerr {e:.2e}', flush=True)
        assert e <= tol, f'{name} relerr {e:.3e}'
