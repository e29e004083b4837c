"""qk-norm on the fused path (GPU only): ``nxa_rms_norm_fwd`` / ``_bwd``
through the C ABI against the oracle's ``qk_rms_norm`` and
``qk_rms_norm_vjp`` (pinned in ``test_oracle.py``), and attention with
``qk_norm=True`` end to end with gradients.

Budgets (``max|a-b| / max|b|`` against float64): the forward and the VJP are
one rounding of an fp32 computation to the I/O dtype, which can land one
output ulp from the float64 value: bf16 <= 8e-3 (2^-7), fp16 <= 2e-3 (twice
2^-10), fp32 <= 1e-5.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from _golden import relerr

from oracle import attention as O

pytestmark = pytest.mark.gpu

DT = {'bf16': torch.bfloat16, 'f16': torch.float16, 'f32': torch.float32}
ROUND = {'bf16': O.round_bf16, 'f16': O.round_f16, 'f32': lambda x: x}
TOL = {'bf16': 8e-3, 'f16': 2e-3, 'f32': 1e-5}


def _dev():
    return torch.device('cuda:0')


@pytest.mark.parametrize('name', ['bf16', 'f16', 'f32'])
@pytest.mark.parametrize('shape,width', [
    ((2, 3, 50, 64), 64),
    ((1, 2, 7, 256), 256),
    ((3, 40), 40),
    ((2, 33, 64), 96),   # rows of a wider buffer: row stride 96, D = 64
], ids=['bhld64', 'd256', 'd40', 'strided'])
def test_rms_norm_forward_and_vjp(name, shape, width):
    from nitrix_amd.attention import _RmsNormHip

    rng = np.random.default_rng(1000 * ['bf16', 'f16', 'f32'].index(name) + width)
    dtype = DT[name]
    full = ROUND[name](rng.standard_normal(shape[:-1] + (width,)).astype(np.float32) * 3)
    full[..., 0, :] *= 1e-3  # small rows: mean square near eps
    x = full[..., : shape[-1]]
    g = ROUND[name](rng.standard_normal(shape).astype(np.float32))
    print(f'[case] rms norm {name} shape={shape} width={width}', flush=True)
    tfull = torch.from_numpy(np.ascontiguousarray(full)).to(_dev(), dtype)
    tx = tfull[..., : shape[-1]].detach().requires_grad_(True)
    y = _RmsNormHip.apply(tx)
    y.backward(torch.from_numpy(g).to(_dev(), dtype))
    torch.cuda.synchronize()
    want_y = O.qk_rms_norm(x.astype(np.float64))
    want_dx = O.qk_rms_norm_vjp(x.astype(np.float64), g.astype(np.float64))
    ey = relerr(y.detach().float().cpu().numpy(), want_y)
    ed = relerr(tx.grad.float().cpu().numpy(), want_dx)
    print(f'  y relerr {ey:.2e}  dx relerr {ed:.2e}', flush=True)
    assert ey <= TOL[name], ey
    assert ed <= TOL[name], ed


def test_attention_qk_norm_bf16_with_grads():
    """bf16 attention with qk_norm through the fused path: the norm in the
    I/O dtype before the kernel (``nn/attention/__init__.py:196-197``), the
    cotangents of q and k through the norm's VJP."""
    from nitrix_amd import scaled_dot_product_attention

    rng = np.random.default_rng(31)
    B, H, s, t, d = 2, 2, 90, 110, 64
    q, k, v, g = (O.round_bf16(rng.standard_normal(sh).astype(np.float32) * c)
                  for sh, c in (((B, H, s, d), 3), ((B, H, t, d), 3), ((B, H, t, d), 1),
                                ((B, H, s, d), 1)))
    tq, tk, tv = (torch.from_numpy(a).to(_dev(), torch.bfloat16).requires_grad_(True)
                  for a in (q, k, v))
    print('[case] attention qk_norm bf16', flush=True)
    out = scaled_dot_product_attention(tq, tk, tv, qk_norm=True, causal=True, backend='hip')
    out.backward(torch.from_numpy(g).to(_dev(), torch.bfloat16))
    torch.cuda.synchronize()
    qh = O.round_bf16(O.qk_rms_norm(q))  # the fused path normalises in bf16
    kh = O.round_bf16(O.qk_rms_norm(k))
    ref = O.sdpa_forward(qh, kh, v, causal=True, acc_dtype=np.float64)
    dqh, dkh, dv, _ = O.sdpa_backward(qh, kh, v, g, causal=True, acc_dtype=np.float64)
    dq = O.qk_rms_norm_vjp(q.astype(np.float64), dqh)
    dk = O.qk_rms_norm_vjp(k.astype(np.float64), dkh)
    for nm, got, want in (('out', out.detach(), ref), ('dq', tq.grad, dq),
                          ('dk', tk.grad, dk), ('dv', tv.grad, dv)):
        e = relerr(got.float().cpu().numpy(), want)
        print(f'  {nm} relerr {e:.2e}', flush=True)
        assert e <= 2e-2, (nm, e)
