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

import zlib

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


@pytest.mark.parametrize('name,B,H,s,t,d,dv,kw', [
    ('bf16', 2, 2, 130, 96, 128, 128, {'causal': True}),
    ('f16', 2, 3, 70, 150, 64, 64, {'mask': 'keypad'}),
    ('bf16', 1, 2, 100, 136, 64, 32, {'bias': (1, 2, 1, 136)}),
    ('bf16', 2, 2, 64, 200, 40, 40, {'bias': (2, 2, 64, 200), 'mask': 'random'}),
    ('f16', 3, 1, 257, 129, 128, 64, {'bias': (129,)}),
    ('bf16', 2, 2, 150, 140, 256, 256, {'mask': 'keypad'}),
    ('f16', 1, 2, 100, 130, 192, 256, {'causal': True, 'bias': (1, 2, 1, 130)}),
], ids=['bf16_causal_d128', 'f16_keypad_cross', 'bf16_rowbias_dv32', 'bf16_bias_mask_d40',
        'f16_shared_bias_tails', 'bf16_keypad_d256', 'f16_causal_rowbias_d192_dv256'])
def test_fused_qk_norm_backward(name, B, H, s, t, d, dv, kw):
    """qk_norm=True on the fused path with the norm's VJP inside the dQ and
    dK kernels (``nxa_bwd_normed``): every gradient against the float64
    chain rule through the oracle (normalise, round to the I/O dtype,
    attention, attention VJP, norm VJP); no separate norm backward pass
    runs."""
    from nitrix_amd import _lib, scaled_dot_product_attention

    dtype = DT[name]
    rnd = ROUND[name]
    rng = np.random.default_rng(zlib.crc32(repr((name, B, H, s, t, d, dv)).encode()))
    q = rnd(rng.standard_normal((B, H, s, d)).astype(np.float32) * 3)
    k = rnd(rng.standard_normal((B, H, t, d)).astype(np.float32) * 3)
    v = rnd(rng.standard_normal((B, H, t, dv)).astype(np.float32))
    g = rnd(rng.standard_normal((B, H, s, dv)).astype(np.float32))
    bias = None if 'bias' not in kw else rnd(rng.standard_normal(kw['bias']).astype(np.float32))
    mask = None
    if kw.get('mask') == 'keypad':
        valid = rng.integers(1, t + 1, size=B)
        mask = (np.arange(t)[None, :] < valid[:, None])[:, None, None, :]
    elif kw.get('mask') == 'random':
        mask = rng.random((B, H, s, t)) < 0.5
        mask[..., 0] = True
    causal = kw.get('causal', False)
    to = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(_dev(), dtype).requires_grad_(True)  # noqa: E731
    tq, tk, tv = to(q), to(k), to(v)
    tb = None if bias is None else to(bias)
    tm = None if mask is None else torch.from_numpy(mask).to(_dev())
    print(f'[case] fused qk-norm {name} B{B} H{H} s{s} t{t} d{d} dv{dv} {kw}', flush=True)
    _lib.profile_reset()
    _lib.profile_enable(True)
    try:
        out = scaled_dot_product_attention(tq, tk, tv, bias=tb, mask=tm, causal=causal,
                                           qk_norm=True, backend='hip')
        out.backward(torch.from_numpy(g).to(_dev(), dtype))
        torch.cuda.synchronize()
        _, n_norm_bwd = _lib.profile_read('rms_norm_bwd')
        _, n_norm_fwd = _lib.profile_read('rms_norm_fwd')
    finally:
        _lib.profile_enable(False)
        _lib.profile_reset()
    # k's norm is one pass; q's runs inside the forward kernel.
    assert n_norm_fwd == 1 and n_norm_bwd == 0, (n_norm_fwd, n_norm_bwd)
    qh = rnd(O.qk_rms_norm(q))
    kh = rnd(O.qk_rms_norm(k))
    ref = O.sdpa_forward(qh, kh, v, bias=bias, mask=mask, causal=causal, acc_dtype=np.float64)
    dqh, dkh, dvr, dbr = O.sdpa_backward(qh, kh, v, g, bias=bias, mask=mask, causal=causal,
                                         acc_dtype=np.float64)
    dq = O.qk_rms_norm_vjp(q.astype(np.float64), dqh)
    dk = O.qk_rms_norm_vjp(k.astype(np.float64), dkh)
    tol = 2e-2 if name == 'bf16' else 2e-3
    checks = [('out', out.detach(), ref), ('dq', tq.grad, dq), ('dk', tk.grad, dk),
              ('dv', tv.grad, dvr)]
    if bias is not None:
        checks.append(('dbias', tb.grad, dbr))
    for nm, got, want in checks:
        assert got.shape == want.shape, (nm, got.shape, want.shape)
        e = relerr(got.float().cpu().numpy(), want)
        print(f'  {nm} relerr {e:.2e}', flush=True)
        assert e <= tol, (nm, e)


@pytest.mark.parametrize('name,d,kw', [
    ('bf16', 128, {'mask': 'keypad'}),
    ('f16', 64, {'causal': True}),
    ('bf16', 256, {}),
    ('f16', 40, {'bias': True}),
], ids=['bf16_d128_keypad', 'f16_d64_causal', 'bf16_d256', 'f16_d40_bias'])
def test_forward_normalises_q_in_the_kernel(name, d, kw):
    """``nxa_fwd_normed``: the forward normalises its stationary q rows in
    registers and writes q_hat and the per-row rsqrt for the backward.  q_hat
    against the oracle's qk_rms_norm rounded to the I/O dtype (one rounding
    of an fp32 value: at most one ulp from the float64 result), rstd against
    float64, and the output against the same forward on q normalised by the
    separate pass (``nxa_rms_norm_fwd``)."""
    from nitrix_amd import attention as A

    dtype = DT[name]
    rnd = ROUND[name]
    rng = np.random.default_rng(zlib.crc32(repr((name, d, sorted(kw))).encode()))
    B, H, s, t = 2, 3, 300, 170
    q = rnd(rng.standard_normal((B, H, s, d)).astype(np.float32) * 3)
    q[0, 0, 5] = rnd(q[0, 0, 5] * 1e-3)  # a row whose mean square is near eps
    k = rnd(rng.standard_normal((B, H, t, d)).astype(np.float32) * 3)
    v = rnd(rng.standard_normal((B, H, t, d)).astype(np.float32))
    to = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(_dev(), dtype)  # noqa: E731
    tq, tk, tv = to(q), to(k), to(v)
    tb = to(rng.standard_normal((B, H, s, t)).astype(np.float32)) if kw.get('bias') else None
    tm = None
    if kw.get('mask') == 'keypad':
        valid = rng.integers(1, t + 1, size=B)
        tm = torch.from_numpy((np.arange(t)[None, :] < valid[:, None])[:, None, None, :]).to(_dev())
    causal = kw.get('causal', False)
    print(f'[case] nxa_fwd_normed {name} d{d} {kw}', flush=True)
    kn, _, _ = A._rms_norm_rows(tk)
    qn = torch.empty_like(tq)
    rq = torch.empty((B * H * s,), dtype=torch.float32, device=_dev())
    scale = 1.0 / np.sqrt(d)
    prep = A._Prepared(tq, kn, tv, tb, tm, scale, causal)
    o_fused, lse_fused, _ = A._forward(prep, qnorm=(qn, rq))
    o_nowrite, _, _ = A._forward(prep, qnorm=(None, None))  # a forward without a backward
    qn2, _, rq2 = A._rms_norm_rows(tq)
    o_two, lse_two, _ = A._forward(A._Prepared(qn2, kn, tv, tb, tm, scale, causal))
    torch.cuda.synchronize()
    want_q = rnd(O.qk_rms_norm(q.astype(np.float64)).astype(np.float32))
    e_q = relerr(qn.float().cpu().numpy(), want_q)
    ms = (q.astype(np.float64) ** 2).mean(-1).reshape(-1)
    e_r = np.abs(rq.cpu().numpy() / (1.0 / np.sqrt(ms + 1e-6)) - 1).max()
    differ = (qn != qn2).float().mean().item()
    e_o = relerr(o_fused.float().cpu().numpy(), o_two.float().cpu().numpy())
    e_l = np.abs(lse_fused.cpu().numpy() - lse_two.cpu().numpy()).max()
    print(f'  q_hat relerr {e_q:.2e}  rstd relerr {e_r:.2e}  q_hat differing from the '
          f'separate pass {differ:.2e}  out {e_o:.2e}  lse {e_l:.2e}', flush=True)
    assert e_q <= TOL[name], e_q
    assert e_r <= 1e-6, e_r
    assert differ <= 1e-3, differ  # only fp32 values at a rounding tie can differ
    assert e_o <= TOL[name] and e_l <= 1e-2, (e_o, e_l)
    assert torch.equal(o_nowrite, o_fused)


def test_qk_norm_outside_the_fused_backward_uses_the_norm_passes():
    """Shapes the fused qk-norm backward does not take (fp32 I/O; q
    broadcast over the batch) run the norm kernels as separate passes, with
    the same results as the oracle chain."""
    from nitrix_amd import _lib, scaled_dot_product_attention

    rng = np.random.default_rng(77)
    for dtype, qshape in ((torch.float32, (2, 2, 40, 32)), (torch.bfloat16, (1, 2, 40, 32))):
        rnd = O.round_bf16 if dtype == torch.bfloat16 else (lambda x: x)
        q = rnd(rng.standard_normal(qshape).astype(np.float32) * 2)
        k = rnd(rng.standard_normal((2, 2, 50, 32)).astype(np.float32) * 2)
        v = rnd(rng.standard_normal((2, 2, 50, 32)).astype(np.float32))
        g = rnd(rng.standard_normal((2, 2, 40, 32)).astype(np.float32))
        tq, tk, tv = (torch.from_numpy(a).to(_dev(), dtype).requires_grad_(True) for a in (q, k, v))
        _lib.profile_reset()
        _lib.profile_enable(True)
        try:
            out = scaled_dot_product_attention(tq, tk, tv, qk_norm=True, backend='hip')
            out.backward(torch.from_numpy(g).to(_dev(), dtype))
            torch.cuda.synchronize()
            _, n_norm_bwd = _lib.profile_read('rms_norm_bwd')
        finally:
            _lib.profile_enable(False)
            _lib.profile_reset()
        assert n_norm_bwd == 2
        qb = np.broadcast_to(q, (2, 2, 40, 32))
        qh = rnd(O.qk_rms_norm(qb))
        kh = rnd(O.qk_rms_norm(k))
        dqh, dkh, dvr, _ = O.sdpa_backward(qh, kh, v, g, acc_dtype=np.float64)
        dq = O.unbroadcast(O.qk_rms_norm_vjp(qb.astype(np.float64), dqh), q.shape)
        dk = O.qk_rms_norm_vjp(k.astype(np.float64), dkh)
        tol = 2e-2 if dtype == torch.bfloat16 else 1e-5
        for nm, got, want in (('dq', tq.grad, dq), ('dk', tk.grad, dk), ('dv', tv.grad, dvr)):
            e = relerr(got.float().cpu().numpy(), want)
            assert e <= tol, (dtype, nm, e)


@pytest.mark.parametrize('seed', range(64))
def test_fused_qk_norm_random_configuration(seed):
    """Seeded random problems on the fused qk-norm path (bf16 / fp16): head
    dims 8-256 with d_v != d in about a third, ragged lengths, key padding
    or random masks, full or query-broadcast biases, causal; out at the
    dtype's attention budget, every gradient against the float64 chain
    (normalise, round, attention, attention VJP with delta from the stored
    output as the reference's backward forms it, norm VJP)."""
    from nitrix_amd import scaled_dot_product_attention

    rng = np.random.default_rng(5000 + seed)
    name = ('bf16', 'f16')[seed % 2]
    dtype, rnd = DT[name], ROUND[name]
    tol = 2e-2 if name == 'bf16' else 2e-3
    d = int(rng.choice([8, 40, 64, 72, 96, 128, 136, 192, 256]))
    dv = d if rng.random() < 0.7 else int(rng.choice([8, 32, 64, 128, 256]))
    B, H = int(rng.integers(1, 3)), int(rng.integers(1, 3))
    s, t = int(rng.integers(2, 260)), int(rng.integers(2, 300))
    causal = bool(rng.random() < 0.3)
    mk = str(rng.choice(['none', 'keypad', 'random']))
    bk = str(rng.choice(['none', 'full', 'row']))
    q = rnd(rng.standard_normal((B, H, s, d)).astype(np.float32) * 3)
    k = rnd(rng.standard_normal((B, H, t, d)).astype(np.float32) * 3)
    v = rnd(rng.standard_normal((B, H, t, dv)).astype(np.float32))
    g = rnd(rng.standard_normal((B, H, s, dv)).astype(np.float32))
    bshape = {'none': None, 'full': (B, H, s, t), 'row': (B, H, 1, t)}[bk]
    bias = None if bshape is None else rnd(rng.standard_normal(bshape).astype(np.float32))
    mask = None
    if mk == 'keypad':
        valid = rng.integers(1, t + 1, size=B)
        mask = (np.arange(t)[None, :] < valid[:, None])[:, None, None, :]
    elif mk == 'random':
        mask = rng.random((B, H, s, t)) < 0.5
        mask[..., 0] = True
    print(f'[case] qk-norm seed {seed}: {name} B{B} H{H} s{s} t{t} d{d} dv{dv} '
          f'causal={causal} mask={mk} bias={bk}', flush=True)
    to = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(_dev(), dtype).requires_grad_(True)  # noqa: E731
    tq, tk, tv = to(q), to(k), to(v)
    tb = None if bias is None else to(bias)
    tm = None if mask is None else torch.from_numpy(np.ascontiguousarray(mask)).to(_dev())
    out = scaled_dot_product_attention(tq, tk, tv, bias=tb, mask=tm, causal=causal,
                                       qk_norm=True, backend='hip')
    out.backward(torch.from_numpy(g).to(_dev(), dtype))
    torch.cuda.synchronize()
    qh, kh = rnd(O.qk_rms_norm(q)), rnd(O.qk_rms_norm(k))
    ref = O.sdpa_forward(qh, kh, v, bias=bias, mask=mask, causal=causal, acc_dtype=np.float64)
    o = out.detach().float().cpu().numpy().astype(np.float64)
    e = relerr(o, ref)
    print(f'  out relerr {e:.2e}', flush=True)
    assert e <= tol, ('out', e)
    dqh, dkh, dvr, dbr = O.sdpa_backward(qh, kh, v, g, bias=bias, mask=mask, causal=causal,
                                         acc_dtype=np.float64, out=o)
    checks = [('dq', tq.grad, O.qk_rms_norm_vjp(q.astype(np.float64), dqh)),
              ('dk', tk.grad, O.qk_rms_norm_vjp(k.astype(np.float64), dkh)),
              ('dv', tv.grad, dvr)]
    if bias is not None:
        checks.append(('dbias', tb.grad, dbr))
    for nm, got, want in checks:
        e = relerr(got.float().cpu().numpy(), want)
        print(f'  {nm} relerr {e:.2e}', flush=True)
        assert e <= tol, (nm, e)
