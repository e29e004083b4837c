"""Fused selective scan on the GPU: ``nxa_ssm_fwd`` / ``nxa_ssm_bwd`` through
the host API against the pinned CPU oracle (``oracle/ssm.py``).

Budgets, ``max|a-b| / max|b|`` against the float64 oracle: forward 2e-5 and
every cotangent 2e-4 for float32 inputs (the reference holds its fused path
to 2e-3 forward, ``tests/tolerance.toml:33-35``, and 3e-3 on gradients,
``tests/test_nn_ssm_kernel.py:47``); bfloat16 / float16 inputs the reference's
reduced-precision rows (``tolerance.toml:71-76``, as relative budgets 2e-2 /
1e-2) against the oracle on the same rounded inputs.  At the Mamba-sized bench
shape, where the float64 oracle VJP does not fit in seconds, the forward is
compared with the oracle and the backward with identities any correct VJP
satisfies: y is linear in x, in B and in C, so <dx, x> = <dB, B> = <dC, C> =
<dy, y - D x> (+ <dy, D x> for dx); y is unchanged by (delta, A, B) ->
(s delta, A / s, B / s), so <ddelta, delta> = <dA, A> + <dB, B>; and
dD = sum dy x.
"""

from __future__ import annotations

import warnings

import numpy as np
import pytest
import torch
from _golden import relerr

from nitrix_amd._backend import NitrixBackendFallback, reset_fallback_state
from nitrix_amd.ssm import selective_scan, selective_scan_hip
from oracle import ssm as S

pytestmark = pytest.mark.gpu

FWD_TOL = 2e-5
GRAD_TOL = 2e-4


def _dev():
    return torch.device('cuda:0')


def _inputs(lead, length, d, n, seed, with_d=True, regime='softplus'):
    """float32 numpy inputs.  'softplus': tests/test_nn_ssm.py:44-57 of the
    reference (delta = softplus(randn), A = -exp(randn)); 'mamba':
    tests/test_nn_ssm_kernel.py:50-62 (delta in [0.01, 0.1], A = -(1..n))."""
    rng = np.random.RandomState(seed)
    lead = tuple(lead)
    x = rng.standard_normal(lead + (length, d))
    if regime == 'mamba':
        delta = 0.01 + 0.09 / (1.0 + np.exp(-rng.standard_normal(lead + (length, d))))
        A = -np.repeat((np.arange(n) + 1.0)[None, :], d, 0)
    else:
        delta = np.log1p(np.exp(rng.standard_normal(lead + (length, d))))
        A = -np.exp(rng.standard_normal((d, n)))
    B = rng.standard_normal(lead + (length, n))
    C = rng.standard_normal(lead + (length, n))
    D = rng.standard_normal((d,)) if with_d else None
    return [None if t is None else t.astype(np.float32) for t in (x, delta, A, B, C, D)]


def _gpu(arrs, dtype=torch.float32, grad=False):
    out = []
    for a in arrs:
        if a is None:
            out.append(None)
            continue
        t = torch.from_numpy(np.ascontiguousarray(a)).to(_dev(), dtype)
        out.append(t.requires_grad_(grad))
    return out


def _run(arrs, dy, dtype=torch.float32):
    ts = _gpu(arrs, dtype, grad=True)
    y = selective_scan_hip(*ts)
    y.backward(torch.from_numpy(dy).to(_dev(), dtype))
    torch.cuda.synchronize()
    grads = [None if t is None else t.grad.float().cpu().numpy() for t in ts]
    return y.detach().float().cpu().numpy(), grads


CASES = [
    # (lead, L, d, n, with_d, regime)
    ((2,), 64, 8, 4, True, 'mamba'),     # the reference's kernel-test shape
    ((2,), 64, 8, 4, False, 'mamba'),
    ((), 128, 4, 4, True, 'mamba'),      # no batch axis, longer sequence
    ((3,), 100, 300, 5, True, 'softplus'),   # ragged L, d > 256, n not a power of two
    ((1,), 1, 1, 1, True, 'softplus'),   # smallest
    ((2,), 33, 257, 16, True, 'mamba'),
    ((1,), 257, 64, 32, True, 'mamba'),  # widest state
    ((2, 3), 40, 8, 8, False, 'softplus'),   # two batch axes
    ((1,), 7, 3, 3, True, 'softplus'),
    ((2,), 96, 128, 16, True, 'softplus'),
]
IDS = ['ref64', 'ref64_noD', 'nobatch128', 'ragged', 'one', 'd257n16', 'n32', 'lead2',
       'tiny', 'n16']


@pytest.mark.parametrize('case', CASES, ids=IDS)
def test_forward_and_gradients_match_oracle(case):
    lead, length, d, n, with_d, regime = case
    seed = 7 * length + d + n
    print(f'[case] ssm lead={lead} L={length} d={d} n={n} D={with_d} {regime}', flush=True)
    arrs = _inputs(lead, length, d, n, seed, with_d, regime)
    dy = np.random.RandomState(seed + 1).standard_normal(arrs[0].shape).astype(np.float32)
    y, grads = _run(arrs, dy)
    a64 = [None if a is None else a.astype(np.float64) for a in arrs]
    want = S.selective_scan(*a64)
    ey = relerr(y, want)
    wg = S.selective_scan_vjp(*a64, dy.astype(np.float64))
    eg = [relerr(g, w) for g, w in zip(grads, wg) if w is not None]
    print(f'  y {ey:.2e}  grads ' + ' '.join(f'{e:.2e}' for e in eg), flush=True)
    assert ey <= FWD_TOL, ey
    for g in grads:
        if g is not None:
            assert np.all(np.isfinite(g))
    assert max(eg) <= GRAD_TOL, eg


def test_loss_of_squares_gradient_like_the_reference():
    # tests/test_nn_ssm_kernel.py:151-170: grad of sum(y^2), with and without D.
    for with_d in (False, True):
        arrs = _inputs((2,), 64, 8, 4, 3, with_d, 'mamba')
        ts = _gpu(arrs, grad=True)
        y = selective_scan_hip(*ts)
        (y ** 2).sum().backward()
        torch.cuda.synchronize()
        a64 = [None if a is None else a.astype(np.float64) for a in arrs]
        want = S.selective_scan_vjp(*a64, 2 * S.selective_scan(*a64))
        for t, w in zip(ts, want):
            if t is not None:
                assert relerr(t.grad.cpu().numpy(), w) < GRAD_TOL


def test_broadcast_B_C_gradients_are_summed():
    arrs = _inputs((2,), 48, 16, 4, 21, True, 'softplus')
    arrs[3] = arrs[3][0]  # B (l, n) shared over the batch
    dy = np.random.RandomState(22).standard_normal(arrs[0].shape).astype(np.float32)
    y, grads = _run(arrs, dy)
    a64 = [a.astype(np.float64) for a in arrs]
    Bb = np.broadcast_to(a64[3], a64[4].shape)
    want = S.selective_scan(a64[0], a64[1], a64[2], Bb, a64[4], a64[5])
    assert relerr(y, want) <= FWD_TOL
    wg = S.selective_scan_vjp(a64[0], a64[1], a64[2], Bb, a64[4], a64[5], dy.astype(np.float64))
    assert grads[3].shape == arrs[3].shape
    assert relerr(grads[3], wg[3].sum(0)) <= GRAD_TOL


@pytest.mark.parametrize('name,dtype,tol', [('bf16', torch.bfloat16, 2e-2),
                                            ('f16', torch.float16, 1e-2)])
def test_half_precision_inputs(name, dtype, tol):
    """bf16 / fp16 inputs: upcast at the boundary, fp32 kernels, outputs and
    gradients cast back to the input dtype (and B / C gradients summed over
    a broadcast batch), against the oracle and its VJP on the same rounded
    inputs and cotangent."""
    arrs = _inputs((2,), 64, 96, 16, 31, True, 'mamba')
    arrs[3] = arrs[3][0]  # B shared over the batch
    ts = _gpu(arrs, dtype, grad=True)
    print(f'[case] ssm {name}', flush=True)
    y = selective_scan_hip(*ts)
    assert y.dtype == dtype
    rounded = [t.detach().float().cpu().numpy().astype(np.float64) for t in ts]
    Bb = np.broadcast_to(rounded[3], rounded[4].shape)
    want = S.selective_scan(rounded[0], rounded[1], rounded[2], Bb, rounded[4], rounded[5])
    e = relerr(y.detach().float().cpu().numpy(), want)
    print(f'  y {e:.2e}', flush=True)
    assert e <= tol
    dy = torch.from_numpy(
        np.random.RandomState(32).standard_normal(arrs[0].shape).astype(np.float32)
    ).to(_dev(), dtype)
    y.backward(dy)
    torch.cuda.synchronize()
    wg = list(S.selective_scan_vjp(rounded[0], rounded[1], rounded[2], Bb, rounded[4],
                                   rounded[5], dy.float().cpu().numpy().astype(np.float64)))
    wg[3] = wg[3].sum(0)
    for name_, t, w in zip(('dx', 'ddelta', 'dA', 'dB', 'dC', 'dD'), ts, wg):
        assert t.grad is not None and t.grad.dtype == dtype, name_
        assert t.grad.shape == t.shape, name_
        e = relerr(t.grad.float().cpu().numpy(), w)
        print(f'  {name_} {e:.2e}', flush=True)
        assert e <= tol, f'{name_} relerr {e:.3e}'


def test_in_place_change_before_backward_raises():
    """The inputs are kept with save_for_backward: editing one in place
    between forward and backward raises instead of giving wrong gradients."""
    arrs = _inputs((2,), 40, 64, 8, 33, True)
    ts = _gpu(arrs, torch.float32, grad=True)
    y = selective_scan_hip(*ts)
    with torch.no_grad():
        ts[1].mul_(2.0)
    # torch words it as a version-counter error or, for a view made inside
    # the forward, as an in-place change of that view's base.
    with pytest.raises(RuntimeError, match='inplace'):
        y.backward(torch.ones_like(y))


def test_deterministic():
    arrs = _inputs((2,), 200, 600, 16, 41, True, 'softplus')
    dy = np.random.RandomState(42).standard_normal(arrs[0].shape).astype(np.float32)
    y1, g1 = _run(arrs, dy)
    y2, g2 = _run(arrs, dy)
    assert np.array_equal(y1, y2)
    for a, b in zip(g1, g2):
        assert np.array_equal(a, b)


def test_auto_dispatch_uses_kernel_without_warning():
    arrs = _gpu(_inputs((2,), 64, 8, 4, 4, True, 'mamba'))
    reset_fallback_state()
    with warnings.catch_warnings(record=True) as rec:
        warnings.simplefilter('always')
        out = selective_scan(*arrs, backend='auto')
    assert not [w for w in rec if issubclass(w.category, NitrixBackendFallback)]
    a64 = [None if a is None else a.double().cpu().numpy() for a in arrs]
    assert relerr(out.cpu().numpy(), S.selective_scan(*a64)) <= FWD_TOL


def test_float64_falls_back_loudly():
    arrs = _gpu(_inputs((2,), 64, 8, 4, 6, True, 'mamba'), torch.float64)
    reset_fallback_state()
    with warnings.catch_warnings(record=True) as rec:
        warnings.simplefilter('always')
        out = selective_scan(*arrs, backend='hip')
    assert len([w for w in rec if issubclass(w.category, NitrixBackendFallback)]) == 1
    a64 = [a.cpu().numpy() for a in arrs]
    assert relerr(out.cpu().numpy(), S.selective_scan(*a64)) < 1e-12


def test_bench_shape_forward_and_vjp_identities():
    # The bench workload: batch 8, L 2048, d 1536, n 16, with D.
    lead, length, d, n = (8,), 2048, 1536, 16
    print('[case] ssm bench shape', flush=True)
    arrs = _inputs(lead, length, d, n, 51, True, 'mamba')
    dy = np.random.RandomState(52).standard_normal(arrs[0].shape).astype(np.float32)
    y, (dx, ddelta, dA, dB, dC, dD) = _run(arrs, dy)
    a64 = [a.astype(np.float64) for a in arrs]
    ey = relerr(y, S.selective_scan(*a64))
    x, delta, A, B, C, D = a64
    dy = dy.astype(np.float64)
    y = y.astype(np.float64)
    core = float(np.sum(dy * (y - D * x)))   # <dy, y - D x>
    skip = float(np.sum(dy * D * x))
    checks = {
        'dx': (float(np.sum(dx * x)), core + skip),
        'dB': (float(np.sum(dB * B)), core),
        'dC': (float(np.sum(dC * C)), core),
        'ddelta': (float(np.sum(ddelta * delta)), float(np.sum(dA * A) + np.sum(dB * B))),
    }
    ed = relerr(dD, np.sum(dy * x, axis=(0, 1)))
    print(f'  y {ey:.2e} dD {ed:.2e} ' + ' '.join(
        f'{k} {abs(a - b) / abs(b):.2e}' for k, (a, b) in checks.items()), flush=True)
    assert ey <= FWD_TOL
    assert ed <= GRAD_TOL
    for k, (a, b) in checks.items():
        assert abs(a - b) <= 1e-4 * abs(b), (k, a, b)


def test_inference_forward_matches_training_forward():
    # Without gradients the forward keeps no sub-chunk states (state NULL);
    # the output is the same bits.
    arrs = _inputs((3,), 77, 200, 12, 61, True, 'softplus')
    with torch.no_grad():
        y0 = selective_scan_hip(*_gpu(arrs)).cpu().numpy()
    y1 = selective_scan_hip(*_gpu(arrs, grad=True)).detach().cpu().numpy()
    assert np.array_equal(y0, y1)


@pytest.mark.parametrize('seed', range(64))
def test_random_shapes(seed):
    rng = np.random.RandomState(100 + seed)
    lead = tuple(int(v) for v in rng.randint(1, 3, size=rng.randint(0, 3)))
    length, d, n = int(rng.randint(1, 300)), int(rng.randint(1, 700)), int(rng.randint(1, 33))
    with_d = bool(rng.randint(2))
    regime = ('mamba', 'softplus')[seed % 2]
    print(f'[case] ssm random lead={lead} L={length} d={d} n={n} D={with_d} {regime}',
          flush=True)
    arrs = _inputs(lead, length, d, n, 200 + seed, with_d, regime)
    dy = rng.standard_normal(arrs[0].shape).astype(np.float32)
    y, grads = _run(arrs, dy)
    a64 = [None if a is None else a.astype(np.float64) for a in arrs]
    assert relerr(y, S.selective_scan(*a64)) <= FWD_TOL
    wg = S.selective_scan_vjp(*a64, dy.astype(np.float64))
    for g, w in zip(grads, wg):
        if w is not None:
            assert relerr(g, w) <= GRAD_TOL

