"""Selective scan on the CPU (no GPU needed): the C ABI's host checks and
workspace sizes, the reference engine's three drivers against the pinned
oracle (``oracle/ssm.py``) and the reference's golden fixture, its autograd
against the oracle VJP, and the dispatcher's validation / backend rules
(``src/nitrix/nn/ssm/__init__.py:40-202``)."""

from __future__ import annotations

import warnings

import numpy as np
import pytest
import torch
from _golden import load_golden

from nitrix_amd import _lib
from nitrix_amd._backend import NitrixBackendError, NitrixBackendFallback, reset_fallback_state
from nitrix_amd.attention import HipNotTileable
from nitrix_amd.ssm import (
    _check_tileable,
    reference_selective_scan,
    selective_scan,
)
from oracle import ssm as S


@pytest.fixture(scope='module')
def lib():
    if not _lib.LIB_PATH.exists():
        from nitrix_amd import _build

        _build.build()
    return _lib.lib()


def _inputs(b, length, d, n, seed, with_d=True, dtype=np.float64):
    # tests/test_nn_ssm.py:44-57 of the reference: softplus delta, A = -exp(randn).
    rng = np.random.RandomState(seed)
    lead = () if b is None else (b,)
    x = rng.standard_normal(lead + (length, d))
    delta = np.log1p(np.exp(rng.standard_normal(lead + (length, d))))
    A = -np.exp(rng.standard_normal((d, n)))
    B = rng.standard_normal(lead + (length, n))
    C = rng.standard_normal(lead + (length, n))
    D = rng.standard_normal((d,)) if with_d else None
    return tuple(None if t is None else t.astype(dtype) for t in (x, delta, A, B, C, D))


def _t(arrs):
    return tuple(None if a is None else torch.from_numpy(np.ascontiguousarray(a)) for a in arrs)


# --- C ABI host checks ------------------------------------------------------


def test_check_codes(lib):
    assert lib.nxa_ssm_check(2, 64, 8, 4) == _lib.NXA_OK
    assert lib.nxa_ssm_check(1, 1, 1, 1) == _lib.NXA_OK
    assert lib.nxa_ssm_check(1, 100, 300, 32) == _lib.NXA_OK
    assert lib.nxa_ssm_check(1, 64, 8, 33) == _lib.NXA_E_UNSUPPORTED
    assert b'33' in lib.nxa_last_error()
    for bad in [(0, 64, 8, 4), (1, 0, 8, 4), (1, 64, 0, 4), (1, 64, 8, 0), (-1, 64, 8, 4)]:
        assert lib.nxa_ssm_check(*bad) == _lib.NXA_E_SHAPE, bad


def test_state_and_workspace_sizes(lib):
    nb, length, d, n = 2, 100, 300, 5
    np_, nc, ns, ndblk = 8, 4, 13, 2  # padded states, 32-step chunks, 8-step sub-chunks
    assert lib.nxa_ssm_state_bytes(nb, length, d, n) == nb * ns * np_ * d * 4

    def a256(x):
        return (x + 255) // 256 * 256

    hc = a256(nb * nc * np_ * d * 4)
    sdt = a256(nb * nc * d * 4)
    dbc = a256(ndblk * nb * length * 2 * np_ * 4)
    dad = a256(16 * (np_ + 1) * d * 4)  # 16 row groups of the dA / dD sums
    assert lib.nxa_ssm_workspace_bytes(nb, length, d, n, 0) == hc + sdt
    assert lib.nxa_ssm_workspace_bytes(nb, length, d, n, 1) == hc + 2 * sdt + dbc + dad
    assert lib.nxa_ssm_state_bytes(1, 64, 8, 40) == 0
    # 16 states: the backward chunk pass runs two lanes per channel, so its
    # dB / dC partials come from blocks of 128 channels
    hc16 = a256(nb * nc * 16 * d * 4)
    dbc16 = a256(3 * nb * length * 2 * 16 * 4)
    dad16 = a256(16 * 17 * d * 4)
    assert lib.nxa_ssm_workspace_bytes(nb, length, d, 16, 1) == hc16 + 2 * sdt + dbc16 + dad16


def test_no_state_trajectory_in_memory(lib):
    # The reference's gross-memory contract (tests/test_nn_ssm_kernel.py:104-145):
    # what the fused path keeps besides its inputs and outputs stays below one
    # (l, d, n) float32 trajectory, forward and backward.
    b, length, d, n = 2, 128, 8, 4
    traj = b * length * d * n * 4
    fwd = lib.nxa_ssm_workspace_bytes(b, length, d, n, 0) + lib.nxa_ssm_state_bytes(b, length, d, n)
    bwd = lib.nxa_ssm_workspace_bytes(b, length, d, n, 1) + lib.nxa_ssm_state_bytes(b, length, d, n)
    assert fwd < traj
    assert bwd < traj
    # and at a Mamba-sized shape the saved states are an eighth of it
    b, length, d, n = 8, 2048, 1536, 16
    assert lib.nxa_ssm_state_bytes(b, length, d, n) * 8 == b * length * d * n * 4


def test_entry_points_reject_null_buffers_without_a_gpu(lib):
    args = [1, 64, 8, 4] + [None] * 9 + [0, None]
    assert lib.nxa_ssm_fwd(*args) == _lib.NXA_E_ARG
    assert b'x is NULL' in lib.nxa_last_error()
    args = [1, 64, 8, 4] + [None] * 15 + [0, None]
    assert lib.nxa_ssm_bwd(*args) == _lib.NXA_E_ARG
    assert lib.nxa_ssm_fwd(1, 64, 8, 40, *([None] * 9), 0, None) == _lib.NXA_E_UNSUPPORTED


def test_entry_points_reject_small_or_misaligned_workspace(lib):
    host = np.zeros(1 << 16, np.uint8)
    base = (host.ctypes.data + 255) // 256 * 256
    f = [base] * 6  # x, delta, A, B, C, D (host addresses: never dereferenced)
    need = lib.nxa_ssm_workspace_bytes(1, 64, 8, 4, 0)
    assert lib.nxa_ssm_fwd(1, 64, 8, 4, *f, base, None, base, need - 1, None) == _lib.NXA_E_WORKSPACE
    assert lib.nxa_ssm_fwd(1, 64, 8, 4, *f, base, None, base + 4, need, None) == _lib.NXA_E_WORKSPACE
    assert lib.nxa_ssm_fwd(1, 64, 8, 4, base + 2, *f[1:], base, None, base, need, None) == _lib.NXA_E_LAYOUT


# --- reference engine ---------------------------------------------------------


def test_reference_engine_matches_golden_fixture():
    g = load_golden('selective_scan_float32')
    out = reference_selective_scan(*_t([g['x'], g['delta'], g['A'], g['B'], g['C'], g['D']]),
                                   driver='sequential')
    assert out.dtype == torch.float32
    np.testing.assert_allclose(out.numpy(), g['out'], atol=1e-5, rtol=1e-4)


@pytest.mark.parametrize('driver', ['sequential', 'associative', 'chunked', 'auto'])
@pytest.mark.parametrize('with_d', [False, True])
def test_reference_engine_drivers_match_oracle(driver, with_d):
    arrs = _inputs(2, 64, 5, 3, seed=11, with_d=with_d)
    want = S.selective_scan(*arrs)
    got = reference_selective_scan(*_t(arrs), driver=driver, chunk_size=16)
    np.testing.assert_allclose(got.numpy(), want, atol=1e-10, rtol=1e-10)


def test_reference_engine_upcasts_half_precision():
    arrs = _inputs(1, 16, 4, 2, seed=12, dtype=np.float32)
    t = [None if a is None else torch.from_numpy(a).to(torch.bfloat16) for a in arrs]
    got = reference_selective_scan(*t)
    assert got.dtype == torch.bfloat16
    want = S.selective_scan(*[None if a is None else a.float().numpy() for a in t])
    np.testing.assert_allclose(got.float().numpy(), want.astype(np.float32), rtol=1e-2, atol=1e-2)


def test_reference_engine_autograd_matches_oracle_vjp():
    arrs = _inputs(2, 12, 3, 4, seed=13)
    dy = np.random.RandomState(14).standard_normal(arrs[0].shape)
    ts = [t.requires_grad_(True) for t in _t(arrs)]
    y = reference_selective_scan(*ts, driver='sequential')
    y.backward(torch.from_numpy(dy))
    want = S.selective_scan_vjp(*arrs, dy)
    for t, w in zip(ts, want):
        np.testing.assert_allclose(t.grad.numpy(), w, atol=1e-10, rtol=1e-9)


def test_chunked_driver_requires_divisible_length():
    arrs = _t(_inputs(1, 40, 3, 2, seed=15))
    with pytest.raises(ValueError, match='chunk_size'):
        reference_selective_scan(*arrs, driver='chunked', chunk_size=16)


# --- dispatcher ----------------------------------------------------------------


@pytest.mark.parametrize('mutate,msg', [
    (lambda a: (a[0], a[1][..., :-1], *a[2:]), 'x and delta must match'),
    (lambda a: (a[0], a[1], a[2][:, :1].T, *a[3:]), 'A must be'),
    (lambda a: (*a[:3], a[3][..., :-1], *a[4:]), 'B/C last dim'),
    (lambda a: (*a[:4], a[4][..., :-1, :], a[5]), 'B/C sequence dim'),
    (lambda a: (*a[:5], a[5][:-1]), 'D must be'),
])
def test_validation_messages(mutate, msg):
    arrs = _t(_inputs(2, 8, 4, 3, seed=16))
    with pytest.raises(ValueError, match=msg):
        selective_scan(*mutate(arrs))


def test_driver_contradicts_fused_backend():
    arrs = _t(_inputs(1, 8, 4, 3, seed=17))
    with pytest.raises(NitrixBackendError, match='driver'):
        selective_scan(*arrs, driver='sequential', backend='hip')


def test_cpu_tensors_run_the_reference_engine_quietly():
    arrs = _inputs(1, 8, 4, 3, seed=18)
    reset_fallback_state()
    with warnings.catch_warnings():
        warnings.simplefilter('error', NitrixBackendFallback)
        out = selective_scan(*_t(arrs))
    np.testing.assert_allclose(out.numpy(), S.selective_scan(*arrs), atol=1e-12)


def test_explicit_hip_backend_on_cpu_tensors_raises():
    with pytest.raises(NitrixBackendError, match='gfx950'):
        selective_scan(*_t(_inputs(1, 8, 4, 3, seed=19)), backend='hip')


@pytest.mark.parametrize('case', ['float64', 'n33'])
def test_tileability_gate(case):
    if case == 'float64':
        arrs = _t(_inputs(1, 8, 4, 3, seed=20))
    else:
        arrs = _t(_inputs(1, 8, 4, 33, seed=20, dtype=np.float32))
    with pytest.raises(HipNotTileable):
        _check_tileable(*arrs)
    _check_tileable(*_t(_inputs(1, 8, 4, 32, seed=20, dtype=np.float32)))
