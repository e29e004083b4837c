"""Host-side behaviour of the drop-in on the CPU (no GPU needed).

Mirrors the reference's dispatch / fallback / validation tests
(``tests/test_nn_attention.py:259-340``, ``tests/test_backend.py:19-131``,
``tests/test_nn_attention_kernel.py:283-347``):

* backend resolution: keyword > ``NITRIX_BACKEND`` > auto, reproducible mode,
  explicit fused backends on a host without gfx950 raise;
* the loud, deduplicated fallback warning and its env knobs;
* input validation raises ``ValueError`` as the reference does;
* the tileability gate of the fused path;
* the unfused reference engine (``backend='jax'``) against the reference's
  golden fixtures and the oracle, and ``_unbroadcast`` / descriptor building.
"""

from __future__ import annotations

import warnings

import numpy as np
import pytest
import torch
from _golden import ATTENTION_CASES, CROSS_ATOL, TOL, load_golden

import nitrix_amd
from nitrix_amd import _backend, attention
from oracle import attention as O


@pytest.fixture(autouse=True)
def _clean_env(monkeypatch):
    for k in ('NITRIX_BACKEND', 'NITRIX_SILENCE_FALLBACK', 'NITRIX_STRICT_BACKEND'):
        monkeypatch.delenv(k, raising=False)
    _backend.reset_fallback_state()
    yield
    _backend.reset_fallback_state()


CPU = torch.device('cpu')


def test_auto_on_cpu_is_reference_and_silent():
    with warnings.catch_warnings():
        warnings.simplefilter('error')
        assert _backend.resolve_backend('auto', CPU) == 'jax'


def test_explicit_hip_on_cpu_raises():
    with pytest.raises(_backend.NitrixBackendError):
        _backend.resolve_backend('hip', CPU)


def test_pallas_cuda_raises_on_this_build():
    with pytest.raises(_backend.NitrixBackendError):
        _backend.resolve_backend('pallas-cuda', CPU)


def test_invalid_backend_raises():
    with pytest.raises(_backend.NitrixBackendError):
        _backend.resolve_backend('triton', CPU)


def test_env_backend(monkeypatch):
    monkeypatch.setenv('NITRIX_BACKEND', 'jax')
    assert _backend.resolve_backend('auto', CPU) == 'jax'
    monkeypatch.setenv('NITRIX_BACKEND', 'hip')
    with pytest.raises(_backend.NitrixBackendError):
        _backend.resolve_backend('auto', CPU)
    monkeypatch.setenv('NITRIX_BACKEND', 'bogus')
    with pytest.raises(_backend.NitrixBackendError):
        _backend.resolve_backend('auto', CPU)
    # an explicit keyword wins over the env var
    monkeypatch.setenv('NITRIX_BACKEND', 'hip')
    assert _backend.resolve_backend('jax', CPU) == 'jax'


def test_reproducible_forces_reference():
    with nitrix_amd.reproducible():
        assert _backend.reproducible_enabled()
        assert _backend.auto_backend(CPU) == 'jax'
    assert not _backend.reproducible_enabled()


def _warn_once():
    return _backend.fallback(
        function='f', requested='hip', resolved='jax', reason='r',
        shapes=((1, 2),), dtype='float32',
    )


def test_fallback_warns_once_per_key():
    with pytest.warns(_backend.NitrixBackendFallback):
        assert _warn_once() == 'jax'
    with warnings.catch_warnings():
        warnings.simplefilter('error')
        _warn_once()  # deduplicated
    _backend.reset_fallback_state()
    with pytest.warns(_backend.NitrixBackendFallback):
        _warn_once()


def test_fallback_silence_and_strict(monkeypatch):
    monkeypatch.setenv('NITRIX_SILENCE_FALLBACK', '1')
    with warnings.catch_warnings():
        warnings.simplefilter('error')
        _warn_once()
    monkeypatch.setenv('NITRIX_STRICT_BACKEND', '1')
    with pytest.raises(_backend.NitrixBackendError):
        _warn_once()


def test_no_fallback_when_requested_equals_resolved():
    with warnings.catch_warnings():
        warnings.simplefilter('error')
        assert _backend.fallback(
            function='f', requested='jax', resolved='jax', reason='r'
        ) == 'jax'


# --- validation (__init__.py:40-60) ------------------------------------------


@pytest.mark.parametrize(
    'shapes',
    [((3, 4), (2, 3, 4), (2, 3, 4)), ((2, 3, 4), (2, 3, 5), (2, 3, 5)),
     ((2, 3, 4), (2, 3, 4), (2, 5, 4))],
)
def test_validate_raises_value_error(shapes):
    q, k, v = (torch.zeros(s) for s in shapes)
    with pytest.raises(ValueError):
        nitrix_amd.scaled_dot_product_attention(q, k, v)


# --- tileability gate ---------------------------------------------------------


@pytest.mark.parametrize(
    'dtype, d, dv, ok',
    [
        (torch.bfloat16, 64, 64, True),
        (torch.bfloat16, 128, 128, True),
        (torch.bfloat16, 40, 40, True),
        (torch.float32, 12, 12, True),
        (torch.float16, 64, 64, True),
        (torch.float16, 24, 24, True),
        (torch.float16, 12, 12, False),
        (torch.float64, 64, 64, False),
        (torch.bfloat16, 64, 32, True),
        (torch.float32, 64, 12, True),
        (torch.bfloat16, 64, 136, True),
        (torch.bfloat16, 256, 256, True),
        (torch.float32, 196, 128, True),
        (torch.bfloat16, 64, 20, False),
        (torch.bfloat16, 264, 264, False),
        (torch.float16, 64, 512, False),
        (torch.bfloat16, 12, 12, False),
    ],
)
def test_check_tileable(dtype, d, dv, ok):
    q = torch.zeros(1, 2, 5, d, dtype=dtype)
    k = torch.zeros(1, 2, 7, d, dtype=dtype)
    v = torch.zeros(1, 2, 7, dv, dtype=dtype)
    if ok:
        attention._check_tileable(q, k, v)
    else:
        with pytest.raises(attention.HipNotTileable):
            attention._check_tileable(q, k, v)


def test_mixed_dtypes_are_not_tileable():
    q = torch.zeros(1, 2, 5, 64, dtype=torch.bfloat16)
    k = torch.zeros(1, 2, 7, 64, dtype=torch.float32)
    with pytest.raises(attention.HipNotTileable):
        attention._check_tileable(q, k, k)


# --- the reference engine -----------------------------------------------------


@pytest.mark.parametrize('name', ATTENTION_CASES)
def test_reference_engine_golden(name):
    data = load_golden(name)
    t = {k: torch.from_numpy(v) for k, v in data.items() if v.ndim > 0}
    out = nitrix_amd.scaled_dot_product_attention(
        t['q'], t['k'], t['v'], bias=t.get('bias'),
        causal=bool(data['causal']),
        qk_norm=bool(data['qk_norm']) if 'qk_norm' in data else False,
        backend='jax',
    ).numpy()
    if name == 'attention_cross_float32':
        np.testing.assert_allclose(out, data['out'], atol=CROSS_ATOL, rtol=0)
    else:
        atol, rtol = TOL[('attention', 'float32')]
        np.testing.assert_allclose(out, data['out'], atol=atol, rtol=rtol)


def test_reference_engine_matches_oracle_float64_with_mask_and_grads():
    rng = np.random.default_rng(4)
    q = rng.standard_normal((2, 3, 5, 4))
    k = rng.standard_normal((2, 3, 6, 4))
    v = rng.standard_normal((2, 3, 6, 4))
    bias = rng.standard_normal((3, 5, 6))
    mask = rng.random((2, 1, 5, 6)) < 0.7
    mask[..., 0] = True
    g = rng.standard_normal((2, 3, 5, 4))
    tq, tk, tv, tb = (torch.from_numpy(x).requires_grad_() for x in (q, k, v, bias))
    out = nitrix_amd.scaled_dot_product_attention(
        tq, tk, tv, bias=tb, mask=torch.from_numpy(mask), causal=True,
        backend='jax',
    )
    out.backward(torch.from_numpy(g))
    want = O.sdpa_forward(q, k, v, bias=bias, mask=mask, causal=True)
    np.testing.assert_allclose(out.detach().numpy(), want, atol=1e-12)
    dq, dk, dv, db = O.sdpa_backward(q, k, v, g, bias=bias, mask=mask, causal=True)
    for got, ref in ((tq.grad, dq), (tk.grad, dk), (tv.grad, dv), (tb.grad, db)):
        np.testing.assert_allclose(got.numpy(), ref, atol=1e-10)


def test_reference_engine_bf16_invariant():
    # reduced precision == float32 path on the bf16 inputs, cast back
    # (tests/test_nn_mixed_precision.py:127-135)
    rng = np.random.default_rng(5)
    x = [torch.from_numpy(rng.standard_normal((2, 2, 7, 8)).astype(np.float32))
         for _ in range(3)]
    xb = [t.to(torch.bfloat16) for t in x]
    a = nitrix_amd.scaled_dot_product_attention(*xb, backend='jax')
    b = nitrix_amd.scaled_dot_product_attention(
        *(t.float() for t in xb), backend='jax'
    ).to(torch.bfloat16)
    assert a.dtype == torch.bfloat16
    assert torch.equal(a, b)


def test_qk_norm_false_is_identical():
    rng = np.random.default_rng(6)
    q, k, v = (torch.from_numpy(rng.standard_normal((1, 2, 4, 8))) for _ in range(3))
    a = nitrix_amd.scaled_dot_product_attention(q, k, v, backend='jax')
    b = nitrix_amd.reference_scaled_dot_product_attention(q, k, v)
    assert torch.equal(a, b)


def test_default_scale():
    assert attention.default_scale(64) == 0.125


# --- host-side plumbing of the fused path -------------------------------------


@pytest.mark.parametrize(
    'g_shape, target',
    [((2, 3, 4, 5), (3, 4, 5)), ((2, 3, 4, 5), (1, 3, 1, 5)), ((2, 3, 4, 5), (5,))],
)
def test_unbroadcast_matches_oracle(g_shape, target):
    g = np.random.default_rng(7).standard_normal(g_shape)
    got = attention._unbroadcast(torch.from_numpy(g), target).numpy()
    np.testing.assert_allclose(got, O.unbroadcast(g, target), atol=1e-12)


def test_descriptor_uses_zero_strides_for_broadcast_operands():
    q = torch.zeros(2, 4, 100, 64, dtype=torch.bfloat16)
    k = torch.zeros(2, 4, 70, 64, dtype=torch.bfloat16)
    bias = torch.zeros(4, 1, 70, dtype=torch.bfloat16)        # over batch and queries
    mask = torch.ones(2, 1, 1, 70, dtype=torch.bool)          # key padding
    prep = attention._Prepared(q, k, k, bias, mask, 0.125, True)
    d = prep.desc
    assert (d.B, d.H, d.Lq, d.Lk, d.D) == (2, 4, 100, 70, 64)
    assert tuple(d.bias_str) == (0, 70, 0)
    assert tuple(d.mask_str) == (70, 0, 0)
    assert tuple(d.q_str) == (4 * 100 * 64, 100 * 64, 64)
    assert d.causal == 1 and abs(d.scale - 0.125) < 1e-9
    assert attention._dbias_geometry(prep) == (1, 4, 1)


def test_descriptor_flattens_leading_axes():
    q = torch.zeros(2, 3, 4, 10, 8, dtype=torch.float32)
    k = torch.zeros(1, 3, 4, 12, 8, dtype=torch.float32)      # broadcast over axis 0
    prep = attention._Prepared(q, k, k, None, None, 1.0, False)
    assert prep.nb == 6 and prep.h == 4
    assert prep.desc.B == 6 and prep.desc.k_str[0] % 4 == 0
