"""The ``qk_upcast`` stage-precision knob of the reference engine (CPU).

The reference keeps the knob open and unbuilt; its own determination
(``docs/feature-requests/attention-no-upcast-knob.md``, "nitrix
determination" and "Tests") fixes what it must do, and these tests follow
that list:

* the default (``qk_upcast=None``) is the unchanged reference, and with
  float32 / float64 inputs ``True`` and ``False`` give the same bits;
* ``qk_upcast=True`` casts the float32 softmax probabilities back to the
  I/O dtype before the value product (the ``upcast_attention=True``
  regime): pinned on a case where that rounding decides the result, and
  against a float64 emulation of the regime;
* ``qk_upcast=False`` keeps every stage in the I/O dtype, so fp16 logits
  above 65504 overflow (the documented footgun) where the default and
  ``qk_upcast=True`` stay finite;
* a sub-float32 request with ``backend='hip'`` (or ``'pallas-cuda'``)
  raises, ``'auto'`` resolves to the reference engine (the reference's
  ``SPEC.md`` tenet 11, corollary (a)).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from nitrix_amd import (
    NitrixBackendError,
    reference_scaled_dot_product_attention as ref_sdpa,
    scaled_dot_product_attention,
)
from oracle import attention as O


def _rand(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32).to(dtype)


def _bf16_round(x: np.ndarray) -> np.ndarray:
    """float64 -> nearest bf16 (ties to even), returned as float64."""
    f = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((f + 0x7FFF + ((f >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32).astype(np.float64)


def _round_to(x: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    if dtype == torch.bfloat16:
        return _bf16_round(x)
    return np.asarray(x, np.float16).astype(np.float64)


@pytest.mark.parametrize('dtype', [torch.float32, torch.float64])
@pytest.mark.parametrize('causal', [False, True])
def test_full_precision_inputs_are_unchanged(dtype, causal):
    q, k, v = (_rand((2, 3, 40, 16), dtype, s) for s in (1, 2, 3))
    bias = _rand((3, 40, 40), dtype, 4)
    mask = _rand((2, 1, 40, 40), torch.float32, 5) > -1.0
    base = ref_sdpa(q, k, v, bias=bias, mask=mask, causal=causal)
    for up in (True, False):
        got = scaled_dot_product_attention(q, k, v, bias=bias, mask=mask, causal=causal,
                                           qk_upcast=up, backend='jax')
        assert torch.equal(got, base), up


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16])
def test_default_is_the_reference(dtype):
    q, k, v = (_rand((2, 2, 24, 8), dtype, s) for s in (6, 7, 8))
    a = scaled_dot_product_attention(q, k, v, backend='jax')
    b = scaled_dot_product_attention(q, k, v, qk_upcast=None, backend='jax')
    assert torch.equal(a, b)
    want = O.sdpa_forward(*(x.double().numpy() for x in (q, k, v)),
                          scale=1 / np.sqrt(8), acc_dtype=np.float64)
    assert np.max(np.abs(a.double().numpy() - want)) / np.max(np.abs(want)) < 1e-2


def test_upcast_rounds_the_probabilities_to_the_io_dtype():
    """Two keys whose probabilities (0.50035, 0.49965) both round to 0.5 in
    bf16, values +-1000: the value product of the rounded probabilities is
    0, that of the float32 ones 0.69."""
    d = 8
    q = torch.zeros(1, 1, 1, d)
    q[..., 0] = 1.0
    k = torch.zeros(1, 1, 2, d)
    k[..., 0, 0] = 0.5
    k[..., 1, 0] = 0.5 - 2.0 ** -8
    v = torch.zeros(1, 1, 2, d)
    v[..., 0, :] = 1000.0
    v[..., 1, :] = -1000.0
    q, k, v = (x.to(torch.bfloat16) for x in (q, k, v))
    up = scaled_dot_product_attention(q, k, v, qk_upcast=True, backend='jax')
    full = scaled_dot_product_attention(q, k, v, backend='jax')
    assert float(up.abs().max()) == 0.0
    assert 0.6 < float(full[..., 0, 0]) < 0.8


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16])
def test_upcast_matches_an_emulation_of_the_regime(dtype):
    """Scores and softmax exact (float64) on the I/O-dtype inputs, the
    probabilities rounded to the I/O dtype, the value product exact, the
    output rounded: within one rounding of the I/O dtype of the knob."""
    q, k, v = (_rand((2, 2, 33, 16), dtype, s) for s in (9, 10, 11))
    got = scaled_dot_product_attention(q, k, v, qk_upcast=True, backend='jax')
    qn, kn, vn = (x.double().numpy() for x in (q, k, v))
    s = qn @ np.swapaxes(kn, -1, -2) / 4.0
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    want = _round_to(_round_to(p, dtype) @ vn, dtype)
    ulp = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10
    err = np.abs(got.double().numpy() - want)
    assert np.all(err <= ulp * np.maximum(np.abs(want), 1e-3) + 1e-6), float(err.max())


def test_native_fp16_overflows_where_the_upcast_does_not():
    """Logits of 60 * 60 * 64 = 230,400 exceed fp16's 65,504."""
    q = torch.full((1, 1, 4, 64), 60.0, dtype=torch.float16)
    k = torch.full((1, 1, 5, 64), 60.0, dtype=torch.float16)
    v = _rand((1, 1, 5, 64), torch.float16, 12)
    native = scaled_dot_product_attention(q, k, v, qk_upcast=False, backend='jax')
    assert not torch.isfinite(native).all()
    for up in (None, True):
        assert torch.isfinite(scaled_dot_product_attention(q, k, v, qk_upcast=up,
                                                           backend='jax')).all()


@pytest.mark.parametrize('backend', ['hip', 'pallas-cuda'])
@pytest.mark.parametrize('up', [True, False])
def test_sub_fp32_request_on_the_fused_backend_raises(backend, up):
    q, k, v = (_rand((1, 2, 16, 8), torch.bfloat16, s) for s in (13, 14, 15))
    with pytest.raises(NitrixBackendError, match='below float32'):
        scaled_dot_product_attention(q, k, v, qk_upcast=up, backend=backend)


@pytest.mark.parametrize('up', [True, False])
def test_auto_resolves_to_the_reference(up):
    q, k, v = (_rand((1, 2, 16, 8), torch.float16, s) for s in (16, 17, 18))
    got = scaled_dot_product_attention(q, k, v, qk_upcast=up, backend='auto')
    assert torch.equal(got, ref_sdpa(q, k, v, qk_upcast=up))


def test_gradients_flow_through_the_upcast_regime():
    q, k, v = (_rand((1, 2, 12, 8), torch.bfloat16, s).requires_grad_() for s in (19, 20, 21))
    out = scaled_dot_product_attention(q, k, v, qk_upcast=True, backend='jax')
    out.float().sum().backward()
    for t in (q, k, v):
        assert t.grad is not None and torch.isfinite(t.grad.float()).all()
