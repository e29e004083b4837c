"""Dispatch, loud fallback and the memory contract on the GPU.

Mirrors the reference's device-side dispatch and memory tests
(``tests/test_nn_attention_kernel.py:159-170`` qk_norm=False byte identity,
``:197-252`` no (s, t) temporary in the forward or the backward,
``:258-270`` ``auto`` uses the fused kernel without a warning, ``:283-316``
an untileable shape falls back loudly to a byte-identical reference output):

* ``backend='auto'`` on a gfx950 device runs the HIP library (no warning)
  and matches the oracle;
* shapes the fused gate declines (float64, a head dim above 256, a bf16
  head dim that is not a multiple of 8) each give exactly one
  ``NitrixBackendFallback`` and the reference engine's output, byte for
  byte; ``NITRIX_STRICT_BACKEND=1`` turns that into ``NitrixBackendError``;
* ``qk_norm=False`` is byte-identical to leaving qk_norm out;
* ``qk_upcast`` with bf16 inputs runs the reference engine under ``auto``
  and raises under ``hip``; with float32 inputs the fused kernel runs;
* the peak memory a forward, and a forward + backward, allocate stays below
  one fp32 (s, t) score matrix (``torch.cuda.max_memory_allocated``), and
  the dbias of a bias shared over many (batch, head) pairs needs far less
  than one fp32 score matrix per pair.
"""

from __future__ import annotations

import warnings

import numpy as np
import pytest
import torch

from nitrix_amd import (
    NitrixBackendError,
    NitrixBackendFallback,
    reset_fallback_state,
    scaled_dot_product_attention,
)
from oracle import attention as O

pytestmark = pytest.mark.gpu


def _dev():
    return torch.device('cuda:0')


def _rand(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32).to(_dev(), dtype)


def _relerr(a, b):
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


@pytest.fixture(autouse=True)
def _clean(monkeypatch):
    for k in ('NITRIX_BACKEND', 'NITRIX_SILENCE_FALLBACK', 'NITRIX_STRICT_BACKEND'):
        monkeypatch.delenv(k, raising=False)
    reset_fallback_state()
    yield
    reset_fallback_state()


def _fallbacks(rec):
    return [w for w in rec if issubclass(w.category, NitrixBackendFallback)]


def test_auto_dispatch_uses_the_hip_library_without_warning():
    from nitrix_amd import _lib

    print('[case] auto dispatch', flush=True)
    q, k, v = (_rand((2, 2, 128, 64), torch.bfloat16, s) for s in (1, 2, 3))
    _lib.profile_reset()
    _lib.profile_enable(True)
    try:
        with warnings.catch_warnings(record=True) as rec:
            warnings.simplefilter('always')
            out = scaled_dot_product_attention(q, k, v, backend='auto')
        torch.cuda.synchronize()
        _, launches = _lib.profile_read('fwd')
    finally:
        _lib.profile_enable(False)
        _lib.profile_reset()
    assert not _fallbacks(rec)
    assert launches == 1, 'auto did not run the fused forward'
    ref = O.sdpa_forward(*(x.float().cpu().numpy() for x in (q, k, v)), acc_dtype=np.float64)
    assert _relerr(out.float().cpu().numpy(), ref) <= 2e-2
    hip = scaled_dot_product_attention(q, k, v, backend='hip')
    assert torch.equal(out, hip)


@pytest.mark.parametrize('up', [True, False])
def test_qk_upcast_dispatch_on_the_device(up):
    """bf16 with ``qk_upcast`` set asks for sub-float32 accumulation: ``auto``
    runs the reference engine (no fused launch, no warning, the reference's
    bits) and ``hip`` raises; with float32 inputs the knob changes nothing
    and ``hip`` runs the fused kernel."""
    from nitrix_amd import _lib
    from nitrix_amd import reference_scaled_dot_product_attention as ref_sdpa

    print(f'[case] qk_upcast={up} dispatch', flush=True)
    q, k, v = (_rand((2, 2, 96, 64), torch.bfloat16, s) for s in (31, 32, 33))
    _lib.profile_reset()
    _lib.profile_enable(True)
    try:
        with warnings.catch_warnings(record=True) as rec:
            warnings.simplefilter('always')
            out = scaled_dot_product_attention(q, k, v, qk_upcast=up, backend='auto')
        torch.cuda.synchronize()
        _, launches = _lib.profile_read('fwd')
    finally:
        _lib.profile_enable(False)
        _lib.profile_reset()
    assert not _fallbacks(rec)
    assert launches == 0, 'a sub-float32 request ran the fused forward'
    assert torch.equal(out, ref_sdpa(q, k, v, qk_upcast=up))
    with pytest.raises(NitrixBackendError, match='below float32'):
        scaled_dot_product_attention(q, k, v, qk_upcast=up, backend='hip')
    qf, kf, vf = (x.float() for x in (q, k, v))
    fused = scaled_dot_product_attention(qf, kf, vf, qk_upcast=up, backend='hip')
    want = O.sdpa_forward(*(x.cpu().numpy() for x in (qf, kf, vf)), acc_dtype=np.float64)
    assert _relerr(fused.cpu().numpy(), want) <= 1e-5


UNTILEABLE = {
    'float64': ((2, 2, 64, 32), (2, 2, 64, 32), torch.float64),
    'head_dim_264': ((2, 2, 64, 264), (2, 2, 64, 264), torch.bfloat16),
    'bf16_head_dim_12': ((2, 2, 64, 12), (2, 2, 64, 12), torch.bfloat16),
}


@pytest.mark.parametrize('reason', sorted(UNTILEABLE))
def test_untileable_shape_falls_back_loudly(reason):
    print(f'[case] fallback {reason}', flush=True)
    qs, ks, dtype = UNTILEABLE[reason]
    q, k, v = _rand(qs, dtype, 4), _rand(ks, dtype, 5), _rand(ks, dtype, 6)
    with warnings.catch_warnings(record=True) as rec:
        warnings.simplefilter('always')
        out = scaled_dot_product_attention(q, k, v, backend='hip')
        again = scaled_dot_product_attention(q, k, v, backend='hip')
    assert len(_fallbacks(rec)) == 1  # once per (shape, dtype), then quiet
    ref = scaled_dot_product_attention(q, k, v, backend='jax')
    assert torch.equal(out, ref) and torch.equal(again, ref)


def test_strict_backend_turns_the_fallback_into_an_error(monkeypatch):
    monkeypatch.setenv('NITRIX_STRICT_BACKEND', '1')
    qs, ks, dtype = UNTILEABLE['head_dim_264']
    q, k, v = _rand(qs, dtype, 4), _rand(ks, dtype, 5), _rand(ks, dtype, 6)
    with pytest.raises(NitrixBackendError):
        scaled_dot_product_attention(q, k, v, backend='hip')


def test_qk_norm_false_is_byte_identical_to_no_norm():
    q, k, v = (_rand((2, 2, 96, 64), torch.bfloat16, s) for s in (7, 8, 9))
    a = scaled_dot_product_attention(q, k, v, qk_norm=False, backend='hip')
    b = scaled_dot_product_attention(q, k, v, backend='hip')
    assert torch.equal(a, b)


def _peak_bytes(fn):
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    res = fn()
    torch.cuda.synchronize()
    return torch.cuda.max_memory_allocated() - base, res


@pytest.mark.parametrize('with_mask', [False, True], ids=['plain', 'keypad'])
def test_forward_and_backward_hold_no_score_matrix(with_mask):
    """At s = 4096 one fp32 (s, t) score matrix is 64 MiB; the fused forward
    and forward + backward allocate far less (outputs, lse, tile map and
    per-row values), while the reference engine needs several."""
    b, h, s, d = 1, 1, 4096, 64
    print(f'[case] peak memory s={s} mask={with_mask}', flush=True)
    q, k, v = (_rand((b, h, s, d), torch.bfloat16, i).requires_grad_(True) for i in (1, 2, 3))
    g = _rand((b, h, s, d), torch.bfloat16, 4)
    mask = None
    if with_mask:
        mask = (torch.arange(s, device=_dev()) < 3000)[None, None, None, :]
    score = b * h * s * s * 4

    def fwd(backend):
        def run():
            with torch.no_grad():
                return scaled_dot_product_attention(q, k, v, mask=mask, backend=backend)
        return run

    def fwd_bwd(backend):
        def run():
            out = scaled_dot_product_attention(q, k, v, mask=mask, backend=backend)
            out.backward(g)
            return out
        return run

    pk, _ = _peak_bytes(fwd('hip'))
    pr, _ = _peak_bytes(fwd('jax'))
    print(f'  forward peak: hip {pk / 2**20:.1f} MiB, reference {pr / 2**20:.1f} MiB', flush=True)
    assert pk < score and pk < pr
    pk, _ = _peak_bytes(fwd_bwd('hip'))
    for x in (q, k, v):
        x.grad = None
    pr, _ = _peak_bytes(fwd_bwd('jax'))
    print(f'  fwd+bwd peak: hip {pk / 2**20:.1f} MiB, reference {pr / 2**20:.1f} MiB', flush=True)
    assert pk < score and pk < pr


def test_shared_bias_gradient_memory_is_bounded():
    """A bias shared by 128 batch entries ([1, 1, 2048, 2048]): the dbias
    reduction runs over the (batch, head) pairs in chunks, so the backward
    needs the fp32 accumulator of the bias plus one chunk of partials --
    here well under half of the 2 GiB that one fp32 partial per pair would
    take -- and its gradient matches the reference engine's."""
    B, H, L, D = 128, 1, 2048, 64
    print(f'[case] shared-bias dbias memory B{B} L{L}', flush=True)
    q, k, v = (_rand((B, H, L, D), torch.bfloat16, i).requires_grad_(True) for i in (1, 2, 3))
    bias = _rand((L, L), torch.bfloat16, 4).requires_grad_(True)
    g = _rand((B, H, L, D), torch.bfloat16, 5)
    per_pair = B * H * L * L * 4

    def run():
        out = scaled_dot_product_attention(q, k, v, bias=bias, backend='hip')
        out.backward(g)
        return out

    peak, _ = _peak_bytes(run)
    print(f'  fwd+bwd peak {peak / 2**20:.1f} MiB (one partial per pair: '
          f'{per_pair / 2**20:.0f} MiB)', flush=True)
    assert peak < per_pair / 2
    got = bias.grad.float()
    bias.grad = None
    qf, kf, vf = (x.detach().float().requires_grad_(True) for x in (q, k, v))
    bf = bias.detach().float().requires_grad_(True)
    ref = scaled_dot_product_attention(qf, kf, vf, bias=bf, backend='jax')
    ref.backward(g.float())
    e = float((got - bf.grad).abs().max() / bf.grad.abs().max())
    print(f'  dbias relerr vs reference engine {e:.2e}', flush=True)
    assert e <= 2e-2
