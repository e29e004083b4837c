"""Parity of the fused gfx950 path against the CPU oracle (GPU only).

Every case runs the public drop-in (``scaled_dot_product_attention(...,
backend='hip')``, which calls ``nxa_fwd`` / ``nxa_bwd`` through the C ABI)
on seeded inputs and compares it with the float64 oracle on the same values:

* bf16 I/O: the oracle sees the bf16-rounded inputs upcast to float; the
  budget is ``max|a-b| / max|b| <= 2e-2`` for the output and every gradient;
* fp16 I/O: the same on fp16-rounded inputs, budget ``<= 2e-3`` (the
  reference's fused-path budget, ``tests/tolerance.toml:20-22``, twice its
  fp16 quantisation budget ``:62-64``);
* fp32 I/O: ``<= 1e-5`` for the output and the gradients.

Cases mirror the reference's fused-path tests
(``tests/test_nn_attention_kernel.py:60-140``: dense / bias / causal / mask /
cross, grads incl. dbias) and add what this kernel must get right: tails
(lengths that are not tile multiples), head dims below the padded width,
every bias broadcast pattern, key-padding / random / block-sparse masks,
causal with s != t, and fully masked rows (NaN, as the reference).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from _golden import ATTENTION_CASES, CROSS_ATOL, TOL, load_golden, relerr

from oracle import attention as O

pytestmark = pytest.mark.gpu

REL = {torch.bfloat16: 2e-2, torch.float16: 2e-3, torch.float32: 1e-5}


def _dev():
    return torch.device('cuda:0')


def _draw(rng, shape, dtype):
    x = rng.standard_normal(shape).astype(np.float32)
    if dtype == torch.bfloat16:
        x = O.round_bf16(x)
    elif dtype == torch.float16:
        x = O.round_f16(x)
    return x


def _to(x, dtype, req=False):
    t = torch.from_numpy(np.ascontiguousarray(x)).to(_dev(), dtype)
    return t.requires_grad_(req)


def _make_mask(rng, kind, B, H, s, t):
    if kind is None:
        return None
    if kind == 'keypad':
        valid = rng.integers(1, t + 1, size=B)
        m = np.arange(t)[None, :] < valid[:, None]
        return m[:, None, None, :]
    if kind == 'random':
        m = rng.random((B, H, s, t)) < 0.6
        m[..., 0] = True
        return m
    if kind == 'block':
        nbq, nbk = -(-s // 64), -(-t // 64)
        blk = rng.random((nbq, nbk)) < 0.35
        for i in range(min(nbq, nbk)):
            blk[i, i] = True
        m = np.kron(blk, np.ones((64, 64), bool))[:s, :t]
        m[:, 0] = True
        return m[None, None]
    if kind == 'rowbcast':
        m = rng.random((1, H, 1, t)) < 0.5
        m[..., 0] = True
        return m
    if kind == 'gaps':
        # 64-blocks kept with p = 0.3 plus the diagonal, nothing else: the
        # kept tiles of a row or column of blocks have gaps anywhere,
        # including before the first, and every query keeps itself.
        nbq, nbk = -(-s // 64), -(-t // 64)
        blk = rng.random((nbq, nbk)) < 0.3
        for i in range(min(nbq, nbk)):
            blk[i, i] = True
        return np.kron(blk, np.ones((64, 64), bool))[:s, :t][None, None]
    if kind == 'blocky':
        # 64-blocks kept with a density that differs per block row (2-90 %):
        # the blocks of one head differ widely in work, so the kernels run
        # them far from index order (longest first).
        nbq, nbk = -(-s // 64), -(-t // 64)
        dens = rng.uniform(0.02, 0.9, size=(nbq, 1))
        blk = rng.random((nbq, nbk)) < dens
        blk[:, 0] = True
        return np.kron(blk, np.ones((64, 64), bool))[:s, :t][None, None]
    if kind == 'blocky_bh':
        # the same, drawn per batch and head: every head has its own order
        nbq, nbk = -(-s // 64), -(-t // 64)
        dens = rng.uniform(0.02, 0.9, size=(B, H, nbq, 1))
        blk = rng.random((B, H, nbq, nbk)) < dens
        blk[..., 0] = True
        return np.kron(blk, np.ones((64, 64), bool))[..., :s, :t]
    raise ValueError(kind)


def _check(dtype, B, H, s, t, d, *, bias_shape=None, bias_dtype=None,
           mask_kind=None, causal=False, seed=0, grads=True, scale=None, dv=None):
    rng = np.random.default_rng(seed)
    dv = d if dv is None else dv
    q = _draw(rng, (B, H, s, d), dtype)
    k = _draw(rng, (B, H, t, d), dtype)
    v = _draw(rng, (B, H, t, dv), dtype)
    bdt = bias_dtype or dtype
    bias = None if bias_shape is None else _draw(rng, bias_shape, bdt)
    mask = _make_mask(rng, mask_kind, B, H, s, t)
    g = _draw(rng, (B, H, s, dv), dtype)
    explicit_scale = scale
    if scale is None:
        scale = 1.0 / np.sqrt(d)

    tq, tk, tv = _to(q, dtype, grads), _to(k, dtype, grads), _to(v, dtype, grads)
    tb = None if bias is None else _to(bias, bdt, grads)
    tm = None if mask is None else torch.from_numpy(mask).to(_dev())
    from nitrix_amd import scaled_dot_product_attention

    print(f'[case] {dtype} B{B} H{H} s{s} t{t} d{d} dv{dv} bias={bias_shape} '
          f'mask={mask_kind} causal={causal} seed={seed}', flush=True)
    out = scaled_dot_product_attention(
        tq, tk, tv, bias=tb, mask=tm, causal=causal, scale=explicit_scale,
        backend='hip'
    )
    ref = O.sdpa_forward(q, k, v, bias=bias, mask=mask, scale=scale,
                         causal=causal, acc_dtype=np.float64)
    tol = REL[dtype]
    got = out.detach().float().cpu().numpy()
    assert got.shape == ref.shape
    assert np.all(np.isfinite(got)), 'unexpected non-finite output'
    err = relerr(got, ref)
    print(f'  out relerr {err:.2e}', flush=True)
    assert err <= tol, f'out relerr {err:.3e} > {tol}'
    if not grads:
        return
    out.backward(_to(g, dtype))
    torch.cuda.synchronize()
    dq, dk, dv, db = O.sdpa_backward(q, k, v, g, bias=bias, mask=mask,
                                     scale=scale, causal=causal,
                                     acc_dtype=np.float64)
    pairs = [('dq', tq.grad, dq), ('dk', tk.grad, dk), ('dv', tv.grad, dv)]
    if bias is not None:
        pairs.append(('dbias', tb.grad, db))
    for name, got_t, want in pairs:
        assert got_t is not None, name
        got = got_t.float().cpu().numpy()
        assert got.shape == want.shape, (name, got.shape, want.shape)
        e = relerr(got, want)
        # dbias is stored in the bias dtype: its rounding sets the floor.
        t_ = max(tol, REL[bdt]) if name == 'dbias' else tol
        print(f'  {name} relerr {e:.2e}', flush=True)
        assert e <= t_, f'{name} relerr {e:.3e} > {t_}'


DTYPES = [torch.bfloat16, torch.float16, torch.float32]
IDS = ['bf16', 'f16', 'f32']


@pytest.mark.parametrize('dtype', DTYPES, ids=IDS)
@pytest.mark.parametrize('d', [64, 128])
def test_dense(dtype, d):
    _check(dtype, 2, 2, 256, 256, d)


@pytest.mark.parametrize('dtype', DTYPES, ids=IDS)
@pytest.mark.parametrize('s,t,d', [(100, 77, 64), (33, 200, 128), (6, 9, 8),
                                   (130, 129, 40), (1, 65, 64)])
def test_tails_and_padded_head_dim(dtype, s, t, d):
    _check(dtype, 2, 3, s, t, d, seed=s + t)


@pytest.mark.parametrize('dtype', DTYPES, ids=IDS)
@pytest.mark.parametrize('d,dv,kw', [
    (64, 128, {}),
    (128, 64, {'causal': True}),
    (40, 24, {'bias_shape': (2, 2, 150, 170), 'mask_kind': 'random'}),
    (64, 32, {'bias_shape': (1, 2, 1, 176), 'mask_kind': 'keypad'}),
], ids=['64_128', '128_64_causal', '40_24_bias_mask', '64_32_rowbias'])
def test_value_head_dim_differs(dtype, d, dv, kw):
    """v / out / dO / dv with their own head dim d_v != d (the kernels pad
    both to the same width; q.k runs over d, P.v over d_v)."""
    t = 176 if kw.get('bias_shape', (0,))[-1] == 176 else 170
    _check(dtype, 2, 2, 150, t, d, dv=dv, seed=30 + d + dv, **kw)


@pytest.mark.parametrize('dtype', DTYPES, ids=IDS)
@pytest.mark.parametrize('d,dv,s,t,kw', [
    (256, 256, 160, 150, {}),
    (256, 256, 150, 150, {'causal': True}),
    (192, 256, 130, 170, {'bias_shape': (2, 2, 130, 170), 'mask_kind': 'random'}),
    (256, 64, 100, 136, {'bias_shape': (1, 2, 1, 136), 'mask_kind': 'keypad'}),
    (136, 136, 70, 77, {'bias_shape': (2, 70, 77)}),
], ids=['256', '256_causal', '192_256_bias_mask', '256_64_rowbias', '136_tails'])
def test_wide_head_dim(dtype, d, dv, s, t, kw):
    """Head dims above 128 (padded to 256): one wave per SIMD.  16-bit I/O:
    the forward and dQ kernels with two 64 KB tile stages, dK / dV with 32-row
    query tiles and every product of a key in one wave; fp32: dV, dK and dQ
    column halves in passes of their own."""
    _check(dtype, 2, 2, s, t, d, dv=dv, seed=40 + d + dv, **kw)


def _check_levels(dtype, B, H, s, t, d, levels, *, causal=False, mask_kind=None, seed=0):
    """Forward and gradients against the float64 oracle for q, k whose logits
    follow `levels` (natural-log units, one value per 64-key tile) along the
    keys: q_i = 8 u + noise, k_j = levels[j // 64] sqrt(d) / 8 u + noise with
    u a unit vector, so that with the default scale 1/sqrt(d) the logit
    scale q_i . k_j is levels[j // 64] plus noise of order one."""
    rng = np.random.default_rng(seed)
    u = np.ones(d, np.float32) / np.sqrt(d)
    lv = np.repeat(np.asarray(levels, np.float32), 64)[:t]
    q = 8.0 * u[None, None, None, :] + 0.5 * rng.standard_normal((B, H, s, d)).astype(np.float32)
    k = (lv[None, None, :, None] * u[None, None, None, :] * (np.sqrt(d) / 8.0)
         + 0.5 * rng.standard_normal((B, H, t, d)).astype(np.float32))
    v = rng.standard_normal((B, H, t, d)).astype(np.float32)
    g = rng.standard_normal((B, H, s, d)).astype(np.float32)
    rnd = {torch.bfloat16: O.round_bf16, torch.float16: O.round_f16}.get(dtype, lambda x: x)
    q, k, v, g = rnd(q), rnd(k), rnd(v), rnd(g)
    mask = _make_mask(rng, mask_kind, B, H, s, t)
    scale = 1.0 / np.sqrt(d)
    tq, tk, tv = _to(q, dtype, True), _to(k, dtype, True), _to(v, dtype, True)
    tm = None if mask is None else torch.from_numpy(mask).to(_dev())
    from nitrix_amd import scaled_dot_product_attention

    logits = scale * np.einsum('bhsd,bhtd->bhst', q.astype(np.float64), k.astype(np.float64))
    print(f'[case] levels {dtype} B{B} H{H} s{s} t{t} d{d} causal={causal} mask={mask_kind} '
          f'logits [{logits.min():.0f}, {logits.max():.0f}]', flush=True)
    out = scaled_dot_product_attention(tq, tk, tv, mask=tm, causal=causal, backend='hip')
    ref = O.sdpa_forward(q, k, v, mask=mask, causal=causal, acc_dtype=np.float64)
    # fp32: scores this large are ill-conditioned in fp32 itself -- |q . k|
    # reaches ~3,500 (ulp 2.4e-4) before the scale, so the logits carry
    # ~1e-4 of rounding whatever the kernel; a reference that failed to
    # follow the row maximum would be off by order one.
    tol = 1e-3 if dtype == torch.float32 else REL[dtype]
    e = relerr(out.detach().float().cpu().numpy(), ref)
    print(f'  out relerr {e:.2e}', flush=True)
    assert e <= tol, f'out relerr {e:.3e}'
    out.backward(_to(g, dtype))
    torch.cuda.synchronize()
    dq, dk, dv, _ = O.sdpa_backward(q, k, v, g, mask=mask, causal=causal, acc_dtype=np.float64)
    # dQ_i = scale sum_j dS_ij k_j: along u the keys' large shared component
    # meets sum_j dS_ij = 0, so the 16-bit rounding of dS in the dQ product
    # is amplified by |k . u| / |noise| (~90 here) there -- a property of
    # any bf16 / fp16 backward, not of the row reference.  dQ is compared
    # orthogonal to u; dK and dV in full.
    def perp(x):
        return x - (x @ u.astype(np.float64))[..., None] * u.astype(np.float64)
    errs = {}
    for name, got, want in (('dq_perp_u', tq.grad, dq), ('dk', tk.grad, dk), ('dv', tv.grad, dv)):
        a = got.float().cpu().numpy().astype(np.float64)
        if name == 'dq_perp_u':
            a, want = perp(a), perp(want)
        errs[name] = relerr(a, want)
        print(f'  {name} relerr {errs[name]:.2e}', flush=True)
    for name, e in errs.items():
        assert e <= tol, f'{name} relerr {e:.3e}'


# Tile levels that rise steeply (every tile's row maximum exceeds the last by
# ~25 in natural-log units, so the forward's optimistic pass fails and the
# reference is raised on every tile), fall (the first tile holds the maximum),
# and jump up and down.
LEVELS = {
    'rising': [25.0 * i for i in range(16)],
    'falling': [25.0 * (15 - i) for i in range(16)],
    'jumps': [0, 60, -40, 90, 10, 150, 149, 30, 200, -100, 210, 0, 260, 255, 5, 300],
}


@pytest.mark.parametrize('dtype', DTYPES, ids=IDS)
@pytest.mark.parametrize('pattern', sorted(LEVELS))
def test_logits_far_above_the_running_max(dtype, pattern):
    """Rows whose maximum grows (or drops) by orders of magnitude from one
    key tile to the next: the forward's row reference must follow, with
    every output and gradient as the oracle's."""
    _check_levels(dtype, 1, 2, 96, 1000, 64, LEVELS[pattern], seed=90)


@pytest.mark.parametrize('dtype', DTYPES, ids=IDS)
@pytest.mark.parametrize('d,kw', [(128, {'mask_kind': 'keypad'}), (128, {'causal': True}),
                                  (256, {})], ids=['d128_keypad', 'd128_causal', 'd256'])
def test_rising_logits_other_kernels(dtype, d, kw):
    t = 700 if kw.get('causal') else 1000
    _check_levels(dtype, 2, 1, t if kw.get('causal') else 130, t, d, LEVELS['rising'],
                  seed=91, **kw)


@pytest.mark.parametrize('dtype', DTYPES, ids=IDS)
@pytest.mark.parametrize('s,t', [(256, 256), (200, 130), (96, 300)])
def test_causal(dtype, s, t):
    _check(dtype, 2, 2, s, t, 64, causal=True, seed=3)


@pytest.mark.parametrize('dtype', DTYPES, ids=IDS)
@pytest.mark.parametrize('bias_shape', [
    (2, 2, 192, 160),   # full
    (2, 192, 160),      # shared over batch (the windowed-bias fixture pattern)
    (1, 2, 1, 160),     # query-broadcast (distance / ALiBi-style column bias)
    (192, 160),         # shared over batch and heads
    (2, 1, 192, 160),   # shared over heads
], ids=['full', 'batchbc', 'qbc', 'bhbc', 'headbc'])
def test_bias_broadcast(dtype, bias_shape):
    _check(dtype, 2, 2, 192, 160, 64, bias_shape=bias_shape, seed=5)


@pytest.mark.parametrize('d', [64, 128])
@pytest.mark.parametrize('kind', ['full', 'qbc'])
@pytest.mark.parametrize('causal,mask_kind,scale', [
    (False, None, None),
    (True, None, None),
    (False, 'block', None),
    (True, 'random', 0.37),
], ids=['plain', 'causal', 'blockmask', 'causal_mask_scale'])
def test_bf16_bias_through_mfma(d, kind, causal, mask_kind, scale):
    """bf16 bias with Lk a multiple of 8: the forward adds the bias by MFMA
    (bias^T x diag(1/scale), 1/scale split into two bf16 terms when it is not
    a power of two), streamed through the LDS ring (full tiles) or as one key
    row per tile (query-broadcast).  Lengths leave query and key tails."""
    shape = (2, 2, 200, 136) if kind == 'full' else (1, 2, 1, 136)
    _check(torch.bfloat16, 2, 2, 200, 136, d, bias_shape=shape,
           mask_kind=mask_kind, causal=causal, seed=12 + d, scale=scale)


@pytest.mark.parametrize('d', [64, 128])
@pytest.mark.parametrize('kind', ['full', 'qbc'])
@pytest.mark.parametrize('causal,mask_kind,scale', [
    (False, None, None),
    (True, 'random', 0.37),
], ids=['plain', 'causal_mask_scale'])
def test_f16_bias_through_mfma(d, kind, causal, mask_kind, scale):
    """fp16 bias on fp16 I/O: the MFMA bias modes with 1/scale split into two
    fp16 terms (and log2(e) split likewise in the dQ row-bias product)."""
    shape = (2, 2, 200, 136) if kind == 'full' else (1, 2, 1, 136)
    _check(torch.float16, 2, 2, 200, 136, d, bias_shape=shape,
           mask_kind=mask_kind, causal=causal, seed=20 + d, scale=scale)


def test_bias_fp32_with_bf16_io():
    _check(torch.bfloat16, 2, 2, 128, 128, 64, bias_shape=(2, 2, 128, 128),
           bias_dtype=torch.float32, seed=6)


def test_bias_bf16_with_f16_io():
    """A bias dtype other than the I/O dtype takes the element-wise path."""
    _check(torch.float16, 2, 2, 128, 136, 64, bias_shape=(1, 2, 1, 136),
           bias_dtype=torch.bfloat16, seed=16)


@pytest.mark.parametrize('dtype', DTYPES, ids=IDS)
@pytest.mark.parametrize('kind', ['keypad', 'random', 'block', 'rowbcast'])
def test_masks(dtype, kind):
    _check(dtype, 2, 2, 320, 256, 64, mask_kind=kind, seed=7)


@pytest.mark.parametrize('dtype', DTYPES, ids=IDS)
@pytest.mark.parametrize('d', [64, 128])
@pytest.mark.parametrize('causal', [False, True], ids=['full', 'causal'])
def test_block_sparse_tile_lists(dtype, d, causal):
    """Block-sparse mask over 11 x 11 tiles with gaps before, between and
    after the kept tiles, with and without causality, and a
    query-broadcast bias: the kernels walk their lists of active tiles
    (read an iteration ahead) over runs that are neither contiguous nor of
    one class."""
    _check(dtype, 2, 2, 704, 700, d, bias_shape=(1, 2, 1, 700), mask_kind='gaps',
           causal=causal, seed=40 + d + int(causal))


def test_mask_bias_causal_combined():
    _check(torch.bfloat16, 2, 2, 300, 300, 128, bias_shape=(2, 300, 300),
           mask_kind='random', causal=True, seed=8)


def test_fully_masked_row_is_nan():
    rng = np.random.default_rng(9)
    q = _draw(rng, (1, 2, 70, 64), torch.bfloat16)
    k = _draw(rng, (1, 2, 90, 64), torch.bfloat16)
    v = _draw(rng, (1, 2, 90, 64), torch.bfloat16)
    mask = rng.random((1, 2, 70, 90)) < 0.5
    mask[..., 0] = True
    mask[0, 1, 5] = False
    mask[0, 0, 69] = False
    from nitrix_amd import scaled_dot_product_attention

    out = scaled_dot_product_attention(
        _to(q, torch.bfloat16), _to(k, torch.bfloat16), _to(v, torch.bfloat16),
        mask=torch.from_numpy(mask).to(_dev()), backend='hip',
    ).float().cpu().numpy()
    ref = O.sdpa_forward(q, k, v, mask=mask, acc_dtype=np.float64)
    assert np.all(np.isnan(out[0, 1, 5])) and np.all(np.isnan(out[0, 0, 69]))
    ok = ~np.isnan(ref)
    assert np.array_equal(np.isnan(out), ~ok)
    assert relerr(out[ok], ref[ok]) <= 2e-2


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16], ids=['bf16', 'f16'])
def test_key_padding_with_an_empty_batch(dtype):
    """Key padding that keeps no key of one batch (its rows are NaN, as the
    reference's) beside batches with a partial key tile: the blocks of the
    empty batch have no active tile at all, so they must end without
    staging mask bytes."""
    rng = np.random.default_rng(57)
    B, H, s, t, d = 3, 2, 200, 1000, 64
    q = _draw(rng, (B, H, s, d), dtype)
    k = _draw(rng, (B, H, t, d), dtype)
    v = _draw(rng, (B, H, t, d), dtype)
    valid = np.array([700, 0, 1000])
    mask = (np.arange(t)[None, :] < valid[:, None])[:, None, None, :]
    from nitrix_amd import scaled_dot_product_attention

    print(f'[case] key padding with an empty batch {dtype}', flush=True)
    out = scaled_dot_product_attention(
        _to(q, dtype), _to(k, dtype), _to(v, dtype),
        mask=torch.from_numpy(mask).to(_dev()), backend='hip',
    ).float().cpu().numpy()
    torch.cuda.synchronize()
    assert np.all(np.isnan(out[1]))
    ref = O.sdpa_forward(q[[0, 2]], k[[0, 2]], v[[0, 2]], mask=mask[[0, 2]],
                         acc_dtype=np.float64)
    assert np.all(np.isfinite(out[[0, 2]]))
    assert relerr(out[[0, 2]], ref) <= REL[dtype]


@pytest.mark.parametrize('name', ATTENTION_CASES)
def test_reference_golden_fixtures_fp32(name):
    """The reference's own fixtures through the fused fp32 path (d=8, s=6,
    t=6/9: head-dim padding and length tails)."""
    from nitrix_amd import scaled_dot_product_attention

    data = load_golden(name)
    kw = {}
    if 'bias' in data:
        kw['bias'] = _to(data['bias'], torch.float32)
    out = scaled_dot_product_attention(
        _to(data['q'], torch.float32),
        _to(data['k'], torch.float32),
        _to(data['v'], torch.float32),
        causal=bool(data['causal']),
        qk_norm=bool(data['qk_norm']) if 'qk_norm' in data else False,
        backend='hip',
        **kw,
    ).cpu().numpy()
    if name == 'attention_cross_float32':
        np.testing.assert_allclose(out, data['out'], atol=CROSS_ATOL, rtol=0)
    else:
        atol, rtol = TOL[('attention', 'float32')]
        np.testing.assert_allclose(out, data['out'], atol=atol, rtol=rtol)


def test_leading_batch_dims_and_broadcast_kv():
    """``(..., h, s, d)`` with two leading axes; k / v broadcast over one of
    them (zero strides in the forward, materialised for the backward)."""
    rng = np.random.default_rng(10)
    dtype = torch.bfloat16
    q = _draw(rng, (2, 3, 2, 64, 64), dtype)
    k = _draw(rng, (1, 3, 2, 80, 64), dtype)
    v = _draw(rng, (1, 3, 2, 80, 64), dtype)
    g = _draw(rng, (2, 3, 2, 64, 64), dtype)
    tq, tk, tv = _to(q, dtype, True), _to(k, dtype, True), _to(v, dtype, True)
    from nitrix_amd import scaled_dot_product_attention

    out = scaled_dot_product_attention(tq, tk, tv, backend='hip')
    out.backward(_to(g, dtype))
    kb = np.broadcast_to(k, q.shape[:-2] + k.shape[-2:])
    vb = np.broadcast_to(v, q.shape[:-2] + v.shape[-2:])
    ref = O.sdpa_forward(q, kb, vb, acc_dtype=np.float64)
    dq, dk, dv, _ = O.sdpa_backward(q, kb, vb, g, acc_dtype=np.float64)
    dk = O.unbroadcast(dk, k.shape)
    dv = O.unbroadcast(dv, v.shape)
    assert relerr(out.detach().float().cpu().numpy(), ref) <= 2e-2
    for got, want in ((tq.grad, dq), (tk.grad, dk), (tv.grad, dv)):
        assert got.shape == want.shape
        assert relerr(got.float().cpu().numpy(), want) <= 2e-2


def test_qk_norm_matches_oracle():
    rng = np.random.default_rng(11)
    dtype = torch.float32
    q = _draw(rng, (2, 2, 50, 64), dtype) * 3
    k = _draw(rng, (2, 2, 70, 64), dtype) * 3
    v = _draw(rng, (2, 2, 70, 64), dtype)
    from nitrix_amd import scaled_dot_product_attention

    out = scaled_dot_product_attention(
        _to(q, dtype), _to(k, dtype), _to(v, dtype), qk_norm=True, backend='hip'
    ).cpu().numpy()
    ref = O.sdpa_forward(q, k, v, qk_norm=True, acc_dtype=np.float64)
    assert relerr(out, ref) <= 1e-5


def test_c1_configuration_fp32():
    """BASELINE configs[0] at its exact configuration: fp32, B1 H4 L256 D64,
    full additive bias [1,4,256,256] ~N(0,1), no mask, non-causal, default
    scale; forward and every gradient (dbias included) against the float64
    oracle on the whole problem at 1e-5."""
    _check(torch.float32, 1, 4, 256, 256, 64, bias_shape=(1, 4, 256, 256), seed=101)


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32], ids=['bf16', 'f32'])
@pytest.mark.parametrize('B,bias_shape', [
    (8, (4, 64, 4096)),       # shared over the batch: 2 chunks of 16 pairs
    (8, (8, 1, 64, 4096)),    # shared over heads
    (5, (64, 4096)),          # shared over batch and heads: chunks of 16 + 4
    (8, (1, 4, 1, 4096)),     # query-broadcast, shared over the batch
], ids=['batch', 'head', 'both_uneven', 'qbc_batch'])
def test_shared_bias_gradient_in_chunks(dtype, B, bias_shape):
    """dbias of a bias shared across (batch, head) pairs, with more pairs
    than one chunk of the reduction (the dK/dV kernel runs over the pairs in
    chunks of 512 / key-blocks = 16 here, each followed by a fixed-order
    reduction into an accumulator of the bias's extent)."""
    _check(dtype, B, 4, 64, 4096, 64, bias_shape=bias_shape, mask_kind='keypad', seed=B)


def _run_twice(dtype, B, H, s, t, d, **kw):
    rng = np.random.default_rng(55)
    q = _draw(rng, (B, H, s, d), dtype)
    k = _draw(rng, (B, H, t, d), dtype)
    v = _draw(rng, (B, H, t, d), dtype)
    g = _to(_draw(rng, (B, H, s, d), dtype), dtype)
    bias = _draw(rng, kw.pop('bias_shape'), dtype)
    mask = torch.from_numpy(_make_mask(rng, kw.pop('mask_kind'), B, H, s, t)).to(_dev())
    from nitrix_amd import scaled_dot_product_attention

    runs = []
    for _ in range(2):
        tq, tk, tv = _to(q, dtype, True), _to(k, dtype, True), _to(v, dtype, True)
        tb = _to(bias, dtype, True)
        out = scaled_dot_product_attention(tq, tk, tv, bias=tb, mask=mask,
                                           backend='hip', **kw)
        out.backward(g)
        torch.cuda.synchronize()
        runs.append([out.detach(), tq.grad, tk.grad, tv.grad, tb.grad])
    return runs


@pytest.mark.parametrize('dtype', DTYPES, ids=IDS)
def test_bitwise_deterministic_reruns(dtype):
    """Two runs of forward + backward on the same inputs agree bit for bit
    (no atomics; dbias of a shared bias summed in a fixed order), including
    a bias shared over the batch whose gradient takes several chunks."""
    print(f'[case] determinism {dtype}', flush=True)
    a, b = _run_twice(dtype, 8, 4, 200, 4096, 64, bias_shape=(4, 200, 4096),
                      mask_kind='random', causal=True)
    for name, x, y in zip(('out', 'dq', 'dk', 'dv', 'dbias'), a, b):
        assert torch.equal(x, y), f'{name} differs between identical runs'


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16], ids=['bf16', 'f16'])
@pytest.mark.parametrize('d', [64, 128])
@pytest.mark.parametrize('kind', ['keypad', 'rowbcast'])
@pytest.mark.parametrize('t', [1000, 1001])
def test_query_broadcast_mask_partial_tiles(dtype, d, kind, t):
    """A mask shared by every query row: the forward copies the mask bytes
    of a block's first four partial key tiles into LDS (rows of a multiple
    of four bytes, t = 1000) and reads the rest, or every tile when the rows
    are not 4-byte aligned (t = 1001), with global loads.  Key padding has
    one partial tile per batch; the row-broadcast mask (half the keys
    dropped at random) has every tile partial."""
    _check(dtype, 3, 2, 300, t, d, mask_kind=kind, seed=31)


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16], ids=['bf16', 'f16'])
def test_bitwise_deterministic_reruns_with_block_order(dtype):
    """The same with a non-causal mask whose block densities differ per row,
    so the 16-bit kernels run each head's blocks longest first."""
    print(f'[case] determinism with block order {dtype}', flush=True)
    a, b = _run_twice(dtype, 4, 2, 1500, 1700, 64, bias_shape=(2, 1500, 1700),
                      mask_kind='blocky')
    for name, x, y in zip(('out', 'dq', 'dk', 'dv', 'dbias'), a, b):
        assert torch.equal(x, y), f'{name} differs between identical runs'


def test_in_place_change_before_backward_raises():
    """The inputs are kept with save_for_backward: editing one in place
    between forward and backward raises instead of giving wrong gradients."""
    rng = np.random.default_rng(56)
    dtype = torch.bfloat16
    q, k, v = (_to(_draw(rng, (1, 2, 64, 64), dtype), dtype, True) for _ in range(3))
    from nitrix_amd import scaled_dot_product_attention

    out = scaled_dot_product_attention(q, k, v, backend='hip')
    with torch.no_grad():
        k.mul_(2.0)
    with pytest.raises(RuntimeError, match='modified by an inplace operation'):
        out.backward(torch.ones_like(out))
