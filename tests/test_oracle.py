"""Pin the CPU oracle before trusting it (CPU only).

Each check is chosen so that a plausible mistake in the restatement -- a
dropped or mis-ordered term, a wrong sign, a transposed operand, a wrong
reduction axis -- fails at least one of them:

* the reference's golden fixtures (exact-fp32 ones at the reference's own
  ``tol('attention', float32)``; the TF32-generated cross fixture both at
  2e-3 and, reproduced with TF32-rounded operands, at 1e-6);
* an independent per-row loop (``tests/test_nn_attention.py:76-94`` of the
  reference) in float64 with bias, causal and a random keep-mask;
* the reference's invariants (``tests/test_nn_attention.py:147-221``);
* central finite differences of the closed-form backward, float64, on q, k,
  v and the bias -- full, head-shared and query-broadcast bias shapes;
* the bf16 invariant (``tests/test_nn_mixed_precision.py:127-135``) with the
  bf16 rounding itself pinned against torch's independent conversion;
* planted mistakes (in a copy of the oracle, on the CPU) are caught.
"""

from __future__ import annotations

import numpy as np
import pytest
from _golden import (
    ATTENTION_CASES,
    CROSS_ATOL,
    TOL,
    load_golden,
)
from hypothesis import given
from hypothesis import strategies as st

from oracle import attention as O


def _run_golden(data, **kw):
    return O.sdpa_forward(
        data['q'],
        data['k'],
        data['v'],
        bias=data.get('bias'),
        mask=data.get('mask'),
        causal=bool(data['causal']),
        qk_norm=bool(data['qk_norm']) if 'qk_norm' in data else False,
        **kw,
    )


@pytest.mark.parametrize('name', ATTENTION_CASES)
def test_oracle_reproduces_reference_golden(name):
    data = load_golden(name)
    out = _run_golden(data).astype(np.float32)
    if name == 'attention_cross_float32':
        np.testing.assert_allclose(out, data['out'], atol=CROSS_ATOL, rtol=0)
    else:
        atol, rtol = TOL[('attention', 'float32')]
        np.testing.assert_allclose(out, data['out'], atol=atol, rtol=rtol)


def _tf32(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    lsb = (u >> 13) & 1
    r = (((u + 0xFFF + lsb) >> 13) << 13).astype(np.uint32)
    return r.view(np.float32)


def test_cross_fixture_is_tf32_generated():
    # Reproducing the cross fixture with TF32-rounded matmul operands (and the
    # oracle's op order otherwise) closes the 8e-4 gap to ~1e-7, which pins
    # both the op order and the fixture's provenance.
    d = load_golden('attention_cross_float32')
    q, k, v = d['q'], d['k'], d['v']
    logits = np.matmul(_tf32(q), np.swapaxes(_tf32(k), -1, -2))
    logits = logits * np.float32(O.default_scale(q.shape[-1]))
    w = np.exp(logits - logits.max(-1, keepdims=True))
    w = (w / w.sum(-1, keepdims=True)).astype(np.float32)
    out = np.matmul(_tf32(w), _tf32(v))
    np.testing.assert_allclose(out, d['out'], atol=1e-6, rtol=0)
    exact = _run_golden(d, acc_dtype=np.float64)
    assert np.max(np.abs(exact - d['out'])) > 1e-4  # it really is TF32


@pytest.mark.parametrize('causal', [False, True])
@pytest.mark.parametrize('with_mask', [False, True])
def test_oracle_matches_naive_rows(causal, with_mask):
    rng = np.random.RandomState(7)
    s, t, d, dv = 5, 7, 3, 2
    if causal:
        t = s
    q = rng.standard_normal((s, d))
    k = rng.standard_normal((t, d))
    v = rng.standard_normal((t, dv))
    bias = rng.standard_normal((s, t))
    keep = None
    if with_mask:
        keep = rng.rand(s, t) > 0.4
        keep[:, 0] = True
    got = O.sdpa_forward(
        q[None, None],
        k[None, None],
        v[None, None],
        bias=bias[None, None],
        mask=None if keep is None else keep[None, None],
        causal=causal,
    )[0, 0]
    want = O.naive_rows(q, k, v, bias=bias, causal=causal, keep=keep)
    np.testing.assert_allclose(got, want, atol=1e-12, rtol=0)


def test_fully_masked_row_is_nan():
    rng = np.random.RandomState(3)
    q = rng.standard_normal((1, 1, 3, 4))
    k = rng.standard_normal((1, 1, 5, 4))
    v = rng.standard_normal((1, 1, 5, 4))
    keep = np.ones((1, 1, 3, 5), bool)
    keep[0, 0, 1] = False
    out = O.sdpa_forward(q, k, v, mask=keep)
    assert np.all(np.isnan(out[0, 0, 1]))
    assert np.all(np.isfinite(out[0, 0, [0, 2]]))


# --- invariants (tests/test_nn_attention.py:147-221) -------------------------


def test_convex_hull_of_values():
    rng = np.random.RandomState(11)
    q = rng.standard_normal((2, 3, 5, 4))
    k = rng.standard_normal((2, 3, 6, 4))
    v = rng.standard_normal((2, 3, 6, 4))
    out = O.sdpa_forward(q, k, v)
    assert (out >= v.min(axis=2)[:, :, None] - 1e-12).all()
    assert (out <= v.max(axis=2)[:, :, None] + 1e-12).all()


def test_zero_query_gives_mean_value():
    rng = np.random.RandomState(12)
    v = rng.standard_normal((2, 2, 7, 3))
    q = np.zeros((2, 2, 4, 5))
    k = rng.standard_normal((2, 2, 7, 5))
    out = O.sdpa_forward(q, k, v)
    np.testing.assert_allclose(
        out, np.broadcast_to(v.mean(2, keepdims=True), out.shape), atol=1e-12
    )


@given(n=st.integers(2, 9), seed=st.integers(0, 2**16))
def test_causal_equals_tril(n, seed):
    rng = np.random.RandomState(seed)
    q = rng.standard_normal((1, 2, n, 4))
    k = rng.standard_normal((1, 2, n, 4))
    v = rng.standard_normal((1, 2, n, 3))
    a = O.sdpa_forward(q, k, v, causal=True)
    b = O.sdpa_forward(q, k, v, mask=np.tril(np.ones((n, n), bool)))
    np.testing.assert_allclose(a, b, atol=1e-12)


@given(seed=st.integers(0, 2**16))
def test_key_permutation_equivariance(seed):
    rng = np.random.RandomState(seed)
    q = rng.standard_normal((1, 1, 4, 4))
    k = rng.standard_normal((1, 1, 6, 4))
    v = rng.standard_normal((1, 1, 6, 3))
    bias = rng.standard_normal((1, 1, 4, 6))
    perm = rng.permutation(6)
    a = O.sdpa_forward(q, k, v, bias=bias)
    b = O.sdpa_forward(
        q, k[:, :, perm], v[:, :, perm], bias=bias[..., perm]
    )
    np.testing.assert_allclose(a, b, atol=1e-12)


@given(seed=st.integers(0, 2**16))
def test_masking_a_key_equals_deleting_it(seed):
    rng = np.random.RandomState(seed)
    t = 6
    q = rng.standard_normal((1, 1, 3, 4))
    k = rng.standard_normal((1, 1, t, 4))
    v = rng.standard_normal((1, 1, t, 2))
    keep = np.ones((1, 1, 3, t), bool)
    keep[..., t - 1] = False
    a = O.sdpa_forward(q, k, v, mask=keep)
    b = O.sdpa_forward(q, k[:, :, : t - 1], v[:, :, : t - 1])
    np.testing.assert_allclose(a, b, atol=1e-12)


def test_causal_cross_is_top_left_aligned():
    # s != t: query i keeps keys j <= i (indices aligned at 0), so with
    # s < t the keys j >= s are never seen.
    rng = np.random.RandomState(5)
    q = rng.standard_normal((1, 1, 3, 4))
    k = rng.standard_normal((1, 1, 8, 4))
    v = rng.standard_normal((1, 1, 8, 2))
    a = O.sdpa_forward(q, k, v, causal=True)
    b = O.sdpa_forward(q, k[:, :, :3], v[:, :, :3], causal=True)
    np.testing.assert_allclose(a, b, atol=1e-12)


# --- backward: central finite differences (float64) -------------------------


def _fd_check(bias_shape, causal, with_mask, seed=21, dv=3):
    rng = np.random.RandomState(seed)
    b, h, s, t, d = 2, 2, 3, 4, 3
    if causal:
        t = s
    q = rng.standard_normal((b, h, s, d))
    k = rng.standard_normal((b, h, t, d))
    v = rng.standard_normal((b, h, t, dv))
    bias = None if bias_shape is None else rng.standard_normal(bias_shape(s, t))
    mask = None
    if with_mask:
        mask = rng.rand(b, 1, s, t) > 0.3
        mask[..., 0] = True
    g = rng.standard_normal((b, h, s, dv))
    scale = 0.7

    def loss(q, k, v, bias):
        out = O.sdpa_forward(
            q, k, v, bias=bias, mask=mask, scale=scale, causal=causal
        )
        return float(np.sum(out * g))

    grads = O.sdpa_backward(
        q, k, v, g, bias=bias, mask=mask, scale=scale, causal=causal
    )
    args = [q, k, v, bias]
    eps = 1e-6
    for which in range(4):
        if args[which] is None:
            assert grads[which] is None
            continue
        x = args[which]
        assert grads[which].shape == x.shape
        fd = np.zeros_like(x)
        for idx in np.ndindex(x.shape):
            xp = x.copy()
            xp[idx] += eps
            xm = x.copy()
            xm[idx] -= eps
            ap = list(args)
            ap[which] = xp
            am = list(args)
            am[which] = xm
            fd[idx] = (loss(*ap) - loss(*am)) / (2 * eps)
        np.testing.assert_allclose(grads[which], fd, atol=1e-6, rtol=1e-5)


def test_backward_fd_full_bias():
    _fd_check(lambda s, t: (2, 2, s, t), causal=False, with_mask=False)


def test_backward_fd_head_shared_bias_masked():
    _fd_check(lambda s, t: (2, s, t), causal=False, with_mask=True)


def test_backward_fd_query_broadcast_bias_causal():
    _fd_check(lambda s, t: (1, 2, 1, t), causal=True, with_mask=False)


def test_backward_fd_no_bias_causal_masked():
    _fd_check(None, causal=True, with_mask=True)


@pytest.mark.parametrize('dv', [2, 5])
def test_backward_fd_value_head_dim_differs(dv):
    # v, out, dO and dv carry their own head dim d_v != d.
    _fd_check(lambda s, t: (2, 2, s, t), causal=True, with_mask=True, dv=dv)


def test_backward_delta_from_a_stored_output():
    """``out=``: delta taken from a given forward output, as the reference's
    backward takes it from its stored residual (``attention.py:600-622``).
    Given the exact output it reproduces the default; given a perturbed one
    (O + E), every row of dS sums to delta_exact - delta_out =
    -rowsum(E * dO) (the rows of P sum to one, and sum_j P dP = delta_exact),
    which a full bias returns as dbias; dV does not depend on it."""
    rng = np.random.RandomState(5)
    b, h, s, t, d, dv = 2, 2, 5, 7, 4, 3
    q, k = rng.standard_normal((b, h, s, d)), rng.standard_normal((b, h, t, d))
    v, g = rng.standard_normal((b, h, t, dv)), rng.standard_normal((b, h, s, dv))
    bias = rng.standard_normal((b, h, s, t))
    kw = dict(bias=bias, scale=0.6, acc_dtype=np.float64)
    exact = O.sdpa_forward(q, k, v, **kw)
    ref = O.sdpa_backward(q, k, v, g, **kw)
    same = O.sdpa_backward(q, k, v, g, out=exact, **kw)
    for x, y in zip(ref, same):
        np.testing.assert_allclose(y, x, rtol=1e-12, atol=1e-12)
    e = 1e-3 * rng.standard_normal(exact.shape)
    pert = O.sdpa_backward(q, k, v, g, out=exact + e, **kw)
    np.testing.assert_allclose(pert[3].sum(-1), -(e * g).sum(-1), rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(pert[2], ref[2], rtol=1e-12, atol=1e-12)
    assert np.abs(pert[0] - ref[0]).max() > 1e-6  # dq does move with delta


def test_qk_rms_norm_vjp_matches_finite_differences():
    rng = np.random.RandomState(5)
    z = rng.standard_normal((3, 2, 7))
    z[1, 0] *= 1e-4  # a row whose mean square is near eps
    g = rng.standard_normal((3, 2, 7))
    got = O.qk_rms_norm_vjp(z, g)
    eps = 1e-6
    fd = np.zeros_like(z)
    for idx in np.ndindex(z.shape):
        zp = z.copy()
        zp[idx] += eps
        zm = z.copy()
        zm[idx] -= eps
        fd[idx] = (np.sum(O.qk_rms_norm(zp) * g) - np.sum(O.qk_rms_norm(zm) * g)) / (2 * eps)
    np.testing.assert_allclose(got, fd, atol=1e-7, rtol=1e-6)


def test_qk_rms_norm_vjp_is_orthogonal_to_the_input():
    # The output is invariant to scaling z (up to eps), so the cotangent has
    # no component along z: <z, dz> = 0 up to an O(eps / ms) term.
    rng = np.random.RandomState(6)
    z = rng.standard_normal((4, 16))
    dz = O.qk_rms_norm_vjp(z, rng.standard_normal((4, 16)))
    assert np.max(np.abs(np.sum(z * dz, axis=-1))) < 1e-5


# --- bf16 semantics -----------------------------------------------------------


def test_round_bf16_matches_torch():
    torch = pytest.importorskip('torch')
    rng = np.random.RandomState(0)
    x = np.concatenate(
        [
            rng.standard_normal(10000).astype(np.float32) * 100,
            np.array([0.0, -0.0, np.inf, -np.inf, 3.4e38, 1e-40], np.float32),
        ]
    )
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(O.round_bf16(x), want)


def test_round_f16_matches_torch():
    torch = pytest.importorskip('torch')
    rng = np.random.RandomState(1)
    x = np.concatenate(
        [
            rng.standard_normal(10000).astype(np.float32) * 100,
            rng.standard_normal(1000).astype(np.float32) * 1e-6,  # subnormal halves
            np.array([0.0, -0.0, np.inf, -np.inf, 7e4, -7e4, 65519.0, 1e-9], np.float32),
        ]
    )
    want = torch.from_numpy(x).to(torch.float16).float().numpy()
    np.testing.assert_array_equal(O.round_f16(x), want)


def test_round_f16_known_answers():
    # ulp(1) = 2^-10: 1 + 2^-11 is a tie (to the even 1.0), 1 + 3 * 2^-11 a
    # tie to the even 1 + 2^-9; 65504 is the largest half, 65520 the first
    # value that rounds to inf; 2^-24 is the smallest subnormal.
    x = np.array([1 + 2.0**-11, 1 + 3 * 2.0**-11, 65519.0, 65520.0,
                  2.0**-25, 3 * 2.0**-26, 2.0**-14 + 2.0**-25], np.float32)
    want = np.array([1.0, 1 + 2.0**-9, 65504.0, np.inf, 0.0, 2.0**-24, 2.0**-14],
                    np.float32)
    np.testing.assert_array_equal(O.round_f16(x), want)


def test_f16_invariant_is_fp32_path_on_rounded_inputs():
    d = load_golden('attention_dense_float32')
    qh, kh, vh = (O.round_f16(d[n]) for n in ('q', 'k', 'v'))
    out = O.round_f16(O.sdpa_forward(qh, kh, vh))
    atol, rtol = TOL[('attention', 'float16')]
    np.testing.assert_allclose(out, d['out'], atol=atol, rtol=rtol)


def test_bf16_invariant_is_fp32_path_on_rounded_inputs():
    # reduced-precision reference == fp32 path on the bf16 inputs, cast back.
    d = load_golden('attention_dense_float32')
    qb, kb, vb = (O.round_bf16(d[n]) for n in ('q', 'k', 'v'))
    out = O.round_bf16(O.sdpa_forward(qb, kb, vb))
    atol, rtol = TOL[('attention', 'bfloat16')]
    np.testing.assert_allclose(out, d['out'], atol=atol, rtol=rtol)


# --- planted mistakes are caught ---------------------------------------------


def _mutant_scale_after_bias(q, k, v, bias=None, causal=False, **_):
    s = O.default_scale(q.shape[-1])
    lg = np.matmul(q, np.swapaxes(k, -1, -2))
    if bias is not None:
        lg = lg + bias
    lg = lg * s
    if causal:
        n = lg.shape[-1]
        lg = np.where(np.tril(np.ones((n, n), bool)), lg, -np.inf)
    w = np.exp(lg - lg.max(-1, keepdims=True))
    return np.matmul(w / w.sum(-1, keepdims=True), v)


def _mutant_transposed_causal(q, k, v, bias=None, causal=False, **_):
    return O.sdpa_forward(
        q,
        k,
        v,
        bias=bias,
        mask=np.triu(np.ones((q.shape[-2], k.shape[-2]), bool))
        if causal
        else None,
    )


def test_planted_mistakes_fail_the_goldens():
    wb = load_golden('attention_windowed_bias_float32')
    out = _mutant_scale_after_bias(wb['q'], wb['k'], wb['v'], bias=wb['bias'])
    assert np.max(np.abs(out - wb['out'])) > 1e-2
    c = load_golden('attention_causal_float32')
    out = _mutant_transposed_causal(c['q'], c['k'], c['v'], causal=True)
    assert np.max(np.abs(out - c['out'])) > 1e-2


def test_planted_backward_mistake_fails_fd():
    # dK without the scale factor must disagree with finite differences.
    rng = np.random.RandomState(2)
    q = rng.standard_normal((1, 1, 3, 3))
    k = rng.standard_normal((1, 1, 4, 3))
    v = rng.standard_normal((1, 1, 4, 3))
    g = rng.standard_normal((1, 1, 3, 3))
    _, dk, _, _ = O.sdpa_backward(q, k, v, g, scale=0.5)
    eps = 1e-6
    idx = (0, 0, 1, 2)
    kp = k.copy()
    kp[idx] += eps
    km = k.copy()
    km[idx] -= eps
    fd = (
        np.sum(O.sdpa_forward(q, kp, v, scale=0.5) * g)
        - np.sum(O.sdpa_forward(q, km, v, scale=0.5) * g)
    ) / (2 * eps)
    assert abs(dk[idx] - fd) < 1e-6
    assert abs(dk[idx] / 0.5 - fd) > 1e-3


# --- the chunked single-slice oracle (full-size GPU tests) ------------------


@pytest.mark.parametrize('case', ['bias_rows_mask', 'key_bias_causal', 'blocks', 'cross_dv'])
def test_slice_chunked_matches_whole_slice(case):
    """``sdpa_slice_chunked`` (row blocks, kept columns only) equals the
    whole-matrix oracle -- pinned above by the goldens, the naive loop, the
    invariants and finite differences -- on every output, with chunk sizes
    that do not divide the length."""
    rng = np.random.default_rng(31)
    s, t, d, dv = 150, 130, 16, 16
    causal = False
    bias = keep = bias_key = None
    if case == 'cross_dv':
        dv = 24
    q = rng.standard_normal((s, d))
    k = rng.standard_normal((t, d))
    v = rng.standard_normal((t, dv))
    g = rng.standard_normal((s, dv))
    if case == 'bias_rows_mask':
        bias = rng.standard_normal((s, t))
        keep = rng.random((s, t)) < 0.4
        keep[:, 3] = True
    elif case == 'key_bias_causal':
        bias_key = rng.standard_normal(t)
        causal = True
    elif case == 'blocks':
        blk = rng.random((-(-s // 32), -(-t // 32))) < 0.3
        blk[np.arange(min(blk.shape)), np.arange(min(blk.shape))] = True
        keep = np.kron(blk, np.ones((32, 32), bool))[:s, :t]
        bias_key = rng.standard_normal(t)
    scale = 0.3
    full_bias = bias if bias is not None else (
        None if bias_key is None else np.broadcast_to(bias_key, (s, t)))
    out, lse = O.sdpa_forward_lse(q, k, v, bias=full_bias, mask=keep, scale=scale,
                                  causal=causal, acc_dtype=np.float64)
    dq, dk, dvv, db = O.sdpa_backward(q, k, v, g, bias=full_bias, mask=keep, scale=scale,
                                      causal=causal, acc_dtype=np.float64)
    for chunk in (7, 64, 1000):
        r = O.sdpa_slice_chunked(
            q, k, v, g, scale=scale,
            bias_rows=None if bias is None else (lambda a, b: bias[a:b]),
            bias_key=bias_key,
            keep_rows=None if keep is None else (lambda a, b: keep[a:b]),
            causal=causal, chunk=chunk)
        for name, want in (('out', out), ('lse', lse), ('dq', dq), ('dk', dk),
                           ('dv', dvv)):
            np.testing.assert_allclose(r[name], want, rtol=0, atol=1e-12, err_msg=name)
        if full_bias is not None:
            np.testing.assert_allclose(r['dbias_col'], db.sum(axis=0), rtol=0, atol=1e-12)
    fwd = O.sdpa_slice_chunked(q, k, v, scale=scale, bias_key=bias_key, causal=causal,
                               bias_rows=None if bias is None else (lambda a, b: bias[a:b]),
                               keep_rows=None if keep is None else (lambda a, b: keep[a:b]))
    assert set(fwd) == {'out', 'lse'}
    np.testing.assert_allclose(fwd['out'], out, rtol=0, atol=1e-12)
