"""Host-side call preparation (``attention._Prepared``) on CPU tensors.

The fused path flattens q, k, v (and bias / mask) to ``[nb, h, L, d]``
views and fills the C descriptor from their strides.  Inputs already in that
shape skip the broadcast machinery; these tests check that the skip gives
the same views and descriptor as the general expand / reshape route, and that
broadcast leading axes still resolve as ``torch.broadcast_shapes`` does
(``src/nitrix/nn/attention/__init__.py:126-230`` broadcasts q, k, v and
bias / mask over the leading axes).  No GPU: no kernel is called.
"""
import pytest
import torch

import nitrix_amd.attention as A


def _general_bhld(x, lead, nb, epc):
    L, d = x.shape[-2], x.shape[-1]
    y = x.expand(*lead, L, d).reshape(nb, lead[-1], L, d)
    return y if A._layout_ok(y, epc) else y.contiguous()


def _same_view(a, b):
    return (a.shape == b.shape and a.stride() == b.stride()
            and a.data_ptr() == b.data_ptr() and a.dtype == b.dtype)


def _desc_tuple(desc):
    return (desc.B, desc.H, desc.Lq, desc.Lk, desc.D, desc.Dv, desc.io_dtype,
            desc.bias_dtype, desc.causal, desc.scale, tuple(desc.q_str),
            tuple(desc.k_str), tuple(desc.v_str), tuple(desc.o_str),
            tuple(desc.bias_str), tuple(desc.mask_str))


@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16])
def test_four_dim_inputs_take_the_views_of_the_general_route(dtype):
    g = torch.Generator().manual_seed(0)
    q = torch.randn(2, 3, 40, 64, generator=g).to(dtype)
    k = torch.randn(2, 3, 56, 64, generator=g).to(dtype)
    v = torch.randn(2, 3, 56, 32, generator=g).to(dtype)
    bias = torch.randn(2, 3, 40, 56, generator=g)
    mask = torch.rand(2, 3, 40, 56, generator=g) > 0.3
    p = A._Prepared(q, k, v, bias, mask, 0.125, False)
    epc = 4 if dtype == torch.float32 else 8
    assert p.lead == (2, 3) and p.nb == 2 and p.h == 3
    for got, x in ((p.q, q), (p.k, k), (p.v, v)):
        assert _same_view(got, _general_bhld(x, (2, 3), 2, epc))
        assert got.data_ptr() == x.data_ptr()  # no copy
    assert _same_view(p.bias, bias.expand(2, 3, 40, 56).reshape(2, 3, 40, 56))
    assert _same_view(p.mask, mask.expand(2, 3, 40, 56).reshape(2, 3, 40, 56))
    d = p.desc
    assert (d.B, d.H, d.Lq, d.Lk, d.D, d.Dv) == (2, 3, 40, 56, 64, 32)
    assert tuple(d.q_str) == q.stride()[:3] and tuple(d.k_str) == k.stride()[:3]
    assert tuple(d.o_str) == (3 * 40 * 32, 40 * 32, 32)


def test_strided_four_dim_views_keep_their_strides():
    # A [B, L, H, D] tensor transposed to [B, H, L, D]: non-contiguous, but
    # rows are contiguous, so the view is taken as is.
    g = torch.Generator().manual_seed(1)
    base = torch.randn(2, 48, 4, 64, generator=g)
    q = base.transpose(1, 2)
    k = torch.randn(2, 4, 48, 64, generator=g)
    v = torch.randn(2, 4, 48, 64, generator=g)
    p = A._Prepared(q, k, v, None, None, 0.125, True)
    assert _same_view(p.q, q)
    assert tuple(p.desc.q_str) == q.stride()[:3]
    assert p.desc.causal == 1


def test_broadcast_leading_axes_resolve_as_torch_does():
    g = torch.Generator().manual_seed(2)
    q = torch.randn(5, 2, 3, 16, 64, generator=g)
    k = torch.randn(1, 3, 24, 64, generator=g)  # broadcast over both batch axes
    v = torch.randn(2, 3, 24, 64, generator=g)
    bias = torch.randn(3, 1, 24, generator=g)  # broadcast over batch and queries
    p = A._Prepared(q, k, v, bias, None, 0.125, False)
    lead = tuple(torch.broadcast_shapes(q.shape[:-2], k.shape[:-2], v.shape[:-2]))
    assert p.lead == lead == (5, 2, 3)
    assert p.nb == 10 and p.h == 3
    for got, x in ((p.q, q), (p.k, k), (p.v, v)):
        want = _general_bhld(x, lead, 10, 4)
        assert got.shape == want.shape and torch.equal(got, want)
    want_b = bias.expand(5, 2, 3, 16, 24).reshape(10, 3, 16, 24)
    assert torch.equal(p.bias, want_b)


def test_three_dim_inputs():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(4, 20, 64, generator=g)
    k = torch.randn(4, 30, 64, generator=g)
    v = torch.randn(4, 30, 64, generator=g)
    p = A._Prepared(q, k, v, None, None, 0.125, False)
    assert p.lead == (4,) and p.nb == 1 and p.h == 4
    assert p.q.shape == (1, 4, 20, 64) and p.q.data_ptr() == q.data_ptr()


def test_incompatible_leading_axes_raise_torch_s_error():
    q = torch.randn(2, 3, 8, 64)
    k = torch.randn(4, 3, 8, 64)
    v = torch.randn(4, 3, 8, 64)
    with pytest.raises(RuntimeError):
        A._lead_shape(q, k, v)


def test_fast_and_general_routes_fill_the_same_descriptor():
    g = torch.Generator().manual_seed(4)
    q = torch.randn(2, 2, 24, 64, generator=g).to(torch.bfloat16)
    k = torch.randn(2, 2, 40, 64, generator=g).to(torch.bfloat16)
    v = torch.randn(2, 2, 40, 64, generator=g).to(torch.bfloat16)
    bias = torch.randn(2, 2, 24, 40, generator=g).to(torch.bfloat16)
    fast = A._Prepared(q, k, v, bias, None, 0.2, False)
    # The same tensors behind an extra unit axis take the general route.
    slow = A._Prepared(q[None], k[None], v[None], bias[None], None, 0.2, False)
    assert slow.lead == (1, 2, 2)
    assert _desc_tuple(fast.desc) == _desc_tuple(slow.desc)
    for a, b in ((fast.q, slow.q), (fast.k, slow.k), (fast.v, slow.v),
                 (fast.bias, slow.bias)):
        assert _same_view(a, b)


def test_a_bias_that_does_not_broadcast_still_raises():
    # Leading axes (2, 3) of q, k, v; a bias with a flattened batch of 6
    # has the [nb, h, s, t] shape of neither and must not be taken as one.
    q = torch.randn(2, 3, 4, 8, 64)
    k = torch.randn(2, 3, 4, 8, 64)
    v = torch.randn(2, 3, 4, 8, 64)
    bias = torch.randn(6, 4, 8, 8)
    with pytest.raises(RuntimeError):
        A._Prepared(q, k, v, bias, None, 0.125, False)
