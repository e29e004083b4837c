"""Block order of masks that vary over queries (GPU only).

With such a mask and no causal flag, the 16-bit kernels take each head's
blocks longest first. Per tile-map slice (one batch / head of the mask's own
extent) they use three lists: the 128-row query blocks (dQ, 4-wave forward),
the 256-row query blocks (8-wave forward) and the 128-key blocks (dK/dV).
Each list is sorted by the number of 64 x 64 mask tiles its blocks run, most
first, ties in index order. The lists sit in the workspace after the tile
map, 256-byte aligned, as int32 [slice][128-row | 256-row | 128-key].

The test reads them back after a forward call and compares them with the
same order computed here from the mask (a stable numpy argsort of the tile
counts). It then checks the attention itself against the float64 oracle on
masks whose order is far from the index order. Where no order applies
(causal, fp32, a mask broadcast over queries), the workspace holds only the
tile map.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from nitrix_amd import _lib
from nitrix_amd.attention import _Prepared
from test_hip_parity import _check

pytestmark = pytest.mark.gpu


def _dev():
    return torch.device('cuda:0')


def _align256(n):
    return (n + 255) // 256 * 256


def _expected(mask4):
    """Tile counts and orders of a bool mask [MB, MH, Lq, Lk]."""
    MB, MH, Lq, Lk = mask4.shape
    MQ, MK = -(-Lq // 64), -(-Lk // 64)
    pad = np.zeros((MB, MH, MQ * 64, MK * 64), bool)
    pad[:, :, :Lq, :Lk] = mask4
    tiles = pad.reshape(MB, MH, MQ, 64, MK, 64).any(axis=(3, 5))

    def rows(g):
        n = -(-MQ // g)
        t = np.zeros((MB, MH, n * g, MK), bool)
        t[:, :, :MQ] = tiles
        return t.reshape(MB, MH, n, g, MK).any(axis=3).sum(-1)

    nk = -(-MK // 2)
    t = np.zeros((MB, MH, MQ, nk * 2), bool)
    t[..., :MK] = tiles
    cols = t.reshape(MB, MH, MQ, nk, 2).any(-1).sum(2)
    counts = [rows(2), rows(4), cols]
    orders = [np.argsort(-c, axis=-1, kind='stable') for c in counts]
    return counts, orders, MB * MH * MQ * MK


def _forward_workspace(mask4, B, H, s, t, d, dtype, causal=False):
    g = torch.Generator().manual_seed(5)
    q = torch.randn(B, H, s, d, generator=g).to(_dev(), dtype)
    k = torch.randn(B, H, t, d, generator=g).to(_dev(), dtype)
    v = torch.randn(B, H, t, d, generator=g).to(_dev(), dtype)
    m = torch.from_numpy(mask4).to(_dev())
    prep = _Prepared(q, k, v, None, m, 1.0 / np.sqrt(d), causal)
    ws = prep.workspace(_lib.NXA_WS_FWD)
    assert ws is not None
    ws.fill_(0xAB)  # the lists must be written, not found
    o = torch.empty(prep.nb, prep.h, prep.s, prep.dv, dtype=prep.dtype, device=prep.device)
    lse = torch.empty(prep.nb, prep.h, prep.s, device=prep.device)
    ptrs = [None if x is None else x.data_ptr()
            for x in (prep.q, prep.k, prep.v, prep.bias, prep.mask)]
    rc = _lib.lib().nxa_fwd(ctypes.byref(prep.desc), *ptrs, o.data_ptr(), lse.data_ptr(),
                            ws.data_ptr(), ws.numel(), prep.stream())
    _lib.check(rc)
    torch.cuda.synchronize()
    return ws.cpu().numpy()


def _blocky(rng, MB, MH, s, t, p_row):
    """64-tile blocks kept with a probability that differs per block row, so
    the rows' (and columns') tile counts differ widely."""
    nq, nk = -(-s // 64), -(-t // 64)
    dens = rng.uniform(0.02, p_row, size=(MB, MH, nq, 1))
    blk = rng.random((MB, MH, nq, nk)) < dens
    blk[..., 0] = True
    m = np.kron(blk, np.ones((64, 64), bool))[..., :s, :t]
    return np.ascontiguousarray(m)


@pytest.mark.parametrize('MB,MH,B,H,s,t', [
    (1, 1, 1, 1, 1000, 1100),    # 16 x 18 map: byte loads (18 % 16 != 0)
    (2, 1, 2, 3, 2048, 2048),    # 32 x 32 map: 16-byte loads, slices per batch
    (1, 2, 2, 2, 700, 1024),     # 11 x 16 map: odd map rows, slices per head
    (1, 1, 1, 1, 5000, 3000),    # 79 x 47 map: odd extents, 3 chunks per map row
])
def test_orders_in_the_workspace(MB, MH, B, H, s, t):
    rng = np.random.default_rng(MB * 100 + MH * 10 + s)
    mask4 = _blocky(rng, MB, MH, s, t, 0.9)
    print(f'[case] block order MB{MB} MH{MH} B{B} H{H} s{s} t{t}', flush=True)
    ws = _forward_workspace(mask4, B, H, s, t, 64, torch.bfloat16)
    counts, orders, map_bytes = _expected(mask4)
    nq2, nq4, nk2 = (c.shape[-1] for c in counts)
    ps = nq2 + nq4 + nk2
    off = _align256(map_bytes)
    assert ws.size == off + _align256(MB * MH * ps * 4)
    got = ws[off:off + MB * MH * ps * 4].view(np.int32).reshape(MB, MH, ps)
    for name, lo, n, want in (('q128', 0, nq2, orders[0]), ('q256', nq2, nq4, orders[1]),
                              ('k128', nq2 + nq4, nk2, orders[2])):
        np.testing.assert_array_equal(got[..., lo:lo + n], want, err_msg=name)
    # The sort is not the index order here (else the test pins nothing).
    assert not np.array_equal(orders[0], np.broadcast_to(np.arange(nq2), orders[0].shape))
    assert not np.array_equal(orders[2], np.broadcast_to(np.arange(nk2), orders[2].shape))


@pytest.mark.parametrize('causal,dtype,qbcast', [
    (True, torch.bfloat16, False),
    (False, torch.float32, False),
    (False, torch.bfloat16, True),
])
def test_no_order_where_it_does_not_apply(causal, dtype, qbcast):
    rng = np.random.default_rng(3)
    s, t = 600, 700
    mask4 = _blocky(rng, 1, 1, s, t, 0.8)
    if qbcast:
        mask4 = np.ascontiguousarray(mask4[:, :, :1])
    print(f'[case] no block order causal={causal} {dtype} qbcast={qbcast}', flush=True)
    ws = _forward_workspace(mask4, 1, 1, s, t, 64, dtype, causal=causal)
    _, _, map_bytes = _expected(mask4)
    assert ws.size == _align256(map_bytes)


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16])
@pytest.mark.parametrize('d', [64, 128, 256])
@pytest.mark.parametrize('bias', [None, 'rows'])
def test_parity_with_block_order(dtype, d, bias):
    """fwd + bwd against the float64 oracle with per-row densities from 2 to
    90 %: blocks run far from index order (forward in 4-wave blocks at
    d = 64 and 256, 8-wave at d = 128; the head-dim-256 dK/dV kernel)."""
    B, H, s, t = 1, 2, 1300, 1500
    bias_shape = None if bias is None else (1, H, 1, t)
    _check(dtype, B, H, s, t, d, bias_shape=bias_shape, mask_kind='blocky', seed=11)


@pytest.mark.parametrize('d', [64, 128])
def test_parity_with_per_head_orders(d):
    """A mask drawn per batch and head (one list per head), with a full bias
    shared over the batch, so that dbias is summed over it: the dK/dV kernel
    then runs in chunks of (batch, head) pairs and reads each pair's list
    (36 key blocks: chunks of ceil(512 / 36) = 15 pairs, so 16 pairs take two
    launches, the second starting at pair 15)."""
    B, H, s, t = 8, 2, 200, 4500
    _check(torch.bfloat16, B, H, s, t, d, bias_shape=(1, H, s, t),
           mask_kind='blocky_bh', seed=12)
