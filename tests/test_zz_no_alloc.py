"""``nxa_fwd_noalloc`` (the forward that allocates nothing) against
``nxa_fwd`` through the C ABI (GPU only).

Both entry points run the same kernels; the allocation-free one keeps the
mask's tile map in the library's static device scratch instead of a caller
workspace.  Checked on consecutive calls -- the second smaller than the
first, with a different mask, so a stale tile map left in the scratch by
the first call would show -- and on a call without a mask.  Outputs and
log-sum-exp must agree bit for bit.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from nitrix_amd import _lib
from nitrix_amd.attention import _Prepared

pytestmark = pytest.mark.gpu


def _dev():
    return torch.device('cuda:0')


def _inputs(seed, B, H, s, t, d, mask_kind, bias):
    g = torch.Generator().manual_seed(seed)

    def rnd(*shape):
        return torch.randn(*shape, generator=g).to(_dev(), torch.bfloat16)

    q, k, v = rnd(B, H, s, d), rnd(B, H, t, d), rnd(B, H, t, d)
    b = rnd(B, H, s, t) if bias else None
    m = None
    if mask_kind == 'random':
        m = torch.rand(B, H, s, t, generator=g) < 0.3
        m[..., 0] = True
        m = m.to(_dev())
    elif mask_kind == 'keypad':
        valid = torch.randint(1, t + 1, (B,), generator=g)
        m = (torch.arange(t)[None, :] < valid[:, None])[:, None, None, :].to(_dev())
    return q, k, v, b, m


def _both(q, k, v, bias, mask):
    prep = _Prepared(q, k, v, bias, mask, 1.0 / np.sqrt(q.shape[-1]), False)
    lib = _lib.lib()
    outs = []
    for noalloc in (False, True):
        o = torch.full((prep.nb, prep.h, prep.s, prep.dv), float('nan'),
                       dtype=prep.dtype, device=prep.device)
        lse = torch.full((prep.nb, prep.h, prep.s), float('nan'), device=prep.device)
        ptrs = [None if x is None else x.data_ptr()
                for x in (prep.q, prep.k, prep.v, prep.bias, prep.mask)]
        if noalloc:
            rc = lib.nxa_fwd_noalloc(ctypes.byref(prep.desc), *ptrs, o.data_ptr(),
                                     lse.data_ptr(), prep.stream())
        else:
            ws = prep.workspace(_lib.NXA_WS_FWD)
            rc = lib.nxa_fwd(ctypes.byref(prep.desc), *ptrs, o.data_ptr(), lse.data_ptr(),
                             None if ws is None else ws.data_ptr(),
                             0 if ws is None else ws.numel(), prep.stream())
        _lib.check(rc)
        torch.cuda.synchronize()
        outs.append((o, lse))
    return outs


@pytest.mark.parametrize('calls', [
    [(1, 2, 3, 200, 333, 64, 'random', True), (2, 1, 2, 70, 90, 64, 'keypad', False)],
    [(3, 2, 2, 300, 260, 128, 'keypad', True), (4, 1, 1, 33, 40, 128, 'random', False),
     (5, 1, 2, 64, 64, 64, None, False)],
], ids=['random_then_keypad', 'keypad_then_random_then_nomask'])
def test_noalloc_forward_matches_nxa_fwd(calls):
    for seed, B, H, s, t, d, mask_kind, bias in calls:
        print(f'[case] noalloc B{B} H{H} s{s} t{t} d{d} mask={mask_kind} bias={bias}',
              flush=True)
        (o1, l1), (o2, l2) = _both(*_inputs(seed, B, H, s, t, d, mask_kind, bias))
        assert torch.isfinite(o1.float()).all()
        assert torch.equal(o1, o2), 'output differs from nxa_fwd'
        assert torch.equal(l1, l2), 'lse differs from nxa_fwd'
