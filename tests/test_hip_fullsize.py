"""Parity at the BASELINE configurations' full sizes (GPU only).

The CPU oracle cannot hold these problems whole (8.6-34 GB of fp32 logits per
tensor), so each configuration is checked three ways on the same seeded
inputs:

* **one whole (batch, head) slice** -- out, dQ, dK, dV (and the bias
  gradient of C5's query-broadcast bias) of every row and key of the slice,
  elementwise against the float64 oracle computed in blocks of query rows
  (``oracle.attention.sdpa_slice_chunked``, pinned on the CPU against the
  whole-matrix oracle);
* **sampled rows** -- the float64 oracle (``oracle/attention.py``) on whole
  64-row tiles (start, middle, tail) of a few other (batch, head) slices,
  with the full keys, values, bias row and mask row of each: the output rows
  and the dQ rows are exact functions of those rows alone
  (dQ_i = scale sum_j dS_ij k_j);
* **size-independent identities** of the attention backward, exact in
  arithmetic for every row that keeps at least one key:
    - sum_j dS_ij = 0, hence sum_j dK_j = 0 and sum_j dbias_j = 0 (dbias
      broadcast over queries);
    - sum_j P_ij = 1, hence sum_j dV_j = sum_i dO_i;
    - a key the mask removes gets dK_j = dV_j = 0 exactly.

Budgets: ``max|a-b| / max|b| <= 2e-2`` for sampled bf16 rows (the north
star's bf16 budget), ``|sum| / sum|.| <= 1e-2`` for the identities (sums of
bf16-rounded gradients).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as O

pytestmark = pytest.mark.gpu

REL = 2e-2
IDENT = 1e-2
SEED = 77


def _dev():
    return torch.device('cuda:0')


def _randn(gen, *shape, grad=False, dtype=torch.bfloat16):
    x = torch.empty(*shape, device=_dev(), dtype=dtype)
    flat = x.view(-1)
    step = 1 << 28
    for i in range(0, flat.numel(), step):
        k = min(step, flat.numel() - i)
        flat[i:i + k] = torch.randn(k, generator=gen, device=_dev(), dtype=torch.float32)
    return x.requires_grad_(grad)


def _np(t):
    return t.detach().float().cpu().numpy()


def _relerr(a, b):
    return float(np.max(np.abs(a - b)) / (np.max(np.abs(b)) + 1e-30))


def _check_rows(q, k, v, dout, out, dq, b, h, rows, *, scale, bias_row=None,
                mask_row=None, causal=False):
    """Oracle output and dQ of query ``rows`` of slice (b, h)."""
    qn = _np(q[b, h, rows])[None, None]
    kn = _np(k[b, h])[None, None]
    vn = _np(v[b, h])[None, None]
    L = kn.shape[2]
    keep = np.ones((len(rows), L), bool)
    if mask_row is not None:
        keep &= mask_row
    if causal:
        keep &= np.asarray(rows)[:, None] >= np.arange(L)[None, :]
    bias = None if bias_row is None else bias_row[None, None]
    ref = O.sdpa_forward(qn, kn, vn, bias=bias, mask=keep[None, None], scale=scale,
                         acc_dtype=np.float64)[0, 0]
    got = _np(out[b, h, rows])
    e = _relerr(got, ref)
    assert e <= REL, f'out rows of ({b},{h}) relerr {e:.3e}'
    if dq is not None:
        gn = _np(dout[b, h, rows])[None, None]
        rdq, _, _, _ = O.sdpa_backward(qn, kn, vn, gn, bias=bias, mask=keep[None, None],
                                       scale=scale, acc_dtype=np.float64)
        e = _relerr(_np(dq[b, h, rows]), rdq[0, 0])
        assert e <= REL, f'dq rows of ({b},{h}) relerr {e:.3e}'


def _identities(dk, dv, dout, live_rows, *, dbias=None, dead_keys=None):
    """sum_j dK_j = 0, sum_j dV_j = sum_{live i} dO_i, sum_j dbias_j = 0."""
    dk64 = dk.double()
    s = dk64.sum(dim=2)
    ratio = float((s.abs().max() / dk64.abs().sum(dim=2).max()).cpu())
    assert ratio <= IDENT, f'sum_j dK_j / sum_j |dK_j| = {ratio:.3e}'
    dv64 = dv.double()
    want = (dout.double() * live_rows[..., None]).sum(dim=2)
    err = float(((dv64.sum(dim=2) - want).abs().max() / dv64.abs().sum(dim=2).max()).cpu())
    assert err <= IDENT, f'sum_j dV_j vs sum_i dO_i: {err:.3e}'
    if dbias is not None:
        db = dbias.double()
        r = float((db.sum(dim=-1).abs().max() / db.abs().sum(dim=-1).max()).cpu())
        assert r <= IDENT, f'sum_j dbias_j / sum_j |dbias_j| = {r:.3e}'
    if dead_keys is not None:
        assert torch.count_nonzero(dk[dead_keys]) == 0, 'masked key has dK != 0'
        assert torch.count_nonzero(dv[dead_keys]) == 0, 'masked key has dV != 0'


def _tiles(L):
    """Whole 64-row tiles at the start, the middle and the tail."""
    mid = (L // 2) // 64 * 64
    return list(range(0, 64)) + list(range(mid, mid + 64)) + list(range(L - 64, L))


def _check_slice(q, k, v, dout, out, grads, b, h, *, scale, keep_rows=None,
                 bias_rows=None, bias_key=None, causal=False, dbias_col=None,
                 chunk=512, rel=REL):
    """Every output (and gradient) of slice (b, h) against the chunked
    float64 oracle.  ``grads`` = (dq, dk, dv) tensors or None."""
    r = O.sdpa_slice_chunked(
        _np(q[b, h]), _np(k[b, h]), _np(v[b, h]),
        None if grads is None else _np(dout[b, h]),
        scale=scale, keep_rows=keep_rows, bias_rows=bias_rows, bias_key=bias_key,
        causal=causal, chunk=chunk)
    checks = [('out', out)]
    if grads is not None:
        checks += [('dq', grads[0]), ('dk', grads[1]), ('dv', grads[2])]
    for name, t in checks:
        e = _relerr(_np(t[b, h]), r[name])
        print(f'  slice ({b},{h}) {name} relerr {e:.2e}', flush=True)
        assert e <= rel, f'slice ({b},{h}) {name} relerr {e:.3e}'
    if dbias_col is not None:
        e = _relerr(_np(dbias_col), r['dbias_col'])
        print(f'  slice ({b},{h}) dbias relerr {e:.2e}', flush=True)
        assert e <= REL, f'slice ({b},{h}) dbias relerr {e:.3e}'


def _fwd_bwd(q, k, v, dout, **kw):
    from nitrix_amd import scaled_dot_product_attention

    out = scaled_dot_product_attention(q, k, v, backend='hip', **kw)
    out.backward(dout)
    torch.cuda.synchronize()
    return out


def test_c2_key_padding_b8_h16_l4096_d128():
    """bf16 fwd+bwd, key-padding mask, valid lengths
    uniform in [1024, 4096]."""
    B, H, L, D = 8, 16, 4096, 128
    print(f'[case] C2 B{B} H{H} L{L} D{D} key padding', flush=True)
    gen = torch.Generator(device=_dev())
    gen.manual_seed(SEED)
    rng = np.random.default_rng(SEED)
    valid = rng.integers(1024, L + 1, size=B)
    q, k, v = (_randn(gen, B, H, L, D, grad=True) for _ in range(3))
    dout = _randn(gen, B, H, L, D)
    mask = (torch.arange(L, device=_dev())[None, :]
            < torch.as_tensor(valid, device=_dev())[:, None])[:, None, None, :]
    out = _fwd_bwd(q, k, v, dout, mask=mask)
    scale = 1.0 / math.sqrt(D)
    for b, h in ((0, 0), (2, 15)):
        mrow = np.arange(L) < valid[b]
        _check_rows(q, k, v, dout, out, q.grad, b, h, _tiles(L), scale=scale, mask_row=mrow)
    b, h = 6, 11
    mrow = np.arange(L) < valid[b]
    _check_slice(q, k, v, dout, out, (q.grad, k.grad, v.grad), b, h, scale=scale,
                 keep_rows=lambda r0, r1: np.broadcast_to(mrow, (r1 - r0, L)))
    dead = ~mask[:, 0, 0, :]  # [B, L]
    dead = dead[:, None, :].expand(B, H, L)
    _identities(k.grad, v.grad, dout, torch.ones(B, H, L, device=_dev(), dtype=torch.float64),
                dead_keys=dead)


def test_c3_causal_b4_h32_l8192_d128():
    """bf16 causal fwd+bwd."""
    B, H, L, D = 4, 32, 8192, 128
    print(f'[case] C3 B{B} H{H} L{L} D{D} causal', flush=True)
    gen = torch.Generator(device=_dev())
    gen.manual_seed(SEED + 1)
    q, k, v = (_randn(gen, B, H, L, D, grad=True) for _ in range(3))
    dout = _randn(gen, B, H, L, D)
    out = _fwd_bwd(q, k, v, dout, causal=True)
    scale = 1.0 / math.sqrt(D)
    _check_rows(q, k, v, dout, out, q.grad, 0, 0, _tiles(L), scale=scale, causal=True)
    _check_slice(q, k, v, dout, out, (q.grad, k.grad, v.grad), 3, 31, scale=scale,
                 causal=True)
    _identities(k.grad, v.grad, dout, torch.ones(B, H, L, device=_dev(), dtype=torch.float64))


def test_c4_full_bias_b2_h16_l8192_d64():
    """bf16 fwd with a full per-head bias
    [2,16,8192,8192] (streamed through the LDS ring, added by MFMA)."""
    B, H, L, D = 2, 16, 8192, 64
    print(f'[case] C4 B{B} H{H} L{L} D{D} full bias', flush=True)
    gen = torch.Generator(device=_dev())
    gen.manual_seed(SEED + 2)
    q, k, v = (_randn(gen, B, H, L, D) for _ in range(3))
    bias = _randn(gen, B, H, L, L)
    from nitrix_amd import scaled_dot_product_attention

    with torch.no_grad():
        out = scaled_dot_product_attention(q, k, v, bias=bias, backend='hip')
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    scale = 1.0 / math.sqrt(D)
    for b, h in ((0, 0), (0, 15)):
        rows = _tiles(L)
        brow = _np(bias[b, h, rows])
        _check_rows(q, k, v, None, out, None, b, h, rows, scale=scale, bias_row=brow)
    bslice = _np(bias[1, 9])
    _check_slice(q, k, v, None, out, None, 1, 9, scale=scale,
                 bias_rows=lambda r0, r1: bslice[r0:r1])


def test_c5_block_sparse_row_bias_b1_h8_l32768_d64():
    """bf16 fwd+bwd, block-sparse mask [1,1,L,L] of
    128x128 blocks kept with p=0.25 (diagonal kept), bias [1,8,1,L] with its
    gradient (a column sum over queries)."""
    B, H, L, D = 1, 8, 32768, 64
    print(f'[case] C5 B{B} H{H} L{L} D{D} block-sparse + row bias', flush=True)
    gen = torch.Generator(device=_dev())
    gen.manual_seed(SEED + 3)
    rng = np.random.default_rng(SEED + 3)
    nb = L // 128
    blk = rng.random((nb, nb)) < 0.25
    blk[np.arange(nb), np.arange(nb)] = True
    tb = torch.as_tensor(blk, device=_dev())
    mask = tb.repeat_interleave(128, 0).repeat_interleave(128, 1)[None, None]
    q, k, v = (_randn(gen, B, H, L, D, grad=True) for _ in range(3))
    bias = _randn(gen, 1, H, 1, L, grad=True)
    dout = _randn(gen, B, H, L, D)
    out = _fwd_bwd(q, k, v, dout, bias=bias, mask=mask)
    scale = 1.0 / math.sqrt(D)

    def keep_rows(r0, r1):
        return np.repeat(blk[np.arange(r0, r1) // 128], 128, axis=1)

    rows = _tiles(L)
    brow = _np(bias[0, 0, 0])
    _check_rows(q, k, v, dout, out, q.grad, 0, 0, rows, scale=scale,
                bias_row=brow[None, :].repeat(len(rows), 0),
                mask_row=np.repeat(blk[np.asarray(rows) // 128], 128, axis=1))
    h = 5
    _check_slice(q, k, v, dout, out, (q.grad, k.grad, v.grad), 0, h, scale=scale,
                 keep_rows=keep_rows, bias_key=_np(bias[0, h, 0]),
                 dbias_col=bias.grad[0, h, 0], chunk=128)
    _identities(k.grad, v.grad, dout, torch.ones(B, H, L, device=_dev(), dtype=torch.float64),
                dbias=bias.grad[0, :, 0, :])


# --- more than 1024 tiles per row or column --------------------------------
# Blocks keep the list of their active tiles in LDS for up to 1024 tiles;
# longer problems classify each tile inside the loop instead.


def test_key_padding_more_than_1024_key_tiles():
    """Lk = 66,000 (1,032 key tiles of 64): the forward and dQ kernels run
    without the listed tiles.  Key padding per batch, query tails."""
    B, H, Lq, Lk, D = 2, 2, 300, 66000, 64
    print(f'[case] B{B} H{H} Lq{Lq} Lk{Lk} D{D} key padding, >1024 key tiles', flush=True)
    gen = torch.Generator(device=_dev())
    gen.manual_seed(SEED + 4)
    valid = np.array([41000, 66000])
    q = _randn(gen, B, H, Lq, D, grad=True)
    k, v = (_randn(gen, B, H, Lk, D, grad=True) for _ in range(2))
    dout = _randn(gen, B, H, Lq, D)
    mask = (torch.arange(Lk, device=_dev())[None, :]
            < torch.as_tensor(valid, device=_dev())[:, None])[:, None, None, :]
    out = _fwd_bwd(q, k, v, dout, mask=mask)
    scale = 1.0 / math.sqrt(D)
    for b, h in ((0, 1), (1, 0)):
        mrow = np.arange(Lk) < valid[b]
        _check_slice(q, k, v, dout, out, (q.grad, k.grad, v.grad), b, h, scale=scale,
                     keep_rows=lambda r0, r1: np.broadcast_to(mrow, (r1 - r0, Lk)),
                     chunk=100)


def test_block_sparse_more_than_1024_tiles_both_ways():
    """L = 66,000 with a [1, 1, L, L] mask of 128 x 128 blocks (2 % kept plus
    the diagonal): 1,032 query and key tiles, so the forward, dQ and dK/dV
    kernels all run without the listed tiles; the length leaves tails."""
    B, H, L, D = 1, 1, 66000, 64
    print(f'[case] B{B} H{H} L{L} D{D} block-sparse, >1024 tiles', flush=True)
    gen = torch.Generator(device=_dev())
    gen.manual_seed(SEED + 5)
    rng = np.random.default_rng(SEED + 5)
    nb = -(-L // 128)
    blk = rng.random((nb, nb)) < 0.02
    blk[np.arange(nb), np.arange(nb)] = True
    tb = torch.as_tensor(blk, device=_dev())
    mask = tb.repeat_interleave(128, 0).repeat_interleave(128, 1)[:L, :L][None, None]
    q, k, v = (_randn(gen, B, H, L, D, grad=True) for _ in range(3))
    dout = _randn(gen, B, H, L, D)
    out = _fwd_bwd(q, k, v, dout, mask=mask)
    del mask, tb
    scale = 1.0 / math.sqrt(D)

    def keep_rows(r0, r1):
        return np.repeat(blk[np.arange(r0, r1) // 128], 128, axis=1)[:, :L]

    _check_slice(q, k, v, dout, out, (q.grad, k.grad, v.grad), 0, 0, scale=scale,
                 keep_rows=keep_rows, chunk=128)



def test_more_than_65536_key_tiles():
    """Lk = 4,194,468 (65,539 key tiles of 64, the last one ragged: more than
    a 16-bit tile index holds), no mask: the forward and dQ kernels walk the
    key tiles without a list.  Out and every gradient of the slice against
    the float64 oracle (8 query rows keep it to seconds)."""
    B, H, Lq, Lk, D = 1, 1, 8, 65539 * 64 - 28, 64
    print(f'[case] B{B} H{H} Lq{Lq} Lk{Lk} D{D} no mask, >65536 key tiles', flush=True)
    gen = torch.Generator(device=_dev())
    gen.manual_seed(SEED + 9)
    q = _randn(gen, B, H, Lq, D, grad=True)
    k, v = (_randn(gen, B, H, Lk, D, grad=True) for _ in range(2))
    dout = _randn(gen, B, H, Lq, D)
    out = _fwd_bwd(q, k, v, dout)
    scale = 1.0 / math.sqrt(D)
    qn, kn, vn, gn = _np(q), _np(k), _np(v), _np(dout)
    ref = O.sdpa_forward(qn, kn, vn, scale=scale, acc_dtype=np.float64)
    dq, dk, dv, _ = O.sdpa_backward(qn, kn, vn, gn, scale=scale, acc_dtype=np.float64)
    for name, got, want in (('out', out, ref), ('dq', q.grad, dq), ('dk', k.grad, dk),
                            ('dv', v.grad, dv)):
        e = _relerr(_np(got), want)
        print(f'  {name} relerr {e:.2e}', flush=True)
        assert e <= REL, f'{name} relerr {e:.3e}'


# --- head dim 256 ------------------------------------------------------------


def test_head_dim_256_b4_h16_l4096():
    """The head-dim-256 measurement workload (bench ``w256``): bf16 fwd+bwd,
    no mask.  128 query tiles of 32 per key block in the dK/dV kernel."""
    B, H, L, D = 4, 16, 4096, 256
    print(f'[case] B{B} H{H} L{L} D{D}', flush=True)
    gen = torch.Generator(device=_dev())
    gen.manual_seed(SEED + 6)
    q, k, v = (_randn(gen, B, H, L, D, grad=True) for _ in range(3))
    dout = _randn(gen, B, H, L, D)
    out = _fwd_bwd(q, k, v, dout)
    scale = 1.0 / math.sqrt(D)
    _check_rows(q, k, v, dout, out, q.grad, 1, 7, _tiles(L), scale=scale)
    _check_slice(q, k, v, dout, out, (q.grad, k.grad, v.grad), 3, 12, scale=scale)
    _identities(k.grad, v.grad, dout, torch.ones(B, H, L, device=_dev(), dtype=torch.float64))


def test_head_dim_256_causal_key_padding_ragged():
    """Head dim 256, causal with key padding and a ragged length (partial
    query and key tiles, diagonal tiles, keys removed per batch)."""
    B, H, L, D = 2, 2, 3000, 256
    print(f'[case] B{B} H{H} L{L} D{D} causal + key padding', flush=True)
    gen = torch.Generator(device=_dev())
    gen.manual_seed(SEED + 7)
    valid = np.array([2111, 3000])
    q, k, v = (_randn(gen, B, H, L, D, grad=True) for _ in range(3))
    dout = _randn(gen, B, H, L, D)
    mask = (torch.arange(L, device=_dev())[None, :]
            < torch.as_tensor(valid, device=_dev())[:, None])[:, None, None, :]
    out = _fwd_bwd(q, k, v, dout, mask=mask, causal=True)
    scale = 1.0 / math.sqrt(D)
    for b, h in ((0, 1), (1, 0)):
        mrow = np.arange(L) < valid[b]
        _check_slice(q, k, v, dout, out, (q.grad, k.grad, v.grad), b, h, scale=scale,
                     keep_rows=lambda r0, r1: np.broadcast_to(mrow, (r1 - r0, L)),
                     causal=True)


# --- fp32 at head dim 256 ------------------------------------------------------
# fp32 I/O is held to the parity suite's fp32 budget (1e-5 of the largest
# magnitude) against the float64 oracle.

REL32 = 1e-5


def test_fp32_head_dim_256_b1_h16_l2048():
    """The fp32 head-dim-256 measurement workload (bench ``w256f32``): 32-key
    forward and dQ tiles, the dV and dK launches over 32-query tiles."""
    B, H, L, D = 1, 16, 2048, 256
    print(f'[case] fp32 B{B} H{H} L{L} D{D}', flush=True)
    gen = torch.Generator(device=_dev())
    gen.manual_seed(SEED + 10)
    q, k, v = (_randn(gen, B, H, L, D, grad=True, dtype=torch.float32) for _ in range(3))
    dout = _randn(gen, B, H, L, D, dtype=torch.float32)
    out = _fwd_bwd(q, k, v, dout)
    scale = 1.0 / math.sqrt(D)
    for h in (0, 9, 15):
        _check_slice(q, k, v, dout, out, (q.grad, k.grad, v.grad), 0, h, scale=scale,
                     rel=REL32)
    _identities(k.grad, v.grad, dout, torch.ones(B, H, L, device=_dev(), dtype=torch.float64))


@pytest.mark.parametrize('lq,lk', [(8, 33000), (33000, 8)], ids=['long_keys', 'long_queries'])
def test_fp32_head_dim_256_more_than_1024_tiles(lq, lk):
    """fp32 at head dim 256 with more 32-row tiles than a block lists (1,032):
    long keys take the forward and dQ past the list, long queries the dK/dV
    launches; tails in both."""
    B, H, D = 1, 2, 256
    print(f'[case] fp32 B{B} H{H} Lq{lq} Lk{lk} D{D}', flush=True)
    gen = torch.Generator(device=_dev())
    gen.manual_seed(SEED + 11)
    q = _randn(gen, B, H, lq, D, grad=True, dtype=torch.float32)
    k, v = (_randn(gen, B, H, lk, D, grad=True, dtype=torch.float32) for _ in range(2))
    dout = _randn(gen, B, H, lq, D, dtype=torch.float32)
    out = _fwd_bwd(q, k, v, dout)
    scale = 1.0 / math.sqrt(D)
    qn, kn, vn, gn = _np(q), _np(k), _np(v), _np(dout)
    ref = O.sdpa_forward(qn, kn, vn, scale=scale, acc_dtype=np.float64)
    dq, dk, dv, _ = O.sdpa_backward(qn, kn, vn, gn, scale=scale, acc_dtype=np.float64)
    for name, got, want in (('out', out, ref), ('dq', q.grad, dq), ('dk', k.grad, dk),
                            ('dv', v.grad, dv)):
        e = _relerr(_np(got), want)
        print(f'  {name} relerr {e:.2e}', flush=True)
        assert e <= REL32, f'{name} relerr {e:.3e}'
