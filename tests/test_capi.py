"""The C ABI of ``libnxattn.so`` on the CPU (no GPU needed).

* the library loads and exports every function ``include/nxattn.h`` declares;
* host-side descriptor validation (the counterpart of the reference's
  ``_check_tileable``, ``src/nitrix/_kernels/cuda/attention.py:708-765``)
  returns the documented error codes and a message;
* the workspace sizes follow the documented layout;
* entry points reject NULL / misaligned buffers before touching the GPU.
"""

from __future__ import annotations

import ctypes
import pathlib
import re

import pytest

from nitrix_amd import _lib

HEADER = pathlib.Path(__file__).resolve().parents[1] / 'include' / 'nxattn.h'


@pytest.fixture(scope='module')
def lib():
    if not _lib.LIB_PATH.exists():
        from nitrix_amd import _build

        _build.build()
    return _lib.lib()


def _declared_functions():
    text = HEADER.read_text()
    # drop comments
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    return sorted(set(re.findall(r'\b(nxa_[a-z_]+)\s*\(', text)))


def test_header_declares_the_expected_api():
    assert _declared_functions() == sorted(_lib.EXPORTS)


def test_library_exports_every_declared_function(lib):
    for name in _declared_functions():
        assert hasattr(lib, name), name
    assert lib.nxa_version() == 5


def _desc(B=2, H=3, Lq=100, Lk=70, D=64, dtype=_lib.NXA_BF16):
    d = _lib.NxaDesc()
    d.B, d.H, d.Lq, d.Lk, d.D = B, H, Lq, Lk, D
    d.io_dtype = dtype
    d.bias_dtype = dtype
    d.scale = 0.125
    d.q_str[:] = (H * Lq * D, Lq * D, D)
    d.k_str[:] = (H * Lk * D, Lk * D, D)
    d.v_str[:] = (H * Lk * D, Lk * D, D)
    d.o_str[:] = (H * Lq * D, Lq * D, D)
    d.bias_str[:] = (0, Lq * Lk, Lk)
    d.mask_str[:] = (Lk, 0, 0)
    return d


def _check(lib, d, has_bias=1, has_mask=1):
    return lib.nxa_check(ctypes.byref(d), has_bias, has_mask)


def test_valid_descriptor(lib):
    assert _check(lib, _desc()) == _lib.NXA_OK
    assert _check(lib, _desc(dtype=_lib.NXA_F32, D=12)) == _lib.NXA_OK
    assert _check(lib, _desc(dtype=_lib.NXA_F16, D=40)) == _lib.NXA_OK
    d = _desc(D=64)
    d.Dv = 128  # value head dim different from the query / key one
    assert _check(lib, d) == _lib.NXA_OK
    assert _check(lib, _desc(D=256)) == _lib.NXA_OK
    assert _check(lib, _desc(dtype=_lib.NXA_F32, D=196)) == _lib.NXA_OK


def test_fp16_head_dim_multiple_of_8(lib):
    d = _desc(dtype=_lib.NXA_F16, D=12)
    assert _check(lib, d) == _lib.NXA_E_UNSUPPORTED
    assert 'multiple of 8' in lib.nxa_last_error().decode()


def test_mixed_bias_dtype_is_valid(lib):
    d = _desc(dtype=_lib.NXA_F16)
    d.bias_dtype = _lib.NXA_BF16
    assert _check(lib, d) == _lib.NXA_OK


@pytest.mark.parametrize(
    'mutate, code, text',
    [
        (lambda d: setattr(d, 'io_dtype', 7), _lib.NXA_E_DTYPE, 'io_dtype'),
        (lambda d: setattr(d, 'bias_dtype', 9), _lib.NXA_E_DTYPE, 'bias_dtype'),
        (lambda d: setattr(d, 'Lq', 0), _lib.NXA_E_SHAPE, 'positive'),
        (lambda d: setattr(d, 'D', 264), _lib.NXA_E_UNSUPPORTED, 'exceeds 256'),
        (lambda d: setattr(d, 'D', 12), _lib.NXA_E_UNSUPPORTED, 'multiple of 8'),
        (lambda d: setattr(d, 'Dv', 264), _lib.NXA_E_UNSUPPORTED, 'Dv=264 exceeds 256'),
        (lambda d: setattr(d, 'Dv', 20), _lib.NXA_E_UNSUPPORTED, 'Dv=20 must be a multiple'),
        (lambda d: setattr(d, 'Dv', -8), _lib.NXA_E_SHAPE, 'negative'),
        (lambda d: d.q_str.__setitem__(2, 65), _lib.NXA_E_LAYOUT, 'stride'),
        (lambda d: d.k_str.__setitem__(0, -64), _lib.NXA_E_LAYOUT, 'negative'),
        (lambda d: d.bias_str.__setitem__(1, -1), _lib.NXA_E_LAYOUT, 'bias'),
    ],
)
def test_invalid_descriptors(lib, mutate, code, text):
    d = _desc()
    mutate(d)
    assert _check(lib, d) == code
    assert text in lib.nxa_last_error().decode()


def test_null_descriptor(lib):
    assert lib.nxa_check(None, 0, 0) == _lib.NXA_E_ARG


def test_workspace_layout(lib):
    d = _desc(B=2, H=3, Lq=100, Lk=70)
    # no mask, no bias: the forward needs nothing
    assert lib.nxa_workspace_bytes(ctypes.byref(d), 0, 0, 0) == 0
    # mask [B,1,1,Lk] (zero H / Lq strides): one row of 64-key tiles per batch
    mb = 2 * 1 * 1 * 2  # MB * MH * MQ * MK
    assert lib.nxa_workspace_bytes(ctypes.byref(d), 0, 1, 0) == 256 * (
        (mb + 255) // 256
    )
    # backward: delta and lse2 rows (2 x B*H*Lq fp32), 256-byte aligned each
    rows = 2 * 3 * 100 * 4
    assert lib.nxa_workspace_bytes(ctypes.byref(d), 0, 0, 1) == 2 * 256 * (
        (rows + 255) // 256
    )
    # bias shared over the batch, no dbias wanted: nothing more
    assert lib.nxa_workspace_bytes(ctypes.byref(d), 1, 0, _lib.NXA_WS_BWD) == 2 * 256 * (
        (rows + 255) // 256
    )
    # with dbias: an fp32 accumulator of the bias extent [1,H,Lq,Lk] plus one
    # chunk of per-(batch, head) partials; here every pair fits one chunk
    slot = 100 * 70 * 4
    acc = 3 * slot
    part = min(2 * 3, max(3, -(-512 // 1))) * slot
    got = lib.nxa_workspace_bytes(ctypes.byref(d), 1, 0, _lib.NXA_WS_BWD | _lib.NXA_WS_DBIAS)
    assert got == 2 * 256 * ((rows + 255) // 256) + 256 * ((acc + 255) // 256) + 256 * (
        (part + 255) // 256
    )
    # unknown flags are rejected
    assert lib.nxa_workspace_bytes(ctypes.byref(d), 1, 0, 4) == 0


def test_dbias_workspace_is_bounded_by_the_bias_extent(lib):
    """A bias shared over many (batch, head) pairs: the dbias buffers are the
    fp32 accumulator of the bias's own extent plus one chunk of partials
    (enough pairs for ~512 dK/dV blocks), not B * H * Lq * Lk."""
    B, H, L = 4096, 4, 343  # windowed attention: many windows share a bias
    d = _desc(B=B, H=H, Lq=L, Lk=L, D=32)
    d.bias_str[:] = (0, L * L, L)  # [1, H, L, L]
    base = lib.nxa_workspace_bytes(ctypes.byref(d), 1, 0, _lib.NXA_WS_BWD)
    got = lib.nxa_workspace_bytes(ctypes.byref(d), 1, 0, _lib.NXA_WS_BWD | _lib.NXA_WS_DBIAS)
    slot = L * L * 4
    nkt = -(-L // 128)
    chunk = max(H, -(-512 // nkt))
    assert got - base == 256 * (-(-H * slot // 256)) + 256 * (-(-chunk * slot // 256))
    assert got - base < B * H * slot / 50
    # a full (unshared) bias needs no dbias buffers at all
    d.bias_str[:] = (H * L * L, L * L, L)
    assert lib.nxa_workspace_bytes(ctypes.byref(d), 1, 0, _lib.NXA_WS_BWD | _lib.NXA_WS_DBIAS) == base


def _a256(n):
    return 256 * (-(-n // 256))


def test_block_order_workspace(lib):
    """A mask that varies over queries (16-bit, not causal) adds the block
    order after the tile map: per mask slice, int32 lists of the 128-row,
    256-row and 128-key blocks.  Causal calls, fp32 I/O and masks broadcast
    over queries add nothing."""
    B, H, Lq, Lk = 2, 3, 1000, 1100
    MQ, MK = -(-Lq // 64), -(-Lk // 64)
    lists = -(-MQ // 2) + -(-MQ // 4) + -(-MK // 2)
    d = _desc(B=B, H=H, Lq=Lq, Lk=Lk)
    d.mask_str[:] = (0, Lq * Lk, Lk)  # [1, H, Lq, Lk]: H slices
    fwd = lib.nxa_workspace_bytes(ctypes.byref(d), 0, 1, _lib.NXA_WS_FWD)
    assert fwd == _a256(H * MQ * MK) + _a256(H * lists * 4)
    # the backward's per-row values follow the same mask regions
    rows = _a256(B * H * Lq * 4)
    assert lib.nxa_workspace_bytes(ctypes.byref(d), 0, 1, _lib.NXA_WS_BWD) == fwd + 2 * rows
    d.causal = 1
    assert lib.nxa_workspace_bytes(ctypes.byref(d), 0, 1, _lib.NXA_WS_FWD) == _a256(H * MQ * MK)
    d = _desc(B=B, H=H, Lq=Lq, Lk=Lk, dtype=_lib.NXA_F32)
    d.mask_str[:] = (0, Lq * Lk, Lk)
    assert lib.nxa_workspace_bytes(ctypes.byref(d), 0, 1, _lib.NXA_WS_FWD) == _a256(H * MQ * MK)
    d = _desc(B=B, H=H, Lq=Lq, Lk=Lk)
    d.mask_str[:] = (0, Lk, 0)  # [1, H, 1, Lk]
    assert lib.nxa_workspace_bytes(ctypes.byref(d), 0, 1, _lib.NXA_WS_FWD) == _a256(H * MK)
    # more than 1024 blocks in a list: blocks stay in index order
    d = _desc(B=1, H=1, Lq=131072 + 128, Lk=256)
    d.mask_str[:] = (0, 0, 256)
    MQ = -(-d.Lq // 64)
    assert lib.nxa_workspace_bytes(ctypes.byref(d), 0, 1, _lib.NXA_WS_FWD) == _a256(MQ * 4)


@pytest.mark.parametrize('which', ['q', 'k', 'v', 'o'])
def test_row_stride_bound(lib, which):
    """64 rows of a tile are addressed with 32-bit byte offsets: a row stride
    whose 64 rows reach 2^32 bytes is NXA_E_LAYOUT, one just below is fine."""
    d = _desc()
    limit = ((1 << 32) // 2 - 256) // 64  # bf16 elements; strides are multiples of 8
    ok = (limit - 1) // 8 * 8
    bad = -(-limit // 8) * 8
    getattr(d, f'{which}_str')[2] = ok
    assert _check(lib, d) == _lib.NXA_OK
    getattr(d, f'{which}_str')[2] = bad
    assert _check(lib, d) == _lib.NXA_E_LAYOUT
    assert 'row stride' in lib.nxa_last_error().decode()


def test_bias_row_stride_bound(lib):
    d = _desc()
    d.bias_dtype = _lib.NXA_F32
    limit = ((1 << 32) // 4 - 256) // 64
    d.bias_str[2] = limit - 1
    assert _check(lib, d) == _lib.NXA_OK
    d.bias_str[2] = limit + 1
    assert _check(lib, d) == _lib.NXA_E_LAYOUT
    assert 'bias row stride' in lib.nxa_last_error().decode()
    assert _check(lib, d, has_bias=0) == _lib.NXA_OK  # ignored without a bias


def test_entry_points_reject_null_buffers_without_a_gpu(lib):
    d = _desc()
    rc = lib.nxa_fwd(ctypes.byref(d), None, None, None, None, None, None, None,
                     None, 0, None)
    assert rc == _lib.NXA_E_ARG
    assert 'NULL' in lib.nxa_last_error().decode()
    rc = lib.nxa_bwd(ctypes.byref(d), None, None, None, None, None, None, None,
                     None, None, None, None, None, None, None, 0, 0, None)
    assert rc == _lib.NXA_E_ARG


def test_entry_points_reject_misaligned_buffers(lib):
    d = _desc()
    odd = ctypes.c_void_p(0x1008)
    ok = ctypes.c_void_p(0x2000)
    rc = lib.nxa_fwd(ctypes.byref(d), odd, ok, ok, None, None, ok, None, None,
                     0, None)
    assert rc == _lib.NXA_E_LAYOUT
    assert '16-byte' in lib.nxa_last_error().decode()


def test_forward_with_mask_requires_workspace(lib):
    d = _desc()
    ok = ctypes.c_void_p(0x2000)
    rc = lib.nxa_fwd(ctypes.byref(d), ok, ok, ok, None, ok, ok, None, None, 0,
                     None)
    assert rc == _lib.NXA_E_WORKSPACE


def test_backward_rejects_broadcast_keys(lib):
    d = _desc()
    d.k_str[1] = 0  # k shared over heads
    ok = ctypes.c_void_p(0x2000)
    rc = lib.nxa_bwd(ctypes.byref(d), ok, ok, ok, None, None, ok, ok, ok, ok,
                     ok, ok, None, None, ok, 1 << 20, 0, None)
    assert rc == _lib.NXA_E_UNSUPPORTED


def test_profile_read_without_records(lib):
    _lib.profile_reset()
    assert _lib.profile_read('fwd') == (0.0, 0)


def test_noalloc_forward_rejects_a_tile_map_beyond_the_scratch(lib):
    """nxa_fwd_noalloc keeps the tile map in a static 8 MiB device array: a
    mask whose tile map is larger is NXA_E_WORKSPACE before anything runs
    (no GPU needed to see it)."""
    L = 65536 + 64  # 1025 x 1025 tiles per head
    d = _desc(B=8, H=1, Lq=L, Lk=L, D=64)
    d.mask_str[:] = (L * L, 0, L)  # [B, 1, L, L] mask
    need = lib.nxa_workspace_bytes(ctypes.byref(d), 0, 1, _lib.NXA_WS_FWD)
    assert need > _lib.NXA_NOALLOC_SCRATCH_BYTES
    ok = ctypes.c_void_p(0x2000)
    rc = lib.nxa_fwd_noalloc(ctypes.byref(d), ok, ok, ok, None, ok, ok, None, None)
    assert rc == _lib.NXA_E_WORKSPACE
    assert 'static scratch' in lib.nxa_last_error().decode()
    # and it validates like nxa_fwd
    rc = lib.nxa_fwd_noalloc(ctypes.byref(d), None, ok, ok, None, ok, ok, None, None)
    assert rc == _lib.NXA_E_ARG



@pytest.mark.parametrize('D, code, text', [
    (264, _lib.NXA_E_UNSUPPORTED, 'exceeds 256'),
    (12, _lib.NXA_E_UNSUPPORTED, 'multiple of 8'),
    (0, _lib.NXA_E_SHAPE, 'D > 0'),
])
def test_rms_norm_rejects_head_dims_it_cannot_hold(lib, D, code, text):
    # Validation happens before any launch, so no GPU is needed.
    ok = ctypes.c_void_p(0x2000)
    rc = lib.nxa_rms_norm_fwd(4, D, _lib.NXA_BF16, ok, max(D, 8), ok, None, 1e-6, None)
    assert rc == code
    assert text in lib.nxa_last_error().decode()
    rc = lib.nxa_rms_norm_bwd(4, D, _lib.NXA_BF16, ok, max(D, 8), ok, ok, ok, None)
    assert rc == code


def test_fused_q_norm_forward_rejects_what_it_cannot_take(lib):
    ok = ctypes.c_void_p(0x2000)
    d = _desc()
    d.io_dtype = _lib.NXA_F32
    rc = lib.nxa_fwd_normed(ctypes.byref(d), ok, ok, ok, None, None, ok, ok, ok, ok, 1e-6,
                            None, 0, None)
    assert rc == _lib.NXA_E_UNSUPPORTED and 'bf16 / fp16' in lib.nxa_last_error().decode()
    d = _desc()
    d.B, d.q_str[0] = 2, 0
    rc = lib.nxa_fwd_normed(ctypes.byref(d), ok, ok, ok, None, None, ok, ok, ok, ok, 1e-6,
                            None, 0, None)
    assert rc == _lib.NXA_E_UNSUPPORTED and 'broadcast' in lib.nxa_last_error().decode()
    d = _desc()
    odd = ctypes.c_void_p(0x1008)
    rc = lib.nxa_fwd_normed(ctypes.byref(d), ok, ok, ok, None, None, ok, ok, odd, ok, 1e-6,
                            None, 0, None)
    assert rc == _lib.NXA_E_LAYOUT and 'q_hat' in lib.nxa_last_error().decode()
    rc = lib.nxa_fwd_normed(ctypes.byref(d), ok, ok, ok, None, None, ok, ok, ok, ok, -1.0,
                            None, 0, None)
    assert rc == _lib.NXA_E_ARG
