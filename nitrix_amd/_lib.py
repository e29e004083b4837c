"""ctypes binding of ``libnxattn.so`` (declared in ``include/nxattn.h``).

The library is built in-tree by ``nitrix_amd._build`` (``__graft_entry__.build``)
and loaded from the package directory.  A missing or unloadable library is
an error, never a silent fallback: :func:`lib` raises
:class:`HipLibraryMissing`.
"""

from __future__ import annotations

import ctypes
import pathlib
import threading

LIB_PATH = pathlib.Path(__file__).resolve().parent / 'libnxattn.so'

NXA_BF16 = 0
NXA_F32 = 1
NXA_F16 = 2

# nxa_workspace_bytes flags
NXA_WS_FWD = 0
NXA_WS_BWD = 1
NXA_WS_DBIAS = 2

# static scratch of nxa_fwd_noalloc (NXA_NOALLOC_SCRATCH_BYTES)
NXA_NOALLOC_SCRATCH_BYTES = 8 << 20

NXA_OK = 0
NXA_E_ARG = -1
NXA_E_SHAPE = -2
NXA_E_DTYPE = -3
NXA_E_LAYOUT = -4
NXA_E_WORKSPACE = -5
NXA_E_LAUNCH = -6
NXA_E_UNSUPPORTED = -7

ERROR_NAMES = {
    NXA_E_ARG: 'NXA_E_ARG',
    NXA_E_SHAPE: 'NXA_E_SHAPE',
    NXA_E_DTYPE: 'NXA_E_DTYPE',
    NXA_E_LAYOUT: 'NXA_E_LAYOUT',
    NXA_E_WORKSPACE: 'NXA_E_WORKSPACE',
    NXA_E_LAUNCH: 'NXA_E_LAUNCH',
    NXA_E_UNSUPPORTED: 'NXA_E_UNSUPPORTED',
}

# Every symbol include/nxattn.h declares.
EXPORTS = (
    'nxa_version',
    'nxa_check',
    'nxa_workspace_bytes',
    'nxa_fwd',
    'nxa_fwd_noalloc',
    'nxa_fwd_normed',
    'nxa_bwd',
    'nxa_bwd_normed',
    'nxa_rms_norm_fwd',
    'nxa_rms_norm_bwd',
    'nxa_ssm_check',
    'nxa_ssm_state_bytes',
    'nxa_ssm_workspace_bytes',
    'nxa_ssm_fwd',
    'nxa_ssm_bwd',
    'nxa_last_error',
    'nxa_profile_enable',
    'nxa_profile_read',
    'nxa_profile_reset',
)

_I64x3 = ctypes.c_int64 * 3


class NxaDesc(ctypes.Structure):
    """Mirror of ``nxa_desc``."""

    _fields_ = [
        ('B', ctypes.c_int32),
        ('H', ctypes.c_int32),
        ('Lq', ctypes.c_int32),
        ('Lk', ctypes.c_int32),
        ('D', ctypes.c_int32),
        ('io_dtype', ctypes.c_int32),
        ('bias_dtype', ctypes.c_int32),
        ('causal', ctypes.c_int32),
        ('scale', ctypes.c_float),
        ('q_str', _I64x3),
        ('k_str', _I64x3),
        ('v_str', _I64x3),
        ('o_str', _I64x3),
        ('bias_str', _I64x3),
        ('mask_str', _I64x3),
        ('Dv', ctypes.c_int32),
    ]


class HipLibraryMissing(RuntimeError):
    """``libnxattn.so`` is absent or cannot be loaded."""


class NxaError(RuntimeError):
    """A C-ABI call returned a nonzero status."""

    def __init__(self, code: int, message: str):
        super().__init__(f'{ERROR_NAMES.get(code, code)}: {message}')
        self.code = code


_lock = threading.Lock()
_lib = None


def _declare(lib: ctypes.CDLL) -> None:
    vp = ctypes.c_void_p
    dp = ctypes.POINTER(NxaDesc)
    lib.nxa_version.restype = ctypes.c_int
    lib.nxa_version.argtypes = []
    lib.nxa_check.restype = ctypes.c_int
    lib.nxa_check.argtypes = [dp, ctypes.c_int, ctypes.c_int]
    lib.nxa_workspace_bytes.restype = ctypes.c_size_t
    lib.nxa_workspace_bytes.argtypes = [dp, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    lib.nxa_fwd.restype = ctypes.c_int
    lib.nxa_fwd.argtypes = [dp, vp, vp, vp, vp, vp, vp, vp, vp, ctypes.c_size_t, vp]
    lib.nxa_fwd_noalloc.restype = ctypes.c_int
    lib.nxa_fwd_noalloc.argtypes = [dp, vp, vp, vp, vp, vp, vp, vp, vp]
    lib.nxa_fwd_normed.restype = ctypes.c_int
    lib.nxa_fwd_normed.argtypes = [
        dp, vp, vp, vp, vp, vp, vp, vp, vp, vp, ctypes.c_float, vp, ctypes.c_size_t, vp,
    ]
    lib.nxa_bwd.restype = ctypes.c_int
    lib.nxa_bwd.argtypes = [
        dp,
        vp, vp, vp, vp, vp,  # q k v bias mask
        vp, vp, vp,  # o lse dout
        vp, vp, vp, vp,  # dq dk dv dbias
        ctypes.POINTER(ctypes.c_int64),  # dbias_str
        vp, ctypes.c_size_t, ctypes.c_int, vp,
    ]
    lib.nxa_bwd_normed.restype = ctypes.c_int
    lib.nxa_bwd_normed.argtypes = [
        dp,
        vp, vp, vp, vp, vp,  # q_hat k_hat v bias mask
        vp, vp, vp,  # o lse dout
        vp, vp, vp, vp,  # q k q_rstd k_rstd
        vp, vp, vp, vp,  # dq dk dv dbias
        ctypes.POINTER(ctypes.c_int64),  # dbias_str
        vp, ctypes.c_size_t, ctypes.c_int, vp,
    ]
    i64, i32 = ctypes.c_int64, ctypes.c_int32
    lib.nxa_rms_norm_fwd.restype = ctypes.c_int
    lib.nxa_rms_norm_fwd.argtypes = [i64, i32, i32, vp, i64, vp, vp, ctypes.c_float, vp]
    lib.nxa_rms_norm_bwd.restype = ctypes.c_int
    lib.nxa_rms_norm_bwd.argtypes = [i64, i32, i32, vp, i64, vp, vp, vp, vp]
    lib.nxa_ssm_check.restype = ctypes.c_int
    lib.nxa_ssm_check.argtypes = [i64, i32, i32, i32]
    lib.nxa_ssm_state_bytes.restype = ctypes.c_size_t
    lib.nxa_ssm_state_bytes.argtypes = [i64, i32, i32, i32]
    lib.nxa_ssm_workspace_bytes.restype = ctypes.c_size_t
    lib.nxa_ssm_workspace_bytes.argtypes = [i64, i32, i32, i32, ctypes.c_int]
    lib.nxa_ssm_fwd.restype = ctypes.c_int
    lib.nxa_ssm_fwd.argtypes = [i64, i32, i32, i32] + [vp] * 9 + [ctypes.c_size_t, vp]
    lib.nxa_ssm_bwd.restype = ctypes.c_int
    lib.nxa_ssm_bwd.argtypes = [i64, i32, i32, i32] + [vp] * 15 + [ctypes.c_size_t, vp]
    lib.nxa_last_error.restype = ctypes.c_char_p
    lib.nxa_last_error.argtypes = []
    lib.nxa_profile_enable.restype = ctypes.c_int
    lib.nxa_profile_enable.argtypes = [ctypes.c_int]
    lib.nxa_profile_read.restype = ctypes.c_int
    lib.nxa_profile_read.argtypes = [
        ctypes.c_char_p,
        ctypes.POINTER(ctypes.c_double),
        ctypes.POINTER(ctypes.c_int64),
    ]
    lib.nxa_profile_reset.restype = ctypes.c_int
    lib.nxa_profile_reset.argtypes = []


def lib() -> ctypes.CDLL:
    """Load (once) and return the library; raise if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise HipLibraryMissing(
                    f'{LIB_PATH} is missing: build it with '
                    '`python -m nitrix_amd._build` (hipcc, gfx950)'
                )
            try:
                handle = ctypes.CDLL(str(LIB_PATH))
            except OSError as exc:
                raise HipLibraryMissing(f'cannot load {LIB_PATH}: {exc}') from exc
            _declare(handle)
            _lib = handle
    return _lib


def available() -> bool:
    try:
        lib()
    except HipLibraryMissing:
        return False
    return True


def check(rc: int) -> None:
    """Raise :class:`NxaError` with the library's message for rc != 0."""
    if rc != NXA_OK:
        msg = lib().nxa_last_error().decode('utf-8', 'replace')
        raise NxaError(rc, msg)


def profile_enable(on: bool) -> None:
    check(lib().nxa_profile_enable(1 if on else 0))


def profile_reset() -> None:
    check(lib().nxa_profile_reset())


def profile_read(kernel: str) -> tuple[float, int]:
    ms = ctypes.c_double()
    n = ctypes.c_int64()
    check(lib().nxa_profile_read(kernel.encode(), ctypes.byref(ms), ctypes.byref(n)))
    return ms.value, n.value
