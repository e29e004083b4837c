"""Backend selection and loud fallback.

Mirrors the reference's three-level resolution
(``src/nitrix/_internal/backend.py:227-267``): explicit ``backend=`` keyword >
``NITRIX_BACKEND`` env var > auto-detect, with the same env knobs
(``NITRIX_SILENCE_FALLBACK``, ``NITRIX_STRICT_BACKEND``, ``:141-162``), the same
deduplicated ``NitrixBackendFallback`` warning (``:307-373``) and reproducible
mode forcing ``auto -> 'jax'`` (``:170-198``; ``config.py:78-149``).

The fused engine here is ``'hip'`` (hand-written gfx950 kernels) in place of
``'pallas-cuda'``.  ``'jax'`` names the unfused reference engine, as in the
reference: the same recipe written with stock tensor ops.

``auto`` resolves to ``'hip'`` for tensors on a ROCm gfx950 device (unless
reproducible mode is on) and to ``'jax'`` for tensors on the CPU.  A missing
or broken HIP library on a gfx950 device is an error, not a fallback.
"""

from __future__ import annotations

import contextlib
import contextvars
import os
import threading
import warnings
from typing import Any, Iterator, Literal, Optional

Backend = Literal['auto', 'hip', 'jax', 'pallas-cuda']
ResolvedBackend = Literal['hip', 'jax']

_VALID_BACKENDS = ('auto', 'hip', 'jax', 'pallas-cuda')


class NitrixBackendFallback(UserWarning):
    """Emitted once per ``(function, shapes, dtype, backend)`` when a shape the
    fused kernel declines runs on the reference engine instead
    (``backend.py:40-51`` of the reference).

    Silence with ``NITRIX_SILENCE_FALLBACK=1``; escalate with
    ``NITRIX_STRICT_BACKEND=1``.
    """


class NitrixBackendError(RuntimeError):
    """A backend cannot be honoured on this host (``backend.py:54-60``)."""


def _env_flag(name: str) -> bool:
    return os.environ.get(name, '0').lower() in ('1', 'true', 'yes', 'on')


def silence_fallback() -> bool:
    return _env_flag('NITRIX_SILENCE_FALLBACK')


def strict_backend() -> bool:
    return _env_flag('NITRIX_STRICT_BACKEND')


def env_backend() -> Optional[str]:
    value = os.environ.get('NITRIX_BACKEND')
    if value is None:
        return None
    value = value.strip().lower()
    if value not in _VALID_BACKENDS:
        raise NitrixBackendError(
            f'NITRIX_BACKEND={value!r} not in {_VALID_BACKENDS!r}'
        )
    return value


# --- reproducible mode (config.py:78-149) -----------------------------------

_REPRODUCIBLE: contextvars.ContextVar[bool] = contextvars.ContextVar(
    'nxattn_reproducible', default=_env_flag('NITRIX_REPRODUCIBLE')
)


def reproducible_enabled() -> bool:
    return _REPRODUCIBLE.get()


def set_reproducible(enabled: bool = True) -> None:
    _REPRODUCIBLE.set(bool(enabled))


@contextlib.contextmanager
def reproducible(enabled: bool = True) -> Iterator[None]:
    """Within the block, ``auto`` resolves to the reference engine."""
    token = _REPRODUCIBLE.set(bool(enabled))
    try:
        yield
    finally:
        _REPRODUCIBLE.reset(token)


# --- device probe --------------------------------------------------------------


def device_is_gfx950(device: Any) -> bool:
    """True for a ROCm device whose architecture is gfx950 (MI355X)."""
    import torch

    if getattr(device, 'type', None) != 'cuda' or torch.version.hip is None:
        return False
    try:
        props = torch.cuda.get_device_properties(device)
    except Exception:  # pragma: no cover - no device
        return False
    return str(getattr(props, 'gcnArchName', '')).split(':')[0] == 'gfx950'


def auto_backend(device: Any) -> ResolvedBackend:
    if reproducible_enabled():
        return 'jax'
    if device_is_gfx950(device):
        return 'hip'
    return 'jax'


def resolve_backend(backend: str, device: Any) -> ResolvedBackend:
    """Keyword > env var > auto (``backend.py:227-267``).

    An explicit ``'hip'`` for tensors that are not on a gfx950 device raises,
    whatever ``NITRIX_STRICT_BACKEND`` says; ``'pallas-cuda'`` (NVIDIA only in
    the reference) always raises here.
    """
    if backend not in _VALID_BACKENDS:
        raise NitrixBackendError(
            f'backend={backend!r} not in {_VALID_BACKENDS!r}'
        )
    if backend == 'auto':
        env = env_backend()
        if env is not None and env != 'auto':
            backend = env
        else:
            return auto_backend(device)
    if backend == 'pallas-cuda':
        raise NitrixBackendError(
            "backend='pallas-cuda' requested, but this build targets AMD "
            "gfx950; use backend='hip', 'auto' or 'jax'."
        )
    if backend == 'hip':
        if not device_is_gfx950(device):
            raise NitrixBackendError(
                "backend='hip' requested, but the tensors are not on a ROCm "
                "gfx950 device. Use backend='jax' or backend='auto'."
            )
        return 'hip'
    return 'jax'


# --- fallback warning (backend.py:275-383) -------------------------------------

_warned_keys: set = set()
_warned_lock = threading.Lock()


def _shape_signature(*shapes: Any) -> str:
    parts = []
    for s in shapes:
        if s is None:
            parts.append('None')
        elif isinstance(s, (tuple, list)):
            parts.append('x'.join(str(d) for d in s))
        else:
            parts.append(str(s))
    return ';'.join(parts)


def fallback(
    *,
    function: str,
    requested: str,
    resolved: str,
    reason: str,
    shapes: tuple = (),
    dtype: Any = None,
) -> str:
    if requested == resolved:
        return resolved
    if strict_backend():
        raise NitrixBackendError(
            f'{function}: requested backend={requested!r} but would fall '
            f'back to {resolved!r} ({reason}). NITRIX_STRICT_BACKEND=1 '
            'converted this to an error.'
        )
    if silence_fallback():
        return resolved
    key = (function, _shape_signature(*shapes), str(dtype), requested)
    with _warned_lock:
        if key in _warned_keys:
            return resolved
        _warned_keys.add(key)
    warnings.warn(
        f'{function}: falling back to backend={resolved!r} from '
        f'{requested!r}: {reason}. '
        'Set NITRIX_SILENCE_FALLBACK=1 to suppress this warning, or '
        'NITRIX_STRICT_BACKEND=1 to convert it to an error.',
        category=NitrixBackendFallback,
        stacklevel=3,
    )
    return resolved


def reset_fallback_state() -> None:
    with _warned_lock:
        _warned_keys.clear()
