"""Which engine runs a call, and how a declined fused call is reported.

Behaviour follows the reference's dispatch layer
(``src/nitrix/_internal/backend.py:227-267`` for resolution,
``:307-373`` for the fallback warning, ``config.py:78-149`` for reproducible
mode); the code here is organised differently:

* :class:`_Knobs` is one snapshot of the process environment per call
  (``NITRIX_BACKEND``, ``NITRIX_SILENCE_FALLBACK``, ``NITRIX_STRICT_BACKEND``),
  so a call sees one consistent setting even while another thread edits the
  environment;
* resolution is a chain of rules over (keyword, env choice, device, mode), in
  :func:`resolve_backend`;
* :class:`_Ledger` remembers which fallbacks were already reported, keyed by
  (function, shapes, dtype, requested engine).

Engines: ``'hip'`` is the fused gfx950 library and takes the place of the
reference's ``'pallas-cuda'``, which names NVIDIA hardware and is refused
here; ``'jax'`` names the unfused reference engine, as in the reference.
``'auto'`` picks ``'hip'`` for tensors on a gfx950 device unless reproducible
mode is on, else ``'jax'``.  A gfx950 device whose library cannot be loaded is
an error raised by the caller, never a silent fallback.
"""

from __future__ import annotations

import contextlib
import contextvars
import os
import threading
import warnings
from dataclasses import dataclass
from typing import Any, Iterator, Literal, Optional

Backend = Literal['auto', 'hip', 'jax', 'pallas-cuda']
ResolvedBackend = Literal['hip', 'jax']

# Every spelling the keyword and NITRIX_BACKEND accept.
_CHOICES = ('auto', 'hip', 'jax', 'pallas-cuda')
_TRUTHY = frozenset({'1', 'true', 'yes', 'on'})


class NitrixBackendFallback(UserWarning):
    """A fused call was declined for its shape or dtype and ran on the
    reference engine.  Reported once per (function, shapes, dtype, requested
    engine) per process; ``NITRIX_SILENCE_FALLBACK=1`` mutes it and
    ``NITRIX_STRICT_BACKEND=1`` turns it into :class:`NitrixBackendError`
    (the reference's category, ``backend.py:40-51``)."""


class NitrixBackendError(RuntimeError):
    """The requested engine cannot run here, or a fallback was made strict
    (``backend.py:54-60`` of the reference)."""


def _bad_choice(where: str, value: Any) -> NitrixBackendError:
    return NitrixBackendError(f'{where}={value!r} not in {_CHOICES!r}')


@dataclass(frozen=True)
class _Knobs:
    """The environment as one call sees it."""

    backend: Optional[str]  # normalised NITRIX_BACKEND, None when unset
    silent: bool
    strict: bool

    @classmethod
    def read(cls) -> '_Knobs':
        env = os.environ
        raw = env.get('NITRIX_BACKEND')
        choice = None if raw is None else raw.strip().lower()
        if choice is not None and choice not in _CHOICES:
            raise _bad_choice('NITRIX_BACKEND', choice)
        flag = lambda name: env.get(name, '0').lower() in _TRUTHY  # noqa: E731
        return cls(choice, flag('NITRIX_SILENCE_FALLBACK'), flag('NITRIX_STRICT_BACKEND'))


def silence_fallback() -> bool:
    """``NITRIX_SILENCE_FALLBACK`` is set to a true value."""
    return _Knobs.read().silent


def strict_backend() -> bool:
    """``NITRIX_STRICT_BACKEND`` is set to a true value."""
    return _Knobs.read().strict


def env_backend() -> Optional[str]:
    """The engine named by ``NITRIX_BACKEND`` (lower-cased), or None."""
    return _Knobs.read().backend


# --- reproducible mode ---------------------------------------------------------
# A context variable, so a ``with reproducible():`` block affects only its own
# thread / task (the reference keeps the flag the same way, config.py:33-37).

_reproducible_mode: contextvars.ContextVar[bool] = contextvars.ContextVar(
    'nitrix_amd_reproducible',
    default=os.environ.get('NITRIX_REPRODUCIBLE', '0').lower() in _TRUTHY,
)


def reproducible_enabled() -> bool:
    return _reproducible_mode.get()


def set_reproducible(enabled: bool = True) -> None:
    _reproducible_mode.set(bool(enabled))


@contextlib.contextmanager
def reproducible(enabled: bool = True) -> Iterator[None]:
    """Inside the block ``'auto'`` picks the reference engine, whose results
    do not depend on the hardware."""
    token = _reproducible_mode.set(bool(enabled))
    try:
        yield
    finally:
        _reproducible_mode.reset(token)


# --- hardware --------------------------------------------------------------------


# Architecture test per device index: a device's properties do not change
# within a process, and the lookup costs more host time than a small launch.
_GFX950_BY_INDEX: dict = {}


def device_is_gfx950(device: Any) -> bool:
    """True for a ROCm device whose architecture is gfx950 (MI355X)."""
    if getattr(device, 'type', None) != 'cuda':
        return False
    index = getattr(device, 'index', None)
    hit = _GFX950_BY_INDEX.get(index) if index is not None else None
    if hit is not None:
        return hit
    import torch

    if torch.version.hip is None:
        return False
    try:
        arch = torch.cuda.get_device_properties(device).gcnArchName
    except Exception:  # pragma: no cover - no usable device
        return False
    ok = str(arch).partition(':')[0] == 'gfx950'
    if index is not None:
        _GFX950_BY_INDEX[index] = ok
    return ok


def auto_backend(device: Any) -> ResolvedBackend:
    """What ``'auto'`` means for tensors on ``device``."""
    if not reproducible_enabled() and device_is_gfx950(device):
        return 'hip'
    return 'jax'


def resolve_backend(backend: str, device: Any) -> ResolvedBackend:
    """The engine that runs a call: keyword, else ``NITRIX_BACKEND``, else
    ``'auto'``.

    Explicit fused requests are checked against the hardware whatever
    ``NITRIX_STRICT_BACKEND`` says: ``'hip'`` for tensors off a gfx950 device
    raises, and ``'pallas-cuda'`` (NVIDIA only) always raises in this build.
    """
    if backend not in _CHOICES:
        raise _bad_choice('backend', backend)
    chosen = backend
    if chosen == 'auto':
        chosen = _Knobs.read().backend or 'auto'
    if chosen == 'auto':
        return auto_backend(device)
    if chosen == 'jax':
        return 'jax'
    if chosen == 'hip' and device_is_gfx950(device):
        return 'hip'
    if chosen == 'hip':
        raise NitrixBackendError(
            "backend='hip' requested, but the tensors are not on a ROCm "
            "gfx950 device. Use backend='jax' or backend='auto'."
        )
    raise NitrixBackendError(
        "backend='pallas-cuda' requested, but this build targets AMD "
        "gfx950; use backend='hip', 'auto' or 'jax'."
    )


# --- fallback reporting ------------------------------------------------------------


def _dims(shape: Any) -> str:
    if shape is None:
        return 'None'
    if isinstance(shape, (tuple, list)):
        return 'x'.join(map(str, shape))
    return str(shape)


class _Ledger:
    """The fallbacks already reported in this process."""

    def __init__(self) -> None:
        self._seen: set = set()
        self._mu = threading.Lock()

    def first_time(self, key: tuple) -> bool:
        """Records ``key``; True the first time it is seen."""
        with self._mu:
            fresh = key not in self._seen
            self._seen.add(key)
            return fresh

    def clear(self) -> None:
        with self._mu:
            self._seen.clear()


_ledger = _Ledger()


def fallback(
    *,
    function: str,
    requested: str,
    resolved: str,
    reason: str,
    shapes: tuple = (),
    dtype: Any = None,
) -> str:
    """Reports that ``function`` runs on ``resolved`` instead of
    ``requested`` and returns ``resolved``.

    Nothing happens when the two agree.  Otherwise ``NITRIX_STRICT_BACKEND``
    raises :class:`NitrixBackendError`, ``NITRIX_SILENCE_FALLBACK`` stays
    quiet, and by default one :class:`NitrixBackendFallback` is issued per
    (function, shapes, dtype, requested) in the process.
    """
    if requested == resolved:
        return resolved
    knobs = _Knobs.read()
    if knobs.strict:
        raise NitrixBackendError(
            f'{function}: requested backend={requested!r} but would fall '
            f'back to {resolved!r} ({reason}). NITRIX_STRICT_BACKEND=1 '
            'converted this to an error.'
        )
    key = (function, ';'.join(_dims(s) for s in shapes), str(dtype), requested)
    if not knobs.silent and _ledger.first_time(key):
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
    """Forget the fallbacks already reported, so each warns again."""
    _ledger.clear()
