"""Shared pytest configuration.

* registers the ``gpu`` marker (tests that need an MI355X);
* puts the repository root on ``sys.path`` so ``nitrix_amd`` and ``oracle``
  import from the checkout;
* a hypothesis profile without deadlines (the same policy as the
  reference's ``tests/conftest.py:35-41``: no wall-clock assertions, capped
  example count).
"""

from __future__ import annotations

import os
import sys

_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if _ROOT not in sys.path:
    sys.path.insert(0, _ROOT)

try:
    from hypothesis import HealthCheck, settings

    settings.register_profile(
        'nxattn',
        deadline=None,
        max_examples=25,
        suppress_health_check=[
            HealthCheck.too_slow,
            HealthCheck.data_too_large,
        ],
    )
    settings.load_profile('nxattn')
except ImportError:  # pragma: no cover
    pass


def pytest_configure(config):
    config.addinivalue_line(
        'markers', 'gpu: needs an MI355X (gfx950) and the built HIP library'
    )
