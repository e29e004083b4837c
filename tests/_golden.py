"""Golden-fixture and tolerance helpers.

The fixtures under ``tests/golden/`` are the reference's own
(``tests/golden/attention_*_float32.npz``; see ``tests/golden/NOTICE``).  The
tolerance table restates the attention rows of the reference's
``tests/tolerance.toml:11-22, 59-64`` plus the budgets this build is held to.
"""

from __future__ import annotations

import pathlib

import numpy as np

GOLDEN_DIR = pathlib.Path(__file__).resolve().parent / 'golden'

ATTENTION_CASES = [
    'attention_dense_float32',
    'attention_windowed_bias_float32',
    'attention_causal_float32',
    'attention_cross_float32',
    'attention_qk_norm_float32',
]

# (atol, rtol) -- tolerance.toml:11-13 (float32), 15-17 (float64),
# 20-22 (fused path), 59-64 (bf16 / fp16 reduced-precision reference).
TOL = {
    ('attention', 'float32'): (1e-6, 1e-5),
    ('attention', 'float64'): (1e-12, 1e-12),
    ('attention', 'float32', 'fused'): (2e-3, 2e-3),
    ('attention', 'bfloat16'): (1e-2, 8e-3),
    ('attention', 'float16'): (1e-3, 1e-3),
}

# Max-relative budgets (max|a-b| / max|b|) of this build against the oracle:
# fp32 I/O <= 1e-5, bf16 I/O <= 2e-2 against the fp32 oracle, the same for
# gradients.
REL_FP32 = 1e-5
REL_BF16 = 2e-2

# The cross fixture was generated with TF32 matmul operands (it matches a
# float64 restatement only to ~8e-4), so it is checked at this budget.
CROSS_ATOL = 2e-3


def load_golden(name: str) -> dict:
    with np.load(GOLDEN_DIR / f'{name}.npz') as data:
        return {key: data[key] for key in data.files}


def relerr(a, b) -> float:
    """``max|a - b| / max|b|`` (the reference's ``_relerr``,
    ``tests/test_nn_attention_kernel.py:51-52``)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / (np.max(np.abs(b)) + 1e-30))
