"""``nitrix.nn`` import path for the attention and selective-scan entry
points (``src/nitrix/nn/__init__.py:30-44`` of the reference)."""

from ..attention import (
    reference_scaled_dot_product_attention,
    scaled_dot_product_attention,
)
from ..ssm import reference_selective_scan, selective_scan

__all__ = [
    'reference_scaled_dot_product_attention',
    'reference_selective_scan',
    'scaled_dot_product_attention',
    'selective_scan',
]
