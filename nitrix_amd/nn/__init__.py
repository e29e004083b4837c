"""``nitrix.nn`` import path for the attention entry points
(``src/nitrix/nn/__init__.py:30-44`` of the reference)."""

from ..attention import (
    reference_scaled_dot_product_attention,
    scaled_dot_product_attention,
)

__all__ = [
    'reference_scaled_dot_product_attention',
    'scaled_dot_product_attention',
]
