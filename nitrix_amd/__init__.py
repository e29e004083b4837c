"""nitrix_amd -- MI355X-native (gfx950) fused scaled-dot-product attention.

A drop-in for nitrix's attention path (``nitrix.nn.attention``) and its
sibling fused selective scan (``nitrix.nn.ssm``): the same call signatures,
backed by hand-written HIP kernels behind a C ABI (``include/nxattn.h``,
``libnxattn.so``).
"""

from ._backend import (
    NitrixBackendError,
    NitrixBackendFallback,
    reproducible,
    reset_fallback_state,
    resolve_backend,
)
from .attention import (
    HipNotTileable,
    default_scale,
    qk_rms_norm,
    reference_scaled_dot_product_attention,
    scaled_dot_product_attention,
    scaled_dot_product_attention_hip,
)
from .ssm import (
    reference_selective_scan,
    selective_scan,
    selective_scan_hip,
)

__all__ = [
    'HipNotTileable',
    'NitrixBackendError',
    'NitrixBackendFallback',
    'default_scale',
    'qk_rms_norm',
    'reference_scaled_dot_product_attention',
    'reference_selective_scan',
    'reproducible',
    'reset_fallback_state',
    'resolve_backend',
    'scaled_dot_product_attention',
    'scaled_dot_product_attention_hip',
    'selective_scan',
    'selective_scan_hip',
]
