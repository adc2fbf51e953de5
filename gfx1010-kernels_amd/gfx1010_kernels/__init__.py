"""MI355X (gfx950) fused residual-add + dropout + LayerNorm.

Drop-in replacement for the residual LayerNorm surface of the reference
package (gfx1010_kernels/__init__.py:15-19): ``residual_layer_norm``,
``can_use_residual_layer_norm``, ``residual_layer_norm_status`` and
``BackendStatus``, plus the pre-norm integration helpers ``residual_norm``
and ``prenorm_forward`` (the reference's integration recipe,
docs/residual_layer_norm.md:51-83, as code). The reference's attention,
patch, linear and Triton exports are not part of this build.
"""

from ._status import BackendStatus
from .normalization import (
    can_use_residual_layer_norm,
    residual_layer_norm,
    residual_layer_norm_status,
)
from .prenorm import prenorm_forward, residual_norm

# API version of the reference surface this package reproduces.
__version__ = "0.4.0"

__all__ = [
    "__version__",
    "BackendStatus",
    "can_use_residual_layer_norm",
    "prenorm_forward",
    "residual_layer_norm",
    "residual_layer_norm_status",
    "residual_norm",
]
