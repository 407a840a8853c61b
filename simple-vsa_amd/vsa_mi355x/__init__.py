"""MI355X-native Video Sparse Attention (package ``vsa_mi355x``).

The package is named apart from the reference's own ``vsa`` package so that
both can be imported in one process: the reference registers this backend in
its ``vsa`` namespace with a lazy loader (vsa/__init__.py:28-69 is how it
registers ``triton_vsa`` and the others), and the loader imports
``vsa_mi355x.mi355x`` on the first call.

Importing ``vsa_mi355x`` needs only torch; the gfx950 kernel library is loaded
on the first call.  The tiling helpers and the gate producer keep the
reference's names (vsa/__init__.py:7, 10-25).
"""

from typing import Any

from .gate import CompressionGate
from .tiling import build_vsa_metadata, tile, untile

__all__ = ["mi355x_vsa", "mi355x_sparse_attention", "mi355x_sparse_executor", "mi355x_route",
           "mi355x_vsa_tiled", "CompressionGate", "build_vsa_metadata", "tile", "untile"]


def mi355x_vsa(*args: Any, **kwargs: Any) -> Any:
    """Full VSA (coarse + routed fine branch) on MI355X; see ``vsa_mi355x.mi355x``."""
    from .mi355x import mi355x_vsa as _impl

    return _impl(*args, **kwargs)


def mi355x_sparse_attention(*args: Any, **kwargs: Any) -> Any:
    """Route-explicit sparse executor on MI355X; see ``vsa_mi355x.mi355x``."""
    from .mi355x import mi355x_sparse_attention as _impl

    return _impl(*args, **kwargs)


def mi355x_sparse_executor(*args: Any, **kwargs: Any) -> Any:
    """Sparse-executor callable for a shared orchestrator; see ``vsa_mi355x.mi355x``."""
    from .mi355x import mi355x_sparse_executor as _impl

    return _impl(*args, **kwargs)


def mi355x_route(*args: Any, **kwargs: Any) -> Any:
    """Coarse scores and Top-K route that ``mi355x_vsa`` uses."""
    from .mi355x import mi355x_route as _impl

    return _impl(*args, **kwargs)


def mi355x_vsa_tiled(*args: Any, **kwargs: Any) -> Any:
    """VSA on raster-order video tokens with tile / untile fused into the op;
    see ``vsa_mi355x.tiled``."""
    from .tiled import mi355x_vsa_tiled as _impl

    return _impl(*args, **kwargs)
