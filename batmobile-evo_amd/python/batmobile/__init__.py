"""batmobile on MI355X: hand-written HIP (gfx950) kernels for equivariant GNNs.

Drop-in for the reference package python/batmobile/__init__.py:11-70: the same
names, re-exported from the compiled extension, plus the autograd wrappers.

- Spherical harmonics (L_max up to 6), forward and backward
- 34-path Clebsch-Gordan tensor products (simple and channel-weighted)
- Fused SH + tensor product, with scatter-add into destination nodes
- CSR conversion and cell-list neighbor lists

There is no CPU fallback: importing this package without the built extension
raises ImportError.
"""

import torch  # noqa: F401  (must be imported first: loads the HIP runtime)

try:
    import _batteries  # noqa: F401
except ImportError as exc:  # pragma: no cover - exercised only without a build
    raise ImportError(
        "batmobile: the HIP extension `_batmobile` is not built or not on sys.path; "
        "run `python batmobile-evo_amd/build.py` (or __graft_entry__.build())"
    ) from exc

# Core operations (reference __init__.py:14-32)
from _batteries import (  # noqa: E402
    # Spherical harmonics
    spherical_harmonics,
    spherical_harmonics_inplace,
    spherical_harmonics_backward,
    # Tensor product
    tensor_product_simple,
    tensor_product,
    tensor_product_simple_backward,
    tensor_product_backward,
    # Path info
    get_tp_path_info,
    get_tp_num_paths,
    # Fused operations
    fused_sh_tp_simple,
    # Graph utilities
    edge_index_to_csr,
    fused_message_passing_simple,
    fused_message_passing,
)

# Extensions of this build (no single reference counterpart)
from _batteries import (  # noqa: E402
    spherical_harmonics_normalized,
    spherical_harmonics_normalized_backward,
    sh_tp_scatter,
    sh_tp_scatter_weighted,
    neighbor_list,
    spatial_order,
    mp_schedule,
    sh_tp_scatter_scheduled,
    gemm_f32,
    mace_reverse_edges,
    mace_forward,
    mace_backward,
)
from .graph import Graph  # noqa: E402
from .mace import MACEInteraction, MaceLayerFunction  # noqa: E402

# Autograd-compatible wrappers (reference __init__.py:35-44)
from .autograd import (  # noqa: E402
    SphericalHarmonicsFunction,
    TensorProductSimpleFunction,
    TensorProductFunction,
    spherical_harmonics as spherical_harmonics_autograd,
    tensor_product_simple as tensor_product_simple_autograd,
    tensor_product as tensor_product_autograd,
)

__version__ = "0.1.0"

__all__ = [
    # Core forward operations
    "spherical_harmonics",
    "spherical_harmonics_inplace",
    "tensor_product_simple",
    "tensor_product",
    "fused_sh_tp_simple",
    # Backward operations
    "spherical_harmonics_backward",
    "tensor_product_simple_backward",
    "tensor_product_backward",
    # Path info
    "get_tp_path_info",
    "get_tp_num_paths",
    # Graph utilities
    "edge_index_to_csr",
    "fused_message_passing_simple",
    "fused_message_passing",
    # Autograd classes
    "SphericalHarmonicsFunction",
    "TensorProductSimpleFunction",
    "TensorProductFunction",
    # Extensions
    "spherical_harmonics_normalized",
    "spherical_harmonics_normalized_backward",
    "sh_tp_scatter",
    "sh_tp_scatter_weighted",
    "neighbor_list",
    "spatial_order",
    "mp_schedule",
    "sh_tp_scatter_scheduled",
    "Graph",
    "gemm_f32",
    "mace_reverse_edges",
    "mace_forward",
    "mace_backward",
    "MACEInteraction",
    "MaceLayerFunction",
]
