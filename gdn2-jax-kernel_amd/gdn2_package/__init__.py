"""gdn2_package -- GDN-2 (Gated DeltaNet-2) chunked linear attention on MI355X.

Drop-in for the reference package's exports (tests/test_imports.py:5,12):
``gdn2_pallas_forward``, ``gdn2_pallas_forward_trainable`` and ``__version__``;
beyond them ``gdn2_pallas_forward_raw`` (input activations fused into the
forward), ``gdn2_pallas_forward_varlen`` (variable-length packed batches; trainable as
``gdn2_pallas_forward_varlen_trainable``) and
``gdn2_decode_step`` (one-token recurrent step on the state).  The reference's
per-kernel forward functions (``build_chunk_scores_pallas``, ``wy_solve_pallas``,
``recompute_wy_pallas``, ``gdn2_inter_chunk_combine(_with_state)``) are in
``gdn2_fwd``, and its per-kernel backward functions (``reverse_cumsum_bwd``,
``gdn2_dhu_backward``, ``dav_backward_pallas``, ``wy_dqkg_backward_pallas``,
``intra_backward_pallas``) in ``gdn2_bwd``, as in the reference.
Compute runs in libgdn2_hip.so (hand-written gfx950 HIP kernels, C ABI in
include/gdn2.h); torch supplies device memory and streams.
"""
from . import gdn2_bwd, gdn2_decode, gdn2_fwd, gdn2_pipeline
from ._lib import GDN2LibraryError
from .gdn2_decode import gdn2_decode_step
from .gdn2_fwd import (GDN2Error, GDN2ShapeError, gdn2_pallas_forward,
                       gdn2_pallas_forward_raw, gdn2_pallas_forward_varlen,
                       gdn2_pallas_forward_with_residuals)
from .gdn2_pipeline import (gdn2_pallas_forward_trainable,
                            gdn2_pallas_forward_varlen_trainable)

__version__ = "0.1.0"

__all__ = [
    "gdn2_pallas_forward", "gdn2_pallas_forward_trainable",
    "gdn2_pallas_forward_with_residuals", "gdn2_pallas_forward_raw",
    "gdn2_pallas_forward_varlen", "gdn2_pallas_forward_varlen_trainable", "gdn2_decode_step",
    "GDN2Error", "GDN2ShapeError",
    "GDN2LibraryError", "gdn2_fwd", "gdn2_bwd", "gdn2_pipeline", "__version__",
]
