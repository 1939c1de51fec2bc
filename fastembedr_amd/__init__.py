"""MI355X (gfx950) backend for the openTSNE-style t-SNE gradient loop of fastEmbedR.

The compute path is the HIP library behind include/fastembedr_hip.h; this
package holds its ctypes binding, a session wrapper, the host-side mirror of
the reference's ``opentsne_knn()``, ``transform_tsne()``, ``precompute_knn()``
and ``precompute_query_knn()`` entry points, and synthetic inputs for the
benchmark configurations.
"""

from ._lib import HipBackendError, HipBackendUnavailable, available, last_error
from .knn import KnnResult, exact_knn, exact_query_knn, precompute_knn, precompute_query_knn
from .opentsne import OpenTsneResult, opentsne_knn, opentsne_neighbor_policy, tsne_auto_parameters
from .session import TsneSession
from .transform import TransformResult, transform_tsne

__all__ = [
    "HipBackendError",
    "HipBackendUnavailable",
    "KnnResult",
    "OpenTsneResult",
    "TransformResult",
    "TsneSession",
    "available",
    "exact_knn",
    "exact_query_knn",
    "last_error",
    "opentsne_knn",
    "opentsne_neighbor_policy",
    "precompute_knn",
    "precompute_query_knn",
    "transform_tsne",
    "tsne_auto_parameters",
]
