"""MI355X (gfx950) backend for the openTSNE-style t-SNE gradient loop of fastEmbedR.

The compute path is the HIP library behind include/fastembedr_hip.h; this
package holds its ctypes binding, a session wrapper, the host-side mirror of
the reference's ``opentsne_knn()`` entry point, and synthetic inputs for the
benchmark configurations.
"""

from ._lib import HipBackendError, HipBackendUnavailable, available, last_error
from .opentsne import OpenTsneResult, opentsne_knn, opentsne_neighbor_policy, tsne_auto_parameters
from .session import TsneSession

__all__ = [
    "HipBackendError",
    "HipBackendUnavailable",
    "OpenTsneResult",
    "TsneSession",
    "available",
    "last_error",
    "opentsne_knn",
    "opentsne_neighbor_policy",
    "tsne_auto_parameters",
]
