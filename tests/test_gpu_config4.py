"""Parity at BASELINE.json config 4 (4,000,000 x 50, 200 components with
Dirichlet(0.3) sizes, k = 90, perplexity 30), HIP path vs the CPU oracle on
identical inputs, through the C ABI: P (about 616M stored entries), then the
one-step gradient of both grids at checkpoints of a GPU trajectory through
the late phase (t = 300, 500, 749), where the FIt-SNE grid reaches its
largest box counts and FFT lengths.  At t = 749 the bilinear grid is also
compared with the fp64 evaluation of the same algorithm.  Gates as in
tests/test_gpu_config2.py: P within 1e-5 relative L2 with identical
structure; gradients within 1e-3 relative L2.
"""

import numpy as np
import pytest

from fastembedr_amd import _lib, synthetic
from tests.helpers import rel_l2
from tests.test_gpu_config2 import P_TOL, SCHED, THREADS, _say, _schedule, check_checkpoint

pytestmark = pytest.mark.gpu

LAGRANGE = _lib.REPULSION_LAGRANGE


def test_config4_p_and_late_checkpoint_gradients(hip, oracle_mod):
    spec = synthetic.CONFIGS[4]
    x, _ = synthetic.gaussian_mixture(spec, seed=1)
    n = x.shape[0]
    knn = hip.exact_knn(np.ascontiguousarray(x, np.float32), SCHED["k"], keep_device=True)
    host = knn.to_host()
    idx, dist = np.asarray(host.indices, np.int32), np.asarray(host.distances, np.float32)
    del host
    y0 = synthetic.pca_init(x)
    del x
    _say(f"case: config 4, n={n}: P and the gradients at t in (300, 500, 749)")
    P = oracle_mod.OracleP.build(idx, dist, SCHED["perplexity"], threads=THREADS)
    del idx, dist
    with hip.TsneSession(perplexity=SCHED["perplexity"], index_offset=1, n=n, k=SCHED["k"],
                         device_pointers=(knn.indices_ptr, knn.distances_ptr)) as s:
        rp, col, val = s.csr()
        rp0, col0, val0 = P.csr()
        np.testing.assert_array_equal(rp, rp0)
        np.testing.assert_array_equal(col, col0)
        err = rel_l2(val, val0)
        _say(f"  config 4: nnz {col.size}, P values relL2 {err:.2e}")
        assert err <= P_TOL
        del rp, col, val, rp0, col0, val0
        s.set_repulsion(LAGRANGE, 3, SCHED["min_intervals"], SCHED["ints_in_interval"])
        s.set_state(y0)
        s.center()
        t = 0
        for cp in (300, 500, 749):
            _schedule(s, n, cp, start=t)
            s.sync()
            t = cp
            check_checkpoint(s, P, t, "config 4", yardstick=cp == 749)
