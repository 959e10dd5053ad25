"""NTT launch sizes: launches over at most 96 limbs run the kernels with 8
words per thread, larger ones the 16-word kernels.  Both sides of the switch,
at N=2^16 (256 x 256 split) and N=2^13 (64 x 128), word for word against the
oracle's NTT, and the inverse back to the input."""
import numpy as np
import pytest

from helpers import assert_equal_u64, make_params
from oracle import oracle as O

pytestmark = pytest.mark.gpu

SIZES = [(1, 1), (1, 20), (4, 24), (97, 1), (5, 20)]
IDS = ["1-limb", "20-limbs", "96-limbs", "97-limbs", "100-limbs"]


@pytest.fixture(scope="module", params=[16, 13], ids=["N2^16", "N2^13"])
def ctx(request, hip_lib):
    logn = request.param
    q, p = make_params(logn, [50] * 24, [61])
    hip_lib.NewSchemeWithModuli(logn, q, p, 50, 64, 5)
    orc = O.Oracle(logn, q, p, h=64, seed=5)
    yield hip_lib, orc, q, logn
    orc.close()
    hip_lib.DeleteScheme()


@pytest.mark.parametrize("npoly,nrows", SIZES, ids=IDS)
def test_ntt_launch_sizes(ctx, npoly, nrows):
    lib, orc, q, logn = ctx
    rng = np.random.default_rng(100 * npoly + nrows + logn)
    N = 1 << logn
    x = np.stack([rng.integers(0, q[r], size=(npoly, N), dtype=np.uint64) for r in range(nrows)], axis=1)
    print(f"[ntt] N=2^{logn}: launch of {npoly * nrows} limbs", flush=True)
    dev = lib.device_upload(x)
    lib.NttDevice(dev.ptr, npoly, nrows, 1)
    lib.Synchronize()
    y = dev.download().reshape(npoly, nrows, N)
    for pi in range(npoly):
        for r in range(nrows):
            want = orc.ntt(x[pi, r].copy(), r)
            if not np.array_equal(y[pi, r], want):
                assert_equal_u64(y[pi, r], want, f"NTT {npoly}x{nrows} poly {pi} limb {r}")
    lib.NttDevice(dev.ptr, npoly, nrows, 0)
    lib.Synchronize()
    back = dev.download().reshape(npoly, nrows, N)
    dev.free()
    assert_equal_u64(back, x, f"iNTT(NTT(x)) {npoly}x{nrows}")
