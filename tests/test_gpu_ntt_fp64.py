"""The float64 transform of the limbs whose modulus is at most 2^50 + 2^29
(exact products by fused multiply-add; the other limbs keep the integer
butterflies) on inputs at the edges of its bound schedule: every word q - 1,
alternating 0 and q - 1, runs of q/2 and q/2 + 1, and uniform words.  Forward
and inverse, each against the oracle's transform word for word, at N=2^16
(256 x 256 split) and N=2^13 (64 x 128), in launches small enough for the
8-word kernels and large enough for the 16-word ones, with a 61-bit modulus
(integer path) in the same launch as the 50-bit ones."""
import numpy as np
import pytest

from helpers import assert_equal_u64, make_params
from oracle import oracle as O

pytestmark = pytest.mark.gpu

NROWS = 25  # 24 moduli of 50 bits, then the 61-bit one
PATTERNS = ["all_q-1", "alternating", "halves", "uniform"]


def pattern(name, qq, N, rng):
    i = np.arange(N, dtype=np.uint64)
    q1 = np.uint64(qq - 1)
    if name == "all_q-1":
        return np.full(N, q1, dtype=np.uint64)
    if name == "alternating":
        return np.where(i % 2 == 1, q1, np.uint64(0))
    if name == "halves":
        h = np.uint64(qq // 2)
        return np.where(i % 3 == 0, q1, np.where(i % 3 == 1, h, h + np.uint64(1)))
    return rng.integers(0, qq, size=N, dtype=np.uint64)


@pytest.fixture(scope="module", params=[16, 13], ids=["N2^16", "N2^13"])
def ctx(request, hip_lib):
    logn = request.param
    q, p = make_params(logn, [50] * 24, [61])
    hip_lib.NewSchemeWithModuli(logn, q, p, 50, 64, 5)
    orc = O.Oracle(logn, q, p, h=64, seed=5)
    assert max(q) <= (1 << 50) + (1 << 29) < p[0]
    yield hip_lib, orc, list(q) + list(p), logn
    orc.close()
    hip_lib.DeleteScheme()


@pytest.mark.parametrize("npoly", [1, 4], ids=["25-limbs", "100-limbs"])
def test_fp64_ntt_edges(ctx, npoly):
    lib, orc, mods, logn = ctx
    N = 1 << logn
    rng = np.random.default_rng(7 + npoly + logn)
    for name in PATTERNS:
        x = np.stack([np.stack([pattern(name, mods[r], N, rng) for r in range(NROWS)]) for _ in range(npoly)])
        print(f"[ntt-fp64] N=2^{logn} {npoly * NROWS} limbs, pattern {name}", flush=True)
        dev = lib.device_upload(x)
        lib.NttDevice(dev.ptr, npoly, NROWS, 1)
        lib.Synchronize()
        y = dev.download().reshape(npoly, NROWS, N)
        for pi in range(npoly):
            for r in range(NROWS):
                want = orc.ntt(x[pi, r].copy(), r)
                if not np.array_equal(y[pi, r], want):
                    assert_equal_u64(y[pi, r], want, f"NTT {name} poly {pi} limb {r}")
        # the inverse of the same edge words (not of the forward output)
        dev2 = lib.device_upload(x)
        lib.NttDevice(dev2.ptr, npoly, NROWS, 0)
        lib.Synchronize()
        z = dev2.download().reshape(npoly, NROWS, N)
        for pi in range(npoly):
            for r in range(NROWS):
                want = orc.intt(x[pi, r].copy(), r)
                if not np.array_equal(z[pi, r], want):
                    assert_equal_u64(z[pi, r], want, f"iNTT {name} poly {pi} limb {r}")
        dev.free()
        dev2.free()
