"""Batched negacyclic NTT / inverse NTT and RNS multiply-accumulate on device
buffers, at the kernel-microbenchmark shape: N=2^16, 24 limbs of 50-bit
NTT-friendly primes, 64 polynomials, coefficients uniform mod each prime.
Outputs are bit-exact against the CPU NTT of the oracle on the same primes
and roots; the multiply-accumulate is checked against exact integer sums.
Device buffers come from the library's own allocator (DeviceAlloc)."""
import numpy as np
import pytest

from helpers import assert_equal_u64, make_params
from oracle import oracle as O

pytestmark = pytest.mark.gpu

LOGN, NLIMB, NPOLY = 16, 24, 64


@pytest.fixture(scope="module")
def ntt_ctx(hip_lib):
    q, p = make_params(LOGN, [50] * NLIMB, [61])
    hip_lib.NewSchemeWithModuli(LOGN, q, p, 50, 192, 5)
    orc = O.Oracle(LOGN, q, p, h=192, seed=5)
    rng = np.random.default_rng(11)
    N = 1 << LOGN
    x = np.stack([rng.integers(0, qq, size=(NPOLY, N), dtype=np.uint64) for qq in q], axis=1)
    print(f"[ntt] batch {x.shape}", flush=True)
    yield hip_lib, orc, q, x
    orc.close()
    hip_lib.DeleteScheme()


def test_batched_ntt_bitexact(ntt_ctx):
    lib, orc, q, x = ntt_ctx
    dev = lib.device_upload(x)
    lib.NttDevice(dev.ptr, NPOLY, NLIMB, 1)
    lib.Synchronize()
    y = dev.download()
    for pi in range(NPOLY):
        for r in range(NLIMB):
            want = orc.ntt(x[pi, r].copy(), r)
            if not np.array_equal(y[pi, r], want):
                assert_equal_u64(y[pi, r], want, f"NTT poly {pi} limb {r}")
    # inverse: back to the input word for word
    lib.NttDevice(dev.ptr, NPOLY, NLIMB, 0)
    lib.Synchronize()
    back = dev.download()
    dev.free()
    assert_equal_u64(back, x, "iNTT(NTT(x))")
    # and the inverse alone against the oracle on a few limbs
    for pi, r in [(0, 0), (NPOLY - 1, NLIMB - 1), (17, 5)]:
        assert_equal_u64(orc.intt(y[pi, r].copy(), r), x[pi, r], f"oracle iNTT poly {pi} limb {r}")


def test_rns_multiply_accumulate(ntt_ctx):
    lib, orc, q, x = ntt_ctx
    rng = np.random.default_rng(12)
    N = 1 << LOGN
    b = np.stack([rng.integers(0, qq, size=(NPOLY, N), dtype=np.uint64) for qq in q], axis=1)
    da, db = lib.device_upload(x), lib.device_upload(b)
    out = lib.device_empty((NLIMB, N))
    lib.MulAccDevice(da.ptr, db.ptr, out.ptr, NPOLY, NLIMB)
    lib.Synchronize()
    got = out.download()
    for buf in (da, db, out):
        buf.free()
    pos = rng.integers(0, N, 512)
    for r in range(NLIMB):
        qq = q[r]
        for c in pos:
            want = sum(int(x[pi, r, c]) * int(b[pi, r, c]) for pi in range(NPOLY)) % qq
            assert int(got[r, c]) == want, (r, c)
    assert (got < np.array(q, dtype=np.uint64)[:, None]).all()

