"""Scheme lifecycle through the C ABI: DeleteScheme releases every device
buffer, and a scheme built afterwards works.  Kept in a module of its own:
each test builds and deletes its own scheme, so no module-scoped scheme of
another test file is replaced under it."""
import numpy as np
import pytest

from helpers import make_params, new_hip_scheme
from helrm_amd.backend import HipError

pytestmark = pytest.mark.gpu


def fresh(lib, level=3, scale_bits=30):
    pt = lib.Encode(np.linspace(-1, 1, 16).tolist(), level, 1 << scale_bits)
    ct = lib.Encrypt(pt)
    lib.DeletePlaintext(pt)
    return ct


def test_device_buffer_after_delete_scheme_refused(hip_lib):
    """DeleteScheme releases every device buffer, DeviceAlloc ones included:
    freeing one afterwards is refused, also when the new scheme's own buffers
    reuse its address.  (A pointer that a later DeviceAlloc returns again
    cannot be told from the stale one: pointers carry no owner, which the
    header states.)"""
    q, p = make_params(11, [40, 30, 30, 30], [41, 41])
    new_hip_scheme(hip_lib, 11, q, p, 30, 64, 9)
    stale = hip_lib.device_empty((2, 1 << 11))
    ptr = stale.ptr
    hip_lib.DeleteScheme()
    new_hip_scheme(hip_lib, 11, q, p, 30, 64, 9)
    with pytest.raises(HipError, match="DeviceAlloc"):
        hip_lib.DeviceFree(ptr)
    ct = fresh(hip_lib)
    dec = np.asarray(hip_lib.Decode(hip_lib.Decrypt(ct)))
    np.testing.assert_allclose(dec[:16], np.linspace(-1, 1, 16), atol=1e-4)
    hip_lib.DeleteScheme()


def test_measurement_probes(hip_lib):
    """The measurement entry points bench.py reports: the launch-latency probe
    (an empty dependent launch costs microseconds; a copy's rate is positive
    and below the HBM peak; out-of-range sizes are refused) and the VALU
    issue-rate probe."""
    q, p = make_params(16, [50, 50], [61])
    new_hip_scheme(hip_lib, 16, q, p, 40, 64, 3)
    r = hip_lib.launch_probe(4)
    assert 0.1 < r["empty_launch_us"] < 100
    assert r["copy_us"] > 0 and 0 < r["copy_TBs"] < 8.0
    with pytest.raises(HipError, match="LaunchProbe"):
        hip_lib.launch_probe(0)
    v = hip_lib.valu_peak()
    assert v["cus"] > 0 and v["wave_instr_per_s"] > 0
    hip_lib.DeleteScheme()
