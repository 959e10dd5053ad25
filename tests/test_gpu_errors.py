"""Error paths of the C ABI on a live scheme: every failure the host side can
detect comes back as -1 + GetLastError() (HipError in Python) instead of
aborting the process as a Lattigo panic does (orion/backend/lattigo/
minheap.go:67-75, lineartransform.go:85-87,106-109), and the library keeps
working afterwards.  Every check is made on the host, so no kernel is ever
handed an invalid handle or an unknown key."""
import numpy as np
import pytest

from helpers import make_params, new_hip_scheme
from helrm_amd.backend import HipError

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib(hip_lib):
    q, p = make_params(11, [40, 30, 30, 30], [41, 41])
    new_hip_scheme(hip_lib, 11, q, p, 30, 64, 3)
    yield hip_lib
    hip_lib.DeleteScheme()


def fresh(lib, level=3, scale_bits=30):
    pt = lib.Encode(np.linspace(-1, 1, 16).tolist(), level, 1 << scale_bits)
    ct = lib.Encrypt(pt)
    lib.DeletePlaintext(pt)
    return ct


def test_unknown_handles(lib):
    with pytest.raises(HipError, match="ciphertext not found"):
        lib.RotateNew(12345, 1)
    with pytest.raises(HipError, match="plaintext not found"):
        lib.Decode(777)
    with pytest.raises(HipError, match="linear transform not found"):
        lib.EvaluateLinearTransform(99, fresh(lib))


def test_scale_and_level_mismatch(lib):
    a = fresh(lib)
    b = fresh(lib, scale_bits=29)
    with pytest.raises(HipError, match="scales differ"):
        lib.AddCiphertext(a, b)
    c = fresh(lib, level=0)
    with pytest.raises(HipError, match="level 0"):
        lib.RescaleNew(c)
    with pytest.raises(HipError, match="invalid level"):
        lib.Encode([1.0], 9, 1 << 30)


def test_linear_transform_argument_checks(lib):
    S = 1 << 10
    with pytest.raises(HipError, match="len\\(diag_idxs\\) \\* slots"):
        lib.GenerateLinearTransform([0, 1], np.zeros(S, np.float32), 3, 2.0, "none")
    with pytest.raises(HipError, match="io_mode"):
        lib.GenerateLinearTransform([0], np.zeros(S, np.float32), 3, 2.0, "stream")
    # io_mode "load": no diagonals yet, so evaluation is refused until they are loaded
    tl = lib.GenerateLinearTransform([0], np.zeros(S, np.float32), 3, 2.0, "load")
    with pytest.raises(HipError, match="not loaded"):
        lib.EvaluateLinearTransform(tl, fresh(lib))
    lib.DeleteLinearTransform(tl)
    # rotation keys never generated for this transform: refused before any kernel runs
    tid = lib.GenerateLinearTransform([0, 7, 300], np.ones(3 * S, np.float32), 3, 2.0, "none")
    with pytest.raises(HipError, match="missing Galois key"):
        lib.EvaluateLinearTransform(tid, fresh(lib))
    for g in lib.GetLinearTransformRotationKeys(tid):
        lib.GenerateLinearTransformRotationKey(g)
    out = lib.EvaluateLinearTransform(tid, fresh(lib))
    assert lib.GetCiphertextLevel(out) == 3


def test_library_keeps_working_after_errors(lib):
    ct = fresh(lib)
    with pytest.raises(HipError):
        lib.AddCiphertext(ct, 4242)
    dec = np.asarray(lib.Decode(lib.Decrypt(ct)))
    np.testing.assert_allclose(dec[:16], np.linspace(-1, 1, 16), atol=1e-4)


def test_stream_selection(lib):
    """SetStream / JoinStream take stream 0 or 1; work given to stream 1 and
    joined is seen by stream 0 (a sum computed there, used on stream 0)."""
    with pytest.raises(HipError, match="stream index"):
        lib.SetStream(2)
    with pytest.raises(HipError, match="stream index"):
        lib.JoinStream(-1)
    ct = fresh(lib)
    lib.SetStream(1)
    lib.JoinStream(0)
    two = lib.AddCiphertextNew(ct, ct)
    lib.SetStream(0)
    lib.JoinStream(1)
    three = lib.AddCiphertextNew(two, ct)
    lib.Synchronize()
    dec = np.asarray(lib.Decode(lib.Decrypt(three)))
    np.testing.assert_allclose(dec[:16], 3 * np.linspace(-1, 1, 16), atol=1e-3)


def test_device_buffer_double_free_refused(lib):
    """A DeviceAlloc buffer freed twice is refused (it never enters the buffer
    cache twice, where it could be handed out to two owners)."""
    buf = lib.device_empty((4, 1 << 11))
    ptr = buf.ptr
    buf.free()
    with pytest.raises(HipError, match="freed twice"):
        lib.DeviceFree(ptr)
    a = lib.device_upload(np.arange(8, dtype=np.uint64))
    b = lib.device_upload(np.arange(8, 16, dtype=np.uint64))
    assert a.ptr != b.ptr
    np.testing.assert_array_equal(a.download(), np.arange(8))
    a.free(); b.free()
