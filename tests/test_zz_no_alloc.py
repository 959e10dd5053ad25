"""RotateInto, the entry point that allocates nothing (its key switch runs in
a static device scratch array), against RotateNew through the C ABI: the
same words on two calls in a row, the second with a smaller input (the
library's buffer cache raises if anything inside RotateInto asks it for
memory); sizes beyond the
scratch array are refused with an error and leave the library usable."""
import numpy as np
import pytest

from helpers import assert_equal_u64, make_params, new_hip_scheme
from helrm_amd.backend import HipError

pytestmark = pytest.mark.gpu


def encrypt_at(lib, rng, level, logscale, counter):
    vals = rng.uniform(-1, 1, 1 << 15).astype(np.float32)
    lib.SetEncryptionCounter(counter)
    return lib.Encrypt(lib.Encode(vals.tolist(), level, 1 << logscale))


def test_rotate_into_matches_rotate_new(hip_lib):
    lib = hip_lib
    logq, logp, logscale = [60] + [50] * 23, [61] * 8, 50
    q, p = make_params(16, logq, logp)
    print("[no-alloc] N=2^16, 24 Q + 8 P limbs", flush=True)
    new_hip_scheme(lib, 16, q, p, logscale, 192, 41)
    rng = np.random.default_rng(2)
    k = 1 << 10
    big = encrypt_at(lib, rng, 22, logscale, 0)      # the PCMM's fold level
    small = encrypt_at(lib, rng, 9, logscale, 1)
    ref_big = lib.RotateNew(big, k)                  # generates the key
    ref_small = lib.RotateNew(small, k)
    out = lib.AddCiphertextNew(big, big)             # any ciphertext with room for level 22
    # (inside RotateInto the library's buffer cache raises on any allocation)
    for src, ref, level in ((big, ref_big, 22), (small, ref_small, 9)):
        print(f"[no-alloc] RotateInto at level {level}", flush=True)
        assert lib.RotateInto(src, k, out) == out
        assert lib.GetCiphertextLevel(out) == level
        assert lib.GetCiphertextScaleDouble(out) == lib.GetCiphertextScaleDouble(ref)
        assert_equal_u64(lib.export_ciphertext(out), lib.export_ciphertext(ref), f"RotateInto at level {level}")
    with pytest.raises(HipError, match="no rotation key"):
        lib.RotateInto(big, 3, out)
    with pytest.raises(HipError, match="another ciphertext"):
        lib.RotateInto(big, k, big)
    lib.DeleteScheme()


def test_rotate_into_two_streams(hip_lib):
    """Calls on the scheme's two streams queued back to back: the second
    waits for the first one's key switch before it uses the scratch array,
    so both outputs are RotateNew's words."""
    lib = hip_lib
    logq, logp, logscale = [60] + [50] * 23, [61] * 8, 50
    q, p = make_params(16, logq, logp)
    print("[no-alloc] two streams, N=2^16, 24 Q + 8 P limbs", flush=True)
    new_hip_scheme(lib, 16, q, p, logscale, 192, 47)
    rng = np.random.default_rng(4)
    k = 1 << 9
    a = encrypt_at(lib, rng, 22, logscale, 0)
    b = encrypt_at(lib, rng, 20, logscale, 1)
    ref_a, ref_b = lib.RotateNew(a, k), lib.RotateNew(b, k)
    out_a, out_b = lib.AddCiphertextNew(a, a), lib.AddCiphertextNew(a, a)
    lib.Synchronize()
    for rep in range(3):
        lib.SetStream(0)
        assert lib.RotateInto(a, k, out_a) == out_a
        lib.SetStream(1)
        assert lib.RotateInto(b, k, out_b) == out_b
        lib.SetStream(0)
        assert lib.RotateInto(b, k, out_a) == out_a
        lib.JoinStream(1)
        lib.Synchronize()
        assert_equal_u64(lib.export_ciphertext(out_b), lib.export_ciphertext(ref_b), f"stream 1 RotateInto, round {rep}")
        assert_equal_u64(lib.export_ciphertext(out_a), lib.export_ciphertext(ref_b), f"stream 0 RotateInto, round {rep}")
        lib.SetStream(1)
        assert lib.RotateInto(a, k, out_b) == out_b
        lib.SetStream(0)
        lib.JoinStream(1)
        lib.Synchronize()
        assert_equal_u64(lib.export_ciphertext(out_b), lib.export_ciphertext(ref_a), f"stream 1 RotateInto of a, round {rep}")
    lib.DeleteScheme()


def test_rotate_into_refuses_oversize(hip_lib):
    lib = hip_lib
    logq, logp, logscale = [60] + [50] * 29, [61] * 8, 50
    q, p = make_params(16, logq, logp)
    print("[no-alloc] N=2^16, 30 Q + 8 P limbs", flush=True)
    new_hip_scheme(lib, 16, q, p, logscale, 192, 43)
    rng = np.random.default_rng(3)
    top = encrypt_at(lib, rng, 29, logscale, 0)
    low = encrypt_at(lib, rng, 12, logscale, 1)
    lib.AddRotationKey(1)
    out = lib.AddCiphertextNew(top, top)
    with pytest.raises(HipError, match="bytes of scratch"):
        lib.RotateInto(top, 1, out)
    # the library stays usable and a level that fits still works
    assert lib.RotateInto(low, 1, out) == out
    assert_equal_u64(lib.export_ciphertext(out), lib.export_ciphertext(lib.RotateNew(low, 1)), "RotateInto after a refusal")
    lib.DeleteScheme()
