"""Serialization for Orion's io_mode save / load (key_generator.py:17-31,
lt_evaluator.py:133-161, 440-497): secret key, rotation keys and linear
transform diagonals leave the library as bytes and come back.

* the bytes hold what the layout says: the parsed words, out of Montgomery
  form, are the restatement's secret key / Galois key / diagonal plaintext;
* a loaded key or diagonal makes the library compute exactly what it computed
  before (bit-exact), in another scheme instance;
* malformed bytes are rejected with an error and leave the library usable.
Byte compatibility with Lattigo's own MarshalBinary is parity unpinned: no Go
toolchain or Lattigo module is available to produce reference bytes.
"""
import numpy as np
import pytest

from helpers import (assert_equal_u64, from_montgomery, make_params, new_hip_scheme, parse_wire_poly,
                     parse_wire_qp)
from oracle import oracle as O
from helrm_amd.backend import HipError

pytestmark = pytest.mark.gpu

LOGN, LOGQ, LOGP, LOGSCALE, H = 11, [40, 30, 30, 30], [41, 41], 30, 64


@pytest.fixture(scope="module")
def primes():
    return make_params(LOGN, LOGQ, LOGP)


def _u64(buf, off):
    return int(np.asarray(buf[off:off + 8], dtype=np.uint8).view("<u8")[0]), off + 8


def test_secret_key_bytes_and_reload(hip_lib, primes):
    q, p = primes
    N = 1 << LOGN
    print("[serialize] secret key", flush=True)
    new_hip_scheme(hip_lib, LOGN, q, p, LOGSCALE, H, 31)
    sk_coeffs = hip_lib.export_secret_key()
    data, ptr = hip_lib.SerializeSecretKey()
    hip_lib.FreeCArray(ptr)
    (Q, P), off = parse_wire_qp(data, 0, N)
    assert off == len(data) and Q.shape == (len(q), N) and P.shape == (len(p), N)
    orc = O.Oracle(LOGN, q, p, h=H, seed=31)
    try:
        np.testing.assert_array_equal(orc.secret_key(), sk_coeffs)
        mods = list(q) + list(p)
        words = from_montgomery(np.concatenate([Q, P]), mods)
        for i, m in enumerate(mods):
            want = orc.ntt(np.array([int(c) % m for c in sk_coeffs], dtype=np.uint64), i)
            np.testing.assert_array_equal(words[i], want)
        # a ciphertext of this scheme decrypts in another scheme that loaded the key
        vals = np.random.default_rng(3).uniform(-1, 1, N // 2).astype(np.float32)
        ct = hip_lib.Encrypt(hip_lib.Encode(vals.tolist(), len(q) - 1, 1 << LOGSCALE))
        raw = hip_lib.export_ciphertext(ct)
    finally:
        orc.close()
    hip_lib.DeleteScheme()
    new_hip_scheme(hip_lib, LOGN, q, p, LOGSCALE, H, 99)
    assert not np.array_equal(hip_lib.export_secret_key(), sk_coeffs)
    assert hip_lib.LoadSecretKey(data) == 0
    np.testing.assert_array_equal(hip_lib.export_secret_key(), sk_coeffs)
    ct2 = hip_lib.import_ciphertext(raw, len(q) - 1, float(1 << LOGSCALE))
    dec = np.asarray(hip_lib.Decode(hip_lib.Decrypt(ct2)))
    assert np.abs(dec - vals).max() < 1e-3
    with pytest.raises(HipError):
        hip_lib.LoadSecretKey(data[:-8])
    np.testing.assert_array_equal(hip_lib.export_secret_key(), sk_coeffs)
    hip_lib.DeleteScheme()


def test_rotation_key_bytes_and_reload(hip_lib, primes):
    q, p = primes
    N, L, K = 1 << LOGN, len(q), len(p)
    dnum = (L + K - 1) // K
    print("[serialize] rotation key", flush=True)
    new_hip_scheme(hip_lib, LOGN, q, p, LOGSCALE, H, 41)
    orc = O.Oracle(LOGN, q, p, h=H, seed=41)
    try:
        g = orc.galois_element(5)
        data, ptr = hip_lib.GenerateAndSerializeRotationKey(g)
        hip_lib.FreeCArray(ptr)
        ge, off = _u64(data, 0)
        nth, off = _u64(data, off)
        b2, off = _u64(data, off)
        nd, off = _u64(data, off)
        assert (ge, nth, b2, nd) == (g, 2 * N, 0, dnum)
        want = orc.galois_key(g)
        mods = list(q) + list(p)
        for d in range(dnum):
            one, off = _u64(data, off)
            two, off = _u64(data, off)
            assert (one, two) == (1, 2)
            for part in range(2):
                (Q, P), off = parse_wire_qp(data, off, N)
                got = from_montgomery(np.concatenate([Q, P]), mods)
                assert_equal_u64(got, want[d, part], f"key digit {d} part {part}")
        assert off == len(data)
    finally:
        orc.close()
    hip_lib.DeleteScheme()
    # load into a fresh instance: the key the library then holds is the same key
    new_hip_scheme(hip_lib, LOGN, q, p, LOGSCALE, H, 41)
    assert hip_lib.LoadRotationKey(data, g) == 0
    orc = O.Oracle(LOGN, q, p, h=H, seed=41)
    try:
        assert_equal_u64(hip_lib.export_galois_key(g), orc.galois_key(g), "loaded rotation key")
    finally:
        orc.close()
    with pytest.raises(HipError):
        hip_lib.LoadRotationKey(data, g + 2)
    bad = data.copy()
    bad[64:72] = 0xFF  # the first coefficient of digit 0, b, limb q_0: >= q
    with pytest.raises(HipError):
        hip_lib.LoadRotationKey(bad, g)
    hip_lib.DeleteScheme()


def test_diagonal_save_load_round_trip(hip_lib, primes):
    """lt_evaluator save -> remove -> load (lt_evaluator.py:464-497): the
    transform evaluates bit-exactly as before once every diagonal is back;
    the serialized words are the restatement's diagonal plaintexts."""
    q, p = primes
    N, S, L, K = 1 << LOGN, 1 << (LOGN - 1), len(q), len(p)
    level = L - 1
    print("[serialize] diagonals", flush=True)
    new_hip_scheme(hip_lib, LOGN, q, p, LOGSCALE, H, 51)
    rng = np.random.default_rng(8)
    idx = [0, 1, 2, 5, 17, 40, S - 3]
    data = rng.uniform(-1, 1, (len(idx), S)).astype(np.float32)
    tid = hip_lib.GenerateLinearTransform(idx, data.reshape(-1).tolist(), level, 2.0, "none")
    for ge in hip_lib.GetLinearTransformRotationKeys(tid):
        hip_lib.GenerateLinearTransformRotationKey(ge)
    vals = rng.uniform(-1, 1, S).astype(np.float32)
    ct = hip_lib.Encrypt(hip_lib.Encode(vals.tolist(), level, 1 << LOGSCALE))
    out1 = hip_lib.export_ciphertext(hip_lib.EvaluateLinearTransform(tid, ct))
    orc = O.Oracle(LOGN, q, p, h=H, seed=51)
    mods = list(q[:level + 1]) + list(p)
    blobs = {}
    try:
        t = orc.lt_new(idx, data, level, 2.0)
        for d in idx:
            blob, ptr = hip_lib.SerializeDiagonal(tid, d)
            hip_lib.FreeCArray(ptr)
            (Q, P), off = parse_wire_qp(blob, 0, N)
            assert off == len(blob) and Q.shape[0] == level + 1 and P.shape[0] == K
            want = orc.lt_plaintext(t, d % S)
            assert_equal_u64(from_montgomery(np.concatenate([Q, P]), mods), want, f"diagonal {d}")
            blobs[d] = blob
    finally:
        orc.close()
    with pytest.raises(HipError):
        hip_lib.EvaluateLinearTransform(tid, ct)
    assert hip_lib.RemovePlaintextDiagonals(tid) == 0
    order = list(blobs)
    rng.shuffle(order)
    for d in order[:-1]:
        assert hip_lib.LoadPlaintextDiagonal(blobs[d], tid, d % S) == 0
    with pytest.raises(HipError):
        hip_lib.EvaluateLinearTransform(tid, ct)
    with pytest.raises(HipError):
        hip_lib.LoadPlaintextDiagonal(blobs[order[-1]][:100], tid, order[-1] % S)
    d = order[-1]
    assert hip_lib.LoadPlaintextDiagonal(blobs[d], tid, d % S) == 0
    out2 = hip_lib.export_ciphertext(hip_lib.EvaluateLinearTransform(tid, ct))
    assert_equal_u64(out2, out1, "transform after save / remove / load")
    hip_lib.DeleteScheme()


def _wire_poly(rows):
    """ring.Poly in the library's wire format (the layout parse_wire_poly reads)."""
    parts = [np.array([rows.shape[0]], dtype="<u8").tobytes()]
    for r in rows:
        parts.append(np.array([rows.shape[1]], dtype="<u8").tobytes())
        parts.append(np.ascontiguousarray(r, dtype="<u8").tobytes())
    return b"".join(parts)


def test_packed_diagonal_storage_edges(hip_lib):
    """A dense 16-baby transform keeps its diagonals packed on the device
    (rows of moduli below 2^52 as 52-bit fields, the 60- and 61-bit rows as
    plain words).  Diagonals made of edge words -- every word q - 1, zeros,
    alternating 0 / q - 1, single high bits, a ramp -- are loaded, then read
    back through serialization and export byte for byte, and the transform
    still evaluates bit-exactly as before once its own diagonals are back."""
    logn = 11
    N, S = 1 << logn, 1 << (logn - 1)
    q, p = make_params(logn, [60, 50, 50, 50, 50], [61])
    L, K = len(q), len(p)
    level = L - 1
    mods = list(q) + list(p)
    assert max(q[1:]) < (1 << 52) <= q[0] and p[0] >= (1 << 52)
    print("[serialize] packed diagonal edges", flush=True)
    new_hip_scheme(hip_lib, logn, q, p, 40, 64, 17)
    rng = np.random.default_rng(21)
    idx = list(range(256))
    data = rng.uniform(-1, 1, (len(idx), S)).astype(np.float32)
    tid = hip_lib.GenerateLinearTransform(idx, data.reshape(-1).tolist(), level, 2.0, "none")
    info = hip_lib.lt_info(tid)
    assert info["baby"] == 16 and info["giant"] * 16 == info["plaintexts"], info  # the packed (dense 16-baby) layout
    for ge in hip_lib.GetLinearTransformRotationKeys(tid):
        hip_lib.GenerateLinearTransformRotationKey(ge)
    vals = rng.uniform(-1, 1, S).astype(np.float32)
    ct = hip_lib.Encrypt(hip_lib.Encode(vals.tolist(), level, 1 << 40))
    out1 = hip_lib.export_ciphertext(hip_lib.EvaluateLinearTransform(tid, ct))
    own = {}
    for d in (0, 7, 255):
        blob, ptr = hip_lib.SerializeDiagonal(tid, d)
        hip_lib.FreeCArray(ptr)
        own[d] = bytes(blob)
    i = np.arange(N, dtype=np.uint64)
    patterns = {
        "all_q-1": lambda qq: np.full(N, qq - 1, dtype=np.uint64),
        "zeros": lambda qq: np.zeros(N, dtype=np.uint64),
        "alternating": lambda qq: np.where(i % 2 == 1, np.uint64(qq - 1), np.uint64(0)),
        "high_bits": lambda qq: np.uint64(1) << (i % np.uint64(int(qq).bit_length() - 1)),
        "ramp": lambda qq: (i * np.uint64(0x9E3779B97F4A7C15 % int(qq))) % np.uint64(qq),
    }
    for name, f in patterns.items():
        rows = np.stack([f(int(m)) for m in mods[:level + 1] + list(p)])
        assert all((rows[r] < np.uint64(mods[r] if r <= level else p[r - level - 1])).all() for r in range(rows.shape[0]))
        blob = _wire_poly(rows[:level + 1]) + _wire_poly(rows[level + 1:])
        for d in (0, 7, 255):
            assert hip_lib.LoadPlaintextDiagonal(blob, tid, d) == 0
            got = hip_lib.export_lt_diagonal(tid, d, level)
            assert_equal_u64(np.asarray(got).reshape(-1, N), from_montgomery(rows, mods[:level + 1] + list(p)),
                             f"export {name} diagonal {d}")
            back, ptr = hip_lib.SerializeDiagonal(tid, d)
            hip_lib.FreeCArray(ptr)
            assert bytes(back) == blob, f"{name}: diagonal {d} bytes after the packed round trip"
    for d in (0, 7, 255):
        assert hip_lib.LoadPlaintextDiagonal(own[d], tid, d) == 0
    out2 = hip_lib.export_ciphertext(hip_lib.EvaluateLinearTransform(tid, ct))
    assert_equal_u64(out2, out1, "transform with its own diagonals back")
    hip_lib.DeleteScheme()
