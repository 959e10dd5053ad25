"""Pins of the CPU restatement (oracle/) against what the mathematics fixes,
independently of the oracle's own formulas: schoolbook negacyclic products,
direct evaluation at the roots, exact big-integer CRT, the canonical
embedding evaluated directly, decryption noise bounds and the closed-form
linear transforms of the reference's tests
(tests/oracle/test_linear_transform.py:10-199)."""
import math

import numpy as np
import pytest

from oracle import oracle as O

# ---------------------------------------------------------------- helpers


def mr_prime(n):
    """Miller-Rabin with the first 12 prime bases, written independently."""
    if n < 2:
        return False
    small = [2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37]
    for p in small:
        if n % p == 0:
            return n == p
    d, s = n - 1, 0
    while d % 2 == 0:
        d //= 2
        s += 1
    for a in small:
        x = pow(a, d, n)
        if x in (1, n - 1):
            continue
        for _ in range(s - 1):
            x = x * x % n
            if x == n - 1:
                break
        else:
            return False
    return True


def brv(x, bits):
    return int(format(x, f"0{bits}b")[::-1], 2) if bits else 0


def primitive_2n_root(q, N):
    """psi with psi^N = -1, from the smallest generator of Z_q^* (sympy-free)."""
    n = q - 1
    fac, m, f = [], n, 2
    while f * f <= m:
        if m % f == 0:
            fac.append(f)
            while m % f == 0:
                m //= f
        f += 1
    if m > 1:
        fac.append(m)
    g = 2
    while any(pow(g, n // p, q) == 1 for p in fac):
        g += 1
    return pow(g, n // (2 * N), q)


@pytest.fixture(scope="module")
def tiny():
    """N=16, Q=[30,30,30], P=[31] (primes 1 mod 32)."""
    q, p = O.gen_primes(4, [30, 30, 30], [31])
    o = O.Oracle(4, q, p, h=4, seed=3)
    yield o
    o.close()


@pytest.fixture(scope="module")
def small():
    """N=64, Q=[40,30,30,30], P=[41,41]."""
    q, p = O.gen_primes(6, [40, 30, 30, 30], [41, 41])
    o = O.Oracle(6, q, p, h=16, seed=9)
    yield o
    o.close()


# ---------------------------------------------------------------- primes


@pytest.mark.parametrize("logN,logq,logp", [(13, [60, 40, 40, 40, 40], [61]), (16, [60] + [50] * 23, [61] * 8), (4, [30, 30], [31])])
def test_primes(logN, logq, logp):
    q, p = O.gen_primes(logN, logq, logp)
    allm = q + p
    assert len(set(allm)) == len(allm)
    for m, b in zip(allm, logq + logp):
        assert mr_prime(m)
        assert (m - 1) % (2 << logN) == 0
        assert abs(m.bit_length() - (b + 1)) <= 1
    # 61-bit primes come from below 2^61 (downstream only)
    for m, b in zip(allm, logq + logp):
        if b == 61:
            assert m < (1 << 61)
    # alternation for the 50-bit group: first above 2^50, second below
    if logq.count(50) >= 2:
        fifty = [m for m, b in zip(q, logq) if b == 50]
        assert fifty[0] > (1 << 50) > fifty[1]


# ---------------------------------------------------------------- NTT


def test_ntt_direct_evaluation(tiny):
    N = tiny.N
    for mi, m in enumerate(tiny.q + tiny.p):
        rng = np.random.default_rng(mi)
        a = [int(x) for x in rng.integers(0, m, N)]
        A = tiny.ntt(np.array(a, dtype=np.uint64), mi)
        psi = primitive_2n_root(m, N)
        for j in range(N):
            e = 2 * brv(j, 4) + 1
            want = sum(a[i] * pow(psi, e * i, m) for i in range(N)) % m
            assert int(A[j]) == want


def test_ntt_schoolbook_and_inverse(small):
    N = small.N
    for mi, m in enumerate(small.q + small.p):
        rng = np.random.default_rng(100 + mi)
        a = [int(x) for x in rng.integers(0, m, N)]
        b = [int(x) for x in rng.integers(0, m, N)]
        c = [0] * N
        for i in range(N):
            for j in range(N):
                k = i + j
                if k < N:
                    c[k] = (c[k] + a[i] * b[j]) % m
                else:
                    c[k - N] = (c[k - N] - a[i] * b[j]) % m
        A = small.ntt(np.array(a, dtype=np.uint64), mi)
        B = small.ntt(np.array(b, dtype=np.uint64), mi)
        C = np.array([(int(x) * int(y)) % m for x, y in zip(A, B)], dtype=np.uint64)
        assert [int(v) for v in small.intt(C, mi)] == c
        assert [int(v) for v in small.intt(A, mi)] == a


def test_automorphism_index_is_x_to_xg(small):
    """NTT(sigma_g(a)) = NTT(a)[idx] with sigma_g(a)(X) = a(X^g)."""
    N = small.N
    m = small.q[0]
    rng = np.random.default_rng(5)
    a = [int(x) for x in rng.integers(0, m, N)]
    for k in (1, 3, -1):
        g = small.galois_element(k)
        assert g == pow(5, k % (2 * N), 2 * N)
        s = [0] * N
        for i in range(N):
            t = (i * g) % (2 * N)
            if t < N:
                s[t] = (s[t] + a[i]) % m
            else:
                s[t - N] = (s[t - N] - a[i]) % m
        idx = small.automorphism_index(g)
        A = small.ntt(np.array(a, dtype=np.uint64), 0)
        S = small.ntt(np.array(s, dtype=np.uint64), 0)
        np.testing.assert_array_equal(S, A[idx])


# ---------------------------------------------------------------- RNS


def test_basis_extension_exact_crt(small):
    """For x in [0, S), extend(x mod s_i) = x mod t_k (exact CRT, the float
    overflow count is exact away from integer boundaries)."""
    src, dst = [0, 1, 2], [3, 4, 5]
    mods = small.q + small.p
    S = math.prod(mods[i] for i in src)
    rng = np.random.default_rng(7)
    xs = [int(rng.integers(0, 2 ** 62)) * int(rng.integers(0, 2 ** 62)) * int(rng.integers(1, 2 ** 40)) % S for _ in range(small.N)]
    xs[0], xs[1] = 0, S - 1
    inp = np.array([[x % mods[i] for x in xs] for i in src], dtype=np.uint64)
    out = small.basis_extend(src, dst, inp)
    for r, k in enumerate(dst):
        got = [int(v) for v in out[r]]
        assert got[0] == 0
        # x = S-1: sum y_i/s_i = v + (S-1)/S rounds up in float64, so the
        # overflow count is one too large and the extension returns x - S.
        # This is the float-v method's defined behaviour (not an exact CRT).
        assert got[1] == (xs[1] - S) % mods[k]
        assert got[2:] == [x % mods[k] for x in xs[2:]]


def _crt(residues, mods):
    M = math.prod(mods)
    x = 0
    for r, m in zip(residues, mods):
        Mi = M // m
        x += int(r) * Mi * pow(Mi, -1, m)
    return x % M


def test_mod_down_is_floor_division_by_P(small):
    level = small.L - 1
    rng = np.random.default_rng(11)
    mods = small.q + small.p
    qp = np.array([rng.integers(0, m, small.N) for m in mods], dtype=np.uint64)
    P = math.prod(small.p)
    ntt = np.stack([small.ntt(qp[i], i) for i in range(len(mods))])
    out = small.mod_down(ntt, level)
    coeff = small.to_coeff(out, level)
    for x in range(small.N):
        X = _crt([qp[i][x] for i in range(len(mods))], mods)
        want = (X - (X % P)) // P
        for i, q in enumerate(small.q):
            assert int(coeff[i][x]) == want % q


def test_rescale_is_rounded_division(small):
    level = small.L - 1
    rng = np.random.default_rng(13)
    ct = np.stack([np.array([rng.integers(0, q, small.N) for q in small.q], dtype=np.uint64) for _ in range(2)])
    ntt = np.stack([np.stack([small.ntt(ct[p][i], i) for i in range(small.L)]) for p in range(2)])
    out = small.rescale(ntt, level)
    ql = small.q[level]
    for p in range(2):
        coeff = small.to_coeff(out[p], level - 1)
        for x in range(small.N):
            X = _crt([ct[p][i][x] for i in range(small.L)], small.q)
            u = ((X % ql) + ql // 2) % ql - ql // 2   # representative in [-ql/2, ql/2)
            want = (X - u) // ql
            for i in range(level):
                assert int(coeff[i][x]) == want % small.q[i]


# ---------------------------------------------------------------- encoder


def test_encoding_is_canonical_embedding(small):
    """decode(poly) = poly evaluated at zeta^(5^j) / scale, zeta = exp(i pi / N)."""
    N, S = small.N, small.slots
    rng = np.random.default_rng(17)
    vals = rng.uniform(-1, 1, S).astype(np.float32)
    scale = 2.0 ** 30
    pt = small.encode(vals, 0, scale)
    coeff = small.to_coeff(pt, 0)[0]
    q = small.q[0]
    c = np.array([int(v) - q if int(v) > q // 2 else int(v) for v in coeff], dtype=np.float64)
    for j in range(S):
        z = np.exp(1j * np.pi * pow(5, j, 2 * N) / N)
        slot = np.sum(c * z ** np.arange(N)) / scale
        assert abs(slot.real - vals[j]) < 1e-6 and abs(slot.imag) < 1e-6
    np.testing.assert_allclose(small.decode_f64(pt, 0, scale), vals, atol=1e-6)


def test_complex_encoding_is_canonical_embedding(small):
    """EncodeComplex: the polynomial takes the complex slot value z_j at
    zeta^(5^j) (and its conjugate at zeta^(-5^j)); DecodeComplex returns it."""
    N, S = small.N, small.slots
    rng = np.random.default_rng(18)
    z = (rng.uniform(-1, 1, S) + 1j * rng.uniform(-1, 1, S)).astype(np.complex64)
    scale = 2.0 ** 30
    pt = small.encode_complex(z, 0, scale)
    coeff = small.to_coeff(pt, 0)[0]
    q = small.q[0]
    c = np.array([int(v) - q if int(v) > q // 2 else int(v) for v in coeff], dtype=np.float64)
    for j in range(S):
        r = np.exp(1j * np.pi * pow(5, j, 2 * N) / N)
        slot = np.sum(c * r ** np.arange(N)) / scale
        assert abs(slot - z[j]) < 1e-6
        assert abs(np.sum(c * np.conj(r) ** np.arange(N)) / scale - np.conj(z[j])) < 1e-6
    np.testing.assert_allclose(small.decode_complex(pt, 0, scale), z, atol=1e-6)
    # a purely real input encodes exactly as Encode does
    zr = z.real.astype(np.float32)
    np.testing.assert_array_equal(small.encode_complex(zr.astype(np.complex64), 2, scale), small.encode(zr, 2, scale))


def test_mul_i_is_the_monomial_x_to_the_n_over_2(small):
    """Multiplication by i is multiplication by X^(N/2): decrypted, every
    coefficient moves N/2 places up, negated when it wraps (X^N = -1)."""
    level = small.L - 1
    N = small.N
    vals = np.random.default_rng(21).uniform(-1, 1, small.slots).astype(np.float32)
    ct = small.encrypt(small.encode(vals, level, 2.0 ** 30), level, 2)
    got = small.to_coeff(small.decrypt(small.mul_i(ct, level), level), level)
    base = small.to_coeff(small.decrypt(ct, level), level)
    for i, q in enumerate(small.q[:level + 1]):
        want = np.concatenate([(q - base[i][N // 2:]) % q, base[i][:N // 2]]).astype(np.uint64)
        np.testing.assert_array_equal(got[i], want)
    dec = small.decode_complex(small.decrypt(small.mul_i(ct, level), level), level, 2.0 ** 30)
    np.testing.assert_allclose(dec, 1j * vals, atol=1e-5)


def test_conjugation_conjugates_every_slot(mid):
    """The automorphism X -> X^(2N-1) (Lattigo Conjugate) decrypts to the
    complex conjugate of every slot."""
    level = mid.L - 1
    rng = np.random.default_rng(33)
    z = (rng.uniform(-1, 1, mid.slots) + 1j * rng.uniform(-1, 1, mid.slots)).astype(np.complex64)
    scale = 2.0 ** 30
    ct = mid.encrypt(mid.encode_complex(z, level, scale), level, 4)
    out = mid.automorphism(ct, level, 2 * mid.N - 1)
    np.testing.assert_allclose(mid.decode_complex(mid.decrypt(out, level), level, scale), np.conj(z), atol=1e-4)


# ---------------------------------------------------------------- encryption, keys


def test_encrypt_decrypt_noise(small):
    level = small.L - 1
    rng = np.random.default_rng(19)
    vals = rng.uniform(-1, 1, small.slots).astype(np.float32)
    scale = 2.0 ** 30
    pt = small.encode(vals, level, scale)
    ct = small.encrypt(pt, level, 0)
    d = small.decrypt(ct, level)
    diff = [(_crt(small.to_coeff(d, level)[:, x], small.q[:level + 1]) - _crt(small.to_coeff(pt, level)[:, x], small.q[:level + 1])) for x in range(small.N)]
    Q = math.prod(small.q[:level + 1])
    diff = [v - Q if v > Q // 2 else v for v in (dv % Q for dv in diff)]
    assert max(abs(v) for v in diff) < 64
    np.testing.assert_allclose(small.decode_f64(d, level, scale), vals, atol=1e-6)


def test_seeded_encryption(small):
    """Seeded secret-key encryption: b + a*s - m is a small error (exactly, by
    CRT), `a` is the seed's expansion alone -- the same for any message,
    encryption index and level (a server expands it at the ciphertext's own
    level), different for another seed -- and its words spread over [0, q)."""
    level = small.L - 1
    rng = np.random.default_rng(23)
    vals = rng.uniform(-1, 1, small.slots).astype(np.float32)
    scale = 2.0 ** 30
    pt = small.encode(vals, level, scale)
    ct = small.encrypt_seeded(pt, level, 0x5EED, 4)
    d = small.decrypt(ct, level)
    diff = [(_crt(small.to_coeff(d, level)[:, x], small.q[:level + 1]) - _crt(small.to_coeff(pt, level)[:, x], small.q[:level + 1])) for x in range(small.N)]
    Q = math.prod(small.q[:level + 1])
    diff = [v - Q if v > Q // 2 else v for v in (dv % Q for dv in diff)]
    assert 0 < max(abs(v) for v in diff) < 64
    a = ct[1]
    np.testing.assert_array_equal(a, small.expand_seeded_a(level, 0x5EED))
    other = small.encrypt_seeded(small.encode(-vals, level, scale), level, 0x5EED, 9)
    np.testing.assert_array_equal(other[1], a)
    np.testing.assert_array_equal(small.expand_seeded_a(1, 0x5EED), a[:2])
    assert not np.array_equal(small.expand_seeded_a(level, 0x5EEE), a)
    for i in range(level + 1):
        q = small.q[i]
        assert a[i].max() < q and a[i].mean() / q == pytest.approx(0.5, abs=0.15)
    np.testing.assert_allclose(small.decode_f64(d, level, scale), vals, atol=1e-6)


def test_galois_key_relation(small):
    """b_d + a_d * s' = e_d + P * s on the digit's limbs (s' = sigma_{g^-1}(s))."""
    g = small.galois_element(1)
    key = small.galois_key(g)
    s = small.secret_key()
    N, mods = small.N, small.q + small.p
    ginv = pow(g, -1, 2 * N)
    so = [0] * N
    for i in range(N):
        t = (i * ginv) % (2 * N)
        if t < N:
            so[t] += int(s[i])
        else:
            so[t - N] -= int(s[i])
    P = math.prod(small.p)
    for d in range(small.dnum):
        for i, m in enumerate(mods):
            b = small.intt(key[d][0][i], i)
            a = small.intt(key[d][1][i], i)
            # e = b + a*s' - [P*s] (negacyclic products in Python)
            prod = [0] * N
            for x in range(N):
                if int(a[x]) == 0:
                    continue
                for y in range(N):
                    if so[y] == 0:
                        continue
                    k = x + y
                    v = int(a[x]) * so[y]
                    if k < N:
                        prod[k] += v
                    else:
                        prod[k - N] -= v
            own = i < small.L and d * small.K <= i < (d + 1) * small.K
            e = [(int(b[x]) + prod[x] - (P * int(s[x]) if own else 0)) % m for x in range(N)]
            e = [v - m if v > m // 2 else v for v in e]
            assert max(abs(v) for v in e) <= 21


# ---------------------------------------------------------------- evaluator (closed forms)


@pytest.fixture(scope="module")
def mid():
    q, p = O.gen_primes(11, [45, 35, 35, 35], [46, 46])
    o = O.Oracle(11, q, p, h=64, seed=21)
    yield o
    o.close()


def _enc(o, vals, level, logscale, k):
    return o.encrypt(o.encode(vals, level, float(2 ** logscale)), level, k)


def test_rotation_closed_form(mid):
    level = mid.L - 1
    vals = np.arange(1, mid.slots + 1, dtype=np.float32) / mid.slots
    ct = _enc(mid, vals, level, 35, 1)
    for k in (1, 3, -2, mid.slots // 2):
        r = mid.rotate(ct, level, k)
        out = mid.decode_f64(mid.decrypt(r, level), level, 2.0 ** 35)
        np.testing.assert_allclose(out, np.roll(vals, -k), atol=1e-4)


@pytest.mark.parametrize("case", ["identity", "scale", "shift", "two", "bsgs", "above_level"])
def test_linear_transform_closed_forms(mid, case):
    """tests/oracle/test_linear_transform.py:10-199 closed forms."""
    S, level = mid.slots, mid.L - 1
    vals = (np.arange(S) % 7 - 3.0).astype(np.float32) / 4
    ones = np.ones(S, np.float32)
    lt_level, ratio = level, 1.0
    if case == "identity":
        idx, data, exp = [0], [ones], vals
    elif case == "scale":
        idx, data, exp = [0], [3 * ones], 3 * vals
    elif case == "shift":
        idx, data, exp = [3], [ones], np.roll(vals, -3)
    elif case == "two":
        idx, data, exp = [0, 1], [ones, ones], vals + np.roll(vals, -1)
    elif case == "bsgs":
        idx = [0, 1, 2, 5, 8]
        data = [(d + 1.0) * ones for d in idx]
        exp = sum((d + 1.0) * np.roll(vals, -d) for d in idx)
        ratio = 2.0
    else:
        idx, data, exp = [0, 1], [2 * ones, ones], 2 * vals + np.roll(vals, -1)
        lt_level = 1
    t = mid.lt_new(idx, np.stack(data), lt_level, ratio)
    ct = _enc(mid, vals, level, 35, 2)
    out, l = mid.lt_eval(t, ct, level)
    out = mid.rescale(out, l)
    got = mid.decode_f64(mid.decrypt(out, l - 1), l - 1, 2.0 ** 35 * mid.q[lt_level] / mid.q[l])
    np.testing.assert_allclose(got, exp, atol=1e-3)


def test_linear_transform_random_dense(mid):
    """BSGS result equals the dense mat-vec of the diagonal matrix."""
    S, level = mid.slots, mid.L - 1
    rng = np.random.default_rng(23)
    idx = sorted(rng.choice(S, 30, replace=False).tolist())
    data = rng.uniform(-1, 1, (30, S)).astype(np.float32)
    vals = rng.uniform(-1, 1, S).astype(np.float32)
    t = mid.lt_new(idx, data, level, 2.0)
    out, l = mid.lt_eval(t, _enc(mid, vals, level, 35, 3), level)
    out = mid.rescale(out, l)
    got = mid.decode_f64(mid.decrypt(out, l - 1), l - 1, 2.0 ** 35)
    exp = sum(data[n].astype(np.float64) * np.roll(vals.astype(np.float64), -k) for n, k in enumerate(idx))
    np.testing.assert_allclose(got, exp, atol=1e-3)


@pytest.mark.parametrize("diags,slots,ratio,n1", [
    (list(range(512)), 32768, 2.0, 16),       # the 26-table PCMM: 16 baby x 32 giant
    (list(range(16)), 4096, 2.0, 4),          # single table: 4 x 4
    ([0, 1, 2, 5, 8], 4096, 2.0, 4),          # reference BSGS test diagonals
    ([0], 4096, 1.0, 1),                       # identity
])
def test_bsgs_split(mid, diags, slots, ratio, n1):
    """FindBestBSGSRatio with LogBabyStepGiantStepRatio = int(ln(ratio))
    (lineartransform.go:67): hand-computed baby-step counts."""
    q, p = O.gen_primes(int(math.log2(slots)) + 1, [40, 40], [41])
    o = O.Oracle(int(math.log2(slots)) + 1, q, p, h=8, seed=1)
    try:
        t = o.lt_new(diags, np.ones((len(diags), slots), np.float32) * 0.0 + 1.0, 1, ratio)
        assert o.lt_n1(t) == n1
    finally:
        o.close()


# ---------------------------------------------------------------- products and constants


def _negacyclic(a, b, N):
    prod = [0] * N
    for x in range(N):
        if a[x] == 0:
            continue
        for y in range(N):
            if b[y] == 0:
                continue
            k = x + y
            if k < N:
                prod[k] += a[x] * b[y]
            else:
                prod[k - N] -= a[x] * b[y]
    return prod


def test_relin_key_relation(small):
    """b_d + a_d * s = e_d + P * s^2 on the digit's limbs (key from s^2 to s)."""
    key = small.relin_key()
    s = [int(v) for v in small.secret_key()]
    N, mods = small.N, small.q + small.p
    s2 = _negacyclic(s, s, N)
    P = math.prod(small.p)
    for d in range(small.dnum):
        for i, m in enumerate(mods):
            b = small.intt(key[d][0][i], i)
            a = small.intt(key[d][1][i], i)
            prod = _negacyclic([int(v) for v in a], s, N)
            own = i < small.L and d * small.K <= i < (d + 1) * small.K
            e = [(int(b[x]) + prod[x] - (P * s2[x] if own else 0)) % m for x in range(N)]
            e = [v - m if v > m // 2 else v for v in e]
            assert max(abs(v) for v in e) <= 21


def test_mul_plain_is_decrypt_times_plaintext(mid):
    """Dec(ct x pt) == Dec(ct) * pt slot-wise (exact), and it decodes to the product."""
    level = mid.L - 1
    rng = np.random.default_rng(31)
    a = rng.uniform(-1, 1, mid.slots).astype(np.float32)
    b = rng.uniform(-1, 1, mid.slots).astype(np.float32)
    ct = _enc(mid, a, level, 35, 2)
    pt = mid.encode(b, level - 1, 2.0 ** 35)
    out = mid.mul_plain(ct, level, pt, level - 1)
    assert out.shape == (2, level, mid.N)
    dec = mid.decrypt(out, level - 1)
    base = mid.decrypt(ct, level)[:level]
    for i in range(level):
        q = mid.q[i]
        np.testing.assert_array_equal(dec[i], (base[i].astype(object) * pt[i].astype(object)) % q)
    got = mid.decode_f64(dec, level - 1, 2.0 ** 70)
    np.testing.assert_allclose(got, a.astype(np.float64) * b, atol=1e-4)


@pytest.mark.parametrize("k", [3, -5, 0, 1, -1])
def test_mul_int_scales_the_plaintext(mid, k):
    level = mid.L - 1
    vals = np.linspace(-1, 1, mid.slots).astype(np.float32)
    ct = _enc(mid, vals, level, 35, 3)
    out = mid.mul_int(ct, level, k)
    dec, base = mid.decrypt(out, level), mid.decrypt(ct, level)
    for i in range(level + 1):
        q = mid.q[i]
        np.testing.assert_array_equal(dec[i], (base[i].astype(object) * (k % q)) % q)


def test_scaled_constant_rounds_half_away_from_zero():
    from fractions import Fraction
    rng = np.random.default_rng(5)
    for v in list(rng.uniform(-3, 3, 200).astype(np.float32)) + [0.5, -0.5, 2.5, -2.5, 0.0]:
        for scale in (2.0 ** 35, 2.0 ** 40 + 12345, 1073741827.0):
            exact = Fraction(float(v)) * Fraction(scale)
            if abs(exact) >= 2 ** 52:
                continue
            want = int(exact + Fraction(1, 2)) if exact > 0 else -int(-exact + Fraction(1, 2))
            assert O.Oracle.scaled_constant(float(v), scale) == want


def test_mul_float_and_add_const(mid):
    level = mid.L - 1
    vals = np.linspace(-1, 1, mid.slots).astype(np.float32)
    ct = _enc(mid, vals, level, 35, 4)
    base = mid.decrypt(ct, level)
    # non-integer constant: times round(v * q_level), scale grows by q_level
    out, scaled = mid.mul_float(ct, level, 0.75)
    assert scaled
    k = O.Oracle.scaled_constant(0.75, float(mid.q[level]))
    dec = mid.decrypt(out, level)
    for i in range(level + 1):
        np.testing.assert_array_equal(dec[i], (base[i].astype(object) * (k % mid.q[i])) % mid.q[i])
    got = mid.decode_f64(dec, level, 2.0 ** 35 * mid.q[level])
    np.testing.assert_allclose(got, 0.75 * vals.astype(np.float64), atol=1e-5)
    # integer-valued constant: plain integer product, scale unchanged
    out2, scaled2 = mid.mul_float(ct, level, -2.0)
    assert not scaled2
    np.testing.assert_array_equal(out2, mid.mul_int(ct, level, -2))
    # constants: every NTT slot of part 0 moves by round(v * scale), part 1 untouched
    for sub in (False, True):
        out3 = mid.add_const(ct, level, 0.375, 2.0 ** 35, sub)
        np.testing.assert_array_equal(out3[1], ct[1])
        kk = O.Oracle.scaled_constant(0.375, 2.0 ** 35)
        for i in range(level + 1):
            q = mid.q[i]
            delta = (out3[0][i].astype(object) - ct[0][i].astype(object)) % q
            assert set(delta.tolist()) == {(-kk if sub else kk) % q}
        got = mid.decode_f64(mid.decrypt(out3, level), level, 2.0 ** 35)
        np.testing.assert_allclose(got, vals + (-0.375 if sub else 0.375), atol=1e-6)


def test_mul_relin_decrypts_to_product(mid):
    level = mid.L - 1
    rng = np.random.default_rng(41)
    a = rng.uniform(-1, 1, mid.slots).astype(np.float32)
    b = rng.uniform(-1, 1, mid.slots).astype(np.float32)
    ca, cb = _enc(mid, a, level, 35, 5), _enc(mid, b, level, 35, 6)
    out = mid.mul_relin(ca, cb, level)
    got = mid.decode_f64(mid.decrypt(out, level), level, 2.0 ** 70)
    np.testing.assert_allclose(got, a.astype(np.float64) * b, atol=1e-6)
    # squaring: the same ciphertext twice
    sq = mid.mul_relin(ca, ca, level)
    got = mid.decode_f64(mid.decrypt(sq, level), level, 2.0 ** 70)
    np.testing.assert_allclose(got, a.astype(np.float64) ** 2, atol=1e-6)
    # rescaled once: back to scale 2^70 / q_level
    r = mid.rescale(out, level)
    got = mid.decode_f64(mid.decrypt(r, level - 1), level - 1, 2.0 ** 70 / mid.q[level])
    np.testing.assert_allclose(got, a.astype(np.float64) * b, atol=1e-6)


@pytest.mark.parametrize("coeffs", [[0.25], [0.1, 0.9], [0.05, 0.5, 0.25], [0.047, 0.5, 0.24, -0.003], [0.0, 1.0, 0.0, 0.0]])
def test_eval_poly_decrypts_to_polynomial(mid, coeffs):
    """Degree <= 3 at depth ceil(log2(d + 1)), output at the requested scale."""
    level = mid.L - 1
    vals = np.linspace(-1, 1, mid.slots).astype(np.float32)
    ct = _enc(mid, vals, level, 35, 7)
    out, nl = mid.eval_poly(ct, level, 2.0 ** 35, coeffs, 2.0 ** 35)
    d = len(coeffs) - 1
    while d > 0 and coeffs[d] == 0:
        d -= 1
    assert nl == level - (0 if d == 0 else 1 if d == 1 else 2)
    got = mid.decode_f64(mid.decrypt(out, nl), nl, 2.0 ** 35)
    want = np.polyval(np.asarray(coeffs[::-1], dtype=np.float64), vals.astype(np.float64))
    np.testing.assert_allclose(got, want, atol=1e-5)
