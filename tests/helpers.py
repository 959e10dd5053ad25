"""Shared set-up for parity tests: one parameter set, the oracle and the HIP
library on the same moduli, secret key seed and encryption indices."""
import numpy as np

from oracle import oracle as O


def make_params(logN, logq, logp):
    q, p = O.gen_primes(logN, logq, logp)
    return q, p


def new_hip_scheme(lib, logN, q, p, logscale, h, seed, evaluator=True):
    lib.NewSchemeWithModuli(logN, list(q), list(p), logscale, h, seed)
    lib.NewKeyGenerator()
    lib.GenerateSecretKey()
    lib.GeneratePublicKey()
    lib.NewEncoder()
    lib.NewEncryptor()
    lib.NewDecryptor()
    if evaluator:
        lib.NewEvaluator()
    lib.NewLinearTransformEvaluator()


def cfg1_tables(seed):
    """Single-table cfg: 2 digit sub-tables of 16x16, U[-0.1, 0.1], index in [0, 256)."""
    rng = np.random.default_rng(seed)
    T = [rng.uniform(-0.1, 0.1, (16, 16)).astype(np.float32) for _ in range(2)]
    idx = int(rng.integers(0, 256))
    return T, idx


def assert_equal_u64(a, b, what):
    a = np.asarray(a, dtype=np.uint64)
    b = np.asarray(b, dtype=np.uint64)
    assert a.shape == b.shape, f"{what}: shape {a.shape} vs {b.shape}"
    if not np.array_equal(a, b):
        bad = np.argwhere(a != b)
        raise AssertionError(f"{what}: {len(bad)} of {a.size} words differ, first at {tuple(bad[0])}: {a[tuple(bad[0])]} vs {b[tuple(bad[0])]}")


def oracle_pcmm(orc, diagonals, output_rotations, level, selector, logscale, enc_index, bias=None, bsgs_ratio=2.0):
    """The Orion embedding-PCMM flow (encode + encrypt the selector, LT,
    rescale, hybrid fold, bias) run on the CPU restatement.  Returns the
    output ciphertext, its level and scale."""
    scale = float(1 << logscale)
    idx = list(diagonals.keys())
    data = np.stack([diagonals[i] for i in idx])
    t = orc.lt_new(idx, data, level, bsgs_ratio)
    ct = orc.encrypt(orc.encode(selector, level, scale), level, enc_index)
    out, l = orc.lt_eval(t, ct, level)
    sc = scale * orc.q[level]
    out = orc.rescale(out, l)
    sc /= orc.q[l]
    l -= 1
    slots = orc.slots
    for i in range(1, output_rotations + 1):
        out = orc.add(out, orc.rotate(out, l, slots // (2 ** i)), l)
    b = np.zeros(1, np.float32) if bias is None else bias
    out[0] = orc.add(out[0][None], orc.encode(b, l, scale)[None], l)[0]
    return out, l, sc


def oracle_linear(orc, ct, level, scale, diagonals, output_rotations, logscale, bias=None, bsgs_ratio=2.0):
    """One more Orion Linear (LT at `level`, rescale, hybrid fold, bias) on an
    oracle ciphertext at `level` and `scale`.  Returns (ct, level, scale)."""
    idx = list(diagonals.keys())
    data = np.stack([diagonals[i] for i in idx])
    t = orc.lt_new(idx, data, level, bsgs_ratio)
    out, l = orc.lt_eval(t, ct, level)
    sc = scale * orc.q[level]
    out = orc.rescale(out, l)
    sc /= orc.q[l]
    l -= 1
    for i in range(1, output_rotations + 1):
        out = orc.add(out, orc.rotate(out, l, orc.slots // (2 ** i)), l)
    b = np.zeros(1, np.float32) if bias is None else bias
    out[0] = orc.add(out[0][None], orc.encode(b, l, float(1 << logscale))[None], l)[0]
    return out, l, sc
