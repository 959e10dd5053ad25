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


def oracle_linear(orc, ct, level, scale, diagonals, output_rotations, logscale, bias=None, bsgs_ratio=2.0,
                  lt_level=None):
    """One more Orion Linear (LT compiled at `lt_level`, default `level`;
    rescale, hybrid fold, bias) on an oracle ciphertext at `level` and
    `scale`.  Returns (ct, level, scale)."""
    idx = list(diagonals.keys())
    data = np.stack([diagonals[i] for i in idx])
    lt_level = level if lt_level is None else lt_level
    t = orc.lt_new(idx, data, lt_level, bsgs_ratio)
    out, l = orc.lt_eval(t, ct, level)
    sc = scale * orc.q[lt_level]
    out = orc.rescale(out, l)
    sc /= orc.q[l]
    l -= 1
    for i in range(1, output_rotations + 1):
        out = orc.add(out, orc.rotate(out, l, orc.slots // (2 ** i)), l)
    b = np.zeros(1, np.float32) if bias is None else bias
    out[0] = orc.add(out[0][None], orc.encode(b, l, float(1 << logscale))[None], l)[0]
    return out, l, sc


def oracle_dlrm(orc, w, dense_index=0, sparse_index=1, keep=False):
    """DLRMWorkload.run_stages on the CPU restatement: both inputs encrypted
    at the input level with encryption indices `dense_index` and
    `sparse_index`, then every Linear (oracle_linear) and activation
    (monomial eval_poly at the default scale) in forward order.  Returns
    ((ct, level, scale), {layer name: (ct, level, scale)} when keep)."""
    logscale = w.cfg["logscale"]
    scale = float(1 << logscale)
    L = w.input_level
    trace = {}

    def enc(values, index):
        return orc.encrypt(orc.encode(np.asarray(values, np.float32), L, scale), L, index), L, scale

    def step(name, x):
        ct, l, sc = x
        m = w.modules[name]
        if hasattr(m, "diagonals"):
            y = oracle_linear(orc, ct, l, sc, m.diagonals[(0, 0)], m.output_rotations, logscale, bias=m.bias,
                              lt_level=w.levels[name])
        else:
            out, nl = orc.eval_poly(ct, l, sc, list(m.coeffs[::-1]), scale)
            y = (out, nl, scale)
        if keep:
            trace[name] = y
        return y
    x = enc(w.dense, dense_index)
    for _, name in w.bottom_names:
        x = step(name, x)
    e = step("sparse", enc(w.emb.selector, sparse_index))
    e = step("sparse_to_top", e)
    assert x[1] == e[1] and x[2] == e[2]
    z = (orc.add(x[0], e[0], x[1]), x[1], x[2])
    if keep:
        trace["add"] = z
    for _, name in w.top_names:
        z = step(name, z)
    return z, trace


def parse_wire_poly(buf, off, N):
    """ring.Poly in the library's wire format: u64 rows, then per row u64 N
    and N little-endian u64 words.  Returns (rows x N array, new offset)."""
    buf = np.asarray(buf, dtype=np.uint8)
    rows = int(buf[off:off + 8].view("<u8")[0])
    off += 8
    out = np.zeros((rows, N), dtype=np.uint64)
    for r in range(rows):
        n = int(buf[off:off + 8].view("<u8")[0])
        assert n == N, f"row {r}: length {n}, expected {N}"
        off += 8
        out[r] = buf[off:off + 8 * N].view("<u8")
        off += 8 * N
    return out, off


def parse_wire_qp(buf, off, N):
    """ringqp.Poly: the Q part then the P part.  Returns ((Q, P), offset)."""
    q, off = parse_wire_poly(buf, off, N)
    p, off = parse_wire_poly(buf, off, N)
    return (q, p), off


def from_montgomery(rows, mods):
    """x * 2^-64 mod q for each row (row i under mods[i])."""
    out = np.zeros_like(rows)
    for i, q in enumerate(mods):
        rinv = pow(1 << 64, -1, int(q))
        out[i] = np.array([(int(v) * rinv) % int(q) for v in rows[i]], dtype=np.uint64)
    return out
