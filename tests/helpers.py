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


def row_digests(a):
    """Hex SHA-256 of every row (last axis) of a u64 array, little-endian words,
    as tests/golden/make_fullsize_digests.py writes them."""
    import hashlib
    a = np.ascontiguousarray(a, dtype="<u8")
    return [hashlib.sha256(r.tobytes()).hexdigest() for r in a.reshape(-1, a.shape[-1])]


def fullsize_digests(name):
    """The oracle's digests of one full-size layer (tests/golden/fullsize_digests.json)."""
    import json
    import os
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fullsize_digests.json")
    with open(path) as f:
        return json.load(f)[name]


def assert_rows_match(a, want_rows, what):
    """Row-wise SHA-256 comparison of a u64 array with the oracle's digests;
    names the first rows that differ."""
    got = row_digests(a)
    assert len(got) == len(want_rows), f"{what}: {len(got)} rows, oracle has {len(want_rows)}"
    bad = [i for i, (g, w) in enumerate(zip(got, want_rows)) if g != w]
    assert not bad, f"{what}: {len(bad)} of {len(got)} rows differ from the oracle, first rows {bad[:8]}"


def check_fullsize_layer(lib, w, d, what):
    """A set-up LinearWorkload at N=2^16 against the oracle's digests d: the
    moduli, the input ciphertext, two encoded diagonals, one giant-step key,
    the transform output before the rescale, and the layer output with the
    transform's rescale both separate (Lattigo's convention) and fused into
    its final ModDown (lt_output_prerescaled).  Returns the output."""
    assert lib.GetModuliChain() == d["q"] and lib.GetAuxModuliChain() == d["p"]
    tid = int(list(w.layer.transform_ids.values())[0])
    assert lib.lt_info(tid)["N1"] == d["N1"] and w.layer.output_rotations == d["fold_rotations"]
    cid = w.ct_in.ids[0]
    assert_rows_match(lib.export_ciphertext(cid), d["ct_in"], f"{what} input ciphertext")
    for k in ("diag_first", "diag_last"):
        assert_rows_match(lib.export_lt_diagonal(tid, d[k]["index"], d["level"]), d[k]["rows"],
                          f"{what} diagonal {d[k]['index']}")
    assert_rows_match(lib.export_galois_key(d["galois_key"]["galel"]), d["galois_key"]["rows"],
                      f"{what} Galois key of rotation {d['galois_key']['rotation']}")
    lib.set_lt_output_prerescaled(False)
    lt = lib.EvaluateLinearTransform(tid, cid)
    assert lib.GetCiphertextLevel(lt) == d["lt_out"]["level"]
    assert lib.GetCiphertextScaleDouble(lt) == d["lt_out"]["scale"]
    assert_rows_match(lib.export_ciphertext(lt), d["lt_out"]["rows"], f"{what} transform output")
    lib.DeleteCiphertext(lt)
    out = None
    for pre in (False, True):
        lib.set_lt_output_prerescaled(pre)
        if out is not None:
            out.free()
        out = w.run()
        oid = out.ids[0]
        assert lib.GetCiphertextLevel(oid) == d["out"]["level"]
        assert lib.GetCiphertextScaleDouble(oid) == d["out"]["scale"]
        assert_rows_match(lib.export_ciphertext(oid), d["out"]["rows"], f"{what} layer output (prerescaled {pre})")
    return out
