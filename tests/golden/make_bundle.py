"""Cross-check bundle of the single-table embedding PCMM, written from the
oracle's objects (oracle/) in the library's wire layout, for a machine with
Go and Lattigo v6.2.0 to load and compare against Lattigo's own evaluation.

    python tests/golden/make_bundle.py                  # the committed N=2^10 bundle
    python tests/golden/make_bundle.py --cfg1 OUTDIR    # the same at N=2^13, 5 + 1 limbs
                                                        # (about 60 MB: not committed)

Files (tests/golden/bundle_pcmm_n10/):
  params.json   moduli, scale, secret-key seed, the transform's diagonal
                indices / baby-step size / Galois elements, the fold
                rotations, levels and scales, SHA-256 of every file
  sk.bin        secret key: ringqp.Poly over the whole QP basis (NTT,
                Montgomery form)
  gk_<g>.bin    Galois key of element g: g, 2N, 0, dnum, then per digit
                1, 2 and (b, a) as ringqp.Poly (NTT, Montgomery form)
  diag_<d>.bin  diagonal d of the transform, pre-rotated by its giant step:
                ringqp.Poly at the transform's level (NTT, Montgomery form)
  pt_in.bin     the encoded selector; ct_in.bin its encryption (index 0)
  ct_lt.bin     EvaluateLinearTransform output (before the rescale)
  ct_out.bin    the PCMM output: rescale, hybrid fold, zero bias
Plaintext / ciphertext files: scale (binary64 bits), log2 slots, flags
(0b011: batched, NTT domain, standard representatives), count, then count
ring.Poly.  Every word is little-endian u64.
"""
import argparse
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402
from helrm_amd import orion_host as oh  # noqa: E402

N10 = dict(logn=10, logq=[40, 30, 30], logp=[41, 41], logscale=30, h=32, seed=77, table_seed=5, index=201)
CFG1 = dict(logn=13, logq=[60, 40, 40, 40, 40], logp=[61], logscale=40, h=192, seed=77, table_seed=5, index=201)
OUT = os.path.join(HERE, "bundle_pcmm_n10")


# ---- wire layout ---------------------------------------------------------------
def _u64(x):
    return int(x).to_bytes(8, "little")


def wire_poly(rows):
    rows = np.ascontiguousarray(rows, dtype="<u8")
    out = [_u64(rows.shape[0])]
    for r in rows:
        out.append(_u64(rows.shape[1]))
        out.append(r.tobytes())
    return b"".join(out)


def wire_qp(rows, nq):
    return wire_poly(rows[:nq]) + wire_poly(rows[nq:])


def wire_element(polys, scale, logslots):
    bits = np.array([scale], dtype="<f8").view("<u8")[0]
    out = [_u64(bits), _u64(logslots), _u64(0x3), _u64(len(polys))]
    out += [wire_poly(p) for p in polys]
    return b"".join(out)


def to_montgomery(rows, mods):
    """x * 2^64 mod q, row i under mods[i]."""
    out = np.zeros_like(rows, dtype=np.uint64)
    for i, q in enumerate(mods):
        q = int(q)
        R = (1 << 64) % q
        out[i] = np.array([(int(v) * R) % q for v in rows[i]], dtype=np.uint64)
    return out


# ---- the bundle --------------------------------------------------------------------
def build_bundle(c):
    """{file name: bytes} and the manifest of the single-table PCMM at parameters c."""
    q, p = O.gen_primes(c["logn"], c["logq"], c["logp"])
    orc = O.Oracle(c["logn"], q, p, h=c["h"], seed=c["seed"])
    try:
        N, S, L, K = orc.N, orc.slots, len(q), len(p)
        level, scale = L - 1, float(1 << c["logscale"])
        qp_all = list(q) + list(p)
        rng = np.random.default_rng(c["table_seed"])
        tables = [[rng.uniform(-0.1, 0.1, (16, 16)).astype(np.float32) for _ in range(2)]]
        sel = oh.expanded_sparse([c["index"]], [256], 0, 16)
        d, fold = oh.diagonalize(oh.block_diag_matrix(tables), S)
        d = d[(0, 0)]
        idx = list(d.keys())
        files = {}
        # secret key: NTT of the ternary coefficients in every QP limb
        sk = orc.secret_key()
        sk_rows = np.zeros((L + K, N), dtype=np.uint64)
        for m, mod in enumerate(qp_all):
            row = np.array([(int(v) % int(mod)) for v in sk], dtype=np.uint64)
            sk_rows[m] = orc.ntt(row, m)
        files["sk.bin"] = wire_qp(to_montgomery(sk_rows, qp_all), L)
        t = orc.lt_new(idx, np.stack([d[i] for i in idx]), level, 2.0)
        rots = [r for r in orc.lt_rotations(t) if r]
        fold_rots = [S >> i for i in range(1, fold + 1)]
        galels = sorted({int(orc.galois_element(r)) for r in rots + fold_rots})
        dnum = (L + K - 1) // K
        for g in galels:
            key = orc.galois_key(g)
            parts = [_u64(g), _u64(2 * N), _u64(0), _u64(dnum)]
            for dg in range(dnum):
                parts += [_u64(1), _u64(2)]
                for part in range(2):
                    parts.append(wire_qp(to_montgomery(key[dg, part], qp_all), L))
            files[f"gk_{g}.bin"] = b"".join(parts)
        lt_mods = list(q[:level + 1]) + list(p)
        for i in orc.lt_plaintext_indices(t):
            files[f"diag_{i}.bin"] = wire_qp(to_montgomery(orc.lt_plaintext(t, i), lt_mods), level + 1)
        pt = orc.encode(sel, level, scale)
        files["pt_in.bin"] = wire_element([pt], scale, c["logn"] - 1)
        ct = orc.encrypt(pt, level, 0)
        files["ct_in.bin"] = wire_element([ct[0], ct[1]], scale, c["logn"] - 1)
        lt, l = orc.lt_eval(t, ct, level)
        lt_scale = scale * q[level]
        files["ct_lt.bin"] = wire_element([lt[0], lt[1]], lt_scale, c["logn"] - 1)
        out = orc.rescale(lt, l)
        out_scale = lt_scale / q[l]
        l -= 1
        for r in fold_rots:
            out = orc.add(out, orc.rotate(out, l, r), l)
        out[0] = orc.add(out[0][None], orc.encode(np.zeros(1, np.float32), l, scale)[None], l)[0]
        files["ct_out.bin"] = wire_element([out[0], out[1]], out_scale, c["logn"] - 1)
        manifest = {
            "scheme": {"logN": c["logn"], "ring": "standard", "Q": [int(v) for v in q], "P": [int(v) for v in p],
                       "log_scale": c["logscale"], "h": c["h"], "key_seed": c["seed"]},
            "pcmm": {"table_seed": c["table_seed"], "index": c["index"], "level": level,
                     "diagonal_indices": [int(i) for i in idx], "bsgs_ratio": 2.0, "N1": int(orc.lt_n1(t)),
                     "lt_rotations": [int(r) for r in rots], "fold_rotations": fold_rots,
                     "galois_elements": galels},
            "ct_in": {"level": level, "scale": scale, "encryption_index": 0},
            "ct_lt": {"level": level, "scale": lt_scale},
            "ct_out": {"level": l, "scale": out_scale},
            "sha256": {k: hashlib.sha256(v).hexdigest() for k, v in sorted(files.items())},
        }
        return files, manifest
    finally:
        orc.close()


def write_bundle(files, manifest, outdir):
    os.makedirs(outdir, exist_ok=True)
    for name, data in files.items():
        with open(os.path.join(outdir, name), "wb") as f:
            f.write(data)
    with open(os.path.join(outdir, "params.json"), "w") as f:
        json.dump(manifest, f, indent=1)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--cfg1", metavar="OUTDIR", help="write the N=2^13 single-table bundle to OUTDIR")
    args = ap.parse_args()
    O.set_threads(os.cpu_count() or 1)
    if args.cfg1:
        write_bundle(*build_bundle(CFG1), args.cfg1)
        print(f"wrote {args.cfg1}")
    else:
        write_bundle(*build_bundle(N10), OUT)
        print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
