"""The committed cross-check bundle (tests/golden/bundle_pcmm_n10): the oracle
still writes these bytes, and the words in them are the objects they claim
to be (secret key out of Montgomery form and the inverse NTT is ternary,
ciphertexts decrypt to the PCMM's embedding)."""
import hashlib
import json
import os

import numpy as np

from helpers import from_montgomery, parse_wire_poly, parse_wire_qp
from oracle import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
BUNDLE = os.path.join(HERE, "golden", "bundle_pcmm_n10")


def load_bundle():
    with open(os.path.join(BUNDLE, "params.json")) as f:
        man = json.load(f)
    files = {}
    for name in man["sha256"]:
        with open(os.path.join(BUNDLE, name), "rb") as f:
            files[name] = f.read()
    return man, files


def parse_element(b, N):
    buf = np.frombuffer(b, dtype=np.uint8)
    hdr = buf[:32].view("<u8")
    scale = float(np.array([hdr[0]], dtype="<u8").view("<f8")[0])
    off, polys = 32, []
    for _ in range(int(hdr[3])):
        p, off = parse_wire_poly(buf, off, N)
        polys.append(p)
    assert off == len(buf)
    return scale, int(hdr[1]), int(hdr[2]), np.stack(polys)


def test_bundle_reproduced_by_oracle():
    import sys
    sys.path.insert(0, os.path.join(HERE, "golden"))
    from make_bundle import N10, build_bundle
    man, files = load_bundle()
    for name, data in files.items():
        assert hashlib.sha256(data).hexdigest() == man["sha256"][name], name
    files2, man2 = build_bundle(N10)
    assert sorted(files2) == sorted(files)
    for name in files:
        assert files2[name] == files[name], f"{name} differs from the oracle's bytes"
    assert man2 == man


def test_bundle_words_are_the_objects():
    man, files = load_bundle()
    s = man["scheme"]
    N = 1 << s["logN"]
    q, p = s["Q"], s["P"]
    orc = O.Oracle(s["logN"], q, p, h=s["h"], seed=s["key_seed"])
    try:
        (sq, sp), off = parse_wire_qp(np.frombuffer(files["sk.bin"], dtype=np.uint8), 0, N)
        assert off == len(files["sk.bin"])
        rows = from_montgomery(np.concatenate([sq, sp]), list(q) + list(p))
        for m in range(len(q) + len(p)):
            coef = orc.intt(rows[m], m)
            mod = (list(q) + list(p))[m]
            signed = np.where(coef > mod // 2, coef.astype(np.int64) - int(mod), coef.astype(np.int64))
            assert set(np.unique(signed)) <= {-1, 0, 1}
            np.testing.assert_array_equal(signed, orc.secret_key())
        scale, logslots, flags, ct = parse_element(files["ct_out.bin"], N)
        assert (scale, logslots, flags) == (man["ct_out"]["scale"], s["logN"] - 1, 3)
        level = man["ct_out"]["level"]
        dec = orc.decode_f64(orc.decrypt(ct, level), level, scale)
        rng = np.random.default_rng(man["pcmm"]["table_seed"])
        t0, t1 = [rng.uniform(-0.1, 0.1, (16, 16)).astype(np.float32) for _ in range(2)]
        idx = man["pcmm"]["index"]
        want = t0[idx % 16].astype(np.float64) + t1[idx // 16]
        assert np.abs(dec[:16] - want).max() < 2.0 ** -10
        g = man["pcmm"]["galois_elements"][0]
        key = np.frombuffer(files[f"gk_{g}.bin"], dtype=np.uint8)
        head = key[:32].view("<u8")
        assert list(head) == [g, 2 * N, 0, (len(q) + len(p) - 1) // len(p)]
    finally:
        orc.close()
