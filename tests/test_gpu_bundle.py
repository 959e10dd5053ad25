"""The HIP library against the committed cross-check bundle
(tests/golden/bundle_pcmm_n10, written from the oracle's objects):

* on the bundle's moduli and key seed the library serializes byte for byte
  the same secret key, Galois keys, diagonals, encoded selector and
  ciphertexts (input, transform output, PCMM output);
* in a scheme built with another seed, every object loaded from the bundle
  (secret key, Galois keys, diagonals through io_mode "load", the input
  ciphertext) gives the bundle's PCMM output, byte for byte;
* malformed ciphertext bytes are refused and leave the library usable."""
import json
import os

import numpy as np
import pytest

from helpers import new_hip_scheme
from helrm_amd import orion_host as oh
from helrm_amd.backend import HipError

pytestmark = pytest.mark.gpu

BUNDLE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "bundle_pcmm_n10")


@pytest.fixture(scope="module")
def bundle():
    with open(os.path.join(BUNDLE, "params.json")) as f:
        man = json.load(f)
    files = {}
    for name in man["sha256"]:
        with open(os.path.join(BUNDLE, name), "rb") as f:
            files[name] = f.read()
    return man, files


def pcmm_data(man):
    s, pc = man["scheme"], man["pcmm"]
    S = 1 << (s["logN"] - 1)
    rng = np.random.default_rng(pc["table_seed"])
    tables = [[rng.uniform(-0.1, 0.1, (16, 16)).astype(np.float32) for _ in range(2)]]
    d, fold = oh.diagonalize(oh.block_diag_matrix(tables), S)
    d = d[(0, 0)]
    assert list(d.keys()) == pc["diagonal_indices"] and [S >> i for i in range(1, fold + 1)] == pc["fold_rotations"]
    return d, oh.expanded_sparse([pc["index"]], [256], 0, 16)


def finish_pcmm(lib, man, lt):
    """Rescale, hybrid fold and zero bias of a transform output."""
    s = man["scheme"]
    r = lib.RescaleNew(lt)
    for rot in man["pcmm"]["fold_rotations"]:
        t = lib.RotateNew(r, rot)
        lib.AddCiphertext(r, t)
        lib.DeleteCiphertext(t)
    lib.AddPlaintext(r, lib.Encode([0.0], man["ct_out"]["level"], 1 << s["log_scale"]))
    return r


def same(lib, got, want, what):
    got = bytes(np.asarray(got, dtype=np.uint8))
    assert len(got) == len(want), f"{what}: {len(got)} bytes, bundle {len(want)}"
    assert got == want, f"{what}: bytes differ from the bundle"


def test_library_writes_the_bundle(hip_lib, bundle):
    man, files = bundle
    lib, s, pc = hip_lib, man["scheme"], man["pcmm"]
    print("[bundle] library objects vs bundle bytes", flush=True)
    new_hip_scheme(lib, s["logN"], s["Q"], s["P"], s["log_scale"], s["h"], s["key_seed"])
    same(lib, lib.serialize("SerializeSecretKey"), files["sk.bin"], "secret key")
    for g in pc["galois_elements"]:
        same(lib, lib.serialize("GenerateAndSerializeRotationKey", g), files[f"gk_{g}.bin"], f"Galois key {g}")
    d, sel = pcmm_data(man)
    idx = list(d.keys())
    level = pc["level"]
    tid = lib.GenerateLinearTransform(idx, np.concatenate([d[i] for i in idx]), level, pc["bsgs_ratio"], "none")
    for ge in lib.GetLinearTransformRotationKeys(tid):
        lib.GenerateLinearTransformRotationKey(ge)
    pt = lib.Encode(sel.tolist(), level, 1 << s["log_scale"])
    same(lib, lib.serialize("SerializePlaintext", pt), files["pt_in.bin"], "encoded selector")
    lib.SetEncryptionCounter(man["ct_in"]["encryption_index"])
    ct = lib.Encrypt(pt)
    same(lib, lib.serialize("SerializeCiphertext", ct), files["ct_in.bin"], "input ciphertext")
    lt = lib.EvaluateLinearTransform(tid, ct)
    same(lib, lib.serialize("SerializeCiphertext", lt), files["ct_lt.bin"], "transform output")
    out = finish_pcmm(lib, man, lt)
    same(lib, lib.serialize("SerializeCiphertext", out), files["ct_out.bin"], "PCMM output")
    for i in idx:
        same(lib, lib.serialize("SerializeDiagonal", tid, i), files[f"diag_{i}.bin"], f"diagonal {i}")
    lib.DeleteScheme()


def test_bundle_loads_and_reproduces_output(hip_lib, bundle):
    man, files = bundle
    lib, s, pc = hip_lib, man["scheme"], man["pcmm"]
    print("[bundle] loading the bundle into a scheme with another seed", flush=True)
    lib.NewSchemeWithModuli(s["logN"], s["Q"], s["P"], s["log_scale"], s["h"], s["key_seed"] + 1000)
    lib.NewKeyGenerator()
    lib.LoadSecretKey(files["sk.bin"])
    for f in ("NewEncoder", "NewEncryptor", "NewDecryptor", "NewEvaluator", "NewLinearTransformEvaluator"):
        getattr(lib, f)()
    for g in pc["galois_elements"]:
        lib.LoadRotationKey(files[f"gk_{g}.bin"], g)
    idx = pc["diagonal_indices"]
    tid = lib.GenerateLinearTransform(idx, np.zeros(0, np.float32), pc["level"], pc["bsgs_ratio"], "load")
    for i in idx:
        lib.LoadPlaintextDiagonal(files[f"diag_{i}.bin"], tid, i)
    ct = lib.LoadCiphertext(files["ct_in.bin"])
    assert lib.GetCiphertextLevel(ct) == man["ct_in"]["level"]
    assert lib.GetCiphertextScaleDouble(ct) == man["ct_in"]["scale"]
    pt = lib.LoadPlaintext(files["pt_in.bin"])
    same(lib, lib.serialize("SerializePlaintext", pt), files["pt_in.bin"], "reloaded plaintext")
    lt = lib.EvaluateLinearTransform(tid, ct)
    same(lib, lib.serialize("SerializeCiphertext", lt), files["ct_lt.bin"], "transform output from loaded objects")
    out = finish_pcmm(lib, man, lt)
    same(lib, lib.serialize("SerializeCiphertext", out), files["ct_out.bin"], "PCMM output from loaded objects")
    # malformed input is refused and the library stays usable
    good = bytearray(files["ct_in.bin"])
    for bad, msg in ((bytes(good[:-8]), "truncated"), (bytes(good) + b"\0" * 8, "trailing"),
                     (bytes(good[:16]) + (5).to_bytes(8, "little") + bytes(good[24:]), "NTT domain")):
        with pytest.raises(HipError, match=msg):
            lib.LoadCiphertext(bad)
    assert lib.GetCiphertextLevel(lib.LoadCiphertext(files["ct_out.bin"])) == man["ct_out"]["level"]
    lib.DeleteScheme()
