"""End-to-end embedding PCMM on the GPU through the host mirror of Orion's
callers (helrm_amd.orion_host): selector -> encode -> encrypt -> BSGS linear
transform -> rescale -> hybrid fold -> bias -> decrypt -> decode.

* single_table, pcmm26_n13 and the ragged selector: the output ciphertext is
  bit-exact with the same flow run on the CPU restatement (oracle/);
* pcmm26 and pcmm26 + sparse_to_top (N=2^16): bit-exact with the oracle's
  words through committed per-row SHA-256 digests
  (tests/golden/make_fullsize_digests.py).
* queries issued on the library's two HIP streams: word for word what the
  same queries give one at a time;
* every config: decrypted embeddings within 2^-20 of the fp32 plaintext
  lookup (tolerance from the task statement).
"""
import numpy as np
import pytest

from helpers import assert_equal_u64, assert_rows_match, check_fullsize_layer, fullsize_digests, oracle_linear, oracle_pcmm
from oracle import oracle as O
from helrm_amd.workloads import PCMMWorkload, SparseToTopWorkload

pytestmark = pytest.mark.gpu

TOL = 2.0 ** -20


@pytest.mark.parametrize("name", ["single_table", "pcmm26_n13", "pcmm_ragged_n13"])
def test_pcmm_bitexact_vs_oracle(hip_lib, name):
    print(f"[pcmm] {name}: building", flush=True)
    w = PCMMWorkload(hip_lib, name, seed=3, key_seed=17).setup()
    info = w.shape_info()
    print(f"[pcmm] {name}: {info}", flush=True)
    out = w.run()
    got = hip_lib.export_ciphertext(out.ids[0])
    c = w.cfg
    orc = O.Oracle(c["logn"], hip_lib.GetModuliChain(), hip_lib.GetAuxModuliChain(), h=c["h"], seed=17)
    try:
        want, l, sc = oracle_pcmm(orc, w.layer.diagonals[(0, 0)], w.layer.output_rotations, w.layer.level,
                                  w.selector, c["logscale"], 0)
        assert hip_lib.GetCiphertextLevel(out.ids[0]) == l
        assert hip_lib.GetCiphertextScaleDouble(out.ids[0]) == sc
        assert_equal_u64(got, want, f"{name} PCMM output")
    finally:
        orc.close()
    y = w.decrypt_output(out)
    err = np.abs(y - w.expected).max()
    print(f"[pcmm] {name}: max |decrypted - lookup| = {err:.3e}", flush=True)
    assert err < TOL
    hip_lib.DeleteScheme()


@pytest.mark.parametrize("name", ["single_table", "pcmm26_n13"])
def test_pcmm_prerescaled_bitexact_vs_oracle(hip_lib, name):
    """lt_output_prerescaled (lt_evaluator.py:262-273): EvaluateLinearTransform
    returns the rescaled result, its first division fused into the final
    ModDown, and the host skips its Rescale; the PCMM output stays bit-exact
    with the restatement's transform-then-rescale flow."""
    print(f"[pcmm] {name} prerescaled: building", flush=True)
    w = PCMMWorkload(hip_lib, name, seed=5, key_seed=17).setup()
    hip_lib.set_lt_output_prerescaled(True)
    assert hip_lib.lt_output_prerescaled
    out = w.run()
    got = hip_lib.export_ciphertext(out.ids[0])
    c = w.cfg
    orc = O.Oracle(c["logn"], hip_lib.GetModuliChain(), hip_lib.GetAuxModuliChain(), h=c["h"], seed=17)
    try:
        want, l, sc = oracle_pcmm(orc, w.layer.diagonals[(0, 0)], w.layer.output_rotations, w.layer.level,
                                  w.selector, c["logscale"], 0)
        assert hip_lib.GetCiphertextLevel(out.ids[0]) == l
        assert hip_lib.GetCiphertextScaleDouble(out.ids[0]) == sc
        assert_equal_u64(got, want, f"{name} prerescaled PCMM output")
    finally:
        orc.close()
    assert np.abs(w.decrypt_output(out) - w.expected).max() < TOL
    hip_lib.DeleteScheme()
    assert not hip_lib.lt_output_prerescaled  # the setting belongs to the scheme


def test_pcmm_seeded_upload(hip_lib):
    """bench_sweep.py:381-399 seeded upload: the selector is encrypted with a
    seeded `a`, `a` is dropped (only b crossed the wire) and rebuilt on the
    device before the PCMM; the output is bit-exact with the restatement's
    PCMM of the restatement's seeded ciphertext."""
    name = "pcmm26_n13"
    w = PCMMWorkload(hip_lib, name, seed=4, key_seed=17).setup()
    s = w.scheme
    pt = s.encode(w.selector, w.layer.level)
    hip_lib.SetEncryptionCounter(3)
    cid = hip_lib.EncryptSeeded(pt.ids[0], 0xC0FFEE)
    hip_lib.DropAx(cid)
    hip_lib.ExpandSeededAx(cid, 0xC0FFEE)
    from helrm_amd import orion_host as oh
    out = w.layer.forward(oh.CipherTensor(s, [cid], pt.n))
    got = hip_lib.export_ciphertext(out.ids[0])
    c = w.cfg
    orc = O.Oracle(c["logn"], hip_lib.GetModuliChain(), hip_lib.GetAuxModuliChain(), h=c["h"], seed=17)
    try:
        level, scale = w.layer.level, float(1 << c["logscale"])
        ct = orc.encrypt_seeded(orc.encode(w.selector, level, scale), level, 0xC0FFEE, 3)
        want, l, sc = oracle_linear(orc, ct, level, scale, w.layer.diagonals[(0, 0)], w.layer.output_rotations,
                                    c["logscale"])
        assert_equal_u64(got, want, f"{name} seeded-upload PCMM output")
    finally:
        orc.close()
    y = w.decrypt_output(out)
    assert np.abs(y - w.expected).max() < TOL
    hip_lib.DeleteScheme()


def test_pcmm_io_mode_save_load(hip_lib, tmp_path):
    """Orion's io_mode (key_generator.py:17-31, lt_evaluator.py:133-161,
    224-262, 440-497) on the embedding PCMM: "save" serializes the secret key,
    the rotation keys and every diagonal to files and evaluates from the
    reloaded bytes; "load" in a new scheme instance reads them back instead of
    generating them.  All three modes give the same output ciphertext, word
    for word."""
    name = "pcmm26_n13"
    outs = {}
    for mode in ("none", "save", "load"):
        print(f"[pcmm] {name}: io_mode {mode}", flush=True)
        w = PCMMWorkload(hip_lib, name, seed=6, key_seed=17)
        w.params.io_mode = mode
        w.params.keys_path = str(tmp_path / "keys.npz")
        w.params.diags_path = str(tmp_path / "diags.npz")
        w.setup()
        out = w.run()
        outs[mode] = hip_lib.export_ciphertext(out.ids[0])
        if mode == "save":
            w.scheme.flush()
            assert "sk" in w.scheme.key_store
            assert len([k for k in w.scheme.diag_store.keys()]) == w.shape_info()["diagonals"]
        else:
            y = w.decrypt_output(out)
            assert np.abs(y - w.expected).max() < TOL
        hip_lib.DeleteScheme()
    assert_equal_u64(outs["save"], outs["none"], "io_mode save")
    assert_equal_u64(outs["load"], outs["none"], "io_mode load")


def test_pcmm26_bitexact_vs_oracle(hip_lib):
    """The 26-table PCMM at N=2^16 (24 limbs, dnum 3, 512 diagonals, 16 x 32
    BSGS, 6 fold rotations): input, diagonals, a giant-step key, the
    transform output and the layer output (separate and fused rescale) match
    the oracle's words row for row (SHA-256 digests written by
    tests/golden/make_fullsize_digests.py); the embeddings decrypt within
    2^-20 of the lookup."""
    print("[pcmm] pcmm26 (N=2^16): building", flush=True)
    w = PCMMWorkload(hip_lib, "pcmm26", seed=3, key_seed=17).setup()
    info = w.shape_info()
    print(f"[pcmm] pcmm26: {info}", flush=True)
    assert info["diagonals"] == 512 and info["output_rotations"] == 6
    assert hip_lib.lt_info(list(w.layer.transform_ids.values())[0])["N1"] == 16
    out = check_fullsize_layer(hip_lib, w, fullsize_digests("pcmm26"), "pcmm26")
    y = w.decrypt_output(out)
    err = np.abs(y - w.expected).max()
    print(f"[pcmm] pcmm26: bit-exact; max |decrypted - lookup| = {err:.3e}", flush=True)
    assert err < TOL
    # the fold leaves the output periodic with period 512: slot j+512 decrypts to row j as well
    full = np.asarray(w.scheme.decode(w.scheme.decrypt(out.__class__(w.scheme, out.ids, 2 * 512))))
    assert np.abs(full[512:512 + 416] - w.expected).max() < TOL
    hip_lib.DeleteScheme()


def test_pcmm_two_streams_bitexact(hip_lib):
    """Queries issued back to back on the library's two HIP streams (query i
    on stream i % 2, as bench.py's in-flight measurement issues them), at
    N=2^13: every output equals the same query run alone, word for word, and
    the first equals the restatement's PCMM -- the two streams' buffer caches
    and shared tables never mix one query's work into another's."""
    name = "pcmm26_n13"
    print(f"[pcmm] {name}: two streams", flush=True)
    w = PCMMWorkload(hip_lib, name, seed=3, key_seed=17).setup()
    cts = [w.ct_in] + [w.make_query(1000 + k)[0] for k in range(2)]
    ref = []
    for ct in cts:
        o = w.forward(ct)
        ref.append(hip_lib.export_ciphertext(o.ids[0]))
        o.free()
    outs = []
    for i in range(8):
        hip_lib.SetStream(i % 2)
        outs.append(w.forward(cts[i % len(cts)]))
    hip_lib.SetStream(0)
    hip_lib.JoinStream(1)
    hip_lib.Synchronize()
    for i, o in enumerate(outs):
        assert_equal_u64(hip_lib.export_ciphertext(o.ids[0]), ref[i % len(cts)], f"{name} query {i} on stream {i % 2}")
        o.free()
    c = w.cfg
    orc = O.Oracle(c["logn"], hip_lib.GetModuliChain(), hip_lib.GetAuxModuliChain(), h=c["h"], seed=17)
    try:
        want, _, _ = oracle_pcmm(orc, w.layer.diagonals[(0, 0)], w.layer.output_rotations, w.layer.level, w.selector,
                                 c["logscale"], 0)
    finally:
        orc.close()
    assert_equal_u64(ref[0], want, f"{name} serial output vs the restatement")
    for ct in cts[1:]:
        ct.free()
    hip_lib.DeleteScheme()


def test_sparse_to_top_bitexact_vs_oracle(hip_lib):
    """HELRM.sparse then HELRM.sparse_to_top (dlrm.py:226-230) at N=2^13:
    both layers bit-exact with the restatement, then the 416 embeddings
    decrypt at slots [16, 432) of the top-MLP input within 2^-20."""
    name = "pcmm26_top_n13"
    print(f"[pcmm] {name}: building", flush=True)
    w = SparseToTopWorkload(hip_lib, name, seed=3, key_seed=17).setup()
    info = w.shape_info()
    print(f"[pcmm] {name}: {info}", flush=True)
    assert info["repack"]["diagonals"] == 1 and info["repack"]["output_rotations"] == 3
    out = w.run()
    got = hip_lib.export_ciphertext(out.ids[0])
    c = w.cfg
    orc = O.Oracle(c["logn"], hip_lib.GetModuliChain(), hip_lib.GetAuxModuliChain(), h=c["h"], seed=17)
    try:
        ct1, l1, sc1 = oracle_pcmm(orc, w.layer.diagonals[(0, 0)], w.layer.output_rotations, w.layer.level,
                                   w.selector, c["logscale"], 0)
        assert l1 == w.repack.level
        want, l2, sc2 = oracle_linear(orc, ct1, l1, sc1, w.repack.diagonals[(0, 0)], w.repack.output_rotations,
                                      c["logscale"])
        assert hip_lib.GetCiphertextLevel(out.ids[0]) == l2
        assert hip_lib.GetCiphertextScaleDouble(out.ids[0]) == sc2
        assert_equal_u64(got, want, f"{name} sparse_to_top output")
    finally:
        orc.close()
    y = w.decrypt_output(out)
    err = np.abs(y - w.expected).max()
    print(f"[pcmm] {name}: max |decrypted - expected| = {err:.3e}", flush=True)
    assert err < TOL
    hip_lib.DeleteScheme()


def test_sparse_to_top_full_size_bitexact(hip_lib):
    """HELRM.sparse then HELRM.sparse_to_top at N=2^16 (dlrm.py:226-230): the
    PCMM output and the repack output match the oracle's words row for row
    (SHA-256 digests written by tests/golden/make_fullsize_digests.py); the
    416 embeddings decrypt at slots [16, 432) within 2^-20 and slots [0, 16)
    stay empty."""
    d = fullsize_digests("pcmm26_top")
    print("[pcmm] pcmm26_top (N=2^16): building", flush=True)
    w = SparseToTopWorkload(hip_lib, "pcmm26_top", seed=3, key_seed=17).setup()
    info = w.shape_info()
    print(f"[pcmm] pcmm26_top: {info}", flush=True)
    assert info["repack"]["diagonals"] == 1 and info["repack"]["output_rotations"] == 6
    assert hip_lib.GetModuliChain() == d["q"] and hip_lib.GetAuxModuliChain() == d["p"]
    assert sorted(int(i) for i in w.repack.diagonals[(0, 0)].keys()) == d["repack_diagonals"]
    assert w.repack.output_rotations == d["repack_rotations"]
    emb = w.layer.forward(w.ct_in)
    eid = emb.ids[0]
    assert hip_lib.GetCiphertextLevel(eid) == d["pcmm_out"]["level"]
    assert hip_lib.GetCiphertextScaleDouble(eid) == d["pcmm_out"]["scale"]
    assert_rows_match(hip_lib.export_ciphertext(eid), d["pcmm_out"]["rows"], "pcmm26_top PCMM output")
    out = w.repack.forward(emb)
    emb.free()
    oid = out.ids[0]
    assert hip_lib.GetCiphertextLevel(oid) == d["out"]["level"]
    assert hip_lib.GetCiphertextScaleDouble(oid) == d["out"]["scale"]
    assert_rows_match(hip_lib.export_ciphertext(oid), d["out"]["rows"], "pcmm26_top repack output")
    print("[pcmm] pcmm26_top: PCMM and repack outputs bit-exact", flush=True)
    y = w.decrypt_output(out)
    err = np.abs(y - w.expected).max()
    print(f"[pcmm] pcmm26_top: max |decrypted - expected| = {err:.3e}", flush=True)
    assert err < TOL
    assert np.abs(y[:16]).max() < TOL
    hip_lib.DeleteScheme()


def test_golden_vectors_on_gpu(hip_lib):
    """HIP library vs the committed golden vectors (tests/golden/pcmm_n10.npz)."""
    import os
    from helpers import new_hip_scheme
    from helrm_amd import orion_host as oh
    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "pcmm_n10.npz"))
    q, p = g["q"].tolist(), g["p"].tolist()
    logscale = int(g["logscale"])
    new_hip_scheme(hip_lib, int(g["logn"]), q, p, logscale, int(g["h"]), int(g["seed"]))
    np.testing.assert_array_equal(hip_lib.export_secret_key(), g["secret_key"].astype(np.int64))
    level = len(q) - 1
    S = 1 << (int(g["logn"]) - 1)
    pt = hip_lib.Encode(g["selector"].tolist(), level, 1 << logscale)
    hip_lib.SetEncryptionCounter(0)
    ct = hip_lib.Encrypt(pt)
    assert_equal_u64(hip_lib.export_ciphertext(ct), g["ct_in"], "golden ct_in")
    M = oh.block_diag_matrix([[g["table0"], g["table1"]]])
    d, rots = oh.diagonalize(M, S)
    d = d[(0, 0)]
    idx = list(d.keys())
    assert idx == g["diag_indices"].tolist() and rots == int(g["fold_rotations"])
    tid = hip_lib.GenerateLinearTransform(idx, np.concatenate([d[i] for i in idx]), level, 2.0, "none")
    for ge in hip_lib.GetLinearTransformRotationKeys(tid):
        hip_lib.GenerateLinearTransformRotationKey(ge)
    assert_equal_u64(hip_lib.export_lt_diagonal(tid, idx[0], level), g["diag0_plain"], "golden diagonal")
    out = hip_lib.EvaluateLinearTransform(tid, ct)
    assert_equal_u64(hip_lib.export_ciphertext(out), g["lt_out"], "golden lt_out")
    r = hip_lib.RescaleNew(out)
    assert_equal_u64(hip_lib.export_ciphertext(r), g["rescaled"], "golden rescaled")
    assert_equal_u64(hip_lib.export_ciphertext(hip_lib.RotateNew(ct, 1)), g["rot1"], "golden rot1")
    for i in range(1, rots + 1):
        t = hip_lib.RotateNew(r, S // 2 ** i)
        hip_lib.AddCiphertext(r, t)
    b = hip_lib.Encode([0.0], level - 1, 1 << logscale)
    hip_lib.AddPlaintext(r, b)
    assert_equal_u64(hip_lib.export_ciphertext(r), g["pcmm_out"], "golden pcmm_out")
    hip_lib.DeleteScheme()
