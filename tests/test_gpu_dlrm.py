"""Encrypted HE-LRM forward (examples/criteo/dlrm.py:181-231) on the GPU:
bottom MLP, embedding PCMM, both repacking Linears, Add and top MLP with
degree-3 activations, on a 30-limb chain without bootstrapping.

* dlrm_n13: every layer's output ciphertext is bit-exact with the same flow
  on the CPU restatement (oracle/), which itself decrypts to the cleartext
  model.
* dlrm (N=2^16): every layer's output ciphertext, both inputs and a
  relinearised product match the oracle's per-row SHA-256 digests
  (tests/golden/make_fullsize_digests.py: the same flow on the CPU
  restatement), with the transforms' rescale separate and fused; the
  decrypted logit is within 2^-20 of the float64 cleartext forward on the
  same fp32 weights.
"""
import numpy as np
import pytest

from helpers import assert_equal_u64, assert_rows_match, fullsize_digests, oracle_dlrm
from oracle import oracle as O
from helrm_amd.workloads import DLRMWorkload

pytestmark = pytest.mark.gpu

TOL = 2.0 ** -20


@pytest.mark.parametrize("prerescale", [False, True])
def test_dlrm_n13_bitexact_vs_oracle(hip_lib, prerescale):
    """prerescale: every Linear's transform returns its rescaled result
    (lt_output_prerescaled) -- the same residues layer by layer."""
    name = "dlrm_n13"
    print(f"[dlrm] {name} prerescale={prerescale}: building", flush=True)
    w = DLRMWorkload(hip_lib, name, seed=3, key_seed=17).setup()
    hip_lib.set_lt_output_prerescaled(prerescale)
    print(f"[dlrm] {name}: {w.shape_info()}", flush=True)
    out, kept = w.run_stages(keep=True)
    got = {n: (hip_lib.export_ciphertext(t.ids[0]), hip_lib.GetCiphertextLevel(t.ids[0]),
               hip_lib.GetCiphertextScaleDouble(t.ids[0])) for n, t in kept.items()}
    y = w.decrypt_output(out)
    c = w.cfg
    print(f"[dlrm] {name}: running the restatement", flush=True)
    orc = O.Oracle(c["logn"], hip_lib.GetModuliChain(), hip_lib.GetAuxModuliChain(), h=c["h"], seed=17)
    try:
        (want, l, sc), trace = oracle_dlrm(orc, w, keep=True)
        clear = w.clear_trace()
        for n, (ct, lv, s) in trace.items():
            g, glv, gs = got[n]
            assert glv == lv and gs == s, f"{n}: level/scale {glv}/{gs} vs {lv}/{s}"
            assert_equal_u64(g, ct, f"{name} {n} output")
            ref = clear[n]
            dec = orc.decode_f64(orc.decrypt(ct, lv), lv, s)[: len(ref)]
            assert np.abs(dec - ref).max() < TOL, n
        print(f"[dlrm] {name}: {len(trace)} layer outputs bit-exact", flush=True)
        # the lookup path on the second stream beside the bottom MLP (run()),
        # twice, so that the second forward reuses buffers both streams freed
        final = w.top_names[-1][1]
        want_ct, want_l, want_s = trace[final]
        w.concurrent = True
        for rep in range(2):
            o = w.run()
            assert hip_lib.GetCiphertextLevel(o.ids[0]) == want_l
            assert hip_lib.GetCiphertextScaleDouble(o.ids[0]) == want_s
            assert_equal_u64(hip_lib.export_ciphertext(o.ids[0]), want_ct, f"{name} concurrent forward {rep}")
            o.free()
    finally:
        orc.close()
    err = np.abs(y - w.expected).max()
    print(f"[dlrm] {name}: logit {y[0]:.9f} vs {w.expected[0]:.9f} (|err| {err:.3e})", flush=True)
    assert err < TOL
    for t in kept.values():
        t.free()
    hip_lib.DeleteScheme()


def test_dlrm_full_size_bitexact(hip_lib):
    d = fullsize_digests("dlrm")
    print("[dlrm] dlrm (N=2^16): building", flush=True)
    w = DLRMWorkload(hip_lib, "dlrm", seed=d["workload_seed"], key_seed=d["key_seed"]).setup()
    info = w.shape_info()
    print(f"[dlrm] dlrm: {info}", flush=True)
    assert info["bottom.0"]["diagonals"] == 512 and info["sparse"]["diagonals"] == 512
    assert info["top.4"]["output_rotations"] == 0
    assert hip_lib.GetModuliChain() == d["q"] and hip_lib.GetAuxModuliChain() == d["p"]
    assert w.input_level == d["input_level"]
    assert_rows_match(hip_lib.export_ciphertext(w.ct_dense.ids[0]), d["ct_dense"], "dense input")
    assert_rows_match(hip_lib.export_ciphertext(w.ct_sparse.ids[0]), d["ct_sparse"], "selector input")
    # a relinearised product at the input level (evaluator.go:343-364)
    prod = hip_lib.MulRelinCiphertextNew(w.ct_dense.ids[0], w.ct_sparse.ids[0])
    assert hip_lib.GetCiphertextLevel(prod) == d["mul_relin"]["level"]
    assert_rows_match(hip_lib.export_ciphertext(prod), d["mul_relin"]["rows"], "relinearised product")
    hip_lib.DeleteCiphertext(prod)
    for pre in (True, False):
        hip_lib.set_lt_output_prerescaled(pre)
        print(f"[dlrm] dlrm: layer by layer, prerescale={pre}", flush=True)
        out, kept = w.run_stages(keep=True)
        assert set(kept) == set(d["layers"])
        for n, t in kept.items():
            want = d["layers"][n]
            cid = t.ids[0]
            assert hip_lib.GetCiphertextLevel(cid) == want["level"], n
            assert hip_lib.GetCiphertextScaleDouble(cid) == want["scale"], n
            assert_rows_match(hip_lib.export_ciphertext(cid), want["rows"], f"{n} output (prerescale {pre})")
        for t in kept.values():
            t.free()
    print(f"[dlrm] dlrm: {len(d['layers'])} layer outputs match the oracle", flush=True)
    assert w.concurrent  # run(): the lookup path on the second stream
    hip_lib.set_lt_output_prerescaled(True)
    final = d["layers"][w.top_names[-1][1]]
    for rep in range(2):  # the second reuses the buffers both streams freed
        out = w.run()
        assert_rows_match(hip_lib.export_ciphertext(out.ids[0]), final["rows"], f"concurrent forward {rep}")
        if rep == 0:
            out.free()
    assert hip_lib.GetCiphertextLevel(out.ids[0]) == 0
    y = w.decrypt_output(out)
    err = np.abs(y - w.expected).max()
    print(f"[dlrm] dlrm: logit {y[0]:.9f} vs {w.expected[0]:.9f} (|err| {err:.3e})", flush=True)
    assert err < TOL
    assert abs(float(y[0]) - d["logit"]) < TOL
    # the square-packed last layer leaves no partial sums in the other slots
    full = np.asarray(w.scheme.decode(w.scheme.decrypt(out.__class__(w.scheme, out.ids, 4096))))
    assert np.abs(full[1:]).max() < TOL
    hip_lib.DeleteScheme()


def test_dlrm_n13_seeded_upload_concurrent(hip_lib):
    """The selector uploaded as (b, seed) (bench_sweep.py:381-403): every
    forward rebuilds `a` on the device -- on the second stream when the lookup
    path runs beside the bottom MLP.  Concurrent and one-stream forwards give
    the same words, twice each."""
    w = DLRMWorkload(hip_lib, "dlrm_n13", seed=5, key_seed=17).setup()
    hip_lib.set_lt_output_prerescaled(True)
    w.use_seeded_upload(0x5EED)
    outs = []
    for concurrent in (False, True, False, True):
        w.concurrent = concurrent
        o = w.run()
        outs.append(hip_lib.export_ciphertext(o.ids[0]))
        if concurrent:
            assert np.abs(w.decrypt_output(o) - w.expected).max() < TOL
        o.free()
    for i, g in enumerate(outs[1:], 1):
        assert_equal_u64(g, outs[0], f"seeded-upload forward {i}")
    hip_lib.DeleteScheme()
