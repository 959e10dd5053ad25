"""End-to-end embedding PCMM on the GPU through the host mirror of Orion's
callers (helrm_amd.orion_host): selector -> encode -> encrypt -> BSGS linear
transform -> rescale -> hybrid fold -> bias -> decrypt -> decode.

* single_table and pcmm26_n13: the output ciphertext is bit-exact with the
  same flow run on the CPU restatement (oracle/).
* every config: decrypted embeddings within 2^-20 of the fp32 plaintext
  lookup (tolerance from the task statement).
"""
import numpy as np
import pytest

from helpers import assert_equal_u64, oracle_pcmm
from oracle import oracle as O
from helrm_amd.workloads import PCMMWorkload

pytestmark = pytest.mark.gpu

TOL = 2.0 ** -20


@pytest.mark.parametrize("name", ["single_table", "pcmm26_n13"])
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


def test_pcmm26_full_size_decrypts(hip_lib):
    print("[pcmm] pcmm26 (N=2^16): building", flush=True)
    w = PCMMWorkload(hip_lib, "pcmm26", seed=3, key_seed=17).setup()
    info = w.shape_info()
    print(f"[pcmm] pcmm26: {info}", flush=True)
    assert info["diagonals"] == 512 and info["output_rotations"] == 6
    assert hip_lib.lt_info(list(w.layer.transform_ids.values())[0])["N1"] == 16
    out = w.run()
    y = w.decrypt_output(out)
    err = np.abs(y - w.expected).max()
    print(f"[pcmm] pcmm26: max |decrypted - lookup| = {err:.3e}", flush=True)
    assert err < TOL
    # the fold leaves the output periodic with period 512: slot j+512 decrypts to row j as well
    full = np.asarray(w.scheme.decode(w.scheme.decrypt(out.__class__(w.scheme, out.ids, 2 * 512))))
    assert np.abs(full[512:512 + 416] - w.expected).max() < TOL
    hip_lib.DeleteScheme()
