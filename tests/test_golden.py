"""The CPU restatement still reproduces the committed golden vectors
(tests/golden/pcmm_n10.npz, written by tests/golden/make_golden.py)."""
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def test_oracle_reproduces_golden_vectors():
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(HERE, "golden", "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    ref = np.load(os.path.join(HERE, "golden", "pcmm_n10.npz"))
    now = mg.generate()
    for k in ref.files:
        np.testing.assert_array_equal(np.asarray(now[k]), ref[k], err_msg=k)


def test_golden_pcmm_decrypts_to_lookup():
    """The golden PCMM output is a valid encryption of the table lookup."""
    from oracle import oracle as O
    g = np.load(os.path.join(HERE, "golden", "pcmm_n10.npz"))
    o = O.Oracle(int(g["logn"]), g["q"].tolist(), g["p"].tolist(), h=int(g["h"]), seed=int(g["seed"]))
    try:
        out = g["pcmm_out"]
        level = out.shape[1] - 1
        y = o.decode_f64(o.decrypt(out, level), level, float(1 << int(g["logscale"])))
        assert np.abs(y[:16] - g["expected"]).max() < 2.0 ** -20
    finally:
        o.close()
