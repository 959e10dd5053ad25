"""Blocked linear layers (orion/backend/python/lt_evaluator.py:224-275): a
weight wider than the slot count splits the input over several ciphertexts
and each output block row sums one transform per column block before its
rescale; a square-packed last layer taller than the slot count gives one
output ciphertext per block row (orion/core/packing.py:683-688).  Each output
ciphertext is bit-exact with the same flow on the oracle (transforms, sum
over the column blocks, one rescale, fold, bias), with lt_output_prerescaled
off and on, and decrypts within 2^-20 of W x + b in float64."""
import numpy as np
import pytest

from helpers import assert_equal_u64, make_params
from oracle import oracle as O
from helrm_amd import orion_host as oh

pytestmark = pytest.mark.gpu

LOGN, LOGQ, LOGP, LOGSCALE, H, SEED = 11, [55, 45, 45, 45], [56, 56], 45, 64, 29
TOL = 2.0 ** -20


def oracle_blocked(orc, layer, xs, level, scale):
    """lt_evaluator.evaluate_transforms + linear.py fold and bias on the
    oracle: xs are the input ciphertexts (one per column block)."""
    outs = []
    nbr = max(r for r, _ in layer.diagonals) + 1
    for r in range(nbr):
        acc = None
        for c, x in enumerate(xs):
            d = layer.diagonals[(r, c)]
            idx = list(d.keys())
            t = orc.lt_new(idx, np.stack([d[i] for i in idx]), layer.level, layer.bsgs_ratio)
            y, l = orc.lt_eval(t, x, level)
            orc.lt_free(t)
            acc = y if acc is None else orc.add(acc, y, l)
        out = orc.rescale(acc, l)
        l -= 1
        for i in range(1, layer.output_rotations + 1):
            out = orc.add(out, orc.rotate(out, l, orc.slots // (2 ** i)), l)
        outs.append((out, l))
    return outs


@pytest.mark.parametrize("shape,last", [((200, 2500), False), ((1500, 700), True)],
                         ids=["three_column_blocks", "two_block_rows_square"])
@pytest.mark.parametrize("prerescaled", [False, True])
def test_blocked_linear_bitexact(hip_lib, shape, last, prerescaled):
    q, p = make_params(LOGN, LOGQ, LOGP)
    params = oh.Params(LOGN, LOGQ, LOGP, LOGSCALE, H, seed=SEED)
    scheme = oh.Scheme(params, hip_lib)
    hip_lib.set_lt_output_prerescaled(prerescaled)
    rng = np.random.default_rng(shape[0])
    W = rng.uniform(-0.05, 0.05, shape).astype(np.float32)
    b = rng.uniform(-0.5, 0.5, shape[0]).astype(np.float32)
    x = rng.uniform(-1, 1, shape[1]).astype(np.float32)
    layer = oh.LinearLayer(scheme, W, bias=b, last=last, name=f"blocked{shape[0]}").compile()
    S = params.get_slots()
    nbr, nbc = -(-shape[0] // S), -(-shape[1] // S)
    assert len(layer.diagonals) == nbr * nbc
    print(f"[blocks] {shape} last={last} prerescaled={prerescaled}: {nbr} x {nbc} blocks, "
          f"{sum(len(d) for d in layer.diagonals.values())} diagonals", flush=True)
    hip_lib.SetEncryptionCounter(0)
    ct = scheme.encrypt(scheme.encode(x, layer.level))
    assert len(ct.ids) == nbc
    out = layer.forward(ct)
    assert hip_lib.lt_output_prerescaled == prerescaled
    assert len(out.ids) == nbr
    orc = O.Oracle(LOGN, q, p, h=H, seed=SEED)
    try:
        scale = float(1 << LOGSCALE)
        xs = []
        for j in range(nbc):
            chunk = np.zeros(S, np.float32)
            part = x[j * S:(j + 1) * S]
            chunk[:len(part)] = part
            xs.append(orc.encrypt(orc.encode(chunk, layer.level, scale), layer.level, j))
        want = oracle_blocked(orc, layer, xs, layer.level, scale)
        bias_slots = np.zeros(nbr * S, np.float32)
        bias_slots[:shape[0]] = b
        for r, (w_ct, l) in enumerate(want):
            bp = orc.encode(bias_slots[r * S:(r + 1) * S], l, scale)
            w_ct[0] = orc.add(w_ct[0][None], bp[None], l)[0]
            assert hip_lib.GetCiphertextLevel(out.ids[r]) == l
            assert_equal_u64(hip_lib.export_ciphertext(out.ids[r]), w_ct, f"block row {r}")
    finally:
        orc.close()
    y = scheme.decode(scheme.decrypt(out))
    exp = W.astype(np.float64) @ x.astype(np.float64) + b
    if not last:
        y = y[:shape[0]]
    err = np.abs(np.asarray(y)[:shape[0]] - exp).max()
    print(f"[blocks] max |decrypted - (Wx + b)| = {err:.3e}", flush=True)
    assert err < TOL
    hip_lib.DeleteScheme()
