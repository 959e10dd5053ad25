"""The reference's BSGS linear-transform tests (tests/test_bsgs_linear_transform.py)
on the HIP library, each output ciphertext bit-exact with the oracle's
transform + rescale and decrypted within the reference's own tolerance of
the cleartext sum  expected[i] = sum_k w_k * x[(i + d_k) mod slots].

Parameters are the reference's (test_bsgs_linear_transform.py:18-26): N=2^13,
LogQ [29, 26, 26, 26], LogP [29], LogScale 26, H 8192, on the standard ring
(4096 slots; the reference uses the ConjugateInvariant ring, which this
library does not implement).  bsgs_ratio 2 as BSGS_RATIO (line 33); the
naive path of the consistency case is Lattigo's LogBabyStepGiantStepRatio < 0
(ratio 0.1 -> int(ln 0.1) = -2), the reference's "none".

The stress sets give 26 / 31 / 55 baby steps (Lattigo's FindBestBSGSRatio at
4096 slots): the 55-step set runs the diagonal MAC in two chunks (32 + 23
baby steps, the second accumulating into the first's output).  At 4096
slots and ratio 2 a transform cannot have more than 64 baby steps, so one
more case uses bsgs_ratio 8 (int(ln 8) = 2, giant:baby up to 1:4) on a
structured set with 100 baby steps (four chunks)."""
import numpy as np
import pytest

from helpers import assert_equal_u64, make_params, new_hip_scheme
from oracle import oracle as O

pytestmark = pytest.mark.gpu

LOGN, LOGQ, LOGP, LOGSCALE, H, SEED = 13, [29, 26, 26, 26], [29], 26, 8192, 23
BSGS_RATIO = 2.0


class Ctx:
    def __init__(self, lib):
        self.lib = lib
        self.q, self.p = make_params(LOGN, LOGQ, LOGP)
        self.slots = 1 << (LOGN - 1)
        self.level = len(self.q) - 1
        new_hip_scheme(lib, LOGN, self.q, self.p, LOGSCALE, H, SEED)
        self.orc = O.Oracle(LOGN, self.q, self.p, h=H, seed=SEED)
        self.enc = 0

    def run(self, idx, weights, values, ratio=BSGS_RATIO, per_slot=None):
        """GenerateLinearTransform + EvaluateLinearTransform + Rescale on both
        sides; returns (decoded output, LT info)."""
        S, lib, orc = self.slots, self.lib, self.orc
        data = (np.repeat(np.asarray(weights, np.float32)[:, None], S, axis=1) if per_slot is None
                else np.asarray(per_slot, np.float32))
        values = np.asarray(values, np.float32)
        tid = lib.GenerateLinearTransform(list(idx), data.reshape(-1), self.level, ratio, "none")
        for ge in lib.GetLinearTransformRotationKeys(tid):
            lib.GenerateLinearTransformRotationKey(ge)
        info = lib.lt_info(tid)
        pt = lib.Encode(values.tolist(), self.level, 1 << LOGSCALE)
        lib.SetEncryptionCounter(self.enc)
        ct = lib.Encrypt(pt)
        out = lib.Rescale(lib.EvaluateLinearTransform(tid, ct))
        got = lib.export_ciphertext(out)
        t = orc.lt_new(list(idx), data, self.level, ratio)
        assert orc.lt_n1(t) == info["N1"]
        ref = orc.encrypt(orc.encode(values, self.level, float(1 << LOGSCALE)), self.level, self.enc)
        want, l = orc.lt_eval(t, ref, self.level)
        want = orc.rescale(want, l)
        orc.lt_free(t)
        self.enc += 1
        assert_equal_u64(got, want, f"transform of {len(idx)} diagonals (N1={info['N1']})")
        res = np.asarray(lib.Decode(lib.Decrypt(out)), np.float64)
        lib.DeleteLinearTransform(tid)
        return res, info


def expected_sum(values, idx, weights, slots):
    x = np.asarray(values, np.float64)
    out = np.zeros(slots)
    for d, w in zip(idx, weights):
        out += float(np.float32(w)) * np.roll(x, -d)
    return out


@pytest.fixture(scope="module")
def ctx(hip_lib):
    c = Ctx(hip_lib)
    print(f"[bsgs] N=2^{LOGN} Q={c.q} P={c.p}", flush=True)
    yield c
    c.orc.close()
    hip_lib.DeleteScheme()


def close(res, exp, atol):
    err = np.abs(np.asarray(res)[: len(exp)] - exp).max()
    assert err <= atol, f"max error {err} > {atol}"


def test_identity_bsgs(ctx):
    vals = np.arange(1, ctx.slots + 1, dtype=np.float64)
    res, _ = ctx.run([0], [1.0], vals)
    close(res, vals, 1e-1)


def test_scale_by_constant_bsgs(ctx):
    vals = np.arange(1, ctx.slots + 1, dtype=np.float64)
    res, _ = ctx.run([0], [3.0], vals)
    close(res, 3.0 * vals, 5e-1)


def test_cyclic_permutation_bsgs(ctx):
    vals = np.arange(1, ctx.slots + 1, dtype=np.float64)
    res, _ = ctx.run([3], [1.0], vals)
    close(res, np.roll(vals, -3), 1e-1)


def test_multi_diagonal_bsgs(ctx):
    vals = np.arange(1, ctx.slots + 1, dtype=np.float64)
    res, _ = ctx.run([0, 1], [1.0, 1.0], vals)
    close(res, vals + np.roll(vals, -1), 5e-1)


def test_many_diagonals_bsgs(ctx):
    vals = np.arange(1, ctx.slots + 1, dtype=np.float64)
    idx = [0, 1, 2, 3, 5, 7, 9, 11]
    w = [0.5, -0.3, 0.2, 0.1, -0.4, 0.6, -0.2, 0.3]
    res, info = ctx.run(idx, w, vals)
    close(res, expected_sum(vals, idx, w, ctx.slots), 5e-1)


@pytest.mark.parametrize("num_diags,babies", [(50, 26), (100, 31), (144, 55)])
def test_stress_many_diagonals_bsgs(ctx, num_diags, babies):
    rng = np.random.default_rng(seed=42 + num_diags)
    vals = np.array([float(i % 17) * 0.1 for i in range(ctx.slots)])
    idx = sorted(rng.choice(ctx.slots, size=num_diags, replace=False).tolist())
    w = rng.uniform(-0.5, 0.5, size=num_diags).tolist()
    print(f"[bsgs] stress {num_diags} diagonals", flush=True)
    res, info = ctx.run(idx, w, vals)
    assert info["baby"] == babies
    close(res, expected_sum(vals, idx, w, ctx.slots), 1.0)


def test_bsgs_vs_naive_consistency(ctx):
    rng = np.random.default_rng(seed=99)
    vals = np.array([float(i % 13) * 0.2 for i in range(ctx.slots)])
    idx = sorted(rng.choice(ctx.slots, size=30, replace=False).tolist())
    w = rng.uniform(-0.3, 0.3, size=30).tolist()
    r_bsgs, i_bsgs = ctx.run(idx, w, vals)
    r_naive, i_naive = ctx.run(idx, w, vals, ratio=0.1)
    assert i_bsgs["N1"] > 0 and i_naive["N1"] == 0
    close(r_bsgs, r_naive, 1.0)
    close(r_bsgs, expected_sum(vals, idx, w, ctx.slots), 1.0)


def test_more_than_64_baby_steps(ctx):
    """100 baby steps x 26 giant steps (N1 = 128): the diagonal MAC runs four
    chunks of at most 32 baby steps, the later ones accumulating; per-slot
    diagonal values so that a misplaced diagonal or rotation shows."""
    idx = sorted(set(range(100)) | {128 * j for j in range(26)})
    rng = np.random.default_rng(7)
    data = rng.uniform(-0.05, 0.05, (len(idx), ctx.slots))
    vals = rng.uniform(-1, 1, ctx.slots)
    res, info = ctx.run(idx, None, vals, ratio=8.0, per_slot=data)
    assert (info["N1"], info["giant"], info["baby"]) == (128, 26, 100)
    x = vals.astype(np.float32).astype(np.float64)
    exp = np.zeros(ctx.slots)
    for k, d in enumerate(idx):
        exp += data[k].astype(np.float32).astype(np.float64) * np.roll(x, -d)
    close(res, exp, 1.0)
