"""Host-side callers (helrm_amd.orion_host) against the reference's
documented examples and against plain numpy algebra."""
import math

import numpy as np
import pytest

from helrm_amd import orion_host as oh


def test_diagonalize_docstring_example():
    """orion/core/packing.py:653-686 docstring: 4x4 matrix, slots=4 and 2."""
    M = np.arange(16, dtype=np.float32).reshape(4, 4)
    d, r = oh.diagonalize(M, 4, "square")
    assert r == 0
    assert {k: v.tolist() for k, v in d[(0, 0)].items()} == {
        0: [0., 5., 10., 15.], 1: [1., 6., 11., 12.], 2: [2., 7., 8., 13.], 3: [3., 4., 9., 14.]}
    d2, _ = oh.diagonalize(M, 2, "square")
    assert {k: v.tolist() for k, v in d2[(0, 0)].items()} == {0: [0., 5.], 1: [1., 4.]}
    assert {k: v.tolist() for k, v in d2[(0, 1)].items()} == {0: [2., 7.], 1: [3., 6.]}
    assert {k: v.tolist() for k, v in d2[(1, 0)].items()} == {0: [8., 13.], 1: [9., 12.]}
    assert {k: v.tolist() for k, v in d2[(1, 1)].items()} == {0: [10., 15.], 1: [11., 14.]}


@pytest.mark.parametrize("H,W,S", [(16, 32, 4096), (416, 1248, 32768), (10, 7, 64)])
def test_hybrid_diagonals_and_fold_compute_matvec(H, W, S):
    """sum_i diag_i[j] * x[(i+j) mod S], then the fold sum_k y[j + k*bh] == (M x)[j]."""
    rng = np.random.default_rng(H)
    M = rng.standard_normal((H, W)).astype(np.float32)
    x = np.zeros(S)
    x[:W] = rng.standard_normal(W)
    d, rots = oh.diagonalize(M, S, "hybrid", False)
    bh = 2 ** math.ceil(math.log2(H))
    assert rots == int(math.log2(S // bh))
    y = np.zeros(S)
    for i, v in d[(0, 0)].items():
        y += v.astype(np.float64) * np.roll(x, -i)
    for i in range(1, rots + 1):
        y = y + np.roll(y, -(S // 2 ** i))
    np.testing.assert_allclose(y[:H], M.astype(np.float64) @ x[:W], rtol=1e-5, atol=1e-4)
    np.testing.assert_allclose(y[bh:bh + H], y[:H])


def test_pcmm26_shapes():
    """512 nonzero diagonals, 6 fold rotations for 26 x (48 -> 16) blocks at 2^15 slots."""
    from helrm_amd.workloads import PCMMWorkload
    w = PCMMWorkload(None, "pcmm26", seed=0)
    d, r = oh.diagonalize(w.matrix, 32768)
    assert len(d[(0, 0)]) == 512 and r == 6
    assert w.matrix.shape == (416, 1248)
    assert w.selector.sum() == 26 * 3
    np.testing.assert_allclose(w.matrix @ w.selector, w.expected, atol=1e-6)


@pytest.mark.parametrize("S", [4096, 32768])
def test_sparse_to_top_repack(S):
    """HELRM.sparse_to_top = copy_into(416, 432, 16) (dlrm.py:174-178, 194-198):
    the hybrid packing keeps diagonals i < 512 only, so the shift by 16 is the
    single diagonal 512 - 16, nonzero in the last 512-slot block alone (the
    fold adds the blocks); log2(S/512) fold rotations; on the periodic PCMM
    output layout (slot j holds row j mod 512, rows >= 416 zero) the LT + fold
    puts the 416 embeddings at slots [16, 432)."""
    W = oh.copy_into(416, 432, 16)
    assert W.shape == (432, 416) and W[16:, :].trace() == 416 and W.sum() == 416
    d, rots = oh.diagonalize(W, S, "hybrid", False)
    assert rots == int(math.log2(S // 512))
    assert list(d[(0, 0)]) == [496]
    nz = np.nonzero(d[(0, 0)][496])[0]
    assert nz.min() == S - 512 + 16 and nz.max() == S - 512 + 431 and len(nz) == 416
    rng = np.random.default_rng(S)
    emb = rng.standard_normal(416)
    x = np.zeros(S)
    for k in range(S // 512):
        x[512 * k:512 * k + 416] = emb
    y = np.zeros(S)
    for i, v in d[(0, 0)].items():
        y += v.astype(np.float64) * np.roll(x, -i)
    for i in range(1, rots + 1):
        y = y + np.roll(y, -(S // 2 ** i))
    want = np.zeros(432)
    want[16:] = emb
    np.testing.assert_allclose(y[:432], want, atol=1e-12)


def test_digits_and_selector():
    """examples/criteo/dlrm.py:66-82, 202-221."""
    assert oh.digits(201, 16, 2).tolist() == [9, 12]
    assert oh.digits(4095, 16, 3).tolist() == [15, 15, 15]
    assert oh.radix_width(4096, 16) == 3 and oh.radix_width(256, 16) == 2
    assert oh.expanded_width(4096, 20000, 16) == 4096 and oh.expanded_width(4096, 100, 16) == 48
    sel = oh.expanded_id(201, 256, 0, 16)
    assert sel.shape == (32,) and sel[9] == 1 and sel[16 + 12] == 1 and sel.sum() == 2
    plain = oh.expanded_id(3, 10, 20000, 16)
    assert plain.tolist() == [0, 0, 0, 1, 0, 0, 0, 0, 0, 0]


def test_radix_lookup_is_block_matrix_product():
    rng = np.random.default_rng(2)
    tabs = [[rng.standard_normal((16, 16)).astype(np.float32) for _ in range(3)] for _ in range(4)]
    idx = [5, 4095, 0, 1234]
    M = oh.block_diag_matrix(tabs)
    sel = oh.expanded_sparse(idx, [4096] * 4, 0, 16)
    want = np.concatenate([oh.radix_lookup(t, i, 16) for t, i in zip(tabs, idx)])
    np.testing.assert_allclose(M @ sel, want, atol=1e-5)


def test_encode_padding_matches_orion():
    """orion/backend/python/encoder.py:70-85: zero-pad to a multiple of slots."""
    class B:
        def __init__(self):
            self.calls = []

        def Encode(self, vals, level, scale):
            self.calls.append((len(vals), level, scale))
            return len(self.calls) - 1
    s = oh.Scheme.__new__(oh.Scheme)
    s.params = oh.Params(13, [60, 40], [61], 40)
    s.backend = B()
    pt = s.encode(np.ones(5000), 1)
    assert [c[0] for c in s.backend.calls] == [4096, 4096] and pt.n == 5000
    assert s.backend.calls[0][2] == 1 << 40


def test_ragged_selector_and_matrix():
    """Mixed FullTable / RadixTable packing (dlrm.py:85-124, 202-221, 241-247):
    the block-diagonal matrix times the selector is the fp32 lookup."""
    from helrm_amd.workloads import PCMMWorkload
    w = PCMMWorkload(None, "pcmm_ragged_n13", seed=5)
    widths = [oh.expanded_width(s, w.threshold, 16) for s in w.sizes]
    assert widths == [3, 7, 16, 32, 32, 32, 32, 48, 48, 64]
    assert w.matrix.shape == (16 * len(w.sizes), sum(widths)) and len(w.selector) == sum(widths)
    assert w.selector.sum() == sum(1 if s <= 16 else oh.radix_width(s, 16) for s in w.sizes)
    np.testing.assert_allclose(w.matrix.astype(np.float64) @ w.selector, w.expected, atol=1e-6)
    d, r = oh.diagonalize(w.matrix, 4096)
    assert r == 4  # block height 256 for 160 outputs


def test_dlrm_levels_follow_orion_solver():
    """Lowest-cost level plan of orion/core/auto_bootstrap.py for HE-LRM with
    no bootstrap: linear layers cost level x diagonals (level_dag.py:167-197),
    activations nothing, so the chain is tight and ends at level 0; the
    degree-3 activations take 2 levels (activation.py:23-25)."""
    from helrm_amd.workloads import DLRMWorkload
    w = DLRMWorkload(None, "dlrm", seed=0)
    assert w.levels == {"bottom.0": 20, "bottom.1": 19, "bottom.2": 17, "bottom.3": 16, "bottom.4": 14,
                        "bottom.5": 13, "bottom.6": 11, "bottom.7": 10, "bottom_to_top": 8,
                        "sparse": 9, "sparse_to_top": 8,
                        "top.0": 7, "top.1": 6, "top.2": 4, "top.3": 3, "top.4": 1}
    assert w.input_level == 20 and w.add_level == 7
    assert w.input_level < len(w.cfg["logq"])


@pytest.mark.parametrize("name", ["dlrm_n13", "dlrm"])
def test_dlrm_slot_algebra_matches_cleartext(name):
    """The encrypted forward's slot algebra in float64 -- hybrid diagonals and
    fold (periodic copies without bias), bias in the first rows only, the
    activation on every slot, square packing for the last Linear
    (orion/core/orion.py:255-285) -- gives the cleartext model on the live
    rows of every layer, and zeros outside slot 0 at the end."""
    from helrm_amd.workloads import DLRMWorkload
    w = DLRMWorkload(None, name, seed=1)
    S = 1 << (w.cfg["logn"] - 1)
    clear = w.clear_trace()

    def linear(x, W, b=None, last=False):
        d, rots = oh.diagonalize(W, S, "hybrid", last)
        y = np.zeros(S)
        for i, v in d[(0, 0)].items():
            y += v.astype(np.float64) * np.roll(x, -i)
        for i in range(1, rots + 1):
            y = y + np.roll(y, -(S // 2 ** i))
        if b is not None:
            y[:len(b)] += b
        return y
    x = np.zeros(S)
    x[:13] = w.dense
    for k, (W, b) in enumerate(w.bottom_w):
        x = linear(x, W, b)
        np.testing.assert_allclose(x[:W.shape[0]], clear[f"bottom.{2 * k}"], atol=1e-12)
        x = w.act(x)
    x = linear(x, w.bottom_to_top_w)
    e = np.zeros(S)
    e[:len(w.emb.selector)] = w.emb.selector
    e = linear(linear(e, w.emb.matrix), w.sparse_to_top_w)
    z = x + e
    np.testing.assert_allclose(z[:432], clear["add"], atol=1e-12)
    for k, (W, b) in enumerate(w.top_w):
        last = k == len(w.top_w) - 1
        z = linear(z, W, b, last)
        np.testing.assert_allclose(z[:W.shape[0]], clear[f"top.{2 * k}"], atol=1e-12)
        if not last:
            z = w.act(z)
    assert abs(z[0] - w.expected[0]) < 1e-12
    assert np.abs(z[1:]).max() < 1e-12


def test_wire_store_round_trip(tmp_path):
    """The io_mode stores persist byte blobs as a .npz of uint8 arrays and read
    them back without unpickling."""
    path = str(tmp_path / "keys.npz")
    st = oh.WireStore(path)
    blobs = {"sk": np.arange(40, dtype=np.uint8), "5": np.frombuffer(b"\x00\xff" * 9, dtype=np.uint8),
             "sparse/0_0/17": np.zeros(0, dtype=np.uint8)}
    for k, v in blobs.items():
        st[k] = v
    st.flush()
    back = oh.WireStore(path)
    assert set(back.keys()) == set(blobs)
    for k, v in blobs.items():
        np.testing.assert_array_equal(back[k], v)
        assert back[k].dtype == np.uint8


@pytest.mark.parametrize("n,slots", [(10, 4), (8, 4), (3, 4), (4096 * 3 - 5, 4096)])
def test_pack_lanes_pairs_chunks(n, slots):
    """lane_packing.py:42-81: chunk 2m in the real lane, chunk 2m+1 in the
    imaginary lane of packed chunk m, pre-scaled by 0.5; an odd chunk count is
    padded with a zero partner; p + conj(p) and -i (p - conj(p)) give the chunks
    back."""
    v = np.random.default_rng(n).uniform(-1, 1, n)
    packed, nreal = oh.pack_lanes(v, slots)
    assert nreal == -(-n // slots)
    assert oh.plan_packing(n, slots) == (nreal, -(-nreal // 2))
    assert len(packed) == -(-nreal // 2) * slots
    flat = np.concatenate([v, np.zeros(-(-nreal // 2) * 2 * slots - n)])
    for m in range(len(packed) // slots):
        p = packed[m * slots:(m + 1) * slots]
        np.testing.assert_allclose(p + np.conj(p), flat[2 * m * slots:(2 * m + 1) * slots], atol=1e-15)
        np.testing.assert_allclose((-1j * (p - np.conj(p))).real, flat[(2 * m + 1) * slots:(2 * m + 2) * slots], atol=1e-15)
