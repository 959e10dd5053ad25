"""Synthetic workloads of the encrypted linear-transform path (seeded data).

  single_table  N=2^13, Q=[60,40x4], P=[61], scale 2^40; one table of 256 rows
                x 16 dims, 2 base-16 digit sub-tables U[-0.1, 0.1]
  pcmm26        N=2^16, Q=[60,50x23], P=[61x8] (dnum 3), scale 2^50; 26 tables
                of 4096 rows x 16 dims, 3 base-16 digit sub-tables N(0, 0.05),
                block-diagonally packed so the 416 outputs share one ciphertext
  pcmm26_n13    the pcmm26 structure (26 tables, dnum 3, 512 diagonals) at
                N=2^13 with 9 Q limbs, small enough for the CPU restatement
  pcmm_ragged_n13  HE-LRM's mixed packing at N=2^13: 10 tables of 3 .. 65536
                rows, the ones at or below the compression threshold (16) as
                plain one-hots (FullTable), the others digit-decomposed
                (RadixTable), so the block-diagonal matrix has ragged blocks
  pcmm26_top    pcmm26 followed by HELRM.sparse_to_top (dlrm.py:194-198,
                228): the repacking Linear copy_into(416, 432, 16) at the
                next level, on the same kernels (64 diagonals, 6 fold
                rotations); output slots [16, 432) hold the embeddings
  pcmm26_top_n13  the same two layers at N=2^13
  dense_lt      encrypted dense layer, W 512 outputs x 256 inputs
                U[-1/sqrt(512), 1/sqrt(512)], input 512 values U[-1, 1];
                N=2^16, 16 Q limbs, P=[61x6] (dnum 3): 512 diagonals,
                16 baby x 32 giant steps, 6 fold rotations
  dense_lt_n13  the dense_lt structure at N=2^13

The embedding selector is the digit one-hot of examples/criteo/dlrm.py:202-221,
the plaintext matrix block_diag(W_0..W_25)^T of dlrm.py:241-247 and the
reference lookup the fp32 RadixTable sum (dlrm.py:111-119).  The dense layer
is orion.nn.Linear (orion/nn/linear.py:143-225) on the same path.
"""
import numpy as np

from . import orion_host as oh

CONFIGS = {
    "single_table": dict(kind="pcmm", logn=13, logq=[60, 40, 40, 40, 40], logp=[61], logscale=40, h=192,
                         fields=1, rows=256, dim=16, base=16, init="uniform", init_arg=0.1),
    "pcmm26_n13": dict(kind="pcmm", logn=13, logq=[60] + [50] * 8, logp=[61] * 3, logscale=50, h=192,
                       fields=26, rows=4096, dim=16, base=16, init="normal", init_arg=0.05),
    "pcmm26": dict(kind="pcmm", logn=16, logq=[60] + [50] * 23, logp=[61] * 8, logscale=50, h=192,
                   fields=26, rows=4096, dim=16, base=16, init="normal", init_arg=0.05),
    "pcmm_ragged_n13": dict(kind="pcmm", logn=13, logq=[60] + [50] * 6, logp=[61] * 3, logscale=50, h=192,
                            sizes=[3, 7, 16, 17, 100, 255, 256, 1000, 4096, 65536], threshold=16,
                            dim=16, base=16, init="uniform_bound"),
    "pcmm26_top": dict(kind="pcmm", logn=16, logq=[60] + [50] * 23, logp=[61] * 8, logscale=50, h=192,
                       fields=26, rows=4096, dim=16, base=16, init="normal", init_arg=0.05, repack=(432, 16)),
    "pcmm26_top_n13": dict(kind="pcmm", logn=13, logq=[60] + [50] * 8, logp=[61] * 3, logscale=50, h=192,
                           fields=26, rows=4096, dim=16, base=16, init="normal", init_arg=0.05, repack=(432, 16)),
    "dense_lt": dict(kind="dense", logn=16, logq=[60] + [50] * 15, logp=[61] * 6, logscale=50, h=192,
                     out_features=512, in_features=256, inputs=512),
    "dense_lt_n13": dict(kind="dense", logn=13, logq=[60] + [50] * 15, logp=[61] * 6, logscale=50, h=192,
                         out_features=512, in_features=256, inputs=512),
}


class LinearWorkload:
    """One encrypted linear layer (LT + rescale + fold + bias) on a seeded
    matrix and input vector; subclasses define the data."""

    def __init__(self, backend, name, key_seed):
        c = CONFIGS[name]
        self.name, self.cfg = name, c
        self.params = oh.Params(c["logn"], c["logq"], c["logp"], c["logscale"], c["h"], seed=key_seed)
        self.backend = backend
        self.scheme = None
        self.layer = None
        self.ct_in = None
        self.matrix = None
        self.input = None
        self.expected = None

    def setup(self):
        self.scheme = oh.Scheme(self.params, self.backend)
        self.layer = oh.LinearLayer(self.scheme, self.matrix).compile()
        pt = self.scheme.encode(self.input, self.layer.level)
        self.ct_in = self.scheme.encrypt(pt)
        for i in pt.ids:
            self.backend.DeletePlaintext(i)
        return self

    def run(self):
        """One forward of the layer. Returns the output CipherTensor."""
        return self.layer.forward(self.ct_in)

    def decrypt_output(self, out):
        vals = self.scheme.decode(self.scheme.decrypt(out))
        return vals[: self.matrix.shape[0]]

    def shape_info(self):
        d = self.layer.diagonals[(0, 0)]
        return {"diagonals": len(d), "output_rotations": self.layer.output_rotations,
                "matrix": list(self.matrix.shape), "slots": self.params.get_slots()}


class PCMMWorkload(LinearWorkload):
    """HE-LRM embedding PCMM (HELRM.sparse): digit one-hot selector times the
    block-diagonal table matrix."""

    def __init__(self, backend, name="pcmm26", seed=0, key_seed=1):
        super().__init__(backend, name, key_seed)
        c = self.cfg
        rng = np.random.default_rng(seed)
        base, dim = c["base"], c["dim"]
        sizes = c.get("sizes") or [c["rows"]] * c["fields"]
        threshold = c.get("threshold", 0)
        self.sizes, self.threshold = sizes, threshold
        self.tables = []
        for size in sizes:
            if size <= threshold:
                # FullTable (dlrm.py:85-96): one row per category, plain one-hot selector
                bound = 1.0 / np.sqrt(max(size, 5))
                self.tables.append([rng.uniform(-bound, bound, (size, dim)).astype(np.float32)])
                continue
            # RadixTable (dlrm.py:99-124): one base x dim table per digit
            width = oh.radix_width(size, base)
            if c["init"] == "uniform":
                ts = [rng.uniform(-c["init_arg"], c["init_arg"], (base, dim)).astype(np.float32) for _ in range(width)]
            elif c["init"] == "uniform_bound":
                bound = 1.0 / np.sqrt(size)
                ts = [rng.uniform(-bound, bound, (base, dim)).astype(np.float32) for _ in range(width)]
            else:
                ts = [rng.normal(0.0, c["init_arg"], (base, dim)).astype(np.float32) for _ in range(width)]
            self.tables.append(ts)
        self.indices = np.array([rng.integers(0, s) for s in sizes])
        self.fields = len(sizes)
        self.selector = oh.expanded_sparse(self.indices, sizes, threshold, base)
        self.input = self.selector
        self.matrix = oh.block_diag_matrix(self.tables)
        self.expected = np.concatenate([
            t[0][int(i)] if s <= threshold else oh.radix_lookup(t, int(i), base)
            for t, i, s in zip(self.tables, self.indices, sizes)])


class SparseToTopWorkload(PCMMWorkload):
    """HELRM.sparse then HELRM.sparse_to_top (dlrm.py:226-230): the embedding
    PCMM and the repacking Linear copy_into(416, 432, 16), compiled one level
    below it, evaluated back to back on the same kernels."""

    def __init__(self, backend, name="pcmm26_top", seed=0, key_seed=1):
        super().__init__(backend, name, seed=seed, key_seed=key_seed)
        out_width, start = self.cfg["repack"]
        width = self.matrix.shape[0]
        self.repack_matrix = oh.copy_into(width, out_width, start)
        self.lookup = self.expected
        self.expected = np.zeros(out_width, dtype=np.float64)
        self.expected[start:start + width] = self.lookup
        self.repack = None

    def setup(self):
        super().setup()
        self.repack = oh.LinearLayer(self.scheme, self.repack_matrix, level=self.layer.level - 1).compile()
        return self

    def run(self):
        emb = self.layer.forward(self.ct_in)
        out = self.repack.forward(emb)
        emb.free()
        return out

    def decrypt_output(self, out):
        vals = self.scheme.decode(self.scheme.decrypt(out))
        return vals[: self.repack_matrix.shape[0]]

    def shape_info(self):
        info = super().shape_info()
        info["repack"] = {"diagonals": len(self.repack.diagonals[(0, 0)]),
                          "output_rotations": self.repack.output_rotations,
                          "matrix": list(self.repack_matrix.shape)}
        return info


class DenseLTWorkload(LinearWorkload):
    """Encrypted dense layer y = W x (orion.nn.Linear without bias)."""

    def __init__(self, backend, name="dense_lt", seed=0, key_seed=1):
        super().__init__(backend, name, key_seed)
        c = self.cfg
        rng = np.random.default_rng(seed)
        bound = 1.0 / np.sqrt(c["out_features"])
        self.matrix = rng.uniform(-bound, bound, (c["out_features"], c["in_features"])).astype(np.float32)
        self.input = rng.uniform(-1.0, 1.0, c["inputs"]).astype(np.float32)
        self.expected = self.matrix.astype(np.float64) @ self.input[: c["in_features"]].astype(np.float64)


def make_workload(backend, name, seed=0, key_seed=1):
    c = CONFIGS[name]
    if c["kind"] == "pcmm":
        cls = SparseToTopWorkload if c.get("repack") else PCMMWorkload
    else:
        cls = DenseLTWorkload
    return cls(backend, name, seed=seed, key_seed=key_seed)
