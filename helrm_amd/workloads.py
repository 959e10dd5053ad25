"""Synthetic HE-LRM embedding-PCMM workloads (seeded tables and indices).

  single_table  N=2^13, Q=[60,40x4], P=[61], scale 2^40; one table of 256 rows
                x 16 dims, 2 base-16 digit sub-tables U[-0.1, 0.1]
  pcmm26        N=2^16, Q=[60,50x23], P=[61x8] (dnum 3), scale 2^50; 26 tables
                of 4096 rows x 16 dims, 3 base-16 digit sub-tables N(0, 0.05),
                block-diagonally packed so the 416 outputs share one ciphertext

The selector is the digit one-hot of examples/criteo/dlrm.py:202-221, the
plaintext matrix block_diag(W_0..W_25)^T of dlrm.py:241-247, and the
reference lookup the fp32 RadixTable sum (dlrm.py:111-119).
"""
import numpy as np

from . import orion_host as oh

CONFIGS = {
    "single_table": dict(logn=13, logq=[60, 40, 40, 40, 40], logp=[61], logscale=40, h=192,
                         fields=1, rows=256, dim=16, base=16, init="uniform", init_arg=0.1),
    # same structure as pcmm26 (26 tables, dnum 3, 512 diagonals) at N=2^13, small
    # enough for the CPU restatement to check bit for bit
    "pcmm26_n13": dict(logn=13, logq=[60] + [50] * 8, logp=[61] * 3, logscale=50, h=192,
                       fields=26, rows=4096, dim=16, base=16, init="normal", init_arg=0.05),
    "pcmm26": dict(logn=16, logq=[60] + [50] * 23, logp=[61] * 8, logscale=50, h=192,
                   fields=26, rows=4096, dim=16, base=16, init="normal", init_arg=0.05),
}


class PCMMWorkload:
    def __init__(self, backend, name="pcmm26", seed=0, key_seed=1):
        c = CONFIGS[name]
        self.name, self.cfg = name, c
        self.params = oh.Params(c["logn"], c["logq"], c["logp"], c["logscale"], c["h"], seed=key_seed)
        rng = np.random.default_rng(seed)
        width = oh.radix_width(c["rows"], c["base"])
        self.width = width
        self.tables = []
        for _ in range(c["fields"]):
            if c["init"] == "uniform":
                ts = [rng.uniform(-c["init_arg"], c["init_arg"], (c["base"], c["dim"])).astype(np.float32) for _ in range(width)]
            else:
                ts = [rng.normal(0.0, c["init_arg"], (c["base"], c["dim"])).astype(np.float32) for _ in range(width)]
            self.tables.append(ts)
        self.indices = rng.integers(0, c["rows"], c["fields"])
        sizes = [c["rows"]] * c["fields"]
        # every table is above the compression threshold: digit one-hots
        self.selector = oh.expanded_sparse(self.indices, sizes, 0, c["base"])
        self.matrix = oh.block_diag_matrix(self.tables)
        self.expected = np.concatenate([oh.radix_lookup(t, int(i), c["base"]) for t, i in zip(self.tables, self.indices)])
        self.backend = backend
        self.scheme = None
        self.layer = None
        self.ct_in = None

    def setup(self):
        self.scheme = oh.Scheme(self.params, self.backend)
        self.layer = oh.LinearLayer(self.scheme, self.matrix).compile()
        pt = self.scheme.encode(self.selector, self.layer.level)
        self.ct_in = self.scheme.encrypt(pt)
        for i in pt.ids:
            self.backend.DeletePlaintext(i)
        return self

    def run(self):
        """One PCMM (HELRM.sparse): LT + rescale + fold + bias. Returns the output CipherTensor."""
        return self.layer.forward(self.ct_in)

    def decrypt_output(self, out):
        vals = self.scheme.decode(self.scheme.decrypt(out))
        return vals[: self.matrix.shape[0]]

    def shape_info(self):
        d = self.layer.diagonals[(0, 0)]
        return {"diagonals": len(d), "output_rotations": self.layer.output_rotations,
                "matrix": list(self.matrix.shape), "slots": self.params.get_slots()}
