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
  dlrm          encrypted HE-LRM forward at batch 1 (dlrm.py:181-231): bottom
                MLP 13-512-256-64-16, the pcmm26 embedding PCMM, both
                repacking Linears, Add, top MLP 432-512-256-1, degree-3
                activations after every Linear but the last; weights and
                biases N(0, 0.05), 13 dense features log-normal(0, 1);
                N=2^16, Q=[60,50x29] (30 limbs), P=[61x8], scale 2^50, no
                bootstrapping
  dlrm_n13      the dlrm network at N=2^13 on the same 30-limb chain

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
    "dlrm": dict(kind="dlrm", logn=16, logq=[60] + [50] * 29, logp=[61] * 8, logscale=50, h=192,
                 fields=26, rows=4096, dim=16, base=16, init="normal", init_arg=0.05, weight_std=0.05),
    "dlrm_n13": dict(kind="dlrm", logn=13, logq=[60] + [50] * 29, logp=[61] * 8, logscale=50, h=192,
                     fields=26, rows=4096, dim=16, base=16, init="normal", init_arg=0.05, weight_std=0.05),
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
        self.upload_seed = None
        self.layer_name = "linear"

    def use_seeded_upload(self, seed):
        """Seeded selector upload (bench_sweep.py:381-403): the input is
        encrypted with `a` expanded from `seed`, `a` is dropped (only b and the
        seed cross the wire) and every run() rebuilds it on the device first."""
        pt = self.scheme.encode(self.input, self.layer.level)
        cid = self.backend.EncryptSeeded(pt.ids[0], seed)
        self.backend.DropAx(cid)
        for i in pt.ids:
            self.backend.DeletePlaintext(i)
        self.ct_in.free()
        self.ct_in = oh.CipherTensor(self.scheme, [cid], pt.n)
        self.upload_seed = seed
        return self

    def expand_upload(self):
        if self.upload_seed is not None:
            for cid in self.ct_in.ids:
                self.backend.ExpandSeededAx(cid, self.upload_seed)

    def setup(self):
        self.scheme = oh.Scheme(self.params, self.backend)
        self.layer = oh.LinearLayer(self.scheme, self.matrix, name=self.layer_name).compile()
        pt = self.scheme.encode(self.input, self.layer.level)
        self.ct_in = self.scheme.encrypt(pt)
        for i in pt.ids:
            self.backend.DeletePlaintext(i)
        return self

    def run(self):
        """One forward of the layer. Returns the output CipherTensor."""
        self.expand_upload()
        return self.forward(self.ct_in)

    def forward(self, ct):
        """The layer's forward on the encrypted input ct."""
        return self.layer.forward(ct)

    def decrypt_output(self, out):
        vals = self.scheme.decode(self.scheme.decrypt(out))
        return vals[: self.matrix.shape[0]]

    def linear_layers(self):
        return [self.layer]

    def shape_info(self):
        d = self.layer.diagonals[(0, 0)]
        return {"diagonals": len(d), "output_rotations": self.layer.output_rotations,
                "matrix": list(self.matrix.shape), "slots": self.params.get_slots()}


class PCMMWorkload(LinearWorkload):
    """HE-LRM embedding PCMM (HELRM.sparse): digit one-hot selector times the
    block-diagonal table matrix."""

    def __init__(self, backend, name="pcmm26", seed=0, key_seed=1):
        super().__init__(backend, name, key_seed)
        self.layer_name = "sparse"
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
        self.expected = self.lookup_of(self.indices)

    def lookup_of(self, indices):
        """The plaintext embedding lookup of one query (one index per table)."""
        base = self.cfg["base"]
        return np.concatenate([
            t[0][int(i)] if s <= self.threshold else oh.radix_lookup(t, int(i), base)
            for t, i, s in zip(self.tables, indices, self.sizes)])

    def make_query(self, seed):
        """Another query on the same tables: indices drawn from `seed`, its
        selector encoded and encrypted at the layer's level.  Returns
        (CipherTensor, plaintext lookup)."""
        rng = np.random.default_rng(seed)
        idx = np.array([rng.integers(0, s) for s in self.sizes])
        pt = self.scheme.encode(oh.expanded_sparse(idx, self.sizes, self.threshold, self.cfg["base"]), self.layer.level)
        ct = self.scheme.encrypt(pt)
        for i in pt.ids:
            self.backend.DeletePlaintext(i)
        return ct, self.lookup_of(idx)


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
        self.repack = oh.LinearLayer(self.scheme, self.repack_matrix, level=self.layer.level - 1,
                                     name="sparse_to_top").compile()
        return self

    def forward(self, ct):
        emb = self.layer.forward(ct)
        out = self.repack.forward(emb)
        emb.free()
        return out

    def decrypt_output(self, out):
        vals = self.scheme.decode(self.scheme.decrypt(out))
        return vals[: self.repack_matrix.shape[0]]

    def linear_layers(self):
        return [self.layer, self.repack]

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


# Degree-3 activation, highest-degree coefficient first (orion.nn.Activation
# order): the least-squares cubic fit of ReLU on [-2, 4], rounded to four
# places.  It stands in for HE-LRM's on.ReLU (dlrm.py:133-139), whose
# minimax sign composite needs bootstrapping.
ACTIVATION3 = (-0.0320, 0.2195, 0.5706, 0.2048)
BOTTOM_WIDTHS = (13, 512, 256, 64, 16)   # dlrm.py:19
TOP_WIDTHS = (432, 512, 256, 1)          # dlrm.py:20


def plan_levels(bottom_layers, top_layers, sparse_depth, linear_depth=1, act_depth=2):
    """Levels Orion's bootstrap solver (orion/core/auto_bootstrap.py:114-158)
    gives HE-LRM when the chain is long enough to need no bootstrap: a linear
    layer's cost grows with its level (level_dag.py:167-197) and activations
    cost nothing, so every layer sits at the lowest level its successors
    allow and the network ends at level 0.  Layers are ('L', name) or ('A',
    name) in forward order; returns ({name: level}, add_level, input_level)."""
    levels, lvl = {}, 0
    for kind, name in reversed(top_layers):
        lvl += linear_depth if kind == "L" else act_depth
        levels[name] = lvl
    add_level = lvl
    for kind, name in reversed(bottom_layers):
        lvl += linear_depth if kind == "L" else act_depth
        levels[name] = lvl
    input_level = lvl
    levels["sparse_to_top"] = add_level + linear_depth
    levels["sparse"] = add_level + linear_depth + sparse_depth
    return levels, add_level, input_level


class DLRMWorkload:
    """HELRM.forward (dlrm.py:224-231) under encryption:
        top(add(bottom_to_top(bottom(dense)), sparse_to_top(sparse(selector))))
    with every on.Linear a LinearLayer (hybrid packing; the network's last
    Linear square-packed, orion/core/orion.py:255-285), every activation an
    Activation of ACTIVATION3, and both inputs encrypted at the input level
    (bench_sweep.py:346-349, 395-399).  The embedding part is the
    PCMMWorkload of the same config and seed."""

    def __init__(self, backend, name="dlrm", seed=0, key_seed=1):
        c = CONFIGS[name]
        self.name, self.cfg = name, c
        self.backend = backend
        self.params = oh.Params(c["logn"], c["logq"], c["logp"], c["logscale"], c["h"], seed=key_seed)
        self.emb = PCMMWorkload(None, name, seed=seed, key_seed=key_seed)
        rng = np.random.default_rng([seed, 5])
        std = c["weight_std"]

        def linear(i, o):
            return (rng.normal(0.0, std, (o, i)).astype(np.float32), rng.normal(0.0, std, o).astype(np.float32))
        self.bottom_w = [linear(i, o) for i, o in zip(BOTTOM_WIDTHS, BOTTOM_WIDTHS[1:])]
        self.top_w = [linear(i, o) for i, o in zip(TOP_WIDTHS, TOP_WIDTHS[1:])]
        self.dense = rng.lognormal(0.0, 1.0, BOTTOM_WIDTHS[0]).astype(np.float32)
        # coefficients cross the backend ABI as fp32 (polyeval.go GenerateMonomial)
        self.coeffs = tuple(float(np.float32(cf)) for cf in ACTIVATION3)
        dim = c["dim"]
        width = self.emb.matrix.shape[0]
        self.bottom_to_top_w = oh.copy_into(dim, TOP_WIDTHS[0], 0)        # dlrm.py:194
        self.sparse_to_top_w = oh.copy_into(width, TOP_WIDTHS[0], dim)    # dlrm.py:198
        self.bottom_names = []
        for k in range(len(self.bottom_w)):
            self.bottom_names += [("L", f"bottom.{2 * k}"), ("A", f"bottom.{2 * k + 1}")]
        self.bottom_names.append(("L", "bottom_to_top"))
        self.top_names = []
        for k in range(len(self.top_w)):
            self.top_names.append(("L", f"top.{2 * k}"))
            if k < len(self.top_w) - 1:
                self.top_names.append(("A", f"top.{2 * k + 1}"))
        self.levels, self.add_level, self.input_level = plan_levels(self.bottom_names, self.top_names, 1)
        self.expected = self.clear_forward()
        self.scheme = None
        self.modules = {}
        self.ct_dense = self.ct_sparse = None
        self.upload_seed = None
        # run(): the lookup path on the backend's second stream, beside the bottom MLP,
        # given to it once the first `lookup_after` bottom layers are queued (5: after
        # the 256->64 Linear, so that it overlaps the bottom MLP's small, latency-bound
        # key switches rather than its large transforms; measured 28.0 ms per forward
        # against 28.7 when forked first and 29.4 on one stream)
        self.concurrent = True
        self.lookup_after = 5

    def use_seeded_upload(self, seed):
        """The selector uploaded as (b, seed) at the input level
        (bench_sweep.py:381-403); every forward rebuilds `a` on the device."""
        pt = self.scheme.encode(self.emb.selector, self.input_level)
        cid = self.backend.EncryptSeeded(pt.ids[0], seed)
        self.backend.DropAx(cid)
        for i in pt.ids:
            self.backend.DeletePlaintext(i)
        self.ct_sparse.free()
        self.ct_sparse = oh.CipherTensor(self.scheme, [cid], pt.n)
        self.upload_seed = seed
        return self

    # ---- cleartext model (float64 on the fp32 weights) ----
    def act(self, x):
        out = np.zeros_like(x)
        for cf in self.coeffs:
            out = cf + x * out
        return out

    def clear_trace(self):
        """Every layer's cleartext output, keyed by layer name."""
        tr = {}
        x = self.dense.astype(np.float64)
        for k, (w, b) in enumerate(self.bottom_w):
            x = w.astype(np.float64) @ x + b
            tr[f"bottom.{2 * k}"] = x
            x = self.act(x)
            tr[f"bottom.{2 * k + 1}"] = x
        dense = self.bottom_to_top_w.astype(np.float64) @ x
        tr["bottom_to_top"] = dense
        emb = self.emb.matrix.astype(np.float64) @ self.emb.selector
        tr["sparse"] = emb
        sparse = self.sparse_to_top_w.astype(np.float64) @ emb
        tr["sparse_to_top"] = sparse
        z = dense + sparse
        tr["add"] = z
        for k, (w, b) in enumerate(self.top_w):
            z = w.astype(np.float64) @ z + b
            tr[f"top.{2 * k}"] = z
            if k < len(self.top_w) - 1:
                z = self.act(z)
                tr[f"top.{2 * k + 1}"] = z
        return tr

    def clear_forward(self):
        return self.clear_trace()[self.top_names[-1][1]]

    # ---- encrypted model ----
    def layer_specs(self):
        """Every module of the network: (name, "linear", weight, bias, level,
        last) or (name, "activation", coefficients)."""
        L = self.levels
        specs = []
        for k, (w, b) in enumerate(self.bottom_w):
            specs.append((f"bottom.{2 * k}", "linear", w, b, L[f"bottom.{2 * k}"], False))
            specs.append((f"bottom.{2 * k + 1}", "activation", self.coeffs))
        specs.append(("bottom_to_top", "linear", self.bottom_to_top_w, None, L["bottom_to_top"], False))
        specs.append(("sparse", "linear", self.emb.matrix, None, L["sparse"], False))
        specs.append(("sparse_to_top", "linear", self.sparse_to_top_w, None, L["sparse_to_top"], False))
        for k, (w, b) in enumerate(self.top_w):
            last = k == len(self.top_w) - 1
            specs.append((f"top.{2 * k}", "linear", w, b, L[f"top.{2 * k}"], last))
            if not last:
                specs.append((f"top.{2 * k + 1}", "activation", self.coeffs))
        return specs

    def setup(self):
        s = self.scheme = oh.Scheme(self.params, self.backend)
        mods = {}
        for spec in self.layer_specs():
            if spec[1] == "linear":
                name, _, w, b, level, last = spec
                mods[name] = oh.LinearLayer(s, w, b, level=level, last=last, name=name)
            else:
                mods[spec[0]] = oh.Activation(s, spec[2])
        for m in mods.values():
            m.compile()
        self.modules = mods
        pd = s.encode(self.dense, self.input_level)
        self.ct_dense = s.encrypt(pd)
        ps = s.encode(self.emb.selector, self.input_level)
        self.ct_sparse = s.encrypt(ps)
        for i in pd.ids + ps.ids:
            self.backend.DeletePlaintext(i)
        return self

    def run_stages(self, keep=False, concurrent=False):
        """One encrypted forward; with keep=True also returns every layer's
        output ciphertext tensor (the caller frees them).  concurrent: the
        lookup path (PCMM + sparse_to_top), which depends on nothing of the
        bottom MLP, is given to the backend's second stream first and runs
        beside the bottom MLP; the Add joins the two (the same calls and
        results, in another order)."""
        m = self.modules
        b = self.backend
        kept = {}

        def step(name, x, free_in):
            y = m[name].forward(x)
            if keep:
                kept[name] = y
            elif free_in:
                x.free()
            return y

        def lookup():
            if self.upload_seed is not None:
                for cid in self.ct_sparse.ids:
                    b.ExpandSeededAx(cid, self.upload_seed)
            e = step("sparse", self.ct_sparse, False)
            return step("sparse_to_top", e, True)

        def fork():
            b.SetStream(1)
            b.JoinStream(0)  # after everything already given to stream 0 (inputs, keys)
            e = lookup()
            b.SetStream(0)
            return e

        e = None
        x = self.ct_dense
        for i, (_, name) in enumerate(self.bottom_names):
            if concurrent and i == self.lookup_after:
                e = fork()
            x = step(name, x, i > 0)
        if concurrent:
            if e is None:
                e = fork()
            b.JoinStream(1)
        else:
            e = lookup()
        z = x.add(e)
        if keep:
            kept["add"] = z
        else:
            x.free()
            e.free()
        for i, (_, name) in enumerate(self.top_names):
            z = step(name, z, True)
        return z, kept

    def run(self):
        return self.run_stages(False, self.concurrent)[0]

    # stage split of bench_sweep.py:186-192 (HELRM_STAGES)
    STAGES = {"bottom_mlp": ("bottom", "bottom_to_top"), "lookup": ("sparse",), "sparse_to_top": ("sparse_to_top",),
              "add": ("add",), "top_mlp": ("top",)}

    def stage_of(self, name):
        for stage, prefixes in self.STAGES.items():
            if any(name == p or name.startswith(p + ".") for p in prefixes):
                return stage
        raise KeyError(name)

    def run_staged(self, sync, clock):
        """One forward with `sync()` before each timestamp around every
        layer (the stage hooks of bench_sweep.py:195-219); returns (output,
        {stage: seconds}); the per-layer seconds are kept in self.layer_s."""
        times = {}
        self.layer_s = {}
        m = self.modules
        if self.upload_seed is not None:
            for cid in self.ct_sparse.ids:
                self.backend.ExpandSeededAx(cid, self.upload_seed)

        def step(name, x, free_in):
            sync()
            t0 = clock()
            y = m[name].forward(x) if name != "add" else x[0].add(x[1])
            sync()
            st = self.stage_of(name)
            dt = clock() - t0
            times[st] = times.get(st, 0.0) + dt
            self.layer_s[name] = dt
            if free_in:
                for c in (x if isinstance(x, tuple) else (x,)):
                    c.free()
            return y
        x = self.ct_dense
        for i, (_, name) in enumerate(self.bottom_names):
            x = step(name, x, i > 0)
        e = step("sparse", self.ct_sparse, False)
        e = step("sparse_to_top", e, True)
        z = step("add", (x, e), True)
        for _, name in self.top_names:
            z = step(name, z, True)
        return z, times

    def linear_layers(self):
        return [m for m in self.modules.values() if isinstance(m, oh.LinearLayer)]

    def activations(self):
        return [(n, m) for n, m in self.modules.items() if isinstance(m, oh.Activation)]

    def decrypt_output(self, out):
        return self.scheme.decode(self.scheme.decrypt(out))[: TOP_WIDTHS[-1]]

    def shape_info(self):
        info = {}
        for kind, name in self.bottom_names + [("L", "sparse"), ("L", "sparse_to_top")] + self.top_names:
            m = self.modules.get(name)
            if kind == "L":
                d = m.diagonals[(0, 0)] if m is not None else None
                info[name] = {"level": self.levels[name], "diagonals": None if d is None else len(d),
                              "output_rotations": None if m is None else m.output_rotations}
            else:
                info[name] = {"level": self.levels[name]}
        info["input_level"], info["add_level"] = self.input_level, self.add_level
        return info


def make_workload(backend, name, seed=0, key_seed=1):
    c = CONFIGS[name]
    if c["kind"] == "dlrm":
        return DLRMWorkload(backend, name, seed=seed, key_seed=key_seed)
    if c["kind"] == "pcmm":
        cls = SparseToTopWorkload if c.get("repack") else PCMMWorkload
    else:
        cls = DenseLTWorkload
    return cls(backend, name, seed=seed, key_seed=key_seed)
