"""Host-side callers of the embedding PCMM, restated from the reference so the
path runs end to end without the reference tree:

  * HE-LRM selector / plaintext lookup   examples/criteo/dlrm.py:66-124,202-247
  * hybrid diagonal extraction           orion/core/packing.py:510-529,626-865
  * encode padding                        orion/backend/python/encoder.py:14-107
  * transform generation + rotation keys  orion/backend/python/lt_evaluator.py:29-57,132-160
  * block loop + rescale                  orion/backend/python/lt_evaluator.py:224-275
  * output fold + bias                    orion/nn/linear.py:99-140,191-209
  * CipherTensor roll / add               orion/backend/python/tensors.py:154-186,256-262

Everything here is host bookkeeping; all ciphertext arithmetic goes through
the backend object (a HipLibrary, or any object with the Lattigo method set).
"""
import math
import os

import numpy as np

# --------------------------------------------------------------------------
# parameters (orion/backend/python/parameters.py:168-358, the getters used)
# --------------------------------------------------------------------------


class Params:
    def __init__(self, logn, logq, logp, logscale=None, h=192, ringtype="standard",
                 embedding_method="hybrid", io_mode="none", seed=None, keys_path="", diags_path=""):
        self.logn, self.logq, self.logp = int(logn), list(logq), list(logp)
        self.logscale = int(logscale or self.logq[-1])
        self.h, self.ringtype = int(h), ringtype.lower()
        self.embedding_method, self.io_mode, self.seed = embedding_method, io_mode, seed
        self.keys_path, self.diags_path = keys_path, diags_path

    @classmethod
    def from_config(cls, cfg, seed=None):
        ck = {k.lower(): v for k, v in cfg.get("ckks_params", {}).items()}
        on = {k.lower(): v for k, v in cfg.get("orion", {}).items()}
        return cls(ck["logn"], ck["logq"], ck["logp"], ck.get("logscale"), ck.get("h", 192),
                   ck.get("ringtype", "standard"), on.get("embedding_method", "hybrid"),
                   on.get("io_mode", "none"), seed)

    def get_logn(self): return self.logn
    def get_logq(self): return self.logq
    def get_logp(self): return self.logp
    def get_logscale(self): return self.logscale
    def get_default_scale(self): return 1 << self.logscale
    def get_hamming_weight(self): return self.h
    def get_ringtype(self): return self.ringtype
    def get_max_level(self): return len(self.logq) - 1
    def get_slots(self): return 1 << (self.logn - 1)
    def get_embedding_method(self): return self.embedding_method
    def get_io_mode(self): return self.io_mode
    def get_keys_path(self): return self.keys_path
    def get_diags_path(self): return self.diags_path
    def get_seed(self): return self.seed


# --------------------------------------------------------------------------
# HE-LRM selector and plaintext reference (examples/criteo/dlrm.py)
# --------------------------------------------------------------------------

def digits(index, base, width):
    """dlrm.py:66-72: little-endian base-`base` digits of `index`."""
    index = np.asarray(index, dtype=np.int64)
    out = []
    for _ in range(width):
        out.append(np.remainder(index, base))
        index = np.floor_divide(index, base)
    return np.stack(out)


def radix_width(categories, base):
    """dlrm.py:75-76"""
    return math.ceil(math.log(categories, base))


def expanded_width(categories, compress_threshold, base):
    """dlrm.py:79-82"""
    if categories > compress_threshold:
        return base * radix_width(categories, base)
    return categories


def expanded_id(index, size, compress_threshold, base):
    """dlrm.py:202-213: one-hot of each digit (digit 0 first), or a plain one-hot."""
    if size <= compress_threshold:
        out = np.zeros(size, dtype=np.float32)
        out[index] = 1.0
        return out
    pieces = []
    for d in digits(index, base, radix_width(size, base)):
        piece = np.zeros(base, dtype=np.float32)
        piece[int(d)] = 1.0
        pieces.append(piece)
    return np.concatenate(pieces)


def expanded_sparse(indices, sizes, compress_threshold, base):
    """dlrm.py:215-221: concatenation of the fields' selectors."""
    return np.concatenate([expanded_id(int(i), s, compress_threshold, base) for i, s in zip(indices, sizes)])


def radix_lookup(tables, index, base):
    """RadixTable.forward (dlrm.py:111-119): sum of the digit rows (fp32)."""
    width = len(tables)
    out = np.zeros(tables[0].shape[1], dtype=np.float32)
    for t, d in zip(tables, digits(index, base, width)):
        out = out + t[int(d)]
    return out


def block_diag_matrix(field_tables):
    """export (dlrm.py:241-247): block_diag(W_0..W_F).T with W_f = cat of the
    field's digit tables; rows = outputs, columns = selector positions."""
    blocks = [np.concatenate(t, axis=0) for t in field_tables]  # (width*base) x dim
    rows = sum(b.shape[1] for b in blocks)
    cols = sum(b.shape[0] for b in blocks)
    M = np.zeros((rows, cols), dtype=np.float32)
    r = c = 0
    for b in blocks:
        M[r:r + b.shape[1], c:c + b.shape[0]] = b.T
        r += b.shape[1]
        c += b.shape[0]
    return M


def copy_into(width, output_width, start):
    """Weight of the repacking Linear of examples/criteo/dlrm.py:174-178
    (bias=False): output_width x width, identity block at rows
    [start, start + width) -- HELRM.sparse_to_top moves the 416 embedding
    outputs behind the 16 bottom-MLP features of the top MLP input."""
    w = np.zeros((output_width, width), dtype=np.float32)
    w[start:start + width, :width] = np.eye(width, dtype=np.float32)
    return w


# --------------------------------------------------------------------------
# hybrid diagonal extraction (orion/core/packing.py:626-865, uniform path)
# --------------------------------------------------------------------------

def diagonalize(matrix, num_slots, embed_method="hybrid", is_last_layer=False):
    """Generalised diagonals per (num_slots x num_slots) block.

    Returns ({(row, col): {diag_index: float32 values}}, output_rotations).
    Hybrid (one block row, not the last layer): block_height = 2^ceil(log2 H),
    diagonal i holds M[row0 + (j mod bh), col0 + (i + j) mod slots], zero
    diagonals dropped (a block with none keeps diagonal 0 of zeros) and the
    output needs log2(slots / bh) fold rotations.
    """
    M = np.asarray(matrix, dtype=np.float32)
    H, W = M.shape
    nbr = math.ceil(H / num_slots)
    nbc = math.ceil(W / num_slots)
    if nbr == 1 and embed_method == "hybrid" and not is_last_layer:
        block_height = 2 ** math.ceil(math.log2(H))
        output_rotations = int(math.log2(num_slots // block_height))
    else:
        block_height = num_slots
        output_rotations = 0
    padded = np.zeros((nbr * block_height, nbc * num_slots), dtype=np.float32)
    padded[:H, :W] = M
    j = np.arange(num_slots)
    row_idx = np.tile(np.arange(block_height), num_slots // block_height)
    out = {}
    for br in range(nbr):
        for bc in range(nbc):
            block = padded[br * num_slots: br * num_slots + block_height, bc * num_slots:(bc + 1) * num_slots]
            diags = {}
            for i in range(block_height):
                col_idx = (i + j) % num_slots
                d = block[row_idx, col_idx]
                if np.any(d):
                    diags[i] = d.astype(np.float32)
            out[(br, bc)] = diags or {0: np.zeros(num_slots, dtype=np.float32)}
    return out, output_rotations


# --------------------------------------------------------------------------
# scheme, tensors and the linear layer
# --------------------------------------------------------------------------

class WireStore:
    """Named byte blobs standing in for the HDF5 files of Orion's io_mode
    (keys_path: "sk" and one entry per Galois element; diags_path: one entry
    per layer / block / diagonal, lt_evaluator.py:160-215, 440-497).  With a
    path the store is a .npz file of uint8 arrays (written on flush, read
    without pickle); without one it lives in memory."""

    def __init__(self, path=""):
        self.path = path
        self.blobs = {}
        if path and os.path.exists(path):
            with np.load(path, allow_pickle=False) as z:
                self.blobs = {k: z[k].copy() for k in z.files}

    def __contains__(self, key):
        return key in self.blobs

    def __getitem__(self, key):
        return self.blobs[key]

    def __setitem__(self, key, data):
        self.blobs[key] = np.asarray(data, dtype=np.uint8).copy()

    def keys(self):
        return self.blobs.keys()

    def flush(self):
        if self.path:
            np.savez(self.path, **self.blobs)


class Scheme:
    """Minimal counterpart of orion.core.orion.Scheme for this path: creates
    the backend, keys, encoder/encryptor/evaluator (init_scheme order,
    orion/core/orion.py:66-126 and orion/backend/python/*).  io_mode "save"
    serializes the secret key, rotation keys and diagonals into the stores,
    "load" reads them back instead of generating them
    (key_generator.py:17-31, lt_evaluator.py)."""

    def __init__(self, params, backend):
        self.params = params
        self.backend = backend
        self.io_mode = params.get_io_mode()
        self.key_store = WireStore(params.get_keys_path())
        self.diag_store = WireStore(params.get_diags_path())
        backend.setup_bindings(params)
        backend.NewKeyGenerator()
        if self.io_mode != "load":
            backend.GenerateSecretKey()
            if self.io_mode == "save":
                self._store(self.key_store, "sk", backend.SerializeSecretKey())
        else:
            backend.LoadSecretKey(self.key_store["sk"])
        backend.GeneratePublicKey()
        backend.GenerateRelinearizationKey()
        backend.GenerateEvaluationKeys()
        backend.NewEncoder()
        backend.NewEncryptor()
        backend.NewDecryptor()
        backend.NewEvaluator()
        backend.NewLinearTransformEvaluator()
        backend.NewPolynomialEvaluator()
        self.saved_rotation_keys = set()

    def _store(self, store, key, result):
        data, ptr = result
        try:
            store[key] = data
        finally:
            self.backend.FreeCArray(ptr)

    def flush(self):
        self.key_store.flush()
        self.diag_store.flush()

    # orion/backend/python/encoder.py:14-88 (real values, default path)
    def encode(self, values, level=None, scale=None):
        values = np.asarray(values, dtype=np.float64).reshape(-1)
        if level is None:
            level = self.params.get_max_level()
        if not scale:
            scale = self.params.get_default_scale()
        slots = self.params.get_slots()
        pad = (-len(values)) % slots
        vec = np.concatenate([values, np.zeros(pad)]) if pad or len(values) == 0 else values
        if len(vec) == 0:
            vec = np.zeros(slots)
        ids = [self.backend.Encode(vec[i * slots:(i + 1) * slots].tolist(), level, int(scale))
               for i in range(len(vec) // slots)]
        return PlainTensor(self, ids, len(values))

    def decode(self, pt):
        vals = []
        for i in pt.ids:
            vals.extend(self.backend.Decode(i))
        return np.asarray(vals[: pt.n], dtype=np.float64)

    def encrypt(self, pt):
        return CipherTensor(self, [self.backend.Encrypt(i) for i in pt.ids], pt.n)

    def decrypt(self, ct):
        return PlainTensor(self, [self.backend.Decrypt(i) for i in ct.ids], ct.n)

    def moduli(self):
        return self.backend.GetModuliChain()


class PlainTensor:
    def __init__(self, scheme, ids, n):
        self.scheme, self.ids, self.n = scheme, list(ids), n


class CipherTensor:
    """tensors.py:154-186 (add), 256-262 (roll)."""

    def __init__(self, scheme, ids, n):
        self.scheme, self.ids, self.n = scheme, list(ids), n

    def add(self, other, in_place=False):
        b = self.scheme.backend
        out = []
        for i, cid in enumerate(self.ids):
            if isinstance(other, PlainTensor):
                f = b.AddPlaintext if in_place else b.AddPlaintextNew
            else:
                f = b.AddCiphertext if in_place else b.AddCiphertextNew
            out.append(f(cid, other.ids[i]))
        if in_place:
            return self
        return CipherTensor(self.scheme, out, self.n)

    def __add__(self, other):
        return self.add(other, False)

    def __iadd__(self, other):
        return self.add(other, True)

    def roll(self, amount, in_place=False):
        b = self.scheme.backend
        f = b.Rotate if in_place else b.RotateNew
        return CipherTensor(self.scheme, [f(c, int(amount)) for c in self.ids], self.n)

    def add_rolled(self, amount):
        """self += self.roll(amount), in place: the fold step of linear.py:115-117.
        One backend call per ciphertext (RotateAdd, the add inside the key
        switch's last pass) when the backend has it; else roll + add."""
        b = self.scheme.backend
        if hasattr(b, "RotateAdd"):
            for c in self.ids:
                b.RotateAdd(c, int(amount))
            return self
        rolled = self.roll(amount)
        self.add(rolled, True)
        rolled.free()
        return self

    def free(self):
        for c in self.ids:
            self.scheme.backend.DeleteCiphertext(c)
        self.ids = []


class LinearLayer:
    """Linear / Embedding (orion/nn/linear.py:143-225, orion/nn/embedding.py:12-21)
    compiled at `level` with the hybrid packing; bias zeros for Embedding."""

    _count = 0

    def __init__(self, scheme, weight, bias=None, level=None, bsgs_ratio=2.0, last=False, name=None):
        self.scheme = scheme
        if name is None:
            name = f"linear{LinearLayer._count}"
            LinearLayer._count += 1
        self.name = name
        self.weight = np.asarray(weight, dtype=np.float32)
        self.out_features = self.weight.shape[0]
        self.bias = np.zeros(self.out_features, dtype=np.float32) if bias is None else np.asarray(bias, np.float32)
        self.level = scheme.params.get_max_level() if level is None else level
        self.depth = 1
        self.bsgs_ratio = float(bsgs_ratio)
        self.last = last
        self.transform_ids = {}

    def compile(self):
        p = self.scheme.params
        slots = p.get_slots()
        self.diagonals, self.output_rotations = diagonalize(self.weight, slots, p.get_embedding_method(), self.last)
        # linear.py:191-209: bias encoded at level - depth, then the transforms
        self.on_bias_ptxt = self.scheme.encode(self.bias, self.level - self.depth)
        self.transform_ids = self.generate_transforms()
        return self

    # lt_evaluator.py:29-57
    def generate_transforms(self):
        b = self.scheme.backend
        mode = self.scheme.io_mode
        ids = {}
        for (row, col), diags in self.diagonals.items():
            idxs = list(diags.keys())
            data = np.concatenate([diags[i] for i in idxs]).astype(np.float32)
            tid = b.GenerateLinearTransform(idxs, data, self.level, self.bsgs_ratio, mode)
            ids[(row, col)] = tid
            self.generate_rotation_keys(tid)
            if mode == "save":
                # lt_evaluator.py:453-464: each diagonal leaves the transform as bytes
                for d in idxs:
                    self.scheme._store(self.scheme.diag_store, f"{self.name}/{row}_{col}/{d}", b.SerializeDiagonal(tid, d))
        return ids

    # lt_evaluator.py:132-161
    def generate_rotation_keys(self, tid):
        b = self.scheme.backend
        keys = b.GetLinearTransformRotationKeys(tid)
        new = set(keys).difference(self.scheme.saved_rotation_keys)
        self.scheme.saved_rotation_keys.update(new)
        for k in new:
            if self.scheme.io_mode == "none":
                b.GenerateLinearTransformRotationKey(k)
            elif self.scheme.io_mode == "save" and str(k) not in self.scheme.key_store:
                self.scheme._store(self.scheme.key_store, str(k), b.GenerateAndSerializeRotationKey(k))

    # lt_evaluator.py:466-497
    def load_transform(self, row, col, tid):
        b = self.scheme.backend
        for k in b.GetLinearTransformRotationKeys(tid):
            b.LoadRotationKey(self.scheme.key_store[str(k)], int(k))
        prefix = f"{self.name}/{row}_{col}/"
        for key in self.scheme.diag_store.keys():
            if key.startswith(prefix):
                b.LoadPlaintextDiagonal(self.scheme.diag_store[key], tid, int(key[len(prefix):]))

    # lt_evaluator.py:224-275 (uniform path)
    def evaluate_lt(self, x):
        b = self.scheme.backend
        tids = np.array(list(self.transform_ids.values()))
        cols = len(x.ids)
        rows = len(tids) // cols
        tids = tids.reshape(rows, cols)
        cts_out = []
        io = self.scheme.io_mode != "none"
        # A prerescaled transform returns Rescale(block result): summed over
        # several column blocks that would round each block separately, not
        # Rescale(sum) as the Lattigo flow does, so a layer with more than
        # one column block evaluates its transforms unrescaled and rescales
        # the sum once.
        pre = bool(getattr(b, "lt_output_prerescaled", False))
        if pre and cols > 1:
            b.set_lt_output_prerescaled(False)
        try:
            for i in range(rows):
                ct_out = None
                for j in range(cols):
                    if io:
                        self.load_transform(i, j, int(tids[i][j]))
                    res = CipherTensor(self.scheme, [b.EvaluateLinearTransform(int(tids[i][j]), x.ids[j])], x.n)
                    if io:
                        b.RemoveRotationKeys()
                        b.RemovePlaintextDiagonals(int(tids[i][j]))
                    if ct_out is None:
                        ct_out = res
                    else:
                        ct_out = ct_out + res
                        res.free()
                if pre and cols == 1:
                    cts_out.append(ct_out.ids[0])
                else:
                    cts_out.append(b.RescaleNew(ct_out.ids[0]))
                    ct_out.free()
        finally:
            if pre and cols > 1:
                b.set_lt_output_prerescaled(True)
        return CipherTensor(self.scheme, cts_out, self.out_features)

    # linear.py:99-140 (no slicing, no fold-retag on the Lattigo path)
    def forward(self, x):
        out = self.evaluate_lt(x)
        slots = self.scheme.params.get_slots()
        for i in range(1, self.output_rotations + 1):
            out.add_rolled(slots // (2 ** i))
        out += self.on_bias_ptxt
        return out

    def free(self):
        for t in self.transform_ids.values():
            self.scheme.backend.DeleteLinearTransform(int(t))
        self.transform_ids = {}


class Activation:
    """orion.nn.Activation (orion/nn/activation.py:12-48): a polynomial given
    highest-degree coefficient first (the Horner order of its cleartext
    forward), compiled through PolynomialEvaluator.generate_monomial, which
    hands the backend the coefficients lowest degree first
    (orion/backend/python/poly_evaluator.py:15-18), and evaluated on every
    ciphertext of the tensor at `output_scale` (the default scale when unset,
    poly_evaluator.py:25-35).  Consumes ceil(log2(len(coeffs))) levels."""

    def __init__(self, scheme, coeffs):
        self.scheme = scheme
        self.coeffs = [float(c) for c in coeffs]
        self.depth = int(math.ceil(math.log2(len(self.coeffs)))) if len(self.coeffs) > 1 else 0
        self.output_scale = None
        self.poly = None

    def compile(self):
        self.poly = self.scheme.backend.GenerateMonomial(self.coeffs[::-1])
        return self

    def clear(self, x):
        out = 0.0
        for c in self.coeffs:
            out = c + x * out
        return out

    def forward(self, x):
        b = self.scheme.backend
        scale = self.output_scale or self.scheme.params.get_default_scale()
        return CipherTensor(self.scheme, [b.EvaluatePolynomial(c, self.poly, int(scale)) for c in x.ids], x.n)


# --------------------------------------------------------------------------
# complex-lane upload (orion/core/lane_packing.py)
# --------------------------------------------------------------------------

def plan_packing(num_elements, num_slots):
    """(real ciphertexts, packed ciphertexts) of a real vector (lane_packing.py:42-51)."""
    num_real = -(-num_elements // num_slots)
    return num_real, -(-num_real // 2)


def pack_lanes(values, num_slots):
    """Client side (lane_packing.py:59-81): chunk 2m in the real lane and chunk
    2m+1 in the imaginary lane of packed chunk m, pre-scaled by 0.5.  Returns
    (complex values, number of real chunks)."""
    flat = np.asarray(values, dtype=np.float64).reshape(-1)
    pad = (-len(flat)) % num_slots
    if pad:
        flat = np.concatenate([flat, np.zeros(pad)])
    chunks = flat.reshape(-1, num_slots)
    num_real = chunks.shape[0]
    if num_real % 2:
        chunks = np.concatenate([chunks, np.zeros((1, num_slots))])
    return (0.5 * (chunks[0::2] + 1j * chunks[1::2])).reshape(-1), num_real


def encode_complex(scheme, values, level, scale=None):
    """Complex values, one plaintext per `slots` of them (EncodeComplex takes
    interleaved fp32 (re, im) pairs)."""
    z = np.asarray(values, dtype=np.complex128).reshape(-1)
    slots = scheme.params.get_slots()
    scale = scale or scheme.params.get_default_scale()
    ids = []
    for i in range(0, len(z), slots):
        c = z[i:i + slots]
        v = np.empty(2 * len(c), dtype=np.float32)
        v[0::2], v[1::2] = c.real, c.imag
        ids.append(scheme.backend.EncodeComplex(v, level, int(scale)))
    return PlainTensor(scheme, ids, len(z))


def unpack_lanes(scheme, packed, num_real):
    """Server side (lane_packing.py:84-114): x = p + conj(p), y = -i (p - conj(p))
    per packed ciphertext, the zero-padded partner of an odd count dropped."""
    b = scheme.backend
    real_ids = []
    for pid in packed.ids:
        conj = b.ConjugateNew(pid)
        even = b.AddCiphertextNew(pid, conj)
        diff = b.SubCiphertextNew(pid, conj)
        b.MulImaginaryUnit(diff)
        odd = b.Negate(diff)
        b.DeleteCiphertext(conj)
        b.DeleteCiphertext(diff)
        real_ids.extend([even, odd])
    for extra in real_ids[num_real:]:
        b.DeleteCiphertext(extra)
    return CipherTensor(scheme, real_ids[:num_real], num_real * scheme.params.get_slots())


def embedding_pcmm(scheme, layer, selector):
    """One query: encode + encrypt the selector at the layer's level and run
    the embedding PCMM (HELRM.sparse, dlrm.py:226-230).  Returns (ct, pt_in)."""
    pt = scheme.encode(selector, layer.level)
    ct = scheme.encrypt(pt)
    return layer.forward(ct), ct
