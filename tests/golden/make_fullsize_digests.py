"""Writes tests/golden/fullsize_digests.json: SHA-256 digests, one per
polynomial row, of the oracle's words for the two full-size linear layers at
N=2^16 that the GPU suite cannot afford to recompute on the CPU at test time
(the oracle needs several minutes for the keys and the 512 diagonals):

  pcmm26    26-table embedding PCMM (workload seed 3, key seed 17):
            N=2^16, Q=[60,50x23], P=[61x8], dnum 3, 512 diagonals, 16 x 32 BSGS
  dense_lt  dense layer W 512x256 (workload seed 4, key seed 19):
            N=2^16, Q=[60,50x15], P=[61x6], dnum 3, 512 diagonals, 16 x 32 BSGS

For each: the input ciphertext (encryption index 0 at the top level), the
first and last encoded diagonals, one giant-step Galois key, the linear
transform output before the rescale, and the layer output after rescale,
hybrid fold and the (zero) bias -- each as the hex SHA-256 of the
little-endian u64 words of every row.

  pcmm26_top  HELRM.sparse then HELRM.sparse_to_top (workload seed 3, key
            seed 17): the pcmm26 layer, then the repacking Linear
            copy_into(416, 432, 16) compiled at the PCMM's output level
            (one hybrid diagonal, 6 fold rotations) -- the PCMM output and
            the repack output.

  dlrm      the encrypted HE-LRM forward (workload seed 3, key seed 17):
            N=2^16, Q=[60,50x29], P=[61x8]; both inputs encrypted at the
            input level (encryption indices 0 and 1), then every layer's
            output ciphertext (10 Linears, 6 degree-3 activations, the Add),
            and the relinearised product of the two inputs at that level.

Run in the build container:

    python tests/golden/make_fullsize_digests.py [threads] [case ...]
"""
import hashlib
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402
from helrm_amd import orion_host as oh  # noqa: E402
from helrm_amd.workloads import DenseLTWorkload, DLRMWorkload, PCMMWorkload, SparseToTopWorkload  # noqa: E402
sys.path.insert(0, os.path.dirname(HERE))
from helpers import oracle_dlrm, oracle_linear, oracle_pcmm  # noqa: E402

CASES = {
    "pcmm26": (PCMMWorkload, 3, 17),
    "dense_lt": (DenseLTWorkload, 4, 19),
}
OUT = os.path.join(HERE, "fullsize_digests.json")


def row_digests(a):
    """Hex SHA-256 of every row of a u64 array (last axis = coefficients)."""
    a = np.ascontiguousarray(a, dtype="<u8")
    rows = a.reshape(-1, a.shape[-1])
    return [hashlib.sha256(r.tobytes()).hexdigest() for r in rows]


def case_digests(name, cls, seed, key_seed, log=print):
    w = cls(None, name, seed=seed, key_seed=key_seed)
    c = w.cfg
    q, p = O.gen_primes(c["logn"], c["logq"], c["logp"])
    orc = O.Oracle(c["logn"], q, p, h=c["h"], seed=key_seed)
    try:
        S, level, scale = orc.slots, len(q) - 1, float(1 << c["logscale"])
        d, rots = oh.diagonalize(w.matrix, S)
        d = d[(0, 0)]
        idx = list(d.keys())
        t0 = time.time()
        ct = orc.encrypt(orc.encode(w.input, level, scale), level, 0)
        t = orc.lt_new(idx, np.stack([d[i] for i in idx]), level, 2.0)
        n1 = orc.lt_n1(t)
        log(f"{name}: {len(idx)} diagonals encoded, N1 {n1} ({time.time() - t0:.0f} s)")
        giant = n1  # the first nonzero giant step
        gk = orc.galois_key(orc.galois_element(giant))
        lt_out, l = orc.lt_eval(t, ct, level)
        log(f"{name}: transform done ({time.time() - t0:.0f} s)")
        out = orc.rescale(lt_out, l)
        sc = scale * q[level] / q[l]
        l -= 1
        for i in range(1, rots + 1):
            out = orc.add(out, orc.rotate(out, l, S // (2 ** i)), l)
        zero = orc.encode(np.zeros(1, np.float32), l, scale)
        out[0] = orc.add(out[0][None], zero[None], l)[0]
        log(f"{name}: layer done ({time.time() - t0:.0f} s)")
        return {
            "workload_seed": seed, "key_seed": key_seed, "q": [int(v) for v in q], "p": [int(v) for v in p],
            "level": level, "diagonals": len(idx), "N1": n1, "fold_rotations": rots,
            "ct_in": row_digests(ct),
            "diag_first": {"index": idx[0], "rows": row_digests(orc.lt_plaintext(t, idx[0]))},
            "diag_last": {"index": idx[-1], "rows": row_digests(orc.lt_plaintext(t, idx[-1]))},
            "galois_key": {"rotation": giant, "galel": int(orc.galois_element(giant)), "rows": row_digests(gk)},
            "lt_out": {"level": level, "scale": scale * q[level], "rows": row_digests(lt_out)},
            "out": {"level": l, "scale": sc, "rows": row_digests(out)},
        }
    finally:
        orc.close()


class _Module:
    """What oracle_dlrm reads of a compiled module, built on the host alone."""

    def __init__(self, **kw):
        self.__dict__.update(kw)


def dlrm_digests(seed=3, key_seed=17, log=print):
    w = DLRMWorkload(None, "dlrm", seed=seed, key_seed=key_seed)
    c = w.cfg
    q, p = O.gen_primes(c["logn"], c["logq"], c["logp"])
    slots = w.params.get_slots()
    method = w.params.get_embedding_method()
    for spec in w.layer_specs():
        if spec[1] == "linear":
            name, _, weight, bias, level, last = spec
            weight = np.asarray(weight, np.float32)
            d, rots = oh.diagonalize(weight, slots, method, last)
            b = np.zeros(weight.shape[0], np.float32) if bias is None else np.asarray(bias, np.float32)
            w.modules[name] = _Module(diagonals=d, output_rotations=rots, bias=b)
        else:
            w.modules[spec[0]] = _Module(coeffs=list(spec[2]))
    orc = O.Oracle(c["logn"], q, p, h=c["h"], seed=key_seed)
    try:
        t0 = time.time()
        (out, l, sc), trace = oracle_dlrm(orc, w, keep=True)
        log(f"dlrm: forward done ({time.time() - t0:.0f} s)")
        L = w.input_level
        scale = float(1 << c["logscale"])
        xd = orc.encrypt(orc.encode(np.asarray(w.dense, np.float32), L, scale), L, 0)
        xs = orc.encrypt(orc.encode(np.asarray(w.emb.selector, np.float32), L, scale), L, 1)
        prod = orc.mul_relin(xd, xs, L)
        log(f"dlrm: relinearised product done ({time.time() - t0:.0f} s)")
        logit = float(orc.decode_f64(orc.decrypt(out, l), l, sc)[0])
        return {
            "workload_seed": seed, "key_seed": key_seed, "q": [int(v) for v in q], "p": [int(v) for v in p],
            "input_level": L, "logit": logit,
            "ct_dense": row_digests(xd), "ct_sparse": row_digests(xs),
            "mul_relin": {"level": L, "rows": row_digests(prod)},
            "layers": {name: {"level": int(lv), "scale": float(s), "rows": row_digests(ct)}
                       for name, (ct, lv, s) in trace.items()},
        }
    finally:
        orc.close()


def top_digests(seed=3, key_seed=17, log=print):
    w = SparseToTopWorkload(None, "pcmm26_top", seed=seed, key_seed=key_seed)
    c = w.cfg
    q, p = O.gen_primes(c["logn"], c["logq"], c["logp"])
    orc = O.Oracle(c["logn"], q, p, h=c["h"], seed=key_seed)
    try:
        S, level = orc.slots, len(q) - 1
        d, rots = oh.diagonalize(w.matrix, S)
        t0 = time.time()
        ct1, l1, sc1 = oracle_pcmm(orc, d[(0, 0)], rots, level, w.selector, c["logscale"], 0)
        log(f"pcmm26_top: PCMM done ({time.time() - t0:.0f} s)")
        rd, rrots = oh.diagonalize(w.repack_matrix, S)
        rd = rd[(0, 0)]
        out, l2, sc2 = oracle_linear(orc, ct1, l1, sc1, rd, rrots, c["logscale"])
        log(f"pcmm26_top: repack done ({time.time() - t0:.0f} s)")
        return {
            "workload_seed": seed, "key_seed": key_seed, "q": [int(v) for v in q], "p": [int(v) for v in p],
            "level": level, "repack_diagonals": sorted(int(i) for i in rd.keys()), "repack_rotations": rrots,
            "pcmm_out": {"level": l1, "scale": sc1, "rows": row_digests(ct1)},
            "out": {"level": l2, "scale": sc2, "rows": row_digests(out)},
        }
    finally:
        orc.close()


def main():
    threads = int(sys.argv[1]) if len(sys.argv) > 1 else (os.cpu_count() or 1)
    names = sys.argv[2:] or list(CASES) + ["pcmm26_top", "dlrm"]
    O.set_threads(threads)
    log = lambda m: print(m, flush=True)  # noqa: E731
    res = {}
    if os.path.exists(OUT):
        with open(OUT) as f:
            res = json.load(f)
    for name in names:
        if name == "dlrm":
            res[name] = dlrm_digests(log=log)
        elif name == "pcmm26_top":
            res[name] = top_digests(log=log)
        else:
            res[name] = case_digests(name, *CASES[name], log=log)
    with open(OUT, "w") as f:
        json.dump(res, f, indent=1)
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
