"""Writes tests/golden/pcmm_n10.npz: input/output vectors of the embedding
PCMM flow on the CPU restatement (oracle/) at N=2^10, Q=[40,30,30],
P=[41,41], scale 2^30, h=32, key seed 77.

    python tests/golden/make_golden.py

Contents: moduli, secret key, the selector and its ciphertext (encryption
index 0), one encoded diagonal, the linear-transform output, the rescaled
output, one rotation, and the folded PCMM output; plus NTT vectors of a
fixed input for every modulus.  The CPU suite checks the oracle still
reproduces these words; the GPU suite checks the HIP library against them.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402
from helrm_amd import orion_host as oh  # noqa: E402

LOGN, LOGQ, LOGP, LOGSCALE, H, SEED = 10, [40, 30, 30], [41, 41], 30, 32, 77


def generate():
    q, p = O.gen_primes(LOGN, LOGQ, LOGP)
    o = O.Oracle(LOGN, q, p, h=H, seed=SEED)
    S, level = o.slots, len(q) - 1
    rng = np.random.default_rng(5)
    tables = [[rng.uniform(-0.1, 0.1, (16, 16)).astype(np.float32) for _ in range(2)]]
    index = 201
    M = oh.block_diag_matrix(tables)
    sel = oh.expanded_sparse([index], [256], 0, 16)
    d, rots = oh.diagonalize(M, S)
    d = d[(0, 0)]
    idx = list(d.keys())
    data = np.stack([d[i] for i in idx])
    t = o.lt_new(idx, data, level, 2.0)
    scale = float(1 << LOGSCALE)
    ct = o.encrypt(o.encode(sel, level, scale), level, 0)
    lt_out, l = o.lt_eval(t, ct, level)
    resc = o.rescale(lt_out, l)
    rot1 = o.rotate(ct, level, 1)
    out = resc
    ll = l - 1
    for i in range(1, rots + 1):
        out = o.add(out, o.rotate(out, ll, S // 2 ** i), ll)
    out[0] = o.add(out[0][None], o.encode(np.zeros(1, np.float32), ll, scale)[None], ll)[0]
    base = np.arange(o.N, dtype=np.uint64) * np.uint64(2654435761)
    ntt = np.stack([o.ntt(base % np.uint64(m), i) for i, m in enumerate(q + p)])
    fx = dict(logn=LOGN, q=np.array(q, np.uint64), p=np.array(p, np.uint64), logscale=LOGSCALE, h=H, seed=SEED,
              secret_key=o.secret_key().astype(np.int8), selector=sel, table0=tables[0][0], table1=tables[0][1], index=index,
              diag_indices=np.array(idx, np.int32), diag0_plain=o.lt_plaintext(t, idx[0]), ct_in=ct, lt_out=lt_out,
              rescaled=resc, rot1=rot1, pcmm_out=out, fold_rotations=rots, ntt_in=base, ntt_out=ntt,
              expected=oh.radix_lookup(tables[0], index, 16))
    o.close()
    return fx


if __name__ == "__main__":
    fx = generate()
    np.savez_compressed(os.path.join(HERE, "pcmm_n10.npz"), **fx)
    print("wrote", os.path.join(HERE, "pcmm_n10.npz"))
