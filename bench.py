"""Benchmark: encrypted embedding lookups/s of the 26-table HE-LRM PCMM at
N=2^16 on one MI355X (libhelrm_hip.so), with the fused diagonal-MAC kernel's
HBM roofline and a bounded CPU-restatement baseline timed on the host.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

One step = one PCMM (one query = 26 lookups): BSGS linear transform of the
encrypted digit one-hot selector by the block-diagonal 416x1248 table matrix
(512 diagonals, 16 baby x 32 giant steps), rescale, 6-rotation hybrid fold,
bias add.  The selector ciphertext, diagonals and keys are resident in HBM
before the timed region.  Prints one JSON line.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "encrypted embedding lookups/sec (26-table PCMM, N=2^16)"
HBM_PEAK_GBS = 8000.0


def mac_unit_bytes(N=1 << 16, L=24, K=8, D=512, n1=16, n2=32, w=8):
    """Algorithmic bytes of the fused diagonal MAC by its per-unit definition:
    every QP diagonal read once, 2*n1 baby-step and 2*n2 giant-step QP
    polynomials (the rotated inputs read, the accumulators written):
    D*(L+K)*N*w + 2*n1*(L+K)*N*w + 2*n2*(L+K)*N*w."""
    return (D + 2 * n1 + 2 * n2) * (L + K) * N * w


# Parts of each key-switching key read from HBM: the library samples the a
# half of every key it generates from a seed and regenerates it inside the
# key product, so only the b half is read (2 for keys loaded whole)
KEY_PARTS = 1


# a diagonal row stored packed (modulus below 2^52) holds 64 words in 104 of 128 dwords
PACKED_ROW_FRACTION = 104 / 128


def algorithmic_bytes(N=1 << 16, L=24, K=8, D=512, n1=16, n2=32, f=6, dnum=3, w=8, chunks=1, fused_babies=True,
                      key_parts=KEY_PARTS, packed_rows=0):
    """Per-PCMM and per-diag-MAC-launch algorithmic HBM bytes (every word once).

    PCMM: the diagonals, the read parts of each of the R rotation keys, the
    input and the output ciphertext.  Diagonal MAC launch, counted as this kernel works (the giant
    groups split evenly over `chunks` launches): its share of the diagonals
    and P*c (2 Q polys, baby step 0) read, one QP accumulator pair per giant
    group of the launch written, and the n1-1 hoisted baby rotations --
    computed in the kernel's prologue from their keys (dnum*key_parts QP polys each)
    and with packed_rows of the (L+K) diagonal rows stored packed (dense
    16-baby transforms: the rows of moduli below 2^52)
    and the decomposed input (dnum QP polys, once) when fused_babies, else
    read (2 QP polys each).  mac_unit_bytes is the per-unit definition the
    roofline is quoted on."""
    R = (n1 - 1) + (n2 - 1) + f
    diag_rows = (L + K) - packed_rows * (1 - PACKED_ROW_FRACTION)
    pcmm = int(D * diag_rows * N * w) + R * dnum * key_parts * (L + K) * N * w + 2 * L * N * w + 2 * (L - 1) * N * w
    if fused_babies:
        babies = (n1 - 1) * dnum * key_parts * (L + K) * N * w + (dnum * (L + K) * N * w if n1 > 1 else 0)
    else:
        babies = (n1 - 1) * 2 * (L + K) * N * w
    diag_mac = int(D * diag_rows * N * w + n2 * 2 * (L + K) * N * w) // chunks + babies + 2 * L * N * w
    return pcmm, diag_mac


def keyswitch_rotation_bytes(level, K, N=1 << 16, w=8, key_parts=KEY_PARTS):
    """Algorithmic bytes of one single key switch (a rotation) at `level`:
    the key (dnum digits x key_parts halves), the dnum decomposed digits and
    the two output parts, each a QP polynomial of level + 1 + K rows.
    key_parts=2 is the per-unit definition (whole keys read); the library
    reads only the b halves of the keys it generated (KEY_PARTS)."""
    nqp = level + 1 + K
    dn = (nqp - 1) // K
    return (dn * key_parts + dn + 2) * nqp * N * w


def keyswitch_pass_rows(level, K, fold_add=False, key_parts=KEY_PARTS):
    """Rows of N words that one single key switch at `level` moves, pass by
    pass (a transform is 2 passes, each reading and writing its limb);
    fold_add: the fold step ct + Rotate(ct) (RotateAdd), whose last pass also
    reads both parts of ct at the output positions."""
    ql = level + 1
    nqp = ql + K
    dn = (nqp - 1) // K
    ext = dn * nqp - ql  # extended digit rows: every QP row but each digit's own
    rows = {
        "inverse NTT of c1": 4 * ql,
        "extension of the digits": ql + ext,
        "forward NTT of the extended rows": 4 * ext,
        "key product": (dn * key_parts + dn + 2) * nqp,
        "inverse NTT of the P rows, both parts": 4 * 2 * K,
        "extension P -> Q, both parts": 2 * K + 2 * ql,
        "forward NTT with the ModDown epilogue": 2 * 2 * ql + (2 * ql + 2 * ql + ql + 2 * ql),
    }
    if fold_add:
        rows["the fold's addend, read in the epilogue"] = 2 * ql
    return rows


def read_traffic(kernel="diag_mac"):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC summary, if present."""
    path = os.path.join(ROOT, "profiles", f"{kernel}_pcmm26_traffic.json")
    if not os.path.exists(path):
        return None
    try:
        with open(path) as f:
            return json.load(f).get("bytes_per_launch")
    except Exception:
        return None


def measured_step_traffic(workload, ms):
    """HBM bytes one PCMM actually moves (every dispatch, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary) and the rate they imply at
    this run's step time; empty for other workloads or without the summary."""
    path = os.path.join(ROOT, "profiles", "pcmm26_traffic.json")
    if workload != "pcmm26" or not os.path.exists(path):
        return {}
    with open(path) as f:
        b = json.load(f)["bytes_per_pcmm"]
    return {"measured_traffic_bytes": b, "measured_traffic_GBs": b / (ms / 1000.0) / 1e9,
            "measured_traffic_frac": b / (ms / 1000.0) / 1e9 / HBM_PEAK_GBS}


def cpu_baseline(q, p, h, key_seed, diagonals, selector, level, logscale, threads, per_step=26, fold=6, repeats=3,
                 single_thread=True):
    """The same PCMM on the CPU restatement (oracle/), whole: encode and
    encrypt of the selector, the BSGS transform over every giant group, rescale,
    fold and bias, with keys and diagonals prepared before the timed region;
    1 warm-up + `repeats` timed runs at `threads` OpenMP threads, the mean
    reported and every trial kept (the reference's protocol,
    examples/criteo/README.md:95-96); then the same on one thread (the
    reference times Lattigo with GOMAXPROCS=1, table2.py:48), whole PCMMs as
    well (about 20 s each).  Returns a dict of the figures."""
    from oracle import oracle as O
    O.set_threads(threads)
    orc = O.Oracle(16, q, p, h=h, seed=key_seed)
    try:
        idx = list(diagonals.keys())
        t_prep = time.perf_counter()
        t = orc.lt_new(idx, np.stack([diagonals[i] for i in idx]), level, 2.0)
        ng = orc.lt_num_giant(t)
        rots = orc.lt_rotations(t)
        for r in rots:
            if r:
                orc.galois_key(orc.galois_element(r))
        slots = orc.slots
        for i in range(1, fold + 1):
            orc.galois_key(orc.galois_element(slots >> i))
        scale = float(1 << logscale)
        t_prep = time.perf_counter() - t_prep

        def pcmm():
            ct = orc.encrypt(orc.encode(selector, level, scale), level, 0)
            out, l = orc.lt_eval(t, ct, level)
            out = orc.rescale(out, l)
            l -= 1
            for i in range(1, fold + 1):
                out = orc.add(out, orc.rotate(out, l, slots >> i), l)
            out[0] = orc.add(out[0][None], orc.encode(np.zeros(1, np.float32), l, scale)[None], l)[0]
            return out
        pcmm()
        trials = []
        for _ in range(repeats):
            t0 = time.perf_counter()
            pcmm()
            trials.append(time.perf_counter() - t0)
        t_pcmm = float(np.mean(trials))
        res = {"value": per_step / t_pcmm, "seconds_per_pcmm": t_pcmm, "trials_s": trials, "prep_s": t_prep,
               "sample": (f"CPU restatement (oracle/), {threads} threads: whole PCMMs (encode + encrypt, BSGS transform "
                          f"of {len(idx)} diagonals over all {ng} giant groups, rescale, {fold}-rotation fold, bias), "
                          f"1 warm-up + {repeats} timed, mean {t_pcmm:.2f} s; keys and diagonals prepared beforehand "
                          f"({t_prep:.1f} s)")}
        if single_thread:
            O.set_threads(1)
            pcmm()
            trials1 = []
            for _ in range(repeats):
                t0 = time.perf_counter()
                pcmm()
                trials1.append(time.perf_counter() - t0)
            t1 = float(np.mean(trials1))
            res["single_thread"] = {
                "value": per_step / t1, "seconds_per_pcmm": t1, "trials_s": trials1, "extrapolated": False,
                "sample": (f"CPU restatement (oracle/), 1 thread: whole PCMMs as above, 1 warm-up + {repeats} timed, "
                           f"mean {t1:.2f} s")}
        return res
    finally:
        orc.close()


def cpu_baseline_dlrm(q, p, w, threads):
    """The whole encrypted DLRM forward (both inputs encrypted at the input
    level, every Linear and activation) on the CPU restatement (oracle/);
    key generation and diagonal encoding happen before the timed region.
    Returns (inferences/s, seconds per forward, sample description)."""
    from oracle import oracle as O
    O.set_threads(threads)
    c = w.cfg
    orc = O.Oracle(c["logn"], q, p, h=c["h"], seed=1)
    try:
        scale = float(1 << c["logscale"])
        slots = orc.slots
        lts = {}
        for name, m in w.modules.items():
            if not hasattr(m, "diagonals"):
                continue
            d = m.diagonals[(0, 0)]
            idx = list(d.keys())
            t = orc.lt_new(idx, np.stack([d[i] for i in idx]), w.levels[name], 2.0)
            for r in orc.lt_rotations(t):
                if r:
                    orc.galois_key(orc.galois_element(r))
            for i in range(1, m.output_rotations + 1):
                orc.galois_key(orc.galois_element(slots >> i))
            lts[name] = (t, m)
        orc.relin_key()
        L = w.input_level
        xd = orc.encrypt(orc.encode(w.dense, L, scale), L, 0)
        xs = orc.encrypt(orc.encode(w.emb.selector, L, scale), L, 1)

        def step(name, x):
            ct, lv, sc = x
            if name in lts:
                t, m = lts[name]
                out, l = orc.lt_eval(t, ct, lv)
                sc2 = sc * orc.q[w.levels[name]]
                out = orc.rescale(out, l)
                sc2 /= orc.q[l]
                l -= 1
                for i in range(1, m.output_rotations + 1):
                    out = orc.add(out, orc.rotate(out, l, slots >> i), l)
                out[0] = orc.add(out[0][None], orc.encode(m.bias, l, scale)[None], l)[0]
                return out, l, sc2
            m = w.modules[name]
            out, nl = orc.eval_poly(ct, lv, sc, list(m.coeffs[::-1]), scale)
            return out, nl, scale
        t0 = time.perf_counter()
        x = (xd, L, scale)
        for _, name in w.bottom_names:
            x = step(name, x)
        e = step("sparse_to_top", step("sparse", (xs, L, scale)))
        z = (orc.add(x[0], e[0], x[1]), x[1], x[2])
        for _, name in w.top_names:
            z = step(name, z)
        t_fwd = time.perf_counter() - t0
        logit = orc.decode_f64(orc.decrypt(z[0], z[1]), z[1], z[2])[0]
        sample = (f"CPU restatement (oracle/), {threads} threads: one whole encrypted forward "
                  f"({len(lts)} Linears, {len(w.activations())} activations; keys and diagonals prepared "
                  f"beforehand), {t_fwd:.2f} s, logit {logit:.6f}")
        return 1.0 / t_fwd, t_fwd, sample
    finally:
        orc.close()


def keyswitch_bytes(N, Lq, K, nb, ng, w=8, key_parts=KEY_PARTS):
    """Algorithmic bytes of one launch of the BSGS key-switch kernels of a
    Linear with Lq active Q limbs: keymac_baby (the nb-1 hoisted baby
    rotations: their keys, the decomposed input once, P*c0 once, the rotated
    QP pairs written) and giant_acc (the ng-1 giant groups: keys, decomposed
    c1 parts and c0 accumulators read, one QP pair written)."""
    nqp, dn = Lq + K, (Lq + K - 1) // K
    nbr, ngk = max(nb - 1, 0), max(ng - 1, 0)
    baby = nbr * dn * key_parts * nqp * N * w + dn * nqp * N * w + Lq * N * w + nbr * 2 * nqp * N * w
    giant = ngk * (dn * key_parts + dn + 1) * nqp * N * w + 2 * nqp * N * w
    return baby, giant


def lt_roofline_bytes(lib, layer, N, K, w=8):
    """(whole-layer, diagonal-MAC) algorithmic bytes of one compiled Linear
    at its level: algorithmic_bytes with L = level + 1 active Q limbs and the
    transform's own baby / giant counts and fold rotations."""
    tid = list(layer.transform_ids.values())[0]
    lti = lib.lt_info(tid)
    Lq = layer.level + 1
    # dense 16-baby transforms keep the rows of moduli below 2^52 packed
    dense16 = lti["baby"] == 16 and lti["plaintexts"] == lti["baby"] * lti["giant"]
    packed = sum(1 for qq in lib.GetModuliChain()[:Lq] if qq < (1 << 52)) if dense16 else 0
    return algorithmic_bytes(N=N, L=Lq, K=K, D=lti["plaintexts"], n1=lti["baby"], n2=lti["giant"],
                             f=layer.output_rotations, dnum=(Lq + K - 1) // K, w=w, packed_rows=packed), lti


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), or None."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def describe(cfg):
    if cfg["kind"] == "dlrm":
        return ("encrypted HE-LRM forward at batch 1: bottom MLP 13-512-256-64-16, 26-table embedding PCMM "
                f"(tables {cfg['rows']}x{cfg['dim']}, base-{cfg['base']} digits), repacking Linears, Add, "
                "top MLP 432-512-256-1, degree-3 activations, no bootstrapping")
    if cfg["kind"] == "pcmm":
        if cfg.get("sizes"):
            return f"{len(cfg['sizes'])}-table embedding PCMM, tables of {cfg['sizes']} rows x {cfg['dim']}"
        d = (f"{cfg['fields']}-table embedding PCMM, tables {cfg['rows']}x{cfg['dim']} as base-{cfg['base']} "
             f"digit sub-tables")
        if cfg.get("repack"):
            w, start = cfg["repack"]
            d += f" + sparse_to_top repack Linear copy_into({cfg['fields'] * cfg['dim']}, {w}, {start})"
        return d
    return f"encrypted dense layer {cfg['out_features']}x{cfg['in_features']}"


def ntt_microbench(lib, reps=5):
    """Batched negacyclic NTT / inverse NTT and RNS multiply-accumulate at the
    kernel-microbenchmark shape (N=2^16, 24 limbs of 50-bit primes, 64
    polynomials), data resident in HBM; per-launch times from HIP events on
    the library's stream.  Replaces the current scheme."""
    import ctypes
    logn, nl, npoly = 16, 24, 64
    qb, pb = (ctypes.c_uint64 * nl)(), (ctypes.c_uint64 * 1)()
    lib.GeneratePrimes(logn, [50] * nl, [61], qb, pb)
    q, p = list(qb), list(pb)
    lib.NewSchemeWithModuli(logn, q, p, 50, 192, 5)
    N = 1 << logn
    rng = np.random.default_rng(1)
    x = np.stack([rng.integers(0, qq, size=(npoly, N), dtype=np.uint64) for qq in q], axis=1)
    d = lib.device_upload(x)
    d2 = lib.device_upload(np.stack([rng.integers(0, qq, size=(npoly, N), dtype=np.uint64) for qq in q], axis=1))
    out = lib.device_empty((nl, N))
    lib.NttDevice(d.ptr, npoly, nl, 1)
    lib.NttDevice(d.ptr, npoly, nl, 0)
    lib.Synchronize()
    lib.KernelTimingEnable(1)
    for _ in range(reps):
        lib.NttDevice(d.ptr, npoly, nl, 1)
        lib.NttDevice(d.ptr, npoly, nl, 0)
        lib.MulAccDevice(d.ptr, d2.ptr, out.ptr, npoly, nl)
    lib.Synchronize()
    res = {}
    for name in ("ntt_batch", "intt_batch", "mulacc"):
        c, tot = lib.kernel_time(name)
        res[name + "_ms"] = tot / c if c else None
    lib.KernelTimingEnable(0)
    ok = np.array_equal(d.download(), x)
    d.free(); d2.free(); out.free()
    butterflies = npoly * nl * (N // 2) * logn
    limb_bytes = npoly * nl * N * 8
    res.update({
        "config": "N=2^16, 24 limbs of 50-bit primes, 64 polynomials, u64 words",
        "butterflies_per_transform": butterflies,
        "ntt_Gbutterflies_per_s": butterflies / (res["ntt_batch_ms"] / 1e3) / 1e9,
        "intt_Gbutterflies_per_s": butterflies / (res["intt_batch_ms"] / 1e3) / 1e9,
        # two passes, each reading and writing every word once
        "ntt_hbm_GBs": 4 * limb_bytes / (res["ntt_batch_ms"] / 1e3) / 1e9,
        # multiply-accumulate reads two batches and writes one sum
        "mulacc_hbm_GBs": (2 * limb_bytes + nl * N * 8) / (res["mulacc_ms"] / 1e3) / 1e9,
        "roundtrip_exact": bool(ok),
    })
    # VALU utilisation: wave-instructions per limb and pass from the committed
    # PMC summary (SQ_INSTS_VALU), times the limbs of the batch, over the
    # measured time, against the integer issue rate probed on this device
    counts = read_valu_counts()
    peak = lib.valu_peak()
    res["valu_peak"] = peak
    if counts:
        limbs = npoly * nl
        for key, kernels in (("ntt", ("ntt_col_fwd", "ntt_row_fwd")), ("intt", ("ntt_row_inv", "ntt_col_inv"))):
            if all(k in counts for k in kernels) and res[key + "_batch_ms"]:
                instr = limbs * sum(counts[k] for k in kernels)
                res[key + "_valu_wave_instr"] = instr
                res[key + "_valu_frac"] = instr / (res[key + "_batch_ms"] / 1e3) / peak["wave_instr_per_s"]
        res["valu_frac"] = res.get("ntt_valu_frac")
    return res


def inflight_bench(lib, w, depth=2, queries=12):
    """Throughput with `depth` different queries in flight on one GPU: query i
    goes to the library's stream i % 2 and the queries are issued back to
    back, so one query's fold and small key switches share the chip with the
    next one's diagonal MAC.  Every output is compared word for word with the
    same query run alone.  Reported beside the batch-1 latency, not instead
    of it."""
    cts = [w.ct_in] + [w.make_query(1000 + k)[0] for k in range(depth - 1)]
    ref = []
    for ct in cts:
        o = w.forward(ct)
        ref.append(lib.export_ciphertext(o.ids[0]))
        o.free()

    def burst(n):
        outs = []
        for i in range(n):
            lib.SetStream(i % 2)
            outs.append(w.forward(cts[i % depth]))
        lib.SetStream(0)
        lib.JoinStream(1)
        return outs
    for o in burst(2 * depth):
        o.free()
    lib.Synchronize()
    t0 = time.perf_counter()
    outs = burst(queries)
    lib.Synchronize()
    t1 = time.perf_counter()
    exact = all(np.array_equal(lib.export_ciphertext(o.ids[0]), ref[i % depth]) for i, o in enumerate(outs))
    for o in outs:
        o.free()
    for ct in cts[1:]:
        ct.free()
    ms = (t1 - t0) * 1000.0 / queries
    return {"depth": depth, "queries": queries, "ms_per_query": ms, "queries_per_s": 1000.0 / ms,
            "outputs_bit_exact_with_serial": bool(exact),
            "note": f"{queries} queries issued back to back, query i on HIP stream i % 2, wall time / queries"}


def read_valu_counts():
    """VALU wave-instructions per limb and pass of the NTT kernels, from the
    committed rocprofv3 PMC summary, if present."""
    path = os.path.join(ROOT, "profiles", "ntt_valu_counts.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("valu_wave_instr_per_limb")


def copy_calibration(mib):
    """A plain device-to-device copy kernel of known size (torch elementwise
    copy), run 3 times, so that the FETCH_SIZE / WRITE_SIZE counters can be
    scaled against bytes that are known exactly."""
    import torch
    n = mib * (1 << 20) // 8
    a = torch.arange(n, dtype=torch.int64, device="cuda")
    b = torch.empty_like(a)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    b.copy_(a)
    e0.record()
    for _ in range(3):
        b.copy_(a)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / 3
    print(json.dumps({"copy_calibration_bytes_read": n * 8, "bytes_written": n * 8, "launches": 4,
                      "copy_GBs": 2 * n * 8 / (ms / 1000.0) / 1e9}), flush=True)


def hbm_ceiling(gib_list=(1, 4)):
    """The streaming rates plain torch kernels reach on this GPU, for reading
    the roofline fractions against what a copy achieves: a device copy (read +
    write), a fill (write only) and a sum (read only) of 1 and 4 GiB of
    int64, 5 launches each after one untimed, HIP events on torch's stream.
    One JSON line per size."""
    import torch

    def per_launch_s(f, reps=5):
        f()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            f()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps / 1000.0

    for gib in gib_list:
        n = gib * (1 << 30) // 8
        a = torch.ones(n, dtype=torch.int64, device="cuda")
        b = torch.empty_like(a)
        cp = per_launch_s(lambda: b.copy_(a))
        fl = per_launch_s(lambda: b.fill_(3))
        sm = per_launch_s(lambda: torch.sum(a))
        print(json.dumps({"hbm_ceiling_GiB": gib, "copy_rw_GBs": 2 * n * 8 / cp / 1e9,
                          "fill_w_GBs": n * 8 / fl / 1e9, "sum_r_GBs": n * 8 / sm / 1e9}), flush=True)
        del a, b
        torch.cuda.empty_cache()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="pcmm26")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-ntt-microbench", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--no-single-thread-baseline", action="store_true",
                    help="skip the one-thread timing of the CPU restatement's sample")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--seeded-upload", action="store_true",
                    help="upload the selector as (b, seed) and rebuild a on the device inside every step")
    ap.add_argument("--no-concurrent", action="store_true",
                    help="dlrm: run the lookup path after the bottom MLP on one stream instead of beside it")
    ap.add_argument("--no-lt-prerescale", action="store_true",
                    help="transforms return the un-rescaled result and the host rescales (Lattigo's convention); "
                         "by default they return the rescaled one (lt_output_prerescaled: the first rescale fused "
                         "into the final ModDown, the same residues)")
    ap.add_argument("--inflight", type=int, default=2, metavar="D",
                    help="also measure throughput with D different queries in flight on two HIP streams "
                         "(embedding PCMM workloads; 0: skip)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (PMC counter calibration) and exit")
    ap.add_argument("--hbm-ceiling", action="store_true",
                    help="only measure the copy / fill / sum rates of plain torch kernels over 1 and 4 GiB and exit")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.hbm_ceiling:
        hbm_ceiling()
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: the PCMM runs on a single MI355X (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE {world}); sharding the PCMM over several GPUs is not built.", file=sys.stderr)
        sys.exit(2)

    from helrm_amd.backend import HipLibrary
    from helrm_amd.workloads import make_workload, CONFIGS

    lib = HipLibrary()
    t_setup = time.perf_counter()
    w = make_workload(lib, args.workload, seed=args.seed, key_seed=1).setup()
    t_setup = time.perf_counter() - t_setup
    info = w.shape_info()
    cfg = CONFIGS[args.workload]
    lib.set_lt_output_prerescaled(not args.no_lt_prerescale)
    prerescaled = bool(lib.lt_output_prerescaled)
    if hasattr(w, "concurrent"):
        w.concurrent = not args.no_concurrent
    if args.seeded_upload:
        w.use_seeded_upload(0x5EED + args.seed)
    sel = w.ct_sparse if cfg["kind"] == "dlrm" else w.ct_in
    upload = {"seeded": bool(args.seeded_upload),
              "bytes": sum((lib.GetCiphertextBxBytes(c) + 8) if args.seeded_upload else lib.GetCiphertextBytes(c)
                           for c in sel.ids),
              "full_ciphertext_bytes": sum(lib.GetCiphertextBytes(c) for c in sel.ids)}

    # correctness of the benchmarked path (outside the timed region)
    out = w.run()
    err = float(np.abs(w.decrypt_output(out) - w.expected).max())
    out.free()

    for _ in range(args.warmup):
        o = w.run()
        o.free()
    lib.Synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        o = w.run()
        o.free()
    lib.Synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) * 1000.0 / args.steps
    # one step = one query: one lookup per table for the embedding PCMM, one forward of the dense layer or DLRM
    per_step = len(cfg.get("sizes") or [0] * cfg.get("fields", 1)) if cfg["kind"] == "pcmm" else 1
    lookups = per_step / (ms / 1000.0)
    if cfg["kind"] == "pcmm":
        metric, unit = (METRIC if args.workload == "pcmm26" else f"encrypted embedding lookups/sec ({args.workload})"), "lookups/s"
    elif cfg["kind"] == "dlrm":
        metric, unit = f"encrypted DLRM inferences/sec (HE-LRM forward, batch 1, {args.workload})", "inferences/s"
    else:
        metric, unit = f"encrypted dense-layer forwards/sec ({args.workload})", "forwards/s"
    stages = None
    if cfg["kind"] == "dlrm":
        o, st = w.run_staged(lib.Synchronize, time.perf_counter)
        o.free()
        stages = {k: v * 1000.0 for k, v in st.items()}
        layer_ms = {k: v * 1000.0 for k, v in w.layer_s.items()}

    # per-kernel HIP-event timings (separate, untimed passes): a 50 ms idle gap
    # on either side marks them in a kernel trace of this run; the first step
    # after the gap (clocks coming back up) is not timed.  A DLRM forward runs
    # them on one stream, so that no kernel shares the chip with another.
    nprof = 3
    concurrent = getattr(w, "concurrent", False)
    if concurrent:
        w.concurrent = False
    lib.Synchronize()
    time.sleep(0.05)
    o = w.run()
    o.free()
    lib.KernelTimingEnable(1)
    for _ in range(nprof):
        o = w.run()
        o.free()
    lib.Synchronize()
    kt = {}
    for name in ("diag_mac", "giant_acc", "rotate"):
        c, tot = lib.kernel_time(name)
        kt[name] = {"launches": c, "avg_ms": tot / c if c else None}
    lib.KernelTimingEnable(0)
    time.sleep(0.05)
    if concurrent:
        w.concurrent = True

    L, K = len(cfg["logq"]), len(cfg["logp"])
    N = 1 << cfg["logn"]
    # diagonal-MAC launches per step (one per 32 baby steps of every Linear)
    launches = max(1, round(kt["diag_mac"]["launches"] / nprof)) if kt["diag_mac"]["launches"] else 1
    layers = w.linear_layers()
    step_bytes, mac_bytes, mac_unit, lt_shapes = 0, 0, 0, []
    ks_bytes = {"giant_acc": 0}
    for layer in layers:
        (b_layer, b_mac), lti = lt_roofline_bytes(lib, layer, N, K)
        step_bytes += b_layer
        mac_bytes += b_mac
        mac_unit += mac_unit_bytes(N=N, L=layer.level + 1, K=K, D=lti["plaintexts"], n1=lti["baby"], n2=lti["giant"])
        _, kg = keyswitch_bytes(N, layer.level + 1, K, lti["baby"], lti["giant"])
        ks_bytes["giant_acc"] += kg if lti["giant"] > 1 else 0
        lt_shapes.append({"level": layer.level, "diagonals": lti["plaintexts"], "baby": lti["baby"],
                          "giant": lti["giant"], "fold": layer.output_rotations})
    if cfg["kind"] == "dlrm":
        # each degree-3 activation reads the relinearisation key twice at its level
        for name, _ in w.activations():
            lq = w.levels[name] + 1
            step_bytes += 2 * ((lq + K - 1) // K) * KEY_PARTS * (lq + K) * N * 8
    # algorithmic bytes per diagonal-MAC launch over one step: the per-unit
    # definition (diagonals + 2*n1 baby-step + 2*n2 giant-step QP polynomials)
    # is the roofline; the kernel's own count (it computes the baby rotations
    # in its prologue from their keys and the decomposed input, so it reads
    # those instead of rotated polynomials) is reported beside it
    unit_per_launch = mac_unit / launches
    mac_per_launch = mac_bytes / launches
    mac_ms = kt["diag_mac"]["avg_ms"]
    achieved = unit_per_launch / (mac_ms / 1000.0) / 1e9 if mac_ms else None
    achieved_k = mac_per_launch / (mac_ms / 1000.0) / 1e9 if mac_ms else None
    roofline = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": (achieved / HBM_PEAK_GBS) if achieved else None,
                "traffic": read_traffic("diag_mac") if args.workload == "pcmm26" else None,
                "kernel": "diag_mac_d16_kernel", "algorithmic_bytes_per_launch": unit_per_launch,
                "launches_per_step": launches,
                "definition": "D*(L+K)*N*w diagonals + 2*n1*(L+K)*N*w + 2*n2*(L+K)*N*w baby- and giant-step QP polynomials",
                "kernel_count": {"algorithmic_bytes_per_launch": mac_per_launch, "achieved": achieved_k,
                                 "frac": (achieved_k / HBM_PEAK_GBS) if achieved_k else None,
                                 "definition": ("diagonals (rows of moduli below 2^52 packed, 104 of 128 dwords), the b "
                                                "halves of the hoisted baby rotations' keys (the a halves "
                                                "regenerated from their seed) and the decomposed input (the "
                                                "rotations computed in the prologue), P*c, one QP accumulator "
                                                "pair per giant group")}}
    lti = lib.lt_info(list(layers[0].transform_ids.values())[0])
    # the key-switch kernels of the transforms against the same peak
    kernel_rooflines = {"diag_mac": {"algorithmic_bytes_per_launch": unit_per_launch, "avg_ms": mac_ms,
                                     "achieved_GBs": achieved, "frac": roofline["frac"],
                                     "kernel_count_bytes_per_launch": mac_per_launch,
                                     "kernel_count_frac": roofline["kernel_count"]["frac"]}}
    for name, total in ks_bytes.items():
        n_l = kt[name]["launches"] / nprof if kt[name]["launches"] else 0
        if not n_l or not kt[name]["avg_ms"]:
            continue
        per = total / n_l
        gbs = per / (kt[name]["avg_ms"] / 1000.0) / 1e9
        kernel_rooflines[name] = {"algorithmic_bytes_per_launch": per, "avg_ms": kt[name]["avg_ms"],
                                  "achieved_GBs": gbs, "frac": gbs / HBM_PEAK_GBS}

    # the single-ciphertext key switch: the fold's rotations (one key switch
    # each at the transform's output level, the fold's add inside its last
    # pass) against the per-rotation bytes
    if kt["rotate"]["launches"] and len(layers) == 1:
        lf = layers[0].level - 1  # the fold runs on the rescaled transform output
        nqp, dn = lf + 1 + K, (lf + 1 + K - 1) // K
        rb = keyswitch_rotation_bytes(lf, K, N)
        r_ms = kt["rotate"]["avg_ms"]
        pb = sum(keyswitch_pass_rows(lf, K, fold_add=True).values()) * N * 8
        # the per-unit definition counts whole keys (both halves read)
        ub = keyswitch_rotation_bytes(lf, K, N, key_parts=2)
        kernel_rooflines["keyswitch_rotation"] = {
            "level": lf, "algorithmic_bytes_per_rotation": rb, "avg_ms": r_ms,
            "rotations_per_step": kt["rotate"]["launches"] / nprof,
            "achieved_GBs": rb / (r_ms / 1000.0) / 1e9, "frac": rb / (r_ms / 1000.0) / 1e9 / HBM_PEAK_GBS,
            "per_unit_bytes_per_rotation": ub, "per_unit_frac": ub / (r_ms / 1000.0) / 1e9 / HBM_PEAK_GBS,
            "pass_bytes_per_rotation": pb, "pass_GBs": pb / (r_ms / 1000.0) / 1e9,
            "pass_frac": pb / (r_ms / 1000.0) / 1e9 / HBM_PEAK_GBS}
        # the floor the rotation's 11 dependent launches sit on: an empty
        # dependent launch, and plain copies of the Q rows and of the
        # extended QP rows (LaunchProbe, same stream)
        lp_q, lp_x = lib.launch_probe(lf + 1), lib.launch_probe(dn * nqp - (lf + 1))
        kernel_rooflines["keyswitch_rotation"]["launch_probe"] = {
            "empty_launch_us": lp_q["empty_launch_us"], "copy_q_rows_us": lp_q["copy_us"],
            "copy_q_rows_TBs": lp_q["copy_TBs"], "copy_extended_rows_us": lp_x["copy_us"],
            "copy_extended_rows_TBs": lp_x["copy_TBs"], "q_rows": lf + 1, "extended_rows": dn * nqp - (lf + 1)}

    cpu = None
    if not args.no_cpu_baseline and cfg["kind"] == "dlrm":
        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
        v, t_cpu, sample = cpu_baseline_dlrm(lib.GetModuliChain(), lib.GetAuxModuliChain(), w, threads)
        cpu = {"value": v, "unit": unit, "cores": threads, "kind": "port", "sample": sample,
               "seconds_per_forward": t_cpu}
    elif not args.no_cpu_baseline:
        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
        d = w.layer.diagonals[(0, 0)]
        r = cpu_baseline(lib.GetModuliChain(), lib.GetAuxModuliChain(), cfg["h"], 1, d, w.input, w.layer.level,
                         cfg["logscale"], threads, per_step, fold=w.layer.output_rotations,
                         single_thread=not args.no_single_thread_baseline)
        cpu = {"value": r["value"], "unit": unit, "cores": threads, "kind": "port", "sample": r["sample"],
               "seconds_per_pcmm": r["seconds_per_pcmm"], "trials_s": r["trials_s"], "prep_s": r["prep_s"],
               "cpu_model": cpu_model(), "host_cpus": os.cpu_count()}
        if "single_thread" in r:
            cpu["single_thread"] = r["single_thread"]

    inflight = None
    if args.inflight > 1 and cfg["kind"] == "pcmm" and not args.seeded_upload:
        inflight = inflight_bench(lib, w, args.inflight)
        inflight["lookups_per_s"] = inflight["queries_per_s"] * per_step
    ntt = None if args.no_ntt_microbench else ntt_microbench(lib)

    line = {
        "metric": metric,
        "value": lookups,
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u64",
        "data": "synthetic (seeded tables / weights and inputs, seeded keys and encryption randomness)",
        "config": {"workload": f"{args.workload}: {describe(cfg)}, N=2^{cfg['logn']}, "
                               f"L={L} (60+50x{L - 1} bit), K={K} (61 bit), dnum={(L + K - 1) // K}, scale 2^{cfg['logscale']}"},
        "end_to_end_hbm": {"algorithmic_bytes": step_bytes,
                           "achieved_GBs": step_bytes / (ms / 1000.0) / 1e9,
                           "frac": step_bytes / (ms / 1000.0) / 1e9 / HBM_PEAK_GBS,
                           **measured_step_traffic(args.workload, ms)},
        "kernels": kt,
        "linear_transforms": lt_shapes,
        "selector_upload": upload,
        "lt_output_prerescaled": prerescaled,
        "roofline": roofline,
        "kernel_rooflines": kernel_rooflines,
        "cpu_baseline": cpu,
        "max_abs_err_vs_plaintext": err,
        "inflight": inflight,
        "ntt_microbench": ntt,
        "setup_s": t_setup,
    }
    if cfg["kind"] == "dlrm":
        line["concurrent_lookup"] = bool(w.concurrent)
        line["stage_ms"] = stages
        line["layer_ms"] = layer_ms
        line["levels"] = {"input": w.input_level, "add": w.add_level, "output": 0}
    else:
        line["config"].update({"diagonals": info["diagonals"], "baby_steps": lti["baby"], "giant_steps": lti["giant"],
                               "fold_rotations": info["output_rotations"], "matrix": info["matrix"]})
        line["pcmm_ms"] = ms
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
