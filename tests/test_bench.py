"""bench.py's contract pieces that need no GPU: the refusal of more than one
GPU and the algorithmic byte counts its rooflines divide by."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr or "single MI355X" in r.stderr


def test_pcmm26_algorithmic_bytes():
    """N=2^16, L=24, K=8, D=512, 16 baby x 32 giant steps, 6 fold rotations,
    dnum=3: diagonals + the b halves of 52 rotation keys (the a halves are
    regenerated from their seed) + input + output ciphertexts, and the
    diagonal-MAC launch: diagonals, the key halves of the 15 hoisted baby
    rotations and the 3 decomposed digits (the rotations are computed in its
    prologue), P*c, 32 QP accumulator pairs; with the rotations read instead,
    15 rotated QP pairs take the place of keys and digits."""
    pcmm, mac = bench.algorithmic_bytes()
    assert pcmm == 11_256_463_360
    assert mac == 10_494_148_608
    N, w, nqp = 1 << 16, 8, 32
    assert pcmm == (512 * nqp + 52 * 3 * nqp) * N * w + 2 * 24 * N * w + 2 * 23 * N * w
    assert mac == (512 * nqp + 15 * 3 * nqp + 3 * nqp + 32 * 2 * nqp) * N * w + 2 * 24 * N * w
    # keys read whole (both halves), as for keys loaded from outside
    pcmm2, mac2 = bench.algorithmic_bytes(key_parts=2)
    assert pcmm2 - pcmm == 52 * 3 * nqp * N * w
    assert mac2 == 11_249_123_328
    # the 23 rows of 50-bit moduli stored packed: 104 of 128 dwords per 64 words
    pcmm3, mac3 = bench.algorithmic_bytes(packed_rows=23)
    assert pcmm - pcmm3 == mac - mac3 == 512 * 23 * (N // 64) * (128 - 104) * 4
    assert mac3 == 9_336_520_704
    _, unfused = bench.algorithmic_bytes(fused_babies=False)
    assert unfused == 10_192_158_720
    assert unfused == 512 * nqp * N * w + 15 * 2 * nqp * N * w + 2 * 24 * N * w + 32 * 2 * nqp * N * w


def test_mac_unit_bytes():
    """The fused MAC by its per-unit definition: 512 QP diagonals, 2 x 16
    baby-step and 2 x 32 giant-step QP polynomials of 32 rows of 2^16 words."""
    assert bench.mac_unit_bytes() == 10_200_547_328
    assert bench.mac_unit_bytes() == (512 + 2 * 16 + 2 * 32) * 32 * (1 << 16) * 8
    # the dense 512x256 layer at 16 limbs (K=6): same split, 22 QP rows
    assert bench.mac_unit_bytes(L=16, K=6) == (512 + 32 + 64) * 22 * (1 << 16) * 8


def test_keyswitch_kernel_bytes():
    """keymac_baby: 15 key b halves of 3 digits x 32 QP rows, the 3 digits
    once, P*c0 (24 rows) once, 15 rotated QP pairs; giant_acc: 31 key b
    halves, their digits and c0 accumulators, one QP pair out."""
    baby, giant = bench.keyswitch_bytes(1 << 16, 24, 8, 16, 32)
    row = (1 << 16) * 8
    assert baby == (15 * 3 * 32 + 3 * 32 + 24 + 15 * 2 * 32) * row
    assert giant == (31 * (3 + 3 + 1) * 32 + 2 * 32) * row
    baby2, giant2 = bench.keyswitch_bytes(1 << 16, 24, 8, 16, 32, key_parts=2)
    assert (baby2 - baby, giant2 - giant) == (15 * 3 * 32 * row, 31 * 3 * 32 * row)


@pytest.mark.parametrize("lq,nb,ng", [(1, 1, 1), (8, 4, 4)])
def test_keyswitch_bytes_without_rotations(lq, nb, ng):
    baby, giant = bench.keyswitch_bytes(1 << 13, lq, 8, nb, ng)
    assert baby >= 0 and giant >= 0
    if nb == 1:
        assert baby == ((lq + 7) // 8) * (lq + 8) * (1 << 13) * 8 + lq * (1 << 13) * 8


def test_keyswitch_rotation_bytes():
    """One rotation at level 22 of the 24-limb chain (23 Q + 8 P rows of 2^16
    words, 3 digits): whole keys 3 x 2 x 31 rows, digits 3 x 31, output
    2 x 31 = 341 rows of 512 KiB = 178,782,208 B by the per-unit definition;
    with the b halves only (a halves regenerated), 248 rows."""
    assert bench.keyswitch_rotation_bytes(22, 8, key_parts=2) == 341 * (1 << 16) * 8 == 178_782_208
    assert bench.keyswitch_rotation_bytes(22, 8, key_parts=1) == 248 * (1 << 16) * 8 == 130_023_424
    # a smaller chain: level 3, K = 1 -> 5 QP rows, 4 digits
    assert bench.keyswitch_rotation_bytes(3, 1, N=1 << 13, key_parts=2) == (4 * 2 + 4 + 2) * 5 * (1 << 13) * 8


def test_keyswitch_pass_rows():
    """One rotation at level 22 (23 Q limbs, K=8, 3 digits of 8, 8, 7 rows):
    inverse NTT of 23 limbs (92 rows), extension 23 -> 70 rows (93), forward
    NTT of 70 limbs (280), key product 8 x 31 rows (248: 3 key b halves, 3
    digits, 2 outputs), inverse NTT of 16 P limbs (64), extension 16 -> 46 rows
    (62), forward NTT of 46 limbs whose last pass also reads x and c0
    (92 + 161): 1,092 rows = 572,522,496 B."""
    rows = bench.keyswitch_pass_rows(22, 8)
    assert list(rows.values()) == [92, 93, 280, 248, 64, 62, 253]
    assert sum(rows.values()) * (1 << 16) * 8 == 572_522_496
    # the key product alone is the per-rotation figure of the key-switch roofline
    assert rows["key product"] * (1 << 16) * 8 == 130_023_424
    # keys read whole: 3 more halves of 31 rows
    assert bench.keyswitch_pass_rows(22, 8, key_parts=2)["key product"] == 341
    # the fold step ct + Rotate(ct): its last pass also reads both parts of ct
    folded = bench.keyswitch_pass_rows(22, 8, fold_add=True)
    assert sum(folded.values()) == 1092 + 2 * 23


def test_measured_step_traffic():
    """The whole-PCMM traffic of the committed PMC summary, as a rate at a step time."""
    r = bench.measured_step_traffic("pcmm26", 7.0)
    # the key switches' passes move more than the algorithmic bytes
    assert r["measured_traffic_bytes"] > 2 * bench.algorithmic_bytes(packed_rows=23)[0]
    assert abs(r["measured_traffic_GBs"] - r["measured_traffic_bytes"] / 7e-3 / 1e9) < 1e-6
    assert bench.measured_step_traffic("dlrm", 7.0) == {}
