"""CPU model of the multi-pass mat-vec's plan and indexing (csrc/gemv_pass.hip,
csrc/gemv_pass.hpp): the launcher's choice of rows per pass R and loads per
lane J, every worker's passes, the buffer range of each pass and the LDS
offsets of its chunks. Checks, for the shapes the kernel takes: every row is
computed exactly once, no chunk load starts outside the matrix's dwords (the
descriptor's range ends at the dword boundary at or above the matrix end),
every chunk lands inside the wave's J KB slot, and the pieces a pass reads
(superblock q/4 of the pass, its bytes from the run's dword base) lie inside
the chunks written.
"""
from __future__ import annotations

import numpy as np
import pytest

Q4, Q6 = 12, 14
B = {Q4: 144, Q6: 210}
WAVES, SUMS, MAX_J = 16, 64, 8


def pass_plan(S: int, qtype: int):
    """gemv_pass.hip pass_plan: the (R, J) reading the fewest wasted chunk bytes."""
    rb = S * B[qtype]
    best, R, J = 0.0, 0, 0
    for j in range(4, MAX_J + 1):
        r = min(16, SUMS // S, (1024 * j - 2) // rb)
        if r < 1:
            continue
        eff = r * rb / (1024.0 * j)
        if eff > best + 1e-9:
            best, R, J = eff, r, j
    return R, J


def pass_rows(p, k, W, R, full, last_a, last_b):
    if p < full:
        return (p * W + k) * R, R
    return last_a, last_b - last_a


def check_shape(qtype: int, K: int, N: int, G: int = 256, base_offset: int = 0):
    S = K // 256
    rb = S * B[qtype]
    R, J = pass_plan(S, qtype)
    assert R >= 1
    W = G * WAVES
    full = N // (W * R)
    rest = N - full * W * R
    npass = full + (rest > 0)
    end4 = (N * rb + 3) & ~3
    seen = np.zeros(N, np.int32)
    for k in range(W):
        last_a = full * W * R + k * rest // W
        last_b = full * W * R + (k + 1) * rest // W
        for p in range(npass):
            ra, nr = pass_rows(p, k, W, R, full, last_a, last_b)
            assert 0 <= nr <= R and 4 * nr * S <= 4 * SUMS
            seen[ra:ra + nr] += 1
            run = base_offset + ra * rb  # the weight pointer is dword-aligned
            o = run & 3
            run4 = run - o - base_offset
            cmax = max((o + nr * rb + 15) >> 4, 1) - 1
            rng = end4 - run4  # buffer range from the run's dword base
            assert rng >= 0
            # loads: chunk c = min(lane + 64 j, cmax) at 16 c; bytes past rng read as zero
            assert 16 * cmax < max(rng, 16)
            # LDS: chunks at 16 c of the J KB slot
            assert 16 * cmax + 16 <= 1024 * J
            # pieces: superblock q/4 at o + 210/144 * (q/4), read from its dword base
            if nr:
                last_sb = nr * S - 1
                end_byte = o + last_sb * B[qtype] + B[qtype]
                assert end_byte <= 16 * cmax + 16 and end_byte <= 1024 * J
                # every byte the pieces need was loaded (within the range)
                assert run4 + ((end_byte + 3) & ~3) <= end4 + 0
    assert (seen == 1).all(), (seen.min(), seen.max())
    return R, J, full, rest, npass


@pytest.mark.parametrize("qtype,K,N", [
    (Q6, 2560, 151936),   # lm_head
    (Q6, 2560, 20001), (Q4, 2560, 40003), (Q6, 2816, 20001), (Q4, 9728, 17000), (Q6, 256, 200003),
    (Q6, 9728, 2560), (Q4, 2560, 9728), (Q4, 256, 77), (Q6, 2560, 19), (Q6, 2560, 4096),
])
def test_pass_plan_covers_every_row_in_bounds(qtype, K, N):
    check_shape(qtype, K, N)


def test_pass_plan_lm_head_values():
    """The lm_head runs passes of 3 rows (6300 B) in 7 KB, 12 full rounds over
    4096 waves, then 4480 rows split over the waves."""
    assert check_shape(Q6, 2560, 151936) == (3, 7, 12, 4480, 13)


def test_pass_plan_rejects_rows_over_8_kb():
    assert pass_plan(39, Q6) == (1, 8)  # 8190 B + 2 fit
    assert pass_plan(40, Q6)[0] == 0    # 8400 B do not
