"""CPU index model of the multi-pass batched mat-vec (csrc/bmv_pass.hpp,
csrc/bmv_pass.hip): the pass plan, every lane's 16-byte chunk of a pass, its
place in the wave's LDS slot, and the superblock bytes the tile reads take
from the slot. A matrix of known bytes goes through the model; every tile
must read exactly its own superblock's bytes, and no access leaves the slot
or the matrix's dwords."""
from __future__ import annotations

import numpy as np
import pytest

Q4, Q6 = 12, 14
BYTES = {Q4: 144, Q6: 210}
MAX_J = 8


def plan(S, qtype):
    """bmv_pass_plan: columns per pass C, chunks per run, chunks per lane J."""
    B = BYTES[qtype]
    best, out = 0.0, None
    for c in range(1, S + 1):
        chunks = (c * B + 11 + 15) // 16
        j = (16 * chunks + 63) // 64
        if j > MAX_J:
            break
        if j < 4:
            continue
        eff = c * B / (16 * 64 * j)
        if eff > best + 1e-9:
            best, out = eff, (c, chunks, j)
    return out


def tile_reads(qtype, o, cc, B):
    """Slot byte offsets (relative to the row's run) that ws_tile reads for
    the superblock at run offset o + cc * B (bmv_ws.hpp): Q4_K 16-byte reads
    of the header and two qs pieces per lane quarter; Q6_K dwords 0..53 from
    the dword boundary at or below the superblock."""
    start = o + cc * B
    if qtype == Q4:
        assert start % 16 == 0
        return list(range(start, start + 144))
    base = start - (start & 3)
    return list(range(base, base + 4 * 54))


@pytest.mark.parametrize("qtype,N,S", [(Q6, 40, 10), (Q6, 37, 3), (Q4, 35, 10), (Q4, 50, 7), (Q6, 20, 38)])
def test_bmv_pass_slot_image(qtype, N, S):
    B = BYTES[qtype]
    C, cpr, J = plan(S, qtype)
    assert 16 * cpr * 16 <= J * 1024  # the pass fits the wave's slot
    row_bytes = S * B
    total = N * row_bytes
    end4 = (total + 3) & ~3
    mat = (np.arange(end4, dtype=np.int64) * 2654435761 % 251).astype(np.uint8)
    mat[total:] = 0
    ppg = (S + C - 1) // C
    groups = (N + 15) // 16
    nchunks = 16 * cpr
    lanes = np.arange(64)
    for g in range(groups):
        for pi in range(ppg):
            c0 = pi * C
            slot = np.full(J * 1024, -1, dtype=np.int64)
            for j in range(J):
                c = np.minimum(lanes + 64 * j, nchunks - 1)
                run, q = c // cpr, c % cpr
                row = np.minimum(16 * g + run, N - 1)
                first = row * row_bytes + min(c0, S - 1) * B
                off = (first & ~3) + 16 * q
                assert np.all(off >= 0)
                for ln in range(64):
                    src = mat[off[ln]:off[ln] + 16] if off[ln] + 16 <= end4 else np.concatenate(
                        [mat[off[ln]:end4], np.zeros(max(0, off[ln] + 16 - max(off[ln], end4)), np.uint8)])
                    dst = 16 * (run[ln] * cpr + q[ln])
                    assert dst + 16 <= J * 1024
                    slot[dst:dst + 16] = src
            for n in range(16):
                row = min(16 * g + n, N - 1)
                o = (row * row_bytes + c0 * B) & 3
                run_base = 16 * cpr * n
                for cc in range(C):
                    s = c0 + cc
                    if s >= S:
                        continue
                    reads = tile_reads(qtype, o, cc, B)
                    assert reads[0] >= 0 and reads[-1] < 16 * cpr  # inside the row's run
                    sb = row * row_bytes + s * B
                    got = slot[run_base + o + cc * B:run_base + o + cc * B + B]
                    assert np.array_equal(got, mat[sb:sb + B].astype(np.int64)), (g, pi, n, cc)
                    # every byte a tile read touches was written by this pass
                    assert np.all(slot[[run_base + r for r in reads]] >= 0)


def test_bmv_pass_plan_lm_head():
    """The lm_head (Q6_K, 10 superblocks a row): passes of 2 columns, 27 chunks
    a run, 7 chunks a lane (432 of 448 loaded), 5 passes per 16-row group."""
    assert plan(10, Q6) == (2, 27, 7)
    assert plan(10, Q4) is not None
