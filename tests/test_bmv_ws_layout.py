"""CPU model of the whole-share batched mat-vec
(qwen3-4b-q4_k_m-inference-engine_amd/csrc/bmv_ws.hip, bmv_ws.hpp), M = 2..8.

For each shape the model restates the launcher's plan (workgroups per
segment, at most 16 rows each, region and LDS sizes, the staged-activation
and per-lane load limits) and the kernel's addressing, then, for every wave
of a workgroup:
  - every 16-byte weight load lies inside its matrix's dwords;
  - every LDS chunk write lies inside the wave's region of the phase's buffer;
and it simulates the LDS image byte by byte (which global byte each LDS byte
holds, and in which phase it was written), so that every tile field a lane
reads (the Q4_K header and quarter loads, the Q6_K dword runs with their
realignment) is shown to hold exactly the bytes of its row and superblock,
with every read inside the LDS allocation.
Each (part, row, superblock) is computed by exactly one wave, each sums slot
written once, and the totals read only written slots. The arithmetic of the
tiles is the batched kernel's (its lane-level emulation is in
test_bmv_layout.py). The model is its own code restating the kernel's integer
arithmetic; a change to either file must be mirrored here."""
import numpy as np
import pytest

CUS, MAX_LDS, WAVES = 256, 160 * 1024, 8
BYTES = {12: 144, 14: 210}
J, XS, Q8S = 6, 8, 4
LANE = np.arange(64)
LN, LKQ = LANE & 15, LANE >> 4


def act_bytes(K):
    return (8 * (K + 16) + 16 + 4 * K + 15) // 16 * 16


def sums_bytes(parts):
    return parts * 16 * (WAVES // parts) * 8 * 4


def reg_bytes(rpw, row_bytes):
    return (rpw * row_bytes + 2 + 15 + 15) // 16 * 16


def plan(rows, types, K, mode, M, q8in=False):
    """(workgroups per segment, reg, lds) or None when the launcher declines."""
    if not 2 <= M <= 8 or mode not in (0, 1) or (q8in and mode != 0):
        return None
    nseg = 1 if mode == 1 else len(rows)
    parts = 2 if mode == 1 else 1
    S = K // 256
    if nseg > CUS:
        return None
    byt = [rows[j] * S * BYTES[types[j]] * parts for j in range(nseg)]
    total = float(sum(byt))
    count = [min(max(int(CUS * b / total + 0.5), 1), rows[j]) for j, b in enumerate(byt)]
    while sum(count) > CUS:
        count[count.index(max(count))] -= 1
    rpw = 16 // (WAVES // parts)
    rows_max, reg = 0, 0
    for j in range(nseg):
        rows_max = max(rows_max, -(-rows[j] // count[j]))
        rb = S * BYTES[types[j]]
        if (2 + rpw * rb + 15) // 16 > 64 * J:
            return None
        reg = max(reg, reg_bytes(rpw, rb))
    if rows_max > 16:
        return None
    staged = M * (K // 32) - 64 * WAVES * Q8S if q8in else M * (K // 8) - 64 * WAVES * XS
    if staged > 0:
        return None
    lds = act_bytes(K) + sums_bytes(parts) + 8 * reg
    if lds > MAX_LDS:
        return None
    return count, reg, lds


def issue_share(base, nmat_rows, r0, S, B, sb_a, sb_b):
    """The lanes' (global chunk address, LDS offset) of issue_share<J> (gemv_stream.hpp)."""
    rb = S * B
    run = base + r0 * rb + (sb_a if sb_b > sb_a else 0) * B
    o = run & 3
    run4 = run - o
    cmax = max((o + (sb_b - sb_a) * B + 15) >> 4, 1) - 1
    last = base + ((nmat_rows * rb + 3) & ~3) - 16
    lim = last - run4
    c = np.minimum(LANE[:, None] + 64 * np.arange(J)[None, :], cmax)
    a = np.minimum(run4 + 16 * c, last)
    off = np.minimum(16 * c, lim)
    assert np.all(a - run4 == off)
    return a, off, o, run4


def tile_fields(qtype, kq):
    """(first used byte of each field from the superblock start, length) per lane."""
    if qtype == 12:
        return [(np.zeros_like(kq), 16), (16 + 16 * kq, 16), (80 + 16 * kq, 16)]
    return [(16 * kq, 16), (64 + 16 * kq, 16), (128 + 16 * (kq & 1), 16), (160 + 16 * (kq & 1), 16),
            (np.full_like(kq, 192), 16), (np.full_like(kq, 208), 2)]


def check_indices(rows, types, K, mode, M, bases, q8in=False):
    cfg = plan(rows, types, K, mode, M, q8in)
    assert cfg is not None
    count, reg, lds = cfg
    G = 1
    S = K // 256
    parts = 2 if mode == 1 else 1
    wp = WAVES // parts
    rpw = 16 // wp
    nseg = 1 if mode == 1 else len(rows)
    regions = act_bytes(K) + sums_bytes(parts)
    for j in range(nseg):
        B = BYTES[types[j]]
        rb = S * B
        per, rem = rows[j] // count[j], rows[j] % count[j]
        shares = [(g * per + min(g, rem), per + (1 if g < rem else 0)) for g in range(count[j])]
        assert shares[0][0] == 0 and sum(n for _, n in shares) == rows[j]
        assert all(a + n == b for (a, n), (b, _) in zip(shares, shares[1:])), "shares partition the rows"
        chosen = shares if len(shares) <= 24 else [shares[0], shares[max(rem - 1, 0)], shares[min(rem, len(shares) - 1)],
                                                   shares[-1]]
        for r0, nrows in chosen:
            assert nrows <= 16 * G
            holds = np.full(lds, -1, np.int64)    # global byte held by each LDS byte
            phase_of = np.full(lds, -1, np.int64)  # phase that wrote it
            slots = set()
            computed = set()
            for g in range(G):
                buf = regions
                # loads and chunk writes of every wave
                for wave in range(WAVES):
                    part, wv = wave // wp, wave % wp
                    base = bases[1] if (mode == 1 and part) else bases[j]
                    nmat = rows[j]
                    ra, rbn = min(16 * g + rpw * wv, nrows), min(16 * g + rpw * (wv + 1), nrows)
                    a, off, o, run4 = issue_share(base, nmat, r0, S, B, ra * S, rbn * S)
                    assert np.all(a >= base) and np.all(a + 16 <= base + ((nmat * rb + 3) & ~3)), "load outside the matrix"
                    if types[j] == 12:
                        assert np.all(off % 16 == 0)
                    dst = buf + wave * reg + off
                    assert np.all(dst >= buf + wave * reg) and np.all(dst + 16 <= buf + (wave + 1) * reg), \
                        "chunk outside its region"
                    for t in range(16):
                        holds[(dst + t).ravel()] = (a + t).ravel()
                        phase_of[(dst + t).ravel()] = g
                nr = nrows - 16 * g
                if nr <= 0:
                    continue
                # tile reads of every wave
                for wave in range(WAVES):
                    part, wv = wave // wp, wave % wp
                    base = bases[1] if (mode == 1 and part) else bases[j]
                    ic = np.minimum(LN, nr - 1)
                    ra = 16 * g + rpw * (ic // rpw)
                    o = 0 if types[j] == 12 else ((r0 + ra) * rb) & 3
                    rowp = buf + (part * wp + ic // rpw) * reg + o + (ic % rpw) * rb
                    s_lo, s_hi = S * wv // wp, S * (wv + 1) // wp
                    for s in range(s_lo, s_hi):
                        sb = rowp + s * B
                        if types[j] == 12:
                            assert np.all(sb % 16 == 0), "Q4_K superblocks 16-byte aligned in LDS"
                        mis = sb & 3
                        if types[j] == 14:
                            # dword reads dw..dw+4 from sb - mis for each 16-byte field, dwords 52-53 for d
                            for f, _ in tile_fields(14, LKQ)[:5]:
                                lo, hi = sb - mis + f, sb - mis + f + 20
                                assert np.all(lo >= 0) and np.all(hi <= lds), "Q6_K field read outside LDS"
                            assert np.all(sb - mis + 216 <= lds)
                        for f, n in tile_fields(types[j], LKQ):
                            for t in range(n):
                                addr = sb + f + t
                                want = base + (r0 + 16 * g + ic) * rb + s * B + f + t
                                assert np.all(addr < lds)
                                assert np.array_equal(holds[addr], want), "tile byte is not its weight byte"
                                assert np.all(phase_of[addr] == g), "tile byte from another phase"
                        for n_ in range(min(16, nr)):
                            key = (part, r0 + 16 * g + n_, s)
                            assert key not in computed, "tile computed twice"
                            computed.add(key)
                    key = (part, g, wv)
                    assert key not in slots, "sums slot written twice"
                    slots.add(key)
                    slot = ((part * G + g) * 16 + LN) * wp + wv
                    off = act_bytes(K) + 4 * (slot * 8)
                    assert np.all(off + 32 <= regions), "sums slot outside the sums"
            # totals: every wave's slot of every valid row
            for part in range(parts):
                for row in range(nrows):
                    for wv in range(wp):
                        assert (part, row >> 4, wv) in slots
                    for s in range(S):
                        assert (part, r0 + row, s) in computed, "tile never computed"
    return cfg


SHAPES = [  # rows, types, K, mode, M, q8in
    ([2560], [12], 4096, 0, 8, False),                         # attn_output
    ([2560], [12], 4096, 0, 8, True),
    ([2560], [12], 4096, 0, 2, False),
    ([4096], [12], 2560, 0, 8, False),                         # attn_q alone
    ([1024], [14], 2560, 0, 2, False),                         # attn_v alone
    ([1024], [14], 2560, 0, 7, True),
    ([1024, 1024], [12, 14], 2560, 0, 5, False),               # attn k and v
    ([3000, 3000], [14, 14], 1024, 1, 6, False),               # gate/up, 12 rows a workgroup
    ([3000, 3000], [12, 12], 1536, 1, 2, False),
    ([19], [12], 2560, 0, 5, False),
    ([45], [14], 768, 0, 3, False),
    ([101], [14], 1280, 0, 5, True),
    ([3, 1, 2], [12, 12, 14], 256, 0, 7, False),
    ([300, 17], [14, 12], 512, 0, 8, False),
]


@pytest.mark.parametrize("rows,types,K,mode,M,q8in", SHAPES)
def test_bmv_ws_indices_in_bounds(rows, types, K, mode, M, q8in):
    bases = [(1 << 30) * (i + 1) + (4 if t == 14 else 0) for i, t in enumerate(types)]
    check_indices(rows, types, K, mode, M, bases, q8in)


def test_bmv_ws_plan_for_qwen3_shapes():
    """Which M = 8 decode launches the kernel takes (one workgroup per CU, at
    most 16 rows each)."""
    assert plan([2560], [12], 4096, 0, 8)[0] == [256]                 # attn_output: 10 rows a workgroup
    assert plan([4096, 1024, 1024], [12, 12, 14], 2560, 0, 8) is None  # q/k/v: 26 rows
    assert plan([9728, 9728], [12, 12], 2560, 1, 8) is None            # gate/up: 38 rows
    assert plan([2560], [14], 9728, 0, 8, True) is None                # ffn_down: 8 x 9728 activations
    assert plan([151936], [14], 2560, 0, 8) is None                    # lm_head: 593 rows
    assert plan([2560], [12], 4096, 0, 1) is None                      # M = 1: the whole-share kernels
    assert plan([2560], [12], 4096, 0, 9) is None                      # M > 8: the prefill GEMM
    assert plan([1024], [12], 2560, 0, 8, True)[1] == 2 * 1440 + 32    # Q8 input, mode 0
