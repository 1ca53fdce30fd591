"""CPU model of the whole-share mat-vec's work split and addressing
(qwen3-4b-q4_k_m-inference-engine_amd/csrc/gemv_stream.hip, gemv_stream.hpp):
for each shape, every global read, LDS write, piece read, Q8-block read and
superblock-sum index of every lane of every wave of every workgroup is checked
against its buffer, and every superblock of every row is shown to be covered
exactly once. The model restates the launcher's and kernel's integer arithmetic
(its own code, vectorised over workgroups, waves and lanes); a change to either
file must be mirrored here."""
import numpy as np
import pytest

CUS, MAX_LDS, WAVES, MAX_J, XSTAGED = 256, 160 * 1024, 16, 8, 2
BYTES = {12: 144, 14: 210}
MAX_K = 8 * 64 * WAVES * XSTAGED


def launcher(rows, types, K, mode):
    """(workgroups per segment, J, max_sb, lds bytes) or None when the streaming kernel is used."""
    S = K // 256
    if K > MAX_K:
        return None
    nseg = 1 if mode in (1, 3) else len(rows)
    parts = 2 if mode in (1, 3) else 1
    wpp = WAVES // parts
    byt = [rows[j] * S * BYTES[types[j]] * parts for j in range(nseg)]
    total = float(sum(byt))
    count = [min(max(int(CUS * b / total + 0.5), 1), rows[j]) for j, b in enumerate(byt)]
    while sum(count) > CUS:
        count[count.index(max(count))] -= 1
    J, max_sb = 0, 0
    for j in range(nseg):
        rows_max = -(-rows[j] // count[j])
        sb = rows_max * S
        wave_bytes = 2 + -(-sb // wpp) * BYTES[types[j]]
        J = max(J, min(-(-(-(-wave_bytes // 16)) // 64), MAX_J + 1))
        max_sb = max(max_sb, sb)
    if J > MAX_J:
        return None
    lds = S * 8 * 48 + WAVES * J * 1024 + parts * max_sb * 4 + (4 * WAVES if mode == 3 else 0)
    if lds > MAX_LDS:
        return None
    return count, J, max_sb, lds


def check_shape(rows, types, K, mode, bases):
    cfg = launcher(rows, types, K, mode)
    if cfg is None:
        return False
    count, J, max_sb, lds = cfg
    S = K // 256
    parts = 2 if mode in (1, 3) else 1
    wpp = WAVES // parts
    nseg = 1 if mode in (1, 3) else len(rows)
    seen = [np.zeros((parts, rows[j] * S), np.int64) for j in range(nseg)]
    wave = np.arange(WAVES)[:, None, None]
    lane = np.arange(64)[None, :, None]
    jj = np.arange(J)[None, None, :]
    for j in range(nseg):
        B = BYTES[types[j]]
        rb = S * B
        per, rem = rows[j] // count[j], rows[j] % count[j]
        for g in range(count[j]):
            r0 = g * per + min(g, rem)
            r1 = r0 + per + (1 if g < rem else 0)
            assert 0 <= r0 < r1 <= rows[j]
            nsb = (r1 - r0) * S
            assert nsb <= max_sb
            part, wv = wave // wpp, wave % wpp
            sb_a, sb_b = nsb * wv // wpp, nsb * (wv + 1) // wpp
            base = np.where(part == 1, bases[1] if mode in (1, 3) else 0, bases[j])
            run = base + r0 * rb + np.where(sb_b > sb_a, sb_a, 0) * B
            o = run & 3
            if types[j] == 12:
                assert np.all(run % 16 == 0)
            run4 = run - o
            L = np.maximum((o + (sb_b - sb_a) * B + 15) >> 4, 1)
            end = base + rows[j] * rb
            last = base + ((rows[j] * rb + 3) & ~3) - 16
            c = np.minimum(lane + 64 * jj, L - 1)
            a = np.minimum(run4 + 16 * c, last)
            # global reads: 16 bytes inside the matrix's dwords, dword aligned
            assert np.all(a >= base) and np.all(a + 16 <= ((end + 3) & ~3)) and np.all(a % 4 == 0)
            off = a - run4
            # LDS writes inside the wave's region
            assert np.all(off >= 0) and np.all(off + 16 <= J * 1024)
            # the written bytes cover the run: chunk c < L-1 unmoved, so [0, 16(L-1)) and the last chunk
            cov_end = np.maximum(16 * (L - 1), np.minimum(16 * (L - 1), last - run4) + 16)
            assert np.all(cov_end >= o + (sb_b - sb_a) * B)
            # pieces: superblock offsets and Q6_K field reads inside the superblock
            for w in range(WAVES):
                a_, b_ = int(sb_a[w, 0, 0]), int(sb_b[w, 0, 0])
                seen[j][int(part[w, 0, 0]), r0 * S + a_: r0 * S + b_] += 1
                q = np.arange(4 * (b_ - a_))
                s = (a_ + (q >> 2)) % S
                pc = q & 3
                blk = s * 8 + np.where(types[j] == 12, 2 * pc, 4 * (pc >> 1) + (pc & 1))
                step = 1 if types[j] == 12 else 2
                assert np.all(blk + step < S * 8)
                assert np.all(int(part[w, 0, 0]) * max_sb + a_ + (q >> 2) < parts * max_sb)
    for j in range(nseg):
        assert np.all(seen[j] == 1), "every superblock of every row exactly once"
    assert lds <= MAX_LDS
    if mode == 3:
        # the norm scale is staged like x: task t reads scale[8t, 8t+8), t
        # clamped to the last task; the quantiser waves' partial sums of
        # squares follow the superblock sums of both parts
        groups = K // 8
        nq = min(WAVES, -(-groups // (64 * XSTAGED)))
        t = np.minimum(np.arange(64 * nq)[:, None] + 64 * nq * np.arange(XSTAGED)[None, :], groups - 1)
        assert t.min() >= 0 and 8 * t.max() + 8 <= K
        norm_part = S * 8 * 48 + WAVES * J * 1024 + 4 * (2 * max_sb)
        assert norm_part % 4 == 0 and norm_part + 4 * nq <= lds
    return True


SHAPES = [
    ([2560], [14], 9728, 0),             # ffn_down / config 1
    ([9728], [12], 2560, 0),             # config 0
    ([9728, 9728], [12, 12], 2560, 1),   # gate + up
    ([2560], [12], 4096, 0),             # attn_output
    ([4096, 1024, 1024], [12, 12, 14], 2560, 0),  # q/k/v
    ([3, 1, 2], [12, 12, 14], 256, 0),
    ([1], [14], 256, 0),
    ([5], [14], 2560, 0),
    ([101], [12], 3328, 0),
    ([101], [14], 9728, 0),
    ([1000], [14], 2560, 0),
    ([64], [14], 9728, 0),
    ([5, 5], [14, 14], 2560, 1),
    ([9728, 9728], [12, 12], 2560, 3),   # ffn_norm + gate + up
    ([5, 5], [12, 12], 256, 3),
    ([37, 37], [14, 14], 512, 3),
    ([300, 300], [12, 12], 4096, 3),
    ([300, 300], [14, 14], 9728, 3),
    ([257], [14], 768, 0),
]


@pytest.mark.parametrize("rows,types,K,mode", SHAPES)
def test_whole_share_indices_in_bounds(rows, types, K, mode):
    # Q6_K bases only 4-byte aligned; Q4_K bases 16-byte aligned (the C-ABI's rules)
    bases = [(1 << 24) * (i + 1) + (4 if t == 14 else 0) for i, t in enumerate(types)]
    assert check_shape(rows, types, K, mode, bases)


def test_lm_head_takes_the_streaming_kernel():
    assert launcher([151936], [14], 2560, 0) is None


def test_q6k_gate_up_does_not_fit_the_whole_share_kernel():
    # 2 x 9728 Q6_K rows of width 2560: the FFN (and its norm fold) goes to
    # the norm kernel and the streaming kernel instead
    assert launcher([9728, 9728], [14, 14], 2560, 3) is None


# ---- the batched whole-share kernel (gemv_stream_mt.hpp), M = 2..8 ----

MT_XSTAGED = 4


def launcher_mt(rows, types, K, mode, M):
    """(counts, per/rem, J, region, sums_stride, lds, MT) or None (streaming kernel)."""
    S = K // 256
    MT = 4 if M <= 4 else 8
    if MT * (K // 8) > 64 * WAVES * MT_XSTAGED:
        return None
    nseg = 1 if mode == 1 else len(rows)
    parts = 2 if mode == 1 else 1
    wpp = WAVES // parts
    if any(types[j] != types[0] for j in range(nseg)):
        return None  # one weight type per launch
    byt = [rows[j] * S * BYTES[types[j]] * parts for j in range(nseg)]
    total = float(sum(byt))
    count = [min(max(int(CUS * b / total + 0.5), 1), rows[j]) for j, b in enumerate(byt)]
    while sum(count) > CUS:
        count[count.index(max(count))] -= 1
    region, sums = 16, 0
    for j in range(nseg):
        per, rem = rows[j] // count[j], rows[j] % count[j]
        rb = S * BYTES[types[j]]
        rows_max = per + (1 if rem else 0)
        rpw = -(-rows_max // wpp)
        region = max(region, (2 + rpw * rb + 15) // 16 * 16)
        for n in (per, rows_max):
            if n == 0:
                continue
            groups = -(-n // 16)
            ranges = min(S, max(1, -(-WAVES // (parts * groups))))
            sums = max(sums, n * ranges * MT)
    J = -(-region // 1024)
    if J > MAX_J:
        return None
    lds = MT * S * 8 * 48 + WAVES * region + parts * sums * 4
    if lds > MAX_LDS:
        return None
    return count, J, region, sums, lds, MT


def check_shape_mt(rows, types, K, mode, M, bases):
    cfg = launcher_mt(rows, types, K, mode, M)
    if cfg is None:
        return False
    count, J, region, sums_stride, lds, MT = cfg
    S = K // 256
    parts = 2 if mode == 1 else 1
    wpp = WAVES // parts
    nseg = 1 if mode == 1 else len(rows)
    for j in range(nseg):
        B = BYTES[types[j]]
        rb = S * B
        per, rem = rows[j] // count[j], rows[j] % count[j]
        seen = np.zeros((parts, rows[j]), np.int64)
        for g in range(count[j]):
            r0 = g * per + min(g, rem)
            nrows = per + (1 if g < rem else 0)
            rpw = -(-nrows // wpp)
            images = {}
            for wave in range(WAVES):
                part, wv = wave // wpp, wave % wpp
                first = min(wv * rpw, nrows)
                wrows = min(rpw, nrows - first)
                base = bases[1] if (mode == 1 and part == 1) else bases[j]
                run = base + (r0 + (first if wrows > 0 else 0)) * rb
                o = run & 3
                run4 = run - o
                L = max((o + wrows * rb + 15) >> 4, 1)
                end = base + rows[j] * rb
                last = base + ((rows[j] * rb + 3) & ~3) - 16
                c = np.minimum(np.arange(64)[:, None] + 64 * np.arange(J)[None, :], L - 1)
                a = np.minimum(run4 + 16 * c, last)
                assert np.all(a >= base) and np.all(a + 16 <= ((end + 3) & ~3)) and np.all(a % 4 == 0)
                off = a - run4
                assert np.all(off >= 0) and np.all(off + 16 <= region)
                cov = np.zeros(region, bool)
                for x in np.unique(off):
                    cov[x:x + 16] = True
                images[wave] = (cov, o, first, wrows)
                if wrows > 0:
                    assert cov[o:o + wrows * rb].all()
                    seen[part, r0 + first: r0 + first + wrows] += 1
            # compute units: every (part, row, s) piece read lies in its owner's written bytes
            groups = -(-nrows // 16)
            ranges = min(S, max(1, -(-WAVES // (parts * groups))))
            o_base = (bases[j] + r0 * rb) & 3
            for part in range(parts):
                for row in range(nrows):
                    owner = part * wpp + row // rpw
                    first = (row // rpw) * rpw
                    o_owner = (o_base + first * (rb & 3)) & 3
                    cov, o, f2, wrows = images[owner]
                    assert f2 == first and o == o_owner
                    rowp = o_owner + (row - first) * rb
                    assert cov[rowp:rowp + rb].all()
                    for rr in range(ranges):
                        assert (row * ranges + rr) * MT + MT - 1 < sums_stride
            assert nrows * M <= 64 * WAVES * 64  # row-total threads loop
        assert np.all(seen == 1), "every row of every part exactly once"
    assert lds <= MAX_LDS
    return True


MT_SHAPES = [
    ([9728, 9728], [12, 12], 2560, 1, 8),           # gate + up, M = 8
    ([4096, 1024, 1024], [12, 12, 12], 2560, 0, 8),  # q/k/v all Q4_K, M = 8
    ([2560], [12], 4096, 0, 8),                      # attn_output, M = 8
    ([4096, 1024, 1024], [14, 14, 14], 2560, 0, 3),
    ([5], [14], 2560, 0, 3),
    ([1000], [12], 2560, 0, 2),
    ([4096, 4096], [14, 14], 2560, 1, 2),
    ([101], [14], 1280, 0, 5),
    ([3, 1, 2], [12, 12, 12], 256, 0, 7),
]


@pytest.mark.parametrize("rows,types,K,mode,M", MT_SHAPES)
def test_batched_whole_share_indices_in_bounds(rows, types, K, mode, M):
    bases = [(1 << 24) * (i + 1) + (4 if t == 14 else 0) for i, t in enumerate(types)]
    assert check_shape_mt(rows, types, K, mode, M, bases)


def test_batched_mixed_types_take_the_streaming_kernel():
    assert launcher_mt([4096, 1024, 1024], [12, 12, 14], 2560, 0, 8) is None  # Q4_K q/k, Q6_K v


def test_batched_ffn_down_takes_the_streaming_kernel():
    assert launcher_mt([2560], [14], 9728, 0, 8) is None  # 8 x 9728 activations exceed the staging


def test_batched_q6k_gate_up_too_wide_takes_the_streaming_kernel():
    assert launcher_mt([9728, 9728], [14, 14], 2560, 1, 2) is None  # 5 rows of 2100 B per wave: J > 8


# ---- the fused FFN block (ffn_fused.hip / ffn_fused.hpp), M = 1 ----

H_WAVES = 1           # the last wave: it stores h, its down share is empty
JG_CHOICES = (2, 4, 6, 7, 8)
JD_CHOICES = (2, 4, 6, 8)      # 16-byte chunks per lane of the down share
PD_CHOICES = (1, 2, 3)         # Q6_K down: pieces per lane unpacked ahead of h
Q6_PAIRS = {(2, 1), (4, 1), (4, 2), (6, 2), (8, 2), (8, 3)}  # instantiated (JD, PD)
SYNC_BYTES = 8192


def _round_up(j, choices):
    return next((c for c in choices if j <= c), 0)


def _depth(sb, nbytes):
    return -(-(-(-(2 + sb * nbytes) // 16)) // 64)


def ffn_down_offset(S, JG, max_sb, Sd, JD):
    """ffn_fused.hpp ffn_down_offset: phase B's down region after the Q8 of h, or
    after phase A's sums when it would overlap them."""
    sums_a = S * 8 * 48 + WAVES * JG * 1024
    sums_a_end = sums_a + 2 * max_sb * 4 + 4 * WAVES
    after_h = Sd * 8 * 48
    return after_h if after_h + WAVES * JD * 1024 <= sums_a else sums_a_end


def ffn_launcher(K, N, down_type, gate_up_type=12):
    """(G, per, rem, dper, drem, max_sb, max_sbd, JG, JD, PD, lds) or None (two-launch path)."""
    if gate_up_type != 12 or K > MAX_K or N > MAX_K or K % 256 or N % 256:
        return None
    G = CUS
    if G > N or G > K:
        return None
    S, Sd = K // 256, N // 256
    per, rem, dper, drem = N // G, N % G, K // G, K % G
    max_sb, max_sbd = (per + (1 if rem else 0)) * S, (dper + (1 if drem else 0)) * Sd
    wpp, dwaves = WAVES // 2, WAVES - H_WAVES
    jg = _round_up(_depth(-(-max_sb // wpp), 144), JG_CHOICES)
    down_sb = -(-max_sbd // dwaves)
    jd = _round_up(_depth(down_sb, BYTES[down_type]), JD_CHOICES)
    pd = _round_up(-(-4 * down_sb // 64), PD_CHOICES) if down_type == 14 else 0
    if jg == 0 or jd == 0 or (down_type == 14 and (pd == 0 or (jd, pd) not in Q6_PAIRS)) or jg + jd > 14:
        return None
    lds_a = S * 8 * 48 + WAVES * jg * 1024 + 2 * max_sb * 4 + 4 * WAVES
    lds_b = ffn_down_offset(S, jg, max_sb, Sd, jd) + WAVES * jd * 1024 + max_sbd * 4
    lds = max(lds_a, lds_b)
    if lds > MAX_LDS:
        return None
    return G, per, rem, dper, drem, max_sb, max_sbd, jg, jd, pd, lds


def _share_reads(base, rows, r0, S, B, sb_a, sb_b, J):
    """Global addresses and LDS offsets of one wave's issue_share (per lane, per chunk)."""
    rb = S * B
    run = base + r0 * rb + (sb_a if sb_b > sb_a else 0) * B
    o = run & 3
    run4 = run - o
    cmax = max((o + (sb_b - sb_a) * B + 15) >> 4, 1) - 1
    last = base + ((rows * rb + 3) & ~3) - 16
    lim = last - run4
    c = np.minimum(np.arange(64)[:, None] + 64 * np.arange(J)[None, :], cmax)
    a = np.minimum(run4 + 16 * c, last)
    off = np.minimum(16 * c, lim)
    assert np.array_equal(off, a - run4)  # the lazily recomputed offset is the load's
    end = base + rows * rb
    assert np.all(a >= base) and np.all(a + 16 <= ((end + 3) & ~3)) and np.all(a % 4 == 0)
    assert np.all(off >= 0) and np.all(off + 16 <= J * 1024)
    cov_end = max(16 * cmax, min(16 * cmax, lim) + 16)
    assert cov_end >= o + (sb_b - sb_a) * B
    return o


def check_ffn(K, N, down_type, bases):
    cfg = ffn_launcher(K, N, down_type)
    if cfg is None:
        return False
    G, per, rem, dper, drem, max_sb, max_sbd, JG, JD, PD, lds = cfg
    S, Sd = K // 256, N // 256
    wpp, dwaves = WAVES // 2, WAVES - H_WAVES
    seen = np.zeros((2, N * S), np.int64)
    seen_d = np.zeros(K * Sd, np.int64)
    for g in range(G):
        r0 = g * per + min(g, rem)
        r1 = r0 + per + (1 if g < rem else 0)
        d0 = g * dper + min(g, drem)
        d1 = d0 + dper + (1 if g < drem else 0)
        assert 0 <= r0 < r1 <= N and 0 <= d0 < d1 <= K
        nsb, nsbd = (r1 - r0) * S, (d1 - d0) * Sd
        assert nsb <= max_sb and nsbd <= max_sbd
        for w in range(WAVES):
            part, wv = w // wpp, w % wpp
            sb_a, sb_b = nsb * wv // wpp, nsb * (wv + 1) // wpp
            _share_reads(bases[part], N, r0, S, 144, sb_a, sb_b, JG)
            seen[part, r0 * S + sb_a: r0 * S + sb_b] += 1
            da, db = (nsbd * w // dwaves, nsbd * (w + 1) // dwaves) if w < dwaves else (0, 0)
            o = _share_reads(bases[2], K, d0, Sd, BYTES[down_type], da, db, JD)
            if down_type == 14:
                # pieces read back from the wave's LDS region: lane q = l + 64 i takes piece q % 4
                # of superblock q // 4 of the run (lanes past the share redo its last piece; an
                # empty share reads piece 0); each read spans [base of the dword, superblock end)
                npc = 4 * (db - da)
                assert npc <= 64 * PD, "every piece of the share has a lane"
                q = np.arange(64)[:, None] + 64 * np.arange(PD)[None, :]
                qc = np.minimum(q, npc - 1) if npc > 0 else np.zeros_like(q)
                start = o + (qc >> 2) * 210
                assert np.all((start & ~3) >= 0) and np.all(start + 210 <= JD * 1024)
                stored = (q < npc) & ((q & 3) == 0)
                assert np.all(da + (q[stored] >> 2) < max_sbd)
            seen_d[d0 * Sd + da: d0 * Sd + db] += 1
            # piece reads of Q8 blocks: gate/up over K (x), down over N (h)
            for (a_, b_, SS) in ((sb_a, sb_b, S), (da, db, Sd)):
                q = np.arange(4 * (b_ - a_))
                s = (a_ + (q >> 2)) % SS
                assert np.all(s * 8 + 7 < SS * 8)
        # row totals of phase A by the first H_WAVES waves, a quad per row
        assert (r1 - r0) <= 10_000
    assert np.all(seen == 1) and np.all(seen_d == 1), "every superblock exactly once"
    # h staging: all 16 waves stage tasks l, l + 1024 (lane l of the
    # workgroup); every task of 8 values is staged, and the buffer range of
    # the loads (N floats) makes the tasks past N / 8 read zeros
    nqh = WAVES
    t = np.arange(64 * nqh)[:, None] + 64 * nqh * np.arange(XSTAGED)[None, :]
    assert np.array_equal(np.sort(t[t < N // 8]), np.arange(N // 8))
    # LDS: phase A (Q8 of x, wave regions, both parts' sums, norm partials);
    # phase B (Q8 of h, wave regions, sums) reuse the same bytes
    assert S * 8 * 48 + WAVES * JG * 1024 + 2 * max_sb * 4 + 4 * WAVES <= lds <= MAX_LDS
    dl = ffn_down_offset(S, JG, max_sb, Sd, JD)
    assert dl >= Sd * 8 * 48 and dl + WAVES * JD * 1024 + max_sbd * 4 <= lds
    # the down regions, written while the h wave still reads phase A's sums
    # (and norm partials), do not overlap them
    sums_a, sums_a_end = S * 8 * 48 + WAVES * JG * 1024, S * 8 * 48 + WAVES * JG * 1024 + 2 * max_sb * 4 + 4 * WAVES
    assert dl + WAVES * JD * 1024 <= sums_a or dl >= sums_a_end
    # barrier words: 3 + 2 x 8 lines of 256 bytes
    assert (3 + 2 * 8) * 256 <= SYNC_BYTES
    return True


FFN_SHAPES = [
    (2560, 9728, 14),   # Qwen3-4B: gate/up Q4_K, down Q6_K
    (2560, 9728, 12),   # Q4_K down (layers of Q4_K_M files that keep it at 4 bits)
    (2048, 6144, 14),   # Qwen3-1.7B
    (1024, 3072, 14),   # Qwen3-0.6B
    (4096, 4096, 12),
    (2816, 2560, 14),   # ragged rows per workgroup
]


@pytest.mark.parametrize("K,N,down_type", FFN_SHAPES)
def test_fused_ffn_indices_in_bounds(K, N, down_type):
    bases = [1 << 24, 2 << 24, (3 << 24) + (4 if down_type == 14 else 0)]
    assert check_ffn(K, N, down_type, bases)


def test_fused_ffn_plan_for_qwen3_4b():
    G, per, rem, dper, drem, max_sb, max_sbd, JG, JD, PD, lds = ffn_launcher(2560, 9728, 14)
    assert (per, rem, dper, drem, JG, JD, PD) == (38, 0, 10, 0, 7, 6, 2)
    assert lds > MAX_LDS // 2  # one workgroup per CU


def test_fused_ffn_declines_shapes_that_do_not_fit():
    assert ffn_launcher(4096, 12288, 14) is None   # gate/up share too deep (Qwen3-8B)
    assert ffn_launcher(2560, 9728, 14, gate_up_type=14) is None
    assert ffn_launcher(2560, 20480, 14) is None   # h wider than the quantiser staging
