"""CPU model of the batched mat-vec on the int8 matrix cores
(qwen3-4b-q4_k_m-inference-engine_amd/csrc/bmv.hip, bmv.hpp), M = 2..8.

For each shape the model restates the launcher's plan (workgroups per
segment, superblock runs per row group, LDS size) and the kernel's cursors,
then checks every global load of every lane of every wave of every workgroup
(inside its superblock and its matrix, including the ring's refills past a
wave's last tile), every LDS read and write against its region, and that each
(part, row, superblock) is computed by exactly one tile and each unit's sums
slot written once. A lane-level emulation of the arithmetic (the block-
diagonal A tiles as the lanes read them from the LDS image, the B operands as
the lanes build them, v_mfma_i32_16x16x64_i8 as an integer product with the
probed lane layout: lane l holds A[l%16][16(l/16)+t], B[16(l/16)+t][l%16] and
receives C[4(l/16)+i][l%16]) is compared with the oracle's product, with
garbage planted in the LDS rows the kernel leaves unwritten. The model is its
own code restating the kernel's integer arithmetic; a change to either file
must be mirrored here."""
import numpy as np
import pytest

CUS, MAX_LDS, WAVES = 256, 160 * 1024, 8
BYTES = {12: 144, 14: 210}
P = {12: 6, 14: 4}
P_MIXED6 = 3


def lds_bytes(K, stride, parts, groups, ranges):
    return 8 * stride + 16 + 4 * K + parts * groups * 16 * ranges * 32


def wave_tiles(rows, parts, S, ranges):
    if rows <= 0:
        return 0
    groups = -(-rows // 16)
    units = parts * groups * ranges
    return -(-units // WAVES) * -(-S // ranges)


def plan(rows, types, K, mode, M):
    """(workgroups per segment, ranges, groups_max, lds) or None when the launcher declines."""
    if not 2 <= M <= 8 or mode not in (0, 1):
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
    stride = K + 16
    groups_max = max(-(-(-(-rows[j] // count[j])) // 16) for j in range(nseg))
    ranges, best = 0, None
    for r in range(1, S + 1):
        if lds_bytes(K, stride, parts, groups_max, r) > MAX_LDS:
            break
        tiles = units = 0
        for j in range(nseg):
            per = rows[j] // count[j]
            for n in (per, per + 1):
                tiles = max(tiles, wave_tiles(n, parts, S, r))
                units = max(units, -(-(parts * -(-n // 16) * r) // WAVES))
        cost = 8 * tiles + units
        if best is None or cost < best:
            best, ranges = cost, r
    if ranges == 0:
        return None
    return count, ranges, groups_max, lds_bytes(K, stride, parts, groups_max, ranges)


class Share:
    def __init__(self, r0, nrows, S, ranges, parts):
        self.r0, self.nrows, self.S, self.ranges, self.parts = r0, nrows, S, ranges, parts
        self.groups = (nrows + 15) >> 4
        self.run_q, self.run_r = S // ranges, S % ranges

    def run_begin(self, rr):
        return rr * self.run_q + min(rr, self.run_r)


class Cursor:
    def __init__(self, sh, u, left):
        self.sh = sh
        self.rr = u % sh.ranges
        pg = u // sh.ranges
        self.part = pg // sh.groups
        self.g = pg - self.part * sh.groups
        self.s, self.s_end = sh.run_begin(self.rr), sh.run_begin(self.rr + 1)
        self.left = left

    def copy(self):
        c = Cursor.__new__(Cursor)
        c.__dict__.update(self.__dict__)
        return c

    def next(self):
        sh = self.sh
        if self.left > 1:
            self.left -= 1
            self.s += 1
            if self.s == self.s_end:
                self.rr += 1
                if self.rr == sh.ranges:
                    self.rr = 0
                    self.g += 1
                    if self.g == sh.groups:
                        self.g = 0
                        self.part += 1
                self.s, self.s_end = sh.run_begin(self.rr), sh.run_begin(self.rr + 1)


def wave_streams(sh, wave, depth):
    """(compute tiles, load tiles) of a wave: tiles as (part, g, rr, s, last_of_unit)."""
    units = sh.parts * sh.groups * sh.ranges
    u_lo, u_hi = units * wave // WAVES, units * (wave + 1) // WAVES
    ntiles = sum(sh.run_begin(u % sh.ranges + 1) - sh.run_begin(u % sh.ranges) for u in range(u_lo, u_hi))
    start = Cursor(sh, u_lo if u_lo < u_hi else 0, ntiles)
    lc, cc = start.copy(), start.copy()
    loads, comps = [], []
    for _ in range(depth):
        loads.append((lc.part, lc.g, lc.rr, lc.s))
        lc.next()
    for base in range(0, ntiles, depth):
        for j in range(depth):
            if base + j < ntiles:
                comps.append((cc.part, cc.g, cc.rr, cc.s, cc.s + 1 == cc.s_end))
                cc.next()
            loads.append((lc.part, lc.g, lc.rr, lc.s))
            lc.next()
    return comps, loads


LANE = np.arange(64)
LN, LKQ = LANE & 15, LANE >> 4


def load_ranges(qtype, sb):
    """Byte ranges [a, b) each lane reads of its superblock at offset sb (array per lane)."""
    kq = LKQ
    if qtype == 12:
        return [(sb, sb + 16), (sb + 16 + 16 * kq, sb + 32 + 16 * kq), (sb + 80 + 16 * kq, sb + 96 + 16 * kq)]
    return [(sb + 16 * kq, sb + 16 + 16 * kq), (sb + 64 + 16 * kq, sb + 80 + 16 * kq),
            (sb + 128 + 16 * (kq & 1), sb + 144 + 16 * (kq & 1)),
            (sb + 160 + 16 * (kq & 1), sb + 176 + 16 * (kq & 1)), (sb + 192, sb + 208), (sb + 208, sb + 210)]


def workgroups(rows, types, K, mode, cfg):
    count, ranges, groups_max, lds = cfg
    nseg = 1 if mode == 1 else len(rows)
    parts = 2 if mode == 1 else 1
    for j in range(nseg):
        per, rem = rows[j] // count[j], rows[j] % count[j]
        for g in range(count[j]):
            yield j, Share(g * per + min(g, rem), per + (1 if g < rem else 0), K // 256, ranges, parts)


def check_indices(rows, types, K, mode, M, bases):
    """Workgroups of one segment with the same row count differ only by their
    first row, so beyond 32 workgroups the first of each row count and the
    last are checked lane by lane; the shares' partition of the rows is
    checked for all of them."""
    cfg = plan(rows, types, K, mode, M)
    assert cfg is not None
    count, ranges, groups_max, lds = cfg
    assert lds <= MAX_LDS
    S, stride = K // 256, K + 16
    Z = 8 * stride + 16
    mixed = mode == 0 and len(set(types)) > 1
    parts = 2 if mode == 1 else 1
    nseg = 1 if mode == 1 else len(rows)
    chosen = set()
    for j in range(nseg):
        per, rem = rows[j] // count[j], rows[j] % count[j]
        shares = [(g * per + min(g, rem), per + (1 if g < rem else 0)) for g in range(count[j])]
        assert shares[0][0] == 0 and shares[-1][0] + shares[-1][1] == rows[j]
        assert all(a + n == b for (a, n), (b, _) in zip(shares, shares[1:])), "shares partition the rows"
        if count[j] <= 32:
            chosen |= {(j, r0) for r0, _ in shares}
        else:
            chosen |= {(j, shares[0][0]), (j, shares[rem - 1][0] if rem else 0), (j, shares[rem][0] if rem < count[j] else 0),
                       (j, shares[-1][0])}
    seen = {}
    for j, sh in workgroups(rows, types, K, mode, cfg):
        if (j, sh.r0) not in chosen:
            continue
        qtype = types[j]
        B = BYTES[qtype]
        depth = P_MIXED6 if (mixed and qtype == 14) else P[qtype]
        rb = S * B
        slots = {}
        for wave in range(WAVES):
            comps, loads = wave_streams(sh, wave, depth)
            for part, g, rr, s in loads:
                w = bases[1] if (mode == 1 and part) else bases[j]
                n_mat = rows[1] if (mode == 1 and part) else rows[j]
                row = np.minimum(16 * g + LN, sh.nrows - 1)
                sb = w + (sh.r0 + row) * rb + s * B
                for a, b in load_ranges(qtype, sb):
                    assert np.all(a >= sb) and np.all(b <= sb + B), "read outside the superblock"
                    assert np.all(a >= w) and np.all(b <= w + n_mat * rb), "read outside the matrix"
                    if qtype == 12 and (b - a)[0] == 16:
                        assert np.all(a % 16 == 0), "Q4_K loads are 16-byte aligned"
            for part, g, rr, s, last in comps:
                for rw in range(16 * g, min(16 * g + 16, sh.nrows)):
                    key = (j, part, sh.r0 + rw, s)
                    assert key not in seen, "tile computed twice"
                    seen[key] = True
                # LDS reads of the tile
                khi, klo = LKQ >> 1, LKQ & 1
                if qtype == 12:
                    valid = (LN < 8) == (LKQ < 2)
                    base = (LN & 7) * stride + 16 * klo
                    for h in range(2):
                        for nib in range(2):
                            jj = 4 * h + nib + 2 * khi
                            aoff = np.where(valid, base + 256 * s + 32 * jj, 8 * stride)
                            assert np.all(aoff + 16 <= 8 * stride + 16) and np.all(aoff % 16 == 0)
                            assert np.all(np.where(valid, aoff + 16 <= 8 * stride, True))
                            for reg in (0, K):  # xs, xss
                                off = Z + reg + 4 * ((8 * s + jj) * 8 + 4 * klo)
                                assert np.all(off >= Z + reg) and np.all(off + 16 <= Z + reg + K)
                else:
                    valid = (LN >> 2) == LKQ
                    base = (LN & 3) * stride + 16 * LKQ
                    for h in range(2):
                        for nib in range(2):
                            for mh in range(2 if M > 4 else 1):
                                aoff = np.where(valid, base + 4 * mh * stride + 256 * s + 128 * h + 64 * nib, 8 * stride)
                                assert np.all(aoff % 16 == 0) and np.all(aoff + 16 <= 8 * stride + 16)
                                blk = 4 * h + 2 * nib + khi
                                sb16 = 8 * h + 4 * nib + LKQ
                                off = Z + 4 * ((8 * s + blk) * 8 + 4 * mh)
                                assert np.all(off + 16 <= Z + K)
                                off = Z + 2 * K + 4 * ((16 * s + sb16) * 8 + 4 * mh)
                                assert np.all(off >= Z + 2 * K) and np.all(off + 16 <= Z + 4 * K)
                if last:
                    assert (part, g, rr) not in slots, "unit flushed twice"
                    slots[(part, g, rr)] = True
                    slot = ((part * groups_max + g) * 16 + LN) * ranges + rr
                    off = Z + 4 * K + 4 * (slot * 8)
                    assert np.all(off + 32 <= lds)
        assert len(slots) == parts * sh.groups * ranges, "every unit flushed"
        # totals read every run of every valid row
        for part in range(parts):
            for rw in range(sh.nrows):
                for rr in range(ranges):
                    off = Z + 4 * K + 4 * ((((part * groups_max) * 16 + rw) * ranges + rr) * 8 + 7)
                    assert off + 4 <= lds
    for j, sh in workgroups(rows, types, K, mode, cfg):
        if (j, sh.r0) in chosen:
            for part in range(parts):
                for rw in range(sh.r0, sh.r0 + sh.nrows):
                    for s in range(S):
                        assert (j, part, rw, s) in seen, "tile never computed"
    return cfg


SHAPES = [  # rows, types, K, mode, M
    ([4096, 1024, 1024], [12, 12, 14], 2560, 0, 8),   # attn q/k/v
    ([4096, 1024, 1024], [12, 12, 14], 2560, 0, 3),
    ([2560], [12], 4096, 0, 8),                         # attn_output
    ([9728, 9728], [12, 12], 2560, 1, 8),               # ffn gate/up
    ([9728, 9728], [12, 12], 2560, 1, 5),
    ([2560], [14], 9728, 0, 8),                         # ffn_down
    ([2560], [14], 9728, 0, 4),
    ([151936], [14], 2560, 0, 8),                       # lm_head
    ([1024], [14], 2560, 0, 2),
    ([9728, 9728], [14, 14], 2560, 1, 6),
    ([19], [12], 2560, 0, 5),
    ([19], [14], 9728, 0, 7),
    ([45], [14], 768, 0, 3),
    ([101], [14], 1280, 0, 5),
    ([3, 1, 2], [12, 12, 14], 256, 0, 7),
    ([300, 17], [14, 12], 512, 0, 8),
]


@pytest.mark.parametrize("rows,types,K,mode,M", SHAPES)
def test_bmv_indices_in_bounds(rows, types, K, mode, M):
    bases = [(1 << 30) * (i + 1) + (4 if t == 14 else 0) for i, t in enumerate(types)]
    check_indices(rows, types, K, mode, M, bases)


def test_bmv_plan_for_qwen3_shapes():
    """LDS plans of the decode batch's launches (one workgroup per CU)."""
    assert plan([2560], [14], 9728, 0, 8)[3] <= MAX_LDS           # ffn_down: 8 x 9728 codes + scales
    assert plan([151936], [14], 2560, 0, 8)[2] == 38              # lm_head: 593-594 rows per CU
    assert plan([9728, 9728], [12, 12], 2560, 1, 8)[0] == [256]
    assert plan([2560], [12], 4096, 0, 1) is None                 # M = 1: the whole-share kernels
    assert plan([2560], [12], 4096, 0, 9) is None                 # M > 8: the prefill GEMM


# ---------------------------------------------------------------- arithmetic

def _u32(b):
    return np.frombuffer(np.ascontiguousarray(b, dtype=np.uint8).tobytes(), dtype=np.uint32)


def _f16(bits):
    return float(np.array([bits], dtype=np.uint16).view(np.float16)[0])


def emulate(oracle, rows, types, K, mode, M, weights, x, rng):
    """The kernel's arithmetic at lane level; returns y per segment (mode 0) or h (mode 1)."""
    cfg = plan(rows, types, K, mode, M)
    count, ranges, groups_max, lds = cfg
    S, stride = K // 256, K + 16
    parts = 2 if mode == 1 else 1
    codes_q, scales_q = oracle.quantize_q8(x)
    codes_q = codes_q.reshape(M, K)
    scales_q = scales_q.reshape(M, K // 32)
    # LDS image: written rows from the oracle's Q8, garbage elsewhere
    codes = rng.integers(-128, 128, size=(8, stride), dtype=np.int64)
    codes[:M, :K] = codes_q
    zero = np.zeros(16, dtype=np.int64)
    xs = rng.standard_normal((K // 32, 8)) * 1e3
    xss = rng.standard_normal((K // 32, 8)) * 1e3
    xf = rng.integers(-(1 << 20), 1 << 20, size=(K // 16, 8), dtype=np.int64)
    c32 = codes_q.reshape(M, K // 32, 32).astype(np.int64)
    xs[:, :M] = scales_q.T
    xss[:, :M] = (scales_q * c32.sum(axis=2)).T
    xf[0::2, :M] = (-32 * c32[:, :, :16].sum(axis=2)).T  # int32: the Q6_K MFMA's accumulator input
    xf[1::2, :M] = (-32 * c32[:, :, 16:].sum(axis=2)).T

    def a_tile(offs):  # A[r][16kq+t] from lane (r, kq) = (l%16, l/16) reading 16 bytes at offs[l]
        A = np.zeros((16, 64), dtype=np.int64)
        for l in range(64):
            o = offs[l]
            if o == 8 * stride:
                vals = zero
            else:
                m, k = divmod(int(o), stride)
                vals = codes[m, k:k + 16]
            A[l % 16, 16 * (l // 16):16 * (l // 16) + 16] = vals
        return A

    def b_tile(byte_rows):  # B[16kq+t][n] from lane (n, kq) holding 16 bytes byte_rows[l]
        Bm = np.zeros((64, 16), dtype=np.int64)
        for l in range(64):
            Bm[16 * (l // 16):16 * (l // 16) + 16, l % 16] = byte_rows[l]
        return Bm

    def lane_c(C):  # lane l's four results C[4(l/16)+i][l%16]
        return np.stack([C[4 * (LANE // 16) + i, LANE % 16] for i in range(4)], axis=1)

    nseg = 1 if mode == 1 else len(rows)
    out = [np.full((M, rows[j]), np.nan) for j in range(nseg)]
    for j, sh in workgroups(rows, types, K, mode, cfg):
        qtype = types[j]
        B = BYTES[qtype]
        sums = np.full((parts, groups_max, 16, ranges, 8), np.nan)
        for wave in range(WAVES):
            comps, _ = wave_streams(sh, wave, P[qtype])
            acc = np.zeros((64, 8))
            for part, g, rr, s, last in comps:
                w = weights[1] if (mode == 1 and part) else weights[j]
                row = np.minimum(16 * g + LN, sh.nrows - 1) + sh.r0
                sbs = w.reshape(-1, S, B)[row, s]  # [64 lanes][B bytes]
                kq, khi, klo = LKQ, LKQ >> 1, LKQ & 1
                if qtype == 12:
                    head = np.stack([_u32(sbs[l, :16]) for l in range(64)])
                    qa = np.stack([sbs[l, 16 + 16 * kq[l]:32 + 16 * kq[l]] for l in range(64)]).astype(np.int64)
                    qb = np.stack([sbs[l, 80 + 16 * kq[l]:96 + 16 * kq[l]] for l in range(64)]).astype(np.int64)
                    valid = (LN < 8) == (kq < 2)
                    base = (LN & 7) * stride + 16 * klo
                    mainv, minv = np.zeros((64, 4)), np.zeros((64, 4))
                    for h in range(2):
                        for nib in range(2):
                            jj = 4 * h + nib + 2 * khi
                            A = a_tile(np.where(valid, base + 256 * s + 32 * jj, 8 * stride))
                            q = qb if h else qa
                            Bm = b_tile((q >> 4) & 15 if nib else q & 15)
                            C = lane_c(A @ Bm)
                            o = 8 * (nib + 2 * khi)
                            s0, s1, s2 = head[:, 1], head[:, 2], head[:, 3]
                            if h == 0:
                                sc, mn = (s0 >> o) & 63, (s1 >> o) & 63
                            else:
                                sc = ((s2 >> o) & 15) | (((s0 >> (o + 6)) & 3) << 4)
                                mn = ((s2 >> (o + 4)) & 15) | (((s1 >> (o + 6)) & 3) << 4)
                            x4 = np.stack([xs[8 * s + jj[l], 4 * klo[l]:4 * klo[l] + 4] for l in range(64)])
                            y4 = np.stack([xss[8 * s + jj[l], 4 * klo[l]:4 * klo[l] + 4] for l in range(64)])
                            mainv += C * x4 * sc[:, None]
                            minv += mn[:, None] * y4
                    d = np.array([_f16(v & 0xFFFF) for v in head[:, 0]])
                    dmin = np.array([_f16(v >> 16) for v in head[:, 0]])
                    acc[:, :4] += d[:, None] * mainv - dmin[:, None] * minv
                else:
                    ql = [np.stack([sbs[l, 64 * h + 16 * kq[l]:64 * h + 16 * kq[l] + 16] for l in range(64)]).astype(np.int64) for h in range(2)]
                    qh = [np.stack([sbs[l, 128 + 32 * h + 16 * klo[l]:128 + 32 * h + 16 * klo[l] + 16] for l in range(64)]).astype(np.int64) for h in range(2)]
                    scb = np.stack([sbs[l, 192:208] for l in range(64)]).view(np.int8).astype(np.int64)
                    d = np.array([_f16(int(sbs[l, 208]) | int(sbs[l, 209]) << 8) for l in range(64)])
                    valid = (LN >> 2) == kq
                    base = (LN & 3) * stride + 16 * kq
                    accsb = np.zeros((64, 8))
                    for h in range(2):
                        for nib in range(2):
                            # the kernel's dword ops: lo nibbles, qh rotated right by
                            # sh = 28 + 2*khi (nib 0) or 2*khi (nib 1), bits 4-5 inserted
                            sh_r = (28 + 2 * khi) if nib == 0 else 2 * khi
                            codes16 = np.zeros((64, 16), dtype=np.int64)
                            for l in range(64):
                                lw = _u32(ql[h][l].astype(np.uint8)).astype(np.uint64)
                                hw = _u32(qh[h][l].astype(np.uint8)).astype(np.uint64)
                                lo = ((lw >> 4) if nib else lw) & 0x0F0F0F0F
                                r = int(sh_r[l])
                                hs = ((hw >> r) | (hw << (32 - r))) & 0xFFFFFFFF if r else hw
                                word = (hs & 0x30303030) | (lo & ~np.uint64(0x30303030) & 0xFFFFFFFF)
                                codes16[l] = np.frombuffer(word.astype(np.uint32).tobytes(), dtype=np.uint8)
                            Bm = b_tile(codes16)
                            sb16 = 8 * h + 4 * nib + kq
                            scf = scb[LANE, 4 * (2 * h + nib) + kq]
                            blk = 4 * h + 2 * nib + khi
                            for mh in range(2 if M > 4 else 1):
                                A = a_tile(np.where(valid, base + 4 * mh * stride + 256 * s + 128 * h + 64 * nib, 8 * stride))
                                n4 = np.stack([xf[16 * s + sb16[l], 4 * mh:4 * mh + 4] for l in range(64)])
                                C = lane_c(A @ Bm) + n4  # D = A B + C, exact in int32
                                x4 = np.stack([xs[8 * s + blk[l], 4 * mh:4 * mh + 4] for l in range(64)])
                                accsb[:, 4 * mh:4 * mh + 4] += scf[:, None] * (x4 * C)
                    acc += d[:, None] * accsb
                if last:
                    if qtype == 12:
                        v = acc[:, :4] + acc[LANE ^ 32, :4]
                        for l in range(32):
                            sums[part, g, l & 15, rr, 4 * (l >> 4):4 * (l >> 4) + 4] = v[l]
                    else:
                        v = acc + acc[LANE ^ 32]
                        v = v + v[LANE ^ 16]
                        for l in range(16):
                            sums[part, g, l, rr, :] = v[l]
                    acc[:] = 0.0
        for m in range(M):
            for rw in range(sh.nrows):
                a = sums[0, rw >> 4, rw & 15, :, m].sum()
                if mode == 0:
                    out[j][m, sh.r0 + rw] = a
                else:
                    b = sums[1, rw >> 4, rw & 15, :, m].sum()
                    out[j][m, sh.r0 + rw] = a / (1.0 + np.exp(-a)) * b
    return out


EMULATED = [  # rows, types, K, mode, M
    ([40], [12], 512, 0, 8),
    ([37], [14], 768, 0, 8),
    ([23], [14], 512, 0, 3),
    ([20, 9, 13], [12, 12, 14], 256, 0, 5),
    ([33, 33], [12, 12], 512, 1, 2),
]


@pytest.mark.parametrize("rows,types,K,mode,M", EMULATED)
def test_bmv_arithmetic_matches_oracle(oracle, rows, types, K, mode, M):
    rng = np.random.default_rng(5)
    x = oracle.synth_normal(M * K, 20261300 + K + M)
    nmat = len(rows)
    weights = [oracle.synth_superblocks(types[i], rows[i], K, 20261400 + i, 0.01 if types[i] == 12 else 0.005, 0.01)
               for i in range(nmat)]
    got = emulate(oracle, rows, types, K, mode, M, weights, x, rng)
    if mode == 0:
        for j in range(nmat):
            ref = oracle.reference_product(x, weights[j], types[j], K, rows[j])
            assert oracle.row_norm_error(got[j], ref) <= 1e-6
    else:
        g = oracle.reference_product(x, weights[0], types[0], K, rows[0])
        u = oracle.reference_product(x, weights[1], types[1], K, rows[1])
        ref = g / (1.0 + np.exp(-g)) * u
        assert oracle.row_norm_error(got[0], ref) <= 1e-6



def _owner(r, per, rem):
    big = rem * (per + 1)
    return r // (per + 1) if r < big else rem + (r - big) // per


@pytest.mark.parametrize("N,M,count", [(9728, 8, 256), (9728, 2, 256), (512, 5, 7), (2048, 8, 100),
                                       (96, 3, 50), (6144, 8, 256), (256, 8, 256)])
def test_bmv_q8h_blocks_close_once(N, M, count):
    """Q8(h) in the gate/up launch (bmv_close_blocks): whatever order the
    workgroups arrive in, each 32-value block of h is completed by exactly one
    workgroup, after every workgroup owning one of its rows arrived, every
    counter is back at zero for the next launch, and the closing quads fit the
    workgroup (the launcher's bound on blocks per share holds)."""
    count = min(count, N)
    per, rem = divmod(N, count)
    rows_max = per + (1 if rem else 0)
    bound = (rows_max + 30) // 32 + 1
    if not (N % 32 == 0 and bound <= 16 and 4 * bound * M <= 64 * WAVES):
        return  # the launcher declines; the separate quantise launch runs
    rng = np.random.default_rng(N + M + count)
    for trial in range(3):
        arrive = np.zeros(N // 32, dtype=np.int64)
        closed = np.zeros(N // 32, dtype=np.int64)
        arrived = np.zeros(N // 32, dtype=np.int64)
        for g in rng.permutation(count):
            r0, nrows = g * per + min(g, rem), per + (1 if g < rem else 0)
            b0 = r0 >> 5
            nb = ((r0 + nrows - 1) >> 5) - b0 + 1
            assert nb <= bound
            for i in range(nb):
                b = b0 + i
                first, last = _owner(32 * b, per, rem), _owner(min(32 * b + 31, N - 1), per, rem)
                assert first <= g <= last
                arrive[b] += 1
                arrived[b] += 1
                if arrive[b] == last - first + 1:
                    arrive[b] = 0
                    closed[b] += 1
                    assert arrived[b] == last - first + 1  # every owner's h is stored
                    quads = [(i * M + m) for m in range(M)]
                    assert max(quads) * 4 + 3 < 64 * WAVES
        assert np.all(closed == 1) and np.all(arrive == 0)
    # the owner function restates the cut
    for r in range(0, N, max(1, N // 97)):
        g = _owner(r, per, rem)
        assert g * per + min(g, rem) <= r < g * per + min(g, rem) + per + (1 if g < rem else 0)
