"""CPU model of the Q4_K / Q6_K prefill GEMM (qwen3-4b-q4_k_m-inference-engine_amd/
csrc/gemm_kquant.hip) and of the prep kernel's sub-block sums (csrc/gemm.hip):
every load address (activation pieces, weight qs bytes and headers, sub-block
sums, rows clamped into the matrices), the LDS slot image the workgroup
writes, every lane's fragment reads from it, the k order shared by the A and
B operands of each 16-deep step, the MFMA lane rule and the per-superblock
folds are restated in numpy (float64 arithmetic); every access is checked
against its buffer or slot and the product is compared with the oracle. A
change to either file must be mirrored here."""
import numpy as np
import pytest

WAVES, STAGE_K = 4, 64
BYTES = {12: 144, 14: 210}


class Cfg:
    def __init__(self, TM, TN):
        self.TM, self.TN = TM, TN
        self.BM = 32 * TM
        self.BN = 32 * TN * WAVES
        self.SLOT = self.BM * 2 * 2 * STAGE_K
        self.PIECES = self.SLOT // 16 // (64 * WAVES)
        assert self.PIECES >= 1 and self.SLOT % (16 * 64 * WAVES) == 0


def headroom_exponent(bound):
    if not bound > 0:
        return 0
    return min(14 - (np.frexp(np.float32(bound))[1] - 1), 100)


def prep(oracle, x, M, K):
    """hi, lo planes (float16 [M, K]), row scales, sub-block sums [M][S][hi 8, lo 8]."""
    S = K // 256
    x = x.reshape(M, K)
    x8 = oracle.q8_roundtrip(x.reshape(-1)).reshape(M, K).astype(np.float32)
    hi = np.empty((M, K), np.float16)
    lo = np.empty((M, K), np.float16)
    scale = np.empty(M, np.float32)
    xs = np.zeros(M * S * 16, np.float16)
    for m in range(M):
        s = headroom_exponent(float(np.max(np.abs(x[m]))))
        v = (x8[m] * np.float32(2.0 ** s)).astype(np.float32)
        hi[m] = v.astype(np.float16)
        lo[m] = (v - hi[m].astype(np.float32)).astype(np.float16)
        scale[m] = np.float32(2.0 ** -s)
        blocks = v.reshape(K // 32, 4, 8)
        lane = np.zeros((K // 32, 4), np.float32)
        for e in range(8):  # each lane adds its 8 values in order
            lane = (lane + blocks[:, :, e]).astype(np.float32)
        pair = (lane + lane[:, [1, 0, 3, 2]]).astype(np.float32)  # DPP quad_perm 1,0,3,2
        tot = (pair + pair[:, [2, 3, 0, 1]]).astype(np.float32)[:, 0]  # then 2,3,0,1
        t = (tot * np.float32(0.03125)).astype(np.float32)
        th = t.astype(np.float16)
        tl = (t - th.astype(np.float32)).astype(np.float16)
        for jb in range(K // 32):
            at = (m * S + (jb >> 3)) * 16 + (jb & 7)
            xs[at], xs[at + 8] = th[jb], tl[jb]
    return hi, lo, scale, xs


def scale_min_k4(j, sc12):
    if j < 4:
        return sc12[j] & 63, sc12[j + 4] & 63
    return (sc12[j + 4] & 15) | ((sc12[j - 4] >> 6) << 4), (sc12[j + 4] >> 4) | ((sc12[j] >> 6) << 4)


def stage_k(q6, c):
    """First half of stage c in a row: Q4_K 64c; Q6_K 256 sb + 128 (half) + 32 a."""
    return 256 * (c >> 2) + 128 * ((c >> 1) & 1) + 32 * (c & 1) if q6 else STAGE_K * c


def run_model(cfg, oracle, qtype, M, N, K, seed, splits=1):
    S, nst = K // 256, K // STAGE_K
    q6 = qtype == 14
    SB = BYTES[qtype]
    x = oracle.synth_normal(M * K, seed)
    if q6:  # scales over the whole int8 range, so sc*q reaches past 2048
        w = oracle.synth_superblocks(14, N, K, seed + 1, 0.005)
        sbv = w.reshape(N * S, SB)
        sbv[:, 192:208] = np.random.default_rng(seed).integers(0, 256, (N * S, 16), dtype=np.uint8)
    else:
        w = oracle.synth_superblocks(12, N, K, seed + 1, 0.01, 0.01)
    hi, lo, scale, xs = prep(oracle, x, M, K)
    planes = np.concatenate([hi.reshape(-1), lo.reshape(-1)])  # halves, lo at M*K
    n_tiles = -(-N // cfg.BN)
    tiles = n_tiles * -(-M // cfg.BM)
    y = np.full((M, N), np.nan)
    seen = np.zeros((M, N), np.int64)
    lane = np.arange(64)
    h, l32 = lane >> 5, lane & 31
    swz = l32 & 15
    tid = np.arange(64 * WAVES)
    partial = np.zeros((splits, M, N))
    for u in range(tiles * splits):
        t, split = u // splits, u % splits
        sb0, sb1 = split * S // splits, (split + 1) * S // splits
        mt, nt = t // n_tiles, t % n_tiles
        m0, n0 = mt * cfg.BM, nt * cfg.BN
        # activation piece addresses (halves) of every thread
        pa = []
        for v in range(cfg.PIECES):
            f = tid + 64 * WAVES * v
            row, piece = f >> 4, (f & 15) ^ ((f >> 4) & 15)
            p8 = piece & 7
            koff = 64 * (p8 >> 2) + 8 * (p8 & 3) if q6 else 8 * p8
            pa.append(np.where(piece >> 3 == 1, M * K, 0) + np.minimum(m0 + row, M - 1) * K + koff)
        acc = np.zeros((WAVES, cfg.TM, cfg.TN, 32, 32))
        ph = np.zeros_like(acc)
        for sb in range(sb0, sb1):
            min_b = np.zeros((WAVES, cfg.TN, 64, 8))
            for g in range(4):
                c = 4 * sb + g
                slot = np.zeros(cfg.SLOT, np.uint8)
                for v in range(cfg.PIECES):
                    a = pa[v] + stage_k(q6, c)
                    assert np.all(a >= 0) and np.all(a + 8 <= planes.size)
                    f = tid + 64 * WAVES * v
                    assert np.all(16 * f + 16 <= cfg.SLOT)
                    for th_ in range(tid.size):
                        slot[16 * f[th_]:16 * f[th_] + 16] = planes[a[th_]:a[th_] + 8].view(np.uint8)
                for wv in range(WAVES):
                    n_rows = np.minimum(n0 + wv * 32 * cfg.TN + 32 * np.arange(cfg.TN)[:, None] + l32, N - 1)
                    for j in range(cfg.TN):
                        base = n_rows[j] * S * SB + sb * SB
                        assert np.all(base + SB <= w.size)
                        bw = np.zeros((4, 64, 8))
                        if q6:
                            hf, a_ = g >> 1, g & 1
                            qlo = base + 64 * hf + 32 * a_ + 16 * h
                            qho = base + 128 + 32 * hf + 16 * h
                            assert np.all(qlo + 16 <= base + 128) and np.all(qho + 16 <= base + 192)
                        else:
                            qoff = base + 16 + 32 * g + 16 * h
                            assert np.all(qoff + 16 <= base + SB)
                        for L in range(64):
                            if q6:
                                ql = w[qlo[L]:qlo[L] + 16].astype(np.int64)
                                qh = w[qho[L]:qho[L] + 16].astype(np.int64)
                                scl = w[base[L] + 192:base[L] + 208].view(np.int8).astype(np.int64)
                                for step in range(4):
                                    U, s = step >> 1, step & 1
                                    lo4 = (ql[8 * s:8 * s + 8] >> (4 * U)) & 15
                                    hi2 = (qh[8 * s:8 * s + 8] >> (2 * a_ + 4 * U)) & 3
                                    q = (lo4 | (hi2 << 4)) - 32
                                    sc = scl[8 * hf + 2 * (a_ + 2 * U) + h[L]]
                                    v = sc * q
                                    bh = v.astype(np.float16).astype(np.float64)
                                    assert np.all(np.abs(v - bh) <= 1)  # the exact remainder plane
                                    bw[step, L] = v
                                continue
                            head = w[base[L]:base[L] + 16].astype(np.int64)
                            qs = w[qoff[L]:qoff[L] + 16].astype(np.int64)
                            sc0, mn0 = scale_min_k4(2 * g, head[4:16])
                            sc1, mn1 = scale_min_k4(2 * g + 1, head[4:16])
                            min_b[wv, j, L, 2 * g:2 * g + 2] = (mn0, mn1)
                            for step in range(4):
                                U, s = step >> 1, step & 1
                                byt = qs[8 * s:8 * s + 8]
                                bw[step, L] = (sc1 * (byt >> 4)) if U else (sc0 * (byt & 15))
                        for step in range(4):
                            p = 4 * (step >> 1) + 2 * h + (step & 1)
                            for i in range(cfg.TM):
                                row_off = (32 * i + l32) * 256
                                oh, ol = row_off + 16 * (p ^ swz), row_off + 16 * ((8 + p) ^ swz)
                                assert np.all(ol + 16 <= cfg.SLOT) and np.all(oh + 16 <= cfg.SLOT)
                                ah = np.stack([slot[o:o + 16] for o in oh]).view(np.float16).astype(np.float64)
                                al = np.stack([slot[o:o + 16] for o in ol]).view(np.float16).astype(np.float64)
                                for A in (ah, al):  # lane (m, h) of A pairs with lane (n, h) of B
                                    ph[wv, i, j] += np.einsum("hme,hne->mn", A.reshape(2, 32, 8),
                                                              bw[step].reshape(2, 32, 8))
            # superblock end: acc += d * part - 32 dmin * (X . m)
            for wv in range(WAVES):
                n_rows = np.minimum(n0 + wv * 32 * cfg.TN + 32 * np.arange(cfg.TN)[:, None] + l32, N - 1)
                for i in range(cfg.TM):
                    if q6:
                        for j in range(cfg.TN):
                            base = n_rows[j] * S * SB + sb * SB
                            d = np.array([np.frombuffer(w[o + 208:o + 210].tobytes(), np.float16)[0] for o in base[:32]], np.float64)
                            acc[wv, i, j] += d[None, :] * ph[wv, i, j]
                            ph[wv, i, j] = 0.0
                        continue
                    xo = np.minimum(m0 + 32 * i + l32, M - 1) * S * 16 + 8 * h + 16 * sb
                    assert np.all(xo + 8 <= xs.size)
                    xa = np.stack([xs[o:o + 8] for o in xo]).astype(np.float64)
                    for j in range(cfg.TN):
                        base = n_rows[j] * S * SB + sb * SB
                        d = np.array([np.frombuffer(w[o:o + 2].tobytes(), np.float16)[0] for o in base[:32]], np.float64)
                        dmin = np.array([np.frombuffer(w[o + 2:o + 4].tobytes(), np.float16)[0] for o in base[:32]], np.float64)
                        mp = np.einsum("hme,hne->mn", xa.reshape(2, 32, 8), min_b[wv, j].reshape(2, 32, 8))
                        acc[wv, i, j] += d[None, :] * ph[wv, i, j] - 32.0 * dmin[None, :] * mp
                        ph[wv, i, j] = 0.0
        # epilogue: D lane l, register r -> row 8(r/4) + 4(l/32) + r%4, column l%32
        rows = np.array([[8 * (r >> 2) + 4 * hh + (r & 3) for r in range(16)] for hh in range(2)])
        assert sorted(rows.reshape(-1)) == list(range(32))
        for wv in range(WAVES):
            for i in range(cfg.TM):
                for j in range(cfg.TN):
                    for mm in range(32):
                        m = m0 + 32 * i + mm
                        if m >= M:
                            continue
                        for nn in range(32):
                            n = n0 + wv * 32 * cfg.TN + 32 * j + nn
                            if n < N:
                                partial[split, m, n] = acc[wv, i, j, mm, nn]
                                seen[m, n] += 1
    assert np.all(seen == splits), "every output written once per split"
    y = partial[0]
    for k in range(1, splits):  # the reduce kernel adds the splits in order
        y = y + partial[k]
    y = y * scale[:, None].astype(np.float64)
    ref = oracle.reference_product(x, w, qtype, K, N)
    return y, np.asarray(ref, np.float64).reshape(M, N)


@pytest.mark.parametrize("qtype", [12, 14])
@pytest.mark.parametrize("TM,TN", [(2, 1), (1, 1)])  # the two tiles the launcher uses
@pytest.mark.parametrize("K,splits", [(768, 1), (1024, 3), (1280, 5)])
def test_gemm_model_matches_oracle(oracle, qtype, TM, TN, K, splits):
    y, ref = run_model(Cfg(TM, TN), oracle, qtype, M=70, N=300, K=K, seed=91, splits=splits)
    err = oracle.row_norm_error(y, ref)
    print(f"row-norm error {err:.3e}")
    assert err <= 1e-6


@pytest.mark.parametrize("q6", [False, True])
def test_short_prompt_prep_writes_the_staged_slot_images(q6):
    """At M <= 32 the GEMM forms a superblock's four stages in LDS itself
    (thread t: row t // 8, the 32-value block t % 8 of the superblock, 4
    pieces of 8 values per plane). Every (stage, row, 16-byte position) of the
    four slots is written exactly once, with the plane and the k range that
    the staging of prepared planes (thread f: row f // 16, position f % 16,
    piece (f % 16) ^ (row % 16)) puts there; the sub-block sums land where a
    lane (row l32, half h) reads its 16 bytes."""
    expect = {}
    for g in range(4):
        for r in range(32):
            for pos in range(16):
                L = pos ^ (r & 15)
                plane, p = L >> 3, L & 7
                k0 = stage_k(q6, g) + (64 * (p >> 2) + 8 * (p & 3) if q6 else 8 * p)
                expect[(g, r, pos)] = (plane, k0)
    got, xs = {}, {}
    for t in range(256):
        r, j = t >> 3, t & 7
        stage = 2 * (j >> 2) + (j & 1) if q6 else j >> 1
        p0 = 4 * ((j >> 1) & 1) if q6 else 4 * (j & 1)
        for q in range(4):
            for plane in range(2):
                key = (stage, r, (8 * plane + p0 + q) ^ (r & 15))
                assert key not in got
                got[key] = (plane, 32 * j + 8 * q)
        xs[2 * (16 * r + j)] = ("hi", r, j)       # byte offsets in the 32 x 16 halves
        xs[2 * (16 * r + 8 + j)] = ("lo", r, j)
    assert got == expect
    for l32 in range(32):
        for h in range(2):
            for i in range(8):
                assert xs[32 * l32 + 16 * h + 2 * i] == (("hi", "lo")[h], l32, i)


def test_a_slot_swizzle_is_conflict_free():
    """The 16 rows one ds_read_b128 pass serves (lanes 16k .. 16k+15 of a half-wave)
    read 16 different 16-byte positions of their 256-byte rows, for every piece."""
    l32 = np.arange(32)
    for plane in range(2):
        for p in range(8):
            pos = (8 * plane + p) ^ (l32 & 15)
            for k in range(2):
                assert len(set(pos[16 * k:16 * k + 16])) == 16


def test_weight_operand_fma_is_exact():
    """(1024 + q)*sc - 1024*sc and (1024 + 16q)*(sc/16) - 64*sc, fused and rounded
    once to fp16, give sc*q for every 4-bit q and 6-bit sc."""
    q = np.arange(16)[:, None].astype(np.float64)
    sc = np.arange(64)[None, :].astype(np.float64)
    lo = np.float16(1024.0 + q).astype(np.float64) * np.float16(sc).astype(np.float64) - 1024.0 * sc
    hi = np.float16(1024.0 + 16 * q).astype(np.float64) * (sc / 16.0) - 64.0 * sc
    for v in (lo, hi):
        assert np.array_equal(v.astype(np.float16).astype(np.float64), q * sc)
    assert np.all(np.float16(sc / 16.0).astype(np.float64) == sc / 16.0)
    assert np.all(np.float16(-1024.0 * sc).astype(np.float64) == -1024.0 * sc)
