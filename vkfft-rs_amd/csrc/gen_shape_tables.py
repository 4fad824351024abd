"""Shape tables of the fixed-shape kernels (kf_pow2_*.hip, kf_fam_*.hip,
kf_real_rows_*.hip): the shape lists, the LDS bank-conflict model that chose
each shape's LDS line stride LS and pad shift PS, and the emitter of the
registration files.

    python3 gen_shape_tables.py emit      # rewrite the sixteen kf_*.hip tables
    python3 gen_shape_tables.py check     # re-run the model search per shape
    python3 gen_shape_tables.py round     # re-derive the round-length rows by rule

Bank model (fitted to the SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE ratios the
fixed kernels measured on gfx950): 32 banks of 4 bytes; an 8-byte access of a
wave is served 16 lanes per cycle, a 16-byte access 8 lanes per cycle; a
group costs its largest number of lanes on one bank. A shape's score is the
cost of all its LDS accesses (Stockham stage reads and writes between the
direct first and last stages; staged rows add the cooperative load and store
copies) over the cost of the same accesses laid out conflict-free. `check`
searches PS in {2, 3, 4, 5, 6, 30 (no padding)} and LS from the smallest line
that fits upward, under the LDS cap of the shape (80 KiB for several lines
per block, 156 KiB for one), and prints the recorded choice beside the best
score. Real-transform rows (kf_real_rows_*) reuse the PS/LS of the C2C row of
the same half length.

Nontemporal roles registered per shape: rows -- both directions, input
streamed, output streamed or cached; columns -- both directions, input
cached, output cached or streamed; four-step column passes (FS_A) -- both
directions, cached; R2C half rows -- forward, input streamed; C2R half rows
-- inverse, output streamed.
"""
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))

# ------------------------------------------------------------ bank model

BANKS = 32


def lpad(e, ps):
    return e + (e >> ps)


def wave_lanes(col, G, TT, wave):
    """(line, thread) of each lane of wave `wave` (None past the block)."""
    out = []
    for lane in range(64):
        tid = wave * 64 + lane
        if tid >= G * TT:
            out.append(None)
        elif col:
            out.append((tid % G, tid // G))
        else:
            out.append((tid // TT, tid % TT))
    return out


def cost(addrs, eb):
    """Cycles of one wave access: dword addresses (None = inactive lane)."""
    per = BANKS * 4 // eb
    total = 0
    for s in range(0, 64, per):
        cnt = {}
        for a in addrs[s:s + per]:
            if a is None:
                continue
            for w in range(eb // 4):
                b = (a + w) % BANKS
                cnt[b] = cnt.get(b, 0) + 1
        total += max(cnt.values()) if cnt else 0
    return total


def ideal(addrs, eb):
    return cost([None if a is None else 2 * k * (eb // 8) for k, a in enumerate(addrs)], eb)


def stage_accesses(N, TT, G, PS, LS, col, radices, first_lds, last_lds, eb):
    """LDS addresses of the Stockham stages (kernel_ir.rs:4565-4608 stage
    semantics) run over G lines of length N by TT threads each."""
    P = 1
    waves = (G * TT + 63) // 64
    out = []
    for si, R in enumerate(radices):
        NB = N // R
        MJ = (NB + TT - 1) // TT
        for w in range(waves):
            lanes = wave_lanes(col, G, TT, w)
            for j in range(MJ):
                if si > 0 or first_lds:
                    for i in range(R):
                        ad = []
                        for gt in lanes:
                            bb = None if gt is None else gt[1] + j * TT
                            if gt is None or bb >= NB:
                                ad.append(None)
                            else:
                                ad.append((gt[0] * LS + lpad(bb + i * NB, PS)) * eb // 4)
                        out.append(ad)
                if si < len(radices) - 1 or last_lds:
                    for q in range(R):
                        ad = []
                        for gt in lanes:
                            bb = None if gt is None else gt[1] + j * TT
                            if gt is None or bb >= NB:
                                ad.append(None)
                            else:
                                k = bb % P
                                ad.append((gt[0] * LS + lpad((bb - k) * R + k + q * P, PS)) * eb // 4)
                        out.append(ad)
        P *= R
    return out


def coop(G, N, PS, LS, nthreads, eb):
    """The staged copies (coop_for over contiguous lines)."""
    out = []
    total = G * N
    for base in range(0, total, nthreads):
        for w0 in range(base, min(base + nthreads, total), 64):
            ad = []
            for idx in range(w0, w0 + 64):
                if idx >= total or idx >= base + nthreads:
                    ad.append(None)
                else:
                    ad.append(((idx // N) * LS + lpad(idx % N, PS)) * eb // 4)
            out.append(ad)
    return out


def score(N, TT, G, PS, LS, col, radices, staged, eb):
    if staged:
        acc = coop(G, N, PS, LS, G * TT, eb) + stage_accesses(N, TT, G, PS, LS, col, radices, True, True, eb) + \
            coop(G, N, PS, LS, G * TT, eb)
    else:
        acc = stage_accesses(N, TT, G, PS, LS, col, radices, False, False, eb)
    a = sum(cost(x, eb) for x in acc)
    i = sum(ideal(x, eb) for x in acc)
    return a / i if i else 1.0


def search(N, TT, G, col, radices, staged, eb):
    cap = 80 * 1024 if G > 1 else 160 * 1024 - 4096
    res = []
    for PS in (2, 3, 4, 5, 6, 30):
        base = N + ((N - 1) >> PS if PS < 30 else 0)
        for LS in range(base, base + 20):
            if G * LS * eb > cap:
                break
            res.append((round(score(N, TT, G, PS, LS, col, radices, staged, eb), 3), G * LS, PS, LS))
    res.sort()
    return res[0] if res else None


# ------------------------------------------------------------ shape lists

# (kind, io, N, threads per line, lines per block, columns?, radices, PS, LS);
# strings are comment lines of the table
TABLES = {
    "kf_pow2_f32": [
        ('PLAIN', 'PlainStaged', 8, 1, 64, False, [8], 2, 9),
        ('PLAIN', 'PlainStaged', 16, 1, 64, False, [16], 4, 17),
        ('PLAIN', 'PlainStaged', 32, 8, 32, False, [8, 4], 4, 36),
        ('PLAIN', 'PlainStaged', 64, 8, 32, False, [8, 8], 4, 72),
        ('PLAIN', 'PlainStaged', 128, 16, 16, False, [16, 8], 4, 135),
        ('PLAIN', 'Plain', 256, 16, 16, False, [16, 16], 4, 271),
        ('PLAIN', 'Plain', 512, 64, 4, False, [8, 8, 8], 4, 543),
        ('PLAIN', 'Plain', 2048, 256, 1, False, [16, 16, 8], 4, 2175),
        ('PLAIN', 'Plain', 8192, 512, 1, False, [16, 16, 8, 4], 4, 8703),
        ('PLAIN', 'Plain', 16384, 1024, 1, False, [16, 16, 16, 4], 4, 17407),
        ('PLAIN', 'Plain', 8, 1, 64, True, [8], 3, 8),
        ('PLAIN', 'Plain', 16, 1, 64, True, [16], 4, 16),
        ('PLAIN', 'Plain', 32, 8, 32, True, [8, 4], 4, 33),
        ('PLAIN', 'Plain', 128, 16, 16, True, [16, 8], 6, 129),
        ('PLAIN', 'Plain', 256, 16, 16, True, [16, 16], 30, 257),
        ('PLAIN', 'Plain', 512, 64, 16, True, [8, 8, 8], 30, 513),
        ('FS_A', 'FsA', 32, 8, 32, True, [8, 4], 4, 33),
        ('FS_A', 'FsA', 128, 16, 16, True, [16, 8], 6, 129),
    ],
    "kf_pow2_f64": [
        ('PLAIN', 'PlainStaged', 8, 1, 64, False, [8], 3, 9),
        ('PLAIN', 'PlainStaged', 16, 1, 64, False, [16], 3, 17),
        ('PLAIN', 'PlainStaged', 32, 8, 32, False, [8, 4], 3, 35),
        ('PLAIN', 'Plain', 64, 8, 32, False, [8, 8], 3, 71),
        ('PLAIN', 'Plain', 128, 16, 16, False, [16, 8], 4, 135),
        ('PLAIN', 'Plain', 256, 16, 16, False, [16, 16], 4, 271),
        ('PLAIN', 'Plain', 1024, 128, 2, False, [16, 8, 8], 4, 1087),
        ('PLAIN', 'Plain', 2048, 256, 1, False, [16, 16, 8], 4, 2175),
        ('PLAIN', 'Plain', 4096, 256, 1, False, [16, 16, 16], 4, 4351),
        ('PLAIN', 'Plain', 8192, 512, 1, False, [16, 16, 8, 4], 4, 8703),
        ('PLAIN', 'Plain', 8, 1, 64, True, [8], 3, 8),
        ('PLAIN', 'Plain', 16, 1, 64, True, [16], 4, 16),
        ('PLAIN', 'Plain', 32, 8, 32, True, [8, 4], 4, 33),
        ('PLAIN', 'Plain', 64, 8, 32, True, [8, 8], 5, 65),
        ('PLAIN', 'Plain', 128, 16, 16, True, [16, 8], 6, 129),
        ('PLAIN', 'Plain', 256, 16, 16, True, [16, 16], 30, 257),
        ('FS_A', 'FsA', 32, 8, 32, True, [8, 4], 4, 33),
        ('FS_A', 'FsA', 64, 8, 32, True, [8, 8], 5, 65),
        ('FS_A', 'FsA', 128, 16, 16, True, [16, 8], 6, 129),
    ],
    "kf_fam_f32": [
        ('PLAIN', 'PlainStaged', 12, 3, 64, False, [4, 3], 4, 19),
        ('PLAIN', 'PlainStaged', 24, 3, 64, False, [8, 3], 5, 35),
        ('PLAIN', 'PlainStaged', 48, 3, 64, False, [16, 3], 4, 51),
        ('PLAIN', 'PlainStaged', 96, 6, 42, False, [16, 6], 4, 102),
        ('PLAIN', 'PlainStaged', 192, 12, 21, False, [16, 12], 4, 204),
        ('PLAIN', 'Plain', 384, 24, 10, False, [16, 8, 3], 4, 409),
        ('PLAIN', 'Plain', 768, 48, 5, False, [16, 16, 3], 4, 815),
        ('PLAIN', 'Plain', 1536, 96, 2, False, [16, 16, 6], 4, 1631),
        ('PLAIN', 'Plain', 3072, 192, 1, False, [16, 16, 12], 4, 3263),
        ('PLAIN', 'Plain', 6144, 384, 1, False, [16, 16, 8, 3], 4, 6527),
        ('PLAIN', 'Plain', 12288, 768, 1, False, [16, 16, 16, 3], 4, 13055),
        ('PLAIN', 'PlainStaged', 20, 4, 64, False, [4, 5], 5, 20),
        ('PLAIN', 'PlainStaged', 40, 5, 51, False, [8, 5], 5, 53),
        ('PLAIN', 'PlainStaged', 80, 5, 51, False, [16, 5], 4, 85),
        ('PLAIN', 'PlainStaged', 160, 10, 25, False, [16, 10], 4, 170),
        ('PLAIN', 'Plain', 320, 40, 6, False, [8, 8, 5], 3, 360),
        ('PLAIN', 'Plain', 640, 40, 6, False, [16, 8, 5], 4, 680),
        ('PLAIN', 'Plain', 1280, 80, 3, False, [16, 16, 5], 4, 1359),
        ('PLAIN', 'Plain', 2560, 160, 1, False, [16, 16, 10], 4, 2719),
        ('PLAIN', 'Plain', 5120, 320, 1, False, [16, 16, 4, 5], 4, 5439),
        ('PLAIN', 'Plain', 10240, 640, 1, False, [16, 16, 8, 5], 4, 10879),
        ('PLAIN', 'PlainStaged', 100, 10, 25, False, [10, 10], 6, 106),
        ('PLAIN', 'Plain', 1000, 100, 2, False, [10, 10, 10], 30, 1012),
        ('PLAIN', 'Plain', 10000, 1000, 1, False, [10, 10, 10, 10], 30, 10000),
        ('PLAIN', 'Plain', 360, 40, 6, False, [8, 9, 5], 4, 394),
        "// strided columns (G adjacent columns per block, 128-byte or wider row segments)",
        ('PLAIN', 'Plain', 12, 3, 64, True, [4, 3], 3, 13),
        ('PLAIN', 'Plain', 20, 4, 64, True, [4, 5], 4, 21),
        ('PLAIN', 'Plain', 24, 3, 64, True, [8, 3], 4, 25),
        ('PLAIN', 'Plain', 40, 5, 64, True, [8, 5], 5, 41),
        ('PLAIN', 'Plain', 48, 3, 64, True, [16, 3], 5, 49),
        ('PLAIN', 'Plain', 80, 5, 64, True, [16, 5], 6, 81),
        ('PLAIN', 'Plain', 96, 6, 64, True, [16, 6], 6, 97),
        ('PLAIN', 'Plain', 100, 10, 32, True, [10, 10], 6, 101),
        ('PLAIN', 'Plain', 160, 10, 32, True, [16, 10], 30, 161),
        ('PLAIN', 'Plain', 192, 12, 32, True, [16, 12], 30, 193),
        ('PLAIN', 'Plain', 320, 40, 16, True, [8, 8, 5], 30, 321),
        ('PLAIN', 'Plain', 360, 40, 16, True, [8, 9, 5], 30, 361),
        ('PLAIN', 'Plain', 384, 24, 16, True, [16, 8, 3], 30, 385),
        ('PLAIN', 'Plain', 640, 40, 8, True, [16, 8, 5], 4, 682),
    ],
    "kf_fam_f64": [
        ('PLAIN', 'PlainStaged', 12, 3, 64, False, [4, 3], 4, 19),
        ('PLAIN', 'PlainStaged', 24, 3, 64, False, [8, 3], 3, 27),
        ('PLAIN', 'PlainStaged', 48, 3, 64, False, [16, 3], 4, 51),
        ('PLAIN', 'PlainStaged', 96, 6, 42, False, [16, 6], 4, 102),
        ('PLAIN', 'Plain', 192, 12, 21, False, [16, 12], 4, 204),
        ('PLAIN', 'Plain', 384, 24, 10, False, [16, 8, 3], 4, 407),
        ('PLAIN', 'Plain', 768, 48, 5, False, [16, 16, 3], 4, 815),
        ('PLAIN', 'Plain', 1536, 96, 2, False, [16, 16, 6], 4, 1631),
        ('PLAIN', 'Plain', 3072, 192, 1, False, [16, 16, 12], 4, 3263),
        ('PLAIN', 'Plain', 6144, 384, 1, False, [16, 16, 8, 3], 4, 6527),
        ('PLAIN', 'PlainStaged', 20, 4, 64, False, [4, 5], 5, 20),
        ('PLAIN', 'PlainStaged', 40, 5, 51, False, [8, 5], 3, 45),
        ('PLAIN', 'PlainStaged', 80, 5, 51, False, [16, 5], 4, 85),
        ('PLAIN', 'Plain', 160, 10, 25, False, [16, 10], 4, 170),
        ('PLAIN', 'Plain', 320, 40, 6, False, [8, 8, 5], 3, 359),
        ('PLAIN', 'Plain', 640, 40, 6, False, [16, 8, 5], 4, 679),
        ('PLAIN', 'Plain', 1280, 80, 3, False, [16, 16, 5], 4, 1359),
        ('PLAIN', 'Plain', 2560, 160, 1, False, [16, 16, 10], 4, 2719),
        ('PLAIN', 'Plain', 5120, 320, 1, False, [16, 16, 4, 5], 4, 5439),
        ('PLAIN', 'Plain', 100, 10, 25, False, [10, 10], 6, 106),
        ('PLAIN', 'Plain', 1000, 100, 2, False, [10, 10, 10], 6, 1022),
        ('PLAIN', 'Plain', 360, 40, 6, False, [8, 9, 5], 3, 404),
        "// strided columns (G adjacent columns per block, 128-byte or wider row segments)",
        ('PLAIN', 'Plain', 12, 3, 64, True, [4, 3], 3, 13),
        ('PLAIN', 'Plain', 20, 4, 64, True, [4, 5], 4, 21),
        ('PLAIN', 'Plain', 24, 3, 64, True, [8, 3], 4, 25),
        ('PLAIN', 'Plain', 40, 5, 64, True, [8, 5], 5, 41),
        ('PLAIN', 'Plain', 48, 3, 64, True, [16, 3], 5, 49),
        ('PLAIN', 'Plain', 80, 5, 32, True, [16, 5], 6, 81),
        ('PLAIN', 'Plain', 96, 6, 32, True, [16, 6], 6, 97),
        ('PLAIN', 'Plain', 100, 10, 32, True, [10, 10], 6, 101),
        ('PLAIN', 'Plain', 160, 10, 16, True, [16, 10], 30, 161),
        ('PLAIN', 'Plain', 192, 12, 16, True, [16, 12], 30, 193),
        ('PLAIN', 'Plain', 320, 40, 8, True, [8, 8, 5], 30, 321),
        ('PLAIN', 'Plain', 360, 40, 8, True, [8, 9, 5], 30, 361),
        ('PLAIN', 'Plain', 384, 24, 8, True, [16, 8, 3], 30, 385),
        ('PLAIN', 'Plain', 640, 40, 4, True, [16, 8, 5], 4, 682),
    ],
    "kf_real_rows_f32": [
        ('R2C_HALF', 'R2CHalf', 256, 16, 16, False, [16, 16], 4, 271),
        ('C2R_HALF', 'C2RHalf', 256, 16, 16, False, [16, 16], 4, 271),
        ('R2C_HALF', 'R2CHalf', 512, 64, 4, False, [8, 8, 8], 4, 543),
        ('C2R_HALF', 'C2RHalf', 512, 64, 4, False, [8, 8, 8], 4, 543),
        ('R2C_HALF', 'R2CHalf', 1024, 128, 1, False, [16, 8, 8], 4, 1088),
        ('C2R_HALF', 'C2RHalf', 1024, 128, 1, False, [16, 8, 8], 4, 1088),
        ('R2C_HALF', 'R2CHalf', 2048, 256, 1, False, [16, 16, 8], 4, 2175),
        ('C2R_HALF', 'C2RHalf', 2048, 256, 1, False, [16, 16, 8], 4, 2175),
        ('R2C_HALF', 'R2CHalf', 4096, 256, 1, False, [16, 16, 16], 4, 4352),
        ('C2R_HALF', 'C2RHalf', 4096, 256, 1, False, [16, 16, 16], 4, 4352),
        ('R2C_HALF', 'R2CHalf', 8192, 512, 1, False, [16, 16, 8, 4], 4, 8703),
        ('C2R_HALF', 'C2RHalf', 8192, 512, 1, False, [16, 16, 8, 4], 4, 8703),
        ('R2C_HALF', 'R2CHalf', 384, 24, 10, False, [16, 8, 3], 4, 409),
        ('C2R_HALF', 'C2RHalf', 384, 24, 10, False, [16, 8, 3], 4, 409),
        ('R2C_HALF', 'R2CHalf', 768, 48, 5, False, [16, 16, 3], 4, 815),
        ('C2R_HALF', 'C2RHalf', 768, 48, 5, False, [16, 16, 3], 4, 815),
        ('R2C_HALF', 'R2CHalf', 1536, 96, 2, False, [16, 16, 6], 4, 1631),
        ('C2R_HALF', 'C2RHalf', 1536, 96, 2, False, [16, 16, 6], 4, 1631),
        ('R2C_HALF', 'R2CHalf', 3072, 192, 1, False, [16, 16, 12], 4, 3263),
        ('C2R_HALF', 'C2RHalf', 3072, 192, 1, False, [16, 16, 12], 4, 3263),
        ('R2C_HALF', 'R2CHalf', 6144, 384, 1, False, [16, 16, 8, 3], 4, 6527),
        ('C2R_HALF', 'C2RHalf', 6144, 384, 1, False, [16, 16, 8, 3], 4, 6527),
        ('R2C_HALF', 'R2CHalf', 320, 40, 6, False, [8, 8, 5], 3, 360),
        ('C2R_HALF', 'C2RHalf', 320, 40, 6, False, [8, 8, 5], 3, 360),
        ('R2C_HALF', 'R2CHalf', 640, 40, 6, False, [16, 8, 5], 4, 680),
        ('C2R_HALF', 'C2RHalf', 640, 40, 6, False, [16, 8, 5], 4, 680),
        ('R2C_HALF', 'R2CHalf', 1280, 80, 3, False, [16, 16, 5], 4, 1359),
        ('C2R_HALF', 'C2RHalf', 1280, 80, 3, False, [16, 16, 5], 4, 1359),
        ('R2C_HALF', 'R2CHalf', 2560, 160, 1, False, [16, 16, 10], 4, 2719),
        ('C2R_HALF', 'C2RHalf', 2560, 160, 1, False, [16, 16, 10], 4, 2719),
        ('R2C_HALF', 'R2CHalf', 5120, 320, 1, False, [16, 16, 4, 5], 4, 5439),
        ('C2R_HALF', 'C2RHalf', 5120, 320, 1, False, [16, 16, 4, 5], 4, 5439),
    ],
    "kf_real_rows_f64": [
        ('R2C_HALF', 'R2CHalf', 64, 8, 32, False, [8, 8], 3, 71),
        ('C2R_HALF', 'C2RHalf', 64, 8, 32, False, [8, 8], 3, 71),
        ('R2C_HALF', 'R2CHalf', 128, 16, 16, False, [16, 8], 4, 135),
        ('C2R_HALF', 'C2RHalf', 128, 16, 16, False, [16, 8], 4, 135),
        ('R2C_HALF', 'R2CHalf', 256, 16, 16, False, [16, 16], 4, 271),
        ('C2R_HALF', 'C2RHalf', 256, 16, 16, False, [16, 16], 4, 271),
        ('R2C_HALF', 'R2CHalf', 512, 64, 2, False, [8, 8, 8], 3, 576),
        ('C2R_HALF', 'C2RHalf', 512, 64, 2, False, [8, 8, 8], 3, 576),
        ('R2C_HALF', 'R2CHalf', 1024, 128, 2, False, [16, 8, 8], 4, 1087),
        ('C2R_HALF', 'C2RHalf', 1024, 128, 2, False, [16, 8, 8], 4, 1087),
        ('R2C_HALF', 'R2CHalf', 2048, 256, 1, False, [16, 16, 8], 4, 2175),
        ('C2R_HALF', 'C2RHalf', 2048, 256, 1, False, [16, 16, 8], 4, 2175),
        ('R2C_HALF', 'R2CHalf', 4096, 256, 1, False, [16, 16, 16], 4, 4351),
        ('C2R_HALF', 'C2RHalf', 4096, 256, 1, False, [16, 16, 16], 4, 4351),
        ('R2C_HALF', 'R2CHalf', 192, 12, 21, False, [16, 12], 4, 204),
        ('C2R_HALF', 'C2RHalf', 192, 12, 21, False, [16, 12], 4, 204),
        ('R2C_HALF', 'R2CHalf', 384, 24, 10, False, [16, 8, 3], 4, 407),
        ('C2R_HALF', 'C2RHalf', 384, 24, 10, False, [16, 8, 3], 4, 407),
        ('R2C_HALF', 'R2CHalf', 768, 48, 5, False, [16, 16, 3], 4, 815),
        ('C2R_HALF', 'C2RHalf', 768, 48, 5, False, [16, 16, 3], 4, 815),
        ('R2C_HALF', 'R2CHalf', 1536, 96, 2, False, [16, 16, 6], 4, 1631),
        ('C2R_HALF', 'C2RHalf', 1536, 96, 2, False, [16, 16, 6], 4, 1631),
        ('R2C_HALF', 'R2CHalf', 3072, 192, 1, False, [16, 16, 12], 4, 3263),
        ('C2R_HALF', 'C2RHalf', 3072, 192, 1, False, [16, 16, 12], 4, 3263),
        ('R2C_HALF', 'R2CHalf', 160, 10, 25, False, [16, 10], 4, 170),
        ('C2R_HALF', 'C2RHalf', 160, 10, 25, False, [16, 10], 4, 170),
        ('R2C_HALF', 'R2CHalf', 320, 40, 6, False, [8, 8, 5], 3, 359),
        ('C2R_HALF', 'C2RHalf', 320, 40, 6, False, [8, 8, 5], 3, 359),
        ('R2C_HALF', 'R2CHalf', 640, 40, 6, False, [16, 8, 5], 4, 679),
        ('C2R_HALF', 'C2RHalf', 640, 40, 6, False, [16, 8, 5], 4, 679),
        ('R2C_HALF', 'R2CHalf', 1280, 80, 3, False, [16, 16, 5], 4, 1359),
        ('C2R_HALF', 'C2RHalf', 1280, 80, 3, False, [16, 16, 5], 4, 1359),
        ('R2C_HALF', 'R2CHalf', 2560, 160, 1, False, [16, 16, 10], 4, 2719),
        ('C2R_HALF', 'C2RHalf', 2560, 160, 1, False, [16, 16, 10], 4, 2719),
    ],
}

# Round lengths with factors 2, 3 and 5 outside the families above (common
# decimal-like sizes), as one-upload rows built by rule: the radix plan with
# the fewest stages from {16, 12, 10, 9, 8, 6, 5, 4, 3, 2} (then the largest
# smallest radix, then the largest first radix), largest radix first;
# threads per line = N / the largest radix; about 256 threads per block; LDS
# stride and pad from the bank model's search.
ROUND = [200, 240, 300, 400, 480, 500, 600, 720, 750, 800, 900, 960, 1200, 1500, 1600, 1800, 1920, 2000, 2400,
         2500, 3000, 3200, 3600, 4000, 4800, 5000, 6000, 6400, 7200, 8000, 9000, 9600, 12000, 15000, 16000]
RADICES = (16, 12, 10, 9, 8, 6, 5, 4, 3, 2)


def radix_plan(n, radices=RADICES):
    """Fewest stages, then the largest smallest radix, then the largest first radix."""
    best = None

    def rec(rest, start, acc):
        nonlocal best
        if rest == 1:
            plan = sorted(acc, reverse=True)
            key = (len(plan), -min(plan), -plan[0])
            if best is None or key < best[0]:
                best = (key, plan)
            return
        if len(acc) >= 5:
            return
        for i in range(start, len(radices)):
            r = radices[i]
            if rest % r == 0:
                rec(rest // r, i, acc + [r])

    rec(n, 0, [])
    return best[1] if best else None


def round_rows(prec):
    eb = 16 if prec else 8
    rows = []
    for n in ROUND:
        if prec and n > 8192:
            continue  # longer f64 lines are two uploads (the runtime line with its pad exceeds the LDS)
        rad = radix_plan(n)
        tt = n // max(rad)
        if tt > 1024:
            continue
        g = max(1, min(256 // tt, 64))
        while g > 1 and g * (n + (n >> 2)) * eb > 80 * 1024:
            g -= 1
        best = search(n, tt, g, False, rad, False, eb)
        if best is None:
            continue
        _, _, ps, ls = best
        rows.append(('PLAIN', 'Plain', n, tt, g, False, rad, ps, ls))
    return rows


def _smooth(lo, hi):
    return sorted({2 ** a * 3 ** b * 5 ** c for a in range(15) for b in range(9) for c in range(7)
                   if lo <= 2 ** a * 3 ** b * 5 ** c <= hi})


def _split_pair(n):
    """The two factors a strided axis of length n > 640 is split into (the
    runtime's split_strided_axis: the smallest larger factor)."""
    best = None
    a = 2
    while a * a <= n:
        if n % a == 0 and (best is None or max(a, n // a) < best[0]):
            best = (max(a, n // a), min(a, n // a))
        a += 1
    return best


def nd_rows(prec, have):
    """Shapes the N-D passes of lengths with factors 2, 3 and 5 need beyond the
    other tables (`have`: (kind, N, col) already registered): strided columns of
    every such length up to 640 (the longest strided axis of one pass), the
    first split pass (FS_A columns) of the longer ones, and short rows staged
    through LDS. Columns: threads per line = N / the largest radix, the
    largest power-of-two lines per block up to 64 within 80 KiB and 1024
    threads, an odd LDS stride without pads (lanes walk adjacent lines);
    short rows: about 256 threads per block, LDS stride from the model search."""
    eb = 16 if prec else 8
    rows = []

    def col_shape(kind, io, n):
        rad = radix_plan(n)
        tt = n // max(rad)
        ls = n if n % 2 else n + 1
        G = 64
        while G > 1 and (G * ls * eb > 80 * 1024 or G * tt > 1024):
            G //= 2
        return (kind, io, n, tt, G, True, rad, 30, ls)

    for n in _smooth(6, 640):
        if ('PLAIN', n, True) not in have:
            rows.append(col_shape('PLAIN', 'Plain', n))
    for hi in sorted({_split_pair(n)[0] for n in _smooth(641, 16384)}):
        if ('FS_A', hi, True) not in have:
            rows.append(col_shape('FS_A', 'FsA', hi))
    for n in _smooth(6, 199):
        if ('PLAIN', n, False) in have:
            continue
        rad = radix_plan(n)
        tt = n // max(rad)
        G = max(1, min(64, 256 // tt))
        best = search(n, tt, G, False, rad, True, eb)
        rows.append(('PLAIN', 'PlainStaged', n, tt, G, False, rad, best[2], best[3]))
    return rows


def registered_keys(prec, skip=()):
    """(kind, N, col) of every shape of one precision registered in both
    directions: the generated tables except `skip` (always both), and the
    hand-written kf_plain / kf_nd / kf_real / kf_blue tables."""
    import re
    have = set()
    for other, items in TABLES.items():
        if other in skip or other.endswith("f64") != bool(prec):
            continue
        have |= {(it[0], it[2], it[5]) for it in items if not isinstance(it, str)}
    dirs = {}
    pat = r"KK_(\w+), Io\w+, (float|double), (\d), (-?\d), (\d+), \d+, \d+, \d+, \d+, (true|false)"
    for f in ("kf_plain.hip", "kf_nd.hip", "kf_real.hip", "kf_blue.hip"):
        for m in re.finditer(pat, open(os.path.join(HERE, f)).read()):
            if int(m.group(3)) == prec:
                dirs.setdefault((m.group(1), int(m.group(5)), m.group(6) == "true"), set()).add(int(m.group(4)))
    have |= {k for k, d in dirs.items() if d == {-1, 1}}
    return have


# Factors of the two-upload four-step (the split four_step_split picks: the
# smallest larger factor) for common lengths: powers of two and round ones.
FOURSTEP = [128, 240, 250, 256, 400, 500, 512, 1000, 1024, 2000, 2048]


def fourstep_rows(prec, have):
    """FS_A column passes (threads per line = N / the largest radix, the
    largest power-of-two columns per block up to 32 within 150 KiB and 1024
    threads, odd LDS stride) and FS_B row passes (up to 16 rows per block
    for 128-byte transposed stores, the rows' pad rule) of the FOURSTEP
    lengths not registered yet."""
    eb = 16 if prec else 8
    ps_row = 3 if prec else 4
    rows = []
    for n in FOURSTEP:
        rad = radix_plan(n)
        tt = n // max(rad)
        if ('FS_A', n, True) not in have:
            ls = n if n % 2 else n + 1
            G = 32
            while G > 1 and (G * ls * eb > 150 * 1024 or G * tt > 1024):
                G //= 2
            rows.append(('FS_A', 'FsA', n, tt, G, True, rad, 30, ls))
        if ('FS_B', n, False) not in have:
            ls = n + (n >> ps_row)
            ls += 1 - ls % 2
            G = 16
            while G > 1 and (G * ls * eb > 150 * 1024 or G * tt > 1024):
                G //= 2
            rows.append(('FS_B', 'FsB', n, tt, G, False, rad, ps_row, ls))
    return rows


# The planner's most frequent Bluestein convolution lengths (the padded M of
# the primes up to 8200 that run as Bluestein: 16384, 8192, 6561, 4096, ...)
# Convolution lengths M >= 256 that the planner's Bluestein padding tables
# give (f32: the AMD f32 table plus 16384, which the generic padding gives for
# lengths 4097-8192; f64: the wide table), keeping those with a plan of
# radices 2-16.
BLUE_M = {0: [256, 512, 625, 768, 1024, 1296, 2048, 2187, 2304, 2500, 2592, 3072, 3125, 3136, 4096, 4375, 4608,
              5184, 6561, 8192, 16384],
          1: [256, 270, 512, 625, 640, 750, 756, 768, 875, 1024, 1296, 1323, 1344, 1512, 1792, 2016, 2048, 2187,
              3136, 3430, 3584, 4096, 4375, 4480, 4704, 5103, 5376, 6048, 6144, 8192]}


def blue_rows(prec):
    """One-kernel Bluestein rows (chirp multiply, FFT of M, spectrum multiply
    fused into its last stage, inverse FFT, chirp multiply and truncation):
    the rule's radix plan, threads per line = M / the largest radix, about 256
    threads per block, the rows' pad rule (one slot per 16 f32 / 8 f64)."""
    eb = 16 if prec else 8
    ps = 3 if prec else 4
    rows = []
    for m in BLUE_M[prec]:
        rad = radix_plan(m, (16, 12, 10, 9, 8, 7, 6, 5, 4, 3, 2))
        tt = m // max(rad)
        ls = m + (m >> ps)
        ls += 1 - ls % 2
        if tt > 1024 or ls * eb > 156 * 1024:
            continue
        G = max(1, min(64, 256 // tt))
        while G > 1 and (G * ls * eb > 80 * 1024 or G * tt > 1024):
            G -= 1
        rows.append(('BLUE_1', 'Blue1', m, tt, G, False, rad, ps, ls))
    return rows


HEADS_ROUND = ("// Fixed shapes of round lengths with factors 2, 3 and 5 outside the\n"
               "// power-of-two, 3*2^k and 5*2^k families, {p}: one-upload rows (1-D batches\n"
               "// and the contiguous axis of N-D transforms) in both directions and both\n"
               "// nontemporal roles. Radix plans with the fewest LDS-exchanged stages from\n"
               "// radices 2-16 (composite 6, 9, 10, 12); threads per line = N / the largest\n"
               "// radix; about 256 threads per block; LDS strides minimise bank conflicts\n"
               "// under the 32-bank model of 8-byte accesses.\n")

HEADS = {'kf_pow2_f32': "// Fixed shapes of the power-of-two lengths outside the benchmark\n// configurations, f32: rows of one upload (1-D batches and the contiguous\n// axis of N-D transforms), strided columns up to the length that stays one\n// upload per axis, and the first pass of split strided axes. Each shape is\n// registered for both directions and for the two nontemporal roles its pass\n// can take (rows: the caller's input, with or without the caller's output;\n// columns: cached input, with or without the caller's output). LDS strides\n// minimise bank conflicts under the 32-bank model of 8-byte accesses (16 lanes\n// served per cycle). Short rows, whose first or last Stockham stage would touch\n// HBM in segments narrower than 128 bytes, stage both ends through LDS\n// (IoPlainStaged).\n", 'kf_pow2_f64': "// Fixed shapes of the power-of-two lengths outside the benchmark\n// configurations, f64: rows of one upload (1-D batches and the contiguous\n// axis of N-D transforms), strided columns up to the length that stays one\n// upload per axis, and the first pass of split strided axes. Each shape is\n// registered for both directions and for the two nontemporal roles its pass\n// can take (rows: the caller's input, with or without the caller's output;\n// columns: cached input, with or without the caller's output). LDS strides\n// minimise bank conflicts under the 32-bank model of 8-byte accesses (16 lanes\n// served per cycle). Short rows, whose first or last Stockham stage would touch\n// HBM in segments narrower than 128 bytes, stage both ends through LDS\n// (IoPlainStaged).\n", 'kf_fam_f32': '// Fixed shapes of common lengths with factors 3 and 5, f32: 3*2^k, 5*2^k,\n// 10^k and 360, as rows of one upload (1-D batches and the contiguous axis of\n// N-D transforms) and as strided columns up to 640, each in both directions\n// and both nontemporal roles. Radix plans keep at most three or four\n// LDS-exchanged stages (composite radices 6, 10 and 12 where they save one);\n// threads per line = N / the largest radix; LDS strides minimise bank\n// conflicts under the 32-bank model of 8-byte accesses. Short rows stage both\n// ends through LDS (IoPlainStaged).\n', 'kf_fam_f64': '// Fixed shapes of common lengths with factors 3 and 5, f64: 3*2^k, 5*2^k,\n// 10^k and 360, as rows of one upload (1-D batches and the contiguous axis of\n// N-D transforms) and as strided columns up to 640, each in both directions\n// and both nontemporal roles. Radix plans keep at most three or four\n// LDS-exchanged stages (composite radices 6, 10 and 12 where they save one);\n// threads per line = N / the largest radix; LDS strides minimise bank\n// conflicts under the 32-bank model of 8-byte accesses. Short rows stage both\n// ends through LDS (IoPlainStaged).\n', 'kf_real_rows_f32': "// Fixed shapes of the one-upload even-length real transforms, f32: the\n// half-size packed FFT of R2C (postprocess fused into the staged store) and of\n// C2R (preprocess fused into the direct loads) for half lengths M that have a\n// fixed C2C row shape (powers of two and the 3*2^k / 5*2^k families), with the\n// same radices, threads, lines per block and LDS strides as those rows. R2C is\n// registered for the caller's input with or without the caller's output, C2R\n// for the caller's output with or without the caller's input.\n", 'kf_real_rows_f64': "// Fixed shapes of the one-upload even-length real transforms, f64: the\n// half-size packed FFT of R2C (postprocess fused into the staged store) and of\n// C2R (preprocess fused into the direct loads) for half lengths M that have a\n// fixed C2C row shape (powers of two and the 3*2^k / 5*2^k families), with the\n// same radices, threads, lines per block and LDS strides as those rows. R2C is\n// registered for the caller's input with or without the caller's output, C2R\n// for the caller's output with or without the caller's input.\n"}

# round_rows(0) / round_rows(1) (the model search takes minutes in pure
# Python: `python3 gen_shape_tables.py round` re-derives these lists)
TABLES['kf_round_f32'] = [('PLAIN', 'Plain', 200, 25, 10, False, [8, 5, 5], 5, 217), ('PLAIN', 'Plain', 240, 30, 8, False, [8, 6, 5], 4, 255), ('PLAIN', 'Plain', 300, 25, 10, False, [12, 5, 5], 6, 313), ('PLAIN', 'Plain', 400, 25, 10, False, [16, 5, 5], 4, 425), ('PLAIN', 'Plain', 480, 48, 5, False, [10, 8, 6], 30, 480), ('PLAIN', 'Plain', 500, 50, 5, False, [10, 10, 5], 6, 515), ('PLAIN', 'Plain', 600, 60, 4, False, [10, 10, 6], 30, 604), ('PLAIN', 'Plain', 720, 72, 3, False, [10, 9, 8], 30, 728), ('PLAIN', 'Plain', 750, 125, 2, False, [6, 5, 5, 5], 30, 765), ('PLAIN', 'Plain', 800, 80, 3, False, [10, 10, 8], 6, 812), ('PLAIN', 'Plain', 900, 90, 2, False, [10, 10, 9], 30, 906), ('PLAIN', 'Plain', 960, 80, 3, False, [12, 10, 8], 5, 989), ('PLAIN', 'Plain', 1200, 100, 2, False, [12, 10, 10], 5, 1239), ('PLAIN', 'Plain', 1500, 125, 2, False, [12, 5, 5, 5], 6, 1535), ('PLAIN', 'Plain', 1600, 100, 2, False, [16, 10, 10], 4, 1706), ('PLAIN', 'Plain', 1800, 150, 1, False, [12, 6, 5, 5], 6, 1828), ('PLAIN', 'Plain', 1920, 120, 2, False, [16, 12, 10], 4, 2047), ('PLAIN', 'Plain', 2000, 125, 2, False, [16, 5, 5, 5], 5, 2065), ('PLAIN', 'Plain', 2400, 150, 1, False, [16, 6, 5, 5], 5, 2474), ('PLAIN', 'Plain', 2500, 250, 1, False, [10, 10, 5, 5], 30, 2500), ('PLAIN', 'Plain', 3000, 250, 1, False, [12, 10, 5, 5], 6, 3046), ('PLAIN', 'Plain', 3200, 200, 1, False, [16, 8, 5, 5], 4, 3399), ('PLAIN', 'Plain', 3600, 360, 1, False, [10, 10, 6, 6], 30, 3600), ('PLAIN', 'Plain', 4000, 250, 1, False, [16, 10, 5, 5], 5, 4124), ('PLAIN', 'Plain', 4800, 480, 1, False, [10, 10, 8, 6], 6, 4874), ('PLAIN', 'Plain', 5000, 500, 1, False, [10, 10, 10, 5], 30, 5000), ('PLAIN', 'Plain', 6000, 600, 1, False, [10, 10, 10, 6], 30, 6000), ('PLAIN', 'Plain', 6400, 640, 1, False, [10, 10, 8, 8], 6, 6499), ('PLAIN', 'Plain', 7200, 720, 1, False, [10, 10, 9, 8], 30, 7200), ('PLAIN', 'Plain', 8000, 800, 1, False, [10, 10, 10, 8], 6, 8124), ('PLAIN', 'Plain', 9000, 900, 1, False, [10, 10, 10, 9], 30, 9000), ('PLAIN', 'Plain', 9600, 800, 1, False, [12, 10, 10, 8], 5, 9899), ('PLAIN', 'Plain', 12000, 1000, 1, False, [12, 10, 10, 10], 5, 12374), ('PLAIN', 'Plain', 16000, 1000, 1, False, [16, 10, 10, 10], 4, 16999)]
TABLES['kf_round_f64'] = [('PLAIN', 'Plain', 200, 25, 10, False, [8, 5, 5], 3, 225), ('PLAIN', 'Plain', 240, 30, 8, False, [8, 6, 5], 3, 273), ('PLAIN', 'Plain', 300, 25, 10, False, [12, 5, 5], 5, 314), ('PLAIN', 'Plain', 400, 25, 10, False, [16, 5, 5], 4, 426), ('PLAIN', 'Plain', 480, 48, 5, False, [10, 8, 6], 5, 494), ('PLAIN', 'Plain', 500, 50, 5, False, [10, 10, 5], 30, 506), ('PLAIN', 'Plain', 600, 60, 4, False, [10, 10, 6], 30, 604), ('PLAIN', 'Plain', 720, 72, 3, False, [10, 9, 8], 30, 720), ('PLAIN', 'Plain', 750, 125, 2, False, [6, 5, 5, 5], 30, 757), ('PLAIN', 'Plain', 800, 80, 3, False, [10, 10, 8], 30, 800), ('PLAIN', 'Plain', 900, 90, 2, False, [10, 10, 9], 30, 906), ('PLAIN', 'Plain', 960, 80, 3, False, [12, 10, 8], 5, 989), ('PLAIN', 'Plain', 1200, 100, 2, False, [12, 10, 10], 5, 1242), ('PLAIN', 'Plain', 1500, 125, 2, False, [12, 5, 5, 5], 5, 1552), ('PLAIN', 'Plain', 1600, 100, 2, False, [16, 10, 10], 4, 1706), ('PLAIN', 'Plain', 1800, 150, 1, False, [12, 6, 5, 5], 5, 1856), ('PLAIN', 'Plain', 1920, 120, 2, False, [16, 12, 10], 4, 2039), ('PLAIN', 'Plain', 2000, 125, 2, False, [16, 5, 5, 5], 4, 2125), ('PLAIN', 'Plain', 2400, 150, 1, False, [16, 6, 5, 5], 4, 2549), ('PLAIN', 'Plain', 2500, 250, 1, False, [10, 10, 5, 5], 30, 2500), ('PLAIN', 'Plain', 3000, 250, 1, False, [12, 10, 5, 5], 5, 3093), ('PLAIN', 'Plain', 3200, 200, 1, False, [16, 8, 5, 5], 4, 3399), ('PLAIN', 'Plain', 3600, 360, 1, False, [10, 10, 6, 6], 30, 3600), ('PLAIN', 'Plain', 4000, 250, 1, False, [16, 10, 5, 5], 4, 4249), ('PLAIN', 'Plain', 4800, 480, 1, False, [10, 10, 8, 6], 30, 4800), ('PLAIN', 'Plain', 5000, 500, 1, False, [10, 10, 10, 5], 30, 5000), ('PLAIN', 'Plain', 6000, 600, 1, False, [10, 10, 10, 6], 30, 6000), ('PLAIN', 'Plain', 6400, 640, 1, False, [10, 10, 8, 8], 30, 6400), ('PLAIN', 'Plain', 7200, 720, 1, False, [10, 10, 9, 8], 30, 7200), ('PLAIN', 'Plain', 8000, 800, 1, False, [10, 10, 10, 8], 30, 8000)]
# nd_rows(0 / 1, keys of the other tables and of kf_plain / kf_nd / kf_real /
# kf_blue): `python3 gen_shape_tables.py round` re-derives these lists too
TABLES['kf_round_nd_f32'] = [('PLAIN', 'Plain', 6, 1, 64, True, [6], 30, 7), ('PLAIN', 'Plain', 9, 1, 64, True, [9], 30, 9), ('PLAIN', 'Plain', 10, 1, 64, True, [10], 30, 11), ('PLAIN', 'Plain', 15, 3, 64, True, [5, 3], 30, 15), ('PLAIN', 'Plain', 18, 3, 64, True, [6, 3], 30, 19), ('PLAIN', 'Plain', 25, 5, 64, True, [5, 5], 30, 25), ('PLAIN', 'Plain', 27, 3, 64, True, [9, 3], 30, 27), ('PLAIN', 'Plain', 30, 5, 64, True, [6, 5], 30, 31), ('PLAIN', 'Plain', 36, 6, 64, True, [6, 6], 30, 37), ('PLAIN', 'Plain', 45, 5, 64, True, [9, 5], 30, 45), ('PLAIN', 'Plain', 50, 5, 64, True, [10, 5], 30, 51), ('PLAIN', 'Plain', 54, 6, 64, True, [9, 6], 30, 55), ('PLAIN', 'Plain', 60, 6, 64, True, [10, 6], 30, 61), ('PLAIN', 'Plain', 72, 8, 64, True, [9, 8], 30, 73), ('PLAIN', 'Plain', 75, 15, 64, True, [5, 5, 3], 30, 75), ('PLAIN', 'Plain', 81, 9, 64, True, [9, 9], 30, 81), ('PLAIN', 'Plain', 90, 9, 64, True, [10, 9], 30, 91), ('PLAIN', 'Plain', 108, 9, 64, True, [12, 9], 30, 109), ('PLAIN', 'Plain', 120, 10, 64, True, [12, 10], 30, 121), ('PLAIN', 'Plain', 125, 25, 32, True, [5, 5, 5], 30, 125), ('PLAIN', 'Plain', 135, 15, 64, True, [9, 5, 3], 30, 135), ('PLAIN', 'Plain', 144, 12, 64, True, [12, 12], 30, 145), ('PLAIN', 'Plain', 150, 25, 32, True, [6, 5, 5], 30, 151), ('PLAIN', 'Plain', 162, 18, 32, True, [9, 6, 3], 30, 163), ('PLAIN', 'Plain', 180, 30, 32, True, [6, 6, 5], 30, 181), ('PLAIN', 'Plain', 200, 25, 32, True, [8, 5, 5], 30, 201), ('PLAIN', 'Plain', 216, 36, 16, True, [6, 6, 6], 30, 217), ('PLAIN', 'Plain', 225, 25, 32, True, [9, 5, 5], 30, 225), ('PLAIN', 'Plain', 240, 30, 32, True, [8, 6, 5], 30, 241), ('PLAIN', 'Plain', 243, 27, 32, True, [9, 9, 3], 30, 243), ('PLAIN', 'Plain', 250, 25, 32, True, [10, 5, 5], 30, 251), ('PLAIN', 'Plain', 270, 30, 32, True, [9, 6, 5], 30, 271), ('PLAIN', 'Plain', 288, 36, 16, True, [8, 6, 6], 30, 289), ('PLAIN', 'Plain', 300, 25, 32, True, [12, 5, 5], 30, 301), ('PLAIN', 'Plain', 324, 36, 16, True, [9, 6, 6], 30, 325), ('PLAIN', 'Plain', 375, 75, 8, True, [5, 5, 5, 3], 30, 375), ('PLAIN', 'Plain', 400, 25, 16, True, [16, 5, 5], 30, 401), ('PLAIN', 'Plain', 405, 45, 16, True, [9, 9, 5], 30, 405), ('PLAIN', 'Plain', 432, 36, 16, True, [12, 6, 6], 30, 433), ('PLAIN', 'Plain', 450, 45, 16, True, [10, 9, 5], 30, 451), ('PLAIN', 'Plain', 480, 48, 16, True, [10, 8, 6], 30, 481), ('PLAIN', 'Plain', 486, 54, 16, True, [9, 9, 6], 30, 487), ('PLAIN', 'Plain', 500, 50, 16, True, [10, 10, 5], 30, 501), ('PLAIN', 'Plain', 540, 54, 16, True, [10, 9, 6], 30, 541), ('PLAIN', 'Plain', 576, 64, 16, True, [9, 8, 8], 30, 577), ('PLAIN', 'Plain', 600, 60, 16, True, [10, 10, 6], 30, 601), ('PLAIN', 'Plain', 625, 125, 8, True, [5, 5, 5, 5], 30, 625), ('FS_A', 'FsA', 27, 3, 64, True, [9, 3], 30, 27), ('FS_A', 'FsA', 30, 5, 64, True, [6, 5], 30, 31), ('FS_A', 'FsA', 36, 6, 64, True, [6, 6], 30, 37), ('FS_A', 'FsA', 40, 5, 64, True, [8, 5], 30, 41), ('FS_A', 'FsA', 45, 5, 64, True, [9, 5], 30, 45), ('FS_A', 'FsA', 48, 6, 64, True, [8, 6], 30, 49), ('FS_A', 'FsA', 50, 5, 64, True, [10, 5], 30, 51), ('FS_A', 'FsA', 54, 6, 64, True, [9, 6], 30, 55), ('FS_A', 'FsA', 60, 6, 64, True, [10, 6], 30, 61), ('FS_A', 'FsA', 72, 8, 64, True, [9, 8], 30, 73), ('FS_A', 'FsA', 75, 15, 64, True, [5, 5, 3], 30, 75), ('FS_A', 'FsA', 80, 8, 64, True, [10, 8], 30, 81), ('FS_A', 'FsA', 81, 9, 64, True, [9, 9], 30, 81), ('FS_A', 'FsA', 90, 9, 64, True, [10, 9], 30, 91), ('FS_A', 'FsA', 96, 8, 64, True, [12, 8], 30, 97), ('FS_A', 'FsA', 100, 10, 64, True, [10, 10], 30, 101), ('FS_A', 'FsA', 108, 9, 64, True, [12, 9], 30, 109), ('FS_A', 'FsA', 120, 10, 64, True, [12, 10], 30, 121), ('FS_A', 'FsA', 125, 25, 32, True, [5, 5, 5], 30, 125), ('FS_A', 'FsA', 135, 15, 64, True, [9, 5, 3], 30, 135), ('FS_A', 'FsA', 144, 12, 64, True, [12, 12], 30, 145), ('FS_A', 'FsA', 162, 18, 32, True, [9, 6, 3], 30, 163), ('PLAIN', 'PlainStaged', 6, 1, 64, False, [6], 3, 6), ('PLAIN', 'PlainStaged', 9, 1, 64, False, [9], 4, 9), ('PLAIN', 'PlainStaged', 10, 1, 64, False, [10], 4, 10), ('PLAIN', 'PlainStaged', 15, 3, 64, False, [5, 3], 4, 19), ('PLAIN', 'PlainStaged', 18, 3, 64, False, [6, 3], 5, 19), ('PLAIN', 'PlainStaged', 25, 5, 51, False, [5, 5], 5, 25), ('PLAIN', 'PlainStaged', 27, 3, 64, False, [9, 3], 5, 35), ('PLAIN', 'PlainStaged', 30, 5, 51, False, [6, 5], 5, 37), ('PLAIN', 'PlainStaged', 36, 6, 42, False, [6, 6], 6, 38), ('PLAIN', 'PlainStaged', 45, 5, 51, False, [9, 5], 6, 53), ('PLAIN', 'PlainStaged', 50, 5, 51, False, [10, 5], 6, 53), ('PLAIN', 'PlainStaged', 54, 6, 42, False, [9, 6], 6, 54), ('PLAIN', 'PlainStaged', 60, 6, 42, False, [10, 6], 6, 70), ('PLAIN', 'PlainStaged', 72, 8, 32, False, [9, 8], 30, 72), ('PLAIN', 'PlainStaged', 75, 15, 17, False, [5, 5, 3], 30, 79), ('PLAIN', 'PlainStaged', 81, 9, 28, False, [9, 9], 30, 89), ('PLAIN', 'PlainStaged', 90, 9, 28, False, [10, 9], 30, 105), ('PLAIN', 'PlainStaged', 108, 9, 28, False, [12, 9], 30, 121), ('PLAIN', 'PlainStaged', 120, 10, 25, False, [12, 10], 6, 122), ('PLAIN', 'PlainStaged', 125, 25, 10, False, [5, 5, 5], 30, 137), ('PLAIN', 'PlainStaged', 135, 15, 17, False, [9, 5, 3], 30, 143), ('PLAIN', 'PlainStaged', 144, 12, 21, False, [12, 12], 6, 156), ('PLAIN', 'PlainStaged', 150, 25, 10, False, [6, 5, 5], 30, 153), ('PLAIN', 'PlainStaged', 162, 18, 14, False, [9, 6, 3], 30, 162), ('PLAIN', 'PlainStaged', 180, 30, 8, False, [6, 6, 5], 30, 190)]
TABLES['kf_round_nd_f64'] = [('PLAIN', 'Plain', 6, 1, 64, True, [6], 30, 7), ('PLAIN', 'Plain', 9, 1, 64, True, [9], 30, 9), ('PLAIN', 'Plain', 10, 1, 64, True, [10], 30, 11), ('PLAIN', 'Plain', 15, 3, 64, True, [5, 3], 30, 15), ('PLAIN', 'Plain', 18, 3, 64, True, [6, 3], 30, 19), ('PLAIN', 'Plain', 25, 5, 64, True, [5, 5], 30, 25), ('PLAIN', 'Plain', 27, 3, 64, True, [9, 3], 30, 27), ('PLAIN', 'Plain', 30, 5, 64, True, [6, 5], 30, 31), ('PLAIN', 'Plain', 36, 6, 64, True, [6, 6], 30, 37), ('PLAIN', 'Plain', 45, 5, 64, True, [9, 5], 30, 45), ('PLAIN', 'Plain', 50, 5, 64, True, [10, 5], 30, 51), ('PLAIN', 'Plain', 54, 6, 64, True, [9, 6], 30, 55), ('PLAIN', 'Plain', 60, 6, 64, True, [10, 6], 30, 61), ('PLAIN', 'Plain', 72, 8, 64, True, [9, 8], 30, 73), ('PLAIN', 'Plain', 75, 15, 64, True, [5, 5, 3], 30, 75), ('PLAIN', 'Plain', 81, 9, 32, True, [9, 9], 30, 81), ('PLAIN', 'Plain', 90, 9, 32, True, [10, 9], 30, 91), ('PLAIN', 'Plain', 108, 9, 32, True, [12, 9], 30, 109), ('PLAIN', 'Plain', 120, 10, 32, True, [12, 10], 30, 121), ('PLAIN', 'Plain', 125, 25, 32, True, [5, 5, 5], 30, 125), ('PLAIN', 'Plain', 135, 15, 32, True, [9, 5, 3], 30, 135), ('PLAIN', 'Plain', 144, 12, 32, True, [12, 12], 30, 145), ('PLAIN', 'Plain', 150, 25, 32, True, [6, 5, 5], 30, 151), ('PLAIN', 'Plain', 162, 18, 16, True, [9, 6, 3], 30, 163), ('PLAIN', 'Plain', 180, 30, 16, True, [6, 6, 5], 30, 181), ('PLAIN', 'Plain', 200, 25, 16, True, [8, 5, 5], 30, 201), ('PLAIN', 'Plain', 216, 36, 16, True, [6, 6, 6], 30, 217), ('PLAIN', 'Plain', 225, 25, 16, True, [9, 5, 5], 30, 225), ('PLAIN', 'Plain', 240, 30, 16, True, [8, 6, 5], 30, 241), ('PLAIN', 'Plain', 243, 27, 16, True, [9, 9, 3], 30, 243), ('PLAIN', 'Plain', 250, 25, 16, True, [10, 5, 5], 30, 251), ('PLAIN', 'Plain', 270, 30, 16, True, [9, 6, 5], 30, 271), ('PLAIN', 'Plain', 288, 36, 16, True, [8, 6, 6], 30, 289), ('PLAIN', 'Plain', 300, 25, 16, True, [12, 5, 5], 30, 301), ('PLAIN', 'Plain', 324, 36, 8, True, [9, 6, 6], 30, 325), ('PLAIN', 'Plain', 375, 75, 8, True, [5, 5, 5, 3], 30, 375), ('PLAIN', 'Plain', 400, 25, 8, True, [16, 5, 5], 30, 401), ('PLAIN', 'Plain', 405, 45, 8, True, [9, 9, 5], 30, 405), ('PLAIN', 'Plain', 432, 36, 8, True, [12, 6, 6], 30, 433), ('PLAIN', 'Plain', 450, 45, 8, True, [10, 9, 5], 30, 451), ('PLAIN', 'Plain', 480, 48, 8, True, [10, 8, 6], 30, 481), ('PLAIN', 'Plain', 486, 54, 8, True, [9, 9, 6], 30, 487), ('PLAIN', 'Plain', 500, 50, 8, True, [10, 10, 5], 30, 501), ('PLAIN', 'Plain', 540, 54, 8, True, [10, 9, 6], 30, 541), ('PLAIN', 'Plain', 576, 64, 8, True, [9, 8, 8], 30, 577), ('PLAIN', 'Plain', 600, 60, 8, True, [10, 10, 6], 30, 601), ('PLAIN', 'Plain', 625, 125, 8, True, [5, 5, 5, 5], 30, 625), ('FS_A', 'FsA', 27, 3, 64, True, [9, 3], 30, 27), ('FS_A', 'FsA', 30, 5, 64, True, [6, 5], 30, 31), ('FS_A', 'FsA', 36, 6, 64, True, [6, 6], 30, 37), ('FS_A', 'FsA', 40, 5, 64, True, [8, 5], 30, 41), ('FS_A', 'FsA', 45, 5, 64, True, [9, 5], 30, 45), ('FS_A', 'FsA', 48, 6, 64, True, [8, 6], 30, 49), ('FS_A', 'FsA', 50, 5, 64, True, [10, 5], 30, 51), ('FS_A', 'FsA', 54, 6, 64, True, [9, 6], 30, 55), ('FS_A', 'FsA', 60, 6, 64, True, [10, 6], 30, 61), ('FS_A', 'FsA', 72, 8, 64, True, [9, 8], 30, 73), ('FS_A', 'FsA', 75, 15, 64, True, [5, 5, 3], 30, 75), ('FS_A', 'FsA', 80, 8, 32, True, [10, 8], 30, 81), ('FS_A', 'FsA', 81, 9, 32, True, [9, 9], 30, 81), ('FS_A', 'FsA', 90, 9, 32, True, [10, 9], 30, 91), ('FS_A', 'FsA', 96, 8, 32, True, [12, 8], 30, 97), ('FS_A', 'FsA', 100, 10, 32, True, [10, 10], 30, 101), ('FS_A', 'FsA', 108, 9, 32, True, [12, 9], 30, 109), ('FS_A', 'FsA', 120, 10, 32, True, [12, 10], 30, 121), ('FS_A', 'FsA', 125, 25, 32, True, [5, 5, 5], 30, 125), ('FS_A', 'FsA', 135, 15, 32, True, [9, 5, 3], 30, 135), ('FS_A', 'FsA', 144, 12, 32, True, [12, 12], 30, 145), ('FS_A', 'FsA', 162, 18, 16, True, [9, 6, 3], 30, 163), ('PLAIN', 'PlainStaged', 6, 1, 64, False, [6], 3, 6), ('PLAIN', 'PlainStaged', 9, 1, 64, False, [9], 4, 9), ('PLAIN', 'PlainStaged', 10, 1, 64, False, [10], 3, 11), ('PLAIN', 'PlainStaged', 15, 3, 64, False, [5, 3], 4, 19), ('PLAIN', 'PlainStaged', 18, 3, 64, False, [6, 3], 5, 19), ('PLAIN', 'PlainStaged', 25, 5, 51, False, [5, 5], 5, 29), ('PLAIN', 'PlainStaged', 27, 3, 64, False, [9, 3], 5, 27), ('PLAIN', 'PlainStaged', 30, 5, 51, False, [6, 5], 5, 37), ('PLAIN', 'PlainStaged', 36, 6, 42, False, [6, 6], 6, 38), ('PLAIN', 'PlainStaged', 45, 5, 51, False, [9, 5], 6, 45), ('PLAIN', 'PlainStaged', 50, 5, 51, False, [10, 5], 6, 53), ('PLAIN', 'PlainStaged', 54, 6, 42, False, [9, 6], 6, 54), ('PLAIN', 'PlainStaged', 60, 6, 42, False, [10, 6], 5, 62), ('PLAIN', 'PlainStaged', 72, 8, 32, False, [9, 8], 30, 72), ('PLAIN', 'PlainStaged', 75, 15, 17, False, [5, 5, 3], 30, 79), ('PLAIN', 'PlainStaged', 81, 9, 28, False, [9, 9], 30, 81), ('PLAIN', 'PlainStaged', 90, 9, 28, False, [10, 9], 30, 97), ('PLAIN', 'PlainStaged', 108, 9, 28, False, [12, 9], 5, 113), ('PLAIN', 'PlainStaged', 120, 10, 25, False, [12, 10], 6, 122), ('PLAIN', 'PlainStaged', 125, 25, 10, False, [5, 5, 5], 30, 129), ('PLAIN', 'PlainStaged', 135, 15, 17, False, [9, 5, 3], 30, 135), ('PLAIN', 'PlainStaged', 144, 12, 21, False, [12, 12], 5, 148), ('PLAIN', 'PlainStaged', 150, 25, 10, False, [6, 5, 5], 30, 153), ('PLAIN', 'PlainStaged', 162, 18, 14, False, [9, 6, 3], 30, 162), ('PLAIN', 'PlainStaged', 180, 30, 8, False, [6, 6, 5], 30, 182)]
HEADS_ROUND_ND = ("// Fixed shapes for the N-D passes of lengths with factors 2, 3 and 5\n"
                  "// outside the power-of-two, 3*2^k and 5*2^k families, {p}: strided columns up\n"
                  "// to 640 (the longest strided axis of one pass), the first pass of a split\n"
                  "// strided axis (FS_A columns of its larger factor) and short rows staged\n"
                  "// through LDS. Columns: threads per line = N / the largest radix, the largest\n"
                  "// power-of-two lines per block up to 64 within 80 KiB and 1024 threads, an odd\n"
                  "// LDS stride; rows: about 256 threads per block, LDS stride from the bank model.\n")
# Even-length real rows whose half length has a round-length or 10^k / 360 C2C
# row shape: the same radices, threads, lines per block and LDS strides.
def round_real_rows(prec):
    fam = 'kf_fam_f64' if prec else 'kf_fam_f32'
    src = list(TABLES['kf_round_f64' if prec else 'kf_round_f32'])
    src += [it for it in TABLES[fam] if not isinstance(it, str) and it[0] == 'PLAIN' and not it[5] and
            it[1] == 'Plain' and it[2] in (100, 360, 1000, 10000)]
    rows = []
    for kind, io, N, TT, G, col, rad, PS, LS in sorted(src, key=lambda r: r[2]):
        rows.append(('R2C_HALF', 'R2CHalf', N, TT, G, False, rad, PS, LS))
        rows.append(('C2R_HALF', 'C2RHalf', N, TT, G, False, rad, PS, LS))
    return rows


TABLES['kf_round_real_f32'] = round_real_rows(0)
TABLES['kf_round_real_f64'] = round_real_rows(1)
HEADS_ROUND_REAL = ("// Fixed shapes of the one-upload even-length real transforms whose half\n"
                    "// length M has a round-length (kf_round_{p}) or 10^k / 360 C2C row shape, {p}:\n"
                    "// the half-size packed FFT of R2C (postprocess fused into the staged store)\n"
                    "// and of C2R (preprocess fused into the direct loads), with the same radices,\n"
                    "// threads, lines per block and LDS strides as those rows. R2C is registered\n"
                    "// for the caller's input with or without the caller's output, C2R for the\n"
                    "// caller's output with or without the caller's input.\n")
TABLES['kf_blue_rows_f32'] = blue_rows(0)
TABLES['kf_blue_rows_f64'] = blue_rows(1)
HEADS_BLUE = ("// Fixed shapes of the one-kernel Bluestein transform, {p}, for the planner's\n"
              "// most frequent convolution lengths M (the padded lengths of the primes up\n"
              "// to 8200 that run as Bluestein), streamed input and output. The kernel\n"
              "// always runs its forward FFT first; the transform direction lives in the\n"
              "// chirp and kernel-spectrum tables, so one entry serves both directions.\n"
              "// Radix plans with the fewest stages from radices 2-16; threads per\n"
              "// line = M / the largest radix; about 256 threads per block; one LDS pad\n"
              "// slot per 16 (f32) / 8 (f64) elements.\n")
HEADS['kf_blue_rows_f32'] = HEADS_BLUE.format(p='f32')
HEADS['kf_blue_rows_f64'] = HEADS_BLUE.format(p='f64')
# the same shapes with the 1-D boundary work inside (storage conversion and
# zero intervals), found by kind_variant from the plain entry
TABLES['kf_blue_edge_f32'] = [('BLUE_1_EDGE', 'Blue1Edge') + r[2:] for r in blue_rows(0)]
TABLES['kf_blue_edge_f64'] = [('BLUE_1_EDGE', 'Blue1Edge') + r[2:] for r in blue_rows(1)]
HEADS_BLUE_EDGE = ("// Fixed shapes of the one-kernel Bluestein transform with the 1-D boundary\n"
                   "// work inside, {p}: the caller's input and output in the storage type of\n"
                   "// half the compute precision and the zero intervals of zero padding\n"
                   "// (IoBlue1Edge), one entry for each shape of kf_blue_rows_{p} with the same\n"
                   "// threads, lines per block, radices and LDS strides.\n")
HEADS['kf_blue_edge_f32'] = HEADS_BLUE_EDGE.format(p='f32')
HEADS['kf_blue_edge_f64'] = HEADS_BLUE_EDGE.format(p='f64')
# the real rows with the 1-D boundary work inside, one nontemporal role each
TABLES['kf_real_edge_f32'] = [(r[0] + '_EDGE', r[1] + 'Edge') + r[2:] for r in TABLES['kf_real_rows_f32']]
TABLES['kf_real_edge_f64'] = [(r[0] + '_EDGE', r[1] + 'Edge') + r[2:] for r in TABLES['kf_real_rows_f64']]
HEADS_REAL_EDGE = ("// Fixed shapes of the one-upload even-length real transforms with the 1-D\n"
                   "// boundary work inside, {p}: the caller's buffers in the storage type of\n"
                   "// half the compute precision and the zero interval of the real side\n"
                   "// (IoR2CHalfEdge, IoC2RHalfEdge), one entry for each shape of\n"
                   "// kf_real_rows_{p} with the same threads, lines per block, radices and LDS\n"
                   "// strides.\n")
HEADS['kf_real_edge_f32'] = HEADS_REAL_EDGE.format(p='f32')
HEADS['kf_real_edge_f64'] = HEADS_REAL_EDGE.format(p='f64')
# the one-upload rows with the 1-D boundary work inside, where they beat the
# runtime-shape edge kernels (2048-16384 lines, one box): the 3/5-family rows
# in both precisions (F16 storage 1000: 31.9 against 46.8 us, 1536: 28.6
# against 34.5; F64 compute 1000: 18.6 against 48.2) and the f64 power-of-two
# rows (512: 15.4 against 29.5 us, 2048: 16.5 against 27.9); f32 power-of-two
# rows (256: 30.1 against 23.5 us, 1024: 34.9 against 30.5) and short rows with
# staged ends (96: 49.7 against 36.9 us) keep the runtime-shape edge kernels
PLAIN_CFG_ROWS = {0: [], 1: [('PLAIN', 'Plain', 512, 64, 2, False, [8, 8, 8], 3, 576)]}


def plain_edge_rows(prec):
    p = 'f64' if prec else 'f32'
    tables = ('kf_pow2_f64', 'kf_fam_f64') if prec else ('kf_fam_f32',)
    rows = PLAIN_CFG_ROWS[prec] + [r for t in tables for r in TABLES[t]
                                   if not isinstance(r, str) and r[0] == 'PLAIN' and not r[5] and r[1] == 'Plain']
    return [('PLAIN_EDGE', r[1] + 'Edge') + r[2:] for r in rows]


# the first pass (rows, storage-type input) and the last pass (columns,
# storage-type output) of mixed-storage N-D chunks: every row and column shape
# of the benchmark lengths, kf_pow2_* and kf_fam_* (staged rows excepted)
ND_CFG = {0: [('PLAIN', 'Plain', 1024, 128, 1, False, [16, 8, 8], 4, 1088),
              ('PLAIN', 'Plain', 4096, 256, 1, False, [16, 16, 16], 4, 4352),
              ('PLAIN', 'Plain', 64, 8, 32, True, [8, 8], 30, 65)],
          1: [('PLAIN', 'Plain', 512, 64, 2, False, [8, 8, 8], 3, 576),
              ('PLAIN', 'Plain', 512, 64, 16, True, [8, 8, 8], 30, 513)]}


def nd_edge_rows(prec):
    p = 'f64' if prec else 'f32'
    rows = ND_CFG[prec] + [r for t in ('kf_pow2_' + p, 'kf_fam_' + p) for r in TABLES[t]
                           if not isinstance(r, str) and r[0] == 'PLAIN' and r[1] == 'Plain']
    return [(('PLAIN_EDGE_OUT', 'PlainEdgeOut') if r[5] else ('PLAIN_EDGE_IN', 'PlainEdgeIn')) + r[2:] for r in rows]


TABLES['kf_nd_edge_f32'] = nd_edge_rows(0)
TABLES['kf_nd_edge_f64'] = nd_edge_rows(1)
HEADS_ND_EDGE = ("// Fixed shapes of the first and last passes of mixed-storage N-D chunks,\n"
                 "// {p}: rows reading the caller's storage type of half the compute precision\n"
                 "// (IoPlainEdgeIn) and columns writing it (IoPlainEdgeOut), the middle\n"
                 "// passes running on a compute-type stage; one entry per direction for each\n"
                 "// row and column shape of the benchmark lengths, kf_pow2_{p} and kf_fam_{p},\n"
                 "// with the same threads, lines per block, radices and LDS strides.\n")
HEADS['kf_nd_edge_f32'] = HEADS_ND_EDGE.format(p='f32')
HEADS['kf_nd_edge_f64'] = HEADS_ND_EDGE.format(p='f64')
TABLES['kf_plain_edge_f32'] = plain_edge_rows(0)
TABLES['kf_plain_edge_f64'] = plain_edge_rows(1)
HEADS_PLAIN_EDGE = ("// Fixed one-upload C2C row shapes with the 1-D boundary work inside, {p}:\n"
                    "// the caller's input and output in the storage type of half the compute\n"
                    "// precision and the zero intervals of zero padding (IoPlainEdge), one\n"
                    "// entry per direction for the row shapes where the fixed shape beats the\n"
                    "// runtime-shape edge kernel (the 3/5-family rows; in f64 also the\n"
                    "// power-of-two rows and the 512-point benchmark row), with the same\n"
                    "// threads, lines per block, radices and LDS strides.\n")
HEADS['kf_plain_edge_f32'] = HEADS_PLAIN_EDGE.format(p='f32')
HEADS['kf_plain_edge_f64'] = HEADS_PLAIN_EDGE.format(p='f64')
# fourstep_rows(0 / 1, registered_keys(0 / 1)) before these tables existed
TABLES['kf_round_fs_f32'] = [('FS_B', 'FsB', 128, 8, 16, False, [16, 8], 4, 137), ('FS_A', 'FsA', 240, 30, 32, True, [8, 6, 5], 30, 241), ('FS_B', 'FsB', 240, 30, 16, False, [8, 6, 5], 4, 255), ('FS_A', 'FsA', 250, 25, 32, True, [10, 5, 5], 30, 251), ('FS_B', 'FsB', 250, 25, 16, False, [10, 5, 5], 4, 265), ('FS_A', 'FsA', 256, 16, 32, True, [16, 16], 30, 257), ('FS_B', 'FsB', 256, 16, 16, False, [16, 16], 4, 273), ('FS_A', 'FsA', 400, 25, 32, True, [16, 5, 5], 30, 401), ('FS_B', 'FsB', 400, 25, 16, False, [16, 5, 5], 4, 425), ('FS_A', 'FsA', 500, 50, 16, True, [10, 10, 5], 30, 501), ('FS_B', 'FsB', 500, 50, 16, False, [10, 10, 5], 4, 531), ('FS_A', 'FsA', 512, 64, 16, True, [8, 8, 8], 30, 513), ('FS_B', 'FsB', 512, 64, 16, False, [8, 8, 8], 4, 545), ('FS_A', 'FsA', 1000, 100, 8, True, [10, 10, 10], 30, 1001), ('FS_B', 'FsB', 1000, 100, 8, False, [10, 10, 10], 4, 1063), ('FS_A', 'FsA', 1024, 64, 16, True, [16, 8, 8], 30, 1025), ('FS_A', 'FsA', 2000, 125, 8, True, [16, 5, 5, 5], 30, 2001), ('FS_B', 'FsB', 2000, 125, 8, False, [16, 5, 5, 5], 4, 2125), ('FS_A', 'FsA', 2048, 128, 8, True, [16, 16, 8], 30, 2049), ('FS_B', 'FsB', 2048, 128, 8, False, [16, 16, 8], 4, 2177)]
TABLES['kf_round_fs_f64'] = [('FS_B', 'FsB', 128, 8, 16, False, [16, 8], 3, 145), ('FS_A', 'FsA', 240, 30, 32, True, [8, 6, 5], 30, 241), ('FS_B', 'FsB', 240, 30, 16, False, [8, 6, 5], 3, 271), ('FS_A', 'FsA', 250, 25, 32, True, [10, 5, 5], 30, 251), ('FS_B', 'FsB', 250, 25, 16, False, [10, 5, 5], 3, 281), ('FS_A', 'FsA', 256, 16, 32, True, [16, 16], 30, 257), ('FS_B', 'FsB', 256, 16, 16, False, [16, 16], 3, 289), ('FS_A', 'FsA', 400, 25, 16, True, [16, 5, 5], 30, 401), ('FS_B', 'FsB', 400, 25, 16, False, [16, 5, 5], 3, 451), ('FS_A', 'FsA', 500, 50, 16, True, [10, 10, 5], 30, 501), ('FS_B', 'FsB', 500, 50, 16, False, [10, 10, 5], 3, 563), ('FS_A', 'FsA', 512, 64, 16, True, [8, 8, 8], 30, 513), ('FS_B', 'FsB', 512, 64, 16, False, [8, 8, 8], 3, 577), ('FS_A', 'FsA', 1000, 100, 8, True, [10, 10, 10], 30, 1001), ('FS_B', 'FsB', 1000, 100, 8, False, [10, 10, 10], 3, 1125), ('FS_A', 'FsA', 1024, 64, 8, True, [16, 8, 8], 30, 1025), ('FS_B', 'FsB', 1024, 64, 8, False, [16, 8, 8], 3, 1153), ('FS_A', 'FsA', 2000, 125, 4, True, [16, 5, 5, 5], 30, 2001), ('FS_B', 'FsB', 2000, 125, 4, False, [16, 5, 5, 5], 3, 2251), ('FS_A', 'FsA', 2048, 128, 4, True, [16, 16, 8], 30, 2049), ('FS_B', 'FsB', 2048, 128, 4, False, [16, 16, 8], 3, 2305)]
HEADS_ROUND_FS = ("// Fixed shapes of the two-upload four-step passes, {p}: FS_A column passes\n"
                  "// (FFT over N1 + the W_M twiddle) and FS_B row passes (FFT over N2 + the\n"
                  "// transposed store) for the factors four_step_split picks for common lengths\n"
                  "// (powers of two and round ones: 2^16, 60000, 10^5, 250000, 10^6, 2^22,\n"
                  "// 4*10^6, ...), both directions. Threads per line = N / the largest radix;\n"
                  "// columns: up to 32 per block within 150 KiB, odd LDS stride; rows: up to 16\n"
                  "// per block (128-byte transposed stores), the rows' pad rule.\n")
HEADS['kf_round_fs_f32'] = HEADS_ROUND_FS.format(p='f32')
HEADS['kf_round_fs_f64'] = HEADS_ROUND_FS.format(p='f64')
HEADS['kf_round_real_f32'] = HEADS_ROUND_REAL.format(p='f32')
HEADS['kf_round_real_f64'] = HEADS_ROUND_REAL.format(p='f64')
HEADS['kf_round_nd_f32'] = HEADS_ROUND_ND.format(p='f32')
HEADS['kf_round_nd_f64'] = HEADS_ROUND_ND.format(p='f64')
HEADS['kf_round_f32'] = HEADS_ROUND.format(p='f32')
HEADS['kf_round_f64'] = HEADS_ROUND.format(p='f64')

FUNCS = {'kf_blue_rows_f32': 'fixed_table_blue_rows_f32', 'kf_blue_rows_f64': 'fixed_table_blue_rows_f64',
         'kf_blue_edge_f32': 'fixed_table_blue_edge_f32', 'kf_blue_edge_f64': 'fixed_table_blue_edge_f64',
         'kf_real_edge_f32': 'fixed_table_real_edge_f32', 'kf_real_edge_f64': 'fixed_table_real_edge_f64',
         'kf_plain_edge_f32': 'fixed_table_plain_edge_f32', 'kf_plain_edge_f64': 'fixed_table_plain_edge_f64',
         'kf_nd_edge_f32': 'fixed_table_nd_edge_f32', 'kf_nd_edge_f64': 'fixed_table_nd_edge_f64',
         'kf_round_fs_f32': 'fixed_table_round_fs_f32', 'kf_round_fs_f64': 'fixed_table_round_fs_f64',
         'kf_round_real_f32': 'fixed_table_round_real_f32', 'kf_round_real_f64': 'fixed_table_round_real_f64',
         'kf_round_nd_f32': 'fixed_table_round_nd_f32', 'kf_round_nd_f64': 'fixed_table_round_nd_f64',
         'kf_round_f32': 'fixed_table_round_f32', 'kf_round_f64': 'fixed_table_round_f64', 'kf_pow2_f32': 'fixed_table_pow2_f32', 'kf_pow2_f64': 'fixed_table_pow2_f64', 'kf_fam_f32': 'fixed_table_fam_f32', 'kf_fam_f64': 'fixed_table_fam_f64', 'kf_real_rows_f32': 'fixed_table_real_rows_f32', 'kf_real_rows_f64': 'fixed_table_real_rows_f64'}


def roles(kind, col):
    """(direction, nontemporal input, nontemporal output) registered."""
    if kind in ("BLUE_1", "BLUE_1_EDGE"):
        return [(-1, True, True)]
    if kind in ("FS_A", "FS_B"):
        return [(-1, False, False), (1, False, False)]
    if kind == "R2C_HALF":
        return [(-1, True, True), (-1, True, False)]
    if kind == "C2R_HALF":
        return [(1, True, True), (1, False, True)]
    if kind == "R2C_HALF_EDGE":
        return [(-1, True, True)]
    if kind == "C2R_HALF_EDGE":
        return [(1, True, True)]
    if kind == "PLAIN_EDGE":
        return [(-1, True, True), (1, True, True)]
    if kind == "PLAIN_EDGE_IN":
        return [(-1, True, False), (1, True, False)]
    if kind == "PLAIN_EDGE_OUT":
        return [(-1, False, True), (1, False, True)]
    if col:
        return [(-1, False, False), (-1, False, True), (1, False, False), (1, False, True)]
    return [(-1, True, True), (-1, True, False), (1, True, True), (1, True, False)]


def b(v):
    return "true" if v else "false"


def render(name):
    """Text of table file `name`.hip."""
    prec = 1 if name.endswith("f64") else 0
    T = "double" if prec else "float"
    lines = [HEADS[name].rstrip("\n"),
             "//",
             "// Generated by gen_shape_tables.py (shape lists and LDS bank-conflict",
             "// model); edit the lists there and run `python3 gen_shape_tables.py emit`.",
             '#include "fft_kernels_impl.hpp"', "", "namespace vkfx {", "", "static const FixedKernel kTable[] = {"]
    for it in TABLES[name]:
        if isinstance(it, str):
            lines.append("    " + it)
            continue
        kind, io, N, TT, G, col, rad, PS, LS = it
        for S, nti, nto in roles(kind, col):
            lines.append(f"    VKFX_SHAPE(KK_{kind}, Io{io}, {T}, {prec}, {S}, {N}, {TT}, {G}, {PS}, {LS}, {b(col)}, "
                         f"{b(nti)}, {b(nto)}, {', '.join(map(str, rad))}),")
    lines += ["};", "", f"const FixedKernel* {FUNCS[name]}(int* count) {{",
              "    *count = (int)(sizeof(kTable) / sizeof(kTable[0]));", "    return kTable;", "}", "",
              "}  // namespace vkfx", ""]
    return "\n".join(lines)


def emit(name):
    with open(os.path.join(HERE, name + ".hip"), "w") as f:
        f.write(render(name))


def check():
    for name, items in TABLES.items():
        eb = 16 if name.endswith("f64") else 8
        for it in items:
            if isinstance(it, str) or it[0] in ("R2C_HALF", "C2R_HALF", "R2C_HALF_EDGE", "C2R_HALF_EDGE"):
                continue
            kind, io, N, TT, G, col, rad, PS, LS = it
            staged = io == "PlainStaged"
            cur = score(N, TT, G, PS, LS, col, rad, staged, eb)
            best = search(N, TT, G, col, rad, staged, eb)
            print(f"{name} {kind} N={N} {'col' if col else 'row'} TT={TT} G={G}: PS={PS} LS={LS} "
                  f"ratio {cur:.3f}; model best {best}", flush=True)


if __name__ == "__main__":
    if len(sys.argv) > 1 and sys.argv[1] == "emit":
        for n in (sys.argv[2:] or TABLES):
            emit(n)
    elif len(sys.argv) > 1 and sys.argv[1] == "check":
        check()
    elif len(sys.argv) > 1 and sys.argv[1] == "round":
        for prec, name in ((0, "kf_round_f32"), (1, "kf_round_f64")):
            rows = round_rows(prec)
            print(name, "matches" if rows == TABLES[name] else "DIFFERS", rows, flush=True)
        import re
        for prec, name in ((0, "kf_round_nd_f32"), (1, "kf_round_nd_f64")):
            have = set()
            for other, items in TABLES.items():
                if other.startswith("kf_round_nd") or other.endswith("f64") != bool(prec):
                    continue
                have |= {(it[0], it[2], it[5]) for it in items if not isinstance(it, str)}
            for f in ("kf_plain.hip", "kf_nd.hip", "kf_real.hip", "kf_blue.hip"):
                pat = r"KK_(\w+), Io\w+, (float|double), (\d), -?\d, (\d+), \d+, \d+, \d+, \d+, (true|false)"
                for m in re.finditer(pat, open(os.path.join(HERE, f)).read()):
                    if int(m.group(3)) == prec:
                        have.add((m.group(1), int(m.group(4)), m.group(5) == "true"))
            rows = nd_rows(prec, have)
            print(name, "matches" if rows == TABLES[name] else "DIFFERS", rows, flush=True)
        for prec, name in ((0, "kf_round_fs_f32"), (1, "kf_round_fs_f64")):
            rows = fourstep_rows(prec, registered_keys(prec, skip=(name,)))
            print(name, "matches" if rows == TABLES[name] else "DIFFERS", rows, flush=True)
    else:
        print(__doc__)
