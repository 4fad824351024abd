"""The committed fixed-shape tables are exactly what the shape-table
generator (vkfft-rs_amd/csrc/gen_shape_tables.py) emits, and each recorded
LDS stride scores as well as the generator's bank-conflict model search."""
import importlib.util
import os

import pytest

CSRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "vkfft-rs_amd", "csrc")


def _gen():
    spec = importlib.util.spec_from_file_location("gen_shape_tables", os.path.join(CSRC, "gen_shape_tables.py"))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


@pytest.mark.parametrize("name", ["kf_pow2_f32", "kf_pow2_f64", "kf_fam_f32", "kf_fam_f64", "kf_real_rows_f32",
                                  "kf_real_rows_f64", "kf_round_f32", "kf_round_f64", "kf_round_nd_f32",
                                  "kf_round_nd_f64", "kf_round_real_f32", "kf_round_real_f64",
                                  "kf_round_fs_f32", "kf_round_fs_f64", "kf_blue_rows_f32", "kf_blue_rows_f64"])
def test_tables_match_generator(name):
    g = _gen()
    assert open(os.path.join(CSRC, name + ".hip")).read() == g.render(name)


def test_round_rows_follow_the_rule():
    """The round-length rows' radix plans, threads and lines per block are the
    rule's (the LDS stride search is the slow part and is left to
    `gen_shape_tables.py round`)."""
    g = _gen()
    for prec, name in ((0, "kf_round_f32"), (1, "kf_round_f64")):
        eb = 16 if prec else 8
        for kind, io, N, TT, G, col, rad, PS, LS in g.TABLES[name]:
            assert rad == g.radix_plan(N) and int(__import__("math").prod(rad)) == N, (name, N)
            assert TT == N // max(rad) and 1 <= TT <= 1024, (name, N)
            assert G * TT <= 1024 and G * LS * eb <= (80 * 1024 if G > 1 else 156 * 1024), (name, N)
            assert LS >= N + ((N - 1) >> PS if PS < 30 else 0), (name, N)
    for prec, name in ((0, "kf_round_nd_f32"), (1, "kf_round_nd_f64")):
        eb = 16 if prec else 8
        for kind, io, N, TT, G, col, rad, PS, LS in g.TABLES[name]:
            assert rad == g.radix_plan(N) and TT == N // max(rad), (name, N)
            assert G * TT <= 1024 and G * LS * eb <= 80 * 1024, (name, N)
            if col:
                assert PS == 30 and LS % 2 == 1 and LS >= N and (G == 64 or 2 * G * TT > 1024 or
                                                                 2 * G * LS * eb > 80 * 1024), (name, N)
            else:
                assert io == "PlainStaged" and G == max(1, min(64, 256 // TT)), (name, N)


def test_recorded_strides_are_model_optimal_for_small_shapes():
    g = _gen()
    checked = 0
    for name, items in g.TABLES.items():
        if not name.startswith("kf_pow2"):
            continue
        eb = 16 if name.endswith("f64") else 8
        for it in items:
            if isinstance(it, str) or it[0] in ("R2C_HALF", "C2R_HALF"):
                continue
            kind, io, N, TT, G, col, rad, PS, LS = it
            if N > 64:
                continue  # the search over large lines takes minutes
            cur = g.score(N, TT, G, PS, LS, col, rad, io == "PlainStaged", eb)
            best = g.search(N, TT, G, col, rad, io == "PlainStaged", eb)
            assert round(cur, 3) <= best[0] + 1e-9, (name, it, best)
            checked += 1
    assert checked >= 8
