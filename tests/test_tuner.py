"""The gfx950 tuner (amdgpu-arch-gemm_amd/tuner/sgemm_tuner.py), without a GPU.

The reference tuner (tuner/sgemm_tuner.py:41-128) enumerates knobs, compiles
each point, runs the runner and prints the best; this one adds a gfx950 space,
JSONL resume, per-point isolation and re-emission of the winner.  These tests
drive its pieces with a fake benchmark so no GPU is needed.
"""
import json
import os
from itertools import product

import pytest

from generator import generator as g
from tuner import sgemm_tuner as T


def test_gfx950_stage1_space():
    """Macro-tile {64,128,256}^2 x wave group {2x2, 4x1} x atom {32x32x2,
    16x16x4}: every combination the generator accepts, and nothing else."""
    pts = list(T.geometry_points(T.DEFAULT_KNOBS))
    got = sorted((c.tile_size, c.wave_group, c.mfma) for c, _ in pts)
    want = []
    for (mt0, mt1), wg, mfma in product([(a, b) for a in (64, 128, 256) for b in (64, 128, 256)],
                                        [(2, 2), (4, 1)], [(16, 16, 1, 4), (32, 32, 1, 2)]):
        if mt0 % (mfma[0] * wg[0]) or mt1 % (mfma[1] * wg[1]):
            continue
        wt = (mt0 // (mfma[0] * wg[0]), mt1 // (mfma[1] * wg[1]))
        try:
            g.GemmSolutionConfig(g.DataType.FP32, g.DataType.FP32, g.DataType.FP32, g.DataType.FP32, mfma, wg, wt,
                                 16, False, False, vmem_stage=2)
        except RuntimeError:
            continue
        want.append(((mt0, mt1), wg, mfma))
    assert got == sorted(want)
    # the expressible part of the reference's own sweep of this space (33 points) minus what
    # gfx950's limits reject (wave tiling above 8, LDS above 160 KiB)
    assert 24 <= len(got) <= 33
    assert ((256, 256), (2, 2), (32, 32, 1, 2)) in got   # the headline geometry


def test_stage1_tries_each_geometry_at_each_occupancy():
    """With occs (0, 2) every geometry is a stage-1 candidate twice, so that
    one that only pays with two work-groups per CU (the 4096^3 winner,
    256 x 128) can reach stage 2; the CLI searches both by default."""
    one = [T.point_key(*p) for p in T.geometry_points(T.DEFAULT_KNOBS)]
    two = [T.point_key(*p) for p in T.geometry_points(T.DEFAULT_KNOBS, occs=(0, 2))]
    assert set(one) < set(two)
    assert sorted(k for k in two if not k.endswith("_occ2")) == sorted(one)
    assert "a32_wg2x2_wt4x2_dk16_s2_wgm4_plr3_gw1_mk0_x8_occ2" in two
    # and at each stage-1 depth: the 16x16x4 geometries need depth 32 to rank
    deep = [T.point_key(*p) for p in T.geometry_points(T.DEFAULT_KNOBS, depths=T.STAGE1_DEPTHS)]
    assert "a16_wg2x2_wt4x2_dk32_s2_wgm4_plr3_gw1_mk0_x8" in deep and set(one) < set(deep)



def test_fits_skips_only_tiles_larger_than_the_problem():
    cfg, _ = T.make_point((32, 32, 1, 2), (2, 2), (4, 4), 16, 2, 4, 3, 0, 0, 8)
    assert T.fits(cfg, 256, 256, 16)
    assert T.fits(cfg, 1000, 999, 1001)       # edge tiles are masked in the kernel
    assert not T.fits(cfg, 255, 4096, 4096)   # the tile is larger than the problem
    # 32 x 32 tile, 256 work-items, DK 16: 32*16*4 / 256 = 8 bytes of A per work-item, under the
    # reference's one-16-byte-load filter (sgemm_tuner.py:102-105)
    small, _ = T.make_point((16, 16, 1, 4), (2, 2), (1, 1), 16, 1, 1, 1, 0, 0, 0)
    assert small.num_bytes_per_buffer_load == (8, 8)
    assert not T.fits(small, 64, 64, 64)
    one_wave, _ = T.make_point((16, 16, 1, 4), (1, 1), (1, 1), 16, 1, 1, 1, 0, 0, 0)
    assert T.fits(one_wave, 64, 64, 64)        # 16 x 16 x 16 x 4 / 64 = 16 bytes


def test_point_keys_distinguish_every_knob():
    cfg, _ = T.make_point((16, 16, 1, 4), (2, 2), (4, 2), 16, 1, 1, 1, 0, 0, 0)
    pts = list(T.knob_points(cfg, split_ks=(1, 0, 4), occs=(0, 2)))
    keys = [T.point_key(*p) for p in pts]
    assert len(keys) == len(set(keys))
    opts = {(o.depth_k if hasattr(o, "depth_k") else c.depth_k, c.vmem_stage, o.wgm, o.xcd, o.plr, o.pd, o.split_k, o.occ)
            for c, o in pts}
    assert len(opts) == len(pts)
    assert any(k.endswith("_sk4") for k in keys) and any("_occ2" in k for k in keys)


def _fake_points(out, pts, spilling=(), stale=()):
    """Stand-in code objects for points, with the .toml keys the sweep reads
    (source_sha of the current source unless the key is in ``stale``)."""
    d = T.point_dir(out)
    os.makedirs(d, exist_ok=True)
    for p in pts:
        k = T.point_key(*p)
        open(os.path.join(d, f"{k}.co"), "wb").write(k.encode())
        sha = "0" * 16 if k in stale else T.point_source(p)[1]
        g.write_toml({"name": k, "scratch_bytes_per_lane": 64 if k in spilling else 0, "source_sha": sha},
                     os.path.join(d, f"{k}.toml"))


def test_sweep_resumes_isolates_failures_and_emits_the_best(tmp_path, monkeypatch):
    out = str(tmp_path)
    monkeypatch.setattr(T, "POINTS_DIR", None)
    pts = [T.make_point((32, 32, 1, 2), (2, 2), wt, 16, 2, 4, 3, 1, 0, 8)
           for wt in ((1, 1), (2, 2), (4, 4), (2, 1), (1, 2), (2, 4))]
    keys = [T.point_key(*p) for p in pts]
    _fake_points(out, [pts[i] for i in (0, 1, 2, 4, 5)], spilling={keys[1]}, stale={keys[5]})
    compiled = {keys[0]: 0, keys[1]: 0, keys[2]: 0, keys[3]: 1, keys[4]: 0, keys[5]: 0}   # keys[3] failed to compile
    calls = []
    speed = {keys[2]: 1234.5, keys[4]: 2000.0}

    def bench(co, toml, timeout):
        calls.append(os.path.basename(co))
        if "wt1x1" in co:
            raise RuntimeError("runner crashed")               # isolated, the sweep goes on
        return 0, speed[os.path.basename(co)[:-3]]

    results = os.path.join(out, "results.jsonl")
    recs = T.sweep(pts, out, 256, 256, 64, bench, 10.0, results, compiled)
    status = {r["point"]: r["status"] for r in recs}
    assert status[keys[0]].startswith("error") and status[keys[1]] == "spills"
    assert status[keys[2]] == "ok" and status[keys[3]] == "compile_error" and status[keys[4]] == "ok"
    assert status[keys[5]] == "stale_build"                    # built from another source: never timed
    assert len(calls) == 3
    assert all(r["source_sha"] == T.point_source(p)[1] for r, p in zip(recs, pts))
    # resume: nothing is benchmarked again, the records come back from the JSONL file
    recs2 = T.sweep(pts, out, 256, 256, 64, bench, 10.0, results, compiled)
    assert len(calls) == 3 and [r["status"] for r in recs2] == [r["status"] for r in recs]
    assert len(open(results).read().splitlines()) == 6
    # a record of another source is not resumed: the point is timed again
    lines = [json.loads(x) for x in open(results).read().splitlines()]
    lines[2]["source_sha"] = "f" * 16
    with open(results, "w") as f:
        f.write("".join(json.dumps(x) + "\n" for x in lines))
    T.sweep(pts, out, 256, 256, 64, bench, 10.0, results, compiled)
    assert calls[3:] == [keys[2] + ".co"]
    # emission: the fastest point that validates (keys[4] fails, keys[2] is next)
    checked = []

    def validate(co, toml):
        checked.append(os.path.basename(co)[:-3])
        return os.path.basename(co)[:-3] != keys[4], "fake check"

    best = T.emit_best(out, recs, validate)
    assert checked == [keys[4], keys[2]] and best["point"] == keys[2]
    assert open(os.path.join(out, "generated_gemm.co"), "rb").read() == keys[2].encode()
    assert g.read_toml(os.path.join(out, "generated_gemm.toml"))["name"] == keys[2]
    assert T.emit_best(out, recs, lambda co, toml: (False, "no")) is None


def test_validation_shape_is_clipped():
    assert T.validation_shape(4096, 128, 4096) == (1024, 128, 1024)
    assert T.validation_shape(300, 200, 100) == (300, 200, 100)


def test_compile_only_builds_stage1_with_split_and_occupancy_knobs(tmp_path):
    out = str(tmp_path)
    rc = T.main(["--m", "64", "--n", "64", "--k", "64", "--bench", "unused", "--output-folder", out,
                 "--compile-only", "--jobs", "8"])
    assert rc == 0
    built = sorted(f for f in os.listdir(os.path.join(out, "points")) if f.endswith(".co"))
    assert built and all(f.startswith(("a16_", "a32_")) for f in built)
    for f in built:
        d = g.read_toml(os.path.join(out, "points", f[:-3] + ".toml"))
        assert d["scratch_bytes_per_lane"] == 0 and d["split_k"] == 1
    # the knob lists reach stage 2 (and the keys), checked without compiling
    cfg, _ = T.make_point((16, 16, 1, 4), (2, 2), (2, 2), 16, 2, 4, 3, 0, 0, 8)
    keys = {T.point_key(*p) for p in T.knob_points(cfg, split_ks=(1, 0), occs=(0, 2))}
    assert any(k.endswith("_occ2_sk0") for k in keys) and any(k.endswith("_occ2") for k in keys)
    assert sum(1 for k in keys if k.endswith("_sk0")) * 2 == len(keys)


def test_transposed_layout_flags_reach_every_point(tmp_path):
    """--trans-a / --trans-b build every candidate for op(A) = A^T, op(B) =
    B^T: the keys carry the layout, stage 2 keeps it and the emitted .toml
    records it (the reference's schema fields)."""
    out = str(tmp_path)
    rc = T.main(["--m", "64", "--n", "64", "--k", "64", "--bench", "unused", "--output-folder", out,
                 "--compile-only", "--jobs", "8", "--tiles", "32x32,64x64", "--trans-a", "--trans-b"])
    assert rc == 0
    built = sorted(f for f in os.listdir(os.path.join(out, "points")) if f.endswith(".co"))
    assert built and all(f.endswith("_tt.co") for f in built)
    for f in built:
        d = g.read_toml(os.path.join(out, "points", f[:-3] + ".toml"))
        assert d["trans_a"] is True and d["trans_b"] is True and d["scratch_bytes_per_lane"] == 0
    cfg, _ = T.make_point((16, 16, 1, 4), (2, 2), (2, 2), 16, 2, 4, 3, 0, 0, 8, trans=(True, False))
    keys = {T.point_key(*p) for p in T.knob_points(cfg)}
    assert keys and all(k.endswith("_tn") for k in keys)
    nn, _ = T.make_point((16, 16, 1, 4), (2, 2), (2, 2), 16, 2, 4, 3, 0, 0, 8)
    assert T.point_key(nn, _).endswith("_x8")


@pytest.mark.parametrize("name,occs,depths", [
    ("mt128x64_a16_wg2x4_dk64", (0,), (32, 64)),              # cfg5's instance
    ("mt256x128_a32_wg4x2_dk16_s3_occ4_plr2", (0, 2, 4), (16,)),  # cfg4's instance
])
def test_wide_space_reaches_the_eight_wave_instances(name, occs, depths):
    """With --space gfx950-wide, --occ and --stage1-depths covering them, the
    tuner's stage 1 holds the geometry of the catalog's eight-wave instances
    and stage 2 around it holds the instance's exact knobs."""
    from generator import catalog
    cfg, opt = catalog.SOLUTIONS[name]
    geo = (tuple(cfg.mfma), tuple(cfg.wave_group), tuple(cfg.wave_tiling))
    stage1 = [c for c, o in T.geometry_points(T.DEFAULT_KNOBS, wide=True, occs=occs, depths=depths,
                                              tiles=[tuple(cfg.tile_size)])
              if (tuple(c.mfma), tuple(c.wave_group), tuple(c.wave_tiling)) == geo and o.occ == opt.occ]
    assert stage1, name
    keys = {T.point_key(c, o) for c, o in T.knob_points(stage1[0], split_ks=(opt.split_k,), occs=(opt.occ,),
                                                          gws=(opt.gw,))}
    assert T.point_key(cfg, opt) in keys, name


def test_stage2_wave_specialisation_points():
    """--ws 0,1 adds wave-specialised stage-2 points: no split-K, no
    occupancy cap, a fourth LDS buffer only with them, and keys that tell
    them apart; geometries with odd WT0 get none."""
    from generator.generator import GemmSolutionConfig, MFMA_16x16x4
    base = GemmSolutionConfig(0, 0, 0, 0, MFMA_16x16x4, (1, 4), (4, 1), 32, False, False, vmem_stage=2)
    pts = list(T.knob_points(base, split_ks=(1, 0), occs=(0, 2), gws=(1,), wss=(0, 1)))
    ws = [(c, o) for c, o in pts if o.ws]
    assert ws and all(o.split_k == 1 and o.occ == 0 and o.pd == 1 for _, o in ws)
    assert {c.vmem_stage for c, _ in ws} == {1, 2, 3}
    assert all(c.vmem_stage < 3 for c, o in pts if not o.ws)
    keys = [T.point_key(c, o) for c, o in pts]
    assert len(keys) == len(set(keys)) and all("_ws" in T.point_key(c, o) for c, o in ws)
    odd = GemmSolutionConfig(0, 0, 0, 0, MFMA_16x16x4, (2, 2), (1, 2), 32, False, False, vmem_stage=2)
    assert not [o for _, o in T.knob_points(odd, wss=(1,)) if o.ws]


def test_stage2_k_split_points():
    """--ksplit 0,1 adds in-group K split points: no split-K, no occupancy
    cap, never with ws, no fourth LDS buffer, and keys of their own."""
    from generator.generator import GemmSolutionConfig, MFMA_16x16x4
    base = GemmSolutionConfig(0, 0, 0, 0, MFMA_16x16x4, (1, 4), (4, 1), 32, False, False, vmem_stage=2)
    pts = list(T.knob_points(base, split_ks=(1, 0), occs=(0, 2), gws=(1,), wss=(0, 1), kss=(0, 1)))
    ks = [(c, o) for c, o in pts if o.ksplit]
    assert ks and all(o.split_k == 1 and o.occ == 0 and not o.ws for _, o in ks)
    assert {c.vmem_stage for c, _ in ks} == {1, 2}
    keys = [T.point_key(c, o) for c, o in pts]
    assert len(keys) == len(set(keys)) and all(T.point_key(c, o).endswith("_ks") for c, o in ks)
    odd = GemmSolutionConfig(0, 0, 0, 0, MFMA_16x16x4, (2, 2), (1, 2), 32, False, False, vmem_stage=2)
    assert not [o for _, o in T.knob_points(odd, kss=(1,)) if o.ksplit]



def test_playoff_reranks_by_interleaved_medians(tmp_path, monkeypatch):
    """The playoff re-times the leaders round-robin, the order reversed every
    other round, and emission follows the medians: a point whose single
    timing was lucky loses to one that is faster every time it is re-timed."""
    out = str(tmp_path)
    monkeypatch.setattr(T, "POINTS_DIR", None)
    pts = [T.make_point((32, 32, 1, 2), (2, 2), wt, 16, 2, 4, 3, 1, 0, 8) for wt in ((1, 1), (2, 2), (4, 4), (2, 1))]
    keys = [T.point_key(*p) for p in pts]
    _fake_points(out, pts)
    compiled = {kk: 0 for kk in keys}
    single = {keys[0]: 1100.0, keys[1]: 1000.0, keys[2]: 990.0, keys[3]: 500.0}   # keys[0]'s first timing was lucky
    steady = {keys[0]: 900.0, keys[1]: 980.0, keys[2]: 995.0, keys[3]: 500.0}
    order = []

    def bench(co, toml, timeout):
        kk = os.path.basename(co)[:-3]
        order.append(kk)
        if len(order) <= len(keys):
            return 0, single[kk]
        if kk == keys[2] and len(order) == len(keys) + 3:
            return 0, 1.0       # its first re-timing is bad: the median ignores it
        return 0, steady[kk]

    recs = T.sweep(pts, out, 256, 256, 64, bench, 10.0, os.path.join(out, "results.jsonl"), compiled)
    ranked = T.playoff(recs, out, bench, 3, 4, 10.0)
    played = order[len(keys):]
    assert played == [keys[0], keys[1], keys[2], keys[2], keys[1], keys[0]] * 2   # ABC CBA ABC CBA
    assert [r["point"] for r in ranked] == [keys[2], keys[1], keys[0]]
    assert ranked[0]["playoff"] == [1.0, 995.0, 995.0, 995.0] and ranked[0]["playoff_gflops"] == 995.0
    best = T.emit_best(out, recs, lambda co, toml: (True, "ok"))
    assert best["point"] == keys[2]
    # a participant that fails validation hands over to the next median, not to a single timing
    best = T.emit_best(out, recs, lambda co, toml: (os.path.basename(co)[:-3] != keys[2], "x"))
    assert best["point"] == keys[1]
    T.write_summary(os.path.join(out, "s.md"), recs, best, 256, 256, 64, ["--playoff", "3"])
    text = open(os.path.join(out, "s.md")).read()
    assert "Playoff (4 interleaved rounds" in text and "(playoff median)" in text
