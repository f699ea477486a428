"""E/F/S parity of the HIP path against the CPU oracle.

Tolerance: 1e-10 relative to the max-abs of each quantity (energy, site
energies, forces, stress), the bar stated for fp64 E/F/S.  Every case runs
through the C ABI (libmtpx.so) on cuda:0.
"""
import numpy as np
import pytest

import oracle as O
from helpers import assert_efs_close, oracle_case, rel_err, upload_oracle_lists
from mtpx import synth as S

TOL = 1e-10
pytestmark = pytest.mark.gpu


def _template_model(name, Z, R, rmin, rmax, seed, lo=-0.05, hi=0.05):
    return S.random_model(name, Z, R, rmin, rmax, lo, hi, S.rng_for(100 + seed))


def _cases():
    out = []
    out.append(("lvl10-fcc108", *S.workload_inference(1)))
    out.append(("lvl16-fcc256", *S.scaled_inference(2, (4, 4, 4))))
    out.append(("lvl20-fcc108-z4", *S.scaled_inference(3, (3, 3, 3))))
    rng = S.rng_for(200)
    s = S.displace(S.strain(S.lattice("bcc", (3, 3, 4), 2.87), rng, 0.03), rng, 0.15)
    s.types = (S.uniform(rng, s.n) * 2).astype(np.int32)
    out.append(("shapeev06-bcc", _template_model("shapeev-06.mtp", 2, 6, 1.6, 4.8, 1), s))
    out.append(("ps1-7b-517-M8", _template_model("ps1-7b-517.mtp", 2, 8, 1.6, 4.8, 2), s))
    out.append(("pot4b-M8", _template_model("pot4b.mtp", 2, 8, 1.6, 4.8, 3), s))
    trained = open(S.os.path.join(S.TEMPLATE_DIR, "potential.mtp")).read()
    out.append(("trained-potential.mtp", trained, s))
    liq = S.training_structures(5, 1)[0]
    out.append(("lvl20-liquid-z3", S.training_models(5)[1], liq))
    # dense: > 64 neighbours per atom exercises the multi-chunk neighbour loop
    dense = S.random_model("shapeev-16.mtp", 3, 8, 1.5, 7.5, -0.05, 0.05, S.rng_for(300))
    out.append(("lvl16-dense-liquid", dense, liq))
    # duplicate scalar mapping {0, 4, 5, 6, 4} and rules with l == r
    # (runtime/mtp/cpu/tests/test_mtp_cpu.cpp:30-33)
    dup = S.random_model("dup-scalar.mtp", 2, 6, 1.8, 4.6, -0.5, 0.5, S.rng_for(700))
    out.append(("dup-scalar-map", dup, s))
    return out


CASES = _cases()


@pytest.mark.parametrize("name,model_text,s", CASES, ids=[c[0] for c in CASES])
def test_efs_matches_oracle(ctx, name, model_text, s):
    ref = oracle_case(model_text, s)
    ctx.load_model_text(model_text)
    upload_oracle_lists(ctx, ref["nb"])
    got = ctx.efs()
    assert_efs_close(got, ref, TOL)
    got_det = ctx.efs(deterministic=True)
    assert_efs_close(got_det, ref, TOL)


def test_dense_case_has_long_lists():
    name, model_text, s = CASES[-2]
    ref = oracle_case(model_text, s)
    counts = np.diff(ref["nb"].offsets)
    assert counts.max() > 64


def test_deterministic_mode_is_bitwise_repeatable(ctx):
    model_text, s = S.scaled_inference(2, (4, 4, 4))
    ref = oracle_case(model_text, s)
    ctx.load_model_text(model_text)
    upload_oracle_lists(ctx, ref["nb"])
    a = ctx.efs(deterministic=True)
    b = ctx.efs(deterministic=True)
    for x, y in zip(a, b):
        assert np.array_equal(np.asarray(x).view(np.uint64), np.asarray(y).view(np.uint64))


def test_timings_switch(ctx):
    """mtpx_set_timings: with the HIP events off a call reports zero timings
    and the same results, bit for bit; back on, the kernel time is positive."""
    model_text, s = S.scaled_inference(2, (3, 3, 3))
    pos = O.wrap(s.cell, s.pbc, s.pos)
    ctx.load_model_text(model_text)
    ctx.build_neighbors(s.cell, s.pbc, pos, s.types, 5.0)
    ctx.efs_device(False)
    assert ctx.last_timings()[1] > 0
    on = ctx.efs()
    ctx.set_timings(False)
    ctx.efs_device(False)
    assert not ctx.last_timings().any()
    off = ctx.efs()
    assert not ctx.last_timings().any()
    for x, y in zip(on, off):
        assert np.array_equal(np.asarray(x).view(np.uint64), np.asarray(y).view(np.uint64))
    ctx.set_timings(True)
    ctx.efs_device(False)
    assert ctx.last_timings()[1] > 0


def test_isolated_atom_energy_is_species_coefficient(ctx):
    model_text, _ = S.scaled_inference(2, (2, 2, 2))
    ctx.load_model_text(model_text)
    # one centre without neighbours: E_i = species coefficient of its type
    ctx.set_neighbors(np.array([0, 0]), np.zeros(0), np.zeros(0), np.zeros((0, 3)), np.zeros(0),
                      np.array([1]))
    E, F, St, se = ctx.efs()
    coef = ctx.get_coeffs()
    nrad = ctx.info["Z"] ** 2 * ctx.info["M"] * ctx.info["R"]
    assert E == coef[nrad + 1]
    assert np.all(F == 0) and np.all(St == 0)


def test_empty_structure(ctx):
    model_text, _ = S.scaled_inference(2, (2, 2, 2))
    ctx.load_model_text(model_text)
    ctx.set_neighbors(np.array([0]), np.zeros(0), np.zeros(0), np.zeros((0, 3)), np.zeros(0),
                      np.zeros(0))
    E, F, St, se = ctx.efs()
    assert E == 0 and F.shape == (0, 3) and np.all(St == 0)


def test_entries_beyond_cutoff_are_skipped(ctx):
    """potential_mtp.cpp:2842: list entries with d > cutoff contribute nothing;
    d == cutoff is kept (and contributes zero through (r - r_c)^2)."""
    model_text, s = S.scaled_inference(2, (2, 2, 2))
    ref = oracle_case(model_text, s)
    nb = ref["nb"]
    rc = ref["model"].cutoff
    # append one far entry and one exactly-at-cutoff entry to centre 0
    far = np.array([[rc + 0.3, 0.0, 0.0], [0.0, rc, 0.0]])
    off = nb.offsets.copy()
    ins = off[1]
    idx = np.insert(nb.idx, ins, [1, 2])
    typ = np.insert(nb.types, ins, [nb.center_types[1], nb.center_types[2]])
    vec = np.insert(nb.vec, ins, far, axis=0)
    dist = np.insert(nb.dist, ins, [rc + 0.3, rc])
    off[1:] += 2
    ctx.load_model_text(model_text)
    ctx.set_neighbors(off, idx, typ, vec, dist, nb.center_types)
    E, F, St, se = ctx.efs()
    onb = O.Neighbors.from_csr(off, idx, typ, vec, dist, nb.center_types)
    Eo, Fo, So, seo = O.efs(ref["model"], onb)
    assert rel_err(E, Eo) < TOL and rel_err(F, Fo) < TOL and rel_err(St, So) < TOL
    assert rel_err(E, ref["E"]) < TOL  # identical to the list without the extra entries


def test_coefficient_update_changes_results(ctx):
    model_text, s = S.scaled_inference(2, (3, 3, 3))
    ref = oracle_case(model_text, s)
    ctx.load_model_text(model_text)
    upload_oracle_lists(ctx, ref["nb"])
    x = ctx.get_coeffs()
    x2 = x * 1.1
    ctx.set_coeffs(x2)
    m = ref["model"]
    m.coeffs = x2
    E, F, St, se = O.efs(m, ref["nb"])
    assert_efs_close(ctx.efs(), dict(E=E, F=F, S=St, se=se), TOL)


def test_full_size_workload2_matches_oracle(ctx):
    """The 32,000-atom level-16 cell against the oracle (OpenMP getEFSOMP)."""
    model_text, s = S.workload_inference(2)
    m = O.Model(model_text)
    pos = O.wrap(s.cell, s.pbc, s.pos)
    nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, m.cutoff)
    E, F, St, se = O.efs(m, nb, threads=16)
    ctx.load_model_text(model_text)
    upload_oracle_lists(ctx, nb)
    got = ctx.efs()
    assert_efs_close(got, dict(E=E, F=F, S=St, se=se), TOL)
    # size-independent properties
    Eg, Fg, Sg, seg = got
    assert abs(Eg - seg.sum()) <= 1e-12 * np.abs(seg).sum()
    assert np.abs(Fg.sum(axis=0)).max() < 1e-9 * np.abs(Fg).max() * np.sqrt(len(Fg))
    assert np.abs(Sg - Sg.T).max() < 1e-9 * np.abs(Sg).max()


@pytest.mark.timeout(600)
def test_full_size_workload3_matches_oracle(ctx):
    """The 256,000-atom level-20 four-species cell (about 14.8M directed
    entries): device lists bit-exact against the oracle's BOXED lists, E/F/S
    against the oracle's getEFSOMP at 1e-10, and the size-independent sums."""
    model_text, s = S.workload_inference(3)
    m = O.Model(model_text)
    pos = O.wrap(s.cell, s.pbc, s.pos)
    nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, m.cutoff)
    assert s.n == 256000 and nb.P > 14_000_000
    ctx.load_model_text(model_text)
    ctx.build_neighbors(s.cell, s.pbc, pos, s.types, m.cutoff)
    got = ctx.get_neighbors()
    assert np.array_equal(got["offsets"], nb.offsets)
    assert np.array_equal(got["idx"], nb.idx)
    assert np.array_equal(got["types"], nb.types)
    assert np.array_equal(got["vec"].view(np.uint64), nb.vec.view(np.uint64))
    assert np.array_equal(got["dist"].view(np.uint64), nb.dist.view(np.uint64))
    del got
    E, F, St, se = O.efs(m, nb, threads=16)
    res = ctx.efs()
    assert_efs_close(res, dict(E=E, F=F, S=St, se=se), TOL)
    Eg, Fg, Sg, seg = res
    assert abs(Eg - seg.sum()) <= 1e-12 * np.abs(seg).sum()
    assert np.abs(Fg.sum(axis=0)).max() < 1e-9 * np.abs(Fg).max() * np.sqrt(len(Fg))
    assert np.abs(Sg - Sg.T).max() < 1e-9 * np.abs(Sg).max()
    # the deterministic path at this size too
    assert_efs_close(ctx.efs(deterministic=True), dict(E=E, F=F, S=St, se=se), TOL)


@pytest.mark.parametrize("name,model_text,s", CASES[:4], ids=[c[0] for c in CASES[:4]])
def test_energy_only_matches_oracle_get_e(ctx, name, model_text, s):
    """getE: energies without the gradient, the same numbers as mtpx_efs."""
    m = O.Model(model_text)
    pos = O.wrap(s.cell, s.pbc, s.pos)
    nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, m.cutoff)
    Eo, seo = O.energy(m, nb)
    ctx.load_model_text(model_text)
    ctx.build_neighbors(s.cell, s.pbc, pos, s.types, m.cutoff)
    E, se = ctx.energy()
    assert rel_err(E[0], Eo) < 1e-10 and rel_err(se, seo) < 1e-10
    E2, _, _, se2 = ctx.efs()
    assert np.array_equal(se, se2)


def test_energy_only_per_structure(ctx):
    text, _ = S.training_models(4)
    m = O.Model(text)
    structs = S.training_structures(4, 5)
    for st in structs:
        st.pos = O.wrap(st.cell, st.pbc, st.pos)
    ctx.load_model_text(text)
    off = ctx.set_structures(structs, 5.0)
    E, se = ctx.energy()
    for c, st in enumerate(structs):
        nb = O.Neighbors.build(st.cell, st.pbc, st.pos, st.types, 5.0)
        Eo, seo = O.energy(m, nb)
        assert rel_err(E[c], Eo) < 1e-10
        assert rel_err(se[off[c]:off[c + 1]], seo) < 1e-10


def _oversized_model(K=12001):
    """One basic moment and K-1 product rules m_k = m_0 m_0: a per-wave work
    space far beyond a CU's 160 KB of LDS."""
    times = ", ".join("{0, 0, 1, %d}" % k for k in range(1, K))
    return ("MTP\nversion = 1.1.0\npotential_name = MTP1m\nscaling = 0.01\nspecies_count = 1\n"
            "potential_tag = \nradial_basis_type = RBChebyshev\n\tmin_dist = 2\n\tmax_dist = 5\n"
            "\tradial_basis_size = 8\n\tradial_funcs_count = 1\n"
            "alpha_moments_count = %d\nalpha_index_basic_count = 1\n"
            "alpha_index_basic = {{0, 0, 0, 0}}\nalpha_index_times_count = %d\n"
            "alpha_index_times = {%s}\nalpha_scalar_moments = 1\nalpha_moment_mapping = {%d}\n"
            % (K, K - 1, times, K - 1))


def test_failed_model_load_leaves_previous_model(ctx):
    """A model refused for capacity changes nothing: the loaded model, its
    tables and results stay as they were (no half-installed model)."""
    from mtpx import capi
    model_text, s = S.scaled_inference(2, (3, 3, 3))
    ref = oracle_case(model_text, s)
    ctx.load_model_text(model_text)
    upload_oracle_lists(ctx, ref["nb"])
    before = ctx.efs()
    with pytest.raises(capi.MtpxError) as e:
        ctx.load_model_text(_oversized_model())
    assert e.value.code == -7  # MTPX_E_CAPACITY
    after = ctx.efs()
    for x, y in zip(before, after):
        assert np.allclose(x, y, rtol=1e-13, atol=0)
    assert_efs_close(after, ref, TOL)
