"""Model I/O: PotMTP::Load / PotMTP::Save (potentials/potential_mtp.cpp:
119-571, 647-785, 1052-1061), the potential_tag metadata
(tools/mtp_metadata.h) and the radial bases of basis/basis.cpp.

The product's writer (mtpx_format_model_text, host only) is compared byte
for byte with the oracle's restatement of PotMTP::Save; the tag handling
with answers worked out from the reference's metadata rules; the oracle's
bases with the reference core (oracle/_ref/mlip_ref, where built) and with
closed forms."""
import numpy as np
import pytest

import oracle as O
from helpers import rel_err
from mtpx import capi
from mtpx import synth as S

SPLIT = [("RBChebyshev", 1.7, 4.6), ("RBChebyCos", 1.8, 4.9),
         ("RBChebyshevPoly5", 1.6, 5.2, -0.2), ("RBChebyshevPoly4", 1.9, 4.4, 0.5)]
BASES = {"chebyshev": {}, "chebycos": dict(basis="RBChebyCos"),
         "poly4": dict(basis="RBChebyshevPoly4"), "poly5": dict(basis="RBChebyshevPoly5"),
         "split": dict(pair_bases=SPLIT),
         "configurable": dict(basis=S.configurable("smoothstep7", "exponential_tanh", True)),
         "split-configurable": dict(pair_bases=[
             (S.configurable("poly3", "i2"), 1.7, 4.6), (S.configurable("cosine_left", "exponential"), 1.8, 4.9),
             (S.configurable("sine_squared", "exponential_left", True), 1.6, 5.2), ("RBChebyshevPoly5", 1.9, 4.4, 0.5)])}
DEFAULT_TAG = '{"model":"linear","schema":"gpml.mtp.metadata","type":"MTP","version":1}'


def model_text(kind, template="shapeev-06.mtp", seed=721, **extra):
    kw = dict(BASES[kind])
    kw.update(extra)
    return S.random_model(template, 2, 6, 1.8, 4.8, -0.5, 0.5, S.rng_for(seed), **kw)


def tag_line(text):
    return [l for l in text.splitlines() if l.startswith("potential_tag")][0]


@pytest.mark.parametrize("kind", list(BASES))
def test_writer_matches_oracle_save(kind):
    text = model_text(kind)
    got = capi.format_model_text(text)
    assert got == O.Model(text).save_text()
    # a second pass is the identity (17 significant digits round-trip)
    assert capi.format_model_text(got) == got


@pytest.mark.parametrize("name", ["shapeev-16.mtp", "potential.mtp", "pot4b.mtp", "dup-scalar.mtp"])
def test_writer_templates(name):
    text = S.read_template(name)
    got = capi.format_model_text(text)
    assert got == O.Model(text).save_text()
    assert tag_line(got) == "potential_tag = " + DEFAULT_TAG


def test_round_trip_keeps_every_coefficient():
    text = model_text("split", template="shapeev-16.mtp")
    out = capi.format_model_text(text)
    info = np.zeros(8, np.int32)
    a = np.zeros(4000)
    b = np.zeros(4000)
    import ctypes as C
    for t, x in ((text, a), (out, b)):
        assert capi.lib().mtpx_parse_model_text(t.encode(), info.ctypes.data_as(C.POINTER(C.c_int)),
                                                x.ctypes.data_as(C.POINTER(C.c_double)), None, 0) == 0
    n = int(info[7])
    assert np.array_equal(a[:n].view(np.uint64), b[:n].view(np.uint64))


# Tags: Tag::parse keeps plain text as the legacy text, a JSON object with
# the gpml.mtp.metadata schema as fields; Tag::output drops the model-derived
# keys, adds type / model / schema / version and the legacy text, and the
# writer emits compact JSON with sorted keys and picojson's escapes.
TAGS = [
    ("", DEFAULT_TAG),
    ("NiAl fit v2", '{"legacy_tag":"NiAl fit v2","model":"linear","schema":"gpml.mtp.metadata",'
                    '"type":"MTP","version":1}'),
    ('a/b "q"', '{"legacy_tag":"a\\/b \\"q\\"","model":"linear","schema":"gpml.mtp.metadata",'
                '"type":"MTP","version":1}'),
    ('{"foo": 1}', '{"legacy_tag":"{\\"foo\\": 1}","model":"linear",'
                   '"schema":"gpml.mtp.metadata","type":"MTP","version":1}'),
    ('{"schema": "gpml.mtp.metadata", "version": 1, "type": "MTP", "model": "linear", '
     '"elements": ["Ni", "Al"], "note": "x/y", "w": 0.1, "k": 3.0, "model_coeffs_count": 7}',
     '{"elements":["Ni","Al"],"k":3,"model":"linear","note":"x\\/y","schema":"gpml.mtp.metadata",'
     '"type":"MTP","version":1,"w":0.10000000000000001}'),
    ('{"schema":"gpml.mtp.metadata","version":1,"type":"MTP","model":"linear",'
     '"legacy_tag":"old","units":{"energy":"eV","b":[true,null]}}',
     '{"legacy_tag":"old","model":"linear","schema":"gpml.mtp.metadata","type":"MTP",'
     '"units":{"b":[true,null],"energy":"eV"},"version":1}'),
]


@pytest.mark.parametrize("raw,expected", TAGS, ids=[str(i) for i in range(len(TAGS))])
def test_tag_known_answers(raw, expected):
    text = model_text("chebyshev", tag=raw)
    assert tag_line(capi.format_model_text(text)) == "potential_tag = " + expected
    if not raw.startswith("{"):
        assert tag_line(O.Model(text).save_text()) == "potential_tag = " + expected


@pytest.mark.parametrize("raw", [
    '{"schema":"gpml.mtp.metadata","version":1,"type":"MTP","model":"linear","elements":["Ni"]}',
    '{"schema":"gpml.mtp.metadata","version":1,"type":"MTP_M","model":"mtp_m_li","q":1}',
    '{"schema":"gpml.mtp.metadata","version":2,"type":"MTP","model":"linear"}',
    '{"schema":"gpml.mtp.metadata","version":1,"type":"MTP","model":"linear","elements":["Ni","Xx"]}',
    '{"schema":"gpml.mtp.metadata", "version":1',
    'v1 | imrmlp_meta_v1:{"model_type":"mtp"}',
])
def test_tag_refused(raw):
    with pytest.raises(capi.MtpxError):
        capi.format_model_text(model_text("chebyshev", tag=raw))


def test_unsupported_basis_is_refused():
    text = model_text("chebyshev").replace("RBChebyshev", "RBPolyB")
    with pytest.raises(capi.MtpxError):
        capi.format_model_text(text)


# ---------------------------------------------- the oracle's radial bases --

def test_envelope_closed_forms():
    """Each basis is s T_k(xi) rc(r): rc = (r - max)^2 (RBChebyshev),
    (1 + cos(pi r / max)) / 2 (RBChebyCos), (1 - x)^3 (1 + (3 + b) x) and
    (1 - x)^4 (1 + (4 + b) x) with x = (r - min) / (max - min) (Poly4, Poly5,
    zero outside [min, max]); derivatives against central differences."""
    rmin, rmax, b, s = 1.8, 4.8, -1.0 / 3.0, 0.01
    env = {"chebyshev": lambda r: (r - rmax) ** 2,
           "chebycos": lambda r: 0.5 * (1 + np.cos(np.pi * r / rmax)),
           "poly4": lambda r: (1 - (r - rmin) / (rmax - rmin)) ** 3 * (1 + (3 + b) * (r - rmin) / (rmax - rmin)),
           "poly5": lambda r: (1 - (r - rmin) / (rmax - rmin)) ** 4 * (1 + (4 + b) * (r - rmin) / (rmax - rmin))}
    for kind, f in env.items():
        m = O.Model(model_text(kind))
        for r in np.linspace(1.85, 4.75, 17):
            v, d = m.rb_calc_der(r)
            xi = (2 * r - (rmin + rmax)) / (rmax - rmin)
            T = np.cos(np.arange(6) * np.arccos(xi))
            assert np.allclose(v, s * T * f(r), rtol=1e-11, atol=1e-16), kind
            h = 1e-6
            fd = (m.rb_calc_der(r + h)[0] - m.rb_calc_der(r - h)[0]) / (2 * h)
            assert np.allclose(d, fd, rtol=1e-6, atol=1e-11), kind
        if kind.startswith("poly"):
            assert not m.rb_calc_der(rmin - 0.1)[0].any() and not m.rb_calc_der(rmax + 0.1)[0].any()


def test_split_pairs_use_their_own_basis():
    m = O.Model(model_text("split"))
    assert m.cutoff == 5.2
    for q, pb in enumerate(SPLIT):
        ti, tj = divmod(q, 2)
        one = O.Model(model_text({"RBChebyshev": "chebyshev", "RBChebyCos": "chebycos",
                                  "RBChebyshevPoly4": "poly4", "RBChebyshevPoly5": "poly5"}[pb[0]]))
        for r in (2.0, 3.3, 4.3):
            got = m.rb_calc_der(r, ti, tj)
            # the same kind on the pair's interval (b where it has one)
            lines = S.basis_lines(pb[0], pb[1], pb[2], 6, *pb[3:])
            ref_text = model_text("chebyshev").replace(
                "\n".join(S.basis_lines("RBChebyshev", 1.8, 4.8, 6)), "\n".join(lines))
            exp = O.Model(ref_text).rb_calc_der(r)
            assert np.array_equal(got[0], exp[0]) and np.array_equal(got[1], exp[1])
        del one


def test_split_with_identical_pairs_equals_shared_basis():
    same = [("RBChebyCos", 1.8, 4.8)] * 4
    a, b = model_text("split", pair_bases=same), model_text("chebycos")
    rng = S.rng_for(722)
    s = S.displace(S.lattice("bcc", (3, 3, 3), 2.87), rng, 0.15)
    s.types = (S.uniform(rng, s.n) * 2).astype(np.int32)
    pos = O.wrap(s.cell, s.pbc, s.pos)
    ma, mb = O.Model(a), O.Model(b)
    nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, 4.8)
    for x, y in zip(O.efs(ma, nb), O.efs(mb, nb)):
        assert np.array_equal(np.asarray(x), np.asarray(y))


# every cutoff once, the shifts in turn, both basis function types
CONFIGS = [(c, S.SHIFT_TYPES[k % 5], k % 2 == 1) for k, c in enumerate(S.CUTOFF_TYPES)]


def _cfg_model(cut, shift, om, R=6):
    return O.Model(S.random_model("shapeev-06.mtp", 2, R, 1.8, 4.8, -0.5, 0.5, S.rng_for(723),
                                  basis=S.configurable(cut, shift, om)))


@pytest.mark.parametrize("cut,shift,om", CONFIGS)
def test_configurable_structure(cut, shift, om):
    """RBChebyshevConfigurable (basis.cpp:931-1011) is s raw_k(x(r)) fc(r):
    Q_0 / s gives the cutoff and Q_1 / Q_0 the shift (chebyshev), and every
    Q_k / Q_0 is T_k(x) = cos(k acos x) (or (1 - T_(k+1)) / (1 - x) for
    one_minus); every cutoff vanishes at max_dist, each shift maps the
    interval ends as its definition fixes, derivatives match central
    differences, and the basis is zero outside [min, max]."""
    m = _cfg_model(cut, shift, om)
    s, lo, hi = 0.01, 1.8, 4.8
    ends = {"linear": (-1, 1), "exponential": (-1, 1), "i2": (1, -1), "exponential_tanh": (-1, 1)}
    for r in np.linspace(1.85, 4.75, 13):
        v, d = m.rb_calc_der(r)
        k = np.arange(6)
        if abs(v[0]) > 1e-12:
            if not om:
                x = v[1] / v[0]
                T = np.cos(k * np.arccos(np.clip(x, -1, 1)))
                assert np.allclose(v / v[0], T, rtol=1e-9, atol=1e-9)
            else:
                # Q_k / Q_0 = (1 - T_(k+1)) / (1 - T_1), and Q_1 / Q_0 = 2 (1 + x)
                x = v[1] / (2 * v[0]) - 1
                T = np.cos((k + 1) * np.arccos(np.clip(x, -1, 1)))
                assert np.allclose(v / v[0], (1 - T) / (1 - x), rtol=1e-8, atol=1e-8)
            assert -1 - 1e-12 <= x <= 1 + 1e-12
        h = 1e-6
        fd = (m.rb_calc_der(r + h)[0] - m.rb_calc_der(r - h)[0]) / (2 * h)
        assert np.allclose(d, fd, rtol=1e-6, atol=1e-10)
    at_hi = m.rb_calc_der(hi)[0]
    assert np.abs(at_hi).max() < 1e-13
    assert not m.rb_calc_der(lo - 0.05)[0].any() and not m.rb_calc_der(hi + 0.05)[0].any()
    if not om and shift in ends and cut in ("cosine", "smoothstep5", "poly3"):
        # a cutoff that is positive at min_dist: the shift's value there
        v = m.rb_calc_der(lo)[0]
        assert abs(v[1] / v[0] - ends[shift][0]) < 1e-12


needs_ref = pytest.mark.skipif(not O.ref_available("mlip_ref"),
                               reason="reference binaries not built (make -C oracle ref)")


@needs_ref
@pytest.mark.parametrize("cut,shift,om", CONFIGS)
def test_configurable_matches_reference_core(workdir, cut, shift, om):
    """Every cutoff, every shift and both basis function types against the
    reference core's configurable basis (runtime/mtp/radial_basis.h) at
    1e-12: E, site energies, forces, virial."""
    text = S.random_model("shapeev-06.mtp", 2, 6, 1.8, 4.8, -0.5, 0.5, S.rng_for(724),
                          basis=S.configurable(cut, shift, om))
    m = O.Model(text)
    rng = S.rng_for(725)
    s = S.displace(S.strain(S.lattice("bcc", (3, 3, 3), 2.87), rng, 0.03), rng, 0.15)
    s.types = (S.uniform(rng, s.n) * 2).astype(np.int32)
    pos = O.wrap(s.cell, s.pbc, s.pos)
    nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, m.cutoff)
    E, F, St, se = O.efs(m, nb)
    Er, ser, Fr, vr = O.ref_mlip_efs(text, nb, s.types, m.cutoff, workdir, m.Z)
    sym = 0.5 * (St + St.T)
    v6 = np.array([sym[0, 0], sym[1, 1], sym[2, 2], sym[0, 1], sym[0, 2], sym[1, 2]])
    assert rel_err(E, Er) < 1e-12 and rel_err(se, ser) < 1e-12
    assert rel_err(F, Fr) < 1e-12 and rel_err(v6, vr) < 1e-12


@needs_ref
@pytest.mark.parametrize("kind", ["chebycos", "poly4", "poly5", "split"])
def test_bases_match_reference_core(workdir, kind):
    """E, site energies, forces and the virial against the reference core
    (runtime/mtp/mlip.cpp, radial_basis_setup.cpp) at 1e-12."""
    text = model_text(kind)
    m = O.Model(text)
    rng = S.rng_for(720)
    s = S.displace(S.strain(S.lattice("bcc", (3, 3, 3), 2.87), rng, 0.03), rng, 0.15)
    s.types = (S.uniform(rng, s.n) * 2).astype(np.int32)
    pos = O.wrap(s.cell, s.pbc, s.pos)
    nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, m.cutoff)
    E, F, St, se = O.efs(m, nb)
    Er, ser, Fr, vr = O.ref_mlip_efs(text, nb, s.types, m.cutoff, workdir, m.Z)
    sym = 0.5 * (St + St.T)
    v6 = np.array([sym[0, 0], sym[1, 1], sym[2, 2], sym[0, 1], sym[0, 2], sym[1, 2]])
    assert rel_err(E, Er) < 1e-12 and rel_err(se, ser) < 1e-12
    assert rel_err(F, Fr) < 1e-12 and rel_err(v6, vr) < 1e-12
