"""MTP-M potentials (potentials/potential_mtp_m.h; the short-range runtime's
reader and site executor, runtime/mtp/mlip.cpp:70-296 and
runtime/mtp/cpu/mtp_cpu.cpp:291-442).

The oracle's heads are pinned three ways: against the reference executor
itself (oracle/_ref/mtpm_ref, where it is built) to 1e-12; against closed
forms -- a head that is linear in its descriptors is a linear MTP with
folded species and moment coefficients, checked against the linear oracle
(itself pinned) -- and against finite differences of the energy (forces,
virial), which a dropped chain-rule term or a transposed weight fails.
The product's host-side reader, metadata checks and writer are compared
with the oracle and with the reference reader's verdicts."""
import os
import subprocess

import numpy as np
import pytest

import oracle as O
from helpers import rel_err
from mtpx import capi
from mtpx import synth as S

ACTS = ("TANH", "RELU", "SIGMOID", "LINEAR")
CASES = ([("mtp_m_li", 0, 0, "TANH"), ("mtp_m_q2", 0, 0, "TANH"), ("mtp_m_fs", 0, 0, "TANH")]
         + [("mtp_m_n1", 4, 0, a) for a in ACTS]
         + [("mtp_m_n2", 4, 3, a) for a in ACTS if a != "LINEAR"])
HEAD_IDS = {h: k for k, h in enumerate(capi.HEADS)}

needs_ref = pytest.mark.skipif(not O.ref_available("mtpm_ref"),
                               reason="oracle/_ref/mtpm_ref not built (make -C oracle ref)")


def base_text(seed=40, template="shapeev-10.mtp", Z=2):
    return S.random_model(template, Z, 6, 2.0, 5.0, -0.1, 0.1, S.rng_for(seed))


def head_text(head, h1=0, h2=0, act="TANH", form="both", seed=41, base=None, q=None):
    return S.mtpm_model(base or base_text(), head, S.rng_for(seed), q=q, h1=h1, h2=h2,
                        activation=act, form=form)


def structure(seed=42, reps=(2, 2, 2)):
    rng = S.rng_for(seed)
    s = S.displace(S.strain(S.lattice("fcc", reps, 3.6), rng, 0.02), rng, 0.12)
    s.types = (S.uniform(rng, s.n) * 2).astype(np.int32)
    return s


def efs_of(model, s, pos=None):
    pos = O.wrap(s.cell, s.pbc, s.pos if pos is None else pos)
    nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, model.cutoff)
    return O.efs(model, nb)


def virial6(St):
    sym = 0.5 * (St + St.T)
    return np.array([sym[0, 0], sym[1, 1], sym[2, 2], sym[0, 1], sym[0, 2], sym[1, 2]])


def case_id(c):
    return "%s-%s" % (c[0], c[3])


# ------------------------------------------- the reference site executor --

@needs_ref
@pytest.mark.parametrize("form", ["both", "tag", "footer"])
@pytest.mark.parametrize("case", CASES, ids=case_id)
def test_oracle_matches_reference_executor(workdir, case, form):
    head, h1, h2, act = case
    text = head_text(head, h1, h2, act, form)
    m = O.Model(text)
    assert (m.head, m.h1, m.h2) == (HEAD_IDS[head], h1, h2)
    s = structure()
    pos = O.wrap(s.cell, s.pbc, s.pos)
    nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, m.cutoff)
    E, F, St, se = O.efs(m, nb)
    Er, ser, Fr, vr = O.ref_mlip_efs(text, nb, s.types, m.cutoff, workdir, m.Z, binary="mtpm_ref")
    assert rel_err(E, Er) < 1e-12 and rel_err(se, ser) < 1e-12
    assert rel_err(F, Fr) < 1e-12 and rel_err(virial6(St), vr) < 1e-12


@needs_ref
@pytest.mark.parametrize("case", [CASES[1], CASES[4], CASES[8]], ids=case_id)
def test_duplicate_scalars_match_reference_executor(workdir, case):
    """alpha_moment_mapping {0, 4, 5, 6, 4} (the executor's own test graph,
    runtime/mtp/cpu/tests/test_mtp_cpu.cpp:30-33): each descriptor counts
    moment 4 with the sum of its two coefficients, in energy and forces."""
    head, h1, h2, act = case
    base = S.random_model("dup-scalar.mtp", 2, 6, 1.8, 4.6, -0.5, 0.5, S.rng_for(700))
    text = head_text(head, h1, h2, act, base=base, seed=43)
    m = O.Model(text)
    s = structure(44)
    pos = O.wrap(s.cell, s.pbc, s.pos)
    nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, m.cutoff)
    E, F, St, se = O.efs(m, nb)
    Er, ser, Fr, vr = O.ref_mlip_efs(text, nb, s.types, m.cutoff, workdir, m.Z, binary="mtpm_ref")
    assert rel_err(E, Er) < 1e-12 and rel_err(F, Fr) < 1e-12
    assert rel_err(virial6(St), vr) < 1e-12


# ------------------------------------------------------------ closed forms --

def _coeff_blocks(m, x):
    """(radial, species Z, descriptor species [P, Z], moments [P, S], head)."""
    r, Z, P, S_ = m.nradial, m.Z, m.P, m.S
    sp = x[r:r + Z]
    dsp = x[r + Z:r + Z * (P + 1)].reshape(P, Z)
    C = x[r + Z * (P + 1):r + Z * (P + 1) + P * S_].reshape(P, S_)
    return x[:r], sp, dsp, C, x[r + Z * (P + 1) + P * S_:]


def _linear_equivalent(m, base, a, const):
    """The linear MTP with E_i = species[t] + const + sum_p a_p Q_p."""
    lin = O.Model(base)
    rad, sp, dsp, C, _ = _coeff_blocks(m, m.coeffs)
    lin.coeffs = np.concatenate([rad, sp + const + a @ dsp, a @ C])
    return lin


def _assert_same_efs(m, lin, s, tol=1e-12):
    E, F, St, se = efs_of(m, s)
    El, Fl, Sl, sel = efs_of(lin, s)
    assert rel_err(E, El) < tol and rel_err(se, sel) < tol
    assert rel_err(F, Fl) < tol and rel_err(St, Sl) < tol


def test_li_head_is_a_linear_mtp():
    base = base_text()
    m = O.Model(head_text("mtp_m_li", base=base))
    _assert_same_efs(m, _linear_equivalent(m, base, np.array([1.0]), 0.0), structure())


def test_q2_head_without_quadratic_terms_is_a_linear_mtp():
    base = base_text()
    m = O.Model(head_text("mtp_m_q2", base=base))
    x = m.coeffs
    x[-5:] = [0.7, -1.3, 0.0, 0.0, 0.0]
    m.coeffs = x
    _assert_same_efs(m, _linear_equivalent(m, base, np.array([0.7, -1.3]), 0.0), structure())


def test_q2_head_closed_form():
    """E_i = species + c0 x + c1 y + c2 x^2 + c3 y^2 + c4 x y over the
    descriptors evaluated from the linear oracle's site energies."""
    base = base_text()
    m = O.Model(head_text("mtp_m_q2", base=base))
    rad, sp, dsp, C, c = _coeff_blocks(m, m.coeffs)
    s = structure()
    q = []
    for p in range(2):
        lin = O.Model(base)
        lin.coeffs = np.concatenate([rad, dsp[p], C[p]])
        q.append(efs_of(lin, s)[3])
    x, y = q
    want = sp[s.types] + c[0] * x + c[1] * y + c[2] * x * x + c[3] * y * y + c[4] * x * y
    assert rel_err(efs_of(m, s)[3], want) < 1e-13


def test_fs_head_closed_form():
    base = base_text()
    m = O.Model(head_text("mtp_m_fs", base=base))
    rad, sp, dsp, C, c = _coeff_blocks(m, m.coeffs)
    s = structure()
    q = []
    for p in range(2):
        lin = O.Model(base)
        lin.coeffs = np.concatenate([rad, dsp[p], C[p]])
        q.append(efs_of(lin, s)[3])
    want = sp[s.types] + q[0] + c[0] * np.arcsinh(q[1])
    assert rel_err(efs_of(m, s)[3], want) < 1e-13


def test_nn1_linear_activation_is_a_linear_mtp():
    base = base_text()
    m = O.Model(head_text("mtp_m_n1", 5, 0, "LINEAR", base=base))
    P, h1 = m.P, 5
    c = _coeff_blocks(m, m.coeffs)[4]
    W, out, b1 = c[:P * h1].reshape(h1, P), c[P * h1:P * h1 + h1], c[P * h1 + h1:]
    _assert_same_efs(m, _linear_equivalent(m, base, out @ W, out @ b1), structure())


def test_nn2_relu_in_its_linear_region_is_a_linear_mtp():
    """Large positive biases keep every preactivation positive, where RELU
    is the identity."""
    base = base_text()
    m = O.Model(head_text("mtp_m_n2", 4, 3, "RELU", base=base))
    P, h1, h2 = m.P, 4, 3
    x = m.coeffs
    n0 = x.size - m.Mc
    c = x[n0:].copy()
    W1 = c[:P * h1].reshape(h1, P)
    c[P * h1:P * h1 + h1] = 50.0                       # b1
    W2 = c[P * h1 + h1:P * h1 + h1 + h1 * h2].reshape(h2, h1)
    c[P * h1 + h1 + h1 * h2:P * h1 + h1 + h1 * h2 + h2] = 50.0   # b2
    out = c[-h2:]
    x[n0:] = c
    m.coeffs = x
    b1 = np.full(h1, 50.0)
    b2 = np.full(h2, 50.0)
    a = out @ W2 @ W1
    const = out @ (W2 @ b1 + b2)
    _assert_same_efs(m, _linear_equivalent(m, base, a, const), structure(), 1e-11)


@pytest.mark.parametrize("case", [CASES[1], CASES[2], CASES[3], CASES[5], CASES[7], CASES[9]],
                         ids=case_id)
def test_forces_and_virial_are_energy_derivatives(case):
    head, h1, h2, act = case
    m = O.Model(head_text(head, h1, h2, act, seed=45))
    s = structure(46)
    E, F, St, se = efs_of(m, s)
    assert abs(E - se.sum()) < 1e-12 * np.abs(se).sum()
    assert np.abs(F.sum(axis=0)).max() < 1e-11 * np.abs(F).max()
    h = 1e-5
    for i in (0, 5, 17):
        for a in range(3):
            p1, p2 = s.pos.copy(), s.pos.copy()
            p1[i, a] += h
            p2[i, a] -= h
            fd = -(efs_of(m, s, p1)[0] - efs_of(m, s, p2)[0]) / (2 * h)
            assert abs(F[i, a] - fd) < 1e-7 * max(1.0, np.abs(F).max())
    h = 1e-6
    for a, b in [(0, 0), (1, 2), (2, 1)]:
        eps = np.zeros((3, 3))
        eps[a, b] = h
        sp = S.Structure(s.cell @ (np.eye(3) + eps), s.pos @ (np.eye(3) + eps), s.types, s.pbc)
        sm = S.Structure(s.cell @ (np.eye(3) - eps), s.pos @ (np.eye(3) - eps), s.types, s.pbc)
        dE = (efs_of(m, sp)[0] - efs_of(m, sm)[0]) / (2 * h)
        assert abs(St[b, a] + dE) < 1e-6 * max(1.0, np.abs(St).max())


@pytest.mark.parametrize("case", CASES[:5] + CASES[8:9], ids=case_id)
def test_energy_path_matches_efs(case):
    head, h1, h2, act = case
    m = O.Model(head_text(head, h1, h2, act))
    s = structure()
    pos = O.wrap(s.cell, s.pbc, s.pos)
    nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, m.cutoff)
    E, _, _, se = O.efs(m, nb)
    Ee, see = O.energy(m, nb)
    assert rel_err(Ee, E) < 1e-14 and rel_err(see, se) < 1e-14


def test_oracle_refuses_training_of_heads():
    m = O.Model(head_text("mtp_m_q2"))
    s = structure()
    pos = O.wrap(s.cell, s.pbc, s.pos)
    nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, m.cutoff)
    with pytest.raises(ValueError):
        O.efs_components(m, nb)


# ------------------------------------------------- the product's reader --

@pytest.mark.parametrize("form", ["both", "tag", "footer"])
@pytest.mark.parametrize("case", CASES, ids=case_id)
def test_product_reads_heads_like_the_oracle(case, form):
    head, h1, h2, act = case
    text = head_text(head, h1, h2, act, form)
    m = O.Model(text)
    got = capi.parse_model_head(text)
    assert got == dict(head=head, q=m.P, hidden1=h1, hidden2=h2,
                       activation=act if head in ("mtp_m_n1", "mtp_m_n2") else "TANH",
                       model_coeffs_count=m.Mc)
    info, coef = capi.parse_model_text(text)
    assert info["ncoef"] == m.ncoef
    assert np.array_equal(coef, m.coeffs)


def test_linear_mtp_has_no_head():
    text = base_text()
    assert capi.parse_model_head(text) == dict(head="linear", q=1, hidden1=0, hidden2=0,
                                               activation="TANH", model_coeffs_count=0)


def _footer(head, extra=()):
    return ["# mtp_model = " + head] + list(extra)


# (text transformation, error text of the reference reader, runtime/mtp/
# mlip.cpp:70-296 and tools/mtp_metadata.h)
def _bad_cases():
    n1 = head_text("mtp_m_n1", 4, 0, "TANH", "footer")
    q2 = head_text("mtp_m_q2", form="footer")
    q2t = head_text("mtp_m_q2", form="tag")
    n2 = head_text("mtp_m_n2", 4, 3, "TANH", "footer")
    lin = base_text()
    return [
        ("conflict", n1.replace("# mtp_model = mtp_m_n1", "# mtp_model = mtp_m_n1\nmtp_model = mtp_m_q2"),
         "conflicting JSON/footer metadata for mtp_model"),
        ("tag-footer-conflict", head_text("mtp_m_n1", 4, 0, "TANH", "both").replace(
            "# mtp_hidden1 = 4", "# mtp_hidden1 = 5"), "conflicting JSON/footer metadata for mtp_hidden1"),
        ("unknown-model", q2.replace("mtp_m_q2", "mtp_m_q3"), "invalid value for mtp_model: 'mtp_m_q3'"),
        ("q2-q3", q2.replace("# mtp_descriptor_count = 2", "# mtp_descriptor_count = 3"),
         "analytic q2/fs models require descriptor_count 2"),
        ("nn2-linear", n2.replace("# mtp_activation = TANH", "# mtp_activation = linear"),
         "NN2 does not support LINEAR activation"),
        ("no-model-coeffs", "\n".join(l for l in q2.split("\n") if not l.startswith("model_coeffs")),
         "nonlinear mtp_model requires a model_coeffs section"),
        ("linear-with-model-coeffs", lin + "model_coeffs = {1.0}\n",
         "model_coeffs is present but mtp_model metadata is missing"),
        ("q2-hidden", q2 + "# mtp_hidden1 = 4\n", "non-neural models require zero hidden dimensions"),
        ("n1-hidden2", n1.replace("# mtp_hidden2 = 0", "# mtp_hidden2 = 2"), "NN1 requires zero hidden2"),
        ("n1-count", n1.replace("# mtp_model_coeffs_count = 20", "# mtp_model_coeffs_count = 7"),
         "neural model coefficient count does not match dimensions"),
        ("bad-int", n1.replace("# mtp_hidden1 = 4", "# mtp_hidden1 = 4x"),
         "invalid value for mtp_hidden1: '4x'"),
        ("bad-activation", n1.replace("# mtp_activation = TANH", "# mtp_activation = gelu"),
         "invalid value for mtp_activation: 'GELU'"),
        ("n1-zero-hidden", n1.replace("# mtp_hidden1 = 4", "# mtp_hidden1 = 0"),
         "neural model requires positive descriptor_count and hidden1"),
        ("li-count", head_text("mtp_m_li", form="footer").replace(
            "# mtp_model_coeffs_count = 0", "# mtp_model_coeffs_count = 3"),
         "linear MTP-M requires one descriptor and no head coefficients"),
        ("long-range", n1 + "les_kernel = coulomb\n",
         "long-range payload is unsupported by the short-range runtime"),
        ("tag-q3", q2t.replace('"q":2', '"q":3'), "analytic head requires q=2"),
        ("tag-ordinary-head", q2t.replace('"type":"MTP_M"', '"type":"MTP"'),
         "ordinary MTP cannot declare an external head"),
        ("tag-nn-for-q2", q2t.replace('"q":2', '"nn":{"activation":"TANH","hidden_layers":[3]},"q":2'),
         "nn.hidden_layers conflicts with model"),
    ]


BAD = _bad_cases()


def _ref_load_error(text, workdir):
    """The reference reader's verdict on a potential (oracle/_ref/mtpm_ref
    over one isolated atom): (exit status, stderr)."""
    mpath = os.path.join(workdir, "bad.mtp")
    with open(mpath, "w") as f:
        f.write(text)
    fin = os.path.join(workdir, "one_in.bin")
    with open(fin, "wb") as f:
        f.write(np.int32(2).tobytes() + np.int32(1).tobytes() + np.int32(1).tobytes())
        f.write(np.float64(5.0).tobytes() + np.zeros(3).tobytes())
        f.write(np.int32(0).tobytes() + np.int32(0).tobytes())
    r = subprocess.run([os.path.join(O.REF_DIR, "mtpm_ref"), mpath, fin,
                        os.path.join(workdir, "one_out.bin")], capture_output=True, text=True)
    return r.returncode, r.stderr


@pytest.mark.parametrize("name,text,msg", BAD, ids=[b[0] for b in BAD])
def test_product_refuses_bad_metadata(name, text, msg):
    with pytest.raises(capi.MtpxError) as e:
        capi.parse_model_head(text)
    assert msg in str(e.value)


@needs_ref
@pytest.mark.parametrize("name,text,msg", BAD, ids=[b[0] for b in BAD])
def test_reference_reader_refuses_the_same(workdir, name, text, msg):
    rc, err = _ref_load_error(text, workdir)
    assert rc != 0 and msg in err, err


@needs_ref
def test_reference_reader_accepts_the_good_forms(workdir):
    for head, h1, h2, act in CASES:
        for form in ("both", "tag", "footer"):
            rc, err = _ref_load_error(head_text(head, h1, h2, act, form), workdir)
            assert rc == 0, (head, act, form, err)


@pytest.mark.parametrize("name", ["n1-count", "tag-q3", "unknown-model", "no-model-coeffs"])
def test_oracle_refuses_bad_metadata(name):
    text = dict((b[0], b[1]) for b in BAD)[name]
    with pytest.raises(ValueError):
        O.Model(text)


def test_short_model_coeffs_section_is_refused():
    text = head_text("mtp_m_n1", 4, 0, "TANH")
    lines = text.split("\n")
    k = next(i for i, l in enumerate(lines) if l.startswith("model_coeffs"))
    lines[k] = lines[k].rsplit(",", 1)[0] + "}"
    with pytest.raises(capi.MtpxError) as e:
        capi.parse_model_head("\n".join(lines))
    assert "missing model coefficient" in str(e.value)


# ------------------------------------------------- the product's writer --

@pytest.mark.parametrize("case", CASES, ids=case_id)
def test_save_round_trip(case):
    """PotMTP_M::Save (potential_mtp_m.h:2256-2336): the saved text reads
    back to the same head and the same coefficients bit for bit, declares
    the head in the tag (model_metadata, :1564-1589) and in the "# mtp_*"
    lines, and saving it again gives the same text."""
    head, h1, h2, act = case
    text = head_text(head, h1, h2, act, "footer")
    out = capi.format_model_text(text)
    assert capi.format_model_text(out) == out
    assert capi.parse_model_head(out) == capi.parse_model_head(text)
    assert np.array_equal(capi.parse_model_text(out)[1], capi.parse_model_text(text)[1])
    tag = next(l for l in out.split("\n") if l.startswith("potential_tag"))
    m = O.Model(text)
    nn = ""
    if head == "mtp_m_n1":
        nn = ',"nn":{"activation":"%s","hidden_layers":[%d]}' % (act, h1)
    elif head == "mtp_m_n2":
        nn = ',"nn":{"activation":"%s","hidden_layers":[%d,%d]}' % (act, h1, h2)
    assert tag == ('potential_tag = {"model":"%s","model_coeffs_count":%d%s,"q":%d,'
                   '"schema":"gpml.mtp.metadata","type":"MTP_M","version":1}'
                   % (head, m.Mc, nn, m.P))
    assert "# mtp_model = %s\n# mtp_descriptor_count = %d\n" % (head, m.P) in out
    assert ("model_coeffs = {" in out) and out.count("\nmodel_coeffs") == 1
    # the oracle reads the saved text to the same numbers
    assert np.array_equal(O.Model(out).coeffs, m.coeffs)


@needs_ref
def test_saved_text_evaluates_the_same_in_the_reference(workdir):
    text = head_text("mtp_m_n2", 4, 3, "SIGMOID", "footer")
    out = capi.format_model_text(text)
    m = O.Model(text)
    s = structure()
    pos = O.wrap(s.cell, s.pbc, s.pos)
    nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, m.cutoff)
    a = O.ref_mlip_efs(text, nb, s.types, m.cutoff, workdir, m.Z, binary="mtpm_ref")
    b = O.ref_mlip_efs(out, nb, s.types, m.cutoff, workdir, m.Z, binary="mtpm_ref")
    for x, y in zip(a, b):
        assert np.array_equal(x, y)
