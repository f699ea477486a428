"""mtpx_calc_efs, the calc_efs front end (apps/calc_efs.cpp:179-389) over
the C ABI: configurations in the text MLIP format or a VASP POSCAR
(GPIO::read_vasp_poscar, io/gpio_read_vasp.cpp:1108-1234) in, the
configurations with the device's energy, forces, stress and site energies
out, against the oracle's getEFS of each structure.  POSCAR element names
become species through an index file, the element order the potential
declares, or the periodic table (GPIO::install_species_map,
io/gpio.cpp:103-200).

Tolerances: 1e-10 relative with --lossless (numbers that read back to the
same doubles); the fixed-width form carries 8 significant digits, so 1e-7
relative to the largest magnitude there."""
import os
import subprocess

import numpy as np
import pytest

import oracle as O
from helpers import rel_err
from mtpx import synth as S

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "imr-mlp_amd", "lib", "mtpx_calc_efs")


def _structures():
    rng = S.rng_for(1201)
    out = []
    for k, (kind, reps, a) in enumerate([("bcc", (3, 3, 3), 2.87), ("fcc", (2, 2, 3), 3.6),
                                         ("bcc", (2, 3, 2), 2.9)]):
        s = S.displace(S.strain(S.lattice(kind, reps, a), rng, 0.02), rng, 0.1)
        s.types = (S.uniform(rng, s.n) * 2).astype(np.int32)
        out.append(s)
    # a cluster: no Supercell in the file
    s = S.displace(S.lattice("fcc", (2, 2, 2), 3.6), rng, 0.1)
    s.types = (S.uniform(rng, s.n) * 2).astype(np.int32)
    s.cell = np.zeros((3, 3))
    s.pbc = np.zeros(3, np.int32)
    out.append(s)
    return out


def _write_cfg(path, structs):
    with open(path, "w") as f:
        for k, s in enumerate(structs):
            f.write("BEGIN_CFG\n Size\n    %d\n" % s.n)
            if s.pbc.any():
                f.write(" Supercell\n")
                for r in s.cell:
                    f.write("  %.17g %.17g %.17g\n" % tuple(r))
            f.write(" AtomData:  id type       cartes_x      cartes_y      cartes_z   charge_q\n")
            for i in range(s.n):
                f.write("  %d %d %.17g %.17g %.17g %g\n" % ((i + 1, s.types[i]) + tuple(s.pos[i])
                                                           + (0.5 * i,)))
            f.write(" Energy\n  -1.0\n PlusStress:  xx  yy  zz  yz  xz  xy\n 1 2 3 4 5 6\n")
            f.write(" Feature   EFS_by  test%d\nEND_CFG\n\n" % k)


def _read_cfg(path):
    """(cells, AtomData columns by name, energies, stresses [xx yy zz yz xz xy],
    feature lines) of every configuration."""
    out = []
    lines = open(path).read().splitlines()
    k = 0
    while k < len(lines):
        if "BEGIN_CFG" not in lines[k]:
            k += 1
            continue
        n = int(lines[k + 2].split()[0])
        assert "Supercell" in lines[k + 3]
        cell = np.array([[float(v) for v in lines[k + 4 + r].split()] for r in range(3)])
        head = lines[k + 7].split()[1:]
        rows = np.array([[float(v) for v in lines[k + 8 + i].split()] for i in range(n)])
        cols = {h: rows[:, j] for j, h in enumerate(head)}
        k += 8 + n
        cfg = dict(cell=cell, cols=cols, widths=[len(lines[k - n].split()[2])], features=[])
        while "END_CFG" not in lines[k]:
            t = lines[k].split()
            if t[0] == "Energy":
                cfg["energy"] = float(lines[k + 1])
                k += 1
            elif t[0] == "PlusStress:":
                cfg["stress"] = np.array([float(v) for v in lines[k + 1].split()])
                k += 1
            elif t[0] == "Feature":
                cfg["features"].append(lines[k])
            k += 1
        out.append(cfg)
    return out


def _oracle(model, s):
    pos = O.wrap(s.cell, s.pbc, s.pos) if s.pbc.any() else s.pos
    nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, model.cutoff)
    E, F, St, se = O.efs(model, nb)
    return pos, E, F, St, se


@pytest.fixture(scope="module")
def run_case(tmp_path_factory):
    if not os.path.exists(EXE):
        pytest.fail("mtpx_calc_efs is not built")
    d = tmp_path_factory.mktemp("calc_efs")
    text = S.random_model("shapeev-16.mtp", 2, 8, 1.9, 5.0, -0.05, 0.05, S.rng_for(1202))
    mtp = d / "pot.mtp"
    mtp.write_text(text)
    structs = _structures()
    cfg = d / "in.cfg"
    _write_cfg(cfg, structs)

    def run(*flags):
        out = d / ("out%d.cfg" % len(list(d.iterdir())))
        r = subprocess.run([EXE, "--pot", str(mtp), "--in", str(cfg), "--out", str(out)]
                           + list(flags), capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stderr
        return _read_cfg(out), r.stderr
    return O.Model(text), structs, run


def test_lossless_output_matches_oracle(run_case):
    model, structs, run = run_case
    got, log = run("--lossless", "--gpu-batch-structures", "2")
    assert "2 chunk(s)" in log and len(got) == len(structs)
    for s, g in zip(structs, got):
        pos, E, F, St, se = _oracle(model, s)
        c = g["cols"]
        assert np.array_equal(c["id"], np.arange(1, s.n + 1))
        assert np.array_equal(c["type"], s.types)
        # positions come back wrapped, as Atoms::wrap leaves them
        assert np.array_equal(np.stack([c["cartes_x"], c["cartes_y"], c["cartes_z"]], 1), pos)
        assert np.array_equal(c["charge_q"], 0.5 * np.arange(s.n))
        assert rel_err(g["energy"], E) < 1e-10
        assert rel_err(np.stack([c["fx"], c["fy"], c["fz"]], 1), F) < 1e-10
        assert rel_err(c["site_en"], se) < 1e-10
        voigt = np.array([St[0, 0], St[1, 1], St[2, 2], St[1, 2], St[0, 2], St[0, 1]])
        assert rel_err(g["stress"], voigt) < 1e-10
        assert np.array_equal(g["cell"], s.cell)
        assert len(g["features"]) == 1 and "EFS_by" in g["features"][0]


def test_fixed_width_and_energy_only(run_case):
    model, structs, run = run_case
    got, _ = run()
    for s, g in zip(structs, got):
        _, E, F, St, se = _oracle(model, s)
        c = g["cols"]
        assert g["widths"][0] <= 15
        assert abs(g["energy"] - E) <= 1e-7 * abs(E)
        assert rel_err(np.stack([c["fx"], c["fy"], c["fz"]], 1), F) < 1e-7
    got, _ = run("--energy-only", "--gpu-batch-atoms", "100")
    for s, g in zip(structs, got):
        _, E, _, _, _ = _oracle(model, s)
        assert abs(g["energy"] - E) <= 1e-7 * abs(E)
        assert "fx" not in g["cols"] and "site_en" not in g["cols"] and "stress" not in g
    got, _ = run("--no-site-energy", "--lossless", "--deterministic")
    assert "site_en" not in got[0]["cols"] and "fx" in got[0]["cols"]


# ---- POSCAR ----------------------------------------------------------------

def _poscar(path, s, names, direct=True, scale=1.0, selective=False, cell_scale=1.0):
    """POSCAR of structure s (atoms grouped by species, as POSCAR keeps
    them), the cell written divided by cell_scale.  Returns the structure
    in that order."""
    order = np.argsort(s.types, kind="stable")
    pos, types = s.pos[order], s.types[order]
    cell = s.cell / cell_scale
    with open(path, "w") as f:
        f.write("synthetic test structure\n%.17g\n" % float(scale))
        for r in cell:
            f.write("  %.17g %.17g %.17g\n" % tuple(r))
        present = sorted(set(types.tolist()))
        f.write("  " + " ".join(names[t] for t in present) + "\n")
        f.write("  " + " ".join(str(int((types == t).sum())) for t in present) + "\n")
        if selective:
            f.write("Selective dynamics\n")
        f.write("Direct\n" if direct else "Cartesian\n")
        frac = pos @ np.linalg.inv(s.cell)
        for i in range(s.n):
            v = frac[i] if direct else pos[i]
            f.write("  %.17g %.17g %.17g%s\n" % (tuple(v) + (" T T F" if selective else "",)))
    st = S.Structure(s.cell.copy(), pos.copy(), types.astype(np.int32), s.pbc.copy())
    if direct:
        # the reader's Cartesian positions: row vector times the cell, summed
        # left to right
        c = s.cell
        st.pos = np.stack([(frac[:, 0] * c[0, b] + frac[:, 1] * c[1, b]) + frac[:, 2] * c[2, b]
                           for b in range(3)], 1)
    return st


def _poscar_case(tmp_path, text, s, names, flags=(), **kw):
    mtp = tmp_path / "pot.mtp"
    mtp.write_text(text)
    st = _poscar(tmp_path / "POSCAR", s, names, **kw)
    out = tmp_path / "out.cfg"
    r = subprocess.run([EXE, "--pot", str(mtp), "--in", str(tmp_path / "POSCAR"), "--out",
                        str(out), "--lossless"] + list(flags), capture_output=True, text=True,
                       timeout=120, cwd=str(tmp_path))
    return st, r, out


def _check_against_oracle(model, st, out, tol=1e-10):
    got = _read_cfg(out)
    assert len(got) == 1
    g = got[0]
    pos, E, F, St, se = _oracle(model, st)
    c = g["cols"]
    assert np.array_equal(c["type"], st.types)
    assert np.allclose(np.stack([c["cartes_x"], c["cartes_y"], c["cartes_z"]], 1), pos,
                       rtol=0, atol=1e-12)
    assert rel_err(g["energy"], E) < tol
    assert rel_err(np.stack([c["fx"], c["fy"], c["fz"]], 1), F) < tol
    voigt = np.array([St[0, 0], St[1, 1], St[2, 2], St[1, 2], St[0, 2], St[0, 1]])
    assert rel_err(g["stress"], voigt) < tol


def _two_species_structure(seed):
    rng = S.rng_for(seed)
    s = S.displace(S.strain(S.lattice("fcc", (2, 2, 2), 3.6), rng, 0.03), rng, 0.1)
    s.types = (S.uniform(rng, s.n) * 2).astype(np.int32)
    return s


def test_poscar_direct_with_index_map(tmp_path):
    """Direct coordinates, element names mapped by index.map (found in the
    working directory, as the reference's default): species = line order."""
    text = S.random_model("shapeev-16.mtp", 2, 8, 1.9, 5.0, -0.05, 0.05, S.rng_for(1203))
    (tmp_path / "index.map").write_text("Al 1.43\nNi 1.24\n")
    s = _two_species_structure(1204)
    st, r, out = _poscar_case(tmp_path, text, s, ["Al", "Ni"])
    assert r.returncode == 0, r.stderr
    _check_against_oracle(O.Model(text), st, out)


def test_poscar_cartesian_selective_volume_scale(tmp_path):
    """Cartesian coordinates after a Selective dynamics line (its flags are
    read and dropped) and a negative scale, which sets the cell volume; an
    index file named on the command line."""
    text = S.random_model("shapeev-16.mtp", 2, 8, 1.9, 5.0, -0.05, 0.05, S.rng_for(1205))
    (tmp_path / "elements.txt").write_text("Ni\nAl\n")
    s = _two_species_structure(1206)
    vol = abs(np.linalg.det(s.cell))
    st, r, out = _poscar_case(tmp_path, text, s, ["Ni", "Al"],
                              flags=("--index", "elements.txt", "--input-format", "POSCAR"),
                              direct=False, selective=True, scale=-vol, cell_scale=1.25)
    assert r.returncode == 0, r.stderr
    # the cell comes back scaled to the volume: (vol / (vol / 1.25^3))^(1/3) = 1.25
    g = _read_cfg(out)[0]
    assert np.allclose(g["cell"], s.cell, rtol=1e-13, atol=1e-13)
    st.cell = g["cell"]
    _check_against_oracle(O.Model(text), st, out)


def test_poscar_species_from_model_elements(tmp_path):
    """Without an index file the element order the potential declares (its
    potential_tag "elements") maps the names; an element outside it is
    refused."""
    tag = ('{"elements":["Ta","W"],"model":"linear","schema":"gpml.mtp.metadata",'
           '"type":"MTP","version":1}')
    text = S.random_model("shapeev-16.mtp", 2, 8, 1.9, 5.0, -0.05, 0.05, S.rng_for(1207),
                          tag=tag)
    s = _two_species_structure(1208)
    st, r, out = _poscar_case(tmp_path, text, s, ["Ta", "W"])
    assert r.returncode == 0, r.stderr
    _check_against_oracle(O.Model(text), st, out)
    st, r, _ = _poscar_case(tmp_path, text, s, ["Ta", "Mo"])
    assert r.returncode != 0 and "element Mo is not in the species map" in r.stderr
    # a named index file that is missing: the declared order is used, with a warning
    st, r, out = _poscar_case(tmp_path, text, s, ["Ta", "W"], flags=("--index", "none.map"))
    assert r.returncode == 0 and "using the element order declared by the model" in r.stderr


def test_poscar_periodic_table_and_errors(tmp_path):
    """No index file and no declared elements: species are atomic numbers
    (X = 0, H = 1), so a two-species model takes X and H; a named index file
    that is missing is then an error; a bad coordinate mode is refused."""
    text = S.random_model("shapeev-16.mtp", 2, 8, 1.9, 5.0, -0.05, 0.05, S.rng_for(1209))
    s = _two_species_structure(1210)
    s.types[:] = 1
    st, r, out = _poscar_case(tmp_path, text, s, ["X", "H"])
    assert r.returncode == 0, r.stderr
    assert "using the periodic table" in r.stderr
    _check_against_oracle(O.Model(text), st, out)
    _, r, _ = _poscar_case(tmp_path, text, s, ["X", "H"], flags=("--index", "missing.map"))
    assert r.returncode != 0 and "does not declare an element order" in r.stderr
    (tmp_path / "POSCAR").write_text("x\n1.0\n5 0 0\n0 5 0\n0 0 5\nH\n1\nQ\n0 0 0\n")
    r = subprocess.run([EXE, "--pot", str(tmp_path / "pot.mtp"), "--in",
                        str(tmp_path / "POSCAR"), "--out", str(tmp_path / "o.cfg")],
                       capture_output=True, text=True, timeout=120, cwd=str(tmp_path))
    assert r.returncode != 0 and "unknown POSCAR format" in r.stderr


# ---- binary configurations ----------------------------------------------------

def _bin_frame(s, version=3, extras=True):
    """One frame of the binary configuration format (io/gpio_binary.h): the
    cell as Eigen stores it (column-major), positions, types, periodicity
    (version 3) and, with extras, records the reader passes over."""
    import struct
    out = [b"GPMLBIN2", struct.pack("<Ii", version, s.n)]
    out += [b"l", np.asarray(s.cell, "<f8").T.tobytes()]
    out += [b"p", np.asarray(s.pos, "<f8").tobytes(), b"t", np.asarray(s.types, "<i4").tobytes()]
    if version >= 3:
        out += [b"b", bytes(int(v) for v in s.pbc)]
    if extras:
        name = b"tag"
        out += [b"e", struct.pack("<d", -1.5), b"s", np.zeros(9).tobytes(),
                b"f", np.ones((s.n, 3)).tobytes(), b"c", np.arange(s.n, dtype="<f8").tobytes(),
                b"A", struct.pack("<i", len(name)) + name + np.zeros(s.n).tobytes(),
                b"I", struct.pack("<i", len(name)) + name + struct.pack("<i", 2)
                + np.zeros((2, s.n), "<i4").tobytes(),
                b"D", struct.pack("<i", 1) + b"g" + struct.pack("<i", 3) + np.zeros(3).tobytes(),
                b"F", struct.pack("<i", 6) + b"EFS_by" + struct.pack("<i", 3) + b"dft"]
    out.append(b"#")
    return b"".join(out)


def test_binary_configurations(run_case, tmp_path):
    """Binary frames (found by their magic): a periodic cell with every kind
    of record the reader passes over, a slab periodic along x and y, and a
    version-2 frame without periodicity flags (periodic)."""
    model, structs, _ = run_case
    rng = S.rng_for(1211)
    slab = S.displace(S.lattice("fcc", (3, 3, 2), 3.6), rng, 0.1)
    slab.types = (S.uniform(rng, slab.n) * 2).astype(np.int32)
    slab.pbc = np.array([1, 1, 0], np.int32)
    frames = [(structs[0], 3, True), (slab, 3, False), (structs[1], 2, False)]
    path = tmp_path / "in.bin"
    path.write_bytes(b"".join(_bin_frame(s, v, x) for s, v, x in frames))
    mtp = tmp_path / "pot.mtp"
    mtp.write_text(model.save_text())
    out = tmp_path / "out.cfg"
    r = subprocess.run([EXE, "--pot", str(mtp), "--in", str(path), "--out", str(out),
                        "--lossless"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    got = _read_cfg(out)
    assert len(got) == 3
    for (s, _, x), g in zip(frames, got):
        pos, E, F, St, se = _oracle(model, s)
        c = g["cols"]
        assert np.array_equal(c["type"], s.types)
        assert np.array_equal(np.stack([c["cartes_x"], c["cartes_y"], c["cartes_z"]], 1), pos)
        assert rel_err(g["energy"], E) < 1e-10
        assert rel_err(np.stack([c["fx"], c["fy"], c["fz"]], 1), F) < 1e-10
        voigt = np.array([St[0, 0], St[1, 1], St[2, 2], St[1, 2], St[0, 2], St[0, 1]])
        assert rel_err(g["stress"], voigt) < 1e-10
        assert np.array_equal(g["cell"], s.cell)
        assert len(g["features"]) == (1 if x else 0)
    # a frame with an unknown record is refused
    bad = _bin_frame(structs[0], 3, False)[:-1] + b"Z#"
    path.write_bytes(bad)
    r = subprocess.run([EXE, "--pot", str(mtp), "--in", str(path), "--out", str(out)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and "unsupported binary mlpcfg tag Z" in r.stderr
