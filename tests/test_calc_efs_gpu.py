"""mtpx_calc_efs, the calc_efs front end (apps/calc_efs.cpp:179-389) over
the C ABI: configurations in the text MLIP format in, the same
configurations with the device's energy, forces, stress and site energies
out, against the oracle's getEFS of each structure.

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
