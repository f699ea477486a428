"""GPM bundles on the device: a context loaded from a bundle
(mtpx_load_model_gpm) evaluates the source model's E/F/S as the oracle does
(1e-11 relative), saves a bundle of its current coefficients
(mtpx_save_model_gpm), and mtpx_calc_efs takes a bundle for --pot."""
import os
import subprocess

import numpy as np
import pytest

import oracle as O
from helpers import assert_efs_close, oracle_case, rel_err, upload_oracle_lists
from mtpx import capi
from mtpx import synth as S
from test_gpm import MODELS
from test_mtpm import structure

pytestmark = pytest.mark.gpu
TOL = 1e-11


@pytest.mark.parametrize("kind", ["chebyshev", "split-configurable", "level16", "mtp_m_n2"])
def test_bundle_loads_and_evaluates(ctx, kind):
    text = MODELS[kind]()
    ref = oracle_case(text, structure(90))
    ctx.load_model_gpm(capi.gpm_from_text(text, zstd_level=1 if kind == "level16" else 0))
    upload_oracle_lists(ctx, ref["nb"])
    assert_efs_close(ctx.efs(), ref, TOL)
    assert_efs_close(ctx.efs(deterministic=True), ref, TOL)


def test_save_bundle_after_coefficient_update(ctx):
    text = MODELS["mtp_m_q2"]()
    m = O.Model(text)
    ctx.load_model_text(text)
    x = ctx.get_coeffs() * 1.01
    ctx.set_coeffs(x)
    data = ctx.save_model_gpm()
    assert np.array_equal(capi.parse_model_gpm(data)[1], x)
    m.coeffs = x
    s = structure(91)
    pos = O.wrap(s.cell, s.pbc, s.pos)
    nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, m.cutoff)
    E, F, St, se = O.efs(m, nb)
    ctx.load_model_gpm(data)
    upload_oracle_lists(ctx, nb)
    assert_efs_close(ctx.efs(), dict(E=E, F=F, S=St, se=se), TOL)


def test_calc_efs_reads_a_bundle(tmp_path):
    from test_calc_efs_gpu import EXE, _read_cfg, _write_cfg
    if not os.path.exists(EXE):
        pytest.fail("mtpx_calc_efs is not built")
    text = MODELS["split-configurable"]()
    pot = tmp_path / "pot.gpm"
    pot.write_bytes(capi.gpm_from_text(text))
    structs = [structure(92), structure(93, (2, 2, 3))]
    cfg = tmp_path / "in.cfg"
    _write_cfg(cfg, structs)
    out = tmp_path / "out.cfg"
    r = subprocess.run([EXE, "--pot", str(pot), "--in", str(cfg), "--out", str(out), "--lossless"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    for s, got in zip(structs, _read_cfg(out)):
        ref = oracle_case(text, s)
        c = got["cols"]
        assert rel_err(got["energy"], ref["E"]) < 1e-10
        assert rel_err(np.stack([c["fx"], c["fy"], c["fz"]], 1), ref["F"]) < 1e-10
