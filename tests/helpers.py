"""Shared helpers of the parity tests: structures, oracle runs, comparisons."""
import numpy as np

import oracle as O
from mtpx import synth as S


def rel_err(a, b):
    """max |a - b| / max |b| (per quantity; exact zero reference -> absolute)."""
    a = np.asarray(a, float)
    b = np.asarray(b, float)
    scale = np.max(np.abs(b)) if b.size else 0.0
    diff = np.max(np.abs(a - b)) if b.size else 0.0
    return diff / scale if scale > 0 else diff


def oracle_case(model_text, s: S.Structure):
    """Wrap (Atoms::wrap), build the BOXED lists and evaluate E/F/S on the CPU."""
    m = O.Model(model_text)
    pos = O.wrap(s.cell, s.pbc, s.pos)
    nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, m.cutoff)
    E, F, St, se = O.efs(m, nb)
    return dict(model=m, pos=pos, nb=nb, E=E, F=F, S=St, se=se)


def upload_oracle_lists(ctx, nb):
    ctx.set_neighbors(nb.offsets, nb.idx, nb.types, nb.vec, nb.dist, nb.center_types)


def assert_efs_close(got, ref, tol):
    E, F, St, se = got
    assert rel_err(E, ref["E"]) < tol, (E, ref["E"])
    assert rel_err(se, ref["se"]) < tol
    assert rel_err(F, ref["F"]) < tol, rel_err(F, ref["F"])
    assert rel_err(St, ref["S"]) < tol, (St, ref["S"])
