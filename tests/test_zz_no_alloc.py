"""Allocation-free E/F/S (mtpx_efs_noalloc) against mtpx_efs through the C ABI.

The outputs go to device buffers the test owns (hipMalloc through the HIP
runtime the library links); the library's scratch is its static per-GPU
array.  Two
calls in a row, the second on a smaller structure, each checked against the
allocating entry point's fast path at 1e-10 relative (both sum the force
reactions with atomics, so the order of additions differs)."""
import numpy as np
import pytest

from helpers import DeviceArray, rel_err
from mtpx import capi
from mtpx import synth as S

pytestmark = pytest.mark.gpu
TOL = 1e-10


def _noalloc(ctx, n):
    # stale contents: every output must be written by the call
    f = DeviceArray(np.full((max(n, 1), 3), 123.0))
    se = DeviceArray(np.full(max(n, 1), -7.0))
    es = DeviceArray(np.full(10, 5.0))
    try:
        ctx.efs_noalloc(f.address, se.address, es.address)
        e = es.download()
        return e[0], f.download()[:n], e[1:].reshape(3, 3), se.download()[:n]
    finally:
        for b in (f, se, es):
            b.free()


def test_noalloc_matches_allocating_entry_point():
    ctx = capi.Context(0)
    try:
        for reps in [(6, 6, 6), (3, 3, 2)]:  # the second call on a smaller cell
            text, s = S.scaled_inference(2, reps)
            pos = capi.wrap(s.cell, s.pbc, s.pos)
            ctx.load_model_text(text)
            ctx.build_neighbors(s.cell, s.pbc, pos, s.types, 5.0)
            n, _ = ctx.neighbor_count()
            E, F, St, se = ctx.efs()
            Ea, Fa, Sa, sea = _noalloc(ctx, n)
            assert rel_err(Ea, E) < TOL and rel_err(sea, se) < TOL
            assert rel_err(Fa, F) < TOL and rel_err(Sa, St) < TOL
    finally:
        ctx.close()
