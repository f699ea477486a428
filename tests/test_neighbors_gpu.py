"""Device neighbour lists against the oracle's restatement of the reference
BOXED builder: identical offsets, neighbour indices, species, and
displacements/distances equal bit for bit."""
import numpy as np
import pytest

import oracle as O
from mtpx import synth as S

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def nctx():
    """A context without a model: species indices are not range-checked
    against a model's species count."""
    from mtpx import capi
    c = capi.Context(0)
    yield c
    c.close()


def _structures():
    out = []
    _, s = S.workload_inference(1)
    out.append(("fcc108", s, 5.0))
    _, s = S.scaled_inference(2, (4, 3, 5))
    out.append(("fcc-strained-240", s, 5.0))
    rng = S.rng_for(400)
    for k in range(6):
        s = S.lattice("fcc", (2, 2, 2), 3.6)
        s = S.displace(S.strain(s, rng, 0.15), rng, 0.2)
        cell = s.cell.copy()
        cell[1] += 0.37 * cell[0]
        cell[2] += -0.21 * cell[1] + 0.3 * cell[0]
        s.cell = cell
        s.types = (S.uniform(rng, s.n) * 2).astype(np.int32)
        out.append(("skew%d" % k, s, 3.0 + 2.5 * rng.random()))
    # cell smaller than the cutoff: many images of the same atom in one list
    s = S.displace(S.lattice("bcc", (1, 1, 2), 2.87), rng, 0.05)
    out.append(("tiny-bcc", s, 6.0))
    for k, st in enumerate(S.training_structures(5, 2)):
        out.append(("liquid%d" % k, st, 6.0))
    # slab: periodic in x, y only
    s = S.displace(S.lattice("fcc", (3, 3, 3), 3.6), rng, 0.1)
    s.pbc = np.array([1, 1, 0], np.int32)
    out.append(("slab", s, 5.0))
    # isolated cluster
    s = S.displace(S.lattice("fcc", (2, 2, 2), 3.6), rng, 0.1)
    s.pbc = np.zeros(3, np.int32)
    out.append(("cluster", s, 5.0))
    s = S.Structure(np.eye(3) * 10, np.array([[1.0, 2.0, 3.0]]), np.zeros(1, np.int32),
                    np.ones(3, np.int32))
    out.append(("single-atom", s, 5.0))
    return out


CASES = _structures()


def _compare(got, nb):
    assert np.array_equal(got["offsets"], nb.offsets)
    assert np.array_equal(got["idx"], nb.idx)
    assert np.array_equal(got["types"], nb.types)
    assert np.array_equal(got["center_types"], nb.center_types)
    assert np.array_equal(got["vec"].view(np.uint64), nb.vec.view(np.uint64))
    assert np.array_equal(got["dist"].view(np.uint64), nb.dist.view(np.uint64))


@pytest.mark.parametrize("name,s,rc", CASES, ids=[c[0] for c in CASES])
def test_device_lists_bit_exact(nctx, name, s, rc):
    pos = O.wrap(s.cell, s.pbc, s.pos) if np.any(s.pbc) else s.pos
    nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, rc)
    nctx.build_neighbors(s.cell, s.pbc, pos, s.types, rc)
    _compare(nctx.get_neighbors(), nb)


def test_empty_structure_lists(nctx):
    nctx.build_neighbors(np.eye(3) * 5, [1, 1, 1], np.zeros((0, 3)), np.zeros(0), 5.0)
    got = nctx.get_neighbors()
    assert got["offsets"].tolist() == [0] and len(got["idx"]) == 0


def test_full_size_workload2_lists_bit_exact(nctx):
    model_text, s = S.workload_inference(2)
    pos = O.wrap(s.cell, s.pbc, s.pos)
    nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, 5.0)
    nctx.build_neighbors(s.cell, s.pbc, pos, s.types, 5.0)
    _compare(nctx.get_neighbors(), nb)
    counts = np.diff(nb.offsets)
    assert 40 <= counts.mean() <= 55


def test_one_pass_and_counted_builds_agree():
    """The builder counts the lists on a context's first build and, on the
    next builds, writes them in one pass into bins sized from the longest
    list seen (plus a quarter and 8); a list that outgrows its bin sends the
    build back through the counting pass.  A fresh context walks every path:
    counted (first build), one pass (same cell), overflow then counted (a
    cutoff of 7 gives lists about 2.7 times longer), one pass at the longer
    cutoff, one pass back at the shorter one.  Every result is the oracle's
    lists bit for bit."""
    from mtpx import capi
    _, s = S.workload_inference(1)
    pos = O.wrap(s.cell, s.pbc, s.pos)
    ref = {rc: O.Neighbors.build(s.cell, s.pbc, pos, s.types, rc) for rc in (5.0, 7.0)}
    longest = int(np.diff(ref[5.0].offsets).max())
    assert int(np.diff(ref[7.0].offsets).max()) > longest + longest // 4 + 8
    c = capi.Context(0)
    try:
        for rc in (5.0, 5.0, 7.0, 7.0, 5.0):
            c.build_neighbors(s.cell, s.pbc, pos, s.types, rc)
            _compare(c.get_neighbors(), ref[rc])
    finally:
        c.close()


def _rel(a, b):
    a, b = np.asarray(a, float), np.asarray(b, float)
    return np.abs(a - b).max() / max(np.abs(b).max(), 1e-300)


@pytest.mark.parametrize("name,s,rc", CASES, ids=[c[0] for c in CASES])
def test_mirror_assembly_matches_reaction_atomics(ctx, name, s, rc):
    """Lists built on the device carry each entry's mirror (the entry of the
    neighbour's list that points back, or for an image of the centre the
    opposite image), and E/F/S then assembles the forces from per-entry
    derivatives without atomics: the own force stored, the reactions gathered
    through the mirrors.  The same lists handed over (no mirrors) take the
    reaction atomics and, when ordered, the reverse index.  All three agree
    (1e-13), on every structure above: skewed cells, a cell smaller than the
    cutoff (many images of the centre in its own list), a slab, a cluster and
    a single atom.  The mirror assembly is bitwise repeatable."""
    text, _ = S.scaled_inference(2, (2, 2, 2))  # two species
    cut = O.Model(text).cutoff
    pos = O.wrap(s.cell, s.pbc, s.pos) if np.any(s.pbc) else s.pos
    ctx.load_model_text(text)
    ctx.build_neighbors(s.cell, s.pbc, pos, s.types % 2, cut)
    got = ctx.efs()
    again = ctx.efs(deterministic=True)
    for x, y in zip(got, again):
        assert np.array_equal(np.asarray(x).view(np.uint64), np.asarray(y).view(np.uint64))
    nb = ctx.get_neighbors()
    ctx.set_neighbors(nb["offsets"], nb["idx"], nb["types"], nb["vec"], nb["dist"],
                      nb["center_types"])
    for det in (False, True):
        ref = ctx.efs(deterministic=det)
        assert abs(got[0] - ref[0]) <= 1e-13 * max(abs(ref[0]), 1.0)
        if np.abs(ref[1]).max() > 0:
            assert _rel(got[1], ref[1]) < 1e-13
        else:
            assert np.abs(got[1]).max() < 1e-14
        assert _rel(got[2], ref[2]) < 1e-13
        assert _rel(got[3], ref[3]) < 1e-13


@pytest.mark.parametrize("chunk", ["1", "150"], ids=["chunk1", "chunk150"])
def test_mirror_assembly_of_chunked_batches(ctx, monkeypatch, chunk):
    """A batch built in chunks appends each chunk's mirrors shifted to the
    batch's entries: compute_batch on it equals compute_batch on the batch
    built in one piece (1e-13)."""
    text, _ = S.scaled_inference(2, (2, 2, 2))
    cut = O.Model(text).cutoff
    structs = []
    for _, s, _ in CASES:
        pos = O.wrap(s.cell, s.pbc, s.pos) if np.any(s.pbc) else s.pos
        structs.append(S.Structure(s.cell, pos, (s.types % 2).astype(np.int32), s.pbc))
    ctx.load_model_text(text)
    ctx.set_structures(structs, cut)
    ref = ctx.compute_batch()
    monkeypatch.setenv("MTPX_NEIGHBOR_CHUNK_ATOMS", chunk)
    ctx.set_structures(structs, cut)
    got = ctx.compute_batch()
    for x, y in zip(got, ref):
        assert _rel(x, y) < 1e-13


def test_device_lists_drive_efs(ctx):
    """Build on the device, evaluate on the device, compare with the oracle."""
    model_text, s = S.scaled_inference(2, (4, 4, 4))
    m = O.Model(model_text)
    pos = O.wrap(s.cell, s.pbc, s.pos)
    nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, m.cutoff)
    E, F, St, se = O.efs(m, nb)
    ctx.load_model_text(model_text)
    ctx.build_neighbors(s.cell, s.pbc, pos, s.types, m.cutoff)
    Eg, Fg, Sg, seg = ctx.efs()
    assert abs(Eg - E) < 1e-10 * abs(E)
    assert np.abs(Fg - F).max() < 1e-10 * np.abs(F).max()
    assert np.abs(Sg - St).max() < 1e-10 * np.abs(St).max()


def _concat(lists):
    """The lists of several structures as one batch: offsets and neighbour
    indices shifted by the atoms and entries before each structure."""
    off, idx, types, ct, vec, dist = [np.zeros(1, np.int64)], [], [], [], [], []
    a0 = p0 = 0
    for nb in lists:
        off.append(nb.offsets[1:].astype(np.int64) + p0)
        idx.append(nb.idx.astype(np.int64) + a0)
        types.append(nb.types)
        ct.append(nb.center_types)
        vec.append(nb.vec.reshape(-1, 3))
        dist.append(nb.dist)
        a0 += len(nb.offsets) - 1
        p0 += int(nb.offsets[-1])
    return dict(offsets=np.concatenate(off), idx=np.concatenate(idx),
                types=np.concatenate(types), center_types=np.concatenate(ct),
                vec=np.concatenate(vec), dist=np.concatenate(dist))


@pytest.mark.parametrize("chunk", [None, "1", "150"], ids=["one-chunk", "chunk1", "chunk150"])
def test_batch_lists_bit_exact(nctx, monkeypatch, chunk):
    """Every structure above in one batch (cutoff 5, an empty structure in the
    middle), built in the same launches, and in chunks of at most 1 and 150
    atoms appended in order: the concatenation of the oracle's lists."""
    if chunk is not None:
        monkeypatch.setenv("MTPX_NEIGHBOR_CHUNK_ATOMS", chunk)
    rc = 5.0
    structs = []
    for _, s, _ in CASES:
        pos = O.wrap(s.cell, s.pbc, s.pos) if np.any(s.pbc) else s.pos
        structs.append(S.Structure(s.cell, pos, s.types, s.pbc))
    structs.insert(3, S.Structure(np.eye(3) * 5, np.zeros((0, 3)), np.zeros(0, np.int32),
                                  np.ones(3, np.int32)))
    nctx.set_structures(structs, rc)
    got = nctx.get_neighbors()
    exp = _concat([O.Neighbors.build(s.cell, s.pbc, s.pos, s.types, rc) for s in structs])
    assert np.array_equal(got["offsets"], exp["offsets"])
    assert np.array_equal(got["idx"], exp["idx"])
    assert np.array_equal(got["types"], exp["types"])
    assert np.array_equal(got["center_types"], exp["center_types"])
    assert np.array_equal(got["vec"].view(np.uint64), exp["vec"].view(np.uint64))
    assert np.array_equal(got["dist"].view(np.uint64), exp["dist"].view(np.uint64))
