"""The two training workloads at their full batch sizes against the oracle.

- Linear-fit assembly (TrainLinearFast, train/train_mtp.cpp:2374-2427 over
  AddLinearFast :1289-1395): the level-16 two-species model on all 2,000
  FCC/BCC structures of 64-256 atoms (about 335k atoms, 16.1M neighbour
  entries, 1.02M rows), weights energy/force/stress 1/0.01/0.001.  G = AᵀA
  and b = Aᵀy at 1e-10 relative against the oracle's per-structure normal
  equations summed over the whole set.
- Nonlinear loss and gradient (Trainer_MTP::AccumulateGard,
  train_mtp.cpp:3039-3094): the level-20 three-species model on all 1,000
  liquid structures of 108-216 atoms (about 160k atoms, 8.6M entries),
  the trainer's default loss settings with a penalty.  Loss and gradient at
  1e-9 relative against the oracle.

Labels are a seeded reference model's E/F/S plus noise, drawn as the
benchmark draws them (they are inputs to both sides).  The oracle runs on the host's cores (at most 16
threads); each test takes some tens of seconds."""
import os
import sys
import time

import numpy as np
import pytest

import oracle as O
from helpers import rel_err
from mtpx import capi
from mtpx import synth as S

pytestmark = pytest.mark.gpu
THREADS = max(1, min(16, os.cpu_count() or 1))


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _labelled_set(ctx, config, nconf, cutoff, seed):
    """(start model text, structures, oracle lists, labels).  The labels are
    inputs to both sides; they are drawn as the benchmark draws them, from
    the reference model's E/F/S on the device."""
    ref_text, start_text = S.training_models(config)
    structs = S.training_structures(config, nconf)
    t0 = time.time()
    nbs = []
    for s in structs:
        s.pos = O.wrap(s.cell, s.pbc, s.pos)
        nbs.append(O.Neighbors.build(s.cell, s.pbc, s.pos, s.types, cutoff))
    ctx.load_model_text(ref_text)
    off = ctx.set_structures(structs, cutoff)
    E, F, St, _ = ctx.compute_batch()
    rng = S.rng_for(config, seed)
    labels = []
    for c, s in enumerate(structs):
        e, f, st = S.noisy_labels(rng, s.n, E[c], F[off[c]:off[c + 1]], St[c])
        labels.append(O.Labels(s.n, energy=e, forces=f, stress=st))
    _say("lists and labels of %d structures in %.1f s" % (nconf, time.time() - t0))
    return start_text, structs, nbs, labels


def _upload(ctx, text, structs, labels, settings, cutoff):
    ctx.load_model_text(text)
    off = ctx.set_structures(structs, cutoff)
    nconf = len(structs)
    has = np.ones((nconf, 3), np.int32)
    tF = np.concatenate([lb.forces for lb in labels])
    st = capi.LossSettings.make(*[getattr(settings, f[0]) for f in settings._fields_])
    active, wE, wF, wS = capi.loss_weights(st, off, has, tF)
    tE = np.array([lb.energy for lb in labels])
    tS = np.array([lb.stress for lb in labels])
    ctx.set_labels(active, tE, wE, tF, wF, tS, wS)
    return off


def test_linear_system_2000_structures(ctx):
    _say("linear fit, 2,000 level-16 structures: building the set")
    text, structs, nbs, labels = _labelled_set(ctx, 4, 2000, 5.0, 7)
    sets = O.LossSettings.make(weight_eng=1.0, weight_force=0.01, weight_stress=0.001)
    _upload(ctx, text, structs, labels, sets, 5.0)
    n, P = ctx.neighbor_count()
    assert P == sum(nb.P for nb in nbs)
    _say("device assembly over %d atoms, %d entries" % (n, P))
    G, b = ctx.linear_system()
    rows = int(ctx.last_linear_timings()[3])
    assert rows == sum(3 * s.n + 10 for s in structs)
    t0 = time.time()
    Go, bo = O.linear_system_batch(O.Model(text), nbs, labels, sets, THREADS)
    _say("oracle assembly in %.1f s (%d threads)" % (time.time() - t0, THREADS))
    assert rel_err(G, Go) < 1e-10
    assert rel_err(b, bo) < 1e-10
    # a second assembly is the same bits (fixed-order sums)
    G2, b2 = ctx.linear_system()
    assert np.array_equal(G2.view(np.uint64), G.view(np.uint64))
    assert np.array_equal(b2.view(np.uint64), b.view(np.uint64))


def test_loss_grad_1000_liquids(ctx):
    _say("loss+gradient, 1,000 level-20 liquids: building the set")
    text, structs, nbs, labels = _labelled_set(ctx, 5, 1000, 6.0, 3)
    st = O.LossSettings.make()
    _upload(ctx, text, structs, labels, st, 6.0)
    n, P = ctx.neighbor_count()
    assert P == sum(nb.P for nb in nbs)
    _say("device loss+gradient over %d atoms, %d entries" % (n, P))
    f, g, _ = ctx.loss_grad(penalty_weight=1e-6, reg_l2=1e-10)
    t0 = time.time()
    fo, go = O.loss_grad_batch(O.Model(text), nbs, labels, st, 1e-6, 1e-10, 0.0, THREADS)
    _say("oracle loss+gradient in %.1f s (%d threads)" % (time.time() - t0, THREADS))
    assert rel_err(f, fo) < 1e-9
    assert rel_err(g, go) < 1e-9
    f2, g2, _ = ctx.loss_grad(penalty_weight=1e-6, reg_l2=1e-10, deterministic=True)
    assert rel_err(f2, fo) < 1e-9 and rel_err(g2, go) < 1e-9
