"""Carve the level-10 template from shapeev-16.mtp.

No level-10 template ships with the reference; its inventory is recorded in
unitest/test-data/mtp-basis-corpus/sources.json ("shapeev/10": 41 moments,
25 basic, 42 products, 16 scalars).  Shapeev's level of a basic moment
(mu, a, b, c) is 2 + 4 mu + (a + b + c); a product rule's output has the sum
of its operands' levels.  Scalars with level <= 10 are kept, then orphans are
removed the way PotMTP::remove_orphans does (potentials/potential_mtp.cpp:
7340-7460): keep = closure of the kept scalars through the rules in reverse
order, moments renumbered in index order, radial channels compacted.

usage: python tests/golden/make_level10.py  (writes templates/shapeev-10.mtp)
"""
import os
import re
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(HERE)), "imr-mlp_amd"))
from mtpx.synth import template_topology  # noqa: E402


def carve(text: str, max_level: int):
    t = template_topology(text)
    basic, times, mp, K = t["basic"], t["times"], t["map"], t["K"]
    B = len(basic)
    level = [None] * K
    for i, b in enumerate(basic):
        level[i] = 2 + 4 * int(b[0]) + int(b[1] + b[2] + b[3])
    for l, r, c, o in times:
        lv = level[l] + level[r]
        assert level[o] in (None, lv), "inconsistent rule levels"
        level[o] = lv
    keep_scalar = [s for s in range(len(mp)) if level[mp[s]] <= max_level]
    keep = [False] * K
    for s in keep_scalar:
        keep[mp[s]] = True
    for l, r, c, o in reversed(times.tolist()):
        if keep[o]:
            keep[l] = keep[r] = True
    mmap = {}
    for i in range(K):
        if keep[i]:
            mmap[i] = len(mmap)
    channels = sorted({int(basic[i][0]) for i in range(B) if keep[i]})
    cmap = {mu: q for q, mu in enumerate(channels)}
    nb = [[cmap[int(b[0])], int(b[1]), int(b[2]), int(b[3])] for i, b in enumerate(basic) if keep[i]]
    nt = [[mmap[int(l)], mmap[int(r)], int(c), mmap[int(o)]] for l, r, c, o in times if keep[o]]
    nm = [mmap[int(mp[s])] for s in keep_scalar]
    return dict(K=len(mmap), basic=nb, times=nt, map=nm, M=len(channels))


def render(t, header_text):
    head = header_text.split("alpha_moments_count")[0]
    head = re.sub(r"radial_funcs_count = \d+", "radial_funcs_count = %d" % t["M"], head)
    out = head
    out += "alpha_moments_count = %d\n" % t["K"]
    out += "alpha_index_basic_count = %d\n" % len(t["basic"])
    out += "alpha_index_basic = {" + ", ".join("{%d, %d, %d, %d}" % tuple(b) for b in t["basic"]) + "}\n"
    out += "alpha_index_times_count = %d\n" % len(t["times"])
    out += "alpha_index_times = {" + ", ".join("{%d, %d, %d, %d}" % tuple(r) for r in t["times"]) + "}\n"
    out += "alpha_scalar_moments = %d\n" % len(t["map"])
    out += "alpha_moment_mapping = {" + ", ".join(str(v) for v in t["map"]) + "}\n"
    return out


if __name__ == "__main__":
    src = open(os.path.join(HERE, "templates", "shapeev-16.mtp")).read()
    t = carve(src, 10)
    assert (t["K"], len(t["basic"]), len(t["times"]), len(t["map"]), t["M"]) == (41, 25, 42, 16, 3), \
        (t["K"], len(t["basic"]), len(t["times"]), len(t["map"]), t["M"])
    with open(os.path.join(HERE, "templates", "shapeev-10.mtp"), "w") as f:
        f.write(render(t, src))
    print("wrote shapeev-10.mtp", t["K"], len(t["basic"]), len(t["times"]), len(t["map"]), t["M"])
