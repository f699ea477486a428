"""GPM v2 model bundles (tools/gpm_container.h, tools/gpm_mtp.h; the MTP
node of potentials/gpm_codec.cpp:190-382).

Pinned against the reference's own container code (oracle/_ref/gpm_ref, the
header-only reader, writer and MTP text adapter built from their sources,
where available) and its runtime reader (oracle/_ref/mtpm_ref, which loads
bundles through MLIPCore::read_model_text): the product's GPM -> .mtp text
is byte-equal to GPM::mtp_text; bundles the product writes are read back
by the reference to the same text and evaluate in the reference runtime to
the oracle's E/F/S of the source model at 1e-12; bundles the reference
writer lays out are read by the product to the same coefficients, bit for
bit; malformed containers are refused with the reference's own reasons."""
import ctypes
import json
import os
import struct
import subprocess

import numpy as np
import pytest

import oracle as O
from helpers import rel_err
from mtpx import capi
from mtpx import synth as S
from test_model_io import model_text
from test_mtpm import head_text, structure

needs_gpm_ref = pytest.mark.skipif(not O.ref_available("gpm_ref"),
                                   reason="oracle/_ref/gpm_ref not built (make -C oracle ref)")
needs_mtpm_ref = pytest.mark.skipif(not O.ref_available("mtpm_ref"),
                                    reason="oracle/_ref/mtpm_ref not built (make -C oracle ref)")


def _zstd():
    try:
        return ctypes.CDLL("libzstd.so.1")
    except OSError:
        return None


def _elements_tag(Z):
    els = json.dumps(["Ta", "W", "Mo", "Nb"][:Z]).replace(" ", "")
    return ('{"elements":%s,"model":"linear","schema":"gpml.mtp.metadata","type":"MTP",'
            '"version":1}' % els)


MODELS = {
    "chebyshev": lambda: model_text("chebyshev"),
    "chebyshev-elements": lambda: model_text("chebyshev", tag=_elements_tag(2)),
    "poly4": lambda: model_text("poly4"),
    "chebycos": lambda: model_text("chebycos"),
    "split-configurable": lambda: model_text("split-configurable"),
    "configurable": lambda: model_text("configurable"),
    "level16": lambda: S.random_model("shapeev-16.mtp", 2, 8, 1.9, 5.0, -0.05, 0.05,
                                      S.rng_for(80)),
    "mtp_m_n2": lambda: head_text("mtp_m_n2", 4, 3, "SIGMOID"),
    "mtp_m_q2": lambda: head_text("mtp_m_q2"),
    "mtp_m_li": lambda: head_text("mtp_m_li"),
}


def _ref(*args, check=True):
    r = subprocess.run([os.path.join(O.REF_DIR, "gpm_ref")] + list(args), capture_output=True,
                       text=True)
    if check:
        assert r.returncode == 0, r.stderr
    return r


def _unpack(data):
    """(manifest, payload) of a bundle."""
    assert data[:8] == b"GPMLMODL"
    length, start = struct.unpack_from("<QQ", data, 16)
    return json.loads(data[64:64 + length].decode()), data[start:]


def _pack(manifest, payload, major=2, flags=0):
    """A bundle of a manifest and payload (the container layout of
    GPM::Writer::save, tools/gpm_container.h:681-700)."""
    js = json.dumps(manifest, separators=(",", ":")).encode()
    start = (64 + len(js) + 63) & ~63
    pre = bytearray(64)
    pre[:8] = b"GPMLMODL"
    struct.pack_into("<HHIQQ", pre, 8, major, 0, flags, len(js), start)
    return bytes(pre) + js + b"\0" * (start - 64 - len(js)) + payload


# --------------------------------------------------------------- round trip --

@pytest.mark.parametrize("kind", list(MODELS))
def test_bundle_reads_back_to_the_same_model(kind):
    text = MODELS[kind]()
    data = capi.gpm_from_text(text)
    info, coef = capi.parse_model_gpm(data)
    info_t, coef_t = capi.parse_model_text(text)
    assert info == info_t and np.array_equal(coef, coef_t)
    back = capi.gpm_to_text(data)
    assert capi.parse_model_head(back) == capi.parse_model_head(text)
    # the bundle of the bundle's model is the same bundle
    assert capi.gpm_from_text(back) == data


def test_bundle_layout():
    """The manifest of encode_mtp in ModelBundle::encode's frame: blocks in
    id order at 64-aligned offsets, sizes as decimal strings."""
    text = MODELS["chebyshev-elements"]()
    data = capi.gpm_from_text(text)
    man, payload = _unpack(data)
    assert man["schema"] == "gpml.model" and man["root_model"] == "root"
    assert man["units"] == {"charge": "e", "energy": "eV", "length": "angstrom",
                            "stress": "virial_eV"}
    node = man["models"]["root"]
    assert node["type"] == "mtp" and node["version"] == 1 and node["children"] == {}
    assert man["species"] == node["species"] == [{"id": 0, "symbol": "Ta"},
                                                 {"id": 1, "symbol": "W"}]
    c = node["configuration"]
    m = O.Model(text)
    assert (c["species_count"], c["radial_functions"], c["radial_size"], c["moments_count"],
            c["radial_mode"]) == (m.Z, m.M, m.R, m.K, 0)
    assert c["radial_bases"][0]["radial_basis_type"] == "RBChebyshev"
    assert c["radial_bases"][0]["scaling"] == "0.01"
    ids = [b["id"] for b in man["blocks"]]
    assert ids == sorted(ids)
    for b in man["blocks"]:
        assert int(b["offset"]) % 64 == 0 and b["codec"] == "none"
        assert b["stored_size"] == b["raw_size"]
    radial = next(b for b in man["blocks"] if b["id"] == "root/radial")
    off = int(radial["offset"])
    got = np.frombuffer(payload[off:off + int(radial["raw_size"])], "<f8")
    assert np.array_equal(got, m.coeffs[:m.nradial])
    assert node["common"]["cutoff"] == m.cutoff


@pytest.mark.skipif(_zstd() is None, reason="libzstd.so.1 not present")
def test_zstd_blocks():
    text = MODELS["mtp_m_n2"]()
    data = capi.gpm_from_text(text, zstd_level=3)
    man, _ = _unpack(data)
    assert {b["codec"] for b in man["blocks"]} == {"zstd"}
    assert np.array_equal(capi.parse_model_gpm(data)[1], capi.parse_model_text(text)[1])
    assert capi.gpm_to_text(data) == capi.gpm_to_text(capi.gpm_from_text(text))


@pytest.mark.skipif(_zstd() is None, reason="libzstd.so.1 not present")
def test_zstd_block_beyond_the_read_limit_is_refused():
    """A few-hundred-byte bundle whose zstd block declares 16 GiB of raw
    data is refused before anything is allocated (Reader::read's 8 GiB
    limit, tools/gpm_container.h:512-515)."""
    data = capi.gpm_from_text(MODELS["mtp_m_n2"](), zstd_level=3)
    man, payload = _unpack(data)
    rad = next(b for b in man["blocks"] if b["id"] == "root/radial")
    rad["shape"] = [str(1 << 31)]
    rad["raw_size"] = str(8 << 31)
    with pytest.raises(capi.MtpxError) as e:
        capi.parse_model_gpm(_pack(man, payload))
    assert "block exceeds read limit: root/radial" in str(e.value)


# ------------------------------------------------------ reference container --

@needs_gpm_ref
@pytest.mark.parametrize("kind", list(MODELS))
def test_text_is_the_reference_adapter_text(workdir, kind):
    data = capi.gpm_from_text(MODELS[kind]())
    path = os.path.join(workdir, "m.gpm")
    open(path, "wb").write(data)
    _ref("text", path, os.path.join(workdir, "m.txt"))
    assert capi.gpm_to_text(data) == open(os.path.join(workdir, "m.txt")).read()


@needs_gpm_ref
@pytest.mark.parametrize("kind", ["chebyshev-elements", "split-configurable", "mtp_m_n2"])
def test_reference_writer_layout_reads_the_same(workdir, kind):
    """GPM::Writer re-lays the bundle out (its pretty-printed header, its
    block placement); the product reads it to the same model."""
    data = capi.gpm_from_text(MODELS[kind]())
    a, b = os.path.join(workdir, "a.gpm"), os.path.join(workdir, "b.gpm")
    open(a, "wb").write(data)
    _ref("rewrite", a, b)
    again = open(b, "rb").read()
    assert again != data
    assert np.array_equal(capi.parse_model_gpm(again)[1], capi.parse_model_gpm(data)[1])
    assert capi.gpm_to_text(again) == capi.gpm_to_text(data)


@needs_mtpm_ref
@pytest.mark.parametrize("kind", ["chebyshev", "split-configurable", "poly4", "mtp_m_n2",
                                  "mtp_m_q2"])
def test_reference_runtime_evaluates_the_bundle(workdir, kind):
    """MLIPCore::read_model_text loads the product's bundle (folding each
    pair's scale into its coefficients) and evaluates the source model's
    E/F/S."""
    text = MODELS[kind]()
    m = O.Model(text)
    s = structure(81)
    pos = O.wrap(s.cell, s.pbc, s.pos)
    nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, m.cutoff)
    E, F, St, se = O.efs(m, nb)
    Er, ser, Fr, vr = O.ref_mlip_efs(capi.gpm_from_text(text), nb, s.types, m.cutoff, workdir,
                                     m.Z, binary="mtpm_ref")
    sym = 0.5 * (St + St.T)
    v6 = np.array([sym[0, 0], sym[1, 1], sym[2, 2], sym[0, 1], sym[0, 2], sym[1, 2]])
    assert rel_err(E, Er) < 1e-12 and rel_err(F, Fr) < 1e-12 and rel_err(v6, vr) < 1e-12
    assert rel_err(se, ser) < 1e-12


# ------------------------------------------------------------ refusals --

def _bad_cases():
    data = capi.gpm_from_text(MODELS["mtp_m_q2"]())
    man, payload = _unpack(data)
    out = []

    def edit(name, fn, msg, ref=True):
        m = json.loads(json.dumps(man))
        fn(m)
        out.append((name, _pack(m, payload), msg, ref))

    def block(m, bid):
        return next(b for b in m["blocks"] if b["id"] == bid)
    out.append(("magic", b"GPMLMODX" + data[8:], "invalid magic", True))
    out.append(("major", _pack(man, payload, major=3), "unsupported major version", True))
    out.append(("flags", _pack(man, payload, flags=1), "unsupported required flags", True))
    out.append(("short", data[:40], "truncated preamble", True))
    edit("schema", lambda m: m.update(schema="gpml.other"), "unknown schema")
    edit("features", lambda m: m.update(required_features=["x"]), "unsupported required features")
    edit("leading-zero", lambda m: block(m, "root/radial").update(offset="0" + block(m, "root/radial")["offset"]),
         "invalid uint64")
    edit("shape", lambda m: block(m, "root/radial").update(shape=["3"]), "block shape/size mismatch")
    edit("overlap", lambda m: block(m, "root/species").update(offset=block(m, "root/radial")["offset"]),
         "overlapping blocks")
    edit("unaligned", lambda m: block(m, "root/species").update(
        offset=str(int(block(m, "root/species")["offset"]) + 8)), "invalid block bounds")
    edit("missing", lambda m: m["blocks"].remove(block(m, "root/moments")), "missing block")
    edit("codec", lambda m: block(m, "root/radial").update(codec="lz4"), "unsupported codec")
    edit("dims", lambda m: m["models"]["root"]["configuration"].update(radial_functions=0),
         "invalid MTP dimensions")
    edit("bases", lambda m: m["models"]["root"]["configuration"]["radial_bases"].append(
        m["models"]["root"]["configuration"]["radial_bases"][0]), "invalid radial bases")
    edit("type", lambda m: m["models"]["root"].update(type="lj612"), "mtp and mtp_m", ref=False)
    edit("units", lambda m: m["units"].update(energy="kcal/mol"), "unsupported GPM units",
         ref=False)
    edit("radial-mode", lambda m: m["models"]["root"]["configuration"].update(radial_mode=1),
         "unsupported radial mode", ref=False)
    edit("long-range", lambda m: m["models"]["root"]["configuration"]["metadata"].update(
        long_range={"channels": 1, "kernel": "coulomb"}), "long-range", ref=False)
    return out


BAD = _bad_cases()


@pytest.mark.parametrize("name,data,msg,ref", BAD, ids=[b[0] for b in BAD])
def test_product_refuses_malformed_bundles(name, data, msg, ref):
    with pytest.raises(capi.MtpxError) as e:
        capi.parse_model_gpm(data)
    assert msg in str(e.value)


@needs_gpm_ref
@pytest.mark.parametrize("name,data,msg,ref", [b for b in BAD if b[3]],
                         ids=[b[0] for b in BAD if b[3]])
def test_reference_refuses_the_same(workdir, name, data, msg, ref):
    path = os.path.join(workdir, "bad.gpm")
    open(path, "wb").write(data)
    r = _ref("text", path, os.path.join(workdir, "bad.txt"), check=False)
    assert r.returncode != 0 and msg in r.stderr, r.stderr
