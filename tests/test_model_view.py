"""Model views (mtpx_model_view = MTPGpuPotentialView,
runtime/mtp/gpu-direct/mtp_gpu_direct.h:215-289) on the host.

A view made as the reference's adapter makes it (tests/view_adapter.py,
after potentials/mtp_gpu_adapter.cpp:110-212, 420-468) describes the same
model as the text it came from: mtpx_format_model_view writes the text
mtpx_format_model_text writes, line for line (the potential_tag aside,
which a view does not carry), for every basis kind, split bases and MTP-M
heads.  Inconsistent views are refused with validate_potential_view's texts
(mtp_gpu_direct.cu:419-660); kinds the library does not evaluate with
MTPX_E_MODEL."""
import numpy as np
import pytest

from mtpx import capi
from mtpx import synth as S
from test_gpm import MODELS, _elements_tag
from test_model_io import model_text
from test_mtpm import head_text
from view_adapter import view_of_text, without_tag

VIEW_MODELS = dict(MODELS)
VIEW_MODELS.update({
    "poly5": lambda: model_text("poly5"),
    "split": lambda: model_text("split"),
    "mtp_m_fs": lambda: head_text("mtp_m_fs"),
    "mtp_m_n1": lambda: head_text("mtp_m_n1", 5, 0, "RELU"),
    "level20": lambda: S.random_model("shapeev-20.mtp", 3, 10, 1.5, 6.0, -0.05, 0.05,
                                      S.rng_for(81)),
})


@pytest.mark.parametrize("kind", sorted(VIEW_MODELS))
def test_view_describes_the_text_model(kind):
    text = VIEW_MODELS[kind]()
    view, canon = view_of_text(text)
    got = capi.format_model_view(view)
    assert without_tag(got) == without_tag(canon)
    info, coef = capi.parse_model_text(got)
    info_t, coef_t = capi.parse_model_text(canon)
    assert info == info_t and np.array_equal(coef, coef_t)
    assert capi.parse_model_head(got) == capi.parse_model_head(canon)


def test_shared_basis_passed_as_pair_descriptors():
    """The adapter passes Z^2 copies of a shared non-Chebyshev basis; a
    Chebyshev basis passed the same way is the same model."""
    text = MODELS["chebyshev"]()
    a, canon = view_of_text(text)
    b, _ = view_of_text(text, force_pairs=True)
    assert b.pair_radial_basis_count == 4
    assert capi.format_model_view(a) == capi.format_model_view(b)
    assert "radial_basis_split" not in capi.format_model_view(b)


def _refused(view, code, msg):
    with pytest.raises(capi.MtpxError) as e:
        capi.format_model_view(view)
    assert e.value.code == capi.ERRORS_BY_NAME[code], str(e.value)
    assert msg in str(e.value)


def _fields(kind="chebyshev", **over):
    """The view's fields as a dict (pair bases separately) with overrides."""
    text = VIEW_MODELS[kind]()
    view, _ = view_of_text(text)
    f = {}
    arrays = {}
    for name, ctype in capi.ModelView._fields_:
        if name == "pair_radial_bases":
            continue
        val = getattr(view, name)
        if ctype in (capi._ip, capi._dp):
            arrays[name] = val
        else:
            f[name] = val
    pairs = None
    if view.pair_radial_basis_count:
        pairs = [{k: getattr(view.pair_radial_bases[i], k)
                  for k, _ in capi.RadialBasisView._fields_ if not k.startswith("polynomial")}
                 for i in range(view.pair_radial_basis_count)]
    return view, f, arrays, pairs


def _rebuild(view, f, arrays, pairs, **over):
    """A view with the same pointers and some scalar or pointer fields changed."""
    v = capi.ModelView()
    for name, _ in capi.ModelView._fields_:
        if name in ("pair_radial_bases",):
            continue
        if name in arrays:
            setattr(v, name, arrays[name])
        elif name in f:
            setattr(v, name, f[name])
    keep = [view]
    if pairs is not None:
        arr = (capi.RadialBasisView * len(pairs))()
        for k, b in enumerate(pairs):
            for name, val in b.items():
                setattr(arr[k], name, val)
        keep.append(arr)
        v.pair_radial_bases = capi.C.cast(arr, capi.C.POINTER(capi.RadialBasisView))
        v.pair_radial_basis_count = len(pairs)
    for k, val in over.items():
        setattr(v, k, val)
    v._keep = keep
    return v


def test_species_map_checks():
    view, f, a, p = _fields()
    bad = np.array([0, 2], np.int32)
    _refused(_rebuild(view, f, a, p, spmap=bad.ctypes.data_as(capi._ip)), "MTPX_E_INVALID",
             "species mapping is outside [-1, species_count)")
    _refused(_rebuild(view, f, a, p, max_type=0), "MTPX_E_INVALID",
             "invalid species_count/max_type/spmap in MTPGpuPotentialView")
    # -1 entries are allowed (LAMMPS type 0 is unused)
    ok = np.array([-1, 1, 0], np.int32)
    capi.format_model_view(_rebuild(view, f, a, p, spmap=ok.ctypes.data_as(capi._ip),
                                    max_type=3))


def test_refused_kinds():
    view, f, a, p = _fields("configurable")
    _refused(_rebuild(view, f, a, None, pair_radial_basis_count=0), "MTPX_E_INVALID",
             "configurable radial basis requires explicit pair descriptors")
    polyb = [dict(b, radial_basis=capi.RB_KINDS["RBPolyB"]) for b in p]
    _refused(_rebuild(view, f, a, polyb), "MTPX_E_MODEL", "RBPolyB")
    view, f, a, p = _fields("chebyshev")
    _refused(_rebuild(view, f, a, None, radial_basis=capi.RB_KINDS["RBChebyshevPoly5"]),
             "MTPX_E_MODEL", "RBChebyshevPoly5 basis needs its pair descriptors")
    _refused(_rebuild(view, f, a, None, radial_basis=7), "MTPX_E_INVALID",
             "unsupported radial basis in MTPGpuPotentialView")
    _refused(_rebuild(view, f, a, None, cutoff=f["max_dist"] + 0.5), "MTPX_E_INVALID",
             "cutoff differs from the largest max_dist")
    _refused(_rebuild(view, f, a, None, radial_coeffs_count=3), "MTPX_E_INVALID",
             "radial coefficient count does not match the MTP dimensions")
    _refused(_rebuild(view, f, a, None, model=9), "MTPX_E_INVALID",
             "unsupported site-energy model in MTPGpuPotentialView")
    _refused(_rebuild(view, f, a, None, descriptor_count=2), "MTPX_E_INVALID",
             "invalid classic linear coefficient layout")
    _refused(_rebuild(view, f, a, None, alpha_index_basic_count=f["alpha_moments_count"] + 1),
             "MTPX_E_INVALID", "invalid MTP moment counts in MTPGpuPotentialView")
    _refused(_rebuild(view, f, a, None, scalar_gather=1), "MTPX_E_MODEL", "scalar gather")
    mp = np.array(np.ctypeslib.as_array(a["alpha_moment_mapping"],
                                        shape=(f["alpha_scalar_moments"],)))
    mp[0] = f["alpha_moments_count"]
    _refused(_rebuild(view, f, a, None, alpha_moment_mapping=mp.ctypes.data_as(capi._ip)),
             "MTPX_E_INVALID", "alpha_moment_mapping entry is out of range")


def test_refused_heads():
    view, f, a, p = _fields("mtp_m_n2")
    _refused(_rebuild(view, f, a, p, model_coeffs_count=f["model_coeffs_count"] + 1),
             "MTPX_E_INVALID", "MTP-M model coefficient count does not match its dimensions")
    _refused(_rebuild(view, f, a, p, model_activation=capi.VIEW_ACTIVATIONS["LINEAR"]),
             "MTPX_E_INVALID", "NN2 MTP-M requires two hidden layers")
    mc = np.ones(1)
    _refused(_rebuild(view, f, a, p, moment_coeffs=mc.ctypes.data_as(capi._dp)),
             "MTPX_E_INVALID", "invalid MTP-M descriptor/model coefficient layout")
    view, f, a, p = _fields("mtp_m_q2")
    _refused(_rebuild(view, f, a, p, descriptor_count=3), "MTPX_E_INVALID",
             "invalid analytic MTP-M model dimensions")


def test_split_descriptor_checks():
    view, f, a, p = _fields("split-configurable")
    bad = [dict(b) for b in p]
    bad[1]["max_dist"] = bad[1]["min_dist"]
    _refused(_rebuild(view, f, a, bad), "MTPX_E_INVALID", "invalid split radial basis descriptor")
    _refused(_rebuild(view, f, a, p[:3]), "MTPX_E_INVALID",
             "split radial basis count does not match species_count^2")
    s7 = [dict(b) for b in p]
    s7[0].update(radial_basis=capi.RB_KINDS["RBChebyshevConfigurable"],
                 cutoff=capi.CUTOFFS["smoothstep7"], cutoff_r1=s7[0]["max_dist"] + 1,
                 cutoff_r2=s7[0]["max_dist"] + 2)
    _refused(_rebuild(view, f, a, s7), "MTPX_E_INVALID", "invalid smoothstep7 radial interval")


def test_elements_tag_is_not_part_of_the_view():
    text = model_text("chebyshev", tag=_elements_tag(2))
    view, canon = view_of_text(text)
    assert '"elements"' in canon
    assert '"elements"' not in capi.format_model_view(view)
