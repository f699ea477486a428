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


class DeviceArray:
    """A float64 device buffer from the HIP runtime the library itself links
    (libamdhip64.so.7): hipMalloc / hipMemcpy / hipFree through ctypes, for
    tests of entry points that take device pointers."""
    _hip = None

    @classmethod
    def hip(cls):
        if cls._hip is None:
            import ctypes as C
            h = C.CDLL("libamdhip64.so.7")
            h.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
            h.hipFree.argtypes = [C.c_void_p]
            h.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
            h.hipDeviceSynchronize.argtypes = []
            cls._hip = h
        return cls._hip

    def __init__(self, values):
        import ctypes as C
        self.host = np.ascontiguousarray(values, dtype=np.float64)
        self.ptr = C.c_void_p()
        assert self.hip().hipMalloc(C.byref(self.ptr), max(self.host.nbytes, 8)) == 0
        self.upload(self.host)

    def upload(self, values):
        import ctypes as C
        v = np.ascontiguousarray(values, dtype=np.float64).reshape(self.host.shape)
        assert self.hip().hipMemcpy(self.ptr, v.ctypes.data_as(C.c_void_p), v.nbytes, 1) == 0

    def download(self):
        import ctypes as C
        out = np.empty_like(self.host)
        assert self.hip().hipMemcpy(out.ctypes.data_as(C.c_void_p), self.ptr, out.nbytes, 2) == 0
        return out

    @property
    def address(self):
        return self.ptr.value

    def free(self):
        if self.ptr:
            self.hip().hipFree(self.ptr)
            self.ptr = None
