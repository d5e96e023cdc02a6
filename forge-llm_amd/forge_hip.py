"""ctypes binding of the C ABI in include/forge_hip.h (libforge_hip.so).

Used by the Python tests and bench.py; the product host is the JavaScript
package under forge-llm_amd/src, which reaches the same ABI through the N-API
addon.  Argument types are derived from the header itself, so the binding
cannot drift from the declared ABI.  There is no fallback: if the shared
library is missing, importing this module raises.
"""
import ctypes
import os
import re

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
HEADER = os.path.join(ROOT, "include", "forge_hip.h")
LIBPATH = os.environ.get("FORGE_HIP_LIB", os.path.join(HERE, "lib", "libforge_hip.so"))

_CTYPE = {
    "int": ctypes.c_int,
    "int64_t": ctypes.c_int64,
    "size_t": ctypes.c_size_t,
    "double": ctypes.c_double,
    "float": ctypes.c_float,
}


def parse_header(path=HEADER):
    """Return {name: (restype, [argtype strings])} for every fg_* declaration."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"(int|const char\s*\*)\s+(fg_\w+)\s*\(([^)]*)\)\s*;", text):
        ret, name, args = m.group(1), m.group(2), m.group(3).strip()
        types = []
        if args and args != "void":
            for a in args.split(","):
                a = a.strip()
                if "*" in a:
                    types.append("ptr")
                else:
                    t = re.sub(r"\bconst\b", "", a).strip().rsplit(None, 1)[0].strip()
                    types.append(t)
        decls[name] = (ret.replace(" ", ""), types)
    return decls


DECLS = parse_header()
MISSING = []  # declared in the header but not exported by the library


class ForgeError(RuntimeError):
    pass


def _load():
    if not os.path.exists(LIBPATH):
        raise ImportError("libforge_hip.so is not built (%s); run forge-llm_amd/build.py" % LIBPATH)
    lib = ctypes.CDLL(LIBPATH)
    for name, (ret, types) in DECLS.items():
        fn = getattr(lib, name, None)
        if fn is None:
            MISSING.append(name)
            continue
        fn.restype = ctypes.c_char_p if ret.startswith("constchar") else ctypes.c_int
        fn.argtypes = [ctypes.c_void_p if t == "ptr" else _CTYPE[t] for t in types]
    return lib


lib = _load()


def last_error():
    s = lib.fg_last_error()
    return s.decode() if s else ""


def check(rc, what=""):
    if rc != 0:
        raise ForgeError("%s failed (%d): %s" % (what, rc, last_error()))


def call(name, *args):
    """Call fg_<name>(*args); DeviceArray arguments are passed by pointer."""
    conv = [a.ptr if isinstance(a, DeviceArray) else a for a in args]
    rc = getattr(lib, "fg_" + name)(*conv)
    check(rc, "fg_" + name)


def device_count():
    n = ctypes.c_int(0)
    lib.fg_device_count(ctypes.byref(n))
    return n.value


_initialised = False


def init(device=0):
    global _initialised
    check(lib.fg_init(device), "fg_init")
    _initialised = True


def sync():
    check(lib.fg_sync(), "fg_sync")


class DeviceArray:
    """A device allocation from the library's caching allocator."""

    def __init__(self, shape, dtype=np.float32):
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = ctypes.c_void_p()
        check(lib.fg_malloc(ctypes.byref(p), max(self.nbytes, 1)), "fg_malloc")
        self.ptr = p.value

    @classmethod
    def from_numpy(cls, a):
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        if d.nbytes:
            check(lib.fg_h2d(ctypes.c_void_p(d.ptr), a.ctypes.data_as(ctypes.c_void_p), d.nbytes), "fg_h2d")
        return d

    @classmethod
    def zeros(cls, shape, dtype=np.float32):
        d = cls(shape, dtype)
        if d.nbytes:
            check(lib.fg_zero(ctypes.c_void_p(d.ptr), d.nbytes), "fg_zero")
        return d

    def numpy(self):
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            check(lib.fg_d2h(out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(self.ptr), self.nbytes), "fg_d2h")
        return out

    def upload(self, a):
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes
        check(lib.fg_h2d(ctypes.c_void_p(self.ptr), a.ctypes.data_as(ctypes.c_void_p), self.nbytes), "fg_h2d")

    def free(self):
        if self.ptr:
            lib.fg_free(ctypes.c_void_p(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr and _initialised:
                lib.fg_free(ctypes.c_void_p(self.ptr))
        except Exception:
            pass


class AdamTensor(ctypes.Structure):
    _fields_ = [("p", ctypes.c_void_p), ("g", ctypes.c_void_p), ("m", ctypes.c_void_p),
                ("v", ctypes.c_void_p), ("n", ctypes.c_int64)]


def adam_step(tensors, lr_t, b1, b2, eps, wd, clip, bc1, bc2, stats=None):
    """tensors: list of (p, g, m, v) DeviceArrays."""
    arr = (AdamTensor * len(tensors))()
    for i, (p, g, m, v) in enumerate(tensors):
        arr[i] = AdamTensor(p.ptr, g.ptr, m.ptr, v.ptr, int(np.prod(p.shape)))
    rc = lib.fg_adam_step(ctypes.cast(arr, ctypes.c_void_p), len(tensors), lr_t, b1, b2, eps, wd, clip,
                          bc1, bc2, stats.ptr if stats is not None else None)
    check(rc, "fg_adam_step")


class WgradJob(ctypes.Structure):
    _fields_ = [("gW", ctypes.c_void_p), ("gY", ctypes.c_void_p), ("X", ctypes.c_void_p), ("M", ctypes.c_int),
                ("K", ctypes.c_int), ("N", ctypes.c_int), ("beta", ctypes.c_int), ("xp_gy", ctypes.c_void_p),
                ("xp_x", ctypes.c_void_p)]


class ColsumJob(ctypes.Structure):
    _fields_ = [("out", ctypes.c_void_p), ("partial", ctypes.c_void_p), ("rows", ctypes.c_int), ("n", ctypes.c_int),
                ("beta", ctypes.c_int)]


class DecodeLayer(ctypes.Structure):
    _fields_ = ([(n, ctypes.c_void_p) for n in ("ln1", "wqkv", "wo", "ln2", "gate", "up", "down")]
                + [(n, ctypes.c_int) for n in ("wqkv_type", "wo_type", "gate_type", "up_type", "down_type")])


class DecodeModel(ctypes.Structure):
    _fields_ = ([(n, ctypes.c_int) for n in ("dim", "hidden", "nLayers", "nHeads", "nKvHeads", "vocab", "maxSeq",
                                             "emb_type", "cls_type")]
                + [("normEps", ctypes.c_double)]
                + [(n, ctypes.c_void_p) for n in ("tok_emb", "ln_f", "wcls", "layers", "rope_cos", "rope_sin", "x",
                                                  "q", "h", "attn_part")])


class Event:
    def __init__(self):
        p = ctypes.c_void_p()
        check(lib.fg_event_create(ctypes.byref(p)), "fg_event_create")
        self.ptr = p.value

    def record(self):
        check(lib.fg_event_record(ctypes.c_void_p(self.ptr)), "fg_event_record")

    def elapsed_ms(self, stop):
        ms = ctypes.c_float()
        check(lib.fg_event_elapsed_ms(ctypes.c_void_p(self.ptr), ctypes.c_void_p(stop.ptr), ctypes.byref(ms)),
              "fg_event_elapsed_ms")
        return ms.value


def kprof_report():
    buf = ctypes.create_string_buffer(1 << 20)
    check(lib.fg_kprof_report(buf, len(buf)), "fg_kprof_report")
    import json
    return json.loads(buf.value.decode())
