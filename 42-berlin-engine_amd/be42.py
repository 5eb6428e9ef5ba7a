"""Host-side mirror of the gfx950 decode hot-path library (lib42be_hip.so).

Loads the C-ABI shared library through ctypes and exposes its entry points on
torch device tensors.  torch is imported before the library is loaded so that
the process holds exactly one HIP runtime (torch ships its own
libamdhip64.so.7; the library then binds to the already-loaded copy).

There is no CPU path here: when the library or a GPU is missing, calls raise.
"""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib42be_hip.so")

BE42_OK = 0
ERRORS = {-1: "EINVAL", -2: "EHIP", -3: "ENOMEM", -4: "ENODEV"}

vp, i32, sz, f32 = C.c_void_p, C.c_int, C.c_size_t, C.c_float

# name -> (restype, argtypes); keep in sync with include/*.h
SIGNATURES = {
    "be42_init": (i32, [i32]),
    "be42_last_error": (C.c_char_p, []),
    "be42_device_count": (i32, []),
    "be42_sync": (i32, [vp]),
    "be42_malloc": (vp, [sz]),
    "be42_free": (i32, [vp]),
    "be42_memcpy_h2d": (i32, [vp, vp, sz, vp]),
    "be42_memcpy_d2h": (i32, [vp, vp, sz, vp]),
    "be42_memset": (i32, [vp, i32, sz, vp]),
    "be42_quant_rows_int8": (i32, [vp, vp, vp, i32, i32, vp]),
    "be42_quant_rows_fp8": (i32, [vp, vp, vp, i32, i32, vp]),
    "be42_dequant_rows_int8": (i32, [vp, vp, vp, i32, i32, vp]),
    "be42_fp8_decode": (i32, [vp, vp, sz, vp]),
    "be42_gemv_q8": (i32, [vp, vp, vp, vp, i32, i32, i32, vp]),
    "be42_gemv_fp8": (i32, [vp, vp, vp, vp, i32, i32, i32, vp]),
    "be42_gemv_xdig_bytes": (sz, [i32, i32, i32]),
    "be42_gemv_prepare": (i32, [vp, vp, i32, i32, i32, vp]),
    "be42_gemv_q8_prepared": (i32, [vp, vp, vp, vp, i32, i32, i32, vp]),
    "be42_gemv_fp8_prepared": (i32, [vp, vp, vp, vp, i32, i32, i32, vp]),
}


class Be42Error(RuntimeError):
    pass


def _torch():
    import torch  # noqa: F401  (must precede the library load, see module doc)
    return torch


class Lib:
    def __init__(self, path=LIB_PATH):
        self.torch = _torch()
        if not os.path.exists(path):
            raise Be42Error(f"{path} is not built: run __graft_entry__.build()")
        self.lib = C.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(self.lib, name)
            fn.restype = res
            fn.argtypes = args
        self._inited = False

    # -- plumbing -------------------------------------------------------------
    def device_available(self):
        return self.lib.be42_device_count() > 0

    def init(self, device=0):
        if not self._inited:
            self.check(self.lib.be42_init(device), "be42_init")
            self._inited = True

    def last_error(self):
        return (self.lib.be42_last_error() or b"").decode()

    def check(self, rc, what):
        if rc != BE42_OK:
            raise Be42Error(f"{what}: {ERRORS.get(rc, rc)}: {self.last_error()}")

    def stream(self, s=None):
        t = self.torch
        s = s if s is not None else t.cuda.current_stream()
        return C.c_void_p(s.cuda_stream)

    @staticmethod
    def p(t):
        return C.c_void_p(t.data_ptr()) if t is not None else None

    def _call(self, name, *args):
        self.init()
        self.check(getattr(self.lib, name)(*args), name)

    # -- quant codecs ---------------------------------------------------------
    def quant_rows_int8(self, x):
        t = self.torch
        rows, cols = x.shape
        q = t.empty((rows, cols), dtype=t.int8, device=x.device)
        s = t.empty(rows, dtype=t.float32, device=x.device)
        self._call("be42_quant_rows_int8", self.p(q), self.p(s), self.p(x), rows, cols, self.stream())
        return q, s

    def quant_rows_fp8(self, x):
        t = self.torch
        rows, cols = x.shape
        q = t.empty((rows, cols), dtype=t.uint8, device=x.device)
        s = t.empty(rows, dtype=t.float32, device=x.device)
        self._call("be42_quant_rows_fp8", self.p(q), self.p(s), self.p(x), rows, cols, self.stream())
        return q, s

    def dequant_rows_int8(self, q, s):
        t = self.torch
        rows, cols = q.shape
        out = t.empty((rows, cols), dtype=t.float32, device=q.device)
        self._call("be42_dequant_rows_int8", self.p(out), self.p(q), self.p(s), rows, cols, self.stream())
        return out

    def fp8_decode(self, q):
        t = self.torch
        out = t.empty(q.shape, dtype=t.float32, device=q.device)
        self._call("be42_fp8_decode", self.p(out), self.p(q), q.numel(), self.stream())
        return out

    # -- GEMV -----------------------------------------------------------------
    def gemv(self, w, sw, x, kind, out=None, stream=None):
        t = self.torch
        n, k = w.shape
        batch = x.shape[0] if x.dim() == 2 else 1
        y = out if out is not None else t.empty((batch, n), dtype=t.float32, device=x.device)
        name = "be42_gemv_q8" if kind == "int8" else "be42_gemv_fp8"
        self._call(name, self.p(y), self.p(w), self.p(sw), self.p(x), n, k, batch, self.stream(stream))
        return y


    def gemv_prepare(self, x, kind, buf=None, stream=None):
        """Split activations x [batch][k] into MFMA digit planes (device buffer)."""
        t = self.torch
        batch, k = x.shape
        fp8 = 1 if kind == "fp8" else 0
        nbytes = self.lib.be42_gemv_xdig_bytes(k, batch, fp8)
        if nbytes == 0:
            raise Be42Error("gemv_prepare: unsupported shape")
        if buf is None:
            buf = t.empty(nbytes, dtype=t.uint8, device=x.device)
        self._call("be42_gemv_prepare", self.p(buf), self.p(x), k, batch, fp8, self.stream(stream))
        return buf

    def gemv_prepared(self, w, sw, xdig, batch, kind, out, stream=None):
        n, k = w.shape
        name = "be42_gemv_q8_prepared" if kind == "int8" else "be42_gemv_fp8_prepared"
        self._call(name, self.p(out), self.p(w), self.p(sw), self.p(xdig), n, k, batch, self.stream(stream))
        return out


_LIB = None


def load():
    """The process-wide library handle (raises if the .so is not built)."""
    global _LIB
    if _LIB is None:
        _LIB = Lib()
    return _LIB
