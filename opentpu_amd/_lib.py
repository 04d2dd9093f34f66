"""ctypes binding of libotpu_amd.so (the C ABI of include/otpu.h) and the torch plumbing the
Python API uses: device tensors, their pointers and the current HIP stream.

There is no CPU fallback: every operation runs the HIP kernels, and loading fails loudly when
the library is not built or no GPU is present."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("OTPU_LIB") or os.path.join(HERE, "libotpu_amd.so")

INT8, INT4, FP4, NVFP4 = 0, 1, 2, 3
FMT = {"int8": INT8, "int4": INT4, "fp4": FP4, "nvfp4": NVFP4}
UNIT, ACC, RMAX, ASCALE, PAIR, RSC = 0x1, 0x2, 0x4, 0x8, 0x40, 0x80
Q_ROW, Q_LO, Q_HL = 0x1, 0x10, 0x20             # QACT / QST flags
QALIGN = 64                                     # QACT ST / LDA row alignment
LM_STATE_BYTES = 16640                          # the LM head's state (result word, maxima)
ABI_VERSION = 3                                 # include/otpu.h OTPU_ABI_VERSION this binding follows

# every exported symbol and its argument types (P pointer, L int64, I int32, F float, D double)
_P, _L, _I, _F, _D = C.c_void_p, C.c_int64, C.c_int, C.c_float, C.c_double
SIGNATURES = {
    "otpu_last_error": ([], C.c_char_p),
    "otpu_version": ([], _I),
    "otpu_qact": ([_P, _I, _I, _L, _I, _I, _P, _P, _P, _L, _P, _P, _L, _P, _L, _P], _I),
    "otpu_lda": ([_P, _L, _I, _I, _P, _L, _P, _P, _L, _P], _I),
    "otpu_mm": ([_P, _L, _P, _P, _L, _I, _I, _P, _L, _P, _L, _I, _I, _I, _I, _P, _P, _L, _P, _P], _I),
    "otpu_mm_acc": ([_P, _L, _P, _L, _I, _I, _P, _L, _P, _L, _I, _I, _I, _I, _P, _P], _I),
    "otpu_mm_batched": ([_I, _P, _L, _L, _P, _L, _P, _L, _L, _I, _I, _P, _L, _L, _P, _L, _L, _I, _I, _I,
                         _I, _P, _L, _L, _P], _I),
    "otpu_lm_head_argmax": ([_P, _P, _P, _I, _P, _L, _P, _L, _I, _I, _I, _I, _L, _P, _P, _P, _P], _I),
    "otpu_argmax": ([_P, _I, _I, _L, _L, _P, _L, _P], _I),
    "otpu_pack_int8": ([_P, _I, _I, _L, _I, _P, _L, _P, _L, _P], _I),
    "otpu_pack_x4": ([_P, _I, _I, _L, _I, _P, _L, _P, _L, _P], _I),
    "otpu_qact_ranges": ([_P, _P, _I, _I, _L, _I, _I, _I, _P, _P, _P, _L, _P, _P, _L, _P], _I),
    "otpu_mm_ranges": ([_P, _L, _P, _P, _L, _I, _I, _I, _P, _L, _P, _L, _I, _I, _I, _I, _P, _P, _L, _P], _I),
    "otpu_vmul": ([_P, _P, _P, _L, _P], _I),
    "otpu_mm_qin": ([_P, _P, _P, _P, _I, _L, _I, _I, _P, _L, _P, _L, _I, _I, _I, _I, _P, _L, _L, _P], _I),
    "otpu_mm_qin_fold": ([_P, _P, _P, _P, _I, _I, _P, _L, _P, _L, _I, _I, _I, _I, _P, _P], _I),
    "otpu_mm_spl": ([_P, _L, _P, _P, _L, _I, _I, _P, _L, _L, _P, _L, _I, _I, _P, _L, _P], _I),
    "otpu_acc_rows": ([_P, _I, _L, _I, _P, _P, _P], _I),
    "otpu_chain_plan_bytes": ([_I, _I, _I, _I, _I], _L),
    "otpu_chain_plan": ([_I, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _L], _I),
    "otpu_chain_step": ([_P, _P], _I),
    "otpu_chain_error": ([_P, _P], _I),
    "otpu_chain_stamps": ([_P, _P], _I),
    "otpu_ungroup_rows": ([_P, _I, _I, _I, _I, _I, _L, _P, _L, _P], _I),
    "otpu_ungroup_scales": ([_P, _I, _I, _I, _I, _I, _I, _P, _L, _P], _I),
    "otpu_import_mxfp4": ([_P, _L, _P, _L, _I, _I, _I, _P, _L, _P, _L, _P, _P], _I),
    "otpu_import_nvfp4": ([_P, _L, _P, _L, _F, _I, _I, _P, _L, _P, _L, _P, _P], _I),
    "otpu_sample_work_bytes": ([_I], _L),
    "otpu_sample": ([_P, _I, _P, _P, _D, _I, _F, _F, _P, _I, _P, _P, _P, _P], _I),
    "otpu_sample_static": ([_P, _I, _P, _P, _D, _I, _F, _F, _P, _I, _P, _P, _P], _I),
    "otpu_fake_act": ([_P, _I, _I, _L, _I, _I, _I, _P, _L, _P, _L, _P], _I),
    "otpu_fake_act_f64": ([_P, _I, _I, _L, _I, _I, _I, _P, _L, _P, _L, _P], _I),
    "otpu_dequant": ([_P, _L, _P, _L, _I, _I, _I, _I, _P, _L, _P, _L, _P], _I),
    "otpu_mx_matmul": ([_P, _L, _P, _L, _P, _L, _P, _L, _I, _I, _I, _I, _I, _P, _L, _P], _I),
}


OTPU_ETIMEOUT = -6         # the binding's own code: the persistent step's error word was set


class OtpuError(RuntimeError):
    """A call the C ABI refused (the reference raises SimError for the same checks)."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


_lib = None


def load(path: str = LIB_PATH):
    """The library, with argument types set (no GPU needed to load it)."""
    global _lib
    if _lib is None:
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is not built: run `python -m opentpu_amd.build` "
                               "(there is no CPU fallback)")
        lib = C.CDLL(path)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        if lib.otpu_version() != ABI_VERSION:
            raise RuntimeError(f"{path} has ABI version {lib.otpu_version()}, this binding follows "
                               f"{ABI_VERSION}: rebuild it (python -m opentpu_amd.build)")
        _lib = lib
    return _lib


def call(name: str, *args) -> None:
    rc = getattr(load(), name)(*args)
    if rc != 0:
        raise OtpuError(rc, load().otpu_last_error().decode())


def torch():
    import torch as T
    if not T.cuda.is_available():
        raise RuntimeError("opentpu_amd needs a GPU (HIP device); none is visible")
    return T


def stream():
    """The current torch stream of the current device, as a hipStream_t."""
    return C.c_void_p(torch().cuda.current_stream().cuda_stream)


def ptr(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None


_NP2T = {np.float32: "float32", np.int8: "int8", np.uint8: "uint8", np.int64: "int64",
         np.int32: "int32", np.uint64: "uint64", np.float64: "float64"}


def dev(x, dtype):
    """A contiguous device tensor of dtype (a numpy dtype) from a numpy array or a tensor."""
    T = torch()
    tdt = getattr(T, _NP2T[np.dtype(dtype).type])
    if isinstance(x, T.Tensor):
        if x.dtype != tdt:
            if tdt == T.uint8 and x.dtype == T.int8 or tdt == T.int8 and x.dtype == T.uint8:
                x = x.view(tdt)
            else:
                x = x.to(tdt)
        return x.cuda().contiguous()
    a = np.ascontiguousarray(x)
    if a.dtype != np.dtype(dtype):
        if a.dtype.itemsize == np.dtype(dtype).itemsize and a.dtype.kind in "iu" and np.dtype(dtype).kind in "iu":
            a = a.view(dtype)
        else:
            a = a.astype(dtype)
    return T.from_numpy(a).cuda()


def empty(shape, dtype):
    T = torch()
    return T.empty(shape, dtype=getattr(T, _NP2T[np.dtype(dtype).type]), device="cuda")


def zeros(shape, dtype):
    T = torch()
    return T.zeros(shape, dtype=getattr(T, _NP2T[np.dtype(dtype).type]), device="cuda")


def is_numpy(x) -> bool:
    return isinstance(x, np.ndarray) or np.isscalar(x)


def host(t):
    return t.cpu().numpy()
