"""TEST INFRASTRUCTURE -- ctypes front end of the CPU oracle (liboracle.so).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module; the product (gpt.c_amd/) never does.

The oracle restates gpt.c's CPU attention kernel
(/root/reference/kernels/src/cpu/Attention.c:8-301) in C over OpenBLAS,
which it loads at run time from the scipy/numpy wheels of this image; see
attention_oracle.c for the step-by-step correspondence.  It also carries an
fp64 brute-force version of the same mathematics used to pin it.
"""
import ctypes
import glob
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")


def build():
    """Compile liboracle.so (gcc, seconds)."""
    subprocess.run(["make", "-B", "-C", HERE], check=True, stdout=subprocess.DEVNULL)


def find_openblas():
    """Path of an OpenBLAS shared library shipped with this image's wheels.

    LP64 (scipy) first, then the ILP64 builds.  Raises if none exists: the
    oracle never substitutes a naive loop for BLAS.
    """
    env = os.environ.get("ORACLE_OPENBLAS")
    if env:
        return env
    cands = []
    try:
        import scipy
        cands += sorted(glob.glob(os.path.join(os.path.dirname(scipy.__file__), os.pardir,
                                               "scipy.libs", "libscipy_openblas-*.so")))
    except ImportError:
        pass
    cands += sorted(glob.glob(os.path.join(os.path.dirname(np.__file__), os.pardir,
                                           "numpy.libs", "libscipy_openblas64_*.so")))
    cands += sorted(glob.glob(os.path.join(os.path.dirname(np.__file__), os.pardir,
                                           "numpy.libs", "libopenblas*.so")))
    for c in cands:
        if os.path.exists(c):
            return os.path.realpath(c)
    raise RuntimeError("no OpenBLAS shared library found for the CPU oracle")


class Oracle:
    def __init__(self, threads=None):
        if not os.path.exists(LIB_PATH):
            build()
        lib = ctypes.CDLL(LIB_PATH)
        lib.oracle_init.argtypes = [ctypes.c_char_p]
        lib.oracle_init.restype = ctypes.c_int
        lib.oracle_blas_config.restype = ctypes.c_char_p
        lib.oracle_set_threads.argtypes = [ctypes.c_int]
        ci = ctypes.c_int
        lib.oracle_attention_forward.argtypes = [_f32p, ci, ci, ci, ci, _f32p, ci, _f32p, _f32p, _f32p, _f32p, _f32p]
        lib.oracle_attention_backward.argtypes = [_f32p, ci, ci, ci, ci, _f32p, _f32p, _f32p, _f32p, _f32p]
        lib.oracle_attention_fp64.argtypes = [_f32p, ctypes.c_void_p, ci, ci, ci, ci, _f64p, ctypes.c_void_p,
                                              ctypes.c_void_p]
        self.blas_path = find_openblas()
        if lib.oracle_init(self.blas_path.encode()) != 0:
            raise RuntimeError("oracle: could not load OpenBLAS from " + self.blas_path)
        self.lib = lib
        if threads is not None:
            self.set_threads(threads)

    @property
    def blas_config(self):
        return self.lib.oracle_blas_config().decode()

    def set_threads(self, n):
        self.lib.oracle_set_threads(int(n))

    def forward(self, x, n_heads, mask=None):
        """x (B,T,3C) float32 -> (y (B,T,C), q, k, v (B,H,T,D), P (B,H,T,T)).

        mask defaults to tril(ones(T, T)), the layer's buffer at block = T.
        """
        x = np.ascontiguousarray(x, dtype=np.float32)
        B, T, C3 = x.shape
        C = C3 // 3
        H = n_heads
        D = C // H
        if mask is None:
            mask = np.tril(np.ones((T, T), dtype=np.float32))
        mask = np.ascontiguousarray(mask, dtype=np.float32)
        q = np.empty((B, H, T, D), np.float32)
        k = np.empty_like(q)
        v = np.empty_like(q)
        att = np.empty((B, H, T, T), np.float32)
        y = np.empty((B, T, C), np.float32)
        self.lib.oracle_attention_forward(x, B, T, C, H, mask, mask.shape[-1], q, k, v, att, y)
        return y, q, k, v, att

    def backward(self, dy, n_heads, q, k, v, att):
        """dy (B,T,C) + forward caches -> dqkv (B,T,3C)."""
        dy = np.ascontiguousarray(dy, dtype=np.float32)
        B, T, C = dy.shape
        dqkv = np.empty((B, T, 3 * C), np.float32)
        self.lib.oracle_attention_backward(dy, B, T, C, n_heads, q, k, v, att, dqkv)
        return dqkv

    def fp64(self, x, n_heads, dy=None):
        """fp64 brute force: (y, lse (B,H,T) natural log, dqkv or None)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        B, T, C3 = x.shape
        C = C3 // 3
        y = np.empty((B, T, C), np.float64)
        lse = np.empty((B, n_heads, T), np.float64)
        dqkv = None
        dy_ptr = None
        if dy is not None:
            dy = np.ascontiguousarray(dy, dtype=np.float32)
            dqkv = np.empty((B, T, C3), np.float64)
            dy_ptr = dy.ctypes.data
        self.lib.oracle_attention_fp64(x, dy_ptr, B, T, C, n_heads, y, lse.ctypes.data,
                                       dqkv.ctypes.data if dqkv is not None else None)
        return y, lse, dqkv
