"""TEST INFRASTRUCTURE -- ctypes front end of the CPU oracle (liboracle.so).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module; the product (gpt.c_amd/) never does.

The oracle restates gpt.c's CPU attention kernel
(/root/reference/kernels/src/cpu/Attention.c:8-301) in C over OpenBLAS,
which it loads at run time from the scipy/numpy wheels of this image; see
attention_oracle.c for the step-by-step correspondence.  It also carries an
fp64 brute-force version of the same mathematics used to pin it.  The other
layers of the model (Linear, LayerNorm, GELU, Softmax, Embedding,
CrossEntropy, AdamW) are restated in ops_oracle.c; RefOps loads gpt.c's own
CPU kernels for those layers, compiled in place under oracle/_ref, to check
the restatements.
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
        _declare_ops(lib)
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


_ci, _cl, _cf = ctypes.c_int, ctypes.c_long, ctypes.c_float
_vp = ctypes.c_void_p


def _declare_ops(lib):
    f, v = _f32p, _vp
    sig = {
        "oracle_linear_forward": [f, v, f, _ci, _ci, _ci, f],
        "oracle_linear_backward": [f, f, f, _ci, _ci, _ci, f, v, f],
        "oracle_layer_norm_forward": [f, f, v, _ci, _ci, _cf, f, f, f],
        "oracle_layer_norm_backward": [f, f, f, f, f, _ci, _ci, f, v, f],
        "oracle_gelu_forward": [f, _cl, f],
        "oracle_gelu_backward": [f, f, _cl, f],
        "oracle_softmax_forward": [f, _ci, _ci, f],
        "oracle_softmax_backward": [f, f, _ci, _ci, f],
        "oracle_embedding_forward": [f, f, _ci, _ci, f],
        "oracle_embedding_backward": [f, f, _ci, _ci, _ci, f],
        "oracle_cross_entropy_forward": [f, f, _ci, _ci, f, f],
        "oracle_cross_entropy_backward": [f, f, f, _ci, _ci, f],
        "oracle_adamw": [f, f, f, f, _cl, _cf, _cf, _cf, _cf, _cf, _ci],
    }
    for name, args in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = None


def _c32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a):
    return None if a is None else a.ctypes.data


class Ops:
    """numpy front end of ops_oracle.c (gpt.c's CPU kernels for the non-attention
    layers).  Shapes: rows = product of the leading dimensions."""

    def __init__(self, oracle):
        self.lib = oracle.lib

    def linear_forward(self, W, b, x):
        W, x = _c32(W), _c32(x)
        b = None if b is None else _c32(b)
        out_f, in_f = W.shape
        rows = x.size // in_f
        y = np.empty(x.shape[:-1] + (out_f,), np.float32)
        self.lib.oracle_linear_forward(W, _ptr(b), x, rows, in_f, out_f, y)
        return y

    def linear_backward(self, g, x, W, dW, db):
        """Returns dx; dW and db (float32 arrays or None) are accumulated in place."""
        g, x, W = _c32(g), _c32(x), _c32(W)
        out_f, in_f = W.shape
        rows = g.size // out_f
        dx = np.empty(x.shape, np.float32)
        self.lib.oracle_linear_backward(g, x, W, rows, in_f, out_f, dW, _ptr(db), dx)
        return dx

    def layer_norm_forward(self, x, W, b, eps=1e-5):
        x, W = _c32(x), _c32(W)
        b = None if b is None else _c32(b)
        C = x.shape[-1]
        rows = x.size // C
        y = np.empty_like(x)
        mean = np.empty(x.shape[:-1], np.float32)
        rstd = np.empty(x.shape[:-1], np.float32)
        self.lib.oracle_layer_norm_forward(x, W, _ptr(b), rows, C, eps, mean, rstd, y)
        return y, mean, rstd

    def layer_norm_backward(self, g, x, mean, rstd, W, dW, db, dx):
        """Accumulates into dW, db (or None) and dx in place."""
        g, x, mean, rstd, W = _c32(g), _c32(x), _c32(mean), _c32(rstd), _c32(W)
        C = x.shape[-1]
        self.lib.oracle_layer_norm_backward(g, x, mean, rstd, W, x.size // C, C, dW, _ptr(db), dx)

    def gelu_forward(self, x):
        x = _c32(x)
        y = np.empty_like(x)
        self.lib.oracle_gelu_forward(x, x.size, y)
        return y

    def gelu_backward(self, g, x):
        g, x = _c32(g), _c32(x)
        dx = np.empty_like(x)
        self.lib.oracle_gelu_backward(g, x, x.size, dx)
        return dx

    def softmax_forward(self, x):
        x = _c32(x)
        y = np.empty_like(x)
        self.lib.oracle_softmax_forward(x, x.size // x.shape[-1], x.shape[-1], y)
        return y

    def softmax_backward(self, g, p):
        g, p = _c32(g), _c32(p)
        dx = np.empty_like(p)
        self.lib.oracle_softmax_backward(g, p, p.size // p.shape[-1], p.shape[-1], dx)
        return dx

    def embedding_forward(self, W, ids):
        W, ids = _c32(W), _c32(ids)
        C = W.shape[1]
        y = np.empty(ids.shape + (C,), np.float32)
        self.lib.oracle_embedding_forward(W, ids, ids.size, C, y)
        return y

    def embedding_backward(self, g, ids, dW):
        """dW[ids[i % len(ids)]] += g[i] in place."""
        g, ids = _c32(g), _c32(ids)
        C = dW.shape[1]
        self.lib.oracle_embedding_backward(g, ids, g.size // C, ids.size, C, dW)

    def cross_entropy_forward(self, logits, targets):
        logits, targets = _c32(logits), _c32(targets)
        V = logits.shape[-1]
        lsm = np.empty_like(logits)
        loss = np.zeros(1, np.float32)
        self.lib.oracle_cross_entropy_forward(logits, targets, logits.size // V, V, lsm, loss)
        return lsm, float(loss[0])

    def cross_entropy_backward(self, g, lsm, targets):
        g, lsm, targets = _c32(g), _c32(lsm), _c32(targets)
        V = lsm.shape[-1]
        dx = np.empty_like(lsm)
        self.lib.oracle_cross_entropy_backward(g, lsm, targets, lsm.size // V, V, dx)
        return dx

    def adamw(self, p, g, m, v, lr, beta1, beta2, weight_decay, eps, step):
        """One AdamW step on float32 arrays p, m, v in place."""
        self.lib.oracle_adamw(p, _c32(g), m, v, p.size, lr, beta1, beta2, weight_decay, eps, step)


REF_OPS_PATH = os.path.join(HERE, "_ref", "libgptc_ref_ops.so")


class _RefTensor(ctypes.Structure):
    """gpt.c's tensor_t (include/tensor.h:45-52): 64 bytes, 64-byte aligned."""
    _fields_ = [("t", ctypes.c_void_p), ("ndims", ctypes.c_int), ("length", ctypes.c_int),
                ("shape", ctypes.c_int * 8), ("to", ctypes.c_void_p), ("device", ctypes.c_int),
                ("_pad", ctypes.c_byte * 4)]


class RefOps:
    """gpt.c's own CPU kernels for LayerNorm, GELU, Softmax, Embedding,
    CrossEntropy and AdamW (kernels/src/cpu/*.c compiled unmodified into
    oracle/_ref by `make -C oracle ref`).  Used only to check Ops."""

    def __init__(self, path=REF_OPS_PATH):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        self.lib = ctypes.CDLL(path)
        self._keep = []

    @staticmethod
    def _aligned(arr):
        """64-byte aligned float32 copy (gpt.c's kernels assume 64-byte
        aligned data, __builtin_assume_aligned(..., 64))."""
        arr = np.asarray(arr, dtype=np.float32)
        buf = np.empty(arr.size + 16, np.float32)
        off = (-buf.ctypes.data % 64) // 4
        out = buf[off:off + arr.size].reshape(arr.shape)
        out[...] = arr
        return out

    def _t(self, arr):
        src = arr
        arr = self._aligned(arr)
        t = _RefTensor()
        t.t = arr.ctypes.data
        t.ndims = arr.ndim
        t.length = arr.size
        for i, d in enumerate(arr.shape):
            t.shape[i] = d
        t.device = 0
        self._keep += [arr, t]
        if isinstance(src, np.ndarray) and src.dtype == np.float32:
            self._writeback.append((src, arr))
        return ctypes.pointer(t), arr

    def call(self, name, *arrays):
        """Call name(tensor_t*...) with each array wrapped (None -> NULL; a list
        -> tensor_t**; ctypes scalars passed as they are).  Float32 arrays are
        updated in place; the wrapped copies are returned as well."""
        args, outs = [], []
        self._keep, self._writeback = [], []
        for a in arrays:
            if a is None:
                args.append(None)
                outs.append(None)
            elif isinstance(a, list):
                ptrs = (ctypes.POINTER(_RefTensor) * len(a))()
                arrs = []
                for i, x in enumerate(a):
                    ptrs[i], arr = self._t(x)
                    arrs.append(arr)
                self._keep.append(ptrs)
                args.append(ptrs)
                outs.append(arrs)
            elif isinstance(a, ctypes._SimpleCData):
                args.append(a)
                outs.append(a)
            else:
                p, arr = self._t(a)
                args.append(p)
                outs.append(arr)
        getattr(self.lib, name)(*args)
        for src, arr in self._writeback:  # in-place semantics for the caller's arrays
            src[...] = arr
        return outs
