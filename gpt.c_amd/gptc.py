"""ctypes front end of libgptc_amd.so for Python callers (tests, bench).

The library's interface is gpt.c's C API (include/*.h): tensor_t,
runtime_init/synchronize, Attention() with forward/backward function
pointers, and the C-ABI kernel entry points of include/gpu_kernels.h.
This module only declares those signatures and moves numpy arrays in and
out of tensor_t; all compute happens in the library.  Loading fails
loudly when the library has not been built.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgptc_amd.so")

CPU, CUDA = 0, 1


class Tensor(ctypes.Structure):
    """tensor_t (include/tensor.h): 64-byte aligned, 64 bytes."""


_TO_FN = ctypes.CFUNCTYPE(None, ctypes.POINTER(Tensor), ctypes.c_int)
Tensor._fields_ = [
    ("t", ctypes.POINTER(ctypes.c_float)),
    ("ndims", ctypes.c_int),
    ("length", ctypes.c_int),
    ("shape", ctypes.c_int * 8),
    ("to", ctypes.c_void_p),
    ("device", ctypes.c_int),
    ("_pad", ctypes.c_byte * 4),
]
assert ctypes.sizeof(Tensor) == 64

TensorP = ctypes.POINTER(Tensor)


class AttentionT(ctypes.Structure):
    """attention_t (include/attention.h): 128 bytes with its 64-byte alignment."""
    _fields_ = [
        ("buffer", TensorP),
        ("cache", TensorP * 4),
        ("forward", ctypes.c_void_p),
        ("backward", ctypes.c_void_p),
        ("description", ctypes.c_void_p),
        ("num_parameters", ctypes.c_void_p),
        ("free_layer", ctypes.c_void_p),
        ("free_cache", ctypes.c_void_p),
        ("to", ctypes.c_void_p),
        ("n_embd", ctypes.c_int),
        ("n_heads", ctypes.c_int),
    ]


AttentionP = ctypes.POINTER(AttentionT)
_LAYER_FN = ctypes.CFUNCTYPE(TensorP, AttentionP, TensorP)
_VOID_FN = ctypes.CFUNCTYPE(None, AttentionP)
_INT_FN = ctypes.CFUNCTYPE(ctypes.c_int, AttentionP)
_MOVE_FN = ctypes.CFUNCTYPE(None, AttentionP, ctypes.c_int)

# Every symbol declared in include/*.h, with its ctypes signature.
_ci, _cf, _vp = ctypes.c_int, ctypes.c_float, ctypes.c_void_p
_ip = ctypes.POINTER(ctypes.c_int)
_fp = ctypes.POINTER(ctypes.c_float)
SIGNATURES = {
    # tensor.h
    "create_tensor": (TensorP, [_ip, _ci, _ci]),
    "randn": (TensorP, [_ip, _ci, _ci]),
    "zeros": (TensorP, [_ip, _ci, _ci]),
    "ones": (TensorP, [_ip, _ci, _ci]),
    "fill": (TensorP, [_ip, _ci, _cf, _ci]),
    "arange": (TensorP, [_ci, _ci, _ci, _ci]),
    "tensor_copy": (None, [TensorP, TensorP]),
    "shape": (None, [TensorP, ctypes.c_char_p]),
    "view": (None, [TensorP, _ip, _ci]),
    "tensor_load": (TensorP, [_vp, _ip, _ci, _ci]),
    "tensor_save": (None, [_vp, TensorP]),
    "free_tensor": (None, [TensorP]),
    "get_tensor_device": (None, [TensorP, ctypes.c_char_p]),
    "print_tensor": (None, [TensorP, _ci]),
    "print_shape": (None, [TensorP]),
    # runtime.h
    "runtime_init": (None, [_ci]),
    "runtime_destroy": (None, [_ci]),
    "synchronize": (None, [_ci]),
    # utils.h
    "check_error": (None, [ctypes.c_bool, ctypes.c_char_p, _ci, ctypes.c_char_p]),
    "malloc_check": (_vp, [ctypes.c_size_t, ctypes.c_char_p, _ci]),
    "aligned_malloc_check": (_vp, [ctypes.c_size_t, ctypes.c_size_t, ctypes.c_char_p, _ci]),
    # attention.h
    "Attention": (AttentionP, [_ci, _ci, _ci]),
    # dispatch.h
    "runtime_init_dispatch": (None, [_ci]),
    "runtime_destroy_dispatch": (None, [_ci]),
    "synchronize_dispatch": (None, [_ci]),
    "alloc_dispatch": (_vp, [ctypes.c_size_t, ctypes.c_size_t, _ci]),
    "free_dispatch": (None, [_vp, _ci]),
    "create_tensor_data_dispatch": (None, [TensorP]),
    "zeros_tensor_data_dispatch": (None, [TensorP]),
    "ones_tensor_data_dispatch": (None, [TensorP]),
    "fill_tensor_data_dispatch": (None, [TensorP, _cf]),
    "arange_tensor_data_dispatch": (None, [TensorP, _ci, _ci, _ci]),
    "move_tensor_data_dispatch": (None, [TensorP, _ci]),
    "copy_tensor_data_dispatch": (None, [TensorP, TensorP]),
    "attention_forward_dispatch": (None, [TensorP, TensorP, _ci, ctypes.POINTER(TensorP), TensorP]),
    "attention_backward_dispatch": (None, [TensorP, ctypes.POINTER(TensorP), _ci, TensorP]),
    # gpu_kernels.h
    "runtime_init_cuda": (None, []),
    "runtime_destroy_cuda": (None, []),
    "synchronize_cuda": (None, []),
    "alloc_cuda": (_vp, [ctypes.c_size_t]),
    "free_cuda": (None, [_vp]),
    "move_tensor_to_host_cuda": (None, [TensorP]),
    "move_tensor_to_device_cuda": (None, [TensorP]),
    "create_tensor_data_cuda": (None, [TensorP]),
    "zeros_tensor_data_cuda": (None, [TensorP]),
    "ones_tensor_data_cuda": (None, [TensorP]),
    "fill_tensor_data_cuda": (None, [TensorP, _cf]),
    "arange_tensor_data_cuda": (None, [TensorP, _ci, _ci, _ci]),
    "copy_tensor_data_cuda": (None, [TensorP, TensorP]),
    "attention_forward_cuda_kernel": (None, [TensorP, TensorP, _ci, ctypes.POINTER(TensorP), TensorP]),
    "attention_backward_cuda_kernel": (None, [TensorP, ctypes.POINTER(TensorP), _ci, TensorP]),
    "gptc_stream": (_vp, []),
    "gptc_set_kernel_events": (None, [ctypes.POINTER(_vp), _ci]),
    "gptc_attention_state_floats": (ctypes.c_longlong, [_ci, _ci, _ci, _ci]),
    "attention_decode_cuda_kernel": (None, [TensorP, TensorP, TensorP, _ci, _ci, TensorP]),
    # rand.h
    "manual_seed": (None, [_vp, ctypes.c_uint]),
    "randint32": (ctypes.c_uint, [_vp]),
    "randint64": (ctypes.c_ulonglong, [_vp]),
    "randfloat32": (ctypes.c_float, [_vp]),
    "randfloat64": (ctypes.c_double, [_vp]),
    "uniform_": (None, [_fp, ctypes.c_uint, _cf, _cf, _vp]),
    "normal_": (None, [_fp, ctypes.c_uint, _cf, _cf, _vp]),
    "gptc_normal_seeded": (None, [_fp, ctypes.c_uint, _cf, _cf, ctypes.c_uint]),
}

MT19937_STATE_BYTES = 8 + 4 + 4 + 624 * 4 + 2 * 4  # mt19937_state in include/rand.h


def build():
    """Compile libgptc_amd.so for gfx950 (hipcc + gcc; cross-compiles without a GPU)."""
    subprocess.run(["make", "-B", "-j8", "-C", HERE], check=True, stdout=subprocess.DEVNULL)


def load(path=None):
    """dlopen the library and attach signatures; raises if it is missing.

    The path defaults to the in-tree build, or $GPTC_LIB when set (to compare
    two builds of the library side by side).
    """
    path = path or os.environ.get("GPTC_LIB") or LIB_PATH
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built: run __graft_entry__.build() (make -C gpt.c_amd)")
    lib = ctypes.CDLL(path, mode=ctypes.RTLD_GLOBAL)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def _shape_arr(shape):
    return (ctypes.c_int * len(shape))(*shape)


class Runtime:
    """Thin owner of the loaded library with numpy <-> tensor_t helpers."""

    def __init__(self, lib=None):
        self.lib = lib or load()

    # ---- runtime ----
    def init(self):
        self.lib.runtime_init(CUDA)

    def sync(self):
        self.lib.synchronize(CUDA)

    def stream(self):
        return self.lib.gptc_stream()

    # ---- tensors ----
    def empty(self, shape, device=CUDA):
        return self.lib.create_tensor(_shape_arr(shape), len(shape), device)

    def from_numpy(self, arr, device=CUDA):
        arr = np.ascontiguousarray(arr, dtype=np.float32)
        t = self.lib.create_tensor(_shape_arr(arr.shape), arr.ndim, CPU)
        if arr.size:
            ctypes.memmove(t.contents.t, arr.ctypes.data, arr.nbytes)
        if device != CPU:
            self.lib.move_tensor_data_dispatch(t, device)
        return t

    def to_numpy(self, t):
        """Copy of a tensor's data as a numpy array (the tensor is left in place)."""
        tc = t.contents
        shp = tuple(tc.shape[i] for i in range(tc.ndims))
        if tc.device == CPU:
            out = np.empty(shp, np.float32)
            if out.size:
                ctypes.memmove(out.ctypes.data, tc.t, out.nbytes)
            return out
        tmp = self.lib.create_tensor(_shape_arr(shp), len(shp), tc.device)
        self.lib.tensor_copy(tmp, t)
        self.lib.move_tensor_data_dispatch(tmp, CPU)
        out = self.to_numpy(tmp)
        self.lib.free_tensor(tmp)
        return out

    def free(self, t):
        self.lib.free_tensor(t)

    # ---- inputs ----
    def normal(self, shape, seed, mean=0.0, std=1.0):
        """numpy array drawn with torch-identical manual_seed(seed) + normal_()."""
        out = np.empty(shape, np.float32)
        self.lib.gptc_normal_seeded(out.ctypes.data_as(_fp), out.size, mean, std, seed)
        return out


class AttentionLayer:
    """The library's Attention() object driven through its function pointers."""

    def __init__(self, rt, n_embd, n_heads, block_size):
        self.rt = rt
        self.ptr = rt.lib.Attention(n_embd, n_heads, block_size)
        s = self.ptr.contents
        self._fwd = ctypes.cast(s.forward, _LAYER_FN)
        self._bwd = ctypes.cast(s.backward, _LAYER_FN)
        self._free_layer = ctypes.cast(s.free_layer, _VOID_FN)
        self._free_cache = ctypes.cast(s.free_cache, _VOID_FN)
        self._to = ctypes.cast(s.to, _MOVE_FN)
        self._nparams = ctypes.cast(s.num_parameters, _INT_FN)

    def to(self, device):
        self._to(self.ptr, device)

    def forward(self, x):
        return self._fwd(self.ptr, x)

    def backward(self, dy):
        return self._bwd(self.ptr, dy)

    def num_parameters(self):
        return self._nparams(self.ptr)

    def cache(self, i):
        return self.ptr.contents.cache[i]

    @property
    def buffer(self):
        return self.ptr.contents.buffer

    def free_cache(self):
        self._free_cache(self.ptr)

    def free(self):
        if self.ptr:
            self._free_layer(self.ptr)
            self.ptr = None
