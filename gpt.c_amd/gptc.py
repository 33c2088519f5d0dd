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
    "fopen_check": (_vp, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, _ci]),
    "fread_check": (None, [_vp, ctypes.c_size_t, ctypes.c_size_t, _vp, ctypes.c_char_p, _ci]),
    "fclose_check": (None, [_vp, ctypes.c_char_p, _ci]),
    "fseek_check": (None, [_vp, ctypes.c_long, _ci, ctypes.c_char_p, _ci]),
    "print_table": (None, [ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_char_p), ctypes.c_size_t]),
    "tensor_check": (None, [TensorP, ctypes.c_char_p, _ci]),
    "tensor_device_check": (None, [TensorP, TensorP, ctypes.c_char_p, _ci]),
    # dataloader.h, tokenizer.h, checkpoint.h
    "DataLoader": (_vp, [ctypes.c_char_p, _ci, _ci]),
    "Tokenizer": (_vp, [ctypes.c_char_p]),
    "safe_printf": (None, [ctypes.c_char_p]),
    "gptc_load_model": (_vp, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_size_t)]),
    "gptc_save_model": (None, [ctypes.c_char_p, _vp, ctypes.c_size_t]),
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
    "saxpy_dispatch": (None, [_ci, _cf, TensorP, _ci, _ci, TensorP, _ci, _ci]),
    "sgemm_dispatch": (None, [_ci, _ci, _ci, _ci, _ci, _cf, TensorP, _ci, _ci, TensorP, _ci, _ci, _cf, TensorP, _ci,
                              _ci]),
    "linear_forward_dispatch": (None, [TensorP, TensorP, TensorP, TensorP]),
    "linear_backward_dispatch": (None, [TensorP, TensorP, TensorP, TensorP, TensorP, TensorP]),
    "layer_norm_forward_dispatch": (None, [TensorP, TensorP, TensorP, _cf, ctypes.POINTER(TensorP), TensorP]),
    "layer_norm_backward_dispatch": (None, [TensorP, ctypes.POINTER(TensorP), TensorP, TensorP, TensorP, TensorP]),
    "gelu_forward_dispatch": (None, [TensorP, TensorP]),
    "gelu_backward_dispatch": (None, [TensorP, TensorP, TensorP]),
    "softmax_forward_dispatch": (None, [TensorP, TensorP]),
    "softmax_backward_dispatch": (None, [TensorP, TensorP, TensorP]),
    "embedding_forward_dispatch": (None, [TensorP, TensorP, TensorP]),
    "embedding_backward_dispatch": (None, [TensorP, TensorP, TensorP]),
    "cross_entropy_forward_dispatch": (None, [TensorP, TensorP, ctypes.POINTER(TensorP), TensorP]),
    "cross_entropy_backward_dispatch": (None, [TensorP, ctypes.POINTER(TensorP), TensorP]),
    "step_adamW_dispatch": (None, [ctypes.POINTER(TensorP)] * 4 + [_ci, _cf, _cf, _cf, _cf, _cf, _ci]),
    "zero_grad_adamW_dispatch": (None, [ctypes.POINTER(TensorP), _ci]),
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
    "gptc_attention_set_state_limit": (ctypes.c_longlong, [ctypes.c_longlong]),
    "gptc_attention_set_scratch_limit": (ctypes.c_longlong, [ctypes.c_longlong]),
    "attention_decode_cuda_kernel": (None, [TensorP, TensorP, TensorP, _ci, _ci, TensorP]),
    "attention_decode_noalloc_cuda_kernel": (None, [TensorP, TensorP, TensorP, _ci, _ci, TensorP]),
    "gptc_decode_noalloc_scratch_floats": (ctypes.c_longlong, []),
    "gptc_retain_cuda": (None, [_vp]),
    "gptc_attention_forward_bias": (TensorP, [_vp, TensorP, TensorP]),
    "gptc_attention_backward_bias": (TensorP, [_vp, TensorP, TensorP, TensorP]),
    "gptc_linear_forward_nobias": (TensorP, [_vp, TensorP]),
    "gptc_linear_backward_nodb": (TensorP, [_vp, TensorP]),
    "gptc_gelu_forward_bias": (TensorP, [_vp, TensorP, TensorP]),
    "gptc_gelu_backward_bias": (TensorP, [_vp, TensorP, TensorP, TensorP]),
    "gptc_gelu_forward_bias_cuda": (None, [TensorP, TensorP, TensorP]),
    "gptc_gelu_backward_bias_cuda": (None, [TensorP, TensorP, TensorP, TensorP, TensorP]),
    "gptc_attention_forward_qkv_bias": (None, [TensorP, TensorP, TensorP, _ci, ctypes.POINTER(TensorP), TensorP]),
    "gptc_attention_backward_qkv_bias": (None, [TensorP, ctypes.POINTER(TensorP), TensorP, _ci, TensorP, TensorP]),
    "gptc_attention_block_schedule": (_ci, [_ci, _ci, _ci, _ci, ctypes.POINTER(_ci), ctypes.POINTER(_ci), _ci,
                                             ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_ci)]),
    "gptc_attention_block_schedule_pool": (_ci, [_ci, _ci, _ci, _ci, ctypes.POINTER(_ci), ctypes.POINTER(_ci), _ci,
                                                  ctypes.POINTER(_ci)]),
    "gptc_attention_key_schedule": (_ci, [_ci, _ci, _ci, _ci, ctypes.POINTER(_ci), ctypes.POINTER(_ci), _ci,
                                           ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_ci)]),
    "saxpy_cuda": (None, [_ci, _cf, TensorP, _ci, _ci, TensorP, _ci, _ci]),
    "sgemm_cuda": (None, [_ci, _ci, _ci, _ci, _ci, _cf, TensorP, _ci, _ci, TensorP, _ci, _ci, _cf, TensorP, _ci,
                          _ci]),
    "sgemm_strided_batched_cuda": (None, [_ci, _ci, _ci, _ci, _ci, _cf, TensorP, _ci, _ci, TensorP, _ci, _ci, _cf,
                                          TensorP, _ci, _ci, _ci]),
    "linear_forward_cuda_kernel": (None, [TensorP, TensorP, TensorP, TensorP]),
    "linear_backward_cuda_kernel": (None, [TensorP, TensorP, TensorP, TensorP, TensorP, TensorP]),
    "layer_norm_forward_cuda_kernel": (None, [TensorP, TensorP, TensorP, _cf, ctypes.POINTER(TensorP), TensorP]),
    "layer_norm_backward_cuda_kernel": (None, [TensorP, ctypes.POINTER(TensorP), TensorP, TensorP, TensorP,
                                               TensorP]),
    "gptc_layer_norm_backward_set": (None, [TensorP, ctypes.POINTER(TensorP), TensorP, TensorP, TensorP, TensorP]),
    "gelu_forward_cuda_kernel": (None, [TensorP, TensorP]),
    "gelu_backward_cuda_kernel": (None, [TensorP, TensorP, TensorP]),
    "softmax_forward_cuda_kernel": (None, [TensorP, TensorP]),
    "softmax_backward_cuda_kernel": (None, [TensorP, TensorP, TensorP]),
    "embedding_forward_cuda_kernel": (None, [TensorP, TensorP, TensorP]),
    "embedding_backward_cuda_kernel": (None, [TensorP, TensorP, TensorP]),
    "cross_entropy_forward_cuda_kernel": (None, [TensorP, TensorP, ctypes.POINTER(TensorP), TensorP]),
    "cross_entropy_backward_cuda_kernel": (None, [TensorP, ctypes.POINTER(TensorP), TensorP]),
    "step_adamW_cuda_kernel": (None, [ctypes.POINTER(TensorP)] * 4 + [_ci, _cf, _cf, _cf, _cf, _cf, _ci]),
    "zero_grad_adamW_cuda_kernel": (None, [ctypes.POINTER(TensorP), _ci]),
    "gptc_linear_rows_cuda": (None, [TensorP, TensorP, TensorP, TensorP, _ci, TensorP]),
    "gptc_embed_token_cuda": (None, [TensorP, TensorP, TensorP, _ci, TensorP]),
    "gptc_argmax_cuda": (None, [TensorP, TensorP]),
    # generate.h
    "gptc_kv_cache_create": (_vp, [_vp, _ci, _ci]),
    "gptc_kv_cache_free": (None, [_vp]),
    "gptc_gpt2_decode": (TensorP, [_vp, _vp, TensorP, _ci]),
    "gptc_gpt2_generate": (None, [_vp, _vp, TensorP, _ci, _ci]),
    # tensor.h (BLAS front ends)
    "saxpy": (None, [_ci, _cf, TensorP, _ci, _ci, TensorP, _ci, _ci]),
    "sgemm": (None, [_ci, _ci, _ci, _ci, _ci, _cf, TensorP, _ci, _ci, TensorP, _ci, _ci, _cf, TensorP, _ci, _ci]),
    "uniform": (None, [TensorP, _cf, _cf]),
    # model layers (linear.h, layer_norm.h, embedding.h, activation.h, loss.h, optim.h, blocks.h, transformer.h)
    "Linear": (_vp, [_ci, _ci, _ci]),
    "LayerNorm": (_vp, [_ci, _cf, _ci]),
    "Embedding": (_vp, [_ci, _ci]),
    "GELU": (_vp, []),
    "Softmax": (_vp, []),
    "CrossEntropyLoss": (_vp, []),
    "AdamW": (_vp, [ctypes.POINTER(TensorP), ctypes.POINTER(TensorP), _ci, _cf, _cf, _cf, _cf, _cf]),
    "MLP": (_vp, [_ci, _ci, _ci]),
    "SelfAttention": (_vp, [_ci, _ci, _ci, _ci]),
    "Block": (_vp, [_ci, _ci, _ci, _ci]),
    "GPT2": (_vp, [_vp]),
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
    """Compile libgptc_amd.so for gfx950 (hipcc + gcc; cross-compiles without a GPU), and the GEMM tuner."""
    subprocess.run(["make", "-B", "-j8", "-C", HERE, "all", "tune"], check=True, stdout=subprocess.DEVNULL)


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


# ---- model layers (include/blocks.h, transformer.h, loss.h, optim.h) ----
TensorPP = ctypes.POINTER(TensorP)
_MODEL_FNS = ["forward", "backward", "description", "num_parameters", "free_layer", "free_cache", "parameters",
              "gradients", "load_state_dict", "to"]


class SelfAttentionT(ctypes.Structure):
    """self_attention_t (include/blocks.h)."""
    _fields_ = ([("n_embd", _ci), ("n_heads", _ci), ("use_bias", _ci), ("block_size", _ci),
                 ("_num_param_tensors", _ci), ("_pad", ctypes.c_byte * 4),
                 ("qkv", _vp), ("attn", _vp), ("c_proj", _vp)] + [(n, _vp) for n in _MODEL_FNS])


class GPT2T(ctypes.Structure):
    """gpt2_t (include/transformer.h)."""
    _fields_ = ([("n_embd", _ci), ("n_heads", _ci), ("n_layers", _ci), ("block_size", _ci), ("vocab_size", _ci),
                 ("_num_param_tensors", _ci), ("layers", _vp), ("wpe", _vp), ("wte", _vp), ("lm_head", _vp),
                 ("ln_f", _vp)] + [(n, _vp) for n in _MODEL_FNS[:9]] +
                [("fast_load_state_dict", _vp), ("to", _vp)])


class GPT2Config(ctypes.Structure):
    _fields_ = [("block_size", _ci), ("vocab_size", _ci), ("n_layers", _ci), ("n_heads", _ci), ("n_embd", _ci)]


class CrossEntropyLossT(ctypes.Structure):
    """cross_entropy_loss_t (include/loss.h)."""
    _fields_ = [("softmax", _vp), ("cache", TensorP * 2), ("forward", _vp), ("backward", _vp), ("description", _vp),
                ("num_parameters", _vp), ("free_layer", _vp), ("free_cache", _vp), ("to", _vp)]


class AdamWT(ctypes.Structure):
    """adamW_t (include/optim.h)."""
    _fields_ = [("parameters", TensorPP), ("gradients", TensorPP), ("m", TensorPP), ("v", TensorPP),
                ("lr", _cf), ("beta1", _cf), ("beta2", _cf), ("eps", _cf), ("weight_decay", _cf),
                ("n_parameters", _ci), ("step_t", _ci), ("_pad", ctypes.c_byte * 4),
                ("step", _vp), ("zero_grad", _vp), ("free_layer", _vp)]


def _fn(addr, res, *args):
    return ctypes.CFUNCTYPE(res, *args)(addr)


class _Layer:
    """A gpt.c layer object (forward/backward/parameters/... function pointers)."""

    def __init__(self, rt, ptr, struct):
        self.rt, self.ptr = rt, ctypes.cast(ptr, ctypes.POINTER(struct))
        self.s = self.ptr.contents
        self.raw = ctypes.c_void_p(ptr)

    def forward(self, x):
        return _fn(self.s.forward, TensorP, _vp, TensorP)(self.raw, x)

    def backward(self, g):
        return _fn(self.s.backward, TensorP, _vp, TensorP)(self.raw, g)

    def n_params(self):
        return self.s._num_param_tensors

    def _tensor_list(self, fn):
        """Call a parameters()/gradients() function pointer; the malloc'd array is
        read as plain addresses (indexing it would alias its memory) and freed."""
        arr = _fn(fn, _vp, _vp)(self.raw)
        addrs = ctypes.cast(arr, ctypes.POINTER(ctypes.c_void_p))
        vals = [addrs[i] for i in range(self.n_params())]
        _libc_free(arr)
        return [ctypes.cast(v, TensorP) for v in vals]

    def parameters(self):
        return self._tensor_list(self.s.parameters)

    def gradients(self):
        return self._tensor_list(self.s.gradients)

    def to(self, device):
        _fn(self.s.to, None, _vp, _ci)(self.raw, device)

    def num_parameters(self):
        return _fn(self.s.num_parameters, _ci, _vp)(self.raw)

    def free_cache(self):
        _fn(self.s.free_cache, None, _vp)(self.raw)

    def free(self):
        if self.raw:
            _fn(self.s.free_layer, None, _vp)(self.raw)
            self.raw = None

    def load_arrays(self, arrays):
        """load_state_dict from numpy arrays (host tensors, freed afterwards)."""
        ts = [self.rt.from_numpy(a, CPU) for a in arrays]
        arr = (TensorP * len(ts))(*ts)
        _fn(self.s.load_state_dict, None, _vp, TensorPP)(self.raw, arr)
        for t in ts:
            self.rt.free(t)


def _libc_free(p):
    ctypes.CDLL(None).free(ctypes.cast(p, _vp))


class SelfAttentionBlock(_Layer):
    """SelfAttention(n_embd, n_heads, block_size, use_bias): qkv -> attention -> c_proj."""

    def __init__(self, rt, n_embd, n_heads, block_size, use_bias=1):
        super().__init__(rt, rt.lib.SelfAttention(n_embd, n_heads, block_size, use_bias), SelfAttentionT)


class GPT2Model(_Layer):
    """GPT2(config) driven through its function pointers."""

    def __init__(self, rt, block_size, vocab_size, n_layers, n_heads, n_embd):
        self.cfg = GPT2Config(block_size, vocab_size, n_layers, n_heads, n_embd)
        super().__init__(rt, rt.lib.GPT2(ctypes.byref(self.cfg)), GPT2T)

    @classmethod
    def from_checkpoint(cls, rt, path):
        """gptc_load_model(path): a GPT2 on the CPU; returns (model, steps)."""
        steps = ctypes.c_size_t()
        raw = rt.lib.gptc_load_model(os.fsencode(path), ctypes.byref(steps))
        model = cls.__new__(cls)
        _Layer.__init__(model, rt, raw, GPT2T)
        return model, steps.value

    def save(self, path, steps=0):
        """gptc_save_model(path, model, steps)."""
        self.rt.lib.gptc_save_model(os.fsencode(path), self.raw, steps)

    # Per-block parameters in the order block_t's parameters() lists them
    # (ln1, attention qkv and c_proj, ln2, MLP c_fc and c_proj; weight, bias).
    BLOCK_PARAMS = ("ln1.W", "ln1.b", "qkv.W", "qkv.b", "attn_proj.W", "attn_proj.b",
                    "ln2.W", "ln2.b", "fc.W", "fc.b", "mlp_proj.W", "mlp_proj.b")

    def param_layout(self):
        """(name, shape) of every parameter in parameters() order, the shapes
        read from the model's own tensors."""
        names = ["wte", "wpe"] + [f"h{i}.{n}" for i in range(self.s.n_layers) for n in self.BLOCK_PARAMS] + \
            ["ln_f.W", "ln_f.b"]
        ts = self.parameters()
        assert len(ts) == len(names), (len(ts), len(names))
        return [(n, tuple(t.contents.shape[:t.contents.ndims])) for n, t in zip(names, ts)]

    def random_init_arrays(self, seed_base=1000, std=0.02):
        """The random init of BASELINE's GPT-2 configs: every matrix and
        embedding N(0, std) from seed seed_base + its index in parameters()
        order, biases 0, LayerNorm weights 1.  Returns the host arrays."""
        out = []
        for i, (name, shp) in enumerate(self.param_layout()):
            if name.endswith(("ln1.W", "ln2.W")) or name == "ln_f.W":
                out.append(np.ones(shp, np.float32))
            elif len(shp) == 1:
                out.append(np.zeros(shp, np.float32))
            else:
                out.append(self.rt.normal(shp, seed_base + i, 0.0, std))
        return out

    def fast_load(self, arrays):
        """fast_load_state_dict from numpy arrays in parameters() order."""
        ts = [self.rt.from_numpy(a, CPU) for a in arrays]
        arr = (TensorP * len(ts))(*ts)
        _fn(self.s.fast_load_state_dict, None, _vp, TensorPP)(self.raw, arr)
        for t in ts:
            self.rt.free(t)


class CrossEntropy:
    def __init__(self, rt):
        self.rt = rt
        self.raw = ctypes.c_void_p(rt.lib.CrossEntropyLoss())
        self.s = ctypes.cast(self.raw, ctypes.POINTER(CrossEntropyLossT)).contents

    def forward(self, logits, targets):
        return _fn(self.s.forward, TensorP, _vp, TensorP, TensorP)(self.raw, logits, targets)

    def backward(self, g):
        return _fn(self.s.backward, TensorP, _vp, TensorP)(self.raw, g)

    def free(self):
        _fn(self.s.free_layer, None, _vp)(self.raw)


class AdamWOptimizer:
    """AdamW(model.parameters(), model.gradients(), n, ...); the lists are
    handed to (and freed by) the optimizer, as gpt.c's train_gpt.c does."""

    def __init__(self, rt, model, lr=3e-4, beta1=0.9, beta2=0.99, eps=1e-8, weight_decay=0.0):
        self.rt = rt
        p = _fn(model.s.parameters, TensorPP, _vp)(model.raw)
        g = _fn(model.s.gradients, TensorPP, _vp)(model.raw)
        self.raw = ctypes.c_void_p(rt.lib.AdamW(p, g, model.n_params(), lr, beta1, beta2, eps, weight_decay))
        self.s = ctypes.cast(self.raw, ctypes.POINTER(AdamWT)).contents

    def step(self):
        _fn(self.s.step, None, _vp)(self.raw)

    def zero_grad(self):
        _fn(self.s.zero_grad, None, _vp)(self.raw)

    def free(self):
        _fn(self.s.free_layer, None, _vp)(self.raw)


class KVCache:
    """gptc_kv_cache_create(model, B, L) and the one-token step gptc_gpt2_decode."""

    def __init__(self, rt, model, B, L):
        self.rt = rt
        self.raw = ctypes.c_void_p(rt.lib.gptc_kv_cache_create(model.raw, B, L))
        self.model = model

    def decode(self, ids, pos):
        """ids: device tensor (B, 1); returns the logits tensor (B, 1, V)."""
        return self.rt.lib.gptc_gpt2_decode(self.model.raw, self.raw, ids, pos)

    def free(self):
        if self.raw:
            self.rt.lib.gptc_kv_cache_free(self.raw)
            self.raw = None
