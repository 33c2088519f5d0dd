"""gpt.c's on-disk formats read and written by the library (row f4), on the CPU.

gpt.c ships no sample files, so each format is pinned by an independent
numpy writer/reader that restates the reference's Python tooling:
  * checkpoint   model.py:246-283 (write_model / write_tensors) and
                 train_gpt.c:197-348 (load_model / save_model);
  * tokens       data/common.py:35-48 (raw int32 ids) read by
                 src/dataloader.c:14-101;
  * tokenizer    tokenizer.py:12-40 (header, then length byte + bytes) read by
                 src/tokenizer.c:16-114.
(the writers are in file_formats.py).  A file written by numpy loads into the
same parameters / batches / strings; a file the library writes is
byte-identical to numpy's.  The GPU case (saving
a model whose parameters live on the device) is in test_gpt2_gpu.py's style
at the end, marked gpu.
"""
import ctypes
import os
import subprocess
import sys
import textwrap

import numpy as np
import pytest

import gptc
from file_formats import write_checkpoint, write_tokenizer
from gpt2_oracle import param_shapes

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


class DataLoaderT(ctypes.Structure):
    """dataloader_t (include/dataloader.h)."""
    _fields_ = [("batch_size", ctypes.c_int), ("block_size", ctypes.c_int), ("fp", ctypes.c_void_p),
                ("batch", ctypes.c_void_p), ("_file_size", ctypes.c_size_t), ("_curr_fp_ptr", ctypes.c_size_t),
                ("next", ctypes.c_void_p), ("len", ctypes.c_void_p), ("reset", ctypes.c_void_p),
                ("free_layer", ctypes.c_void_p)]


class TokenizerT(ctypes.Structure):
    """tokenizer_t (include/tokenizer.h)."""
    _fields_ = [("vocab_size", ctypes.c_uint32), ("eot_token", ctypes.c_int), ("token_map", ctypes.c_void_p),
                ("free_layer", ctypes.c_void_p), ("decode", ctypes.c_void_p), ("decode_tokens", ctypes.c_void_p),
                ("decode_length", ctypes.c_void_p)]


@pytest.fixture(scope="module")
def rt():
    return gptc.Runtime(gptc.load())


def test_checkpoint_numpy_file_loads_and_saves_identically(rt, tmp_path):
    cfg = (16, 37, 2, 2, 8)  # block, V, layers, heads, C
    block, V, L, H, C = cfg
    rng = np.random.default_rng(0)
    params = [rng.standard_normal(shp).astype(np.float32) for _, shp in param_shapes(V, block, L, C)]
    src = tmp_path / "model.bin"
    write_checkpoint(src, cfg, params, step=123)
    model, steps = gptc.GPT2Model.from_checkpoint(rt, src)
    assert steps == 123
    s = model.s
    assert (s.block_size, s.vocab_size, s.n_layers, s.n_heads, s.n_embd) == cfg
    assert s._num_param_tensors == len(params)
    for t, p in zip(model.parameters(), params):
        assert np.array_equal(rt.to_numpy(t), p)
    out = tmp_path / "again.bin"
    model.save(out, steps=123)
    assert open(out, "rb").read() == open(src, "rb").read()
    model.free()


def test_checkpoint_errors_are_fatal(tmp_path):
    bad = tmp_path / "bad.bin"
    np.zeros(300, np.int32).tofile(bad)
    code = textwrap.dedent(f"""
        import sys; sys.path.insert(0, {os.path.join(ROOT, 'gpt.c_amd')!r})
        import gptc
        rt = gptc.Runtime(gptc.load())
        gptc.GPT2Model.from_checkpoint(rt, {str(bad)!r})
    """)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and "Bad magic model file" in r.stderr


def test_dataloader_windows_targets_and_wraparound(rt, tmp_path):
    B, T = 3, 5
    toks = np.arange(1000, 1000 + 40, dtype=np.int32)  # 40 ids: windows of 16 advance by 15
    path = tmp_path / "toks.bin"
    toks.tofile(path)
    raw = rt.lib.DataLoader(os.fsencode(path), B, T)
    dl = ctypes.cast(raw, ctypes.POINTER(DataLoaderT)).contents
    nxt = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.POINTER(gptc.TensorP))(dl.next)
    length = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p)(dl.len)(raw)
    assert length == 40 // (B * T + 1)
    batch = (gptc.TensorP * 2)()
    starts = []
    for _ in range(4):
        nxt(raw, batch)
        x, y = rt.to_numpy(batch[0]), rt.to_numpy(batch[1])
        assert x.shape == (B, T) and y.shape == (B, T)
        start = int(x.ravel()[0]) - 1000
        starts.append(start)
        assert np.array_equal(x.ravel(), toks[start:start + B * T].astype(np.float32))
        assert np.array_equal(y.ravel(), toks[start + 1:start + B * T + 1].astype(np.float32))
        rt.free(batch[0])
        rt.free(batch[1])
    # 0, 15, then 30 would need ids 30..45 (past 40): back to 0
    assert starts == [0, 15, 0, 15]
    ctypes.CFUNCTYPE(None, ctypes.c_void_p)(dl.free_layer)(raw)


def test_tokenizer_decodes(rt, tmp_path):
    pieces = [b"Hello", b",", b" world", b"\xe2\x82\xac", b"!", b"<|endoftext|>", bytes(range(1, 256))[:255]]
    path = tmp_path / "tokenizer.bin"
    write_tokenizer(path, pieces, eot=5)
    raw = rt.lib.Tokenizer(os.fsencode(path))
    tk = ctypes.cast(raw, ctypes.POINTER(TokenizerT)).contents
    assert tk.vocab_size == len(pieces) and tk.eot_token == 5
    decode = ctypes.CFUNCTYPE(ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32)(tk.decode)
    for i, b in enumerate(pieces):
        assert ctypes.string_at(decode(raw, i)) == b
    ids = (ctypes.c_uint32 * 5)(0, 1, 2, 4, 3)
    dl = ctypes.CFUNCTYPE(ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t)(tk.decode_length)
    assert dl(raw, ids, 5) == len(b"Hello, world!\xe2\x82\xac")
    buf = ctypes.create_string_buffer(64)
    dt = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t)(
        tk.decode_tokens)
    dt(raw, ids, 5, buf, 64)
    assert buf.value == b"Hello, world!\xe2\x82\xac"
    dt(raw, ids, 5, buf, 6)  # truncated to dest_n - 1 bytes
    assert buf.value == b"Hello"
    ctypes.CFUNCTYPE(None, ctypes.c_void_p)(tk.free_layer)(raw)


def test_dataloader_reset_and_ragged_file(rt, tmp_path):
    """A file whose size is not a whole number of ids (a trailing partial id)
    and reset(): windows restart at id 0, len() counts whole windows."""
    B, T = 2, 3
    toks = np.arange(7, 7 + 20, dtype=np.int32)
    path = tmp_path / "ragged.bin"
    path.write_bytes(toks.tobytes() + b"\x01\x02")  # 82 bytes
    raw = rt.lib.DataLoader(os.fsencode(path), B, T)
    dl = ctypes.cast(raw, ctypes.POINTER(DataLoaderT)).contents
    nxt = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.POINTER(gptc.TensorP))(dl.next)
    assert ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p)(dl.len)(raw) == 82 // (4 * (B * T + 1))
    batch = (gptc.TensorP * 2)()
    starts = []
    for i in range(5):
        if i == 3:
            ctypes.CFUNCTYPE(None, ctypes.c_void_p)(dl.reset)(raw)
        nxt(raw, batch)
        x, y = rt.to_numpy(batch[0]).ravel(), rt.to_numpy(batch[1]).ravel()
        s0 = int(x[0]) - 7
        assert np.array_equal(x, toks[s0:s0 + B * T].astype(np.float32))
        assert np.array_equal(y, toks[s0 + 1:s0 + B * T + 1].astype(np.float32))
        starts.append(s0)
        rt.free(batch[0])
        rt.free(batch[1])
    # 20 whole ids: windows of 7 at 0, 6, 12 (needs ids 12..18), then 18 would
    # need 18..24: wrap to 0; reset before the 4th call restarts at 0 too.
    assert starts == [0, 6, 12, 0, 6]
    ctypes.CFUNCTYPE(None, ctypes.c_void_p)(dl.free_layer)(raw)


@pytest.mark.parametrize("case", ["too_small", "bad_magic", "truncated_piece", "empty_piece"])
def test_format_errors_are_fatal(tmp_path, case):
    """Malformed inputs end the process with the library's error, never a
    read past the data."""
    path = tmp_path / "f.bin"
    if case == "too_small":
        np.arange(6, dtype=np.int32).tofile(path)  # one window needs 2*3+1 = 7 ids
        call = f"lib.DataLoader({os.fsencode(path)!r}, 2, 3)"
    else:
        header = np.zeros(256, np.int32)
        header[:3] = [20240415 if case != "bad_magic" else 1234, 2, 1]
        body = {"bad_magic": b"\x01a\x01b", "truncated_piece": b"\x01a\x05bc", "empty_piece": b"\x01a\x00"}[case]
        path.write_bytes(header.tobytes() + body)
        call = f"lib.Tokenizer({os.fsencode(path)!r})"
    code = textwrap.dedent(f"""
        import sys
        sys.path.insert(0, {os.path.join(ROOT, 'gpt.c_amd')!r})
        import gptc
        lib = gptc.load()
        {call}
    """)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and "[ERROR]" in r.stderr, r.stderr
    expect = {"too_small": "fewer than one window", "bad_magic": "not a tokenizer.bin",
              "truncated_piece": "ends inside", "empty_piece": "empty byte string"}[case]
    assert expect in r.stderr, r.stderr


@pytest.mark.gpu
def test_checkpoint_saved_from_gpu_round_trips(tmp_path):
    lib = gptc.load()
    r = gptc.Runtime(lib)
    r.init()
    block, V, L, H, C = 32, 53, 2, 2, 16
    rng = np.random.default_rng(1)
    params = [rng.standard_normal(shp).astype(np.float32) for _, shp in param_shapes(V, block, L, C)]
    model = gptc.GPT2Model(r, block, V, L, H, C)
    model.fast_load(params)
    model.to(gptc.CUDA)
    path = tmp_path / "gpu.bin"
    model.save(path, steps=7)
    model.free()
    ref = tmp_path / "ref.bin"
    write_checkpoint(ref, (block, V, L, H, C), params, step=7)
    assert open(path, "rb").read() == open(ref, "rb").read()
