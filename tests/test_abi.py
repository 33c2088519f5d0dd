"""The C-ABI library without a GPU: it loads, exports every function that
include/*.h declares, keeps tensor_t / attention_t binary-compatible with
gpt.c, and its host-side logic (constructor, CPU tensor ops, fatal error
convention) behaves like gpt.c's.  No call here reaches the device.
"""
import ctypes
import os
import re
import subprocess
import sys
import textwrap

import numpy as np
import pytest

import gptc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")


def declared_functions():
    names = set()
    for fn in sorted(os.listdir(INCLUDE)):
        if not fn.endswith(".h"):
            continue
        src = open(os.path.join(INCLUDE, fn)).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        src = re.sub(r"//[^\n]*", "", src)
        src = re.sub(r"#[^\n]*", "", src)
        src = re.sub(r"typedef\s+(struct|enum)[^;]*?\{.*?\}[^;]*;", "", src, flags=re.S)
        for m in re.finditer(r"([A-Za-z_][A-Za-z0-9_]*)\s*\([^;{]*\)\s*;", src):
            names.add(m.group(1))
    return names - {"if", "while", "for", "return", "sizeof"}


def test_every_declared_function_is_exported(lib):
    names = declared_functions()
    assert len(names) > 50
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    # The Python front end declares a signature for each of them.
    assert names <= set(gptc.SIGNATURES), sorted(names - set(gptc.SIGNATURES))


def test_struct_layouts_match_gpt_c():
    # tensor_t: float*, ndims, length, shape[8], to, device; aligned(64) -> 64 bytes.
    assert ctypes.sizeof(gptc.Tensor) == 64
    assert gptc.Tensor.device.offset == 56 and gptc.Tensor.shape.offset == 16
    # attention_t: buffer, cache[4], 7 function pointers, n_embd, n_heads; aligned(64) -> 128.
    assert gptc.AttentionT.n_heads.offset == 100
    assert (ctypes.sizeof(gptc.AttentionT) + 63) // 64 * 64 == 128


def test_constructor_builds_causal_mask_on_host(lib):
    rt = gptc.Runtime(lib)
    layer = gptc.AttentionLayer(rt, 64, 4, 9)
    buf = layer.buffer.contents
    assert buf.device == gptc.CPU and buf.ndims == 2 and (buf.shape[0], buf.shape[1]) == (9, 9)
    mask = rt.to_numpy(layer.buffer)
    assert np.array_equal(mask, np.tril(np.ones((9, 9), np.float32)))
    assert layer.num_parameters() == 0
    assert layer.ptr.contents.n_embd == 64 and layer.ptr.contents.n_heads == 4
    assert all(not layer.cache(i) for i in range(4))
    layer.free()


def test_cpu_tensor_ops(lib):
    rt = gptc.Runtime(lib)
    a = np.arange(24, dtype=np.float32).reshape(2, 3, 4)
    t = rt.from_numpy(a, gptc.CPU)
    assert np.array_equal(rt.to_numpy(t), a)
    shp = (ctypes.c_int * 2)(6, 4)
    lib.view(t, shp, 2)
    assert rt.to_numpy(t).shape == (6, 4)
    buf = ctypes.create_string_buffer(64)
    lib.shape(t, buf)
    assert buf.value == b"6, 4"
    z = lib.zeros((ctypes.c_int * 1)(5), 1, gptc.CPU)
    o = lib.ones((ctypes.c_int * 1)(5), 1, gptc.CPU)
    f = lib.fill((ctypes.c_int * 1)(5), 1, ctypes.c_float(2.5), gptc.CPU)
    r = lib.arange(3, 11, 2, gptc.CPU)
    assert np.array_equal(rt.to_numpy(z), np.zeros(5))
    assert np.array_equal(rt.to_numpy(o), np.ones(5))
    assert np.array_equal(rt.to_numpy(f), np.full(5, 2.5))
    assert np.array_equal(rt.to_numpy(r), [[3, 5, 7, 9]])
    c = lib.create_tensor((ctypes.c_int * 2)(6, 4), 2, gptc.CPU)
    lib.tensor_copy(c, t)
    assert np.array_equal(rt.to_numpy(c), a.reshape(6, 4))
    for x in (t, z, o, f, r, c):
        lib.free_tensor(x)


def run_c_snippet(body):
    """Run a few library calls in a child process (errors are fatal exits)."""
    code = textwrap.dedent(f"""
        import ctypes, sys
        sys.path.insert(0, {os.path.join(ROOT, 'gpt.c_amd')!r})
        import gptc
        lib = gptc.load()
        rt = gptc.Runtime(lib)
    """) + textwrap.dedent(body)
    return subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)


def test_fatal_error_bad_head_split():
    r = run_c_snippet("lib.Attention(10, 4, 8)\nprint('survived')")
    assert r.returncode == 1 and "survived" not in r.stdout
    assert "divisible by n_heads" in r.stderr and "[ERROR]" in r.stderr


def test_fatal_error_cpu_attention_is_not_served():
    r = run_c_snippet("""
        import numpy as np
        layer = gptc.AttentionLayer(rt, 8, 2, 4)
        x = rt.from_numpy(np.zeros((1, 4, 24), np.float32), gptc.CPU)
        layer.forward(x)
        print('survived')
    """)
    assert r.returncode == 1 and "survived" not in r.stdout
    assert "GPU attention path only" in r.stderr


def test_fatal_error_gpu_call_before_runtime_init():
    r = run_c_snippet("lib.alloc_cuda(16)\nprint('survived')")
    assert r.returncode == 1 and "survived" not in r.stdout
    assert "runtime_init" in r.stderr


def test_fatal_error_decode_position_past_cache():
    r = run_c_snippet("""
        import numpy as np
        row = rt.from_numpy(np.zeros((1, 1, 24), np.float32), gptc.CPU)
        kc = rt.from_numpy(np.zeros((1, 2, 4, 4), np.float32), gptc.CPU)
        vc = rt.from_numpy(np.zeros((1, 2, 4, 4), np.float32), gptc.CPU)
        out = rt.from_numpy(np.zeros((1, 1, 8), np.float32), gptc.CPU)
        lib.attention_decode_cuda_kernel(row, kc, vc, 4, 2, out)
        print('survived')
    """)
    assert r.returncode == 1 and "survived" not in r.stdout
    assert "0 <= pos < L = 4" in r.stderr


def block_schedule(lib, BH, nqt, per_cu=3, cus=32):
    cap = BH * nqt + 8 * cus * per_cu * 4 + 16
    ws, it = (ctypes.c_int * cap)(), (ctypes.c_int * cap)()
    load, pairs = ctypes.c_double(), ctypes.c_int()
    n = lib.gptc_attention_block_schedule(BH, nqt, per_cu, cus, ws, it, cap, ctypes.byref(load), ctypes.byref(pairs))
    assert n > 0
    starts = list(ws[:n + 1])
    items = list(it[:starts[-1]])
    return n, starts, items, load.value, bool(pairs.value)


@pytest.mark.parametrize("B,H,T", [(8, 12, 1024), (4, 25, 1024), (8, 12, 128), (8, 12, 256), (1, 12, 1024),
                                   (8, 12, 960), (2, 3, 17), (1, 1, 1), (3, 7, 2000), (16, 25, 1024)])
def test_block_schedule_covers_every_block_once(lib, B, H, T):
    """The forward and dq kernels write the rows of exactly the blocks their
    work lists name: every (head, 64-query block) must appear exactly once,
    or rows of y / dq would be left unwritten or written twice."""
    BH, nqt = B * H, (T + 63) // 64
    n, starts, items, load, pairs = block_schedule(lib, BH, nqt)
    assert n % 8 == 0 and starts[0] == 0 and all(a <= b for a, b in zip(starts, starts[1:]))
    seen = sorted((i >> 12, i & 4095) for i in items)
    assert seen == [(bh, j) for bh in range(BH) for j in range(nqt)]
    # The largest per-CU load is at least the even share and, for the paired
    # shape of C2, exactly one CU's three pairs.
    per_cu_share = BH * sum(j + 1.5 for j in range(nqt)) / (8 * 32)
    assert load >= per_cu_share - 1e-9
    if (B, H, T) == (8, 12, 1024):
        assert pairs and abs(load - 3 * (nqt + 1 + 1.0)) < 1e-9


@pytest.mark.parametrize("B,H,T", [(8, 12, 1024), (4, 25, 1024), (16, 25, 1024), (1, 12, 1024), (8, 12, 320),
                                   (8, 12, 256), (2, 3, 17), (3, 7, 2000)])
def test_pooled_block_schedule_covers_every_block_once(lib, B, H, T):
    """With the pool, the lists and the pool together name every (head,
    64-query block) exactly once, and every list keeps a block (a workgroup
    with none would count itself done without running the pool protocol's
    first steps); where that cannot hold there is no pool."""
    BH, nqt = B * H, (T + 63) // 64
    cap = BH * nqt + 8 * 32 * 3 * 4 + 16
    ws, it, j0 = (ctypes.c_int * cap)(), (ctypes.c_int * cap)(), ctypes.c_int()
    n = lib.gptc_attention_block_schedule_pool(BH, nqt, 3, 32, ws, it, cap, ctypes.byref(j0))
    assert n > 0
    starts = list(ws[:n + 1])
    items = list(it[:starts[-1]])
    pool = [(r % BH, j0.value - 1 - r // BH) for r in range(j0.value * BH)]
    seen = sorted([(i >> 12, i & 4095) for i in items] + pool)
    assert seen == [(bh, j) for bh in range(BH) for j in range(nqt)]
    if j0.value > 0:
        assert all(b > a for a, b in zip(starts, starts[1:]))
        assert all((i & 4095) >= j0.value for i in items)
    if (B, H, T) == (8, 12, 1024):
        assert j0.value == 3  # C2 runs with the pool: blocks 0, 1 and 2 of every head
    if (B, H, T) == (2, 3, 17):
        assert j0.value == 0  # one block per head: too few for a pool


def test_block_schedule_uses_every_slot_on_ties(lib):
    """C2's 768 pairs fill three workgroups per CU exactly; for a kernel that
    keeps four per CU (dq16) the pairs would leave a quarter of the slots
    empty, so the longest-first lists over all 1024 slots win while their
    largest per-CU load is within 2 % of the pairs', and they still name
    every block once."""
    BH, nqt = 8 * 12, 16
    n3, _, _, load3, pairs3 = block_schedule(lib, BH, nqt, per_cu=3)
    n4, starts, items, load4, pairs4 = block_schedule(lib, BH, nqt, per_cu=4)
    assert pairs3 and n3 == 768
    assert not pairs4 and n4 == 1024 and all(b > a for a, b in zip(starts, starts[1:]))
    assert load3 - 1e-9 <= load4 <= 1.02 * load3
    assert sorted((i >> 12, i & 4095) for i in items) == [(bh, j) for bh in range(BH) for j in range(nqt)]


def test_block_schedule_balances_c5(lib):
    """C5 (100 heads x 16 blocks) has 800 pairs for 768 resident slots: the
    longest-first lists must keep every CU within 5 % of the even share."""
    BH, nqt = 4 * 25, 16
    n, starts, items, load, pairs = block_schedule(lib, BH, nqt)
    share = BH * sum(j + 1.5 for j in range(nqt)) / (8 * 32)
    assert not pairs and n <= 8 * 32 * 3
    assert load <= 1.05 * share, (load, share)


def key_schedule(lib, BH, nqt, per_cu=2, cus=32):
    nkb = (nqt + 1) // 2
    cap = 4 * (2 * BH * nkb) + 8 * cus * per_cu * 2 + 16
    ws, it = (ctypes.c_int * cap)(), (ctypes.c_int * cap)()
    est, nsplit = ctypes.c_double(), ctypes.c_int()
    n = lib.gptc_attention_key_schedule(BH, nqt, per_cu, cus, ws, it, cap, ctypes.byref(est), ctypes.byref(nsplit))
    assert n > 0
    starts = list(ws[:n + 1])
    items = [tuple(it[4 * i:4 * i + 4]) for i in range(starts[-1])]
    return n, starts, items, est.value, nsplit.value


@pytest.mark.parametrize("B,H,T", [(8, 12, 1024), (4, 25, 1024), (8, 12, 256), (1, 12, 1024), (8, 12, 960),
                                   (3, 7, 2000), (16, 25, 1024), (32, 12, 1024), (1, 1, 200), (2, 12, 4096)])
def test_key_schedule_covers_every_tile_once(lib, B, H, T):
    """The dk/dv kernel writes dK, dV rows of exactly the items its work lists
    name: the items of every (head, 128-key block kb) must cover query tiles
    2kb .. nqt-1 once, as one item, or as two for kb < nsplit (whose adds land
    on rows the delta kernel zeroed: two addends give the same sum in either
    order, three would not)."""
    BH, nqt = B * H, (T + 63) // 64
    nkb = (nqt + 1) // 2
    n, starts, items, est, nsplit = key_schedule(lib, BH, nqt)
    assert n % 8 == 0 and starts[0] == 0 and all(a <= b for a, b in zip(starts, starts[1:]))
    assert 0 <= nsplit <= nkb
    by_block = {}
    for bh, kb, qa, qe in items:
        assert 0 <= bh < BH and 0 <= kb < nkb and 2 * kb <= qa < qe <= nqt
        by_block.setdefault((bh, kb), []).append((qa, qe))
    assert sorted(by_block) == [(bh, kb) for bh in range(BH) for kb in range(nkb)]
    for (bh, kb), parts in by_block.items():
        parts.sort()
        assert parts[0][0] == 2 * kb and parts[-1][1] == nqt
        assert all(a[1] == b[0] for a, b in zip(parts, parts[1:]))
        assert len(parts) <= (2 if kb < nsplit else 1), ((bh, kb), parts, nsplit)


def test_key_schedule_c2_balance(lib):
    """At C2 (96 heads x 8 key blocks over 512 slots) the lists need no split
    and keep every CU within 5 % of the even share of the work."""
    BH, nqt = 96, 16
    n, starts, items, est, nsplit = key_schedule(lib, BH, nqt)
    cost = lambda kb, qa, qe: (qe - qa) - (0.75 if qa == 2 * kb else 0.0) + 0.3
    share = BH * sum(cost(kb, 2 * kb, nqt) for kb in range(nqt // 2)) / (8 * 32)
    assert nsplit == 0 and n == 512
    loads = {}
    for w in range(n):
        cu = (w % 8, (w // 8) % 32)
        loads[cu] = loads.get(cu, 0.0) + sum(cost(kb, qa, qe) for (bh, kb, qa, qe) in items[starts[w]:starts[w + 1]])
    assert max(loads.values()) <= 1.05 * share, (max(loads.values()), share)


# Random shapes and occupancies: the list builders must name every block
# exactly once whichever construction wins (pairs, longest-first lists over
# the slots, the pool, split key blocks), or output rows would be dropped or
# written twice.
from hypothesis import given, settings, strategies as st


@settings(max_examples=200, deadline=None)
@given(BH=st.integers(1, 400), T=st.integers(1, 3000), per_cu=st.integers(1, 4), cus=st.sampled_from([1, 4, 32]))
def test_block_schedule_property(lib, BH, T, per_cu, cus):
    nqt = (T + 63) // 64
    n, starts, items, load, pairs = block_schedule(lib, BH, nqt, per_cu=per_cu, cus=cus)
    assert n % 8 == 0 and starts[0] == 0 and all(a <= b for a, b in zip(starts, starts[1:]))
    assert sorted((i >> 12, i & 4095) for i in items) == [(bh, j) for bh in range(BH) for j in range(nqt)]
    cap = BH * nqt + 8 * cus * per_cu * 4 + 16
    ws, it, j0 = (ctypes.c_int * cap)(), (ctypes.c_int * cap)(), ctypes.c_int()
    m = lib.gptc_attention_block_schedule_pool(BH, nqt, per_cu, cus, ws, it, cap, ctypes.byref(j0))
    assert m > 0
    pstarts = list(ws[:m + 1])
    pool = [(r % BH, j0.value - 1 - r // BH) for r in range(j0.value * BH)]
    seen = sorted([(i >> 12, i & 4095) for i in it[:pstarts[-1]]] + pool)
    assert seen == [(bh, j) for bh in range(BH) for j in range(nqt)]
    if j0.value > 0:
        assert all(b > a for a, b in zip(pstarts, pstarts[1:]))


@settings(max_examples=200, deadline=None)
@given(BH=st.integers(1, 300), T=st.integers(1, 3000), per_cu=st.integers(1, 3), cus=st.sampled_from([1, 4, 32]))
def test_key_schedule_property(lib, BH, T, per_cu, cus):
    nqt = (T + 63) // 64
    nkb = (nqt + 1) // 2
    n, starts, items, est, nsplit = key_schedule(lib, BH, nqt, per_cu=per_cu, cus=cus)
    assert n % 8 == 0 and starts[0] == 0 and all(a <= b for a, b in zip(starts, starts[1:]))
    assert 0 <= nsplit <= nkb
    by_block = {}
    for bh, kb, qa, qe in items:
        assert 0 <= bh < BH and 0 <= kb < nkb and 2 * kb <= qa < qe <= nqt
        by_block.setdefault((bh, kb), []).append((qa, qe))
    assert sorted(by_block) == [(bh, kb) for bh in range(BH) for kb in range(nkb)]
    for (bh, kb), parts in by_block.items():
        parts.sort()
        assert parts[0][0] == 2 * kb and parts[-1][1] == nqt
        assert all(a[1] == b[0] for a, b in zip(parts, parts[1:]))
        assert len(parts) <= (2 if kb < nsplit else 1)
