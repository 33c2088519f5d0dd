"""attention_decode_noalloc_cuda_kernel against attention_decode_cuda_kernel.

The allocation-free entry point runs the same decode kernels; steps past
512 keys (the split-key pair) keep their partials in a fixed device array
instead of a stream-ordered allocation, so its output and the cache rows it
writes must equal the allocating entry point's bit for bit.  Two such calls
in a row share that array: the second, with fewer sequences and keys, must
not see the first's partials.  A step of at most 512 keys (one launch, no
partials) follows them.  A step needing more partials than the array holds
is refused on the host before any launch.
"""
import os
import subprocess
import sys
import textwrap

import numpy as np
import pytest

import gptc

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def decode_both(rt, B, H, D, L, pos, seed):
    """One decode step at `pos` through both entry points, from identical
    caches (rows 0 .. pos-1 filled, the rest N(0,1) noise the step must not
    read).  Returns (allocating, allocation-free) outputs and caches."""
    C = H * D
    lib = rt.lib
    row = rt.normal((B, 1, 3 * C), seed)
    kc0 = rt.normal((B, H, L, D), seed + 1)
    vc0 = rt.normal((B, H, L, D), seed + 2)
    outs = []
    for fn in (lib.attention_decode_cuda_kernel, lib.attention_decode_noalloc_cuda_kernel):
        q, kc, vc, y = rt.from_numpy(row), rt.from_numpy(kc0), rt.from_numpy(vc0), rt.empty((B, 1, C))
        print(f"  {fn.__name__}: B={B} H={H} D={D} L={L} pos={pos}", flush=True)
        fn(q, kc, vc, pos, H, y)
        rt.sync()
        outs.append((rt.to_numpy(y), rt.to_numpy(kc), rt.to_numpy(vc)))
        for t in (q, kc, vc, y):
            rt.free(t)
    return outs


def reference_row(row, kc, vc, pos, H, D):
    """float64 softmax(q k^T / sqrt(D)) v over keys 0 .. pos (the new k, v at pos)."""
    B = row.shape[0]
    C = H * D
    out = np.empty((B, 1, C))
    for b in range(B):
        for h in range(H):
            q = row[b, 0, h * D:(h + 1) * D].astype(np.float64)
            k = kc[b, h, :pos + 1].astype(np.float64)
            v = vc[b, h, :pos + 1].astype(np.float64)
            s = k @ q / np.sqrt(D)
            p = np.exp(s - s.max())
            out[b, 0, h * D:(h + 1) * D] = p @ v / p.sum()
    return out


def test_noalloc_matches_allocating_entry_point_twice(rt):
    # Second call smaller; both use the scratch array.  The third needs none.
    cases = [(4, 12, 64, 1024, 900, 11), (1, 12, 64, 1024, 600, 23), (1, 12, 64, 512, 100, 29)]
    for B, H, D, L, pos, seed in cases:
        (y_a, k_a, v_a), (y_n, k_n, v_n) = decode_both(rt, B, H, D, L, pos, seed)
        assert np.array_equal(y_a, y_n), f"outputs differ at B={B} pos={pos}: {np.abs(y_a - y_n).max():.3e}"
        assert np.array_equal(k_a, k_n) and np.array_equal(v_a, v_n), "cache rows differ"
        row = rt.normal((B, 1, 3 * H * D), seed)
        ref = reference_row(row, k_n, v_n, pos, H, D)
        err = float(np.abs(y_n - ref).max())
        print(f"  B={B} pos={pos}: max abs err vs float64 {err:.2e}")
        assert err <= 1e-4


def test_noalloc_other_head_size(rt):
    """D != 64 takes the one-workgroup kernel, which needs no partials."""
    (y_a, _, _), (y_n, _, _) = decode_both(rt, 2, 4, 48, 64, 40, 5)
    assert np.array_equal(y_a, y_n)


def test_noalloc_rejects_steps_beyond_its_scratch(rt):
    cap = rt.lib.gptc_decode_noalloc_scratch_floats()
    B, H, D = 8, 32, 64
    pos = 8191  # B*H*128 chunks*68 floats > cap
    assert B * H * ((pos + 64) // 64) * 68 > cap
    code = textwrap.dedent(f"""
        import sys
        sys.path.insert(0, {os.path.join(ROOT, 'gpt.c_amd')!r})
        import gptc
        lib = gptc.load()
        rt = gptc.Runtime(lib)
        rt.init()
        q, kc, vc, y = rt.empty(({B}, 1, {3 * H * D})), rt.empty(({B}, {H}, 8192, {D})), \\
            rt.empty(({B}, {H}, 8192, {D})), rt.empty(({B}, 1, {H * D}))
        lib.attention_decode_noalloc_cuda_kernel(q, kc, vc, {pos}, {H}, y)
        print("returned")
    """)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and "fixed" in r.stderr and "returned" not in r.stdout, r.stderr
