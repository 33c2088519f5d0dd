#!/usr/bin/env python3
"""Benchmark of the fused causal attention path (fwd + bwd) on one MI355X.

Metric: causal attention fwd+bwd TFLOP/s and % of the fp32
MFMA peak at B=8 T=1024 H=12 D=64 (config C2).  One "step" = one forward
(attention_forward_cuda_kernel) + one backward
(attention_backward_cuda_kernel) over the same synthetic batch, through the
library's C-ABI, inputs and outputs resident in HBM, nothing allocated in
the timed region.

FLOPs are algorithmic: the two forward and four backward contractions over
the causal triangle only, D*T*(T+1)*B*H flop each (T(T+1)/2 query-key pairs
x D multiply-adds x 2), no recompute, no softmax.  fwd = 2 units, bwd = 4.

Prints ONE JSON line on stdout; progress goes to stderr.
"""
import argparse
import ctypes
import json
import os
import re
import statistics
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "gpt.c_amd"))

import numpy as np  # noqa: E402

import gptc  # noqa: E402

CONFIGS = {
    "c2": dict(B=8, T=1024, C=768, H=12, workload="causal self-attention fwd+bwd, GPT-2 124M shape (C2)"),
    "c5": dict(B=4, T=1024, C=1600, H=25, workload="causal self-attention fwd+bwd, GPT-2 XL shape (C5)"),
    "c1": dict(B=8, T=128, C=768, H=12, forward_only=True,
               workload="causal self-attention forward only (C1), HBM-side of the ridge"),
}
SEED_X, SEED_DY = 1337, 1338
SPEC_CU, SPEC_MHZ = 256, 2400            # MI355X public spec
FLOP_PER_CLK_CU_FP32_MFMA = 256          # v_mfma_f32_32x32x2_f32: 4096 flop / 16 passes of 4 clk, 4 SIMDs
HBM_PEAK_GBS = 8000.0
BOX_CPU_SHARE = 16                       # CPUs a one-GPU box allots to a job


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def device_peak():
    """fp32 MFMA peak from rocminfo's CU count and max clock (spec fallback)."""
    cu, mhz, src = SPEC_CU, SPEC_MHZ, "spec"
    try:
        out = subprocess.run(["rocminfo"], capture_output=True, text=True, timeout=60).stdout
        for block in out.split("Agent ")[1:]:
            if "gfx950" not in block:
                continue
            m_cu = re.search(r"Compute Unit:\s+(\d+)", block)
            m_mhz = re.search(r"Max Clock Freq\. \(MHz\):\s+(\d+)", block)
            if m_cu and m_mhz:
                cu, mhz, src = int(m_cu.group(1)), int(m_mhz.group(1)), "rocminfo"
            break
    except (OSError, subprocess.SubprocessError):
        pass
    return cu * mhz * 1e6 * FLOP_PER_CLK_CU_FP32_MFMA / 1e12, cu, mhz, src


class Hip:
    """The few HIP runtime calls the timer needs (ctypes on libamdhip64)."""

    def __init__(self):
        self.h = ctypes.CDLL("libamdhip64.so")
        self.h.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.h.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.h.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.h.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def check(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed with hipError {rc}")

    def event(self):
        e = ctypes.c_void_p()
        self.check(self.h.hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        return e.value

    def record(self, ev, stream):
        self.check(self.h.hipEventRecord(ev, stream), "hipEventRecord")

    def elapsed_ms(self, a, b):
        self.check(self.h.hipEventSynchronize(b), "hipEventSynchronize")
        ms = ctypes.c_float()
        self.check(self.h.hipEventElapsedTime(ctypes.byref(ms), a, b), "hipEventElapsedTime")
        return ms.value

    def device_sync(self):
        self.check(self.h.hipDeviceSynchronize(), "hipDeviceSynchronize")


def host_cpu():
    """The host CPU as the CPU baselines use it: lscpu's model, threads per
    core, cores per socket and sockets, the logical CPUs this process may run
    on (its affinity set) and the physical cores behind them (distinct
    (package, core) pairs in sysfs).  OpenBLAS runs one thread per physical
    core of that set, capped at BOX_CPU_SHARE, the CPUs a one-GPU box
    allots to a job whatever the machine has."""
    info = {"nproc": os.cpu_count()}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=30).stdout
        for key, name in (("Model name", "model"), ("Thread(s) per core", "threads_per_core"),
                          ("Core(s) per socket", "cores_per_socket"), ("Socket(s)", "sockets")):
            m = re.search(rf"^{re.escape(key)}:\s*(.+)$", out, re.M)
            if m:
                v = m.group(1).strip()
                info[name] = int(v) if v.isdigit() else v
    except (OSError, subprocess.SubprocessError):
        pass
    cpus = sorted(os.sched_getaffinity(0))
    cores = set()
    for c in cpus:
        try:
            with open(f"/sys/devices/system/cpu/cpu{c}/topology/physical_package_id") as f:
                pkg = f.read().strip()
            with open(f"/sys/devices/system/cpu/cpu{c}/topology/core_id") as f:
                core = f.read().strip()
            cores.add((pkg, core))
        except OSError:
            cores.add(("?", str(c)))
    info["affinity_logical_cpus"] = len(cpus)
    info["affinity_physical_cores"] = len(cores)
    info["openblas_threads"] = max(1, min(len(cores), BOX_CPU_SHARE))
    return info


def contraction_flops(B, T, H, D):
    return float(D) * T * (T + 1) * B * H


def cpu_baseline(cfg, x, dy, budget_s, gpu_outs=None):
    """The oracle (C restatement of gpt.c's OpenBLAS CPU path) on this host,
    forward + backward (forward only for a forward-only config).

    gpu_outs = {name: {"y", "lse", "dqkv"}} of timed GPU steps on the same
    inputs: the last oracle run checks each (max abs error per output; the
    LSE against a float64 log-sum-exp of the oracle's q, k), as the parity
    tests do.  The errors come back per name."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as oracle_mod
    cpu = host_cpu()
    threads = cpu["openblas_threads"]
    orc = oracle_mod.Oracle(threads=threads)
    B, T, C, H = cfg["B"], cfg["T"], cfg["C"], cfg["H"]
    fwd_only = bool(cfg.get("forward_only"))
    times = []
    t_start = time.perf_counter()
    for i in range(4):
        t0 = time.perf_counter()
        y_ref, q, k, v, att = orc.forward(x, H)
        t1 = time.perf_counter()
        d_ref = None if fwd_only else orc.backward(dy, H, q, k, v, att)
        t2 = time.perf_counter()
        if i > 0:
            times.append((t1 - t0, t2 - t1))
        log(f"[cpu] run {i}: fwd {t1 - t0:.3f} s bwd {t2 - t1:.3f} s")
        if time.perf_counter() - t_start > budget_s and len(times) >= 1:
            break
    fwd = statistics.median(t[0] for t in times)
    bwd = statistics.median(t[1] for t in times)
    errs = {}
    lse_ref = lse_fp64(q, k) if gpu_outs else None
    for name, gpu_out in (gpu_outs or {}).items():
        def e(a, b):
            return float(np.abs(a.astype(np.float64) - b).max())
        err = {"y": e(gpu_out["y"], y_ref), "lse": e(gpu_out["lse"], lse_ref)}
        if not fwd_only:
            d = gpu_out["dqkv"]
            err.update(dq=e(d[..., :C], d_ref[..., :C]), dk=e(d[..., C:2 * C], d_ref[..., C:2 * C]),
                       dv=e(d[..., 2 * C:], d_ref[..., 2 * C:]))
        err["tolerance"] = 1e-4
        errs[name] = err
    sample = (f"one full {cfg['workload']} call (B={B} T={T} H={H}), 1 warm-up then median of {len(times)}; "
              f"fwd {fwd * 1e3:.1f} ms" + ("" if fwd_only else f" + bwd {bwd * 1e3:.1f} ms") +
              f"; OPENBLAS threads={threads} (one per physical core of the affinity set, at most "
              f"{BOX_CPU_SHARE}); {orc.blas_config}")
    if fwd_only:
        fwd_bytes, _ = compulsory_bytes(B, T, C, H)
        value, unit, ms = fwd_bytes / fwd / 1e9, "GB/s", fwd * 1e3
    else:
        value, unit, ms = 6 * contraction_flops(B, T, H, C // H) / (fwd + bwd) / 1e12, "TFLOP/s", (fwd + bwd) * 1e3
    return {"value": value, "unit": unit, "cores": threads, "kind": "port", "sample": sample,
            "ms_per_step": ms, "host": cpu, "openblas": orc.blas_config, "gpu_max_abs_err": errs}


def copy_calibration(args):
    """Plain device copy of a known size through copy_tensor_data_cuda.

    Used to scale rocprof's FETCH_SIZE / WRITE_SIZE counters (a copy of N
    bytes must fetch N and write N) and as the achievable-bandwidth check.
    """
    n = 64 << 20  # floats: 256 MiB per buffer, larger than the 256 MB MALL
    lib = gptc.load()
    rt = gptc.Runtime(lib)
    rt.init()
    hip = Hip()
    src = lib.fill((ctypes.c_int * 1)(n), 1, ctypes.c_float(1.0), gptc.CUDA)
    dst = rt.empty((n,))
    for _ in range(args.warmup):
        lib.tensor_copy(dst, src)
    rt.sync()
    a, b = hip.event(), hip.event()
    hip.record(a, rt.stream())
    for _ in range(args.steps):
        lib.tensor_copy(dst, src)
    hip.record(b, rt.stream())
    ms = hip.elapsed_ms(a, b) / args.steps
    nbytes = 4 * n
    print(json.dumps({"workload": "copy", "bytes_read_per_launch": nbytes, "bytes_written_per_launch": nbytes,
                      "ms_per_launch": round(ms, 5), "GB_per_s": round(2 * nbytes / (ms * 1e-3) / 1e9, 1),
                      "hbm_peak_GB_per_s": HBM_PEAK_GBS}), flush=True)
    rt.free(src)
    rt.free(dst)
    rt.sync()


def decode_bench(args):
    """C4's attention: the KV-cache decode step at GPT-2 small's heads (B=1,
    C=768, H=12), over the caches of --decode-layers layers (default 12, the
    model's depth, so that the K/V set per position is the model's, not one
    layer's that would stay in L2).

    A 64-token prompt fills the caches, then 448 generated tokens (positions
    64..511) are timed, one attention_decode_cuda_kernel call per layer each,
    inputs resident in HBM: exactly K = 448 x layers back-to-back launches
    between two events on the library stream.  Metric: compulsory HBM bytes per step (cached K
    and V rows 0..pos-1 read once, the new q, k, v row read, its k, v and the
    output row written) over the time per step.  Every step is one kernel
    (attn_decode_head_kernel), so the roofline's duration is the same
    interval: the launch-to-launch time, kernel plus dispatch gap.
    Beside it: the reference-literal step, gpt.c's infer_gpt.c:339-351
    recompute of the full 1024-token window, through this library's forward
    and (cpu_baseline) through the oracle on the host.
    """
    B, C, H, L, prompt, last = 1, 768, 12, 1024, 64, 512
    D = C // H
    layers = args.decode_layers
    lib = gptc.load()
    rt = gptc.Runtime(lib)
    rt.init()
    hip = Hip()
    stream = rt.stream()
    x = rt.normal((B, last, 3 * C), SEED_X)
    rows = [rt.from_numpy(x[:, p:p + 1, :]) for p in range(last)]
    kvs = [(rt.empty((B, H, L, D)), rt.empty((B, H, L, D))) for _ in range(layers)]
    out = rt.empty((B, 1, C))
    for p in range(prompt):
        for kc, vc in kvs:
            lib.attention_decode_cuda_kernel(rows[p], kc, vc, p, H, out)
    rt.sync()
    hip.device_sync()
    a, b = hip.event(), hip.event()
    hip.record(a, stream)
    for p in range(prompt, last):
        for kc, vc in kvs:
            lib.attention_decode_cuda_kernel(rows[p], kc, vc, p, H, out)
    hip.record(b, stream)
    steps = last - prompt
    us = hip.elapsed_ms(a, b) * 1e3 / (steps * layers)
    y_last = rt.to_numpy(out)
    # Compulsory bytes: cached key and value rows 0..pos-1 read once, the new
    # q, k, v row read, its k, v written to the caches and the output row.
    kv_bytes = sum(2 * p * C * 4 for p in range(prompt, last))
    io_bytes = steps * (3 * C + 2 * C + C) * 4
    step_bytes = (kv_bytes + io_bytes) / steps
    gbs = step_bytes / (us * 1e-6) / 1e9

    # Reference-literal: forward over the full window for every token.
    xw = rt.from_numpy(rt.normal((B, L, 3 * C), SEED_X))
    mask = rt.from_numpy(np.tril(np.ones((L, L), np.float32)))
    caches = (gptc.TensorP * 4)(xw, rt.empty((B, L, C)), rt.empty((B, H, L)),
                                rt.empty((lib.gptc_attention_state_floats(B, L, C, H),)))
    yw = rt.empty((B, L, C))
    for _ in range(args.warmup):
        lib.attention_forward_cuda_kernel(xw, mask, H, caches, yw)
    rt.sync()
    hip.record(a, stream)
    for _ in range(args.steps):
        lib.attention_forward_cuda_kernel(xw, mask, H, caches, yw)
    hip.record(b, stream)
    win_us = hip.elapsed_ms(a, b) * 1e3 / args.steps

    kernel = "attn_decode_head_kernel"
    roof = {"kernel": kernel, "bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 5), "traffic": None, "algorithmic_bytes_per_launch": round(step_bytes),
            "duration_ms": round(us * 1e-3, 6),
            "duration_source": "the timed region: K back-to-back decode launches (one kernel each) between two "
                               "events, / K (kernel plus dispatch gap)"}
    traffic_file = os.path.join(ROOT, "profiles", "hbm_traffic_decode.json")
    if os.path.exists(traffic_file):
        with open(traffic_file) as fh:
            tr = json.load(fh)
        k = tr["kernels"].get(kernel)
        if k:
            roof["traffic"] = k["read_bytes"] + k["write_bytes"]
            roof["traffic_source"] = (f"profiles/hbm_traffic_decode.json (rocprofv3 FETCH_SIZE x{tr['fetch_scale']:.2f}"
                                      f" + WRITE_SIZE x{tr['write_scale']:.2f}, mean over the K launches)")
    result = {
        "metric": "C4 decode attention step, compulsory HBM GB/s, B=1 C=768 H=12 D=64, positions 64..511",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": prompt,
        "ms_per_step": round(us * 1e-3, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "step": "one decode launch: one layer's attention for one position",
        "dtype": "fp32", "data": f"synthetic: qkv rows ~ N(0,1) seed {SEED_X} (torch-identical mt19937)",
        "config": {"workload": f"C4 KV-cache decode attention, GPT-2 small's heads (B=1, C=768, H=12) over {layers} "
                               "layers' caches, a 64-token prompt then positions 64..511", "B": B, "C": C, "H": H,
                   "D": D, "L": L, "layers": layers},
        "us_per_step": round(us, 3), "bytes_per_step": round(step_bytes),
        "pct_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 3),
        "window_forward_us_per_step": round(win_us, 2),
        "speedup_vs_window_recompute": round(win_us / us, 1),
        "roofline": roof,
        "note": "latency bound at B=1: 12 workgroups (one per head), one memory round trip per launch",
    }
    for t in rows + [t for kv in kvs for t in kv] + [out, xw, mask, yw, *caches[1:]]:
        rt.free(t)
    rt.sync()

    if args.no_cpu_baseline:
        result["cpu_baseline"] = None
    else:
        # gpt.c's own per-token attention work at C4 (infer_gpt.c:339-351): the
        # oracle's forward over the whole block_size window, on the host; the
        # value is the rate at which it yields the same output rows, in the
        # GPU metric's unit (the decode step's compulsory bytes per token).
        # Its window row 511 also checks the last timed decode output.
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as oracle_mod
        cpu = host_cpu()
        orc = oracle_mod.Oracle(threads=cpu["openblas_threads"])
        xwin = np.concatenate([x, rt.normal((B, L, 3 * C), SEED_X + 7)[:, last:]], axis=1)
        times = []
        t_start = time.perf_counter()
        y_ref = None
        for i in range(6):
            t0 = time.perf_counter()
            y_ref, *_ = orc.forward(xwin, H)
            times.append(time.perf_counter() - t0)
            if i >= 2 and time.perf_counter() - t_start > args.cpu_budget_s:
                break
        sec = statistics.median(times[1:])
        err = float(np.abs(y_last[:, 0].astype(np.float64) - y_ref[:, last - 1]).max())
        result["cpu_baseline"] = {
            "value": round(step_bytes / sec / 1e9, 4), "unit": "GB/s", "cores": cpu["openblas_threads"],
            "kind": "port", "ms_per_step": round(sec * 1e3, 3),
            "sample": (f"gpt.c's per-token step at C4: the oracle's forward over the full {L}-token window "
                       f"(B=1, H={H}), warm-up then median of {len(times) - 1}: {sec * 1e3:.1f} ms per token; "
                       f"OPENBLAS threads={cpu['openblas_threads']} (one per physical core of the affinity set, "
                       f"at most {BOX_CPU_SHARE}); {orc.blas_config}"),
            "host": cpu,
            "gpu_max_abs_err": {"y_pos511_vs_window_row": err, "tolerance": 1e-4},
        }
    print(json.dumps(result), flush=True)


def gpt2_step_flops(B, T, L, C, V):
    """Algorithmic flops of one GPT-2 training step: 2 per multiply-add of every
    Linear (qkv 3C^2, c_proj C^2, c_fc 4C^2, mlp c_proj 4C^2 per layer, lm_head
    C V), x3 for forward + the two backward products, plus the six causal
    attention contractions per layer."""
    linear = 2 * B * T * (L * 12 * C * C + C * V) * 3
    attn = L * 6 * contraction_flops(B, T, 12, C // 12)
    return linear + attn, attn


def c4_bench(args):
    """C4: greedy generation with GPT-2 124M (N(0, 0.02) init), B=1, a 64-token
    uniform prompt, 448 new tokens to T=512.  Two loops on the same model:
    the one-token KV-cache step (gptc_gpt2_decode) and infer_gpt.c's
    reference context handling (the 1024-token window through GPT2.forward
    for every token).  Both produce the same tokens (tests/test_generate_gpu.py);
    here they are timed end to end, host loop included."""
    from generation import graph_generate, kv_generate, window_generate
    V, block, L, H, C, prompt_len, total = 50257, 1024, 12, 12, 768, 64, 512
    lib = gptc.load()
    rt = gptc.Runtime(lib)
    rt.init()
    model = gptc.GPT2Model(rt, block, V, L, H, C)
    params = model.random_init_arrays()
    n_weights = sum(p.size for p in params)
    model.fast_load(params)
    del params
    model.to(gptc.CUDA)
    prompt = np.random.default_rng(SEED_X).integers(0, V, prompt_len)
    new = total - prompt_len
    loops = set(args.c4_loops.split(","))
    toks = gtoks = wtoks = None
    kv_s = graph_s = win_s = float("nan")
    if "eager" in loops:
        kv_generate(rt, model, prompt, prompt_len + 8, block)  # warm-up
        rt.sync()
        t0 = time.perf_counter()
        toks, _ = kv_generate(rt, model, prompt, total, block)
        rt.sync()
        kv_s = time.perf_counter() - t0
    if "graph" in loops:
        cache = gptc.KVCache(rt, model, 1, total)
        graph_generate(rt, model, prompt, total, cache)  # warm-up: captures the step graph
        rt.sync()
        t0 = time.perf_counter()
        gtoks = graph_generate(rt, model, prompt, total, cache)
        graph_s = time.perf_counter() - t0
        cache.free()
    if "window" in loops:
        window_generate(rt, model, prompt, prompt_len + 2, block)  # warm-up
        rt.sync()
        t0 = time.perf_counter()
        wtoks, _ = window_generate(rt, model, prompt, total, block)
        rt.sync()
        win_s = time.perf_counter() - t0
    model.free()
    g_tok = graph_s / (total - 1)
    # Per generated token the decode path reads every weight once (the tied
    # wte twice: embedding row and lm_head) and the cached keys and values.
    kv_bytes = sum(2 * L * (p + 1) * C * 4 for p in range(prompt_len - 1, total - 1)) / new
    step_bytes = n_weights * 4 + kv_bytes
    # The prompt's 63 decode steps are part of the timed loop too.
    per_tok = kv_s / (total - 1)
    print(json.dumps({
        "workload": "C4 greedy generation, GPT-2 124M (N(0,0.02) init), B=1, prompt 64, 448 new tokens to T=512",
        "kv_cache_graph": {"s_total": round(graph_s, 4), "ms_per_step": round(g_tok * 1e3, 4),
                           "tokens_per_s": round(new / graph_s, 1), "bytes_per_step": round(step_bytes),
                           "GB_per_s": round(step_bytes / g_tok / 1e9, 1), "hbm_peak_GB_per_s": HBM_PEAK_GBS,
                           "note": "gptc_gpt2_generate: one captured step replayed per position, no host wait "
                                   "between tokens (511 steps: 63 prompt + 448 generated)"},
        "kv_cache_eager": {"s_total": round(kv_s, 3), "ms_per_step": round(per_tok * 1e3, 3),
                           "tokens_per_s": round(new / kv_s, 1),
                           "note": "gptc_gpt2_decode per token from Python, token id read back each step"},
        "window_recompute": {"s_total": round(win_s, 3), "ms_per_token": round(win_s / new * 1e3, 3),
                             "tokens_per_s": round(new / win_s, 1),
                             "note": "infer_gpt.c's loop: the 1024-token window through GPT2.forward per token"},
        "speedup_graph_vs_window": round(win_s / graph_s, 1),
        "same_tokens": all(np.array_equal(u, v) for u, v in ((toks, wtoks), (gtoks, toks), (gtoks, wtoks))
                           if u is not None and v is not None),
        "loops": sorted(loops),
    }), flush=True)
    rt.sync()


def gpt2_cpu_baseline(rt, V, block, L, H, C):
    """The oracle's GPT-2 step (C restatements of gpt.c's CPU kernels over
    OpenBLAS) on a bounded sample of C3: one sequence (B=1, T=1024) through
    the full 12-layer model, forward + loss + backward + AdamW, median of 2
    after a warm-up."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as oracle_mod
    from gpt2_oracle import GPT2Oracle, param_shapes
    cpu = host_cpu()
    threads = cpu["openblas_threads"]
    orc = oracle_mod.Oracle(threads=threads)
    params = []
    for i, (name, shp) in enumerate(param_shapes(V, block, L, C)):
        if name.endswith(("ln1.W", "ln2.W")) or name == "ln_f.W":
            params.append(np.ones(shp, np.float32))
        elif len(shp) == 1:
            params.append(np.zeros(shp, np.float32))
        else:
            params.append(rt.normal(shp, 1000 + i, 0.0, 0.02))
    rng = np.random.default_rng(SEED_X)
    ids, tg = rng.integers(0, V, (1, block)), rng.integers(0, V, (1, block))
    g = GPT2Oracle(orc, params, L, H)
    del params
    times = []
    for i in range(3):
        t0 = time.perf_counter()
        g.loss(g.forward(ids), tg)
        g.backward()
        g.step()
        times.append(time.perf_counter() - t0)
        log(f"[cpu] GPT-2 step {i}: {times[-1]:.2f} s")
    sec = statistics.median(times[1:])
    return {"value": round(block / sec, 1), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": (f"one GPT-2 124M training step at B=1 T={block} (1/8 of C3's batch), warm-up then median "
                       f"of 2: {sec:.2f} s; OPENBLAS threads={threads} (one per physical core of the affinity "
                       f"set, at most {BOX_CPU_SHARE}); {orc.blas_config}"),
            "host": cpu}


def gpt2_bench(args):
    """C3: one GPT-2 124M training step (train_gpt.c:481-521's loop body:
    zero_grad, forward, CrossEntropyLoss forward and backward, model backward,
    AdamW step) at B=8, T=1024, on the library's layer objects.  Weights are
    C3's random init (N(0, 0.02) matrices and embeddings, zero biases,
    LayerNorm weight 1); token ids and targets uniform in [0, 50257).  The
    batch sits in HBM; each step copies it into the fresh id tensors that the
    model and the loss take ownership of, as train_gpt.c's moves do."""
    B, T, L, H, C, V, block = 8, 1024, 12, 12, 768, 50257, 1024
    lib = gptc.load()
    rt = gptc.Runtime(lib)
    rt.init()
    hip = Hip()
    stream = rt.stream()
    rng = np.random.default_rng(SEED_X)
    ids = rt.from_numpy(rng.integers(0, V, (B, T)).astype(np.float32))
    tgs = rt.from_numpy(rng.integers(0, V, (B, T)).astype(np.float32))
    ones = rt.from_numpy(np.ones((B, T), np.float32))
    model = gptc.GPT2Model(rt, block, V, L, H, C)
    params = model.random_init_arrays()
    model.fast_load(params)
    del params
    model.to(gptc.CUDA)
    opt = gptc.AdamWOptimizer(rt, model, lr=3e-4, beta1=0.9, beta2=0.99, eps=1e-8, weight_decay=0.0)
    loss_fn = gptc.CrossEntropy(rt)
    losses_seen = []

    def step(keep_loss=False):
        x, t, g = rt.empty((B, T)), rt.empty((B, T)), rt.empty((B, T))
        lib.tensor_copy(x, ids)
        lib.tensor_copy(t, tgs)
        lib.tensor_copy(g, ones)
        opt.zero_grad()
        logits = model.forward(x)
        losses = loss_fn.forward(logits, t)
        rt.free(logits)
        g = loss_fn.backward(g)
        g = model.backward(g)
        if g:
            rt.free(g)
        opt.step()
        if keep_loss:
            losses_seen.append(float(rt.to_numpy(losses)[0]))
        rt.free(losses)

    log(f"[bench] C3 GPT-2 124M training step B={B} T={T}; warmup {args.warmup}, steps {args.steps}")
    for i in range(args.warmup):
        step(keep_loss=(i == 0))
    rt.sync()
    hip.device_sync()
    a, b = hip.event(), hip.event()
    t0 = time.perf_counter()
    hip.record(a, stream)
    for _ in range(args.steps):
        step()
    hip.record(b, stream)
    ms = hip.elapsed_ms(a, b) / args.steps
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    step(keep_loss=True)
    rt.sync()
    flops, attn_flops = gpt2_step_flops(B, T, L, C, V)
    peak, cu, mhz, src = device_peak()
    tflops = flops / (ms * 1e-3) / 1e12
    cpu = None
    if not args.no_cpu_baseline:
        cpu = gpt2_cpu_baseline(rt, V, block, L, H, C)
    print(json.dumps({
        "workload": "C3 GPT-2 124M training step (fwd + CrossEntropy + bwd + AdamW), B=8 T=1024, fp32",
        "metric": "tokens/s", "value": round(B * T / (ms * 1e-3), 1), "unit": "tokens/s",
        "ms_per_step": round(ms, 3), "wall_ms_per_step": round(wall_ms, 3), "steps": args.steps,
        "warmup": args.warmup, "tflops": round(tflops, 2), "pct_fp32_mfma_peak": round(100 * tflops / peak, 2),
        "flops_per_step": flops, "attention_flops_per_step": attn_flops,
        "loss_first_step": round(losses_seen[0], 6), "loss_after": round(losses_seen[-1], 6),
        "dtype": "fp32", "data": "synthetic (uniform token ids, N(0,0.02) init)",
        "cpu_baseline": cpu,
    }), flush=True)
    opt.free()
    loss_fn.free()
    model.free()
    for t in (ids, tgs, ones):
        rt.free(t)
    rt.sync()


def attention_metric(cfg):
    """The metric string of a config: BASELINE.json's for C2, the same form
    with each config's own shape otherwise; C1 is forward-only and HBM-side,
    so its metric is compulsory GB/s."""
    B, T, H, D = cfg["B"], cfg["T"], cfg["H"], cfg["C"] // cfg["H"]
    if cfg.get("forward_only"):
        return f"causal attn fwd compulsory HBM GB/s (cold MALL), B={B} T={T} H={H} D={D}"
    return f"causal attn fwd+bwd TFLOP/s + % fp32 MFMA peak, B={B} T={T} H={H} D={D}"


def compulsory_bytes(B, T, C, H):
    """Compulsory HBM bytes: forward reads qkv, writes y and the LSE;
    backward reads qkv, y, dy and the LSE, writes dqkv."""
    fwd = 4.0 * (B * T * (3 * C + C) + B * H * T)
    bwd = 4.0 * (B * T * (3 * C + 2 * C) + B * H * T + B * T * 3 * C)
    return fwd, bwd


def lse_fp64(q, k):
    """Natural-log causal row log-sum-exp of (B, H, T, D) q, k in float64."""
    B, H, T, D = q.shape
    out = np.empty((B, H, T))
    keep = np.tril(np.ones((T, T), bool))
    for b in range(B):
        s = np.matmul(q[b].astype(np.float64), k[b].astype(np.float64).transpose(0, 2, 1)) / np.sqrt(D)
        s = np.where(keep, s, -np.inf)
        m = s.max(-1)
        out[b] = m + np.log(np.exp(s - m[..., None]).sum(-1))
    return out


def attention_bench(args):
    cfg = CONFIGS[args.config]
    B, T, C, H = cfg["B"], cfg["T"], cfg["C"], cfg["H"]
    D = C // H
    fwd_only = bool(cfg.get("forward_only"))
    lib = gptc.load()
    rt = gptc.Runtime(lib)
    rt.init()
    hip = Hip()
    stream = rt.stream()

    x = rt.normal((B, T, 3 * C), SEED_X)
    dy = rt.normal((B, T, C), SEED_DY)
    xt = rt.from_numpy(x)
    dyt = rt.from_numpy(dy)
    mask = rt.from_numpy(np.tril(np.ones((T, T), np.float32)))
    # Compact cache layout of the library's Attention(): cache[0] is the input
    # itself, cache[3] the 1-D backward state (probability blocks and maxima).
    n_state = lib.gptc_attention_state_floats(B, T, C, H)

    def make_set(xin):
        # As Attention() sets it up: cache[1] is the output tensor itself
        # (the layer keeps y for the backward by sharing its storage).
        y = rt.empty((B, T, C))
        return (gptc.TensorP * 4)(xin, y, rt.empty((B, H, T)), rt.empty((n_state,))), y

    caches, yt = make_set(xt)
    dqkv = rt.empty((B, T, 3 * C))
    rt.sync()

    def fwd(c=caches, y=yt):
        lib.attention_forward_cuda_kernel(c[0], mask, H, c, y)

    def step():
        fwd()
        lib.attention_backward_cuda_kernel(dyt, caches, H, dqkv)

    def timed(fn, n):
        """ms per call of n back-to-back calls between two events on the library stream."""
        a, b = hip.event(), hip.event()
        hip.record(a, stream)
        for i in range(n):
            fn(i)
        hip.record(b, stream)
        return hip.elapsed_ms(a, b) / n

    log(f"[bench] {cfg['workload']}: B={B} T={T} H={H} D={D}; warmup {args.warmup}, steps {args.steps}")
    # Device pre-warm, untimed, before the W warm-up steps: a kernel trace of
    # this bench shows the GPU's clocks settling over the first ~40 ms of
    # sustained load (step time 0.53 -> 0.41 ms at C2), so a short warm-up
    # would time the power-management ramp instead of the kernels.  Steps
    # run until prewarm_ms of wall time have passed; the line reports it.
    t_pre = time.perf_counter()
    n_pre = 0
    while (time.perf_counter() - t_pre) * 1e3 < args.prewarm_ms:
        for _ in range(8):
            step()
        n_pre += 8
        rt.sync()
    prewarm = {"ms": round((time.perf_counter() - t_pre) * 1e3, 1), "steps": n_pre,
               "reason": "untimed, before the W warm-up steps: lets the clocks settle under sustained load"}
    for _ in range(args.warmup):
        step()
    rt.sync()
    hip.device_sync()

    # Headline: exactly K fwd+bwd steps between two events, nothing else on the stream.
    ms_step = timed(lambda i: step(), args.steps)
    rt.sync()
    hip.device_sync()
    # The same K-step measurement repeated, for the spread.
    reps = [timed(lambda i: step(), args.steps) for _ in range(args.reps)]

    # Per-kernel durations: K more steps with events recorded by the entry points
    # around every kernel launch (each boundary then carries an event).
    kernels = ("fwd", "bwd_delta", "bwd_dkdv", "bwd_dq")
    k_ms = None
    if not args.no_kernel_pass:
        n_ev = 2 * len(kernels)
        evs = [[hip.event() for _ in range(n_ev)] for _ in range(args.steps)]
        ev_arrays = [(ctypes.c_void_p * n_ev)(*e) for e in evs]
        for i in range(args.steps):
            lib.gptc_set_kernel_events(ev_arrays[i], n_ev)
            step()
        rt.sync()
        hip.device_sync()
        lib.gptc_set_kernel_events(None, 0)
        k_ms = {name: statistics.median(hip.elapsed_ms(e[2 * j], e[2 * j + 1]) for e in evs)
                for j, name in enumerate(kernels)}

    # The layer API as SelfAttention calls it (attn->forward / attn->backward
    # through Attention()'s function pointers), allocation of the caches, y
    # and dqkv included; the fresh input copies the layer takes ownership of
    # are made outside the event pairs.
    layer = gptc.AttentionLayer(rt, C, H, T)
    layer.to(gptc.CUDA)
    api_f, api_b = [], []
    for i in range(args.warmup + args.steps):
        xi, di = rt.empty((B, T, 3 * C)), rt.empty((B, T, C))
        lib.tensor_copy(xi, xt)
        lib.tensor_copy(di, dyt)
        e = [hip.event() for _ in range(4)]
        hip.record(e[0], stream)
        yi = layer.forward(xi)
        hip.record(e[1], stream)
        rt.free(yi)
        hip.record(e[2], stream)
        gi = layer.backward(di)
        hip.record(e[3], stream)
        rt.free(gi)
        if i >= args.warmup:
            api_f.append(hip.elapsed_ms(e[0], e[1]))
            api_b.append(hip.elapsed_ms(e[2], e[3]))
    layer.free()
    rt.sync()

    # Forward alone, warm (one input, resident in the 256 MB MALL) and cold
    # (rotating over enough input sets that every forward's inputs were
    # evicted by the others' traffic).
    ms_fwd_warm = timed(lambda i: fwd(), args.steps)
    set_bytes = 4 * (B * T * 3 * C + B * T * C + B * H * T + n_state)
    n_sets = max(3, int(np.ceil(2 * 256e6 / set_bytes)) + 1)
    cold = [make_set(rt.from_numpy(x)) for _ in range(n_sets)] if n_sets * set_bytes < 8e9 else []
    ms_fwd_cold = None
    if cold:
        for c, y in cold:
            fwd(c, y)
        rt.sync()
        ms_fwd_cold = timed(lambda i: fwd(*cold[i % n_sets]), max(args.steps, 2 * n_sets))
        rt.sync()
        for c, y in cold:
            for t in (c[0], c[2], c[3], y):
                rt.free(t)
    # The floor for moving the forward's compulsory bytes: a plain device
    # copy of fwd_bytes / 2 (it reads and writes that much), timed cold the
    # same way (forward-only configs).
    copy_floor_us = None
    if fwd_only:
        n_copy = int(compulsory_bytes(B, T, C, H)[0] // 8)
        n_cs = int(np.ceil(2 * 256e6 / (8 * n_copy))) + 1
        srcs = [rt.from_numpy(np.ones(n_copy, np.float32)) for _ in range(n_cs)]
        dsts = [rt.empty((n_copy,)) for _ in range(n_cs)]
        for i in range(n_cs):
            lib.tensor_copy(dsts[i], srcs[i])
        rt.sync()
        copy_floor_us = 1e3 * timed(lambda i: lib.tensor_copy(dsts[i % n_cs], srcs[i % n_cs]),
                                    max(args.steps, 2 * n_cs))
        rt.sync()
        for t in srcs + dsts:
            rt.free(t)
    # The LSE-only state (the north star's backward: P recomputed from the
    # saved log-sum-exp; dS handed to the dq kernel through a scratch), timed
    # the same way in the same process: the state limit at 0 makes every
    # D = 64 forward keep only the LSE.  The first forward re-points cache[3]
    # to the shorter state (outside the timed region).
    lse_res, lse_out = None, None
    if not fwd_only and D == 64:
        prev_limit = lib.gptc_attention_set_state_limit(0)
        # The first step re-points the state; the warm-up then runs long
        # enough for the clocks to settle on the new kernel mix (the first
        # K-step pass after 10 steps measured 2 % above the repetitions).
        for _ in range(max(args.warmup, 40)):
            step()
        rt.sync()
        ms_lse = timed(lambda i: step(), args.steps)
        rt.sync()
        reps_lse = [timed(lambda i: step(), args.steps) for _ in range(max(1, args.reps // 2))]
        k_lse = None
        if not args.no_kernel_pass:
            n_ev = 2 * len(kernels)
            evs = [[hip.event() for _ in range(n_ev)] for _ in range(args.steps)]
            ev_arrays = [(ctypes.c_void_p * n_ev)(*e) for e in evs]
            for i in range(args.steps):
                lib.gptc_set_kernel_events(ev_arrays[i], n_ev)
                step()
            rt.sync()
            hip.device_sync()
            lib.gptc_set_kernel_events(None, 0)
            k_lse = {name: round(statistics.median(hip.elapsed_ms(e[2 * j], e[2 * j + 1]) for e in evs), 5)
                     for j, name in enumerate(kernels)}
        step()
        rt.sync()
        if not args.no_cpu_baseline:
            lse_out = {"y": rt.to_numpy(yt), "lse": rt.to_numpy(caches[2]).reshape(B, H, T),
                       "dqkv": rt.to_numpy(dqkv)}
        lib.gptc_attention_set_state_limit(prev_limit)
        t_lse = 6 * contraction_flops(B, T, H, D) / (ms_lse * 1e-3) / 1e12
        lse_res = {
            "ms_per_step": round(ms_lse, 5), "tflops": round(t_lse, 3),
            "reps_ms_per_step": {"n": len(reps_lse), "median": round(statistics.median(reps_lse), 5),
                                 "min": round(min(reps_lse), 5), "max": round(max(reps_lse), 5)},
            "kernel_ms": k_lse,
            "state_floats": lib.gptc_attention_state_floats(B, T, C, H),
            "note": ("the forward keeps only the log-sum-exp (O(T) per head); the dk/dv kernel recomputes P from it "
                     "(S, dP, dV, dK: 4 contractions) and writes dS to a scratch the dq kernel reads (1 contraction); "
                     "kernel_ms keys as in the headline, dkdv = attn_bwd_dkdv_dma_kernel<RECOMP>"),
        }
        log(f"[bench] LSE-only state: {ms_lse:.4f} ms/step, {t_lse:.2f} TFLOP/s; kernels (ms): {k_lse}")

    step()  # leave the headline buffers with one fwd+bwd of the seeded inputs
    rt.sync()

    unit = contraction_flops(B, T, H, D)
    peak, cu, mhz, peak_src = device_peak()
    fwd_bytes, bwd_bytes = compulsory_bytes(B, T, C, H)
    value_tflops = 6 * unit / (ms_step * 1e-3) / 1e12
    fwd_cold_gbs = fwd_bytes / (ms_fwd_cold * 1e-3) / 1e9 if ms_fwd_cold else None
    log(f"[bench] {ms_step:.4f} ms/step, {value_tflops:.2f} TFLOP/s; forward warm {ms_fwd_warm * 1e3:.2f} us, "
        f"cold {ms_fwd_cold and ms_fwd_cold * 1e3:.2f} us; kernels (ms): {k_ms}")

    result = {
        "metric": attention_metric(cfg),
        "value": round(fwd_cold_gbs, 1) if fwd_only else round(value_tflops, 3),
        "unit": "GB/s" if fwd_only else "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "prewarm": prewarm,
        "ms_per_step": round(ms_fwd_cold if fwd_only else ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": f"synthetic: qkv ~ N(0,1) seed {SEED_X}, dout ~ N(0,1) seed {SEED_DY} (torch-identical mt19937)",
        "config": {"workload": cfg["workload"], "B": B, "T": T, "H": H, "D": D, "C": C,
                   "causal_flop_per_step": (2 if fwd_only else 6) * unit},
        "fwd_bwd": {
            "ms_per_step": round(ms_step, 5),
            "tflops": round(value_tflops, 3),
            "pct_fp32_mfma_peak": round(100.0 * value_tflops / peak, 2),
            "reps_ms_per_step": reps and {"n": len(reps), "median": round(statistics.median(reps), 5),
                                          "min": round(min(reps), 5), "max": round(max(reps), 5)},
            # FlashAttention's convention (full T^2 work, backward 2.5x forward), for comparison only.
            "tflops_fa_convention": round(7.0 * B * H * T * T * D / (ms_step * 1e-3) / 1e12, 3),
            "compulsory_gb_per_s": round((fwd_bytes + bwd_bytes) / (ms_step * 1e-3) / 1e9, 1),
            "tokens_per_s": round(B * T / (ms_step * 1e-3), 1),
        },
        "forward": {
            "us_warm": round(ms_fwd_warm * 1e3, 3),
            "us_cold": ms_fwd_cold and round(ms_fwd_cold * 1e3, 3),
            "cold_input_sets": n_sets if cold else 0,
            "compulsory_bytes": fwd_bytes,
            "gb_per_s_warm": round(fwd_bytes / (ms_fwd_warm * 1e-3) / 1e9, 1),
            "gb_per_s_cold": fwd_cold_gbs and round(fwd_cold_gbs, 1),
            "tflops_warm": round(2 * unit / (ms_fwd_warm * 1e-3) / 1e12, 3),
            "copy_floor_us_cold": copy_floor_us and round(copy_floor_us, 3),
        },
        "api_ms": {"forward_median": round(statistics.median(api_f), 5),
                   "backward_median": round(statistics.median(api_b), 5),
                   "step_median": round(statistics.median(a + b for a, b in zip(api_f, api_b)), 5),
                   "note": "attn->forward / attn->backward through Attention(), allocation included"},
        "peak_tflops": round(peak, 2),
        "peak_source": f"{peak_src}: {cu} CU x {mhz} MHz x {FLOP_PER_CLK_CU_FP32_MFMA} flop/clk/CU",
        "kernel_ms": k_ms and {k: round(v, 5) for k, v in k_ms.items()},
    }
    if fwd_only:
        result["pct_hbm_peak"] = round(100.0 * fwd_cold_gbs / HBM_PEAK_GBS, 2)
    else:
        result["pct_fp32_mfma_peak"] = round(100.0 * value_tflops / peak, 2)
        result["tflops_fa_convention"] = result["fwd_bwd"]["tflops_fa_convention"]
        result["tokens_per_s"] = result["fwd_bwd"]["tokens_per_s"]

    # Roofline of the dominant kernel: algorithmic work of one launch over its
    # median duration in the per-kernel pass.  Contractions per kernel: forward
    # S and PV; dk/dv kernel dP, dV, dK; dq kernel dQ (delta does none).
    if k_ms:
        kernel_flops = {"fwd": 2 * unit, "bwd_delta": 0.0, "bwd_dkdv": 3 * unit, "bwd_dq": 1 * unit}
        # Kernel symbols per head size (D == 64: the 16-row kernels; short
        # heads: T <= 64 one workgroup per block, 64 < T <= 128 two per head).
        fwd_sym = "attn_fwd16_kernel" if T > 128 else ("attn_fwd_twotile_kernel" if T > 64 else "attn_fwd_short_kernel")
        # dk/dv: the LDS-direct kernel for D == 64 heads with the stored P'
        # (T > 128), the general one otherwise.
        symbols = {"fwd": "attn_fwd_kernel" if D != 64 else fwd_sym,
                   "bwd_delta": "attn_bwd_delta_kernel",
                   "bwd_dkdv": "attn_bwd_dkdv_dma_kernel" if D == 64 and T > 128 else "attn_bwd_dkdv_kernel",
                   "bwd_dq": "attn_bwd_dq16_kernel" if D == 64 else "attn_bwd_dq_kernel"}
        dom = "fwd" if fwd_only else max(k_ms, key=k_ms.get)
        if fwd_only:
            # The forward is the only kernel of the timed region (K cold
            # launches between two events): its average launch duration is
            # the region over K, the same interval as `value`.
            dur_ms, dur_src = ms_fwd_cold, "the timed region: K cold forward launches between two events, / K"
            achieved = fwd_bytes / (dur_ms * 1e-3) / 1e9
            roof = {"kernel": dom, "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                    "algorithmic_bytes_per_launch": fwd_bytes}
        else:
            # The per-kernel pass brackets every launch with events, which adds
            # a fixed cost to each interval that the headline pass (no events)
            # does not pay: the four medians sum to more than ms_step.  That
            # excess, shared equally, is taken off the dominant kernel's median
            # (a kernel trace of the headline pass gives the same duration).
            ev_ms = k_ms[dom]
            per_event = max(0.0, (sum(k_ms.values()) - ms_step) / len(k_ms))
            dur_ms = ev_ms - per_event
            dur_src = ("median of the per-kernel event pass less the events' cost: (sum of the per-kernel medians "
                       "- headline ms/step) / number of kernels")
            achieved = kernel_flops[dom] / (dur_ms * 1e-3) / 1e12
            roof = {"kernel": dom, "bound": "mfma", "achieved": round(achieved, 3), "peak": round(peak, 2),
                    "unit": "TFLOP/s", "frac": round(achieved / peak, 4), "traffic": None,
                    "algorithmic_flop_per_launch": kernel_flops[dom]}
        roof["duration_ms"] = round(dur_ms, 5)
        roof["duration_source"] = dur_src
        if not fwd_only:
            roof["duration_event_ms"] = round(ev_ms, 5)
        # HBM bytes per launch from the committed rocprof byte-counter runs
        # (FETCH_SIZE and WRITE_SIZE, scaled by a plain copy of known size).
        traffic_file = os.path.join(ROOT, "profiles", f"hbm_traffic_{args.config}.json")
        sym = symbols[dom]
        if os.path.exists(traffic_file):
            with open(traffic_file) as fh:
                tr = json.load(fh)
            k = tr["kernels"].get(sym)
            if k:
                roof["traffic"] = k["read_bytes"] + k["write_bytes"]
                roof["traffic_source"] = (f"profiles/hbm_traffic_{args.config}.json (rocprofv3 FETCH_SIZE "
                                          f"x{tr['fetch_scale']:.2f} + WRITE_SIZE x{tr['write_scale']:.2f})")
        result["roofline"] = roof

    gpu_outs = None
    if not args.no_cpu_baseline:
        gpu_outs = {"default": {"y": rt.to_numpy(yt), "lse": rt.to_numpy(caches[2]).reshape(B, H, T),
                                "dqkv": None if fwd_only else rt.to_numpy(dqkv)}}
        if lse_out is not None:
            gpu_outs["lse_only"] = lse_out
    for t in (dyt, mask, yt, dqkv, caches[0], caches[2], caches[3]):
        rt.free(t)
    rt.sync()

    if lse_res is not None:
        lse_res["pct_fp32_mfma_peak"] = round(100.0 * lse_res["tflops"] / peak, 2)
        result["lse_only"] = lse_res
    # The other workloads, in child processes, when this is the default
    # (driver) run: C2 with the CPU leg.
    if args.config == "c2" and not args.no_cpu_baseline and not args.no_other_configs:
        result["other_configs"] = other_configs(args)
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline (oracle over OpenBLAS) ...")
        cb = cpu_baseline(cfg, x, dy, args.cpu_budget_s, gpu_outs)
        errs = cb.pop("gpu_max_abs_err")
        cb["gpu_max_abs_err"] = errs.get("default")
        if lse_res is not None:
            lse_res["gpu_max_abs_err"] = errs.get("lse_only")
        result["cpu_baseline"] = {k: (round(v, 5) if isinstance(v, float) else v) for k, v in cb.items()}
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


def other_configs(args):
    """The benchmark's other workloads, each measured by this script in a
    child process (no CPU leg there): C5, C1 (cold forward), the C4 decode
    attention, C4 greedy generation (graph loop) and the C3 training step.
    They ride in the default run's one JSON line so that every config has a
    driver-measured figure.  Children start after the parent's GPU work is
    done and its buffers are freed."""
    runs = {
        "c5": ["--config", "c5", "--steps", "30", "--warmup", "5", "--reps", "3", "--no-kernel-pass"],
        "c1": ["--config", "c1", "--steps", "50", "--warmup", "5", "--reps", "3", "--no-kernel-pass"],
        "c4_decode_attention": ["--workload", "decode"],
        "c4_generation": ["--workload", "c4", "--c4-loops", "graph"],
        "c3_training_step": ["--workload", "gpt2", "--steps", "5", "--warmup", "2"],
    }
    keep = ("workload", "metric", "value", "unit", "ms_per_step", "tflops", "pct_fp32_mfma_peak", "pct_hbm_peak",
            "tokens_per_s", "same_tokens",
            "us_per_step", "roofline", "lse_only", "kernel_ms", "forward", "kv_cache_graph", "config", "note")
    out = {}
    for name, extra in runs.items():
        cmd = [sys.executable, os.path.abspath(__file__), "--no-cpu-baseline"] + extra
        log(f"[bench] other config {name}: {' '.join(extra)}")
        t0 = time.perf_counter()
        try:
            r = subprocess.run(cmd, capture_output=True, text=True, timeout=args.other_timeout_s)
        except subprocess.TimeoutExpired:
            out[name] = {"error": f"timed out after {args.other_timeout_s} s"}
            continue
        lines = [ln for ln in r.stdout.splitlines() if ln.startswith("{")]
        if r.returncode != 0 or not lines:
            out[name] = {"error": f"exit {r.returncode}", "stderr_tail": r.stderr[-400:]}
            continue
        d = json.loads(lines[-1])
        o = {k: d[k] for k in keep if k in d}
        if "lse_only" in o:
            o["lse_only"] = {k: o["lse_only"][k] for k in ("ms_per_step", "tflops", "pct_fp32_mfma_peak")
                             if k in o["lse_only"]}
        o["wall_s"] = round(time.perf_counter() - t0, 1)
        o["command"] = "bench.py --no-cpu-baseline " + " ".join(extra)
        out[name] = o
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", choices=sorted(CONFIGS), default="c2")
    ap.add_argument("--workload", choices=["attention", "copy", "decode", "gpt2", "c4"], default="attention",
                    help="copy: HBM copy of known size, to calibrate rocprof byte counters; "
                         "decode: the C4 KV-cache decode step; gpt2: the C3 GPT-2 124M training step; "
                         "c4: C4 greedy generation with GPT-2 124M")
    ap.add_argument("--decode-layers", type=int, default=12,
                    help="decode workload: layers whose caches each position runs through (GPT-2 small: 12)")
    ap.add_argument("--c4-loops", default="eager,graph,window",
                    help="c4 workload: the loops to time (comma list of eager, graph, window)")
    ap.add_argument("--reps", type=int, default=10,
                    help="attention: repetitions of the K-step timing after the headline (median/min)")
    ap.add_argument("--prewarm-ms", type=float, default=300.0,
                    help="attention: untimed steps for this long (wall ms) before the W warm-up steps")
    ap.add_argument("--no-kernel-pass", action="store_true",
                    help="attention: skip the per-kernel event pass (e.g. under a kernel trace of the headline)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="attention C2: skip the other workloads measured in child processes")
    ap.add_argument("--other-timeout-s", type=float, default=240.0)
    ap.add_argument("--cpu-budget-s", type=float, default=20.0)
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only. Every (b, h) pair of causal attention is independent, "
              "so the path shards over batch or heads with no exchange. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if args.workload == "decode":
        decode_bench(args)
        return
    if args.workload == "gpt2":
        gpt2_bench(args)
        return
    if args.workload == "c4":
        c4_bench(args)
        return
    if args.workload == "copy":
        copy_calibration(args)
        return

    attention_bench(args)


if __name__ == "__main__":
    main()
