"""gpt.c's own programs, unmodified, on this library.

oracle/Makefile's `apps` target compiles gpt.c's train_gpt.c and infer_gpt.c
from /root/reference against include/ and links them to libgptc_amd.so
(oracle/_ref/{train,infer}_gpt_amd).  That they compile and link at all shows
the headers and exports are a source-level drop-in for gpt.c's; the GPU tests
below run them end to end and check what they print and save against the CPU
oracle:
  * train_gpt  (train_gpt.c:350-577): per-step training losses, the
    validation loss and the checkpoint it saves after validation, against
    GPT2Oracle's steps over the same DataLoader windows;
  * infer_gpt  (infer_gpt.c:280-430): every sampled token, against the
    softmax of the oracle's logits for the same window row and infer_gpt.c's
    own sampler (xorshift coin and float32 running sum, infer_gpt.c:255-278,
    restated below).
Where the programs are not built (no /root/reference when they were built)
the tests skip.
"""
import os
import re
import subprocess

import numpy as np
import pytest

from file_formats import read_checkpoint, write_checkpoint, write_tokenizer, write_tokens
from gpt2_oracle import GPT2Oracle, param_shapes

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
APPS = os.path.join(ROOT, "oracle", "_ref")
TRAIN = os.path.join(APPS, "train_gpt_amd")
INFER = os.path.join(APPS, "infer_gpt_amd")
EOT = 50256


def need(app):
    if not os.path.exists(app):
        pytest.skip(f"{os.path.basename(app)} is not built (make -C oracle apps, where gpt.c's sources exist)")


def run(args, timeout=300):
    r = subprocess.run(args, capture_output=True, text=True, timeout=timeout)
    print(r.stdout[-3000:])
    print(r.stderr[-3000:])
    return r


def init_params(V, block, L, C, seed, std):
    rng = np.random.default_rng(seed)
    out = []
    for name, shp in param_shapes(V, block, L, C):
        if name.endswith(("ln1.W", "ln2.W")) or name == "ln_f.W":
            out.append((1 + 0.05 * rng.standard_normal(shp)).astype(np.float32))
        elif len(shp) == 1:
            out.append((0.05 * rng.standard_normal(shp)).astype(np.float32))
        else:
            out.append((rng.standard_normal(shp) * std).astype(np.float32))
    return out


def test_programs_start():
    for app in (TRAIN, INFER):
        need(app)
        r = run([app, "--help"], timeout=60)
        assert r.returncode == 0 and "Usage:" in r.stdout


def test_cpu_device_is_refused_loudly(tmp_path):
    """--device=cpu reaches the library's CPU dispatch, which is fatal: the
    library has no CPU fallback."""
    need(TRAIN)
    block, V, L, H, C = 16, 37, 1, 2, 16
    ckpt = tmp_path / "model.bin"
    write_checkpoint(ckpt, (block, V, L, H, C), init_params(V, block, L, C, 0, 0.02), 0)
    data = tmp_path / "train.bin"
    write_tokens(data, np.arange(100) % V)
    r = run([TRAIN, f"--train-data={data}", f"--load-checkpoint={ckpt}", "--max-epochs=1", "--batch-size=2",
             "--block-size=8", f"--log-dir={tmp_path / 'logs'}", "--device=cpu"], timeout=60)
    assert r.returncode != 0
    assert "GPU back end only" in r.stderr


@pytest.mark.gpu
def test_train_gpt_matches_oracle(oracle, tmp_path):
    block, V, L, H, C = 64, 211, 2, 4, 96
    B, T, vB, vT = 4, 48, 2, 64
    lr, wd, eps = 1e-3, 0.1, 1e-4  # eps: see the AdamW note in test_gpt2_gpu.py
    params = init_params(V, block, L, C, 3, 0.05)
    ckpt = tmp_path / "model.bin"
    write_checkpoint(ckpt, (block, V, L, H, C), params, 5)
    rng = np.random.default_rng(4)
    n_steps, n_val = 4, 3
    train = rng.integers(0, V, n_steps * (B * T + 1))
    val = rng.integers(0, V, n_val * (vB * vT + 1))
    write_tokens(tmp_path / "train.bin", train)
    write_tokens(tmp_path / "val.bin", val)
    logs = tmp_path / "logs"
    r = run([TRAIN, f"--train-data={tmp_path / 'train.bin'}", f"--val-data={tmp_path / 'val.bin'}",
             "--max-epochs=1", f"--batch-size={B}", f"--block-size={T}", f"--log-dir={logs}", "--output=ckpt",
             f"--load-checkpoint={ckpt}", "--device=cuda", f"--val-batch-size={vB}", f"--val-block-size={vT}",
             f"--lr={lr}", f"--weight-decay={wd}", f"--eps={eps}"])
    assert r.returncode == 0
    losses = [float(m) for m in re.findall(r"train loss: ([-0-9.naif]+)", r.stdout)]
    val_loss = [float(m) for m in re.findall(r"val loss: ([-0-9.naif]+)", r.stdout)]
    assert len(losses) == n_steps and len(val_loss) == 1

    # The same run on the oracle: DataLoader windows of B*T+1 ids advancing
    # by B*T (src/dataloader.c), inputs ids[:-1], targets ids[1:].
    g = GPT2Oracle(oracle, params, L, H)
    for s in range(n_steps):
        w = train[s * B * T:(s + 1) * B * T + 1]
        logits = g.forward(w[:-1].reshape(B, T))
        ref = float(g.loss(logits, w[1:].reshape(B, T)))
        g.backward()
        g.step(lr=lr, weight_decay=wd, eps=eps)
        print(f"step {s + 1}: train_gpt {losses[s]:.6f} oracle {ref:.6f}")
        assert abs(losses[s] - ref) <= 1e-4 * max(1.0, abs(ref))
    vals = []
    for s in range(n_val):
        w = val[s * vB * vT:(s + 1) * vB * vT + 1]
        vals.append(float(g.loss(g.forward(w[:-1].reshape(vB, vT)), w[1:].reshape(vB, vT))))
    ref_val = float(np.mean(vals))
    print(f"val: train_gpt {val_loss[0]:.6f} oracle {ref_val:.6f}")
    assert abs(val_loss[0] - ref_val) <= 1e-4 * max(1.0, abs(ref_val))

    # The checkpoint saved after validation: gpt.c's header, the trained
    # parameters (steps = the loaded checkpoint's 5 + this run's 4).
    header, saved = read_checkpoint(logs / "ckpt.bin")
    assert header[1:8] == [block, V, L, H, C, header[6], 5 + n_steps]
    assert len(saved) == len(g.p)
    for (name, _), a, b in zip(param_shapes(V, block, L, C), saved, g.p):
        assert a.shape == b.shape, name
        tol = 1e-5 * max(1.0, float(np.abs(b).max()))
        err = float(np.abs(a.astype(np.float64) - b).max())
        assert err <= tol, f"{name}: {err:.3e} > {tol:.1e}"


def xorshift_coins(seed, n):
    """infer_gpt.c:255-264: xorshift* over a uint64 state, the top 24 bits
    of the 32-bit output as a float in [0, 1)."""
    state, mask, out = seed, (1 << 64) - 1, []
    for _ in range(n):
        state ^= state >> 12
        state = (state ^ (state << 25)) & mask
        state ^= state >> 27
        u32 = ((state * 0x2545F4914F6CDD1D) & mask) >> 32
        out.append(np.float32(u32 >> 8) / np.float32(16777216.0))
    return out


@pytest.mark.gpu
def test_infer_gpt_samples_match_oracle(oracle, tmp_path):
    block, V, L, H, C = 32, 50257, 1, 2, 64
    prompt, max_tokens, seed, temp = [11, 500, 7, 42000, 3], 40, 1234, 0.8
    params = init_params(V, block, L, C, 5, 0.3)
    ckpt = tmp_path / "model.bin"
    write_checkpoint(ckpt, (block, V, L, H, C), params, 0)
    tok = tmp_path / "tokenizer.bin"
    write_tokenizer(tok, [b"<%d>" % i for i in range(V)], EOT)
    r = run([INFER, f"--load-checkpoint={ckpt}", f"--tokenizer={tok}",
             "--prompt=[" + ",".join(map(str, prompt)) + "]", f"--max-tokens={max_tokens}",
             f"--temperature={temp}", f"--rand-seed={seed}", "--device=cuda"])
    assert r.returncode == 0
    text = r.stdout.split("Starting Inference")[1].split("Inference Time")[0]
    ids = [int(m) for m in re.findall(r"<(\d+)>", text)]
    total = len(prompt) + max_tokens
    assert len(ids) == total and ids[:len(prompt)] == prompt

    # infer_gpt.c's loop on the oracle, teacher-forced with the program's own
    # tokens: the window, the logits row, softmax(row / temperature), and
    # the token the coin picks from the cumulative sum (sample_mult).
    g = GPT2Oracle(oracle, params, L, H)
    X = np.full(-(-total // block) * block, EOT, np.int64)
    X[:total] = ids
    coins = xorshift_coins(seed, max_tokens)
    start = 0
    for n, i in enumerate(range(len(prompt), total)):
        start += 0 if i < block else 1
        window = X[start:start + block].copy()
        window[i - start:] = EOT  # not generated yet when token i was drawn
        logits = g.forward(window.reshape(1, block))
        row = logits[0, i - 1 if i < block else block - 1].astype(np.float32)
        p = softmax_f32(row * np.float32(1.0 / temp))
        cdf = np.cumsum(p, dtype=np.float32)  # sample_mult's float32 running sum
        t = ids[i]
        lo = float(cdf[t - 1]) if t > 0 else 0.0
        hi = float(cdf[t]) if t < V - 1 else 1.0
        assert lo - 1e-5 <= coins[n] < hi + 1e-5, f"token {i}: {t} with coin {coins[n]} outside [{lo}, {hi})"


def softmax_f32(row):
    """The softmax of a float32 row, rounded once to float32.  The
    normalising sum is taken in float64: a sequential float32 sum over 50257
    terms (the oracle's) is off by about 1e-5 relative, which moves the
    cumulative sum at 0.7 by as much as a whole interval; the library's
    tree-shaped sum is within a few ulp of the exact one."""
    e = np.exp(row.astype(np.float64) - float(row.max()))
    return (e / e.sum()).astype(np.float32)
