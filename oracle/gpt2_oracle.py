"""TEST INFRASTRUCTURE -- gpt.c's GPT-2 training step composed from the CPU
oracle's kernels.  Only tests/ and bench.py's cpu_baseline leg may use it.

The composition follows gpt.c's model code call for call:
  forward   src/transformer.c:69-111 (wte + wpe via saxpy per sequence,
            blocks, ln_f, lm_head tied to wte), src/block.c:54-90,
            src/self_attention.c:47-64, src/mlp.c:46-57;
  backward  src/transformer.c:113-158 (lm_head gradient re-created, added
            into wte's after the embedding backwards), src/block.c:92-135;
  loss      src/loss.c:33-108 with upstream gradient ones(B, T)
            (train_gpt.c:508-510);
  step      src/optim.c:72-108 (AdamW over parameters() in order).
Parameters are float32 numpy arrays in gpt.c's parameters() order
(src/transformer.c:230-262): wte, wpe, then per layer ln1.W, ln1.b,
qkv.W, qkv.b, attn.c_proj.W, attn.c_proj.b, ln2.W, ln2.b, c_fc.W, c_fc.b,
mlp.c_proj.W, mlp.c_proj.b, and finally ln_f.W, ln_f.b.
"""
import numpy as np

from oracle import Ops

PER_LAYER = ["ln1.W", "ln1.b", "qkv.W", "qkv.b", "attn_proj.W", "attn_proj.b",
             "ln2.W", "ln2.b", "fc.W", "fc.b", "mlp_proj.W", "mlp_proj.b"]


def param_shapes(V, block, L, C):
    """(name, shape) of every parameter in gpt.c's parameters() order."""
    out = [("wte", (V, C)), ("wpe", (block, C))]
    shp = {"ln1.W": (C,), "ln1.b": (C,), "qkv.W": (3 * C, C), "qkv.b": (3 * C,),
           "attn_proj.W": (C, C), "attn_proj.b": (C,), "ln2.W": (C,), "ln2.b": (C,),
           "fc.W": (4 * C, C), "fc.b": (4 * C,), "mlp_proj.W": (C, 4 * C), "mlp_proj.b": (C,)}
    for i in range(L):
        out += [(f"h{i}.{n}", shp[n]) for n in PER_LAYER]
    out += [("ln_f.W", (C,)), ("ln_f.b", (C,))]
    return out


class GPT2Oracle:
    def __init__(self, oracle, params, n_layers, n_heads):
        """params: list of float32 arrays in parameters() order (copied)."""
        self.o = oracle
        self.ops = Ops(oracle)
        self.p = [np.array(a, dtype=np.float32, copy=True) for a in params]
        self.L, self.H = n_layers, n_heads
        self.m = self.v = None
        self.t = 0

    def _lp(self, i):
        base = 2 + 12 * i
        return dict(zip(PER_LAYER, self.p[base:base + 12]))

    def forward(self, ids):
        ops, B, T = self.ops, ids.shape[0], ids.shape[1]
        wte, wpe = self.p[0], self.p[1]
        self.ids = ids.astype(np.float32)
        self.pos = np.arange(T, dtype=np.float32)[None, :]
        x = ops.embedding_forward(wte, self.ids)
        x = x + ops.embedding_forward(wpe, self.pos)  # saxpy(1, pos, tok[b])
        self.cache = []
        for i in range(self.L):
            lp = self._lp(i)
            c = {"x": x}
            h, c["m1"], c["r1"] = ops.layer_norm_forward(x, lp["ln1.W"], lp["ln1.b"])
            c["h"] = h
            qkv = ops.linear_forward(lp["qkv.W"], lp["qkv.b"], h)
            c["qkv"] = qkv
            a, q, k, v, att = self.o.forward(qkv, self.H)
            c["att"] = (q, k, v, att)
            c["a"] = a
            x1 = ops.linear_forward(lp["attn_proj.W"], lp["attn_proj.b"], a) + x
            c["x1"] = x1
            h2, c["m2"], c["r2"] = ops.layer_norm_forward(x1, lp["ln2.W"], lp["ln2.b"])
            c["h2"] = h2
            f = ops.linear_forward(lp["fc.W"], lp["fc.b"], h2)
            c["f"] = f
            gl = ops.gelu_forward(f)
            c["g"] = gl
            x = ops.linear_forward(lp["mlp_proj.W"], lp["mlp_proj.b"], gl) + x1
            self.cache.append(c)
        self.xf = x
        self.hf, self.mf, self.rf = ops.layer_norm_forward(x, self.p[-2], self.p[-1])
        return ops.linear_forward(wte, None, self.hf)

    def loss(self, logits, targets):
        self.lsm, loss = self.ops.cross_entropy_forward(logits, targets.astype(np.float32))
        self.targets = targets.astype(np.float32)
        return loss

    def backward(self):
        """Gradients (list in parameters() order) of the mean loss."""
        ops = self.ops
        B, T = self.ids.shape
        grads = [np.zeros_like(a) for a in self.p]
        dlogits = ops.cross_entropy_backward(np.ones((B, T), np.float32), self.lsm, self.targets)
        d_lm = np.zeros_like(self.p[0])
        dx = ops.linear_backward(dlogits, self.hf, self.p[0], d_lm, None)
        dxf = np.zeros_like(self.xf)
        ops.layer_norm_backward(dx, self.xf, self.mf, self.rf, self.p[-2], grads[-2], grads[-1], dxf)
        g = dxf
        for i in reversed(range(self.L)):
            lp, c = self._lp(i), self.cache[i]
            base = 2 + 12 * i
            gi = dict(zip(PER_LAYER, grads[base:base + 12]))
            d = ops.linear_backward(g, c["g"], lp["mlp_proj.W"], gi["mlp_proj.W"], gi["mlp_proj.b"])
            d = ops.gelu_backward(d, c["f"])
            d = ops.linear_backward(d, c["h2"], lp["fc.W"], gi["fc.W"], gi["fc.b"])
            d2 = np.zeros_like(d)
            ops.layer_norm_backward(d, c["x1"], c["m2"], c["r2"], lp["ln2.W"], gi["ln2.W"], gi["ln2.b"], d2)
            d2 = g + d2  # saxpy(1, global_grad, out)
            d = ops.linear_backward(d2, c["a"], lp["attn_proj.W"], gi["attn_proj.W"], gi["attn_proj.b"])
            q, k, v, att = c["att"]
            d = self.o.backward(d, self.H, q, k, v, att)
            d = ops.linear_backward(d, c["h"], lp["qkv.W"], gi["qkv.W"], gi["qkv.b"])
            d3 = np.zeros_like(d)
            ops.layer_norm_backward(d, c["x"], c["m1"], c["r1"], lp["ln1.W"], gi["ln1.W"], gi["ln1.b"], d3)
            g = d2 + d3  # saxpy(1, gg2, out)
        ops.embedding_backward(g, self.pos, grads[1])
        ops.embedding_backward(g, self.ids, grads[0])
        grads[0] += d_lm  # saxpy(1, lm_head.dW, wte.dW)
        self.grads = grads
        return grads

    def step(self, lr=3e-4, beta1=0.9, beta2=0.99, weight_decay=0.0, eps=1e-8):
        """AdamW with train_gpt.c's defaults (train_gpt.c:93-97)."""
        if self.m is None:
            self.m = [np.zeros_like(a) for a in self.p]
            self.v = [np.zeros_like(a) for a in self.p]
        self.t += 1
        for p, g, m, v in zip(self.p, self.grads, self.m, self.v):
            self.ops.adamw(p, g, m, v, lr, beta1, beta2, weight_decay, eps, self.t)
