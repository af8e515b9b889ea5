"""Writes the golden fixtures of this directory: expected outputs computed by an
independent float64 torch (CPU) composition of the reference's block and model
(include/ctd/nn/transformer_block.h:28-35, attention.h:100-143, mlp.h:16-21,
model.h:170-206, loss.cu:253-329 of the reference), for inputs that the tests
regenerate from numpy's legacy RandomState (its streams are frozen across numpy
versions), so the files hold only expected outputs:

- c1_block.npz: BASELINE config 0, one SmolLM2-135M-shaped decoder block
  (hidden 576, 9/3 heads of 64, MLP 1536, eps 1e-5, theta 1e5), B=1, T=256,
  every weight ~N(0, 0.02) (norm weights included), x and dy ~N(0, 1):
  y = block(x) and dx, dW = the backward of sum(y * dy).
- c2_model.npz: BASELINE config 1, the full SmolLM2-135M model (30 layers,
  vocab 49152, tied head), B=4, T=512, weights ~N(0, 0.02) with norm weights
  1, token ids uniform, each row's loss mask 0 on a prefix of 20-60%: the
  masked mean cross-entropy and its gradients.
- c3_model.npz: BASELINE config 2's Qwen3-0.6B shape (hidden 1024, 16/8 heads
  of 128 with per-head QK-RMSNorm, MLP 3072, vocab 151936, eps 1e-6, theta
  1e6) cut to 2 layers, at the config's B=4, T=1024 with the prefix loss mask.
- c4_model.npz: BASELINE config 3's LLaMA-3.2-1B shape (hidden 2048, 32/8
  heads of 64, MLP 8192, vocab 128256, eps 1e-5, theta 5e5 with llama3
  scaling: factor 32, low 1, high 4, original context 8192) cut to 2 layers,
  at T=2048 (positions up to 2047 cross all three llama3 bands) and B=2, with
  the all-ones mask the config implies.
- c5_model.npz: BASELINE config 4's Qwen3-1.7B shape (hidden 2048, 16/8 heads
  of 128 with per-head QK-RMSNorm, MLP 6144, vocab 151936, eps 1e-6, theta
  1e6) cut to 2 layers, at the config's T=4096 with B=1 and the prefix loss
  mask.

Full tensors would be megabytes, so each output is stored as its float64 sum,
sum of squares, maximum magnitude, and values at fixed sampled positions (and,
for y and dx, the sum and sum of squares of every row).  Run from the
repository root: python tests/golden/make_golden.py [c1 c2 c3 c4 c5] (c1 and c2
about a minute each on 8 cores, c3, c4 and c5 a few minutes and up to 30 GB of
memory).
"""
import math
import os
import sys

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))

C1 = dict(hidden=576, inter=1536, heads=9, kv_heads=3, head_dim=64, eps=1e-5, theta=1e5,
          B=1, T=256, seed=0)
C2 = dict(vocab=49152, hidden=576, inter=1536, layers=30, heads=9, kv_heads=3, head_dim=64,
          eps=1e-5, theta=1e5, B=4, T=512, seed=1, masked=True)
C3 = dict(vocab=151936, hidden=1024, inter=3072, layers=2, heads=16, kv_heads=8, head_dim=128,
          eps=1e-6, theta=1e6, qk_norm=True, B=4, T=1024, seed=2, masked=True)
C4 = dict(vocab=128256, hidden=2048, inter=8192, layers=2, heads=32, kv_heads=8, head_dim=64,
          eps=1e-5, theta=5e5, rope=(32.0, 1.0, 4.0, 8192), B=2, T=2048, seed=3, masked=False)
C5 = dict(vocab=151936, hidden=2048, inter=6144, layers=2, heads=16, kv_heads=8, head_dim=128,
          eps=1e-6, theta=1e6, qk_norm=True, B=1, T=4096, seed=4, masked=True)
BLOCK_KEYS = ["input_layernorm", "q_proj", "k_proj", "v_proj", "o_proj",
              "post_attention_layernorm", "gate_proj", "up_proj", "down_proj"]
# collect_parameters' order inside a layer when the model has QK-Norm
QK_BLOCK_KEYS = ["input_layernorm", "q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm",
                 "post_attention_layernorm", "gate_proj", "up_proj", "down_proj"]


N_SAMPLES = 64


def block_keys(c):
    return QK_BLOCK_KEYS if c.get("qk_norm") else BLOCK_KEYS


def block_shapes(c):
    d, I, H, Hk, D = c["hidden"], c["inter"], c["heads"], c["kv_heads"], c["head_dim"]
    return {"input_layernorm": (d,), "q_proj": (H * D, d), "k_proj": (Hk * D, d),
            "v_proj": (Hk * D, d), "o_proj": (d, H * D), "q_norm": (D,), "k_norm": (D,),
            "post_attention_layernorm": (d,), "gate_proj": (I, d), "up_proj": (I, d),
            "down_proj": (d, I)}


def c1_inputs():
    """Weights (BLOCK_KEYS order, all ~N(0, 0.02)), x, dy, from RandomState(seed)."""
    c = C1
    r = np.random.RandomState(c["seed"])
    sh = block_shapes(c)
    w = {k: 0.02 * r.standard_normal(sh[k]) for k in BLOCK_KEYS}
    x = r.standard_normal((c["B"], c["T"], c["hidden"]))
    dy = r.standard_normal((c["B"], c["T"], c["hidden"]))
    return w, x, dy


def model_inputs(c):
    """Parameters in collect_parameters order (embedding, per layer
    block_keys(c), final norm; projections and embedding ~N(0, 0.02), norms
    1), then ids, targets and the loss mask (a prefix of 20-60% of each row
    masked when c["masked"], else all ones), from RandomState(seed)."""
    r = np.random.RandomState(c["seed"])
    params = [0.02 * r.standard_normal((c["vocab"], c["hidden"]))]
    shapes = block_shapes(c)
    for _ in range(c["layers"]):
        for k in block_keys(c):
            params.append(np.ones(shapes[k]) if k.endswith("norm")
                          else 0.02 * r.standard_normal(shapes[k]))
    params.append(np.ones(c["hidden"]))
    B, T = c["B"], c["T"]
    row = r.randint(0, c["vocab"], size=(B, T + 1))
    mask = np.ones((B, T))
    if c["masked"]:
        for b in range(B):
            mask[b, : int(math.floor(r.uniform(0.2, 0.6) * T))] = 0.0
    return params, row[:, :T].copy(), row[:, 1:].copy(), mask


def c2_inputs():
    return model_inputs(C2)


def grad_names(c):
    """Fixture names of the parameters, in collect_parameters order."""
    return (["embed"] + [f"l{i}.{k}" for i in range(c["layers"]) for k in block_keys(c)]
            + ["norm"])


def summarised_grads(c):
    """Indices of the parameters whose gradients a fixture keeps: all of them,
    in collect_parameters order."""
    return list(range(len(grad_names(c))))


def rope_freqs(D, theta, factor=0.0, low_freq=1.0, high_freq=4.0, orig_max_pos=8192):
    """theta^(-2i/D) in float32, as the reference's kernel computes it; with
    factor > 1 the llama3 bands of rope.cu:37-46, written per band in float64:
    wavelength 2*pi/f above L/low_freq divides f by factor, below L/high_freq
    keeps f, and in between takes (1 - s)*f + s*f/factor with
    s = (wavelength - L/high_freq) / (L/low_freq - L/high_freq).  This weight is
    the reference's; HF's llama3 rule weights f/factor by 1 - s' with
    s' = (L/wavelength - low_freq)/(high_freq - low_freq) instead."""
    # float32 theta and exponent, the power in float64 rounded once to float32
    # (numpy's vectorised float32 power is off by an ulp at some i, which moves
    # angles near position 4095 by 1e-4 rad)
    expo = [float(np.float32(-(2.0 * i) / D)) for i in range(D // 2)]
    base = np.array([float(np.float32(theta)) ** e for e in expo]).astype(np.float32)
    if factor <= 1.0:
        return base
    out = np.empty(D // 2, dtype=np.float32)
    lo_wl, hi_wl = orig_max_pos / low_freq, orig_max_pos / high_freq
    for j, b in enumerate(base.astype(np.float64)):
        wl = 2.0 * math.pi / b
        if wl > lo_wl:
            f = b / factor
        elif wl > hi_wl:
            s = (wl - hi_wl) / (lo_wl - hi_wl)
            f = (1.0 - s) * b + s * (b / factor)
        else:
            f = b
        out[j] = np.float32(f)
    return out


def rope(z, freqs, T):
    # angle = float32(pos) * freq rounded to float32, then an accurate rotation
    ang = torch.from_numpy((np.arange(T, dtype=np.float32)[:, None] * freqs[None, :])
                           .astype(np.float32)).double()
    cos, sin = torch.cos(ang)[None, :, None, :], torch.sin(ang)[None, :, None, :]
    half = z.shape[-1] // 2
    a, b = z[..., :half], z[..., half:]
    return torch.cat([a * cos - b * sin, a * sin + b * cos], -1)


def block(c, w, x):
    B, T, d = x.shape
    H, Hk, D = c["heads"], c["kv_heads"], c["head_dim"]
    freqs = rope_freqs(D, c["theta"], *c.get("rope", ()))
    h1 = F.rms_norm(x, (d,), w["input_layernorm"], eps=c["eps"])
    q = (h1 @ w["q_proj"].T).view(B, T, H, D)
    k = (h1 @ w["k_proj"].T).view(B, T, Hk, D)
    if c.get("qk_norm"):  # per-head RMSNorm over D before RoPE (attention.h:115-118)
        q = F.rms_norm(q, (D,), w["q_norm"], eps=c["eps"])
        k = F.rms_norm(k, (D,), w["k_norm"], eps=c["eps"])
    q, k = rope(q, freqs, T), rope(k, freqs, T)
    v = (h1 @ w["v_proj"].T).view(B, T, Hk, D)
    g = H // Hk
    s = (q.transpose(1, 2) @ k.transpose(1, 2).repeat_interleave(g, 1).transpose(-1, -2))
    s = s / math.sqrt(D)
    s = s.masked_fill(torch.triu(torch.ones(T, T, dtype=torch.bool), 1), -math.inf)
    o = torch.softmax(s, -1) @ v.transpose(1, 2).repeat_interleave(g, 1)
    h = x + o.transpose(1, 2).reshape(B, T, H * D) @ w["o_proj"].T
    h2 = F.rms_norm(h, (d,), w["post_attention_layernorm"], eps=c["eps"])
    return h + (F.silu(h2 @ w["gate_proj"].T) * (h2 @ w["up_proj"].T)) @ w["down_proj"].T


def summarise(prefix, a, out, rows=False):
    a = np.asarray(a, dtype=np.float64)
    flat = a.reshape(-1)
    idx = np.random.RandomState(12345).randint(0, flat.size, size=N_SAMPLES)
    out[prefix + ".sum"] = flat.sum()
    out[prefix + ".sumsq"] = (flat * flat).sum()
    out[prefix + ".maxabs"] = np.abs(flat).max()
    out[prefix + ".idx"] = idx
    out[prefix + ".val"] = flat[idx]
    if rows:
        r2 = a.reshape(-1, a.shape[-1])
        out[prefix + ".row_sum"] = r2.sum(1)
        out[prefix + ".row_sumsq"] = (r2 * r2).sum(1)


def make_c1():
    w, x, dy = c1_inputs()
    tw = {k: torch.tensor(v, requires_grad=True) for k, v in w.items()}
    tx = torch.tensor(x, requires_grad=True)
    y = block(C1, tw, tx)
    (y * torch.tensor(dy)).sum().backward()
    out = {}
    summarise("y", y.detach().numpy(), out, rows=True)
    summarise("dx", tx.grad.numpy(), out, rows=True)
    for k in BLOCK_KEYS:
        summarise("d_" + k, tw[k].grad.numpy(), out)
    np.savez(os.path.join(HERE, "c1_block.npz"), **out)


def make_model(c, filename):
    params, ids, tg, mask = model_inputs(c)
    tp = [torch.tensor(p, requires_grad=True) for p in params]
    del params
    emb = tp[0]
    keys = block_keys(c)
    h = emb[torch.from_numpy(ids)]
    for layer in range(c["layers"]):
        w = dict(zip(keys, tp[1 + len(keys) * layer: 1 + len(keys) * (layer + 1)]))
        h = torch.utils.checkpoint.checkpoint(block, c, w, h, use_reentrant=False)
    h = F.rms_norm(h, (c["hidden"],), tp[-1], eps=c["eps"])
    logits = h.reshape(-1, c["hidden"]) @ emb.T
    per = F.cross_entropy(logits, torch.from_numpy(tg.reshape(-1)), reduction="none")
    del logits
    m = torch.tensor(mask.reshape(-1))
    loss = (per * m).sum() / m.sum()
    loss.backward()
    out = {"loss": loss.item(), "mask_sum": mask.sum()}
    names = grad_names(c)
    for i in summarised_grads(c):
        summarise("g." + names[i], tp[i].grad.numpy(), out)
    np.savez(os.path.join(HERE, filename), **out)


if __name__ == "__main__":
    torch.set_default_dtype(torch.float64)
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    which = sys.argv[1:] or ["c1", "c2", "c3", "c4", "c5"]
    if "c1" in which:
        make_c1()
    for name, c in (("c2", C2), ("c3", C3), ("c4", C4), ("c5", C5)):
        if name in which:
            make_model(c, f"{name}_model.npz")
