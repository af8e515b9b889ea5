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

Full tensors would be megabytes, so each output is stored as its float64 sum,
sum of squares, maximum magnitude, and values at fixed sampled positions (and,
for y and dx, the sum and sum of squares of every row).  Run from the
repository root: python tests/golden/make_golden.py (about a minute on 8 cores).
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
          eps=1e-5, theta=1e5, B=4, T=512, seed=1)
BLOCK_KEYS = ["input_layernorm", "q_proj", "k_proj", "v_proj", "o_proj",
              "post_attention_layernorm", "gate_proj", "up_proj", "down_proj"]
N_SAMPLES = 64


def block_shapes(c):
    d, I, H, Hk, D = c["hidden"], c["inter"], c["heads"], c["kv_heads"], c["head_dim"]
    return {"input_layernorm": (d,), "q_proj": (H * D, d), "k_proj": (Hk * D, d),
            "v_proj": (Hk * D, d), "o_proj": (d, H * D), "post_attention_layernorm": (d,),
            "gate_proj": (I, d), "up_proj": (I, d), "down_proj": (d, I)}


def c1_inputs():
    """Weights (BLOCK_KEYS order, all ~N(0, 0.02)), x, dy, from RandomState(seed)."""
    c = C1
    r = np.random.RandomState(c["seed"])
    w = {k: 0.02 * r.standard_normal(s) for k, s in block_shapes(c).items()}
    x = r.standard_normal((c["B"], c["T"], c["hidden"]))
    dy = r.standard_normal((c["B"], c["T"], c["hidden"]))
    return w, x, dy


def c2_inputs():
    """Parameters in collect_parameters order (embedding, per layer BLOCK_KEYS,
    final norm; projections and embedding ~N(0, 0.02), norms 1), then ids,
    targets and the loss mask, from RandomState(seed)."""
    c = C2
    r = np.random.RandomState(c["seed"])
    params = [0.02 * r.standard_normal((c["vocab"], c["hidden"]))]
    shapes = block_shapes(c)
    for _ in range(c["layers"]):
        for k in BLOCK_KEYS:
            params.append(np.ones(shapes[k]) if k.endswith("layernorm")
                          else 0.02 * r.standard_normal(shapes[k]))
    params.append(np.ones(c["hidden"]))
    B, T = c["B"], c["T"]
    row = r.randint(0, c["vocab"], size=(B, T + 1))
    mask = np.ones((B, T))
    for b in range(B):
        mask[b, : int(math.floor(r.uniform(0.2, 0.6) * T))] = 0.0
    return params, row[:, :T].copy(), row[:, 1:].copy(), mask


def rope_freqs(D, theta):
    # theta^(-2i/D) in float32, as the reference's kernel computes it
    i = np.arange(D // 2, dtype=np.float32)
    return np.power(np.float32(theta), -(np.float32(2.0) * i) / np.float32(D)).astype(np.float32)


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
    freqs = rope_freqs(D, c["theta"])
    h1 = F.rms_norm(x, (d,), w["input_layernorm"], eps=c["eps"])
    q = rope((h1 @ w["q_proj"].T).view(B, T, H, D), freqs, T)
    k = rope((h1 @ w["k_proj"].T).view(B, T, Hk, D), freqs, T)
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


def make_c2():
    c = C2
    params, ids, tg, mask = c2_inputs()
    tp = [torch.tensor(p, requires_grad=True) for p in params]
    emb = tp[0]
    h = emb[torch.from_numpy(ids)]
    for layer in range(c["layers"]):
        w = dict(zip(BLOCK_KEYS, tp[1 + 9 * layer: 1 + 9 * (layer + 1)]))
        h = torch.utils.checkpoint.checkpoint(block, c, w, h, use_reentrant=False)
    h = F.rms_norm(h, (c["hidden"],), tp[-1], eps=c["eps"])
    logits = h.reshape(-1, c["hidden"]) @ emb.T
    per = F.cross_entropy(logits, torch.from_numpy(tg.reshape(-1)), reduction="none")
    m = torch.tensor(mask.reshape(-1))
    loss = (per * m).sum() / m.sum()
    loss.backward()
    out = {"loss": loss.item(), "mask_sum": mask.sum()}
    names = ["embed"] + [f"l{i}.{k}" for i in range(c["layers"]) for k in BLOCK_KEYS] + ["norm"]
    for i in [0, 1, 2, 3, 4, 5, 6, 7, 8, 9, len(names) - 2, len(names) - 1]:
        summarise("g." + names[i], tp[i].grad.numpy(), out)
    np.savez(os.path.join(HERE, "c2_model.npz"), **out)


if __name__ == "__main__":
    torch.set_default_dtype(torch.float64)
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    which = sys.argv[1:] or ["c1", "c2"]
    if "c1" in which:
        make_c1()
    if "c2" in which:
        make_c2()
