"""CPU restatement of the training driver's host logic -- TEST INFRASTRUCTURE ONLY.

Follows the reference's tools/ctd_train/main.cpp: the batch assembly of
make_batch (145-168), lr_at_step (176-188), and the order of one optimizer step
(346-376: micro-batch losses scaled by 1/accum and accumulated, clip_grad_norm_
over all parameters, AdamW with the step's learning rate), plus the loss.jsonl
records (378-411).  Only tests import this module.
"""
from __future__ import annotations

import json
import math

import numpy as np

from . import adamw as _adamw

F32 = np.float32


def lr_at_step(step, warmup_steps, total_steps, lr, min_lr_ratio):
    """Linear warmup, then cosine decay to lr*min_lr_ratio (main.cpp:176-188), in float32."""
    lr = F32(lr)
    if step < warmup_steps:
        t = F32(step) / F32(max(1, warmup_steps))
        return F32(lr * t)
    decay = max(1, total_steps - warmup_steps)
    s = min(step - warmup_steps, decay)
    t = F32(s) / F32(decay)
    cos_factor = F32(0.5) * (F32(1.0) + np.cos(F32(math.pi) * t, dtype=F32))
    min_lr = F32(lr * F32(min_lr_ratio))
    return F32(min_lr + (lr - min_lr) * cos_factor)


def make_host_batch(tokens, masks, docs, seq_len):
    """tokens int32 / masks int8, both [num_docs, seq_len] -> (ids, targets, mask, sum_mask).

    inputs are tokens[0:seq_len-1], targets tokens[1:seq_len], and the mask of a
    position is the target token's mask value (main.cpp:151-164); sum_mask is a
    float32 running sum in document order.
    """
    tokens = np.asarray(tokens).reshape(-1, seq_len)
    masks = np.asarray(masks).reshape(-1, seq_len)
    ids = np.stack([tokens[d, :-1] for d in docs]).astype(np.int64)
    tgt = np.stack([tokens[d, 1:] for d in docs]).astype(np.int64)
    mask = np.stack([masks[d, 1:] for d in docs]).astype(np.float32)
    s = F32(0.0)
    for m in mask.reshape(-1):
        s = F32(s + m)
    return ids, tgt, mask, float(s)


def clip_grad_norm(grads, max_norm, eps=1e-6):
    """(total_norm, scaled grads): grads *= max_norm / (norm + eps) when norm > max_norm
    (src/core/optim.cu:219-293), the norm taken in float64."""
    total = math.sqrt(sum(float(np.sum(np.asarray(g, np.float64) ** 2)) for g in grads))
    if total > max_norm:
        sc = max_norm / (total + eps)
        grads = [np.asarray(g, np.float64) * sc for g in grads]
    return total, grads


def adamw_step(params, grads, m, v, step, lr, decay, weight_decay, beta1=0.9, beta2=0.95,
               eps=1e-8):
    """One AdamW step over every parameter with a gradient; decay[i] selects the
    weight-decay group (bias corrections in float, optim.cu:142-143)."""
    bc1 = F32(1.0) - F32(beta1) ** F32(step)
    bc2 = F32(1.0) - F32(beta2) ** F32(step)
    out = []
    for i, (p, g) in enumerate(zip(params, grads)):
        wd = weight_decay if decay[i] else 0.0
        out.append(_adamw(p, g, m[i], v[i], F32(lr), F32(beta1), F32(beta2), F32(eps), F32(wd),
                          bc1, bc2))
    return out  # [(p, m, v)]


def train_event(step, loss, lr, grad_norm, tokens_per_sec, wall_s):
    """One loss.jsonl train record as the reference's JSON library writes it: float
    fields widened to double, keys sorted, compact separators."""
    return json.dumps({"step": int(step), "phase": "train", "loss": float(F32(loss)),
                       "lr": float(F32(lr)), "grad_norm": float(F32(grad_norm)),
                       "tokens_per_sec": float(tokens_per_sec), "wall_s": float(wall_s)},
                      sort_keys=True, separators=(",", ":"))


def val_event(step, loss, wall_s):
    return json.dumps({"step": int(step), "phase": "val", "loss": float(F32(loss)),
                       "wall_s": float(wall_s)}, sort_keys=True, separators=(",", ":"))
