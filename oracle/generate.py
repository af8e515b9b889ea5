"""CPU restatement of the ctd_generate loop -- TEST INFRASTRUCTURE ONLY.

Follows the reference's tools/ctd_generate/main.cpp:52-192: request defaults,
the empty-prompt and prompt-too-long replies, prefill then one token per step,
budget forcing of think_close_ids, the eos / max_seq_len / max_tokens stop
reasons and the reply lines (nlohmann::json dump: sorted keys, compact).  The
model is a callable from the token list so far to the last position's logits.
Only tests import this module.
"""
from __future__ import annotations

import json

from . import sampling as S


def _line(obj):
    return json.dumps(obj, sort_keys=True, separators=(",", ":"))


def generate(last_logits, req: dict):
    """Reply lines for request `req`; last_logits(tokens) -> logits of the last token."""
    ids = list(req["input_ids"])
    max_new = int(req.get("max_new_tokens", 64))
    max_seq = int(req.get("max_seq_len", 2048))
    temperature = float(req.get("temperature", 1.0))
    top_k = int(req.get("top_k", 0))
    top_p = float(req.get("top_p", 0.0))
    rng = S.MT19937_64(int(req.get("seed", 0)))
    eos = set(req.get("eos_ids", []))
    budget = int(req.get("thinking_token_budget", 0))
    t_open = list(req.get("think_open_ids", []))
    t_close = list(req.get("think_close_ids", []))
    active = budget > 0 and t_open and t_close
    if not ids:
        return [_line({"done": True, "reason": "empty_prompt"})]
    if len(ids) >= max_seq:
        return [_line({"done": True, "reason": "max_seq_len"})]
    out = []
    seq = list(ids)
    cur_len = len(ids)
    logits = last_logits(seq)
    window, queue = [], []
    in_think, count = False, 0
    cap = max(len(t_open), len(t_close)) if active else 0
    generated, reason = 0, "max_tokens"
    while generated < max_new:
        if active and queue:
            tok = queue.pop(0)
        else:
            tok = S.sample_row(logits, rng, temperature, top_k, top_p)
        out.append(_line({"token": tok}))
        generated += 1
        if active:
            window.append(tok)
            if len(window) > cap:
                window.pop(0)
            if window[-len(t_open):] == t_open and len(window) >= len(t_open):
                in_think, count = True, 0
            elif window[-len(t_close):] == t_close and len(window) >= len(t_close):
                in_think = False
            elif in_think:
                count += 1
            if in_think and not queue and count >= budget:
                queue = list(t_close)
        if tok in eos:
            reason = "eos"
            break
        if cur_len + 1 > max_seq:
            reason = "max_seq_len"
            break
        seq.append(tok)
        cur_len += 1
        logits = last_logits(seq)
    out.append(_line({"done": True, "generated_tokens": generated, "reason": reason}))
    return out
