"""CPU checks of the training driver's host logic (include/ctd/train.h) against
oracle/driver.py, and of oracle/driver.py against closed forms.

The driver mirrors tools/ctd_train/main.cpp: config, the int32-token /
int8-mask data format, batch assembly, warmup + cosine LR, loss.jsonl records.
Nothing here touches the GPU.
"""
import json
import math
import os

import numpy as np
import pytest

from emberlm_amd import trainer as TR
from oracle import driver as OD

F32 = np.float32


# ------------------------------------------------------- LR schedule (oracle pins)
@pytest.mark.parametrize("warmup,total,lr,ratio", [(100, 2800, 3e-4, 0.1), (10, 50, 1e-3, 0.0),
                                                   (0, 20, 2e-4, 0.5)])
def test_lr_oracle_closed_forms(warmup, total, lr, ratio):
    f = lambda s: float(OD.lr_at_step(s, warmup, total, lr, ratio))  # noqa: E731
    lr32, lo = float(F32(lr)), float(F32(F32(lr) * F32(ratio)))
    if warmup > 0:
        assert f(0) == 0.0
        assert math.isclose(f(warmup // 2), lr32 * (warmup // 2) / warmup, rel_tol=1e-6)
        assert all(f(s) < f(s + 1) for s in range(warmup))  # linear ramp up
    assert math.isclose(f(warmup), lr32, rel_tol=1e-6)       # cos(0) = 1
    assert math.isclose(f(total), lo, rel_tol=1e-6, abs_tol=1e-12)  # cos(pi) = -1
    assert math.isclose(f(total + 37), lo, rel_tol=1e-6, abs_tol=1e-12)  # clamped past the end
    if (total - warmup) % 2 == 0:                            # cos(pi/2) = 0: midpoint
        assert math.isclose(f(warmup + (total - warmup) // 2), (lr32 + lo) / 2, rel_tol=1e-5)
    assert all(f(s) >= f(s + 1) for s in range(warmup, total))  # cosine decays monotonically


@pytest.mark.parametrize("warmup,total,lr,ratio", [(100, 2800, 3e-4, 0.1), (10, 50, 1e-3, 0.0),
                                                   (0, 20, 2e-4, 0.5), (5, 5, 1e-4, 0.1)])
def test_lr_schedule_matches_oracle(warmup, total, lr, ratio):
    # Both evaluate the formula in float32; their cos may differ by one ulp
    # (glibc cosf vs numpy's float32 cos), which 1 + cos can magnify ~4x.
    for s in list(range(0, min(total, 200) + 3)) + [total - 1, total, total + 10]:
        got = TR.lr_at_step(s, warmup, total, lr, ratio)
        ref = float(OD.lr_at_step(s, warmup, total, lr, ratio))
        assert math.isclose(got, ref, rel_tol=1e-6, abs_tol=1e-12), (s, got, ref)


# -------------------------------------------------------------- data format
def write_split(d, name, tokens, masks):
    np.asarray(tokens, np.int32).tofile(os.path.join(d, f"{name}.bin"))
    np.asarray(masks, np.int8).tofile(os.path.join(d, f"{name}_mask.bin"))
    return os.path.join(d, f"{name}.bin"), os.path.join(d, f"{name}_mask.bin")


def test_host_batch_matches_oracle(tmp_path):
    rng = np.random.default_rng(0)
    seq_len, n = 17, 9
    tokens = rng.integers(0, 49152, (n, seq_len)).astype(np.int32)
    masks = (rng.random((n, seq_len)) < 0.6).astype(np.int8)
    tp, mp = write_split(tmp_path, "train", tokens, masks)
    docs = [3, 0, 8, 3]
    ids, tgt, mask, sm, nd = TR.host_batch(tp, mp, seq_len, docs)
    r_ids, r_tgt, r_mask, r_sm = OD.make_host_batch(tokens, masks, docs, seq_len)
    assert nd == n
    assert np.array_equal(ids, r_ids) and np.array_equal(tgt, r_tgt)
    assert np.array_equal(mask, r_mask) and sm == r_sm
    # the shift: target t is input t+1, and the mask follows the target token
    assert np.array_equal(ids[:, 1:], tgt[:, :-1])
    assert np.array_equal(mask[1], masks[0, 1:])


def test_data_format_errors(tmp_path):
    seq_len = 8
    tp, mp = write_split(tmp_path, "a", np.zeros(2 * seq_len + 1), np.zeros(2 * seq_len))
    with pytest.raises(TR.CtdError, match="not whole documents of 8"):
        TR.host_batch(tp, mp, seq_len, [])
    tp, mp = write_split(tmp_path, "b", np.zeros(2 * seq_len), np.zeros(2 * seq_len - 1))
    with pytest.raises(TR.CtdError, match="15 mask values for 16 tokens"):
        TR.host_batch(tp, mp, seq_len, [])
    tp, mp = write_split(tmp_path, "c", np.zeros(2 * seq_len), np.zeros(2 * seq_len))
    with pytest.raises(TR.CtdError, match="out of range"):
        TR.host_batch(tp, mp, seq_len, [2])
    with pytest.raises(TR.CtdError, match="cannot stat"):
        TR.host_batch(os.path.join(tmp_path, "missing.bin"), mp, seq_len, [])
    # a token file that is not a whole number of int32 values
    open(os.path.join(tmp_path, "odd.bin"), "wb").write(b"\0" * 33)
    with pytest.raises(TR.CtdError, match="not a whole number of 4-byte values"):
        TR.host_batch(os.path.join(tmp_path, "odd.bin"), mp, seq_len, [])


# ------------------------------------------------------------ loss.jsonl records
@pytest.mark.parametrize("step,loss,lr,gn,tps,wall", [
    (1, 10.3406, 3e-4, 0.75, 1234.5, 12.0),
    (250, 2.0, 1.5e-5, 1e-7, 98765.4321, 3600.125),
    (7, 0.1, 0.0, 3.0, 0.0, 0.0),
])
def test_train_event_matches_reference_format(step, loss, lr, gn, tps, wall):
    got = TR.event_json(step, loss, lr, gn, tps, wall)
    assert got == OD.train_event(step, loss, lr, gn, tps, wall)
    rec = json.loads(got)
    assert list(rec) == sorted(rec) == ["grad_norm", "loss", "lr", "phase", "step",
                                        "tokens_per_sec", "wall_s"]
    assert rec["phase"] == "train" and rec["step"] == step and rec["loss"] == float(F32(loss))


def test_val_event_matches_reference_format():
    got = TR.event_json(100, 1.875, wall_s=42.5, val=True)
    assert got == OD.val_event(100, 1.875, 42.5) == '{"loss":1.875,"phase":"val","step":100,"wall_s":42.5}'


# ------------------------------------------------------------------- config
@pytest.mark.parametrize("body,msg", [
    ('{"data_dir": "x"}', "init_weights"),
    ('{"init_weights": "w.safetensors"}', "data_dir"),
    ('{"init_weights": "w", "data_dir": "d", "seq_len": "long"}', "seq_len must be a number"),
    ('{"init_weights": "w", "data_dir": "d", "offload_optimizer": 1}', "true/false"),
    ('{"init_weights": "w", "data_dir": "d", "grad_accum_steps": 0}', "grad_accum_steps"),
    ('{"init_weights": "w", "data_dir": "d", "model": {"hidden_size": 64}}', "model needs"),
    ('{"init_weights": "w", "data_dir": "d",', "bad JSON"),
])
def test_config_errors_before_any_device_work(tmp_path, body, msg):
    cfg = tmp_path / "config.json"
    cfg.write_text(body)
    with pytest.raises(TR.CtdError, match=msg):
        TR.train_run(cfg)


def test_cli_usage_and_config_error(tmp_path):
    import subprocess
    exe = os.path.join(os.path.dirname(TR.LIB_PATH), "ctd_train")
    r = subprocess.run([exe], capture_output=True, text=True)
    assert r.returncode == 2 and "usage:" in r.stderr and "--config" in r.stderr
    cfg = tmp_path / "config.json"
    cfg.write_text('{"data_dir": "x"}')
    r = subprocess.run([exe, "--config", str(cfg)], capture_output=True, text=True)
    assert r.returncode == 1 and "ctd_train: error:" in r.stderr and "init_weights" in r.stderr
