"""GPU checks of the ctd_train driver (include/ctd/train.h; reference
tools/ctd_train/main.cpp:346-431).

- Gradient accumulation: two micro-batches at scale 1/2 give the oracle's
  0.5 * (grad_1 + grad_2), per element within 1e-4 (the masked-CE tolerance).
- A whole run on a tiny Qwen3-shaped model (QK-Norm, offloaded AdamW,
  checkpointing) over a data split whose documents are all the same, so every
  sampled batch is known: its final weights and m/v must equal, bit for bit,
  the same steps driven one call at a time through the trainer API
  (accumulate x grad_accum_steps, clip, lr_at_step, AdamW, zero_grad).
- Resume: a run stopped at step 2 and resumed from its checkpoint ends with the
  same bits as the uninterrupted run, appends to loss.jsonl, and restores
  optimizer.step.
"""
import json
import os

import numpy as np
import pytest

import oracle as O
from tests.helpers import assert_close

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from emberlm_amd import trainer as TR  # noqa: E402
from tests.test_gpu_model import batch, oracle_cfg, shapes, tiny_cfg  # noqa: E402


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def shaped_params(tr, c):
    sh = shapes(c)
    out = []
    for i, name in enumerate(tr.names):
        p = tr.get_param(i)
        if name == "model.embed_tokens.weight":
            out.append(p.reshape(c.vocab_size, c.hidden_size))
        elif name == "model.norm.weight":
            out.append(p)
        else:
            out.append(p.reshape(sh[name.split(".")[-2]]))
    return out


def test_grad_accumulation_vs_oracle():
    c = tiny_cfg(qk_norm=True, D=64)
    tr = TR.Trainer(c, seed=11, init_std=0.05)
    params = shaped_params(tr, c)
    micro = [batch(c, 2, 48, seed=20), batch(c, 2, 48, seed=21)]
    ref = [np.zeros(p.shape) for p in params]
    ref_losses = []
    for ids, tg, mask in micro:
        tr.set_batch(ids, tg, mask)
        loss = tr.accumulate(0.5)
        l_ref, g_ref = O.model_loss(oracle_cfg(c), params, ids, tg, mask)
        ref_losses.append(l_ref)
        assert abs(loss - l_ref) <= 1e-4 * abs(l_ref)
        for r, g in zip(ref, g_ref):
            r += 0.5 * g
    for i, name in enumerate(tr.names):
        assert_close(tr.get_grad(i), ref[i].reshape(-1), name=name)
    tr.close()


MODEL = dict(vocab_size=1000, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
             num_attention_heads=4, num_key_value_heads=2, head_dim=64, qk_norm=True,
             rms_norm_eps=1e-6, rope_theta=1e6)


def tr_cfg():
    return TR.make_config(vocab_size=1000, hidden_size=128, intermediate_size=256, num_layers=2,
                          num_heads=4, num_kv_heads=2, head_dim=64, qk_norm=1, rms_norm_eps=1e-6,
                          rope_theta=1e6)


def make_run(root, name, init, data, total, resume=None, **kw):
    d = root / name
    d.mkdir()
    cfg = dict(init_weights=str(init), data_dir=str(data), seq_len=49, batch_size=2,
               grad_accum_steps=2, total_steps=total, warmup_steps=2, lr=1e-3, min_lr_ratio=0.1,
               weight_decay=0.1, clip_grad_norm=0.5, val_every=2, save_every=2, log_every=1,
               seed=7, offload_optimizer=True, gradient_checkpointing=True, model=MODEL)
    if resume:
        cfg["resume_from"] = str(resume)
    cfg.update(kw)
    (d / "config.json").write_text(json.dumps(cfg))
    return d


def read_st(path):
    from safetensors.numpy import load_file
    return load_file(str(path))


@pytest.fixture(scope="module")
def setup(tmp_path_factory):
    root = tmp_path_factory.mktemp("ctd_train")
    c = tr_cfg()
    init_tr = TR.Trainer(c, seed=3, init_std=0.05)
    init = root / "init.safetensors"
    init_tr.save(init)
    init_tr.close()
    # every document the same, so every sampled batch is this one
    rng = np.random.default_rng(5)
    seq_len = 49
    doc = rng.integers(0, 1000, seq_len).astype(np.int32)
    mdoc = np.ones(seq_len, np.int8)
    mdoc[: 20] = 0
    data = root / "data"
    data.mkdir()
    np.tile(doc, 6).tofile(data / "train.bin")
    np.tile(mdoc, 6).tofile(data / "train_mask.bin")
    np.tile(doc, 2).tofile(data / "val.bin")
    np.tile(mdoc, 2).tofile(data / "val_mask.bin")
    return root, c, init, data, doc, mdoc


def replay(c, init, doc, mdoc, steps, cfg):
    """The driver's steps, one trainer call at a time."""
    tr = TR.Trainer(c, seed=0)
    tr.load(init)
    tr.set_checkpointing(True)
    tr.make_optimizer(lr=cfg["lr"], weight_decay=cfg["weight_decay"], offload=True)
    ids = np.tile(doc[:-1], (cfg["batch_size"], 1))
    tg = np.tile(doc[1:], (cfg["batch_size"], 1))
    mask = np.tile(mdoc[1:].astype(np.float32), (cfg["batch_size"], 1))
    tr.set_batch(ids, tg, mask)
    losses = []
    for step in range(1, steps + 1):
        ls = [tr.accumulate(1.0 / cfg["grad_accum_steps"]) for _ in range(cfg["grad_accum_steps"])]
        # the driver's mask-weighted mean in double (main.cpp:363-364, 370-371)
        S = float(mask.sum())
        losses.append(float(np.float32(sum(l * S for l in ls) / (S * len(ls)))))
        tr.set_lr(TR.lr_at_step(step, cfg["warmup_steps"], cfg["total_steps"], cfg["lr"],
                                cfg["min_lr_ratio"]))
        tr.clip(cfg["clip_grad_norm"])
        tr.opt_step()
        tr.zero_grad()
    return tr, losses


def test_ctd_train_run_equals_stepwise_replay(setup):
    root, c, init, data, doc, mdoc = setup
    run = make_run(root, "full", init, data, total=4)
    TR.train_run(run / "config.json")
    cfg = json.loads((run / "config.json").read_text())

    recs = [json.loads(l) for l in (run / "loss.jsonl").read_text().splitlines()]
    train = [r for r in recs if r["phase"] == "train"]
    val = [r for r in recs if r["phase"] == "val"]
    assert [r["step"] for r in train] == [1, 2, 3, 4] and [r["step"] for r in val] == [2, 4]
    for r in train:
        assert list(r) == ["grad_norm", "loss", "lr", "phase", "step", "tokens_per_sec", "wall_s"]
        assert r["lr"] == float(np.float32(TR.lr_at_step(r["step"], 2, 4, 1e-3, 0.1)))
        assert r["tokens_per_sec"] > 0 and np.isfinite(r["loss"]) and r["grad_norm"] > 0
    for f in ("ckpt_step_2.safetensors", "ckpt_step_4.safetensors", "final.safetensors"):
        assert (run / f).exists() and (run / (f + ".opt.safetensors")).exists()

    tr, losses = replay(c, init, doc, mdoc, 4, cfg)
    assert [r["loss"] for r in train] == losses
    final = read_st(run / "final.safetensors")
    opt = read_st(run / "final.safetensors.opt.safetensors")
    assert opt["optimizer.step"][0] == 4.0
    for i, name in enumerate(tr.names):
        assert np.array_equal(final[name].reshape(-1), tr.get_param(i)), name
        m, v = tr.opt_state(i)
        assert np.array_equal(opt["optimizer.m." + name].reshape(-1), m), name
        assert np.array_equal(opt["optimizer.v." + name].reshape(-1), v), name
    # validation loss = the trainer's loss on the (single) validation batch
    tr.set_batch(np.tile(doc[:-1], (1, 1)), np.tile(doc[1:], (1, 1)),
                 mdoc[None, 1:].astype(np.float32))
    assert val[-1]["loss"] == float(np.float32(tr.forward_backward(False)))
    tr.close()


def test_ctd_train_resume_matches_uninterrupted(setup):
    root, c, init, data, doc, mdoc = setup
    first = make_run(root, "first", init, data, total=2)
    TR.train_run(first / "config.json")
    resumed = make_run(root, "resumed", init, data, total=4,
                       resume=first / "final.safetensors")
    TR.train_run(resumed / "config.json")
    steps = [json.loads(l)["step"] for l in (resumed / "loss.jsonl").read_text().splitlines()
             if json.loads(l)["phase"] == "train"]
    assert steps == [3, 4]
    whole = make_run(root, "whole", init, data, total=4)
    TR.train_run(whole / "config.json")
    a = read_st(resumed / "final.safetensors")
    b = read_st(whole / "final.safetensors")
    assert set(a) == set(b)
    for k in a:
        assert np.array_equal(a[k], b[k]), k
    oa = read_st(resumed / "final.safetensors.opt.safetensors")
    ob = read_st(whole / "final.safetensors.opt.safetensors")
    for k in oa:
        assert np.array_equal(oa[k], ob[k]), k
