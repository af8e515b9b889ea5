"""Model-level GPU parity: the C++ Tensor/autograd/Module/AdamW layer (libctd.so)
against the CPU oracle, plus the checkpointing and offload invariants.

- c1: one SmolLM2-135M-shaped decoder block, B1 T256, seed 0,
  weights ~N(0,0.02), x and dy ~N(0,1): forward/backward vs the oracle, then the
  same with gradient checkpointing (bitwise equal), then one AdamW step with m/v
  offloaded (lr 1e-4, betas 0.9/0.95, eps 1e-8, wd 0.1 on 2-D weights).
- tiny full models (embedding + blocks + tied head + masked CE) vs the oracle's
  loss and every gradient, with QK-Norm and with llama3 RoPE scaling.
- c2 full SmolLM2-135M step at B4 T512, and the full c3 (Qwen3-0.6B B4 T1024),
  c4 (LLaMA-3.2-1B B4 T2048, llama3 RoPE) and c5 (Qwen3-1.7B B8 T4096) steps:
  checkpoint on/off bitwise identical (c3-c5: every gradient, by digest), loss
  at its init value.
- c5: two offloaded train steps equal the on-device ones bitwise (p, m, v).
- c1 block, c2 full step and 2-layer c3/c4 models at full width and vocabulary
  against the golden fixtures (tests/golden), an independent float64 torch
  composition frozen in files.
Tolerance: |a-b| <= 1e-4|b| + 1e-4 max|b| and relative L2 <= 1e-4; AdamW 1e-5.
"""
import hashlib
import json
import math
import os
import struct

import numpy as np
import pytest

import oracle as O
from tests.golden import make_golden as MG
from tests.helpers import assert_close, assert_matches_golden

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from emberlm_amd import trainer as TR  # noqa: E402


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


BLOCK_ORDER = ["input_layernorm", "q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm",
               "post_attention_layernorm", "gate_proj", "up_proj", "down_proj"]


def oracle_cfg(c: TR.ModelConfig):
    return O.make_cfg(vocab=c.vocab_size, hidden=c.hidden_size, inter=c.intermediate_size,
                      layers=c.num_layers, heads=c.num_heads, kv_heads=c.num_kv_heads,
                      head_dim=c.head_dim, eps=float(np.float32(c.rms_norm_eps)),
                      theta=c.rope_theta, rope_factor=c.rope_factor,
                      rope_low_freq=c.rope_low_freq_factor, rope_high_freq=c.rope_high_freq_factor,
                      rope_orig_max_pos=c.rope_original_max_pos, qk_norm=c.qk_norm)


def shapes(c):
    d, I, H, Hk, D = c.hidden_size, c.intermediate_size, c.num_heads, c.num_kv_heads, c.head_dim
    return {"input_layernorm": (d,), "q_proj": (H * D, d), "k_proj": (Hk * D, d),
            "v_proj": (Hk * D, d), "o_proj": (d, H * D), "q_norm": (D,), "k_norm": (D,),
            "post_attention_layernorm": (d,), "gate_proj": (I, d), "up_proj": (I, d),
            "down_proj": (d, I)}


def layer_params(tr, c, layer):
    sh = shapes(c)
    out = {}
    for i, name in enumerate(tr.names):
        pre = f"model.layers.{layer}."
        if name.startswith(pre):
            key = name[len(pre):].split(".")[-2]
            out[key] = (i, tr.get_param(i).reshape(sh[key]))
    return out


C1 = dict(vocab_size=256, hidden_size=576, intermediate_size=1536, num_layers=1, num_heads=9,
          num_kv_heads=3, head_dim=64, rms_norm_eps=1e-5, rope_theta=1e5)


def test_c1_block_fwd_bwd_checkpoint_and_offloaded_adamw():
    c = TR.make_config(**C1)
    tr = TR.Trainer(c, seed=0, init_std=0.02, norm_value=None)  # all weights ~N(0,0.02)
    rng = np.random.default_rng(0)
    B, T, d = 1, 256, 576
    x = rng.standard_normal((B, T, d)).astype(np.float32)
    dy = rng.standard_normal((B, T, d)).astype(np.float32)
    lp = layer_params(tr, c, 0)
    w = {k: v[1] for k, v in lp.items()}
    oc = oracle_cfg(c)

    y, dx = tr.block_step(0, x, dy, checkpoint=False)
    grads_off = {k: tr.get_grad(i).reshape(w[k].shape) for k, (i, _) in lp.items()}
    assert_close(y, O.block_fwd(oc, w, x), name="c1 y")
    dx_ref, dw_ref = O.block_bwd(oc, w, x, dy)
    assert_close(dx, dx_ref, name="c1 dx")
    for k in w:
        assert_close(grads_off[k], dw_ref[k], name=f"c1 d{k}")

    # Gradient checkpointing: recomputed activations and every gradient bitwise equal.
    tr.zero_grad()
    y2, dx2 = tr.block_step(0, x, dy, checkpoint=True)
    assert np.array_equal(y, y2) and np.array_equal(dx, dx2)
    for k, (i, _) in lp.items():
        assert np.array_equal(tr.get_grad(i).reshape(w[k].shape), grads_off[k]), k

    # One AdamW step with m/v offloaded to pinned host memory, checked per element
    # against the oracle update from the same gradients.
    tr.make_optimizer(lr=1e-4, weight_decay=0.1, beta1=0.9, beta2=0.95, eps=1e-8, offload=True)
    tr.opt_step()
    bc1, bc2 = np.float32(1 - np.float32(0.9)), np.float32(1 - np.float32(0.95))
    for k, (i, p0) in lp.items():
        g = grads_off[k]
        wd = 0.1 if tr.decay[i] else 0.0
        rp, rm, rv = O.adamw(p0.reshape(-1), g.reshape(-1), np.zeros(g.size), np.zeros(g.size),
                             np.float32(1e-4), np.float32(0.9), np.float32(0.95), np.float32(1e-8),
                             np.float32(wd), bc1, bc2)
        m, v = tr.opt_state(i)
        for got, ref, nm in [(tr.get_param(i), rp, "p"), (m, rm, "m"), (v, rv, "v")]:
            err = np.abs(got - ref)
            bound = 1e-5 * np.abs(ref) + 1e-6 * np.abs(ref).max()
            assert (err <= bound).all(), (k, nm, float(err.max()))
    tr.close()


GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_c1_block_vs_golden():
    # The HIP block against the independent float64 torch fixture for
    # BASELINE config 0 (tests/golden/make_golden.py), checkpointing off and on.
    g = np.load(os.path.join(GOLDEN, "c1_block.npz"), allow_pickle=False)
    w, x, dy = MG.c1_inputs()
    c = TR.make_config(**C1)
    tr = TR.Trainer(c, seed=0, init_std=0.02, norm_value=None)
    lp = layer_params(tr, c, 0)
    assert sorted(lp) == sorted(MG.BLOCK_KEYS)
    for k, (i, _) in lp.items():
        tr.set_param(i, w[k])
    for ckpt in (False, True):
        tr.zero_grad()
        y, dx = tr.block_step(0, x, dy, checkpoint=ckpt)
        assert_matches_golden(g, "y", y, rows=True)
        assert_matches_golden(g, "dx", dx, rows=True)
        for k, (i, _) in lp.items():
            assert_matches_golden(g, "d_" + k, tr.get_grad(i))
    tr.close()


def _model_step_vs_golden(c, mc, fixture):
    """Loads the fixture's inputs (tests/golden/make_golden.py) into a model of
    config mc and checks the loss and the summarised gradients, with
    checkpointing on, against the float64 torch fixture; then checks that the
    step without checkpointing gives the same bits."""
    g = np.load(os.path.join(GOLDEN, fixture), allow_pickle=False)
    params, ids, tg, mask = MG.model_inputs(c)
    tr = TR.Trainer(mc, seed=0, init_std=0.02)
    names = MG.grad_names(c)
    assert tr.num_params() == len(params) == len(names)
    for i, (name, prm) in enumerate(zip(tr.names, params)):
        want = names[i]
        if want == "embed":
            assert name == "model.embed_tokens.weight"
        elif want == "norm":
            assert name == "model.norm.weight"
        else:
            layer, key = want[1:].split(".")
            assert name.startswith(f"model.layers.{layer}.") and name.split(".")[-2] == key, name
        assert tr.numels[i] == prm.size, name
        tr.set_param(i, prm)
    del params
    tr.set_batch(ids, tg, mask)
    tr.set_checkpointing(True)
    loss = tr.forward_backward(True)
    assert abs(loss - float(g["loss"])) <= 1e-4 * abs(float(g["loss"])), (loss, float(g["loss"]))
    kept = MG.summarised_grads(c)
    grads = {i: tr.get_grad(i) for i in kept}
    for i in kept:
        assert_matches_golden(g, "g." + names[i], grads[i])
    tr.zero_grad()
    tr.set_checkpointing(False)
    assert tr.forward_backward(True) == loss
    for i in kept:
        assert np.array_equal(tr.get_grad(i), grads[i]), names[i]
    tr.close()


def test_c2_smollm2_step_vs_golden():
    # BASELINE config 1 at full size (SmolLM2-135M, B=4, T=512, masked loss)
    # against the independent float64 torch fixture: the loss and the
    # gradient of every one of the 272 parameters.
    _model_step_vs_golden(MG.C2, TR.preset("smollm2-135m"), "c2_model.npz")


def _reduced(preset, layers):
    c = TR.preset(preset)
    c.num_layers = layers
    return c


def test_c3_qwen3_06b_two_layers_vs_golden():
    # BASELINE config 2's Qwen3-0.6B at its real width, heads (16/8 of 128, QK-Norm)
    # and vocabulary (151936), B=4, T=1024, masked loss, cut to 2 layers.
    c = _reduced("qwen3-0.6b", MG.C3["layers"])
    assert (c.hidden_size, c.num_heads, c.num_kv_heads, c.head_dim, c.vocab_size, c.qk_norm) == (
        MG.C3["hidden"], MG.C3["heads"], MG.C3["kv_heads"], MG.C3["head_dim"], MG.C3["vocab"], 1)
    _model_step_vs_golden(MG.C3, c, "c3_model.npz")


def test_c4_llama32_1b_two_layers_vs_golden():
    # BASELINE config 3's LLaMA-3.2-1B at its real width, heads (32/8 of 64,
    # GQA group 4) and vocabulary (128256), llama3 RoPE over positions 0..2047,
    # all-ones mask, cut to 2 layers at B=2.  The fixture's frequencies come
    # from the per-band statement pinned in tests/test_oracle.py.
    c = _reduced("llama3.2-1b", MG.C4["layers"])
    assert (c.hidden_size, c.num_heads, c.num_kv_heads, c.head_dim, c.vocab_size) == (
        MG.C4["hidden"], MG.C4["heads"], MG.C4["kv_heads"], MG.C4["head_dim"], MG.C4["vocab"])
    assert (c.rope_factor, c.rope_low_freq_factor, c.rope_high_freq_factor,
            c.rope_original_max_pos) == MG.C4["rope"]
    _model_step_vs_golden(MG.C4, c, "c4_model.npz")


def test_c5_qwen3_17b_two_layers_vs_golden():
    # BASELINE config 4's Qwen3-1.7B at its real width (hidden 2048, MLP 6144),
    # heads (16/8 of 128, QK-Norm) and vocabulary (151936), at T=4096 with the
    # prefix loss mask, cut to 2 layers at B=1.
    c = _reduced("qwen3-1.7b", MG.C5["layers"])
    assert (c.hidden_size, c.intermediate_size, c.num_heads, c.num_kv_heads, c.head_dim,
            c.vocab_size, c.qk_norm) == (MG.C5["hidden"], MG.C5["inter"], MG.C5["heads"],
                                         MG.C5["kv_heads"], MG.C5["head_dim"], MG.C5["vocab"], 1)
    _model_step_vs_golden(MG.C5, c, "c5_model.npz")


def tiny_cfg(qk_norm=False, llama3=False, D=64, vocab=1000):
    # vocab 1000 takes the LM head's all-rows form, a multiple of 16 (1024) the
    # form that computes only rows with a nonzero mask value.
    return TR.make_config(vocab_size=vocab, hidden_size=128, intermediate_size=256, num_layers=2,
                          num_heads=4, num_kv_heads=2, head_dim=D, qk_norm=int(qk_norm),
                          rms_norm_eps=1e-6 if qk_norm else 1e-5,
                          rope_theta=5e5 if llama3 else 1e4, rope_factor=32.0 if llama3 else 0.0,
                          rope_original_max_pos=64 if llama3 else 8192)


def batch(c, B, T, seed):
    rng = np.random.default_rng(seed)
    row = rng.integers(0, c.vocab_size, (B, T + 1))
    mask = np.ones((B, T), np.float32)
    for b in range(B):
        mask[b, : int(rng.uniform(0.2, 0.6) * T)] = 0
    return row[:, :T], row[:, 1:], mask


@pytest.mark.parametrize("qk_norm,llama3,D,vocab", [(False, False, 64, 1000),
                                                    (True, False, 128, 1000),
                                                    (False, True, 64, 1000),
                                                    # head sizes outside the fused kernels'
                                                    # 64/128: the reference's
                                                    # bmm/mask/softmax chain
                                                    (True, False, 16, 1000),
                                                    (False, True, 32, 1000),
                                                    (False, False, 8, 1000),
                                                    # LM head over the active rows only
                                                    (True, False, 128, 1024),
                                                    (False, True, 64, 1024)])
def test_tiny_model_loss_and_grads_vs_oracle(qk_norm, llama3, D, vocab):
    c = tiny_cfg(qk_norm, llama3, D, vocab)
    tr = TR.Trainer(c, seed=1, init_std=0.1, norm_value=None)
    ids, tg, mask = batch(c, 2, 96, seed=2)
    tr.set_batch(ids, tg, mask)
    loss = tr.forward_backward(True)
    params = [tr.get_param(i) for i in range(tr.num_params())]
    sh = shapes(c)
    shaped = []
    for name, p in zip(tr.names, params):
        if name == "model.embed_tokens.weight":
            shaped.append(p.reshape(c.vocab_size, c.hidden_size))
        elif name == "model.norm.weight":
            shaped.append(p)
        else:
            shaped.append(p.reshape(sh[name.split(".")[-2]]))
    ref_loss, ref_grads = O.model_loss(oracle_cfg(c), shaped, ids, tg, mask)
    assert abs(loss - ref_loss) <= 1e-4 * abs(ref_loss), (loss, ref_loss)
    grads_off = []
    for i, name in enumerate(tr.names):
        g = tr.get_grad(i)
        assert g is not None, name
        assert_close(g, ref_grads[i].reshape(-1), name=name)
        grads_off.append(g)
    # checkpointing on: same loss bits, same gradient bits
    tr.zero_grad()
    tr.set_checkpointing(True)
    loss2 = tr.forward_backward(True)
    assert loss2 == loss
    for i, name in enumerate(tr.names):
        assert np.array_equal(tr.get_grad(i), grads_off[i]), name
    tr.close()


@pytest.mark.parametrize("qk_norm,D", [(False, 64), (True, 128)])
def test_kept_attention_scores_with_checkpointing(qk_norm, D):
    # Attention that keeps its scores for the backward (the checkpointed
    # re-run's forward keeps them, its backward reads them): the same loss
    # bits (the forward is unchanged), gradients within fp32 rounding of the
    # default path and against the oracle, and bit for bit on a repeat.
    c = tiny_cfg(qk_norm, False, D, 1024)
    tr = TR.Trainer(c, seed=3, init_std=0.1, norm_value=None)
    ids, tg, mask = batch(c, 2, 130, seed=4)
    tr.set_batch(ids, tg, mask)
    tr.set_checkpointing(True)
    try:
        loss = tr.forward_backward(True)
        ref = [tr.get_grad(i) for i in range(tr.num_params())]
        TR.set_attn_keep_scores(True)
        runs = []
        for _ in range(2):
            tr.zero_grad()
            runs.append((tr.forward_backward(True),
                         [tr.get_grad(i) for i in range(tr.num_params())]))
    finally:
        TR.set_attn_keep_scores(False)
    assert runs[0][0] == loss and runs[1][0] == loss
    for name, a, b, g in zip(tr.names, runs[0][1], runs[1][1], ref):
        assert np.array_equal(a, b), name
        assert_close(a, g, rtol=1e-5, name=name)
    sh = shapes(c)
    params = []
    for name, i in zip(tr.names, range(tr.num_params())):
        pv = tr.get_param(i)
        if name == "model.embed_tokens.weight":
            params.append(pv.reshape(c.vocab_size, c.hidden_size))
        elif name == "model.norm.weight":
            params.append(pv)
        else:
            params.append(pv.reshape(sh[name.split(".")[-2]]))
    _, ref_grads = O.model_loss(oracle_cfg(c), params, ids, tg, mask)
    for i, name in enumerate(tr.names):
        assert_close(runs[0][1][i], ref_grads[i].reshape(-1), name=name)
    tr.close()



@pytest.mark.parametrize("vocab,dead_rows", [(1000, 0), (1024, 0), (1024, 100)])
def test_chunked_lm_head_loss_equals_single_chunk(vocab, dead_rows):
    """The LM head + loss run a chunk of rows at a time; the loss does not
    depend on the chunking (bitwise), the gradients only through the order dW
    is summed in.  vocab 1024 takes the active-rows form, where chunks hold
    active rows only (dead_rows: the first rows all masked out, so that a
    whole chunk's worth of rows has nothing to compute); its loss is the
    all-rows form's (set_head_active_rows(False)) bit for bit and its
    gradients equal within fp32 rounding."""
    c = tiny_cfg(qk_norm=True, D=64, vocab=vocab)
    ids, tg, mask = batch(c, 2, 96, seed=8)
    mask.reshape(-1)[:dead_rows] = 0
    runs = []
    for rows in (0, 64, 40):   # automatic (one chunk), 3 chunks, 5 chunks (ragged)
        TR.set_head_chunk_rows(rows)
        tr = TR.Trainer(c, seed=4, init_std=0.1, norm_value=None)
        tr.set_batch(ids, tg, mask)
        loss = tr.forward_backward(True)
        runs.append((loss, [tr.get_grad(i) for i in range(tr.num_params())], tr.names))
        tr.close()
    if vocab % 16 == 0:  # the same model with every row through the head
        TR.set_head_active_rows(False)
        try:
            tr = TR.Trainer(c, seed=4, init_std=0.1, norm_value=None)
            tr.set_batch(ids, tg, mask)
            loss = tr.forward_backward(True)
            runs.append((loss, [tr.get_grad(i) for i in range(tr.num_params())], tr.names))
            tr.close()
        finally:
            TR.set_head_active_rows(True)
    TR.set_head_chunk_rows(0)
    base_loss, base_grads, names = runs[0]
    for loss, grads, _ in runs[1:]:
        assert loss == base_loss
        for name, g, b in zip(names, grads, base_grads):
            assert_close(g, b, rtol=1e-5, name=name)


@pytest.mark.parametrize("vocab", [1000, 1024])
def test_lm_head_loss_with_every_row_masked_out(vocab):
    # The reference's masked CE: a zero mask gives loss 0 in the forward and an
    # error in the backward (sum(loss_mask) == 0, loss.cu:382-408), through the
    # all-rows form (vocab 1000) and the active-rows form, which then finds no
    # rows at all (vocab 1024).
    c = tiny_cfg(qk_norm=True, D=64, vocab=vocab)
    ids, tg, mask = batch(c, 2, 64, seed=3)
    mask[:] = 0
    tr = TR.Trainer(c, seed=1, init_std=0.1, norm_value=None)
    tr.set_batch(ids, tg, mask)
    assert tr.forward_backward(False) == 0.0
    with pytest.raises(TR.CtdError, match=r"sum\(loss_mask\) == 0"):
        tr.forward_backward(True)
    tr.close()


def test_offload_equals_on_device_over_steps():
    c = tiny_cfg(qk_norm=True, D=128)
    a = TR.Trainer(c, seed=3, init_std=0.05)
    b = TR.Trainer(c, seed=3, init_std=0.05)
    a.make_optimizer(lr=1e-3, weight_decay=0.1, offload=True, chunk_elems=4099)  # many chunks
    b.make_optimizer(lr=1e-3, weight_decay=0.1, offload=False)
    for step in range(3):
        for t in (a, b):
            t.synthetic_batch(2, 64, seed=step, masked=True)
            t.forward_backward(True)
            t.clip(1.0)
            t.opt_step()
            t.zero_grad()
    for i in range(a.num_params()):
        assert np.array_equal(a.get_param(i), b.get_param(i)), a.names[i]
        ma, va = a.opt_state(i)
        mb, vb = b.opt_state(i)
        assert np.array_equal(ma, mb) and np.array_equal(va, vb), a.names[i]
    a.close()
    b.close()


def test_overlapped_offload_train_steps_equal_on_device():
    # train_step returns while the offloaded update still streams; the next
    # forward must see every updated parameter, and the host reads below must
    # see the final state without an explicit synchronize.
    c = tiny_cfg(qk_norm=True, D=64)
    a = TR.Trainer(c, seed=5, init_std=0.05)
    b = TR.Trainer(c, seed=5, init_std=0.05)
    a.make_optimizer(lr=1e-3, weight_decay=0.1, offload=True, chunk_elems=3000)
    b.make_optimizer(lr=1e-3, weight_decay=0.1, offload=False)
    losses = {id(a): [], id(b): []}
    for step in range(4):
        for t in (a, b):
            t.synthetic_batch(2, 96, seed=10 + step, masked=True)
            losses[id(t)].append(t.train_step(1.0).loss)
    assert losses[id(a)] == losses[id(b)]
    for i in range(a.num_params()):
        assert np.array_equal(a.get_param(i), b.get_param(i)), a.names[i]
        ma, va = a.opt_state(i)
        mb, vb = b.opt_state(i)
        assert np.array_equal(ma, mb) and np.array_equal(va, vb), a.names[i]
    ms, nbytes, prefetched = a.offload_stats()
    assert ms > 0 and nbytes >= 8 * sum(a.numels) and prefetched == 0  # no checkpointing
    a.close()
    b.close()


@pytest.mark.parametrize("chunk", [3000, 1 << 20, 50000])
def test_prefetched_offload_with_checkpointing_equals_on_device(chunk):
    # With checkpointing on, train_step's backward stages the m/v of the first
    # parameter in streaming order (the embedding) on the device when it re-runs
    # layer 1 (AdamW::prefetch), and step() updates those chunks from there.
    # chunk 3000: the embedding spans 43 chunks, more than the 32 prefetched;
    # 1 << 20: the whole state is one chunk, so step() copies nothing in;
    # 50000: the third prefetched chunk runs past the embedding into layer 0.
    c = tiny_cfg(qk_norm=True, D=64)
    a = TR.Trainer(c, seed=6, init_std=0.05)
    b = TR.Trainer(c, seed=6, init_std=0.05)
    for t in (a, b):
        t.set_checkpointing(True)
    a.make_optimizer(lr=1e-3, weight_decay=0.1, offload=True, chunk_elems=chunk)
    a.set_prefetch_layer(1)  # the estimate skips the prefetch for a model this small
    b.make_optimizer(lr=1e-3, weight_decay=0.1, offload=False)
    losses = {id(a): [], id(b): []}
    for step in range(4):
        for t in (a, b):
            t.synthetic_batch(2, 96, seed=20 + step, masked=True)
            losses[id(t)].append(t.train_step(1.0).loss)
    assert losses[id(a)] == losses[id(b)]
    for i in range(a.num_params()):
        assert np.array_equal(a.get_param(i), b.get_param(i)), a.names[i]
        ma, va = a.opt_state(i)
        mb, vb = b.opt_state(i)
        assert np.array_equal(ma, mb) and np.array_equal(va, vb), a.names[i]
    # Expected prefetch: whole chunks covering the first parameter, at most 32,
    # within the flat state (each parameter padded to 64 floats).
    assert a.names[0] == "model.embed_tokens.weight"
    chunk_r = (chunk + 63) // 64 * 64
    flat_n = sum((n + 63) // 64 * 64 for n in a.numels)
    nch = min(-(-a.numels[0] // chunk_r), 32)
    ms, nbytes, prefetched = a.offload_stats()
    assert ms > 0 and nbytes == 8 * flat_n
    assert prefetched == 8 * min(nch * chunk_r, flat_n)
    a.close()
    b.close()


def test_train_step_and_checkpoint_roundtrip(tmp_path):
    c = tiny_cfg()
    a = TR.Trainer(c, seed=4)
    a.make_optimizer(lr=1e-3, offload=True)
    a.synthetic_batch(2, 64, seed=5)
    t = a.train_step(1.0)
    assert math.isfinite(t.loss) and t.loss > 0 and t.total_ms > 0
    path = tmp_path / "ckpt.safetensors"
    a.save(path)
    # header: u64 length, compact key-sorted JSON, space padded to 8 bytes
    def header(p):
        raw = open(p, "rb").read()
        (hl,) = struct.unpack("<Q", raw[:8])
        assert hl % 8 == 0
        return raw[8: 8 + hl].decode()
    head = header(path)
    keys = list(json.loads(head).keys())
    assert keys == sorted(keys) and '"data_offsets":' in head and ", " not in head
    b = TR.Trainer(c, seed=99)
    b.make_optimizer(lr=1e-3, offload=True)
    b.load(path)
    for i in range(a.num_params()):
        assert np.array_equal(a.get_param(i), b.get_param(i))
        ma, va = a.opt_state(i)
        mb, vb = b.opt_state(i)
        assert np.array_equal(ma, mb) and np.array_equal(va, vb)
    opt_keys = json.loads(header(str(path) + ".opt.safetensors"))
    assert "optimizer.step" in opt_keys and f"optimizer.m.{a.names[0]}" in opt_keys
    a.close()
    b.close()


def test_c2_smollm2_full_step_checkpoint_bitwise():
    c = TR.preset("smollm2-135m")
    tr = TR.Trainer(c, seed=0, init_std=0.02)
    tr.synthetic_batch(4, 512, seed=0, masked=True)
    loss_off = tr.forward_backward(True)
    g_off = [tr.get_grad(i) for i in (0, 1, 5, tr.num_params() - 1)]
    tr.zero_grad()
    tr.set_checkpointing(True)
    loss_on = tr.forward_backward(True)
    assert loss_on == loss_off
    # At init the logits are ~N(0, s^2) with s^2 = d * 0.02^2 (unit-RMS hidden states
    # times N(0, 0.02) embeddings), so E[loss] ~ ln V + s^2 / 2.
    assert abs(loss_off - (math.log(c.vocab_size) + c.hidden_size * 0.02 ** 2 / 2)) < 0.05
    for j, i in enumerate((0, 1, 5, tr.num_params() - 1)):
        assert np.array_equal(tr.get_grad(i), g_off[j])
    tr.close()


# BASELINE configs 2, 3 and 4 at full size: (preset, B, T, loss mask).  c3 has
# 28 layers, c4 16 with llama3 RoPE and the all-ones mask, c5 28 (about 143 GB of
# HBM without checkpointing).
FULL = [("qwen3-0.6b", 4, 1024, True), ("llama3.2-1b", 4, 2048, False),
        ("qwen3-1.7b", 8, 4096, True)]


def digest(a):
    return hashlib.blake2b(a.tobytes(), digest_size=16).digest()


@pytest.mark.parametrize("preset,B,T,masked", FULL)
def test_full_step_checkpoint_bitwise(preset, B, T, masked):
    # The loss and every gradient with checkpointing on equal the
    # non-checkpointed ones bit for bit, and the loss sits at its value for
    # N(0, 0.02) weights at init.
    c = TR.preset(preset)
    tr = TR.Trainer(c, seed=0, init_std=0.02)
    tr.synthetic_batch(B, T, seed=0, masked=masked)
    loss_off = tr.forward_backward(True)
    d_off = [digest(tr.get_grad(i)) for i in range(tr.num_params())]
    tr.zero_grad()
    tr.set_checkpointing(True)
    loss_on = tr.forward_backward(True)
    assert loss_on == loss_off
    assert abs(loss_off - (math.log(c.vocab_size) + c.hidden_size * 0.02 ** 2 / 2)) < 0.05
    for i in range(tr.num_params()):
        assert digest(tr.get_grad(i)) == d_off[i], tr.names[i]
    tr.close()


@pytest.mark.parametrize("preset,B,T,masked", [("llama3.2-1b", 4, 2048, False),
                                                ("qwen3-1.7b", 8, 4096, True)])
def test_full_size_offloaded_steps_equal_on_device(preset, B, T, masked):
    # Two recompute + offload train steps of BASELINE config 3 (LLaMA-3.2-1B,
    # B=4, T=2048, llama3 RoPE, all-ones mask) and config 4 (Qwen3-1.7B, B=8,
    # T=4096) against the same steps with m/v on the device: every parameter,
    # m and v equal bit for bit.  The offloaded state is one pinned buffer
    # each for m and v (4.9 / 6.9 GB: byte offsets past 2^32), cut into
    # 16M-float chunks that cross parameter boundaries, and the embedding's
    # chunks are prefetched during the backward at the default layer (a), or
    # not at all (p); the second step reads back what the first wrote.
    c = TR.preset(preset)
    a = TR.Trainer(c, seed=0, init_std=0.02)
    p = TR.Trainer(c, seed=0, init_std=0.02)
    b = TR.Trainer(c, seed=0, init_std=0.02)
    a.make_optimizer(lr=1e-4, weight_decay=0.1, offload=True)
    p.make_optimizer(lr=1e-4, weight_decay=0.1, offload=True)
    p.set_prefetch_chunks(0)
    b.make_optimizer(lr=1e-4, weight_decay=0.1, offload=False)
    for t in (a, p, b):
        t.set_checkpointing(True)
    for step in range(2):
        losses = []
        for t in (a, p, b):
            t.synthetic_batch(B, T, seed=step, masked=masked)
            losses.append(t.train_step(1.0).loss)
        assert losses[0] == losses[1] == losses[2], (step, losses)
    ms, nbytes, prefetched = a.offload_stats()
    assert nbytes > 2 ** 32 and prefetched > 0
    assert p.offload_stats()[2] == 0
    for i in range(a.num_params()):
        want = b.get_param(i)
        mb, vb = b.opt_state(i)
        for t in (a, p):
            assert np.array_equal(t.get_param(i), want), a.names[i]
            mt, vt = t.opt_state(i)
            assert np.array_equal(mt, mb), a.names[i]
            assert np.array_equal(vt, vb), a.names[i]
    for t in (a, p, b):
        t.close()
