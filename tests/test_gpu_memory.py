"""The device allocator on BASELINE config 4 (Qwen3-1.7B, B=8, T=4096,
recompute + offloaded AdamW), on the GPU: capped at 1.15x the live high-water
mark of a first step, two more steps run without the allocator emptying its
cache or failing, and give the same loss, parameters and optimizer state bit
for bit as the same three steps without a cap."""
import hashlib

import numpy as np
import pytest

from emberlm_amd import trainer as TR

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def digest(a):
    return hashlib.blake2b(np.ascontiguousarray(a).tobytes(), digest_size=16).digest()


def three_steps(cap_factor):
    TR.set_memory_limit(0)
    TR.empty_cache()
    c = TR.preset("qwen3-1.7b")
    t = TR.Trainer(c, seed=0, init_std=0.02)
    try:
        t.make_optimizer(lr=1e-4, weight_decay=0.1, offload=True)
        t.set_checkpointing(True)
        t.synthetic_batch(8, 4096, seed=0, masked=True)
        TR.reset_peak_memory()
        losses = [t.train_step(1.0).loss]
        t.synchronize()
        first = TR.memory()
        cap = int(cap_factor * first.peak_allocated) if cap_factor else 0
        TR.set_memory_limit(cap)
        for step in (1, 2):
            t.synthetic_batch(8, 4096, seed=step, masked=True)
            losses.append(t.train_step(1.0).loss)
        t.synchronize()
        after = TR.memory()
        state = [(digest(t.get_param(i)),) + tuple(digest(x) for x in t.opt_state(i))
                 for i in range(t.num_params())]
        return losses, state, first, after, cap
    finally:
        TR.set_memory_limit(0)
        t.close()


def test_c5_steps_within_115_percent_of_live_peak():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    ref_losses, ref_state, _, _, _ = three_steps(None)
    losses, state, first, after, cap = three_steps(1.15)
    print(f"live peak {first.peak_allocated / 1e9:.3f} GB, held {first.reserved / 1e9:.3f} GB, "
          f"cap {cap / 1e9:.3f} GB; after: held peak {after.peak_reserved / 1e9:.3f} GB, "
          f"flushes {after.cache_flushes - first.cache_flushes}")
    assert first.reserved <= cap
    assert after.cache_flushes == first.cache_flushes, "the allocator emptied its cache"
    assert after.peak_reserved <= cap
    assert losses == ref_losses
    assert state == ref_state
