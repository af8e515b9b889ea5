"""The device allocator's placement (emberlm_amd/csrc/host/block_arena.cpp),
replayed on the host: the arena that serves every device tensor runs over a
backend that only hands out addresses, so splitting, coalescing, best fit,
the cap and a recorded training step can be checked without a GPU.

The recorded history (tests/golden/alloc_history_qwen3-1.7b_B8_T4096.txt.gz)
is the device allocator's own record (bench.py --alloc-history) of setup, one
warmup and fifteen timed recompute + offload steps of Qwen3-1.7B at B=8,
T=4096 on an MI355X, including the split dS workspaces of the attention
backward ("s" records), which the replay plans again against its own arena,
and the elastic optimizer-state prefetch buffers ("e" records)."""
import gzip
import os
import shutil

import pytest

from emberlm_amd import trainer as TR

MiB = 1 << 20
GOLDEN = os.path.join(os.path.dirname(__file__), "golden",
                      "alloc_history_qwen3-1.7b_B8_T4096.txt.gz")


def replay(tmp_path, lines, limit=0):
    p = tmp_path / "h.txt"
    p.write_text("\n".join(lines) + "\n")
    return TR.alloc_replay(str(p), limit)


def test_split_block_serves_smaller_requests_and_coalesces(tmp_path):
    # One 200 MiB segment; two 100 MiB requests split it, and once both are
    # freed their halves merge so a 200 MiB request fits again.
    r = replay(tmp_path, ["a 0 209715200", "f 0", "a 1 104857600", "a 2 104857600",
                          "f 1", "f 2", "a 3 209715200"])
    assert r.segments_obtained == 1
    assert r.peak_reserved == 200 * MiB
    assert r.peak_allocated == 200 * MiB


def test_best_fit_takes_the_smallest_hole(tmp_path):
    # Holes of 300 and 500 MiB (kept apart by live blocks); 250 MiB goes into
    # the 300 MiB hole, so a following 480 MiB request still fits.
    r = replay(tmp_path, ["a 0 524288000", "a 1 2097152", "a 2 314572800", "a 3 2097152",
                          "f 0", "f 2", "a 4 262144000", "a 5 503316480"])
    assert r.segments_obtained == 4
    assert r.peak_reserved == 500 * MiB + 300 * MiB + 2 * 2 * MiB


def test_small_requests_do_not_pin_large_segments(tmp_path):
    # A long-lived 4 KiB tensor comes from a 2 MiB small-request segment, not
    # from the freed 1 GiB block, which stays whole for the next 1 GiB request.
    r = replay(tmp_path, ["a 0 1073741824", "f 0", "a 1 4096", "a 2 1073741824"])
    assert r.segments_obtained == 2
    assert r.peak_reserved == 1024 * MiB + 2 * MiB


def test_cap_empties_the_cache_then_refuses(tmp_path):
    # Under a 1 GiB cap, a 700 MiB request does not fit beside the cached
    # 600 MiB segment: the cache is emptied (one flush) and the request is
    # served from the room that frees.
    lines = ["a 0 629145600", "a 1 2097152", "f 0", "a 2 734003200"]
    r = replay(tmp_path, lines, limit=1024 * MiB)
    assert r.cache_flushes == 1 and r.peak_reserved <= 1024 * MiB
    # Live blocks alone above the cap: the request is refused.
    with pytest.raises(TR.CtdError, match="out of memory"):
        replay(tmp_path, ["a 0 629145600", "a 1 629145600"], limit=1024 * MiB)


# Three free segments of 300, 200 and 100 MiB, kept apart (each its own
# segment, so they never coalesce).
HOLES = ["a 0 314572800", "a 1 209715200", "a 2 104857600", "f 0", "f 1", "f 2"]
UNIT = 64 * MiB


def test_split_workspace_fills_the_free_blocks_without_growing(tmp_path):
    # 8 units of 64 MiB: 4 in the 300 MiB block, 3 in the 200, 1 in the 100.
    r = replay(tmp_path, HOLES + [f"s {UNIT} 8 4 1 16 1", "a 9 536870912", "f 9",
                                  "a 10 314572800"])
    assert r.segments_obtained == 3
    assert r.peak_reserved == 600 * MiB
    assert r.peak_allocated == 600 * MiB


def test_split_workspace_grows_only_to_least(tmp_path):
    # Only the 100 MiB block is free (1 unit < least 4): the rest of the 4
    # units (192 MiB) is one new piece; the other 4 units wanted are not.
    r = replay(tmp_path, ["a 0 104857600", "f 0", f"s {UNIT} 8 4 1 16 1", "a 9 536870912"])
    assert r.segments_obtained == 2
    assert r.peak_reserved == 100 * MiB + 192 * MiB
    assert r.peak_allocated == 64 * MiB + 192 * MiB


def test_split_workspace_is_cut_to_a_multiple(tmp_path):
    # The 300 and 200 MiB blocks hold 7 units; cut to a multiple of 4, the
    # 200 MiB block stays free and serves the next 200 MiB request.
    lines = ["a 0 314572800", "a 1 209715200", "f 0", "f 1", f"s {UNIT} 16 4 4 16 1",
             "a 9 1073741824", "a 10 209715200"]
    r = replay(tmp_path, lines)
    assert r.segments_obtained == 2 and r.peak_reserved == 500 * MiB
    # At most one piece: only the largest block is used.
    r = replay(tmp_path, ["a 0 314572800", "a 1 209715200", "f 0", "f 1",
                          f"s {UNIT} 7 2 1 2 1", "a 9 1073741824", "a 10 209715200"])
    assert r.segments_obtained == 2 and r.peak_reserved == 500 * MiB


def test_replay_rejects_malformed_histories(tmp_path):
    with pytest.raises(TR.CtdError, match="unknown id"):
        replay(tmp_path, ["f 7"])
    with pytest.raises(TR.CtdError, match="allocated twice"):
        replay(tmp_path, ["a 1 512", "a 1 512"])


def test_recorded_qwen3_step_holds_at_most_115_percent_of_live(tmp_path):
    # The recorded steps replayed from an empty arena: the bytes held from the
    # driver stay within 1.15x the live high-water mark, with no cache flush.
    p = tmp_path / "hist.txt"
    with gzip.open(GOLDEN, "rb") as src, open(p, "wb") as dst:
        shutil.copyfileobj(src, dst)
    r = TR.alloc_replay(str(p))
    assert 21e9 < r.peak_allocated < 23e9
    assert r.cache_flushes == 0
    assert r.peak_reserved <= 1.15 * r.peak_allocated, r.peak_reserved / r.peak_allocated
    # Capped at that bound from the start, it never needs to empty its cache.
    r2 = TR.alloc_replay(str(p), int(1.15 * r.peak_allocated))
    assert r2.cache_flushes == 0 and r2.peak_reserved == r.peak_reserved
