"""The rotating (sliding-window) cache semantics the GPU ring follows, pinned against a
step-by-step restatement of the reference's RotatingCache::append
(crates/kvcache/src/rotating.rs:56-97): after any sequence of appends the cache holds the
positions [max(0, total - window), total), in order, and the ring layout places each of
them in a distinct row p % window."""
import numpy as np
import pytest

import oracle


@pytest.mark.parametrize("window", [1, 7, 64, 300])
def test_rotating_cache_keeps_the_last_window(window):
    rng = np.random.default_rng(window)
    for trial in range(50):
        kept, total = [], 0
        for _ in range(int(rng.integers(1, 12))):
            n = int(rng.integers(1, 2 * window + 3))
            kept = oracle.rotating_append(kept, n, window)
            total += n
            lo, hi = oracle.rotating_window(total, window)
            assert kept == list(range(lo, hi)), (window, total, n)
            rows = oracle.ring_rows(total, window)
            assert sorted(rows.values()) == kept and len(rows) == len(kept) <= window
            assert all(0 <= r < window and p % window == r for r, p in rows.items())


def test_rotating_len_matches_reference():
    # len() = min(write_pos, total_len) (rotating.rs:108-110) = min(total, window)
    for window in (4, 16):
        kept, total = [], 0
        for n in (3, 1, 1, 9, 1, 30):
            kept = oracle.rotating_append(kept, n, window)
            total += n
            assert len(kept) == min(total, window)
