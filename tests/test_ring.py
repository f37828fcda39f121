"""The product's ring bookkeeping (gh_ring_*) against the oracle's
restatement of src/ring_buffer.zig and the reference's own ring tests."""
import numpy as np

import gemma_hip as gh
import oracle as orc


def test_ring_reference_kat_window_eviction():
    # src/ring_buffer.zig:149-166
    r = gh.Ring(2, 4, 8, 4)
    assert r.total_slots == 16
    for c in range(20):
        r.activate_slot(0, c)
    s = r.active_slots(0, 19)
    assert len(s) == 12 and s[0] == 0 and s[3] == 3


def test_ring_reference_kat_recall():
    # src/ring_buffer.zig:168-187
    r = gh.Ring(1, 2, 4, 3)
    r.activate_recall(0, 0, 100)
    r.activate_recall(0, 1, 50)
    assert len(r.active_slots(0, 101)) == 2
    r.clear_recall()
    assert len(r.active_slots(0, 101)) == 0


def test_ring_matches_oracle_random():
    rng = np.random.default_rng(12)
    for A, W, R in [(32, 512, 96), (4, 16, 4), (0, 8, 2), (3, 5, 0)]:
        g = gh.Ring(2, A, W, R)
        o = orc.Ring(2, 1, A, W, R)
        clock = 0
        for step in range(700):
            clock += int(rng.integers(1, 3))
            for layer in (0, 1):
                assert g.activate_slot(layer, clock) == o.activate_slot(layer, clock)
            if R and rng.random() < 0.05:
                rank = int(rng.integers(0, R))
                c = int(rng.integers(0, clock + 20))
                g.activate_recall(0, rank, c)
                o.write_recall_kv(0, rank, np.zeros(1, np.float32), np.zeros(1, np.float32), c)
            if R and rng.random() < 0.02:
                g.clear_recall()
                o.clear_recall()
            q = clock + int(rng.integers(-3, 3))
            q = max(q, 0)
            assert np.array_equal(g.active_slots(0, q), o.active_slots(0, q))
            assert g.slot_index(q) == o.slot_index(q)
