"""Device-resident ring bookkeeping (gh_model_ring_*): the decode graph's
first kernel activates the clock's slot and builds slot_idx, S and the active
list on the device (src/ring_buffer.zig:56-136, as src/model/forward.zig:42-43
drives it).  Checked bit for bit against the host ring (ring.cpp, itself
pinned by the reference's ring tests in test_ring.py) across the anchors, the
window's wraparound and recall slots, and the model's outputs against the
host-list path on an identical model."""
import numpy as np
import pytest

import gemma_hip as gh
import oracle as orc
from tol import assert_close

pytestmark = pytest.mark.gpu


def _cfg(max_slots):
    return gh.model_config(vocab=512, hidden=256, intermediate=512, layers=2, heads=4,
                           kv_heads=2, head_dim=64, max_slots=max_slots, global_kv_heads=2,
                           global_head_dim=128, full_layers=(1,))


@pytest.mark.parametrize("tiers,clocks", [((4, 16, 4), 70), ((32, 512, 96), 600)])
def test_device_ring_matches_host_ring(gpu, tiers, clocks):
    A, W, R = tiers
    cfg = _cfg(A + W + R)
    mh = gh.Model(gpu, cfg, seed=3)  # host lists (gh_dispatch_forward_token)
    md = gh.Model(gpu, cfg, seed=3)  # device ring (gh_model_forward_clock)
    try:
        md.ring_init(A, W, R)
        ring = gh.Ring(1, A, W, R)
        rng = np.random.default_rng(A)
        kvd = [md.read(l, gh.T_K_CACHE, np.float32).size // cfg.max_slots for l in range(2)]
        recall_at, clear_at = clocks // 3, 2 * clocks // 3
        for c in range(clocks):
            if c == recall_at:  # recall slots 0 and R-1, stored at earlier clocks
                for rank, rc in ((0, c - 5), (R - 1, c + 3)):
                    for l in range(2):
                        k = rng.standard_normal(kvd[l]).astype(np.float32)
                        v = rng.standard_normal(kvd[l]).astype(np.float32)
                        md.write_recall_kv(l, rank, k, v, rc)
                        for t, a in ((gh.T_K_CACHE, k), (gh.T_V_CACHE, v)):
                            cache = mh.read(l, t, np.float32).reshape(cfg.max_slots, -1)
                            cache[A + W + rank] = a
                            mh.write(l, t, cache)
                    ring.activate_recall(0, rank, rc)
            if c == clear_at:
                md.ring_clear_recall()
                ring.clear_recall()
            x = md.embed(int(rng.integers(0, cfg.vocab_size)))
            want = c % 4 == 3 or c >= clocks - 3
            slot = ring.activate_slot(0, c)
            active = ring.active_slots(0, c)
            td = md.forward_clock(x, c, want)
            th = mh.forward(x, c, slot, active, want)
            step = md.read(-1, gh.T_STEP, np.uint32)
            dense = np.array_equal(active, np.arange(len(active)))
            assert list(step) == [c, slot, len(active), 1 | (2 if dense else 0)], (c, list(step))
            assert np.array_equal(md.read(-1, gh.T_ACTIVE, np.uint32)[:len(active)], active), c
            assert td == th
            if want:
                assert np.array_equal(md.read(-1, gh.T_LOGITS, np.float32),
                                      mh.read(-1, gh.T_LOGITS, np.float32)), c
        if W == 512:  # the window's wraparound: clock 543 -> slot 543, 544 -> slot 32
            assert ring.slot_index(543) == 543 and ring.slot_index(544) == 32
        for l in range(2):
            for t in (gh.T_K_CACHE, gh.T_V_CACHE):
                assert np.array_equal(md.read(l, t, np.float32), mh.read(l, t, np.float32))
        # the device arrays hold the same state as the host mirror of layer 0
        flags = md.read(-1, gh.T_RING_FLAGS, np.uint32)
        assert flags[:A + W].sum() == min(clocks, A + W)
    finally:
        md.close()
        mh.close()


def test_ring_prefill_lists_and_wrapped_batches(gpu):
    A, W, R = 4, 16, 4
    cfg = _cfg(A + W + R)
    md = gh.Model(gpu, cfg, seed=4)
    mh = gh.Model(gpu, cfg, seed=4)
    try:
        md.ring_init(A, W, R)
        ring = gh.Ring(1, A, W, R)
        xs = np.stack([md.embed(t % cfg.vocab_size) for t in range(48)])
        td = md.ring_prefill(xs[:12], 0, True)  # the batched kernels
        slots = [ring.activate_slot(0, c) for c in range(12)]
        lists = [ring.active_slots(0, c) for c in range(12)]
        th = mh.prefill(xs[:12], np.arange(12), slots, lists, True)
        assert td == th
        assert np.array_equal(md.read(-1, gh.T_LOGITS, np.float32), mh.read(-1, gh.T_LOGITS, np.float32))
        for c in range(12, 30):  # decode continues on the device ring
            slot = ring.activate_slot(0, c)
            active = ring.active_slots(0, c)
            assert md.forward_clock(xs[c], c) == mh.forward(xs[c], c, slot, active)
            assert np.array_equal(md.read(-1, gh.T_ACTIVE, np.uint32)[:len(active)], active)
        # a batch past the window's wraparound (token t attends to the slot
        # token t + 1 overwrites; clocks 30 and 46 share a slot) goes through
        # staging rows: the per-token calls' results, to rounding
        td = md.ring_prefill(xs[30:47], 30, True)
        for c in range(30, 47):
            slot = ring.activate_slot(0, c)
            th = mh.forward(xs[c], c, slot, ring.active_slots(0, c), c == 46)
        ld = md.read(-1, gh.T_LOGITS, np.float32)
        assert_close(ld, mh.read(-1, gh.T_LOGITS, np.float32), what="wrapped batch logits")
        assert td == orc.argmax(ld) and th == orc.argmax(mh.read(-1, gh.T_LOGITS, np.float32))
        for l in range(cfg.num_hidden_layers):
            for t in (gh.T_K_CACHE, gh.T_V_CACHE):
                assert_close(md.read(l, t, np.float32), mh.read(l, t, np.float32),
                             what="wrapped batch cache %d/%d" % (l, t))
        flags = md.read(-1, gh.T_RING_FLAGS, np.uint32)
        assert flags[:A + W].sum() == A + W
        slot = ring.activate_slot(0, 47)
        active = ring.active_slots(0, 47)
        md.forward_clock(xs[47], 47)
        mh.forward(xs[47], 47, slot, active)
        assert_close(md.read(-1, gh.T_LOGITS, np.float32), mh.read(-1, gh.T_LOGITS, np.float32),
                     what="decode after the wrapped batch")
        assert np.array_equal(md.read(-1, gh.T_ACTIVE, np.uint32)[:len(active)], active)
        # a host-list call on a ring model must name the ring's slot
        with pytest.raises(gh.GhError):
            md.forward(xs[0], 48, 3, np.array([3], np.uint32))
    finally:
        md.close()
        mh.close()
