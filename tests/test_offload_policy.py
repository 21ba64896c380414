"""HotCache's policy on the host (hotcache.py:18-121): exponential moving average of use, eviction only past the
margin, at most swaps_per_token copies per token, experts the token uses never evicted, slots off-limits until their
copy lands, and the slot map published only after landing. The copies here are CPU tensor copies; on the GPU they are
host -> device DMAs on the cache's own stream (tests/test_gpu_offload.py)."""
import numpy as np
import torch

from dsv41_amd import offload


class _Slots:
    def __init__(self, n):
        self.w13 = torch.zeros(n, 4, dtype=torch.uint8)


class _Host:
    def __init__(self, E):
        self.data = torch.arange(E * 4, dtype=torch.uint8).view(E, 4)
        self.copies = []

    def copy_to(self, slots, slot, e):
        slots.w13[slot].copy_(self.data[e])
        self.copies.append((slot, e))


class _Layer:
    def __init__(self, E, hot_ids, layer_id=0):
        self.layer_id, self.n_experts = layer_id, E
        self.hx = _Host(E)
        ex = _Slots(len(hot_ids))
        for k, e in enumerate(hot_ids):
            ex.w13[k].copy_(self.hx.data[e])
        self.hot = {"slot": {e: k for k, e in enumerate(hot_ids)}, "dummy": len(hot_ids), "ex": ex}


def _token(hc, layer, ids):
    hc.new_token()
    hc.update(layer.layer_id, ids)
    hc.drain()


def test_swaps_past_margin_and_publish_after_landing():
    layer = _Layer(16, [0, 1, 2, 3])
    hc = offload.HotCache([layer], "cpu", decay=0.9, margin=0.5, swaps_per_token=2)
    _token(hc, layer, [8, 9, 0])
    # two swaps started (budget), the victims left the map at once, the new experts are not in it yet
    assert hc.n_swaps == 2
    assert 8 not in layer.hot["slot"] and 9 not in layer.hot["slot"]
    assert 0 in layer.hot["slot"], "an expert the token uses is never evicted"
    assert len(layer.hot["slot"]) == 2
    _token(hc, layer, [8, 9, 0])      # the landed copies are published by this update
    assert {8, 9, 0} <= set(layer.hot["slot"])
    for e, s in layer.hot["slot"].items():
        assert torch.equal(layer.hot["ex"].w13[s], layer.hx.data[e]), f"slot {s} does not hold expert {e}"
    assert hc.n_hits >= 3
    assert "hit rate" in hc.stats()


def test_no_swap_inside_margin():
    layer = _Layer(16, [0, 1, 2, 3])
    hc = offload.HotCache([layer], "cpu", decay=0.97, margin=2.0, swaps_per_token=2)
    # each cold expert used once: usage 1 < 0 + 2.0 -> no eviction
    _token(hc, layer, [8])
    _token(hc, layer, [9])
    assert hc.n_swaps == 0 and set(layer.hot["slot"]) == {0, 1, 2, 3}
    # a cold expert used repeatedly overtakes the least-used resident by the margin
    for _ in range(3):
        _token(hc, layer, [8])
    assert hc.n_swaps == 1


def test_budget_and_pending_slots():
    layer = _Layer(32, [0, 1, 2, 3, 4, 5])
    hc = offload.HotCache([layer], "cpu", decay=1.0, margin=0.5, swaps_per_token=1)
    hc.new_token()
    hc.update(0, [20, 21, 22])
    assert hc.n_swaps == 1, "at most swaps_per_token copies per token"
    hc.update(0, [20, 21, 22])        # same token: budget spent
    assert hc.n_swaps == 1
    hc.drain()
    pending_before = set(hc.layers[0]["pending"])
    assert len(pending_before) == 1
    hc.new_token()
    hc.update(0, [21])                # publishes the landed copy, then may start one more
    assert not (pending_before & hc.layers[0]["pending"]), "a landed slot is no longer pending"
    usage = hc.layers[0]["usage"]
    assert np.isclose(usage[21], 3.0) and np.isclose(usage[20], 2.0)


def test_split_hot_maps_cold_to_the_dummy_slot():
    m = offload.OffloadMoE.__new__(offload.OffloadMoE)
    m.hot = {"slot": {5: 0, 7: 1}, "dummy": 2}
    gs, gw, cid, cw = m.split_hot([7, 3, 5, 9], [0.4, 0.3, 0.2, 0.1])
    assert gs == [1, 2, 0, 2] and gw == [0.4, 0.0, 0.2, 0.0] and cid == [3, 9] and cw == [0.3, 0.1]
    m.hot = None
    assert m.split_hot([1, 2], [0.5, 0.5]) == (None, None, [1, 2], [0.5, 0.5])
