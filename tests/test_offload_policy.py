"""HotCache's policy on the host (hotcache.py:18-121): decayed use counts, eviction only past the margin, at most
swaps_per_token copies per token, experts the token uses never evicted, slots off-limits until their copy lands, and
the slot map published only after landing. The copies here are CPU tensor copies; on the GPU they are host -> device
DMAs on the cache's own stream (tests/test_gpu_offload.py)."""
import numpy as np
import pytest
import torch

from dsv41_amd import offload


class _Slots:
    def __init__(self, n):
        self.w13 = torch.zeros(n, 4, dtype=torch.uint8)


class _Host:
    """Stands in for HostExpertWeights: expert e's bytes are 4e .. 4e + 3."""

    def __init__(self, E):
        self.E = E
        self.data = torch.arange(E * 4, dtype=torch.uint8).view(E, 4)
        self.copies = []

    def empty_slots(self, n, device):
        return _Slots(n)

    def copy_to(self, slots, slot, e):
        slots.w13[slot].copy_(self.data[e])
        self.copies.append((slot, e))


class _Layer:
    def __init__(self, E, hot_ids, layer_id=0):
        self.layer_id, self.n_experts = layer_id, E
        self.hx = _Host(E)
        self.hot = offload.SlotTable(self.hx, hot_ids, "cpu")


def _token(hc, layer, ids):
    hc.new_token()
    hc.update(layer.layer_id, ids)
    hc.drain()


def test_swaps_past_margin_and_publish_after_landing():
    layer = _Layer(16, [0, 1, 2, 3])
    hc = offload.HotCache([layer], "cpu", decay=0.9, margin=0.5, swaps_per_token=2)
    _token(hc, layer, [8, 9, 0])
    # two swaps started (budget), the victims left the map at once, the new experts are not in it yet
    res = layer.hot.resident()
    assert hc.n_swaps == 2
    assert 8 not in res and 9 not in res
    assert 0 in res, "an expert the token uses is never evicted"
    assert len(res) == 2
    _token(hc, layer, [8, 9, 0])      # the landed copies are published by this update
    res = layer.hot.resident()
    assert {8, 9, 0} <= set(res)
    for e, s in res.items():
        assert torch.equal(layer.hot.ex.w13[s], layer.hx.data[e]), f"slot {s} does not hold expert {e}"
        assert layer.hot.slot_of[e] == s
    assert hc.n_hits >= 3
    assert "hit rate" in hc.stats()


def test_no_swap_inside_margin():
    layer = _Layer(16, [0, 1, 2, 3])
    hc = offload.HotCache([layer], "cpu", decay=0.97, margin=2.0, swaps_per_token=2)
    # each cold expert used once: use 1 < 0 + 2.0 -> no eviction
    _token(hc, layer, [8])
    _token(hc, layer, [9])
    assert hc.n_swaps == 0 and set(layer.hot.resident()) == {0, 1, 2, 3}
    # a cold expert used repeatedly overtakes the least-used resident by the margin: 1 + .97 + .97^2 > 2
    for _ in range(3):
        _token(hc, layer, [8])
    assert hc.n_swaps == 1


def test_budget_and_pending_slots():
    layer = _Layer(32, [0, 1, 2, 3, 4, 5])
    hc = offload.HotCache([layer], "cpu", decay=1.0, margin=0.5, swaps_per_token=1)
    hc.new_token()
    hc.update(0, [20, 21, 22])
    assert hc.n_swaps == 1, "at most swaps_per_token copies per token"
    loading_before = set(hc.state[0]["loading"])
    assert len(loading_before) == 1
    assert all(layer.hot.holder[s] == -1 for s in loading_before), "a slot being rewritten holds no expert"
    hc.drain()
    hc.update(0, [20, 21, 22])        # same token: budget spent; the landed copy is published
    assert hc.n_swaps == 1
    assert not (loading_before & set(hc.state[0]["loading"])), "a landed slot is no longer loading"
    assert 20 in layer.hot.resident()
    hc.new_token()
    hc.update(0, [21])                # may start one more
    heat = hc.state[0]["heat"]
    assert np.isclose(heat[21], 3.0) and np.isclose(heat[20], 2.0)


def test_heat_is_the_decayed_count():
    """heat(e) = sum over the tokens that used e of decay^(age); the lazily scaled form equals the direct sum, also
    across renormalisations."""
    h = offload._Heat(4, 0.5)
    direct = np.zeros(4)
    rng = np.random.default_rng(3)
    for _ in range(600):        # 0.5^600 is far below the renormalisation point
        ids = rng.choice(4, size=2, replace=False)
        h.tick(ids)
        direct *= 0.5
        direct[ids] += 1.0
        assert np.allclose([h[e] for e in range(4)], direct, rtol=1e-12, atol=1e-300)


def _reference_rule(usage, holder, ids, margin, budget):
    """The policy stated one swap at a time: while budget remains, the hottest cold expert of the token replaces the
    coldest resident expert the token does not use (lowest slot among equals), if it beats it by the margin."""
    holder = holder.copy()
    swaps = []
    cold = [e for e in dict.fromkeys(ids) if e not in set(holder.tolist())]
    for e in sorted(cold, key=lambda e: -usage[e]):
        if budget <= 0:
            break
        cand = [(usage[holder[s]], s) for s in range(len(holder)) if holder[s] >= 0 and holder[s] not in ids]
        if not cand:
            break
        u, s = min(cand)
        if usage[e] < u + margin:
            break
        swaps.append((s, e))
        holder[s] = -1
        budget -= 1
    return swaps


@pytest.mark.parametrize("seed", range(5))
def test_greedy_pairing_equals_one_swap_at_a_time(seed):
    """The sorted pairing of contenders and victims picks the same (slot, expert) swaps as applying the rule one swap
    at a time, over random traces (the copies publish at once here: drain + next update)."""
    rng = np.random.default_rng(seed)
    E, n, k = 24, 6, 4
    layer = _Layer(E, list(rng.choice(E, n, replace=False)))
    hc = offload.HotCache([layer], "cpu", decay=0.9, margin=0.7, swaps_per_token=2)
    zipf = 1.0 / np.arange(1, E + 1) ** 1.2
    zipf /= zipf.sum()
    for t in range(60):
        ids = [int(e) for e in rng.choice(E, k, replace=False, p=zipf)]
        hc.new_token()
        hc._publish(hc.state[0])
        heat = hc.state[0]["heat"]
        usage = {e: heat[e] * 0.9 + (1.0 if e in ids else 0.0) for e in range(E)}
        want = _reference_rule(usage, layer.hot.holder, ids, 0.7, 2)
        before = len(layer.hx.copies)
        hc.update(0, ids)
        got = [(s, e) for s, e in layer.hx.copies[before:]]
        assert got == want, f"token {t}: {got} != {want}"
        hc.drain()


def test_split_hot_maps_cold_to_the_dummy_slot():
    m = offload.OffloadMoE.__new__(offload.OffloadMoE)
    m.hot = offload.SlotTable(_Host(16), [5, 7], "cpu")
    gs, gw, cid, cw = m.split_hot([7, 3, 5, 9], [0.4, 0.3, 0.2, 0.1])
    assert gs == [1, 2, 0, 2] and cid == [3, 9]
    assert np.allclose(gw, [0.4, 0.0, 0.2, 0.0]) and np.allclose(cw, [0.3, 0.1])
    m.hot = None
    assert m.split_hot([1, 2], [0.5, 0.5]) == (None, None, [1, 2], [0.5, 0.5])
