"""Single-GPU expert offload (offload.OffloadMoE / HotCache / OffloadDecodeRuntime, the reference's model.py:455-552,
hotcache.py, decode.py:534-795) against the oracle: the gather path and the chunked prefill path equal the all-GPU
layer's oracle; the hot/cold split equals the oracle's GPU part (hot pairs) plus the host library's oracle (cold pairs,
int8 mode); hot-cache swaps land the right bytes in the right slots; the graph-captured runtime equals its eager
form."""
import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from test_gpu_moe import DEV, RTOL_L2, MAXABS_RMS, bf16_vals, close, host_subset, make_experts, rand_x, to_ex

pytestmark = pytest.mark.gpu
E, H, I, K = 16, 1024, 384, 4   # I >= 384: the prefill kernels stream I in 128-k steps, 3 in flight
LIMIT = 10.0


def u16(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.fixture(scope="module")
def layer_weights():
    ws = make_experts(E, H, I, 4242)
    g = torch.Generator(device=DEV).manual_seed(4243)
    gate_w = torch.randn(E, H, generator=g, device=DEV) / H ** 0.5
    bias = torch.randn(E, generator=g, device=DEV) * 0.05
    Ws13 = (torch.randn(2 * I, H, generator=g, device=DEV) / H ** 0.5).to(torch.bfloat16)
    Ws2 = (torch.randn(H, I, generator=g, device=DEV) / I ** 0.5).to(torch.bfloat16)
    return ws, gate_w, bias, Ws13, Ws2


def host_lib(ws):
    from dsv41_amd import cpumoe
    w13, s13, w2, s2 = [w.cpu() for w in ws]
    he = cpumoe.HostExperts(E, I, H)
    he.load_layer([w13[e, :I] for e in range(E)], [w13[e, I:] for e in range(E)], [s13[e, :I] for e in range(E)],
                  [s13[e, I:] for e in range(E)], [w2[e] for e in range(E)], [s2[e] for e in range(E)])
    return he


def make_layer(layer_weights, host=None, hot_ids=None, shared=True, layer_id=0):
    from dsv41_amd import offload
    ws, gate_w, bias, Ws13, Ws2 = layer_weights
    hx = offload.HostExpertWeights.of(to_ex(*ws, True))
    return offload.OffloadMoE(hx, gate_w, bias, topk=K, score_func="sigmoid", route_scale=2.5, swiglu_limit=LIMIT,
                              sh_w13=Ws13 if shared else None, sh_w2=Ws2 if shared else None, host=host, hot_ids=hot_ids,
                              device=DEV, layer_id=layer_id)


def oracle_layer(layer_weights, x, eid, wt, shared=True):
    ws, _, _, Ws13, Ws2 = layer_weights
    W13, S13, W2, S2 = host_subset(ws, set(eid.reshape(-1).tolist()))
    return O.moe_layer(bf16_vals(x), eid, wt, W13, S13, W2, S2, u16(Ws13) if shared else None, u16(Ws2) if shared else None, I, LIMIT)


def check_bf16_layer(got, ref, what):
    rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
    print(f"{what}: rel L2 {O.rel_l2(got, ref):.2e}")
    assert O.rel_l2(got, ref) <= RTOL_L2, what
    assert np.all(np.abs(got - ref) <= MAXABS_RMS * rms + np.abs(ref) * 2.0 ** -7), what


@pytest.mark.parametrize("T", [1, 3, 16])
def test_decode_offload_gather(layer_weights, T):
    """No host library: the selected experts are gathered into staging slots and the decode launches run on them."""
    layer = make_layer(layer_weights)
    x = (rand_x(T, H, 500 + T) * 2).to(DEV)
    y = layer(x).clone()
    eid, wt = [t.cpu().numpy() for t in layer.last_routing]
    check_bf16_layer(bf16_vals(y), oracle_layer(layer_weights, x, eid, wt), f"gather T={T}")


@pytest.mark.parametrize("chunk", [64, 5])
def test_prefill_offload(layer_weights, chunk):
    """40 tokens: the experts stream through staging in chunks (5: four chunks, the last one short)."""
    from dsv41_amd import quant
    layer = make_layer(layer_weights, shared=False)
    T = 40
    x = (rand_x(T, H, 600) * 2).to(DEV)
    wt, eid = layer.gate(x)
    xq = quant.fake_quant_fp8(x)
    y = layer._prefill_offload(xq, eid, wt, chunk=chunk)
    ws = layer_weights[0]
    e, w = eid.cpu().numpy(), wt.cpu().numpy()
    W13, S13, W2, S2 = host_subset(ws, set(e.reshape(-1).tolist()))
    close(y.cpu().numpy(), O.moe_layer_routed(bf16_vals(xq), e, w, W13, S13, W2, S2, I, LIMIT), f"prefill offload chunk={chunk}")
    if chunk == 64:
        out = layer(x)   # the __call__ path (> 16 tokens)
        eid2, wt2 = [t.cpu().numpy() for t in layer.last_routing]
        check_bf16_layer(bf16_vals(out), oracle_layer(layer_weights, x, eid2, wt2, shared=False), "prefill offload __call__")


def hot_cold_ref(ws, xq, eid, wt, hot_ids):
    """The oracle of the split: the hot pairs through the GPU path's oracle, the cold ones through the host library's
    (int8 mode), added."""
    hot_mask = np.array([e in hot_ids for e in eid[0]])
    w13, s13, w2, s2 = [w.cpu().numpy() for w in ws]
    ref = np.zeros(H, np.float64)
    if hot_mask.any():
        ref += O.moe_layer_routed(bf16_vals(xq), eid[:, hot_mask], wt[:, hot_mask], w13, s13, w2, s2, I, LIMIT)[0]
    if (~hot_mask).any():
        _, _, out = O.host_layer(bf16_vals(xq)[0], eid[0, ~hot_mask].tolist(), wt[0, ~hot_mask].tolist(), w13, s13, w2, s2, I, LIMIT)
        ref += out
    return ref.astype(np.float32)


@pytest.mark.parametrize("hot", ["mixed", "all_hot", "all_cold"])
def test_decode_cpu_hot_cold(layer_weights, hot):
    """One token: the hot pairs on the GPU slot table and the cold pairs on the host library at the same time."""
    from dsv41_amd import quant
    ws = layer_weights[0]
    he = host_lib(ws)
    hot_ids = {"mixed": [0, 2, 4, 6, 8, 10, 12, 14], "all_hot": list(range(E)), "all_cold": []}[hot]
    layer = make_layer(layer_weights, host=he, hot_ids=hot_ids, shared=False)
    x = (rand_x(1, H, 700) * 2).to(DEV)
    xq = quant.fake_quant_fp8(x)
    eid = np.array([[3, 8, 11, 0]], np.int32)
    wt = np.array([[0.4, 0.3, 0.2, 0.1]], np.float32)
    y = layer._decode_cpu(xq, torch.from_numpy(eid).to(DEV), torch.from_numpy(wt).to(DEV)).cpu().numpy()[0]
    close(y, hot_cold_ref(ws, xq, eid, wt, hot_ids), f"hot/cold {hot}")
    # through __call__: the gate on the GPU, then the split; bf16 output
    out = layer(x)
    e2, w2 = [t.cpu().numpy() for t in layer.last_routing]
    check_bf16_layer(bf16_vals(out), O.bf16_round(hot_cold_ref(ws, xq, e2, w2, hot_ids)), f"hot/cold {hot} __call__")
    he.close()


def test_hot_cache_swaps(layer_weights):
    """A layer whose tokens keep choosing cold experts: the cache moves them into slots (the slot bytes are those
    experts' bytes), the hit rate rises, and the results still equal the oracle."""
    from dsv41_amd import offload, quant
    ws = layer_weights[0]
    he = host_lib(ws)
    layer = make_layer(layer_weights, host=he, hot_ids=[0, 1, 2, 3], shared=False)
    hc = offload.HotCache([layer], DEV, decay=0.9, margin=0.5, swaps_per_token=2)
    layer.hotcache = hc
    x = (rand_x(1, H, 800) * 2).to(DEV)
    xq = quant.fake_quant_fp8(x)
    eid = torch.tensor([[8, 9, 10, 11]], dtype=torch.int32, device=DEV)
    wt = torch.tensor([[0.25, 0.25, 0.25, 0.25]], dtype=torch.float32, device=DEV)
    for _ in range(6):
        hc.new_token()
        layer._decode_cpu(xq, eid, wt)
        hc.drain()
    smap = layer.hot.resident()
    assert {8, 9, 10, 11} <= set(smap), f"slot map {smap}"
    ex = to_ex(*ws, True)
    for e, s in smap.items():
        for name in ("w13", "s13", "w2", "s2"):
            assert torch.equal(getattr(layer.hot.ex, name)[s], getattr(ex, name)[e]), f"slot {s} does not hold expert {e}"
    assert hc.n_swaps >= 4 and hc.n_hits > 0
    print(hc.stats())
    w13, s13, w2, s2 = [w.cpu().numpy() for w in ws]
    ref = O.moe_layer_routed(bf16_vals(xq), eid.cpu().numpy(), wt.cpu().numpy(), w13, s13, w2, s2, I, LIMIT)
    close(layer._decode_cpu(xq, eid, wt).cpu().numpy(), ref, "all hot after swaps")
    he.close()


@pytest.mark.parametrize("cpu", [True, False])
def test_offload_runtime_graphs_equal_eager(layer_weights, cpu):
    """Two offload layers run by OffloadDecodeRuntime: captured graphs replay to the same bytes as the eager parts,
    token after token; one step equals the layers called one after another."""
    from dsv41_amd import offload
    ws = layer_weights[0]
    hes = [host_lib(ws), host_lib(ws)] if cpu else [None, None]
    layers = [make_layer(layer_weights, host=hes[i], hot_ids=[0, 1, 2, 3, 4, 5] if cpu else None, layer_id=i) for i in range(2)]
    eager = offload.OffloadDecodeRuntime(layers, use_graphs=False)
    graphs = offload.OffloadDecodeRuntime(layers, use_graphs=True)
    graphs.capture()
    for t in range(3):
        x = (rand_x(1, H, 900 + t) * 2).to(DEV)
        a = eager.step(x).clone()
        b = graphs.step(x).clone()
        assert torch.equal(a, b), f"token {t}"
    if not cpu:
        # a step is the two layers applied in turn (gather path)
        x = (rand_x(1, H, 950) * 2).to(DEV)
        y = eager.step(x).clone()
        ref = layers[1](layers[0](x))
        check_bf16_layer(bf16_vals(y), bf16_vals(ref), "runtime step vs layer calls")
    for he in hes:
        if he is not None:
            he.close()
