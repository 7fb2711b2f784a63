"""One decoder layer's projections through ``moat_amd.layer.LayerProjections``
(Q|K|V in one launch, O, gate|up in one launch + SwiGLU -> fp16 h, down(h)),
eager and as one captured HIP graph, against the oracle: ``gemm_ref`` for
each projection and ``swiglu_ref`` -> fp16 h -> ``gemm_ref`` for the MLP
chain (``transformer_engine.mm:582-716``)."""

import numpy as np
import pytest

from oracle import superblock_oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-3


def say(msg):
    print(msg, flush=True)


def rel_err(y, ref):
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.max(np.abs(np.asarray(y, dtype=np.float64) - ref)) / np.sqrt(np.mean(ref ** 2)))


def _shapes(H, q_dim, kv_dim, inter):
    return {"q_proj": (H, q_dim), "k_proj": (H, kv_dim), "v_proj": (H, kv_dim), "o_proj": (q_dim, H),
            "gate_proj": (H, inter), "up_proj": (H, inter), "down_proj": (inter, H)}


def _records(shapes, seed):
    return {name: O.quantize_pack_a(O.synthetic_weights(K, M, 0.02, seed + 31 * i))
            for i, (name, (K, M)) in enumerate(shapes.items())}


def _check(layer, recs, shapes, n, seed, graph):
    H, q_dim, inter = layer.hidden, layer.q_dim, layer.intermediate
    x = O.synthetic_activations(n, H, seed)
    attn = O.synthetic_activations(n, q_dim, seed + 1)
    x_mlp = O.synthetic_activations(n, H, seed + 2)
    out = layer.forward(x, attn, x_mlp, graph=graph)
    got = {k: v.cpu().numpy() for k, v in out.items()}
    for name, key, inp in (("q_proj", "q", x), ("k_proj", "k", x), ("v_proj", "v", x), ("o_proj", "o", attn)):
        K, M = shapes[name]
        err = rel_err(got[key], O.gemm_ref(inp, recs[name], K, M))
        assert err <= TOL, (name, n, graph, err)
    h_ref = O.swiglu_ref(x_mlp, recs["gate_proj"], recs["up_proj"], H, inter)
    h = got["h"].astype(np.float64)
    assert out["h"].dtype.is_floating_point and got["h"].dtype == np.float16
    # fp16 output: half an ulp of each value on top of the GEMM tolerance
    bound = 2.0 ** -11 * np.abs(h_ref) + TOL * np.sqrt(np.mean(h_ref ** 2))
    assert np.all(np.abs(h - h_ref) <= bound), (n, graph, float(np.max(np.abs(h - h_ref) - bound)))
    down_ref = O.gemm_ref(h_ref.astype(np.float16), recs["down_proj"], inter, H)
    err = rel_err(got["down"], down_ref)
    assert err <= TOL, ("down", n, graph, err)


@pytest.mark.parametrize("H,q_dim,kv_dim,inter", [(2048, 2048, 256, 5632), (256, 256, 64, 512)])
def test_layer_projections_match_oracle(H, q_dim, kv_dim, inter):
    from moat_amd.layer import LayerProjections
    shapes = _shapes(H, q_dim, kv_dim, inter)
    recs = _records(shapes, 4000 + H)
    say(f"case: layer H={H} q={q_dim} kv={kv_dim} I={inter}")
    layer = LayerProjections({k: (recs[k], K, M) for k, (K, M) in shapes.items()}, max_batch=32)
    want = "strip" if H >= 2048 else "row"
    assert layer.layouts["qkv"] == want and layer.layouts["gate_up"] == want
    for n in (1, 5, 16, 32):
        say(f"case: layer H={H} n={n} eager")
        _check(layer, recs, shapes, n, 70 + n, graph=False)
        say(f"case: layer H={H} n={n} graph")
        _check(layer, recs, shapes, n, 170 + n, graph=True)
    layer.check()


def test_layer_graph_replays_read_current_inputs():
    """Replays of one captured graph, with eager GEMMs on the same stream and
    synchronisations between them: every replay equals the eager result of
    its own inputs."""
    import torch
    from moat_amd.dequant import batched_int4_matmul
    from moat_amd.layer import LayerProjections
    shapes = _shapes(2048, 2048, 256, 5632)
    recs = _records(shapes, 4100)
    layer = LayerProjections({k: (recs[k], K, M) for k, (K, M) in shapes.items()}, max_batch=16)
    n = 16
    g = layer.capture(n)
    blob = torch.from_numpy(recs["down_proj"].reshape(-1)).cuda()
    for rep in range(4):
        say(f"case: layer graph replay {rep}")
        x = O.synthetic_activations(n, 2048, 900 + rep)
        attn = O.synthetic_activations(n, 2048, 950 + rep)
        x_mlp = O.synthetic_activations(n, 2048, 990 + rep)
        eager = {k: v.clone() for k, v in layer.forward(x, attn, x_mlp, graph=False).items()}
        for t in (layer.q, layer.o, layer.h, layer.down):
            t.zero_()
        g.replay()
        torch.cuda.synchronize()
        for key, t in (("q", layer.q), ("k", layer.k), ("v", layer.v), ("o", layer.o), ("h", layer.h),
                       ("down", layer.down)):
            assert torch.equal(t[:n], eager[key]), (rep, key)
        # unrelated eager work on the default workspace between replays
        hx = torch.from_numpy(O.synthetic_activations(3, 5632, rep)).cuda()
        batched_int4_matmul(hx, blob, 5632, 2048)
        torch.cuda.synchronize()
    layer.check()


def test_layer_from_loader_layers():
    """Layers from the loader (strip order where the shape allows, the
    loader's fp16-scale rule) drive the same launches; the oracle reads the
    loader's records back in row order."""
    import torch
    from moat_amd.layer import LayerProjections
    from moat_amd.loader import ModelWeightLoader
    shapes = _shapes(2048, 2048, 256, 5632)
    loader = ModelWeightLoader(memory_budget_bytes=1 << 30)
    layers = {}
    for i, (name, (K, M)) in enumerate(shapes.items()):
        w = O.synthetic_weights(K, M, 0.02, 4200 + i)
        layers[name] = loader.load_and_repack_layer(name, torch.from_numpy(w).cuda(), keep_q=False)
        assert layers[name]["layout"] == "strip"
    recs = {name: loader.row_records(name).cpu().numpy() for name in shapes}
    layer = LayerProjections(layers, max_batch=8)
    for n in (1, 8):
        say(f"case: loader layer n={n}")
        _check(layer, recs, shapes, n, 300 + n, graph=True)
    with pytest.raises(ValueError):
        layer.forward(np.zeros((9, 2048), np.float16), np.zeros((9, 2048), np.float16),
                      np.zeros((9, 2048), np.float16))
