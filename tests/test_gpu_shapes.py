"""Other model shapes through the GPU engine and the batched prefill.

The reference engine is fixed to Qwen2-0.5B's shapes, so these small
synthetic models (tmq.model_synth) check the shape-general code paths by
consistency: the batched prefill against the one-token-at-a-time prompt,
bit for bit (logits, residual stream, greedy tokens from the KV cache), and
graph-replayed decode against eager launches.

  A  2 layers, hidden 256 (4 heads, 1 KV head), FFN 512, vocab 1000,
     layer 0 Q8_0 attn_v + Q6_K ffn_down, layer 1 Q5_0 + Q4_K
  B  3 layers, hidden 128 (2 heads, 2 KV heads), FFN 256, vocab 517
     (not a multiple of 64), Q8_0 attn_v in layer 1
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SHAPES = {
    "A": dict(n_layers=2, hidden=256, inter=512, vocab=1000, n_heads=4, n_kv_heads=1, q8_v_layers=(0,)),
    "B": dict(n_layers=3, hidden=128, inter=256, vocab=517, n_heads=2, n_kv_heads=2, q8_v_layers=(1,)),
}


@pytest.fixture(scope="module", params=sorted(SHAPES))
def small(ctx, request):
    import tmq
    from tmq import model_synth, tmacfile
    kw = SHAPES[request.param]
    print(f"[shapes] model {request.param}: {kw}", flush=True)
    m = tmq.Model(ctx, tmacfile.to_bytes(model_synth.gen_model(77, **kw)), max_seq=300)
    yield request.param, kw, m
    m.free()


def test_config(small):
    name, kw, m = small
    c = m.config
    assert (c["n_layers"], c["hidden"], c["inter"], c["vocab"]) == (kw["n_layers"], kw["hidden"], kw["inter"],
                                                                    kw["vocab"])
    assert (c["n_heads"], c["n_kv_heads"]) == (kw["n_heads"], kw["n_kv_heads"])


@pytest.mark.parametrize("n", [2, 45, 200])
def test_prefill_matches_sequential(small, n):
    name, kw, m = small
    toks = np.random.default_rng(n).integers(0, kw["vocab"], size=n).astype(np.int32)
    res = []
    for chunk in (0, 512, 64):
        print(f"[shapes] {name} n={n} chunk={chunk}", flush=True)
        m.set_prefill(chunk)
        m.prompt(toks)
        res.append((m.logits(), m.hidden(), m.generate(5)))
    for lg, h, g in res[1:]:
        assert np.array_equal(lg.view(np.uint32), res[0][0].view(np.uint32))
        assert np.array_equal(h.view(np.uint32), res[0][1].view(np.uint32))
        assert g.tolist() == res[0][2].tolist()
    assert np.isfinite(res[0][0]).all()


def test_graphs_match_eager(small):
    name, kw, m = small
    toks = np.array([3, 1, 4, 1, 5], dtype=np.int32)
    out = []
    for graphs in (True, False):
        m.set_graphs(graphs)
        m.set_prefill(0)
        m.prompt(toks)
        out.append(m.generate(12).tolist())
    m.set_graphs(True)
    assert out[0] == out[1]
