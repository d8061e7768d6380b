"""GPU parity of the batched prefill (tmq_model_set_prefill > 0: every layer
takes a chunk of prompt tokens at once, projections on int8 MFMA) against
the engine's one-token-at-a-time prompt (tmq_model_set_prefill(0)), which
is itself bit-exact with the compiled reference (test_gpu_model.py).

The reference's process_prompt (sim/tmac_gguf.cpp:1992-1997) runs one token
at a time, so the batched path must leave the same state bit for bit: the
logits of the last position, the residual stream, and the KV cache (checked
through the greedy tokens generated from it).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

MODEL_SEED = 2024


@pytest.fixture(scope="module")
def model(ctx):
    import tmq
    from tmq import model_synth, tmacfile
    print("[prefill] generating the synthetic C4 model", flush=True)
    blob = tmacfile.to_bytes(model_synth.gen_model(MODEL_SEED))
    m = tmq.Model(ctx, blob, max_seq=1024)
    del blob
    yield m
    m.free()


def run(model, tokens, chunk, gen=4):
    model.set_prefill(chunk)
    model.prompt(tokens)
    assert model.position == len(tokens)
    logits = model.logits()
    hidden = model.hidden()
    out = model.generate(gen)
    return logits, hidden, out


def prompt_of(n, seed):
    return np.random.default_rng(seed).integers(0, 151936, size=n).astype(np.int32)


# (1 token; either side of a 32-token block and of a 128-token GEMM tile)
@pytest.mark.parametrize("n", [1, 2, 31, 33, 37, 100, 127, 128, 129, 200, 257, 300, 512])
def test_prefill_matches_sequential(model, n):
    toks = prompt_of(n, 1000 + n)
    print(f"[prefill] n={n} sequential", flush=True)
    l0, h0, g0 = run(model, toks, 0)
    print(f"[prefill] n={n} batched", flush=True)
    l1, h1, g1 = run(model, toks, 512)
    assert np.array_equal(h1.view(np.uint32), h0.view(np.uint32))
    assert np.array_equal(l1.view(np.uint32), l0.view(np.uint32))
    assert g1.tolist() == g0.tolist()
    assert model.tokens(0, n).tolist() == toks.tolist()


@pytest.mark.parametrize("n, chunk", [(150, 64), (385, 128), (260, 256)])
def test_prefill_chunks(model, n, chunk):
    """chunks of 64-256 tokens, the last one ragged: later chunks attend to
    the cache the earlier ones wrote"""
    toks = prompt_of(n, 77 + n)
    print(f"[prefill] n={n} chunked {chunk} vs sequential", flush=True)
    l0, h0, g0 = run(model, toks, 0)
    l1, h1, g1 = run(model, toks, chunk)
    assert np.array_equal(h1.view(np.uint32), h0.view(np.uint32))
    assert np.array_equal(l1.view(np.uint32), l0.view(np.uint32))
    assert g1.tolist() == g0.tolist()


@pytest.fixture(scope="module")
def long_model(ctx):
    import tmq
    from tmq import model_synth, tmacfile
    print("[prefill] generating the synthetic C4 model (max_seq 3072)", flush=True)
    blob = tmacfile.to_bytes(model_synth.gen_model(MODEL_SEED))
    m = tmq.Model(ctx, blob, max_seq=3072)
    del blob
    yield m
    m.free()


@pytest.mark.parametrize("n,chunk", [(1300, 512), (3000, 1024)])
def test_prefill_long(long_model, n, chunk):
    """past 512 positions the attention keeps its scores in 2, 4 or 8
    register passes of 512 (up to the engine's 3072 positions)"""
    toks = prompt_of(n, 4000 + n)
    print(f"[prefill] n={n} sequential", flush=True)
    l0, h0, g0 = run(long_model, toks, 0)
    print(f"[prefill] n={n} batched, chunks of {chunk}", flush=True)
    l1, h1, g1 = run(long_model, toks, chunk)
    assert np.array_equal(h1.view(np.uint32), h0.view(np.uint32))
    assert np.array_equal(l1.view(np.uint32), l0.view(np.uint32))
    assert g1.tolist() == g0.tolist()


def test_prefill_then_feed(model):
    """a token fed after a batched prompt continues exactly as after a sequential one"""
    toks = prompt_of(20, 5)
    res = []
    for chunk in (0, 512):
        model.set_prefill(chunk)
        model.prompt(toks)
        model.feed(1234)
        res.append((model.logits(), model.hidden()))
    assert np.array_equal(res[0][0].view(np.uint32), res[1][0].view(np.uint32))
    assert np.array_equal(res[0][1].view(np.uint32), res[1][1].view(np.uint32))


def test_prefill_errors(model):
    import tmq
    with pytest.raises(tmq.TmqError):
        model.set_prefill(-1)


@pytest.mark.parametrize("n, chunk", [(300, 512), (150, 64)])
def test_gu_quant_paths(model, monkeypatch, n, chunk):
    """The gate/up GEMM quantises the SwiGLU rows for the down projection in
    its own epilogue (its workgroups of one token tile wait for each other's
    row maxima); TMQ_PF_GUQ=0 takes the separate act kernel instead.  Both
    leave the same bits."""
    toks = prompt_of(n, 3300 + n)
    res = {}
    for guq in ("0", "1"):
        monkeypatch.setenv("TMQ_PF_GUQ", guq)
        print(f"[prefill] n={n} chunk={chunk} TMQ_PF_GUQ={guq}", flush=True)
        res[guq] = run(model, toks, chunk)
    (l0, h0, g0), (l1, h1, g1) = res["0"], res["1"]
    assert np.array_equal(h1.view(np.uint32), h0.view(np.uint32))
    assert np.array_equal(l1.view(np.uint32), l0.view(np.uint32))
    assert g1.tolist() == g0.tolist()


@pytest.mark.parametrize("n, chunk", [(512, 512), (150, 64)])
def test_prefill_graph_replays(model, monkeypatch, n, chunk):
    """A prefill is captured once per prompt length and replayed: every
    replay (with eager decode steps and synchronisations between them)
    leaves the bits of the prefill launched one kernel at a time."""
    toks = prompt_of(n, 5200 + n)
    monkeypatch.setenv("TMQ_PF_GRAPH", "0")
    print(f"[prefill] n={n} chunk={chunk} eager", flush=True)
    l0, h0, g0 = run(model, toks, chunk)
    monkeypatch.setenv("TMQ_PF_GRAPH", "1")
    for rep in range(3):
        print(f"[prefill] n={n} chunk={chunk} graph replay {rep}", flush=True)
        l1, h1, g1 = run(model, toks, chunk)
        assert np.array_equal(h1.view(np.uint32), h0.view(np.uint32)), f"replay {rep}"
        assert np.array_equal(l1.view(np.uint32), l0.view(np.uint32)), f"replay {rep}"
        assert g1.tolist() == g0.tolist()


def test_gu_quant_wait_limit(model, monkeypatch):
    """A gate/up workgroup whose wait for its token tile runs out of polls
    (forced from the host: a limit of 0 polls) flags the prefill, which then
    fails; every kernel still ends.  The next prompt runs normally."""
    import tmq
    toks = prompt_of(100, 4100)
    monkeypatch.setenv("TMQ_PF_GUQ", "1")
    monkeypatch.setenv("TMQ_PF_GUQ_SPIN", "0")
    model.set_prefill(512)
    print("[prefill] gate/up wait limit 0", flush=True)
    with pytest.raises(tmq.TmqError, match="ran out of polls"):
        model.prompt(toks)
    monkeypatch.delenv("TMQ_PF_GUQ_SPIN")
    l0, h0, g0 = run(model, toks, 0)
    l1, h1, g1 = run(model, toks, 512)
    assert np.array_equal(h1.view(np.uint32), h0.view(np.uint32))
    assert g1.tolist() == g0.tolist()


def test_norm_sum_fallback(ctx, model, monkeypatch):
    """RMSNorm's sequential sum of squares runs in segments from speculated
    starting values, each checked against the exact end of the segment
    before it.  With TMQ_SPEC_MISS=1 at load every speculation is rejected
    and every segment re-run from its exact start: the same bits, one token
    at a time, batched, and in the decode steps after the prompt."""
    import tmq
    from tmq import model_synth, tmacfile
    toks = prompt_of(40, 4040)
    exp = {c: run(model, toks, c, gen=3) for c in (0, 512)}
    monkeypatch.setenv("TMQ_SPEC_MISS", "1")
    print("[prefill] model with every norm segment re-run", flush=True)
    blob = tmacfile.to_bytes(model_synth.gen_model(MODEL_SEED))
    m = tmq.Model(ctx, blob, max_seq=64)
    del blob
    try:
        for c in (0, 512):
            l1, h1, g1 = run(m, toks, c, gen=3)
            l0, h0, g0 = exp[c]
            assert np.array_equal(h1.view(np.uint32), h0.view(np.uint32)), f"chunk {c}"
            assert np.array_equal(l1.view(np.uint32), l0.view(np.uint32)), f"chunk {c}"
            assert g1.tolist() == g0.tolist()
    finally:
        m.free()


def test_norm_sum_mixed(ctx, monkeypatch):
    """a prompt token whose embedding row is constant (every Q8_0 block d =
    0x2e66, q = 13: 1.2997 in all 896 columns): the fp32 chain of its
    attn_norm sum of squares drifts past the 64-float window at some segment
    starts and not at others (the 4 segments of that norm, in the QKV
    prologue and the prefill act kernel: taken, re-run, taken -- checked on
    the host below), so the walk mixes taken and re-run segments.  The result must equal the
    all-re-run path (TMQ_SPEC_MISS=1) bit for bit, one token at a time and
    batched."""
    import tmq
    from tmq import model_synth, tmacfile
    tens = model_synth.gen_model(MODEL_SEED)
    emb = tens[0]
    assert emb.name == "token_embd.weight" and emb.cols == 896
    tok = 1234
    rb = (emb.cols // 32) * 34
    row = emb.data[tok * rb:(tok + 1) * rb].reshape(-1, 34)
    row[:, 0], row[:, 1] = 0x66, 0x2E
    row[:, 2:] = 13
    blob = tmacfile.to_bytes(tens)
    del tens
    # the premise, on the host: the chain's distance (in floats) from the
    # rounded fp64 prefix at each segment start is within the window for
    # some segments and outside it for others
    v = np.float32(np.float16(np.frombuffer(bytes([0x66, 0x2E]), np.float16)[0])) * np.float32(13)
    sq = np.full(896, np.float32(v) * np.float32(v), np.float32)
    chain = np.zeros(897, np.float32)
    for i in range(896):
        chain[i + 1] = np.float32(chain[i] + sq[i])
    pref = np.concatenate([[0.0], np.cumsum(sq.astype(np.float64))]).astype(np.float32)
    d = [int(chain[j].view(np.int32)) - int(pref[j].view(np.int32)) for j in (256, 512, 768)]
    inside = [-32 <= x <= 31 for x in d]
    assert any(inside) and not all(inside), d
    toks = np.array([tok, 17, 99000, 4242], dtype=np.int32)
    res = []
    for miss in ("0", "1"):
        monkeypatch.setenv("TMQ_SPEC_MISS", miss)
        print(f"[prefill] constant-embedding model, TMQ_SPEC_MISS={miss}", flush=True)
        m = tmq.Model(ctx, blob, max_seq=64)
        try:
            res.append({c: run(m, toks, c, gen=3) for c in (0, 512)})
        finally:
            m.free()
    for c in (0, 512):
        (l0, h0, g0), (l1, h1, g1) = res[0][c], res[1][c]
        assert np.array_equal(h0.view(np.uint32), h1.view(np.uint32)), f"chunk {c}"
        assert np.array_equal(l0.view(np.uint32), l1.view(np.uint32)), f"chunk {c}"
        assert g0.tolist() == g1.tolist()
    # one token at a time and batched leave the same bits as well
    (l0, h0, g0), (l1, h1, g1) = res[0][0], res[0][512]
    assert np.array_equal(h0.view(np.uint32), h1.view(np.uint32))
    assert np.array_equal(l0.view(np.uint32), l1.view(np.uint32))
    assert g0.tolist() == g1.tolist()


def chain_drift(v, seg, n=896):
    """distance in floats between the sequential fp32 sum of n squares of
    v and the fp64 prefix rounded to float, at every segment start"""
    sq = np.full(n, np.float32(v) * np.float32(v), np.float32)
    chain = np.zeros(n + 1, np.float32)
    for i in range(n):
        chain[i + 1] = np.float32(chain[i] + sq[i])
    pref = np.concatenate([[0.0], np.cumsum(sq.astype(np.float64))]).astype(np.float32)
    return [int(chain[j].view(np.int32)) - int(pref[j].view(np.int32)) for j in range(seg, n, seg)]


def test_norm_sum_mixed_ffn(ctx, monkeypatch):
    """the same constant embedding row, and layer 0's attn_output weights
    all zero (every block d = 0: the projection adds exactly 0), so the
    ffn_norm input of that token is the constant row too.  The decode
    engine sums it in the 16-wave gate/up launch as 8 segments of 128; the
    walk there mixes taken and re-run segments (premise checked on the
    host), and must leave the bits of the all-re-run path and of the batched
    prefill."""
    import tmq
    from tmq import model_synth, tmacfile
    tens = model_synth.gen_model(MODEL_SEED)
    emb = tens[0]
    tok = 1234
    rb = (emb.cols // 32) * 34
    row = emb.data[tok * rb:(tok + 1) * rb].reshape(-1, 34)
    row[:, 0], row[:, 1] = 0x66, 0x2E
    row[:, 2:] = 13
    o0 = [t for t in tens if t.name == "blk.0.attn_output.weight"][0]
    o0.data[:] = 0
    blob = tmacfile.to_bytes(tens)
    del tens
    v = np.float32(np.float16(np.frombuffer(bytes([0x66, 0x2E]), np.float16)[0])) * np.float32(13)
    inside = [-32 <= x <= 31 for x in chain_drift(v, 128)]
    assert any(inside) and not all(inside), inside
    toks = np.array([tok, 5, 151000], dtype=np.int32)
    res = []
    for miss in ("0", "1"):
        monkeypatch.setenv("TMQ_SPEC_MISS", miss)
        print(f"[prefill] zero attn_output model, TMQ_SPEC_MISS={miss}", flush=True)
        m = tmq.Model(ctx, blob, max_seq=64)
        try:
            res.append({c: run(m, toks, c, gen=3) for c in (0, 512)})
        finally:
            m.free()
    ref = res[1][0]
    for r in (res[0][0], res[0][512], res[1][512]):
        assert np.array_equal(r[1].view(np.uint32), ref[1].view(np.uint32))
        assert np.array_equal(r[0].view(np.uint32), ref[0].view(np.uint32))
        assert r[2].tolist() == ref[2].tolist()


@pytest.mark.parametrize("golden,chunk", [("model_prompt.npz", 0), ("model_prompt.npz", 512), ("model_prompt.npz", 8),
                                          ("model_prompt_long.npz", 512), ("model_prompt_long.npz", 64),
                                          ("model_prompt_long.npz", 0)])
def test_prompt_matches_reference(model, golden, chunk):
    """the compiled reference's own process_prompt (sim/tmac_gguf.cpp:
    1992-1997) over a 24-token prompt (tests/golden/model_prompt.npz) and a
    250-token one, close to its 256-position KV cache (MAX_SEQ_LEN,
    :148; model_prompt_long.npz): hidden state, logits and greedy tokens,
    one token at a time (0), in one batch (512) and in chunks (8, 64)"""
    from conftest import load_golden
    g = load_golden(golden)
    assert int(g["model_seed"]) == MODEL_SEED
    print(f"[prefill] reference prompt {golden} ({g['prompt'].size} tokens), chunk {chunk}", flush=True)
    model.set_prefill(chunk)
    model.prompt(g["prompt"])
    h = model.hidden()
    exact = np.mean(h.view(np.uint32) == g["hidden"].view(np.uint32))
    print(f"[prefill] hidden after the prompt: {exact:.4f} bit-exact", flush=True)
    assert exact == 1.0
    lg = model.logits()
    top = np.lexsort((np.arange(lg.size), -lg))[:10]
    assert top.tolist() == g["top_ids"][0].tolist()
    assert np.array_equal(lg[top].view(np.uint32), g["top_vals"][0].view(np.uint32))
    assert np.array_equal(lg[::64].view(np.uint32), g["logits_sub"].view(np.uint32))
    out = model.generate(len(g["tokens"]))
    assert out.tolist() == g["tokens"].tolist()
