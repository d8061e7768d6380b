"""GPU parity of the decode engine (tmq_model_*) against the compiled
reference engine's greedy decode of the synthetic full model
(tests/golden/model_c4.npz, written by tests/golden/gen_model_golden.py).

Bar: bit-exact.  The north star asks for greedy tokens identical and logits
within 1e-3; every fp32 operation of the engine is the reference's in the
reference's order, and expf/logf equal the host libm's on all inputs, so the
hidden states, the layer outputs and the logits are compared bit for bit.
"""
import json
import os

import numpy as np
import pytest
from conftest import load_golden

pytestmark = pytest.mark.gpu



@pytest.fixture(scope="module")
def golden():
    return load_golden("model_c4.npz")


@pytest.fixture(scope="module")
def model(ctx, golden):
    import tmq
    from tmq import model_synth, tmacfile
    print("[model] generating the synthetic C4 model", flush=True)
    blob = tmacfile.to_bytes(model_synth.gen_model(int(golden["model_seed"])))
    m = tmq.Model(ctx, blob, max_seq=512)
    del blob
    yield m
    m.free()


def test_config(model):
    c = model.config
    assert (c["n_layers"], c["hidden"], c["inter"], c["vocab"]) == (24, 896, 4864, 151936)
    assert (c["n_heads"], c["n_kv_heads"], c["head_dim"]) == (14, 2, 64)
    assert model.weight_bytes == 391573504


def test_prompt_hidden(model, golden):
    """hidden state after a one-token prompt (position 0, all 24 layers)"""
    print("[model] prompt of one token", flush=True)
    model.set_graphs(False)
    model.prompt(golden["prompt"])
    h = model.hidden()
    exp = golden["layers0"][-1]
    exact = np.mean(h.view(np.uint32) == exp.view(np.uint32))
    print(f"[model] hidden at position 0: {exact:.4f} bit-exact", flush=True)
    assert exact == 1.0


def test_layer_dump_matches(ctx, golden):
    """tmq_model_feed_dump on a fresh model: every layer's output at position 0"""
    import tmq
    from tmq import model_synth, tmacfile
    blob = tmacfile.to_bytes(model_synth.gen_model(int(golden["model_seed"])))
    m = tmq.Model(ctx, blob, max_seq=16)
    del blob
    d = m.feed(int(golden["prompt"][0]), dump=True)
    exp = golden["layers0"]
    for l in range(exp.shape[0]):
        scale = np.abs(exp[l]).max()
        err = np.abs(d[l] - exp[l]).max() / scale
        ex = np.mean(d[l].view(np.uint32) == exp[l].view(np.uint32))
        print(f"[model] layer {l}: max rel err {err:.3e}, bit-exact {ex:.4f}", flush=True)
        assert ex == 1.0, f"layer {l}: rel err {err}"
    m.free()


def test_greedy_logits_per_step(model, golden):
    """logits of every step vs the reference (top-10 ids and values, every
    64th logit at a few steps), feeding the reference's tokens"""
    model.set_graphs(True)
    model.prompt(golden["prompt"])
    toks = golden["tokens"]
    subs = {int(s): i for i, s in enumerate(golden["sub_steps"])}
    worst = 0.0
    for step in range(toks.size):
        lg = model.logits()
        ids = np.lexsort((np.arange(lg.size), -lg))[:10]
        assert int(ids[0]) == int(toks[step]), f"step {step}: token {ids[0]} != {toks[step]}"
        assert np.array_equal(lg[golden["top_ids"][step]].view(np.uint32), golden["top_vals"][step].view(np.uint32)), \
            f"step {step}: top-10 logits differ"
        worst = max(worst, float(np.abs(lg[golden["top_ids"][step]] - golden["top_vals"][step]).max()))
        if step in subs:
            ref = golden["logits_sub"][subs[step]]
            d = np.abs(lg[::64] - ref).max()
            worst = max(worst, float(d))
            assert np.array_equal(lg[::64].view(np.uint32), ref.view(np.uint32)), \
                f"step {step}: logit subsample max diff {d}"
        model.feed(int(toks[step]))
        if step % 32 == 31:
            print(f"[model] step {step}: worst logit diff so far {worst:.3e}", flush=True)
    print(f"[model] worst logit diff over {toks.size} steps: {worst:.3e}", flush=True)


def test_greedy_generate(model, golden):
    """tmq_model_generate (graph-captured decode steps): the reference's tokens"""
    model.set_graphs(True)
    model.prompt(golden["prompt"])
    got = model.generate(int(golden["tokens"].size))
    exp = golden["tokens"]
    assert np.array_equal(got, exp), f"first difference at {np.flatnonzero(got != exp)[:3]}"
    h = model.hidden()
    assert np.array_equal(h.view(np.uint32), golden["hidden_final"].view(np.uint32))
    assert model.position == 1 + exp.size


def test_graphs_match_eager(model, golden):
    """the captured step replays exactly what the eager launch sequence does"""
    n = 8
    res = []
    for graphs in (False, True):
        model.set_graphs(graphs)
        model.prompt(golden["prompt"])
        toks = model.generate(n)
        res.append((toks, model.hidden(), model.logits()))
    assert np.array_equal(res[0][0], res[1][0])
    assert np.array_equal(res[0][1].view(np.uint32), res[1][1].view(np.uint32))
    assert np.array_equal(res[0][2].view(np.uint32), res[1][2].view(np.uint32))


@pytest.mark.parametrize("max_seq", [61, 130])
def test_cache_capacity_free(ctx, golden, max_seq):
    """The attention's LDS holds the scores, weights and staged V rows of up
    to max_seq positions (16-byte aligned regions, V rows in whole 64s): a
    model whose max_seq is no multiple of 4 or 64 decodes the reference's
    greedy tokens and final state of the same steps."""
    import tmq
    from tmq import model_synth, tmacfile
    n = min(max_seq - 2, int(golden["tokens"].size))
    print(f"[model] max_seq {max_seq}: {n} greedy steps", flush=True)
    blob = tmacfile.to_bytes(model_synth.gen_model(int(golden["model_seed"])))
    m = tmq.Model(ctx, blob, max_seq=max_seq)
    del blob
    try:
        m.prompt(golden["prompt"])
        got = m.generate(n)
        assert np.array_equal(got, golden["tokens"][:n])
        if n == golden["tokens"].size:
            assert np.array_equal(m.hidden().view(np.uint32), golden["hidden_final"].view(np.uint32))
    finally:
        m.free()


def test_engine_mfma_decoders(ctx, golden, monkeypatch):
    """TMQ_ENG_MFMA=1 at load puts the engine's Q5_0 / K-quant projections on
    the int8 MFMA decoders (operand bytes written by the launch prologue,
    K chunks of whole blocks / super-blocks, each chunk adding its own
    columns' corrections): the reference's greedy tokens and the final hidden
    state bit for bit, graph replays equal to eager launches."""
    import tmq
    from tmq import model_synth, tmacfile
    monkeypatch.setenv("TMQ_ENG_MFMA", "1")
    print("[model] synthetic C4 model on the MFMA decoders", flush=True)
    blob = tmacfile.to_bytes(model_synth.gen_model(int(golden["model_seed"])))
    m = tmq.Model(ctx, blob, max_seq=512)
    del blob
    try:
        exp = golden["tokens"]
        res = []
        for graphs in (False, True):
            m.set_graphs(graphs)
            m.prompt(golden["prompt"])
            got = m.generate(int(exp.size))
            assert np.array_equal(got, exp), f"graphs {graphs}: first difference at {np.flatnonzero(got != exp)[:3]}"
            res.append(m.hidden())
            assert np.array_equal(res[-1].view(np.uint32), golden["hidden_final"].view(np.uint32))
    finally:
        m.free()


def test_errors(model, golden):
    import tmq
    with pytest.raises(tmq.TmqError):
        model.prompt(np.array([151936], dtype=np.int32))
    with pytest.raises(tmq.TmqError):
        model.prompt(np.zeros(513, dtype=np.int32))
    model.prompt(golden["prompt"])
    with pytest.raises(tmq.TmqError):
        model.generate(512)  # positions 1..512 exceed max_seq 512
    # still usable afterwards
    model.prompt(golden["prompt"])
    assert np.array_equal(model.generate(3), golden["tokens"][:3])


def test_load_errors(ctx):
    import tmq
    from tmq import tmacfile
    with pytest.raises(tmq.TmqError):
        tmq.Model(ctx, b"NOPE" + b"\0" * 64)
    with pytest.raises(tmq.TmqError):  # truncated
        tmq.Model(ctx, b"TMAC" + (5).to_bytes(8, "little"))
    # a model with only an embedding
    emb = tmacfile.TmacTensor("token_embd.weight", 64, 64, tmacfile.Q8_0, np.zeros(64 * 2 * 34, np.uint8))
    with pytest.raises(tmq.TmqError):
        tmq.Model(ctx, tmacfile.to_bytes([emb]))


def test_cli(golden, tmp_path):
    """tmq_gguf (the tmac_gguf counterpart): --generate prints the greedy
    tokens; without it, the top-10 JSON of the last prompt position"""
    import json
    import subprocess
    from conftest import PKG
    from tmq import model_synth, tmacfile
    exe = os.path.join(PKG, "tmq", "tmq_gguf")
    if not os.path.exists(exe):
        pytest.fail("tmq_gguf is not built (make -C tmac-zynq-fpga_amd)")
    path = tmp_path / "c4.tmac"
    tmacfile.write(path, model_synth.gen_model(int(golden["model_seed"])))
    prompt = f"{int(golden['prompt'][0])}\n"
    allf = ["--fpga-q8", "--fpga-q5-0", "--fpga-q4k", "--fpga-q6-k"]  # the flags of model_c4.npz
    r = subprocess.run([exe, str(path), "--generate", "16"] + allf, input=prompt,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    got = [int(t) for t in r.stdout.split()]
    assert got == golden["tokens"][:16].tolist()
    # the reference's other flag sets (tests/golden/model_flags.npz): Q4_K/Q6_K
    # through matmul_fpga_int16, and no flag at all (the FP32 loop)
    gf = load_golden("model_flags.npz")
    r = subprocess.run([exe, str(path), "--generate", "8", "--fpga-q8", "--fpga-q5-0"], input=prompt,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    assert [int(t) for t in r.stdout.split()] == gf["q8q5_tokens"][:8].tolist()
    r = subprocess.run([exe, str(path)], input=prompt, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    assert [t["id"] for t in json.loads(r.stdout)] == gf["fp32_top_ids"][0].tolist()
    trace = tmp_path / "trace.json"
    r = subprocess.run([exe, str(path), "--perf", "--trace", str(trace)] + allf, input=prompt, capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    top = json.loads(r.stdout)
    assert [t["id"] for t in top] == golden["top_ids"][0].tolist()
    assert [t["logit"] for t in top] == [round(float(v), 3) for v in golden["top_vals"][0]]
    assert "[PERF]" in r.stderr and "PIPELINE TIMING BREAKDOWN" in r.stderr and "ffn_down" in r.stderr
    ev = json.loads(trace.read_text())["traceEvents"]
    assert len(ev) in (2 * 8 * (3 + 5 * 24), 2 * 8 * (3 + 6 * 24)) and {e["ph"] for e in ev} == {"B", "E"}
    # --dump-layers: cpp_layer_0..24.bin of the (one-token) prompt, as the reference writes them
    r = subprocess.run([exe, str(path), "--dump-layers", "--dump-dir", str(tmp_path)] + allf, input=prompt,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    assert [t["id"] for t in json.loads(r.stdout)] == golden["top_ids"][0].tolist()
    exp = golden["layers0"]
    for l in range(exp.shape[0]):
        d = np.fromfile(tmp_path / f"cpp_layer_{l}.bin", dtype=np.float32)
        assert d.shape == exp[l].shape
        assert np.array_equal(d.view(np.uint32), exp[l].view(np.uint32)), f"layer {l}"


SUMMARY_RE = (r"\[FPGA TIMING SUMMARY\] \(GPU\)\n"
              r"  Tiles: (\d+)\s+MACs: (\d+)\s+GPU: ([\d.]+) ms  NAIVE: ([\d.]+) Gop/s\n"
              r"  GPU: (\d+) decode steps profiled, ([\d.]+) us of kernels per step \((\d+) tiles, (\d+) MACs\): "
              r"([\d.]+) Gop/s, ([\d.]+) GB/s of weights")


def test_cli_timing_summary(model, golden, tmp_path):
    """Any --fpga* flag prints the reference's [FPGA TIMING SUMMARY]
    (sim/fpga_sim.hpp:156-172, sim/tmac_gguf.cpp:2168-2171) with GPU figures:
    the run's tiles and MACs equal what the compiled reference's counters
    hold for the same run (tests/golden/timing.npz: per decode step and per
    logits call), NAIVE Gop/s is MACs over the run's wall time, and the
    profiled kernel time per step agrees with tmq_model_profile on the same
    model (the test's own profile of 4 steps); no flag, no summary."""
    import re
    import subprocess
    from conftest import PKG
    from tmq import model_synth, tmacfile
    gt = load_golden("timing.npz")
    exe = os.path.join(PKG, "tmq", "tmq_gguf")
    path = tmp_path / "c4.tmac"
    tmacfile.write(path, model_synth.gen_model(int(golden["model_seed"])))
    prompt = f"{int(golden['prompt'][0])}\n"
    runs = [("all", ["--fpga-q8", "--fpga-q5-0", "--fpga-q4k", "--fpga-q6-k"]), ("q8q5", ["--fpga-q8", "--fpga-q5-0"]),
            ("int16", ["--fpga"])]
    us_cli = []
    for name, fl in runs:
        print(f"[model] CLI --generate 6 {' '.join(fl)}", flush=True)
        r = subprocess.run([exe, str(path), "--generate", "6"] + fl, input=prompt, capture_output=True, text=True,
                           timeout=300)
        assert r.returncode == 0, r.stderr
        m = re.search(SUMMARY_RE, r.stderr)
        assert m, r.stderr[-2000:]
        tiles, macs, wall, naive, steps, us, st, sm, gops, gbps = m.groups()
        step, lg = gt[f"{name}_step"], gt[f"{name}_logits"]
        # one prompt position and 6 generated ones (each fed), 6 logits calls
        assert int(tiles) == 7 * int(step[0]) + 6 * int(lg[0]), name
        assert int(macs) == 7 * int(step[1]) + 6 * int(lg[1]), name
        assert int(st) == int(step[0] + lg[0]) and int(sm) == int(step[1] + lg[1]), name
        assert abs(float(naive) - int(macs) / (float(wall) * 1e-3) / 1e9) <= 0.01 * float(naive) + 0.01
        assert int(steps) == 4
        assert abs(float(gops) - int(sm) / (float(us) * 1e-6) / 1e9) <= 0.01 * float(gops) + 0.01
        assert abs(float(gbps) - model.weight_bytes / (float(us) * 1e-6) / 1e9) <= 0.01 * float(gbps) + 0.1
        if name == "all":
            us_cli.append(float(us))
    model.set_flags(31)
    model.set_graphs(True)
    model.prompt(golden["prompt"])
    prof = model.profile(4)
    us_prof = 1e3 * sum(e - s for _, s, e in prof) / 4
    print(f"[model] kernel time per step: CLI {us_cli[0]:.1f} us, tmq_model_profile {us_prof:.1f} us", flush=True)
    assert 0.7 * us_prof <= us_cli[0] <= 1.4 * us_prof
    r = subprocess.run([exe, str(path), "--generate", "2"], input=prompt, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    assert "TIMING SUMMARY" not in r.stderr


def test_cli_cosim(golden, tmp_path):
    """tmq_gguf --fpga-phaseb --dump-phaseb --dump-tiles 4 --dump-tiles-q5-0 3
    --dump-tiles-q6-k 3 on a one-token prompt against the compiled
    reference's run (tests/golden/cosim.npz): the Q8_0 dump byte for byte;
    the Q5_0 and Q6_K dumps byte for byte in every field but the results of
    the tiles after the first, which carry the values the reference's
    overflowing result array loses (q5_fixed, q6_fixed); tb_phaseb.bin and
    .hdr identical (sha256); the same verification outcome."""
    import hashlib
    import subprocess
    from conftest import PKG
    from tmq import model_synth, tmacfile
    gc = load_golden("cosim.npz")
    exe = os.path.join(PKG, "tmq", "tmq_gguf")
    path = tmp_path / "c4.tmac"
    tmacfile.write(path, model_synth.gen_model(int(gc["model_seed"])))
    out = tmp_path / "cosim"
    out.mkdir()
    print("[model] CLI with --fpga-phaseb and the tile dumps", flush=True)
    r = subprocess.run([exe, str(path), "--fpga-phaseb", "--dump-phaseb", "--dump-tiles", "4", "--dump-tiles-q5-0", "3",
                        "--dump-tiles-q6-k", "3", "--cosim-dir", str(out)], input=f"{int(gc['prompt'][0])}\n",
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-3000:]
    assert [t["id"] for t in json.loads(r.stdout)] == golden["top_ids"][0].tolist()
    assert f"156 descriptors verified, {int(gc['phaseb_errors'])} errors" in r.stderr
    q8 = np.fromfile(out / "cosim_tiles.bin", dtype=np.uint8)
    assert np.array_equal(q8, gc["q8"])
    for k, rec, res_off, fixed in (("q5", 6816, 6752, gc["q5_fixed"]), ("q6", 7616, 7360, gc["q6_fixed"])):
        fn = "cosim_tiles_q5_0.bin" if k == "q5" else "cosim_tiles_q6_k.bin"
        got, exp = np.fromfile(out / fn, dtype=np.uint8), gc[k]
        assert got.size == exp.size and np.array_equal(got[:16 + rec], exp[:16 + rec])
        for t in range(1, 3):
            a, b = got[16 + t * rec: 16 + (t + 1) * rec], exp[16 + t * rec: 16 + (t + 1) * rec]
            assert np.array_equal(a[:res_off], b[:res_off]), f"{k} tile {t}"
            assert np.array_equal(a[res_off:].view(np.int64), fixed[t]), f"{k} tile {t} results"
    for name, key in (("tb_phaseb.bin", "bin"), ("tb_phaseb.hdr", "hdr")):
        data = (out / name).read_bytes()
        assert len(data) == int(gc[f"{key}_size"])
        if key == "hdr":
            assert np.array_equal(np.frombuffer(data[:gc["hdr_head"].size], np.uint8), gc["hdr_head"])
        assert hashlib.sha256(data).hexdigest() == str(gc[f"{key}_sha256"]), name


def test_profile(model, golden):
    """tmq_model_profile: every launch of n decode steps, in order, with the
    same greedy tokens as the graph-replayed generate"""
    model.set_graphs(True)
    model.prompt(golden["prompt"])
    prof = model.profile(3)
    names = [p[0] for p in prof]
    # 5 launches per layer when gate/up finish SwiGLU themselves, 6 with a separate silu_x_up
    per_layer = 6 if "silu_x_up" in names else 5
    assert len(prof) == 3 * (3 + per_layer * 24)
    assert names[:4] == ["output_norm+logits", "argmax", "zero_acc", "embedding+attn_norm+qkv"]
    assert names.count("rope+attention") == 3 * 24 and names.count("ffn_down") == 3 * 24
    starts = [p[1] for p in prof]
    assert starts == sorted(starts) and all(e >= s for _, s, e in prof)
    assert model.position == 4
    assert model.tokens(1, 3).tolist() == golden["tokens"][:3].tolist()
