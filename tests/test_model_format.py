"""CPU tests of the .tmac container, the synthetic model generator and the
whole-model golden fixture (no GPU)."""
import io
import os

import numpy as np
import pytest
from conftest import GOLDEN, load_golden
from tmq import model_synth, synth, tmacfile


def small_model(seed=5):
    return model_synth.gen_model(seed, n_layers=2, hidden=128, inter=256, vocab=96, n_heads=2, n_kv_heads=1,
                                 q8_v_layers=(1,))


def test_roundtrip():
    ts = small_model()
    blob = tmacfile.to_bytes(ts)
    back = tmacfile.read(blob)
    n_q8 = sum(t.type == tmacfile.Q8_0 for t in ts)
    assert len(back) == len(ts) + n_q8
    for a, b in zip(ts, back):
        assert (a.name, a.rows, a.cols, a.type) == (b.name, b.rows, b.cols, b.type)
        assert np.array_equal(a.data, b.data)
    # the aux tensors follow, in order, rows x 1 F32
    aux = back[len(ts):]
    q8 = [t for t in ts if t.type == tmacfile.Q8_0]
    for t, a in zip(q8, aux):
        assert a.name == t.name + "_row_max_abs" and (a.rows, a.cols, a.type) == (t.rows, 1, tmacfile.F32)


def test_header_bytes():
    """field order and widths of scripts/extract_tmac.py:264-273"""
    t = tmacfile.TmacTensor("ab", 3, 1, tmacfile.F32, np.arange(12, dtype=np.uint8))
    blob = tmacfile.to_bytes([t])
    exp = b"TMAC" + (1).to_bytes(8, "little") + (2).to_bytes(8, "little") + b"ab" + \
        (3).to_bytes(8, "little") + (1).to_bytes(8, "little") + (0).to_bytes(4, "little") + \
        (12).to_bytes(8, "little") + bytes(range(12))
    assert blob == exp


def test_row_max_abs_matches_oracle(oracle):
    w = synth.gen_weights(synth.Q8_0, 40, 96, 3)
    got = tmacfile.q8_row_max_abs(w, 40, 96)
    exp = oracle.row_max_abs_q8(w, 40, 96)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


@pytest.mark.parametrize("blob", [
    b"", b"TMA", b"XMAC" + bytes(8),
    b"TMAC" + (1).to_bytes(8, "little"),                                       # truncated entry
    b"TMAC" + (1).to_bytes(8, "little") + (10 ** 6).to_bytes(8, "little"),      # absurd name length
    b"TMAC" + (1).to_bytes(8, "little") + (1).to_bytes(8, "little") + b"a" + bytes(20) + (99).to_bytes(8, "little"),
])
def test_parse_errors(blob):
    with pytest.raises(ValueError):
        tmacfile.read(blob)


def test_file_path(tmp_path):
    ts = small_model(9)
    p = tmp_path / "m.tmac"
    n = tmacfile.write(p, ts)
    assert os.path.getsize(p) == n
    back = tmacfile.read(str(p))
    assert back[0].name == "token_embd.weight" and np.array_equal(back[0].data, ts[0].data)


def test_generator_layout():
    ts = model_synth.gen_model(2024)
    names = [t.name for t in ts]
    assert len(ts) == 1 + 24 * 12 + 1
    by = {t.name: t for t in ts}
    assert (by["token_embd.weight"].rows, by["token_embd.weight"].cols) == (151936, 896)
    for layer in range(24):
        big = layer in model_synth.QWEN_Q8_V_LAYERS
        assert by[f"blk.{layer}.attn_v.weight"].type == (tmacfile.Q8_0 if big else tmacfile.Q5_0)
        assert by[f"blk.{layer}.ffn_down.weight"].type == (tmacfile.Q6_K if big else tmacfile.Q4_K)
        for n in ("attn_q", "attn_k", "attn_output", "ffn_gate", "ffn_up"):
            assert by[f"blk.{layer}.{n}.weight"].type == tmacfile.Q5_0
        assert by[f"blk.{layer}.attn_k.weight"].rows == 128
        assert by[f"blk.{layer}.ffn_down.weight"].cols == 4864
    assert names[-1] == "output_norm.weight"
    # bytes streamed per token (391 573 504: 246 930 432 layers + 144 643 072 logits)
    assert model_synth.weight_bytes(ts) == 391573504
    assert by["token_embd.weight"].n_bytes == 144643072


def test_generator_deterministic():
    a, b = small_model(11), small_model(11)
    c = small_model(12)
    assert all(np.array_equal(x.data, y.data) for x, y in zip(a, b))
    assert not all(np.array_equal(x.data, y.data) for x, y in zip(a, c))


def test_golden_model_fixture():
    if not os.path.exists(os.path.join(GOLDEN, "model_c4.npz")):
        pytest.skip("model_c4.npz not generated")
    g = load_golden("model_c4.npz")
    n = g["tokens"].size
    assert n == 128 and g["top_ids"].shape == (n, 10) and g["layers0"].shape == (25, 896)
    assert np.array_equal(g["top_ids"][:, 0], g["tokens"])
    assert np.all(np.diff(g["top_vals"], axis=1) <= 0)
    assert np.all(g["gap"] >= 0)
    assert 0 <= int(g["prompt"][0]) < 151936
    # the first layer input is the Q8_0 embedding row of the prompt token (exact)
    emb = model_synth.gen_model(int(g["model_seed"]), n_layers=0)[0]
    row = emb.data.reshape(151936, 28, 34)[int(g["prompt"][0])]
    d = row[:, 0:2].copy().view(np.float16).astype(np.float32)
    q = row[:, 2:].view(np.int8).astype(np.float32)
    assert np.array_equal((q * d).reshape(-1).view(np.uint32), g["layers0"][0].view(np.uint32))


def test_golden_prompt_fixture():
    """tests/golden/model_prompt.npz (the reference's process_prompt over 24
    seeded tokens): structure, the seeds it records, and self-consistency"""
    import numpy as np
    from conftest import load_golden
    g = load_golden("model_prompt.npz")
    assert int(g["model_seed"]) == 2024
    exp = np.random.Generator(np.random.PCG64(11)).integers(0, 151936, size=24)
    assert g["prompt"].tolist() == exp.tolist()
    assert g["hidden"].shape == (896,) and np.isfinite(g["hidden"]).all()
    assert g["top_ids"].shape == (9, 10) and g["top_vals"].shape == (9, 10)
    assert g["logits_sub"].shape == (len(range(0, 151936, 64)),)
    assert g["tokens"].shape == (8,)
    # greedy: each generated token is the best of the step before it
    assert g["tokens"].tolist() == g["top_ids"][:8, 0].tolist()
    assert (np.diff(g["top_vals"], axis=1) <= 0).all()
    # a top-10 logit at a multiple of 64 is also in the every-64th sample
    for i, v in zip(g["top_ids"][0], g["top_vals"][0]):
        if i % 64 == 0:
            assert g["logits_sub"][i // 64] == v


def test_timing_counts_match_reference():
    """tmq_matmul_tiles (host only) counts the tiles and MACs the reference's
    matmul_fpga_* add to its [FPGA TIMING SUMMARY] (sim/fpga_sim.hpp:148-174):
    summed over the synthetic C4 model's matmuls of one decode step and one
    logits call, under every flag set of tests/golden/timing.npz (written by
    the compiled reference, tests/golden/gen_timing_golden.py)."""
    import tmq
    from tmq import model_synth
    g = load_golden("timing.npz")
    spec = model_synth.matmul_shapes()
    for key in g.files:
        if not key.endswith("_flags"):
            continue
        name, flags = key[:-6], int(g[key])
        step = np.zeros(2, dtype=np.int64)
        for qt, rows, cols in spec["layers"]:
            step += tmq.matmul_tiles(qt, flags, rows, cols)
        qt, rows, cols = spec["logits"]
        lg = np.array(tmq.matmul_tiles(qt, flags, rows, cols), dtype=np.int64)
        assert step.tolist() == g[f"{name}_step"].tolist(), name
        assert lg.tolist() == g[f"{name}_logits"].tolist(), name
