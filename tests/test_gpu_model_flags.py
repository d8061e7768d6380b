"""GPU parity of the decode engine under the reference's other --fpga* flag
sets (tmq_model_set_flags) against the compiled reference engine run with
the same flags (tests/golden/model_flags.npz, gen_model_flags_golden.py):

  q8q5   --fpga-q8 --fpga-q5-0: Q4_K/Q6_K ffn_down through matmul_fpga_int16
  int16  --fpga: every projection and the logits through matmul_fpga_int16
  fp32   no flag: the FP32 loop of matmul everywhere (get_logits)

Bar: bit-exact (the north star asks for identical greedy tokens and top-10
logits within 1e-3): the hidden states after every layer of position 0, the
top-10 logits of every step, every 64th logit of the first step and the final
hidden state are compared bit for bit."""
import numpy as np
import pytest
from conftest import load_golden

pytestmark = pytest.mark.gpu



@pytest.fixture(scope="module")
def golden():
    return load_golden("model_flags.npz")


@pytest.fixture(scope="module")
def blob(golden):
    from tmq import model_synth, tmacfile
    print("[flags] generating the synthetic C4 model", flush=True)
    return tmacfile.to_bytes(model_synth.gen_model(int(golden["model_seed"])))


@pytest.mark.parametrize("name", ["q8q5", "int16", "fp32"])
def test_flags_decode(ctx, golden, blob, name):
    import tmq
    flags = int(golden[f"{name}_flags"])
    print(f"[flags] {name} (flags {flags:#x}): position 0 with layer dump", flush=True)
    m = tmq.Model(ctx, blob, max_seq=64)
    try:
        m.set_flags(flags)
        assert m.flags == flags
        layers = m.feed(int(golden["prompt"][0]), dump=True)
        exp = golden[f"{name}_layers0"]
        exact = np.mean(layers.view(np.uint32) == exp.view(np.uint32))
        print(f"[flags] {name}: layer dumps {exact:.4f} bit-exact", flush=True)
        for l in range(exp.shape[0]):
            assert np.array_equal(layers[l].view(np.uint32), exp[l].view(np.uint32)), f"layer {l}"
        toks = golden[f"{name}_tokens"]
        for step in range(toks.size):
            lg = m.logits()
            top = np.lexsort((np.arange(lg.size), -lg))[:10]
            assert top.tolist() == golden[f"{name}_top_ids"][step].tolist(), f"step {step}"
            assert np.array_equal(lg[top].view(np.uint32), golden[f"{name}_top_vals"][step].view(np.uint32)), \
                f"step {step}"
            if step == 0:
                assert np.array_equal(lg[::64].view(np.uint32), golden[f"{name}_logits_sub"].view(np.uint32))
            out = m.generate(1)
            assert int(out[0]) == int(toks[step]), f"step {step}"
        h = m.hidden()
        hf = golden[f"{name}_hidden_final"]
        assert np.array_equal(h.view(np.uint32), hf.view(np.uint32))
    finally:
        m.free()


def test_flags_graphs_and_switch(ctx, golden, blob):
    """graph replay after switching flags back and forth gives the eager
    tokens of each set; the default (all four flags) is restored intact"""
    import tmq
    m = tmq.Model(ctx, blob, max_seq=64)
    try:
        assert m.flags == tmq.FLAGS_ALL
        tok = golden["prompt"]
        m.set_flags(int(golden["q8q5_flags"]))
        m.set_graphs(True)
        m.prompt(tok)
        assert m.generate(4).tolist() == golden["q8q5_tokens"][:4].tolist()
        m.set_flags(tmq.FLAGS_ALL)
        m.prompt(tok)
        g = load_golden("model_c4.npz")
        assert m.generate(4).tolist() == g["tokens"][:4].tolist()
        with pytest.raises(tmq.TmqError):
            m.set_flags(64)
        assert m.flags == tmq.FLAGS_ALL
    finally:
        m.free()
