"""Oracle vs the reference's own sim/ sources compiled in place (oracle/_ref).

CPU only; skipped where the reference tree (and so oracle/_ref) is absent,
e.g. on the GPU box.  Random seeded inputs at the BASELINE shapes plus the
corner cases the arithmetic has.
"""
import numpy as np
import pytest
from oracle import Q4_K, Q5_0, Q6_K, Q8_0
from tmq import synth


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("qt,rows,cols", [
    (Q5_0, 896, 896), (Q5_0, 128, 896), (Q5_0, 4864, 896),
    (Q4_K, 896, 4864), (Q6_K, 896, 4864), (Q4_K, 56, 256), (Q6_K, 32, 256),
    (Q8_0, 128, 896), (Q8_0, 2048, 896), (Q8_0, 64, 4864),
])
@pytest.mark.parametrize("seed", [0, 1])
def test_oracle_vs_reference_matmul(oracle, reference, qt, rows, cols, seed):
    w = synth.gen_weights(qt, rows, cols, 1000 + seed)
    x = synth.gen_x(cols, 2000 + seed)
    assert np.array_equal(bits(oracle.matmul(qt, w, x, rows, cols)),
                          bits(reference.matmul(qt, w, x, rows, cols)))


def test_oracle_vs_reference_scaled_activations(oracle, reference):
    """Tiny, huge and sparse activations (x_scale guard and extremes)."""
    w = synth.gen_weights(Q5_0, 64, 896, 7)
    for x in (synth.gen_x(896, 1) * np.float32(1e-12), synth.gen_x(896, 2) * np.float32(1e30),
              np.where(np.arange(896) % 97 == 0, np.float32(5.0), np.float32(0.0)).astype(np.float32)):
        assert np.array_equal(bits(oracle.matmul(Q5_0, w, x, 64, 896)),
                              bits(reference.matmul(Q5_0, w, x, 64, 896)))


def test_q8_combined_scale_wrap_vs_reference(oracle, reference):
    """Blocks whose UQ8.8 scale rounds up to 65536 and wraps to 0 on the
    reference's float->uint16 conversion (sim/tmac_gguf.cpp:1037)."""
    rows, cols = 4, 64
    w = np.zeros((rows, 2, 34), np.uint8)
    # block 0 carries the row maximum d0*127; block 1's scale d1 is chosen
    # so that c = d1*ri lies in [255.998, 256): c*256+0.5 rounds to 65536
    found = None
    for b0 in range(0x3400, 0x4c00):
        d0 = np.array([b0], np.uint16).view(np.float16)[0]
        rs = np.float32(np.float32(d0) * np.float32(127.0)) / np.float32(32767.0)
        ri = np.float32(1.0) / rs
        b1 = int(np.array([np.float16(np.float32(256.0) / ri)], np.float16).view(np.uint16)[0])
        for cand in range(b1 - 2, b1 + 3):
            d1 = np.array([cand], np.uint16).view(np.float16)[0]
            c = np.float32(np.float32(d1) * ri)
            if c < np.float32(256.0) and np.float32(np.float32(c * np.float32(256.0)) + np.float32(0.5)) >= np.float32(65536.0):
                found = (d0, d1, rs)
                break
        if found:
            break
    assert found is not None, "no fp16 scale pair lands in the UQ8.8 wrap window"
    d0, found, rs = found
    w[:, 0, 0:2] = np.array([d0], np.float16).view(np.uint8)
    w[:, 0, 2:] = np.array([127] + [1] * 31, np.int8).view(np.uint8)
    # keep d1*|q| below the row max so row_scale stays d0*127
    w[:, 1, 0:2] = np.array([found], np.float16).view(np.uint8)
    w[:, 1, 2:] = np.array([1, -1] * 16, np.int8).view(np.uint8)
    wf = w.reshape(-1)
    x = synth.gen_x(cols, 3)
    yo, yr = oracle.matmul(Q8_0, wf, x, rows, cols), reference.matmul(Q8_0, wf, x, rows, cols)
    assert np.array_equal(bits(yo), bits(yr))
    assert oracle.lib.tmqo_q8_combined_scale(int(np.array([found], np.float16).view(np.uint16)[0]), float(rs)) == 0


def test_oracle_vs_reference_tiles(oracle, reference):
    rng = np.random.Generator(np.random.PCG64(77))
    for _ in range(3):
        W = rng.integers(-128, 128, size=4096, dtype=np.int8).view(np.uint8)
        cs = rng.integers(0, 65536, size=128, dtype=np.uint16)
        vec = rng.integers(-32768, 32768, size=64, dtype=np.int16)
        assert np.array_equal(oracle.tile_q8(W, cs, vec), reference.tile_q8(W, cs, vec))
    # q5_0 8x896 with large row_inv (exercises the clamp)
    b5 = synth.gen_weights(Q5_0, 8, 896, 5)
    act = rng.integers(-32767, 32768, size=896, dtype=np.int16)
    ri = (rng.random(8, dtype=np.float32) * np.float32(1e6)).astype(np.float32)
    a, b = np.zeros(16, np.int64), np.zeros(16, np.int64)
    oracle.tile_q5_0_8x896(b5, act, ri, a, 4)
    reference.tile_q5_0_8x896(b5, act, ri, b, 4)
    assert np.array_equal(a, b)
    # 4x896 hp_fsm tile (interleaved 48-byte block pairs)
    b56 = rng.integers(0, 256, size=56 * 48, dtype=np.uint8)
    for i in range(56):  # sane fp16 scales
        b56[i * 48: i * 48 + 2] = np.array([np.float16(0.01 * (1 + i % 5))], np.float16).view(np.uint8)
        b56[i * 48 + 22: i * 48 + 24] = np.array([np.float16(0.02)], np.float16).view(np.uint8)
    rn = (rng.random(4, dtype=np.float32) * np.float32(4000.0)).astype(np.float32)
    a, b = np.zeros(8, np.int64), np.zeros(8, np.int64)
    oracle.tile_q5_0_4x896(b56, act, rn, a, 2)
    reference.tile_q5_0_4x896(b56, act, rn, b, 2)
    assert np.array_equal(a, b)
    for qt in (Q6_K, Q4_K):
        blocks = synth.gen_weights(qt, 40, 256, 8)
        act256 = rng.integers(-32767, 32768, size=256, dtype=np.int16)
        ri896 = (rng.random(1024, dtype=np.float32) * np.float32(5e5)).astype(np.float32)  # rows past 896 are read
        for nc in (256, 100):
            a, b = np.zeros(896, np.int64), np.zeros(896, np.int64)
            oracle.tile_kquant(qt, blocks, 40, act256, nc, ri896, a, 870)  # crosses row 896
            reference.tile_kquant(qt, blocks, 40, act256, nc, ri896, b, 870)
            assert np.array_equal(a, b)

