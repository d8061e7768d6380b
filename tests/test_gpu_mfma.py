"""GPU parity of the MFMA decoders: Q5_0, Q4_K and Q6_K GEMVs whose blocks
(K-quants: sub-blocks) are decoded by the upload-time integer fit and summed
on the int8 MFMA, with the codes the fit cannot reproduce applied as
corrections.

Bar: bit-exact int64 row sums and fp32 outputs against the CPU oracle
(oracle/tmq_oracle.c: tmqo_matmul_q5_0, the restatement of
sim/tmac_gguf.cpp:1245-1308), on tensors that take the MFMA decoders and on
the shapes that fall back to the fitted-float decoders (more than 8192
columns); block counts below, at and above the workgroup's four waves.
Forcing one wrong fit on every block (TMQ_IFIT_FORCE=1) routes most codes
through the corrections and must give the same sums.
"""
import numpy as np
import pytest
from oracle import Q4_K, Q5_0, Q6_K
from tmq import synth

pytestmark = pytest.mark.gpu

MFMA_MAX_COLS = 8192


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


def report(name, got, exp):
    bad = np.flatnonzero(got != exp)
    return f"{name}: {bad.size} mismatches, first at {bad[:5]}"


def eligible(cols):
    return cols <= MFMA_MAX_COLS


def check(ctx, oracle, rows, cols, seed, qt=Q5_0):
    w = synth.gen_weights(qt, rows, cols, seed)
    x = synth.gen_x(cols, seed + 1)
    t = ctx.upload(qt, rows, cols, w)
    blocks, corr = t.ifit_stats()
    y = ctx.matmul(t, x)
    acc, xs = ctx.partials(t, x)
    t.free()
    ye = oracle.matmul(qt, w, x, rows, cols)
    xq, _ = oracle.quantize_act(x)
    ae = oracle.acc(qt, w, rows, cols, xq, oracle.row_inv(qt, w, rows, cols))
    assert np.array_equal(acc, ae), report("acc", acc, ae)
    assert np.array_equal(bits(y), bits(ye)), report("y", bits(y), bits(ye))
    return blocks, corr


@pytest.mark.parametrize("rows,cols", [(896, 896), (4864, 896), (100, 896), (64, 4864), (200, 256),
                                       (64, 32), (64, 64), (128, 96), (64, 160), (64, MFMA_MAX_COLS),
                                       (64, MFMA_MAX_COLS + 64)])
def test_mfma_q5_bitexact(ctx, oracle, rows, cols):
    print(f"[mfma] Q5_0 {rows}x{cols}", flush=True)
    blocks, corr = check(ctx, oracle, rows, cols, 1700 + rows + cols)
    if eligible(cols):
        assert blocks == rows * cols // 32
        # the fit leaves about one block in a thousand with a correction
        assert corr <= max(8, blocks // 200)
    else:
        assert (blocks, corr) == (0, 0)


def test_mfma_q5_corrections(ctx, oracle, monkeypatch):
    """Every block on one fixed wrong (AN, BN): nearly every code becomes a
    correction, the sums stay exact."""
    monkeypatch.setenv("TMQ_IFIT_FORCE", "1")
    print("[mfma] Q5_0 896x896 forced fit", flush=True)
    blocks, corr = check(ctx, oracle, 896, 896, 1801)
    assert blocks == 896 * 28
    assert corr > blocks  # several differing codes per block


def test_mfma_q5_misfits_present(ctx, oracle):
    """The BASELINE shapes hold blocks the integer fit cannot reproduce, so
    the natural corrections are exercised."""
    print("[mfma] Q5_0 4864x896 natural corrections", flush=True)
    blocks, corr = check(ctx, oracle, 4864, 896, 1802)
    assert blocks == 4864 * 28 and corr > 0


def test_mfma_q5_off(ctx, oracle, monkeypatch):
    """TMQ_NOMFMA=1 keeps a tensor on the fitted-float decoders."""
    monkeypatch.setenv("TMQ_NOMFMA", "1")
    print("[mfma] Q5_0 896x896 without the MFMA decoders", flush=True)
    assert check(ctx, oracle, 896, 896, 1803) == (0, 0)


# K-quant sub-blocks per 256-column super-block
SUBS = {Q4_K: 8, Q6_K: 16}


@pytest.mark.parametrize("qt", [Q4_K, Q6_K])
@pytest.mark.parametrize("rows,cols", [(896, 4864), (64, 256), (100, 512), (130, 768), (200, 1024),
                                       (64, MFMA_MAX_COLS), (64, MFMA_MAX_COLS + 256)])
def test_mfma_kquant_bitexact(ctx, oracle, qt, rows, cols):
    """K-quants on the MFMA decoders: every row's int64 sum and fp32 output
    bit-exact; one to 32 super-blocks per row (quarters per wave 1 to 32),
    rows not a multiple of 64; wider than 8192 columns stays on the
    fitted-float decoders."""
    print(f"[mfma] type {qt} {rows}x{cols}", flush=True)
    blocks, corr = check(ctx, oracle, rows, cols, 2300 + rows + cols + qt, qt)
    if eligible(cols):
        assert blocks == rows * cols // 256 * SUBS[qt]
        # the fit misses about one Q6_K sub-block in 200 (a few per cent on
        # small tensors) and almost no Q4_K one
        assert corr <= max(32, blocks // 25)
    else:
        assert (blocks, corr) == (0, 0)


@pytest.mark.parametrize("qt", [Q4_K, Q6_K])
def test_mfma_kquant_corrections(ctx, oracle, monkeypatch, qt):
    """Every sub-block on one fixed wrong fit (TMQ_IFIT_FORCE=1): most codes
    become corrections, the sums stay exact."""
    monkeypatch.setenv("TMQ_IFIT_FORCE", "1")
    print(f"[mfma] type {qt} 256x4864 forced fit", flush=True)
    blocks, corr = check(ctx, oracle, 256, 4864, 2401 + qt, qt)
    assert blocks == 256 * 19 * SUBS[qt]
    assert corr > blocks // 2  # most sub-blocks carry corrections


def test_mfma_q6k_misfits_present(ctx, oracle):
    """The BASELINE Q6_K shape holds sub-blocks the integer fit cannot
    reproduce, so the natural corrections are exercised."""
    print("[mfma] Q6_K 896x4864 natural corrections", flush=True)
    blocks, corr = check(ctx, oracle, 896, 4864, 2402, Q6_K)
    assert corr > 0


@pytest.mark.parametrize("qt", [Q4_K, Q6_K])
def test_mfma_kquant_off(ctx, oracle, monkeypatch, qt):
    """TMQ_NOMFMA=1 keeps a K-quant tensor on the fitted-float decoders."""
    monkeypatch.setenv("TMQ_NOMFMA", "1")
    print(f"[mfma] type {qt} without the MFMA decoders", flush=True)
    assert check(ctx, oracle, 128, 1024, 2403 + qt, qt) == (0, 0)
