"""tmq_gemv_dev_noalloc: the GEMV entry point that allocates nothing (its
prepared activation lives in the library's fixed per-device scratch).  It
must give the bits of tmq_gemv_dev on the same inputs -- outputs and int64
partials -- over consecutive calls that reuse the scratch, the second with a
smaller input than the first, and reject tensors wider than its limit."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.device("cuda:0"))


def _run(ctx, torch, t, x_d, noalloc):
    import tmq
    y = torch.full((t.rows,), float("nan"), dtype=torch.float32, device=x_d.device)
    nacc = t.rows * ((t.cols + 63) // 64) if t.qtype == tmq.Q8_0 else t.rows
    acc = torch.full((nacc,), -1, dtype=torch.int64, device=x_d.device)
    f = ctx.gemv_dev_noalloc if noalloc else ctx.gemv_dev
    f(t, x_d.data_ptr(), y.data_ptr(), acc.data_ptr())
    ctx.sync()
    return y.cpu().numpy(), acc.cpu().numpy()


def test_noalloc_matches_gemv_dev(ctx, oracle):
    torch = pytest.importorskip("torch")
    import tmq
    from tmq import synth
    # the first call fills 4864 columns of scratch, the second uses 896
    cases = [(tmq.Q4_K, 896, 4864, 11), (tmq.Q8_0, 128, 896, 12), (tmq.Q5_0, 896, 896, 13)]
    for qt, rows, cols, seed in cases:
        print(f"[noalloc] type {qt} {rows}x{cols} seed {seed}", flush=True)
        w = synth.gen_weights(qt, rows, cols, seed)
        x = synth.gen_x(cols, seed + 100)
        t = ctx.upload(qt, rows, cols, w)
        try:
            x_d = _dev(torch, x)
            y_na, acc_na = _run(ctx, torch, t, x_d, True)
            y_ref, acc_ref = _run(ctx, torch, t, x_d, False)
        finally:
            t.free()
        assert np.array_equal(acc_na, acc_ref)
        assert np.array_equal(y_na.view(np.uint32), y_ref.view(np.uint32))
        ye = oracle.matmul(qt, w, x, rows, cols)
        assert np.array_equal(y_na.view(np.uint32), ye.view(np.uint32))


def test_noalloc_rejects_wide_tensor(ctx):
    torch = pytest.importorskip("torch")
    import tmq
    from tmq import synth
    cols = tmq.NOALLOC_MAX_COLS + 32
    w = synth.gen_weights(tmq.Q5_0, 64, cols, 5)
    t = ctx.upload(tmq.Q5_0, 64, cols, w)
    try:
        x_d = _dev(torch, synth.gen_x(cols, 6))
        y = torch.zeros(64, dtype=torch.float32, device=x_d.device)
        with pytest.raises(tmq.TmqError, match="scratch limit"):
            ctx.gemv_dev_noalloc(t, x_d.data_ptr(), y.data_ptr(), None)
    finally:
        t.free()
