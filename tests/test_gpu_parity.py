"""GPU parity: libtmq.so on gfx950 vs the CPU oracle and the golden vectors.

Bar: bit-exact int64 partials (per row, per Q8 tile) and bit-exact fp32
outputs (the north-star tolerance is 1e-5 relative; exactness is met).
Everything goes through the C ABI (ctypes).
"""
import numpy as np
import pytest
from conftest import load_golden
from oracle import Q4_K, Q5_0, Q6_K, Q8_0
from tmq import synth

pytestmark = pytest.mark.gpu


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


def report(name, got, exp):
    bad = np.flatnonzero(got != exp)
    return f"{name}: {bad.size} mismatches, first at {bad[:5]}"


SHAPES = [
    (Q5_0, 896, 896), (Q5_0, 4864, 896), (Q5_0, 128, 896), (Q5_0, 100, 896),
    (Q4_K, 896, 4864), (Q6_K, 896, 4864), (Q4_K, 40, 512), (Q6_K, 72, 768),
    (Q8_0, 128, 896), (Q8_0, 1000, 896), (Q8_0, 64, 4864), (Q8_0, 8, 96),
]


@pytest.mark.parametrize("qt,rows,cols", SHAPES)
def test_gemv_bitexact(ctx, oracle, qt, rows, cols):
    print(f"[gemv] type={qt} {rows}x{cols}", flush=True)
    w = synth.gen_weights(qt, rows, cols, 500 + rows)
    x = synth.gen_x(cols, 600 + cols)
    t = ctx.upload(qt, rows, cols, w)
    y = ctx.matmul(t, x)
    ye = oracle.matmul(qt, w, x, rows, cols)
    assert np.array_equal(bits(y), bits(ye)), report("y", bits(y), bits(ye))
    acc, xs = ctx.partials(t, x)
    xq, xse = oracle.quantize_act(x)
    assert xs == xse
    if qt == Q8_0:
        rn = t.row_norm()
        rse = oracle.q8_row_scale(oracle.row_max_abs_q8(w, rows, cols))
        assert np.array_equal(bits(rn), bits(rse))
        P = oracle.tiles_q8(w, rows, cols, xq, rse)
        assert np.array_equal(acc, P), report("tiles", acc, P)
    else:
        ri = oracle.row_inv(qt, w, rows, cols)
        assert np.array_equal(bits(t.row_norm()), bits(ri))
        ae = oracle.acc(qt, w, rows, cols, xq, ri)
        assert np.array_equal(acc, ae), report("acc", acc, ae)
    t.free()


FIT_SUB = {Q5_0: 32, Q4_K: 32, Q6_K: 16}  # weights per fitted sub-block


@pytest.mark.parametrize("qt,rows,cols", [(Q5_0, 4864, 896), (Q4_K, 896, 4864), (Q6_K, 896, 4864)])
def test_fit_stats_and_exact_decode(ctx, oracle, qt, rows, cols, monkeypatch):
    """Every sub-block is fitted or flagged; the flagged ones (present in the
    Q5_0 and Q6_K tensors: the linear form has no pair for them) and a
    tensor uploaded with TMQ_NOFIT=1 (every sub-block on the exact decode)
    give the oracle's int64 sums exactly.  The fitted-float decoders are the
    ones the decode engine runs; TMQ_NOMFMA=1 keeps the standalone GEMV on
    them (every tensor here would otherwise take the MFMA decoders)."""
    print(f"[fit] type={qt} {rows}x{cols}", flush=True)
    monkeypatch.setenv("TMQ_NOMFMA", "1")
    w = synth.gen_weights(qt, rows, cols, 900 + rows)
    x = synth.gen_x(cols, 901)
    xq, _ = oracle.quantize_act(x)
    ae = oracle.acc(qt, w, rows, cols, xq, oracle.row_inv(qt, w, rows, cols))
    t = ctx.upload(qt, rows, cols, w)
    fitted, exact = t.fit_stats()
    assert fitted + exact == rows * cols // FIT_SUB[qt]
    assert exact < fitted // 1000
    if qt != Q4_K:
        assert exact > 0, "no sub-block on the exact decode: the mixed case is not covered"
    acc, _ = ctx.partials(t, x)
    assert np.array_equal(acc, ae), report("acc", acc, ae)
    t.free()
    monkeypatch.setenv("TMQ_NOFIT", "1")
    t = ctx.upload(qt, rows, cols, w)
    assert t.fit_stats() == (0, rows * cols // FIT_SUB[qt])
    acc, _ = ctx.partials(t, x)
    assert np.array_equal(acc, ae), report("acc (exact decode)", acc, ae)
    t.free()


def test_q8_logits_full_size(ctx, oracle):
    """151936 x 896 Q8_0 logits matvec, with and without
    the row_max_abs aux tensor."""
    rows, cols = 151936, 896
    print("[gemv] Q8_0 logits 151936x896", flush=True)
    w = synth.gen_weights(Q8_0, rows, cols, 1)
    x = synth.gen_x(cols, 2)
    ye = oracle.matmul(Q8_0, w, x, rows, cols)
    t = ctx.upload(Q8_0, rows, cols, w)
    y = ctx.matmul(t, x)
    assert np.array_equal(bits(y), bits(ye)), report("y", bits(y), bits(ye))
    t.free()
    aux = oracle.row_max_abs_q8(w, rows, cols)
    t2 = ctx.upload(Q8_0, rows, cols, w, row_max_abs=aux)
    assert np.array_equal(bits(ctx.matmul(t2, x)), bits(ye))
    t2.free()


@pytest.mark.parametrize("name", ["q5_0", "q8_0", "q8_0_c64", "q4_k", "q6_k"])
def test_golden_matmul(ctx, name):
    g = load_golden(f"matmul_{name}.npz")
    qt, rows, cols = int(g["qtype"]), int(g["rows"]), int(g["cols"])
    print(f"[golden] {name}", flush=True)
    t = ctx.upload(qt, rows, cols, g["w"])
    assert np.array_equal(bits(ctx.matmul(t, g["x"])), bits(g["y"]))
    t.free()
    if qt == Q8_0:
        t = ctx.upload(qt, rows, cols, g["w"], row_max_abs=g["aux"])
        assert np.array_equal(bits(ctx.matmul(t, g["x"])), bits(g["y_aux"]))
        t.free()


def test_golden_edges(ctx):
    g = load_golden("edge_q5_0.npz")
    t = ctx.upload(Q5_0, 8, 896, g["w"])
    assert np.array_equal(bits(ctx.matmul(t, g["x0"])), bits(g["y0"]))
    assert np.array_equal(bits(ctx.matmul(t, g["xs"])), bits(g["ys"]))
    t.free()


def test_golden_tiles(ctx):
    g = load_golden("tiles.npz")
    print("[tiles]", flush=True)
    assert np.array_equal(ctx.tile_q8(g["W"], g["cs"], g["vec"]), g["tq8"])
    r5 = g["res5_in"].copy()
    ctx.tile_q5_0_8x896(g["b5"], g["act896"], g["ri8"], r5, 8)
    assert np.array_equal(r5, g["res5"])
    r6 = np.zeros(896, np.int64)
    ctx.tile_kquant(Q6_K, g["b6"], 32, g["act256"], 256, g["ri896"], r6, 864)
    assert np.array_equal(r6, g["res6"])
    r4 = np.zeros(896, np.int64)
    ctx.tile_kquant(Q4_K, g["b4"], 56, g["act256"], 200, g["ri896"], r4, 840)
    assert np.array_equal(r4, g["res4"])


def test_tiles_vs_oracle_clamp(ctx, oracle):
    """External row_inv large enough to saturate: the clamp path."""
    rng = np.random.Generator(np.random.PCG64(5))
    b5 = synth.gen_weights(Q5_0, 8, 896, 9)
    act = rng.integers(-32767, 32768, size=896, dtype=np.int16)
    ri = (rng.random(8, dtype=np.float32) * np.float32(1e7)).astype(np.float32)
    a, b = np.zeros(16, np.int64), np.zeros(16, np.int64)
    ctx.tile_q5_0_8x896(b5, act, ri, a, 3)
    oracle.tile_q5_0_8x896(b5, act, ri, b, 3)
    assert np.array_equal(a, b)
    for qt in (Q6_K, Q4_K):
        blocks = synth.gen_weights(qt, 40, 256, 8)
        act256 = rng.integers(-32767, 32768, size=256, dtype=np.int16)
        ri1 = (rng.random(1024, dtype=np.float32) * np.float32(5e5)).astype(np.float32)
        a, b = np.zeros(896, np.int64), np.zeros(896, np.int64)
        ctx.tile_kquant(qt, blocks, 40, act256, 256, ri1, a, 870)
        oracle.tile_kquant(qt, blocks, 40, act256, 256, ri1, b, 870)
        assert np.array_equal(a, b)


def test_tile_q5_0_4x896_vs_oracle(ctx, oracle):
    """The hp_fsm 4x896 tile (56 interleaved 48-byte block pairs, UQ8.8-sized
    row_norm, and large ones that saturate) against the oracle, which
    test_oracle_ref pins to the compiled reference's
    axi_vecmul_tile_q5_0_4x896_axilite."""
    rng = np.random.Generator(np.random.PCG64(11))
    for scale in (np.float32(4.0), np.float32(4000.0), np.float32(1e7)):
        b56 = rng.integers(0, 256, size=56 * 48, dtype=np.uint8)
        for i in range(56):  # finite fp16 scales of both cores
            b56[i * 48: i * 48 + 2] = np.array([np.float16(0.01 * (1 + i % 5))], np.float16).view(np.uint8)
            b56[i * 48 + 22: i * 48 + 24] = np.array([np.float16(-0.02 * (1 + i % 3))], np.float16).view(np.uint8)
        act = rng.integers(-32767, 32768, size=896, dtype=np.int16)
        rn = (rng.random(4, dtype=np.float32) * scale).astype(np.float32)
        a = rng.integers(-1000, 1000, size=10).astype(np.int64)
        b = a.copy()
        ctx.tile_q5_0_4x896(b56, act, rn, a, 5)
        oracle.tile_q5_0_4x896(b56, act, rn, b, 5)
        assert np.array_equal(a, b), f"row_norm scale {scale}"
    with pytest.raises(ValueError):
        ctx.tile_q5_0_4x896(b56, act, rn, np.zeros(6, np.int64), 3)


def test_golden_phaseb(ctx):
    g = load_golden("phaseb.npz")
    arena = g["arena"].copy()
    base, head = int(g["base"]), int(g["head"])
    print("[phaseb]", flush=True)
    n, rows = ctx.phaseb_run(arena, base, head)
    assert n == len(g["rows"]) and list(rows) == list(g["rows"])
    # results written at each descriptor's result_addr
    off, k, got = head, 0, []
    while off:
        d = arena[off - base: off - base + 32]
        ra = int(d[12:16].view(np.uint32)[0])
        got.append(arena[ra - base: ra - base + 8 * int(rows[k])].view(np.int64))
        off = int(d[0:4].view(np.uint32)[0])
        k += 1
    assert np.array_equal(np.concatenate(got), g["acc"])


def test_golden_phaseb_chain(ctx):
    """the compiled reference's in-order replay of a chain with matmul, OP->OP
    (activation = the previous result slot), CPU_OP, Q8_0 and mixed-row_inv
    Q6_K descriptors (tests/golden/phaseb_chain.npz): the arena after
    tmq_phaseb_run equals the reference's byte for byte"""
    g = load_golden("phaseb_chain.npz")
    arena = g["arena"].copy()
    print("[phaseb] chain with OP->OP / CPU_OP / Q8_0 / mixed row_inv", flush=True)
    n, rows = ctx.phaseb_run(arena, int(g["base"]), int(g["head"]))
    assert n == len(g["rows"]) and list(rows) == g["rows"].tolist()
    bad = np.flatnonzero(arena != g["arena_after"])
    assert bad.size == 0, f"{bad.size} bytes differ, first at offset {bad[:4]}"


def test_chain_matches_single_gemvs(ctx, oracle):
    """A device chain (one launch) over mixed formats equals per-GEMV results."""
    torch = pytest.importorskip("torch")
    dev = torch.device("cuda:0")
    specs = [(Q5_0, 896, 896, 224, 4, 1), (Q5_0, 4864, 896, 1216, 4, 1), (Q8_0, 128, 896, 2, 64, 14),
             (Q4_K, 896, 4864, 304, 56, 19), (Q6_K, 896, 4864, 532, 32, 19)]
    xa = synth.gen_x(896, 1)
    xb = synth.gen_x(4864, 2)
    xa_d = torch.from_numpy(xa).to(dev)
    xb_d = torch.from_numpy(xb).to(dev)
    descs, outs, ws, ts = [], [], [], []
    for i, (qt, rows, cols, nt, tr, ncg) in enumerate(specs):
        w = synth.gen_weights(qt, rows, cols, 70 + i)
        t = ctx.upload(qt, rows, cols, w)
        y = torch.zeros(rows, dtype=torch.float32, device=dev)
        x = xa_d if cols == 896 else xb_d
        descs.append((t, x.data_ptr(), y.data_ptr(), None, nt, tr, ncg))
        outs.append(y)
        ws.append(w)
        ts.append(t)
    print("[chain] 5 descriptors", flush=True)
    ch = ctx.chain(descs)
    ch.run()
    ctx.sync()
    for (qt, rows, cols, *_), w, y in zip(specs, ws, outs):
        ye = oracle.matmul(qt, w, xa if cols == 896 else xb, rows, cols)
        assert np.array_equal(bits(y.cpu().numpy()), bits(ye))
    ch.free()
    for t in ts:
        t.free()


@pytest.mark.parametrize("qt", [Q5_0, Q4_K, Q6_K])
def test_chain_tall_tensors(ctx, oracle, qt):
    """A chain segment of 4097 64-row groups over two tall tensors, one of
    them with rows not a multiple of 64: every row bit-exact with the
    oracle."""
    torch = pytest.importorskip("torch")
    dev = torch.device("cuda:0")
    cols = 64 if qt == Q5_0 else 256
    # 2050 + 2047 groups = 4097 = 4 * 1024 + 1
    shapes = [(131200, 11), (131000, 12)]
    x = synth.gen_x(cols, 9)
    x_d = torch.from_numpy(x).to(dev)
    descs, outs, ws, ts = [], [], [], []
    for rows, seed in shapes:
        w = synth.gen_weights(qt, rows, cols, seed)
        t = ctx.upload(qt, rows, cols, w)
        y = torch.zeros(rows, dtype=torch.float32, device=dev)
        tr = 4 if qt == Q5_0 else 8
        descs.append((t, x_d.data_ptr(), y.data_ptr(), None, rows // tr, tr, cols // 256 if qt != Q5_0 else 1))
        outs.append(y)
        ws.append(w)
        ts.append(t)
    print(f"[chain] tall tensors, type {qt}", flush=True)
    ch = ctx.chain(descs)
    ch.run()
    ctx.sync()
    for (rows, _), w, y in zip(shapes, ws, outs):
        ye = oracle.matmul(qt, w, x, rows, cols)
        assert np.array_equal(bits(y.cpu().numpy()), bits(ye))
    ch.free()
    for t in ts:
        t.free()


@pytest.mark.parametrize("qt", [Q4_K, Q6_K])
@pytest.mark.parametrize("force", [False, True])
def test_chain_split_tail(ctx, oracle, monkeypatch, qt, force):
    """A K-quant chain segment of 20 ffn_down tensors (896x4864, 14 groups
    each) and one 130x1024 tensor (3 groups): 283 groups leave a last round
    of 27 on 256 CUs, which the chain splits into pieces over super-block
    ranges (9 a group; 4 for the 4-super-block tensor) that meet through
    tail slots.  Three runs in a row (each slot must be left clear for the
    next): int64 row sums and fp32 outputs bit-exact with the oracle, the
    same as the unsplit chain (TMQ_NOSPLIT=1); with every sub-block forced
    onto corrections (TMQ_IFIT_FORCE=1) too, which only the first piece of a
    group adds."""
    torch = pytest.importorskip("torch")
    dev = torch.device("cuda:0")
    if force:
        monkeypatch.setenv("TMQ_IFIT_FORCE", "1")
    shapes = [(896, 4864)] * 20 + [(130, 1024)]
    xs = {c: synth.gen_x(c, 40 + c) for c in (1024, 4864)}
    xd = {c: torch.from_numpy(v).to(dev) for c, v in xs.items()}
    descs, ys, accs, ws, ts = [], [], [], [], []
    tr = 56 if qt == Q4_K else 32
    for i, (rows, cols) in enumerate(shapes):
        w = synth.gen_weights(qt, rows, cols, 500 + 7 * i + qt)
        t = ctx.upload(qt, rows, cols, w)
        y = torch.zeros(rows, dtype=torch.float32, device=dev)
        a = torch.zeros(rows, dtype=torch.int64, device=dev)
        ncg = cols // 256
        nt = ncg * (rows // tr) if rows % tr == 0 else None
        if nt is None:  # 130 rows: tiles of 10 rows
            nt, trr = ncg * 13, 10
        else:
            trr = tr
        descs.append((t, xd[cols].data_ptr(), y.data_ptr(), a.data_ptr(), nt, trr, ncg))
        ys.append(y)
        accs.append(a)
        ws.append(w)
        ts.append(t)
    exp = []
    for (rows, cols), w in zip(shapes, ws):
        x = xs[cols]
        xq, _ = oracle.quantize_act(x)
        exp.append((oracle.acc(qt, w, rows, cols, xq, oracle.row_inv(qt, w, rows, cols)),
                    oracle.matmul(qt, w, x, rows, cols)))
    for nosplit in (False, True):
        monkeypatch.setenv("TMQ_NOSPLIT", "1" if nosplit else "0")
        print(f"[chain] split tail, type {qt}, forced fit {force}, nosplit {nosplit}", flush=True)
        ch = ctx.chain(descs)
        for run in range(3):
            for y, a in zip(ys, accs):
                y.zero_()
                a.zero_()
            ch.run()
            ctx.sync()
            for i, (y, a, (ae, ye)) in enumerate(zip(ys, accs, exp)):
                got = a.cpu().numpy()
                assert np.array_equal(got, ae), report(f"acc of tensor {i}, run {run}", got, ae)
                assert np.array_equal(bits(y.cpu().numpy()), bits(ye)), f"y of tensor {i}, run {run}"
        ch.free()
    for t in ts:
        t.free()


def test_chain_split_tail_q8(ctx, oracle, monkeypatch):
    """A Q8_0 chain segment of 20 896x896 tensors (4 groups of 256 rows
    each, the last one half empty) and one 130x896 tensor (1 group): 81
    groups leave a last round of 81 on 256 CUs, which the chain runs as one
    workgroup per 64-row quarter, the four waves splitting the row's tiles.
    Three runs: per-tile int64 sums and fp32 outputs bit-exact with the
    oracle, the same as the unsplit chain (TMQ_NOSPLIT=1)."""
    torch = pytest.importorskip("torch")
    dev = torch.device("cuda:0")
    cols = 896
    shapes = [896] * 20 + [130]
    x = synth.gen_x(cols, 77)
    x_d = torch.from_numpy(x).to(dev)
    xq, _ = oracle.quantize_act(x)
    descs, ys, accs, exp, ts = [], [], [], [], []
    nt = cols // 64
    for i, rows in enumerate(shapes):
        w = synth.gen_weights(Q8_0, rows, cols, 900 + i)
        t = ctx.upload(Q8_0, rows, cols, w)
        y = torch.zeros(rows, dtype=torch.float32, device=dev)
        a = torch.zeros(rows * nt, dtype=torch.int64, device=dev)
        tiles, tr = (rows // 64, 64) if rows % 64 == 0 else (13, 10)
        descs.append((t, x_d.data_ptr(), y.data_ptr(), a.data_ptr(), tiles, tr, nt))
        ys.append(y)
        accs.append(a)
        ts.append(t)
        rse = oracle.q8_row_scale(oracle.row_max_abs_q8(w, rows, cols))
        exp.append((oracle.tiles_q8(w, rows, cols, xq, rse).reshape(-1), oracle.matmul(Q8_0, w, x, rows, cols)))
    for nosplit in (False, True):
        monkeypatch.setenv("TMQ_NOSPLIT", "1" if nosplit else "0")
        print(f"[chain] Q8_0 split tail, nosplit {nosplit}", flush=True)
        ch = ctx.chain(descs)
        for run in range(3):
            for y, a in zip(ys, accs):
                y.zero_()
                a.zero_()
            ch.run()
            ctx.sync()
            for i, (y, a, (pe, ye)) in enumerate(zip(ys, accs, exp)):
                got = a.cpu().numpy()
                assert np.array_equal(got, pe), report(f"tiles of tensor {i}, run {run}", got, pe)
                assert np.array_equal(bits(y.cpu().numpy()), bits(ye)), f"y of tensor {i}, run {run}"
        ch.free()
    for t in ts:
        t.free()


def test_error_paths(ctx):
    import tmq
    w = synth.gen_weights(Q5_0, 8, 896, 1)
    with pytest.raises(tmq.TmqError) as e:
        ctx.upload(Q5_0, 8, 900, w)          # cols not a multiple of 32
    assert e.value.code == -1
    with pytest.raises(tmq.TmqError) as e:
        ctx.upload(Q5_0, 8, 896, w[:-1])     # short buffer
    assert e.value.code == -1
    bad = w.copy()
    bad[22 * 5: 22 * 5 + 2] = np.array([np.float16(np.inf)], np.float16).view(np.uint8)
    with pytest.raises(tmq.TmqError) as e:
        ctx.upload(Q5_0, 8, 896, bad)         # Inf scale
    assert e.value.code == -3
    t = ctx.upload(Q5_0, 8, 896, w)
    with pytest.raises(tmq.TmqError):
        tmq._check(tmq.lib().tmq_matmul(ctx.handle, t.handle, None, None, 8, 896))
    t.free()
