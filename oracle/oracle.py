"""ctypes binding for the CPU oracle -- TEST INFRASTRUCTURE ONLY.

Loads oracle/liboracle.so (the C restatement of the reference arithmetic) and,
where it was built, oracle/_ref/libtmacref.so (the reference's own sim/
sources compiled in place).  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg import this module, and only as the checker.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libtmacref.so")

F32, F16, Q8_0, Q5_0, Q4_K, Q6_K = 0, 1, 8, 6, 12, 14

_P = C.c_void_p
_i = C.c_int
_u32 = C.c_uint32
_u64 = C.c_uint64


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _setup(lib, name, res, args):
    f = getattr(lib, name)
    f.restype = res
    f.argtypes = args
    return f


class Oracle:
    """The C restatement (tmq_oracle.c)."""

    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = self.lib = C.CDLL(path)
        _setup(L, "tmqo_f16_to_f32", C.c_float, [C.c_uint16])
        _setup(L, "tmqo_quantize_act", C.c_float, [_P, _i, _P])
        for n in ("q5_0", "q4_k", "q6_k"):
            _setup(L, f"tmqo_row_inv_{n}", None, [_P, _i, _i, _P])
            _setup(L, f"tmqo_acc_{n}", None, [_P, _i, _i, _P, _P, _P])
            _setup(L, f"tmqo_matmul_{n}", None, [_P, _P, _P, _i, _i])
        _setup(L, "tmqo_row_max_abs_q8_0", None, [_P, _i, _i, _P])
        _setup(L, "tmqo_q8_row_scale", C.c_float, [C.c_float])
        _setup(L, "tmqo_q8_combined_scale", C.c_uint16, [C.c_uint16, C.c_float])
        _setup(L, "tmqo_tiles_q8_0", None, [_P, _i, _i, _P, _P, _P])
        _setup(L, "tmqo_finalize_rowinv", C.c_float, [C.c_int64, C.c_float, C.c_float])
        _setup(L, "tmqo_finalize_q8", C.c_float, [_P, _i, C.c_float, C.c_float])
        _setup(L, "tmqo_matmul_q8_0", None, [_P, _P, _P, _i, _i, _P])
        _setup(L, "tmqo_tile_q8", None, [_P, _P, _P, _P])
        _setup(L, "tmqo_tile_q5_0_8x896", None, [_P, _P, _P, _P, _i])
        _setup(L, "tmqo_tile_q6_k", None, [_P, _i, _P, _i, _P, _P, _i])
        _setup(L, "tmqo_tile_q4_k", None, [_P, _i, _P, _i, _P, _P, _i])
        _setup(L, "tmqo_tile_q5_0_4x896", None, [_P, _P, _P, _P, _i])
        _setup(L, "tmqo_phaseb_run", _i, [_P, _u32, _u32, _P])
        _setup(L, "tmqo_read_tensor", C.c_float, [_u32, _P, _i, _i, _i])
        _setup(L, "tmqo_matmul_int16", None, [_u32, _P, _P, _P, _i, _i, _P, _P])
        _setup(L, "tmqo_matmul_fp32", None, [_u32, _P, _P, _P, _i, _i])

    # -- activation / row stats -------------------------------------------
    def quantize_act(self, x: np.ndarray):
        x = np.ascontiguousarray(x, dtype=np.float32)
        xq = np.empty(x.size, dtype=np.int16)
        s = self.lib.tmqo_quantize_act(_ptr(x), x.size, _ptr(xq))
        return xq, np.float32(s)

    def row_inv(self, qtype: int, w: np.ndarray, rows: int, cols: int) -> np.ndarray:
        out = np.empty(rows, dtype=np.float32)
        name = {Q5_0: "q5_0", Q4_K: "q4_k", Q6_K: "q6_k"}[qtype]
        getattr(self.lib, f"tmqo_row_inv_{name}")(_ptr(w), rows, cols, _ptr(out))
        return out

    def row_max_abs_q8(self, w, rows, cols):
        out = np.empty(rows, dtype=np.float32)
        self.lib.tmqo_row_max_abs_q8_0(_ptr(w), rows, cols, _ptr(out))
        return out

    def q8_row_scale(self, max_abs: np.ndarray) -> np.ndarray:
        return np.array([self.lib.tmqo_q8_row_scale(float(m)) for m in max_abs], dtype=np.float32)

    # -- integer partials ---------------------------------------------------
    def acc(self, qtype, w, rows, cols, xq, row_inv) -> np.ndarray:
        out = np.empty(rows, dtype=np.int64)
        name = {Q5_0: "q5_0", Q4_K: "q4_k", Q6_K: "q6_k"}[qtype]
        getattr(self.lib, f"tmqo_acc_{name}")(_ptr(w), rows, cols, _ptr(xq), _ptr(row_inv), _ptr(out))
        return out

    def tiles_q8(self, w, rows, cols, xq, row_scale) -> np.ndarray:
        nt = (cols + 63) // 64
        out = np.empty((rows, nt), dtype=np.int64)
        self.lib.tmqo_tiles_q8_0(_ptr(w), rows, cols, _ptr(xq), _ptr(row_scale), _ptr(out))
        return out

    # -- whole matmul ---------------------------------------------------------
    def matmul(self, qtype, w, x, rows, cols, row_max_abs=None) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(rows, dtype=np.float32)
        if qtype == Q8_0:
            self.lib.tmqo_matmul_q8_0(_ptr(w), _ptr(x), _ptr(y), rows, cols, _ptr(row_max_abs))
        else:
            name = {Q5_0: "q5_0", Q4_K: "q4_k", Q6_K: "q6_k"}[qtype]
            getattr(self.lib, f"tmqo_matmul_{name}")(_ptr(w), _ptr(x), _ptr(y), rows, cols)
        return y

    def read_tensor(self, qtype, w, cols, r, j) -> np.float32:
        return np.float32(self.lib.tmqo_read_tensor(qtype, _ptr(w), cols, r, j))

    def matmul_int16(self, qtype, w, x, rows, cols):
        """matmul_fpga_int16: (y, int64 tiles [rows][ceil(cols/64)], row_scale)"""
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w).view(np.uint8)
        y = np.empty(rows, dtype=np.float32)
        tiles = np.empty((rows, (cols + 63) // 64), dtype=np.int64)
        rs = np.empty(rows, dtype=np.float32)
        self.lib.tmqo_matmul_int16(qtype, _ptr(w), _ptr(x), _ptr(y), rows, cols, _ptr(tiles), _ptr(rs))
        return y, tiles, rs

    def matmul_fp32(self, qtype, w, x, rows, cols) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w).view(np.uint8)
        y = np.empty(rows, dtype=np.float32)
        self.lib.tmqo_matmul_fp32(qtype, _ptr(w), _ptr(x), _ptr(y), rows, cols)
        return y

    # -- tiles ----------------------------------------------------------------
    def tile_q8(self, W, cs, vec):
        r = np.zeros(64, dtype=np.int64)
        self.lib.tmqo_tile_q8(_ptr(W), _ptr(cs), _ptr(vec), _ptr(r))
        return r

    def tile_q5_0_8x896(self, blocks, act, row_inv, result, row_base):
        self.lib.tmqo_tile_q5_0_8x896(_ptr(blocks), _ptr(act), _ptr(row_inv), _ptr(result), row_base)

    def tile_kquant(self, qtype, blocks, nblocks, act, ncols, row_inv, result, row_base):
        f = self.lib.tmqo_tile_q6_k if qtype == Q6_K else self.lib.tmqo_tile_q4_k
        f(_ptr(blocks), nblocks, _ptr(act), ncols, _ptr(row_inv), _ptr(result), row_base)

    def tile_q5_0_4x896(self, blocks56, act, row_norm, result, row_base):
        self.lib.tmqo_tile_q5_0_4x896(_ptr(blocks56), _ptr(act), _ptr(row_norm), _ptr(result), row_base)

    def phaseb_run(self, arena: np.ndarray, arena_base: int, desc_off: int, nrows_max: int):
        acc = np.zeros(max(nrows_max, 1), dtype=np.int64)
        n = self.lib.tmqo_phaseb_run(_ptr(arena), arena_base, desc_off, _ptr(acc))
        return n, acc


class Reference:
    """The reference's sim/ engine compiled in place (oracle/_ref)."""

    @staticmethod
    def available(path: str = REF_SO) -> bool:
        return os.path.exists(path)

    def __init__(self, path: str = REF_SO):
        L = self.lib = C.CDLL(path)
        _setup(L, "ref_f16_to_f32", C.c_float, [C.c_uint16])
        _setup(L, "ref_matmul", _i, [_u32, _P, _u64, _i, _i, _P, _P, _P])
        _setup(L, "ref_matmul_fp32", None, [_u32, _P, _u64, _i, _i, _P, _P])
        _setup(L, "ref_matmul_int16", None, [_u32, _P, _u64, _i, _i, _P, _P])
        _setup(L, "ref_model_set_flags", None, [C.c_uint])
        _setup(L, "ref_dump_tiles_open", _i, [_i, _i, C.c_char_p])
        _setup(L, "ref_dump_tiles_close", None, [])
        _setup(L, "ref_phaseb_verify", _i, [])
        _setup(L, "ref_phaseb_dump_files", None, [])
        _setup(L, "ref_model_logits_auto", None, [_P, _P])
        _setup(L, "ref_tile_q8", None, [_P, _P, _P, _P])
        _setup(L, "ref_tile_q5_0_8x896", None, [_P, _P, _P, _P, _i])
        _setup(L, "ref_tile_q6_k", None, [_P, _i, _P, _i, _P, _P, _i])
        _setup(L, "ref_tile_q4_k", None, [_P, _i, _P, _i, _P, _P, _i])
        _setup(L, "ref_tile_q5_0_4x896", None, [_P, _P, _P, _P, _i])
        _setup(L, "ref_tile_q4k_16", None, [_P, _P, _P])
        _setup(L, "ref_dequant_q4k_block_to_float", None, [_P, _P])
        _setup(L, "ref_phaseb_begin", _i, [])
        _setup(L, "ref_phaseb_end", None, [])
        _setup(L, "ref_phaseb_head", _u32, [])
        _setup(L, "ref_phaseb_next_off", _u32, [])
        _setup(L, "ref_phaseb_count", _i, [])
        _setup(L, "ref_ddr", _P, [])
        _setup(L, "ref_phaseb_run", _i, [_u32, _P])
        _setup(L, "ref_phaseb_alloc", _u32, [_u32])
        _setup(L, "ref_phaseb_add_descriptor", _u32,
               [_u32, _u32, _u32, C.c_uint16, C.c_uint16, C.c_uint8, C.c_uint8, C.c_uint8, C.c_uint16, C.c_uint8])
        _setup(L, "ref_model_load", _i, [C.c_char_p])
        _setup(L, "ref_model_prompt", _i, [_P, _i, _P])
        _setup(L, "ref_model_reset", None, [])
        _setup(L, "ref_model_logits", None, [_P, _P])
        _setup(L, "ref_model_step", None, [_P, _i, _i])
        _setup(L, "ref_model_step_dump", None, [_P, _i, _i, _P])
        _setup(L, "ref_apply_rope", None, [_P, _P, _i])
        _setup(L, "ref_timing_reset", None, [])
        _setup(L, "ref_timing_counts", None, [_P, _P])

    # ---- whole-model engine (sim/tmac_gguf.cpp:1894-2045), 896-wide only
    HIDDEN, VOCAB, LAYERS = 896, 151936, 24

    def model_load(self, path: str) -> None:
        assert self.lib.ref_model_load(path.encode()) == 0, "load_tmac failed"

    def model_prompt(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        h = np.empty(self.HIDDEN, dtype=np.float32)
        assert self.lib.ref_model_prompt(_ptr(t), t.size, _ptr(h)) == 0
        return h

    def model_reset(self) -> None:
        self.lib.ref_model_reset()

    def model_logits(self, hidden) -> np.ndarray:
        h = np.ascontiguousarray(hidden, dtype=np.float32)
        out = np.empty(self.VOCAB, dtype=np.float32)
        self.lib.ref_model_logits(_ptr(h), _ptr(out))
        return out

    def model_step(self, hidden: np.ndarray, token: int, pos: int, dump: bool = False):
        """process_embedding + all layers at pos; hidden updated in place.
        With dump, returns the hidden state after the embedding and each layer."""
        if dump:
            d = np.empty((self.LAYERS + 1, self.HIDDEN), dtype=np.float32)
            self.lib.ref_model_step_dump(_ptr(hidden), int(token), int(pos), _ptr(d))
            return d
        self.lib.ref_model_step(_ptr(hidden), int(token), int(pos))
        return None

    def matmul(self, qtype, w, x, rows, cols, row_max_abs=None) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(rows, dtype=np.float32)
        rc = self.lib.ref_matmul(qtype, _ptr(w), w.size, rows, cols, _ptr(x), _ptr(y), _ptr(row_max_abs))
        assert rc == 0
        return y

    def matmul_fp32(self, qtype, w, x, rows, cols) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(rows, dtype=np.float32)
        self.lib.ref_matmul_fp32(qtype, _ptr(w), w.size, rows, cols, _ptr(x), _ptr(y))
        return y

    def matmul_int16(self, qtype, w, x, rows, cols) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w).view(np.uint8)
        y = np.empty(rows, dtype=np.float32)
        self.lib.ref_matmul_int16(qtype, _ptr(w), w.size, rows, cols, _ptr(x), _ptr(y))
        return y

    def timing_reset(self):
        self.lib.ref_timing_reset()

    def timing_counts(self):
        """(tiles, MACs) of g_timing since the last reset"""
        t = np.zeros(1, dtype=np.int64)
        m = np.zeros(1, dtype=np.int64)
        self.lib.ref_timing_counts(_ptr(t), _ptr(m))
        return int(t[0]), int(m[0])

    def model_set_flags(self, flags: int):
        self.lib.ref_model_set_flags(int(flags))

    def model_logits_auto(self, hidden) -> np.ndarray:
        h = np.ascontiguousarray(hidden, dtype=np.float32)
        out = np.empty(self.VOCAB, dtype=np.float32)
        self.lib.ref_model_logits_auto(_ptr(h), _ptr(out))
        return out

    def tile_q8(self, W, cs, vec):
        r = np.zeros(64, dtype=np.int64)
        self.lib.ref_tile_q8(_ptr(W), _ptr(cs), _ptr(vec), _ptr(r))
        return r

    def tile_q5_0_8x896(self, blocks, act, row_inv, result, row_base):
        self.lib.ref_tile_q5_0_8x896(_ptr(blocks), _ptr(act), _ptr(row_inv), _ptr(result), row_base)

    def tile_kquant(self, qtype, blocks, nblocks, act, ncols, row_inv, result, row_base):
        f = self.lib.ref_tile_q6_k if qtype == Q6_K else self.lib.ref_tile_q4_k
        f(_ptr(blocks), nblocks, _ptr(act), ncols, _ptr(row_inv), _ptr(result), row_base)

    def tile_q5_0_4x896(self, blocks56, act, row_norm, result, row_base):
        self.lib.ref_tile_q5_0_4x896(_ptr(blocks56), _ptr(act), _ptr(row_norm), _ptr(result), row_base)

    def phaseb_build(self, calls):
        """Run matmul_fpga_* calls with descriptor building on; return
        (arena bytes from 0x18000000, base, head, ndesc)."""
        assert self.lib.ref_phaseb_begin() == 0
        try:
            for qtype, w, x, rows, cols in calls:
                self.matmul(qtype, w, x, rows, cols)
        finally:
            self.lib.ref_phaseb_end()
        base = 0x18000000
        end = self.lib.ref_phaseb_next_off()
        ddr = self.lib.ref_ddr()
        arena = np.frombuffer((C.c_uint8 * (end - base)).from_address(ddr + base), dtype=np.uint8).copy()
        return arena, base, self.lib.ref_phaseb_head(), self.lib.ref_phaseb_count()

    def phaseb_run(self, desc_off, nrows_max):
        acc = np.zeros(max(nrows_max, 1), dtype=np.int64)
        n = self.lib.ref_phaseb_run(desc_off, _ptr(acc))
        return n, acc
