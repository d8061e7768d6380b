"""Python binding of libtmq.so, the MI355X quantized-GEMV library (include/tmq.h).

A thin ctypes layer: every numeric result comes from the HIP kernels.  There
is no CPU fallback -- if libtmq.so is missing or the device is not a gfx950,
the calls raise.

    import tmq
    ctx = tmq.Context(0)
    t = ctx.upload(tmq.Q5_0, rows, cols, ggml_bytes)
    y = ctx.matmul(t, x)          # matmul_fpga_q5_0 drop-in
"""
from __future__ import annotations

import ctypes as C
import os
import weakref

import numpy as np

from . import synth  # noqa: F401  (re-export)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtmq.so")

F32, F16, Q5_0, Q8_0, Q4_K, Q6_K, CPU_OP = 0, 1, 6, 8, 12, 14, 15
QK = {Q8_0: 32, Q5_0: 32, Q4_K: 256, Q6_K: 256, F32: 32, F16: 32}
BLOCK_BYTES = {Q8_0: 34, Q5_0: 22, Q4_K: 144, Q6_K: 210, F32: 128, F16: 64}
# matmul branches and the reference's --fpga* flags (include/tmq.h)
PATH_FPGA, PATH_INT16, PATH_FP32 = 0, 1, 2
FLAG_FPGA, FLAG_Q8_0, FLAG_Q5_0, FLAG_Q4_K, FLAG_Q6_K = 1, 2, 4, 8, 16
FLAGS_ALL = 31
NOALLOC_MAX_COLS = 16384  # TMQ_NOALLOC_MAX_COLS

EXPORTS = [
    "tmq_last_error", "tmq_version", "tmq_open", "tmq_close", "tmq_stream", "tmq_sync",
    "tmq_tensor_upload", "tmq_tensor_upload_dev", "tmq_tensor_free", "tmq_tensor_info",
    "tmq_tensor_row_norm", "tmq_tensor_fit_stats", "tmq_tensor_ifit_stats", "tmq_matmul", "tmq_gemv_dev", "tmq_gemv_dev_noalloc",
    "tmq_gemv_partials", "tmq_route", "tmq_matmul_flags", "tmq_matmul_path", "tmq_gemv_dev_path",
    "tmq_gemv_partials_path", "tmq_tensor_prepare_int16",
    "tmq_vecmul_tile_q8", "tmq_vecmul_tile_q5_0_8x896", "tmq_vecmul_tile_q5_0_4x896", "tmq_vecmul_tile_q6_k",
    "tmq_vecmul_tile_q4k", "tmq_phaseb_run", "tmq_chain_create", "tmq_chain_run",
    "tmq_chain_prepare", "tmq_chain_launch",
    "tmq_chain_free", "tmq_chain_weight_bytes",
    "tmq_model_load", "tmq_model_load_mem", "tmq_model_free", "tmq_model_get_config",
    "tmq_model_weight_bytes", "tmq_model_position", "tmq_model_set_graphs", "tmq_model_prompt",
    "tmq_model_feed", "tmq_model_feed_dump", "tmq_model_logits", "tmq_model_generate",
    "tmq_model_generate_async", "tmq_model_tokens", "tmq_model_hidden", "tmq_model_set_prefill",
    "tmq_model_profile", "tmq_model_set_flags", "tmq_model_get_flags", "tmq_quantize_act",
    "tmq_tensor_q8_scales", "tmq_model_feed_capture", "tmq_model_tensor", "tmq_model_logits_capture",
    "tmq_model_reset", "tmq_matmul_tiles",
]


class LaunchTime(C.Structure):
    """tmq_launch_time"""
    _fields_ = [("name", C.c_char_p), ("start_ms", C.c_float), ("end_ms", C.c_float)]


def route(qtype: int, flags: int) -> int:
    """the matmul branch (PATH_*) the reference takes for a type under flags"""
    return _check(lib().tmq_route(qtype, flags))


def matmul_tiles(qtype: int, flags: int, rows: int, cols: int):
    """(tiles, MACs) one matmul adds to the reference's timing summary"""
    t, m = C.c_int64(0), C.c_int64(0)
    _check(lib().tmq_matmul_tiles(qtype, flags, rows, cols, C.byref(t), C.byref(m)))
    return t.value, m.value


class TmqError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"tmq error {code}: {msg}")
        self.code = code


class Desc(C.Structure):
    """tmq_desc"""
    _fields_ = [("weight", C.c_void_p), ("x_dev", C.c_void_p), ("y_dev", C.c_void_p),
                ("acc_dev", C.c_void_p), ("num_tiles", C.c_uint16),
                ("tile_res_rows", C.c_uint8), ("num_col_groups", C.c_uint8)]


_lib = None


def lib(path: str = LIB_PATH):
    """Load libtmq.so (raises if it is not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built: run __graft_entry__.build() "
                                f"or `make -C tmac-zynq-fpga_amd`")
    # PyTorch-ROCm ships its own libamdhip64 (same soname, libamdhip64.so.7).
    # Loading torch first lets libtmq.so bind to that runtime, so a process
    # that uses both has one HIP runtime (two runtimes cannot share the GPU).
    try:
        import torch  # noqa: F401
    except Exception:
        pass
    L = C.CDLL(path)
    P, I, U32, U64 = C.c_void_p, C.c_int, C.c_uint32, C.c_uint64
    sig = {
        "tmq_last_error": (C.c_char_p, []),
        "tmq_version": (C.c_char_p, []),
        "tmq_open": (I, [I, C.POINTER(P)]),
        "tmq_close": (I, [P]),
        "tmq_stream": (P, [P]),
        "tmq_sync": (I, [P]),
        "tmq_tensor_upload": (I, [P, U32, U64, U64, P, U64, P, C.POINTER(P)]),
        "tmq_tensor_upload_dev": (I, [P, U32, U64, U64, P, U64, P, C.POINTER(P)]),
        "tmq_tensor_free": (I, [P]),
        "tmq_tensor_info": (I, [P, P, P, P, P]),
        "tmq_tensor_row_norm": (I, [P, P, P]),
        "tmq_tensor_fit_stats": (I, [P, P, C.POINTER(U64), C.POINTER(U64)]),
        "tmq_tensor_ifit_stats": (I, [P, P, C.POINTER(U64), C.POINTER(U64)]),
        "tmq_matmul": (I, [P, P, P, P, I, I]),
        "tmq_gemv_dev": (I, [P, P, P, P, P]),
        "tmq_gemv_dev_noalloc": (I, [P, P, P, P, P]),
        "tmq_gemv_partials": (I, [P, P, P, P, U64, P]),
        "tmq_route": (I, [U32, U32]),
        "tmq_matmul_tiles": (I, [U32, U32, U64, U64, P, P]),
        "tmq_matmul_flags": (I, [P, P, U32, P, P, I, I]),
        "tmq_matmul_path": (I, [P, P, I, P, P, I, I]),
        "tmq_gemv_dev_path": (I, [P, P, I, P, P, P]),
        "tmq_gemv_partials_path": (I, [P, P, I, P, P, U64, P]),
        "tmq_tensor_prepare_int16": (I, [P, P]),
        "tmq_vecmul_tile_q8": (I, [P, P, P, P, P]),
        "tmq_vecmul_tile_q5_0_8x896": (I, [P, P, P, P, P, I]),
        "tmq_vecmul_tile_q5_0_4x896": (I, [P, P, P, P, P, I]),
        "tmq_vecmul_tile_q6_k": (I, [P, P, I, P, I, P, P, I]),
        "tmq_vecmul_tile_q4k": (I, [P, P, I, P, I, P, P, I]),
        "tmq_phaseb_run": (I, [P, P, U64, U32, U32, P, I]),
        "tmq_chain_create": (I, [P, P, I, C.POINTER(P)]),
        "tmq_chain_run": (I, [P, P]),
        "tmq_chain_prepare": (I, [P, P]),
        "tmq_chain_launch": (I, [P, P]),
        "tmq_chain_free": (I, [P]),
        "tmq_chain_weight_bytes": (U64, [P]),
        "tmq_model_load": (I, [P, C.c_char_p, I, C.POINTER(P)]),
        "tmq_model_load_mem": (I, [P, P, U64, I, C.POINTER(P)]),
        "tmq_model_free": (I, [P]),
        "tmq_model_get_config": (I, [P, P]),
        "tmq_model_weight_bytes": (U64, [P]),
        "tmq_model_position": (I, [P]),
        "tmq_model_set_graphs": (I, [P, I]),
        "tmq_model_set_prefill": (I, [P, I]),
        "tmq_model_set_flags": (I, [P, U32]),
        "tmq_quantize_act": (I, [P, P, I, P, P]),
        "tmq_tensor_q8_scales": (I, [P, P, P]),
        "tmq_model_feed_capture": (I, [P, C.c_int32, P]),
        "tmq_model_tensor": (P, [P, C.c_char_p]),
        "tmq_model_logits_capture": (I, [P, P, P]),
        "tmq_model_reset": (I, [P]),
        "tmq_model_get_flags": (U32, [P]),
        "tmq_model_profile": (I, [P, I, P, I, C.POINTER(C.c_int)]),
        "tmq_model_prompt": (I, [P, P, I]),
        "tmq_model_feed": (I, [P, C.c_int32]),
        "tmq_model_feed_dump": (I, [P, C.c_int32, P]),
        "tmq_model_logits": (I, [P, P]),
        "tmq_model_generate": (I, [P, I, P]),
        "tmq_model_generate_async": (I, [P, I]),
        "tmq_model_tokens": (I, [P, I, I, P]),
        "tmq_model_hidden": (I, [P, P]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def _check(rc: int):
    if rc < 0:
        raise TmqError(rc, lib().tmq_last_error().decode())
    return rc


def _p(a):
    if a is None:
        return None
    if isinstance(a, int):
        return a
    return a.ctypes.data_as(C.c_void_p)


class Tensor:
    def __init__(self, ctx: "Context", handle, qtype: int, rows: int, cols: int):
        self.ctx, self.handle, self.qtype, self.rows, self.cols = ctx, handle, qtype, rows, cols
        ctx._adopt(self)
        wb = C.c_uint64()
        _check(lib().tmq_tensor_info(handle, None, None, None, C.byref(wb)))
        self.weight_bytes = wb.value

    def row_norm(self) -> np.ndarray:
        out = np.empty(self.rows, dtype=np.float32)
        _check(lib().tmq_tensor_row_norm(self.ctx.handle, self.handle, _p(out)))
        return out

    def fit_stats(self):
        """(fitted, exact) sub-block counts of the upload-time decode fits"""
        f, e = C.c_uint64(), C.c_uint64()
        _check(lib().tmq_tensor_fit_stats(self.ctx.handle, self.handle, C.byref(f), C.byref(e)))
        return f.value, e.value

    def ifit_stats(self):
        """(blocks, corrections) of the MFMA decoders' integer fit (0, 0:
        the tensor takes the fitted-float decoders)"""
        b, c = C.c_uint64(), C.c_uint64()
        _check(lib().tmq_tensor_ifit_stats(self.ctx.handle, self.handle, C.byref(b), C.byref(c)))
        return b.value, c.value

    def free(self):
        if self.handle:
            lib().tmq_tensor_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Chain:
    def __init__(self, ctx: "Context", descs):
        self.ctx = ctx
        arr = (Desc * len(descs))()
        self._keep = []
        for i, d in enumerate(descs):
            t, x, y, acc, nt, tr, ncg = d
            self._keep.append(t)
            arr[i] = Desc(t.handle, x, y, acc, nt, tr, ncg)
        h = C.c_void_p()
        _check(lib().tmq_chain_create(ctx.handle, arr, len(descs), C.byref(h)))
        self.handle = h
        ctx._adopt(self)
        self.weight_bytes = lib().tmq_chain_weight_bytes(h)

    def run(self):
        _check(lib().tmq_chain_run(self.ctx.handle, self.handle))

    def prepare(self):
        _check(lib().tmq_chain_prepare(self.ctx.handle, self.handle))

    def launch(self):
        _check(lib().tmq_chain_launch(self.ctx.handle, self.handle))

    def free(self):
        if self.handle:
            lib().tmq_chain_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Context:
    """A device and stream (tmq_open).  Tensors, chains and models made from
    it are freed at the latest by close(): the library needs its context
    alive to free them, so anything still alive then is freed first and
    their own free() becomes a no-op."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        _check(lib().tmq_open(device, C.byref(h)))
        self.handle = h
        self._children = weakref.WeakSet()

    def _adopt(self, obj):
        self._children.add(obj)

    @property
    def stream(self) -> int:
        return lib().tmq_stream(self.handle)

    def sync(self):
        _check(lib().tmq_sync(self.handle))

    def close(self):
        if self.handle:
            for obj in list(self._children):
                obj.free()
            lib().tmq_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- tensors ---------------------------------------------------------
    def upload(self, qtype: int, rows: int, cols: int, data: np.ndarray, row_max_abs=None) -> Tensor:
        data = np.ascontiguousarray(data, dtype=np.uint8)
        if row_max_abs is not None:
            row_max_abs = np.ascontiguousarray(row_max_abs, dtype=np.float32)
        h = C.c_void_p()
        _check(lib().tmq_tensor_upload(self.handle, qtype, rows, cols, _p(data), data.size,
                                       _p(row_max_abs), C.byref(h)))
        return Tensor(self, h, qtype, rows, cols)

    def upload_dev(self, qtype: int, rows: int, cols: int, data_ptr: int, nbytes: int) -> Tensor:
        h = C.c_void_p()
        _check(lib().tmq_tensor_upload_dev(self.handle, qtype, rows, cols, data_ptr, nbytes, None,
                                           C.byref(h)))
        return Tensor(self, h, qtype, rows, cols)

    # -- GEMV ------------------------------------------------------------
    def matmul(self, t: Tensor, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(t.rows, dtype=np.float32)
        _check(lib().tmq_matmul(self.handle, t.handle, _p(x), _p(y), t.rows, t.cols))
        return y

    def matmul_path(self, t: Tensor, x: np.ndarray, path: int) -> np.ndarray:
        """one branch of the reference's matmul (PATH_FPGA / PATH_INT16 / PATH_FP32)"""
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(t.rows, dtype=np.float32)
        _check(lib().tmq_matmul_path(self.handle, t.handle, path, _p(x), _p(y), t.rows, t.cols))
        return y

    def matmul_flags(self, t: Tensor, x: np.ndarray, flags: int) -> np.ndarray:
        """the reference's matmul under its --fpga* flags (FLAG_*)"""
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(t.rows, dtype=np.float32)
        _check(lib().tmq_matmul_flags(self.handle, t.handle, flags, _p(x), _p(y), t.rows, t.cols))
        return y

    def partials_int16(self, t: Tensor, x: np.ndarray):
        """INT16 path: int64 [rows][ceil(cols/64)] tile results and x_scale"""
        x = np.ascontiguousarray(x, dtype=np.float32)
        acc = np.empty((t.rows, (t.cols + 63) // 64), dtype=np.int64)
        xs = np.zeros(1, dtype=np.float32)
        _check(lib().tmq_gemv_partials_path(self.handle, t.handle, PATH_INT16, _p(x), _p(acc), acc.size, _p(xs)))
        return acc, xs[0]

    def gemv_dev_path(self, t: Tensor, path: int, x_ptr: int, y_ptr: int | None, acc_ptr: int | None = None):
        _check(lib().tmq_gemv_dev_path(self.handle, t.handle, path, x_ptr, y_ptr, acc_ptr))

    def partials(self, t: Tensor, x: np.ndarray):
        x = np.ascontiguousarray(x, dtype=np.float32)
        if t.qtype == Q8_0:
            acc = np.empty((t.rows, (t.cols + 63) // 64), dtype=np.int64)
        else:
            acc = np.empty(t.rows, dtype=np.int64)
        xs = np.zeros(1, dtype=np.float32)
        _check(lib().tmq_gemv_partials(self.handle, t.handle, _p(x), _p(acc), acc.size, _p(xs)))
        return acc, xs[0]

    def gemv_dev(self, t: Tensor, x_ptr: int, y_ptr: int | None, acc_ptr: int | None = None):
        _check(lib().tmq_gemv_dev(self.handle, t.handle, x_ptr, y_ptr, acc_ptr))

    def gemv_dev_noalloc(self, t: Tensor, x_ptr: int, y_ptr: int | None, acc_ptr: int | None = None):
        """tmq_gemv_dev from the library's fixed scratch (no device allocation)"""
        _check(lib().tmq_gemv_dev_noalloc(self.handle, t.handle, x_ptr, y_ptr, acc_ptr))

    def quantize_act(self, x: np.ndarray):
        """(int16 xq, x_scale) as every matmul_fpga_* quantises x, on the GPU"""
        x = np.ascontiguousarray(x, dtype=np.float32)
        xq = np.empty(x.size, dtype=np.int16)
        xs = np.zeros(1, dtype=np.float32)
        _check(lib().tmq_quantize_act(self.handle, _p(x), x.size, _p(xq), _p(xs)))
        return xq, xs[0]

    def q8_scales(self, t: Tensor) -> np.ndarray:
        out = np.empty((t.rows, t.cols // 32), dtype=np.uint16)
        _check(lib().tmq_tensor_q8_scales(self.handle, t.handle, _p(out)))
        return out

    # -- tiles -----------------------------------------------------------
    def tile_q8(self, W, cs, vec) -> np.ndarray:
        out = np.zeros(64, dtype=np.int64)
        _check(lib().tmq_vecmul_tile_q8(self.handle, _p(W), _p(cs), _p(vec), _p(out)))
        return out

    def tile_q5_0_8x896(self, blocks, act, row_inv, result, row_base):
        _check(lib().tmq_vecmul_tile_q5_0_8x896(self.handle, _p(blocks), _p(act), _p(row_inv),
                                                _p(result), row_base))

    def tile_q5_0_4x896(self, blocks56, act, row_norm, result, row_base):
        """axi_vecmul_tile_q5_0_4x896_axilite: 56 interleaved 48-byte block
        pairs, act int16[896], row_norm float32[4]; result[row_base+i] += acc_i"""
        if (blocks56.dtype != np.uint8 or blocks56.size < 56 * 48 or act.dtype != np.int16 or act.size < 896
                or row_norm.dtype != np.float32 or row_norm.size < 4 or result.dtype != np.int64
                or not 0 <= row_base <= result.size - 4):
            raise ValueError("tile_q5_0_4x896: uint8[2688], int16[896], float32[4], int64 result with 4 rows "
                             "from row_base")
        _check(lib().tmq_vecmul_tile_q5_0_4x896(self.handle, _p(blocks56), _p(act), _p(row_norm),
                                                _p(result), row_base))

    def tile_kquant(self, qtype, blocks, nblocks, act, ncols, row_inv, result, row_base):
        f = lib().tmq_vecmul_tile_q6_k if qtype == Q6_K else lib().tmq_vecmul_tile_q4k
        _check(f(self.handle, _p(blocks), nblocks, _p(act), ncols, _p(row_inv), _p(result), row_base))

    # -- chains ----------------------------------------------------------
    def phaseb_run(self, arena: np.ndarray, arena_base: int, head: int, max_desc: int = 4096):
        rows = np.zeros(max_desc, dtype=np.uint32)
        n = _check(lib().tmq_phaseb_run(self.handle, _p(arena), arena.size, arena_base, head,
                                        _p(rows), max_desc))
        return n, rows[:n].copy()

    def chain(self, descs) -> Chain:
        return Chain(self, descs)


class ModelConfig(C.Structure):
    """tmq_model_config"""
    _fields_ = [("n_layers", C.c_int32), ("hidden", C.c_int32), ("inter", C.c_int32),
                ("vocab", C.c_int32), ("n_heads", C.c_int32), ("n_kv_heads", C.c_int32),
                ("head_dim", C.c_int32), ("max_seq", C.c_int32), ("rope_base", C.c_float),
                ("norm_eps", C.c_float)]


class Model:
    """A .tmac model resident on the GPU (tmq_model_*): the reference engine's
    load_tmac / process_prompt / get_logits_q8 / generate (greedy)."""

    def __init__(self, ctx: Context, src, max_seq: int = 512):
        h = C.c_void_p()
        if isinstance(src, (str, os.PathLike)):
            _check(lib().tmq_model_load(ctx.handle, os.fspath(src).encode(), max_seq, C.byref(h)))
        else:
            buf = np.frombuffer(src, dtype=np.uint8) if not isinstance(src, np.ndarray) else src
            buf = np.ascontiguousarray(buf, dtype=np.uint8)
            _check(lib().tmq_model_load_mem(ctx.handle, _p(buf), buf.size, max_seq, C.byref(h)))
        self.ctx, self.handle = ctx, h
        ctx._adopt(self)
        cfg = ModelConfig()
        _check(lib().tmq_model_get_config(h, C.byref(cfg)))
        self.config = {f: getattr(cfg, f) for f, _ in ModelConfig._fields_}
        self.weight_bytes = lib().tmq_model_weight_bytes(h)

    @property
    def position(self) -> int:
        return lib().tmq_model_position(self.handle)

    def set_graphs(self, enable: bool):
        _check(lib().tmq_model_set_graphs(self.handle, int(bool(enable))))

    def profile(self, n: int):
        """n greedy decode steps launched one by one with GPU events:
        [(operation, start_ms, end_ms)] per launch (tmq_model_profile)."""
        per = 3 + 6 * self.config["n_layers"]
        buf = (LaunchTime * (n * per))()
        cnt = C.c_int(0)
        _check(lib().tmq_model_profile(self.handle, n, C.cast(buf, C.c_void_p), n * per, C.byref(cnt)))
        return [(buf[i].name.decode(), buf[i].start_ms, buf[i].end_ms) for i in range(cnt.value)]

    def set_flags(self, flags: int):
        """the reference's --fpga* flags (FLAG_*): per-type matmul routing and
        get_logits_q8 vs get_logits"""
        _check(lib().tmq_model_set_flags(self.handle, int(flags)))

    @property
    def flags(self) -> int:
        return lib().tmq_model_get_flags(self.handle)

    def set_prefill(self, chunk: int):
        """0: prompts one token at a time; > 0: batched prefill in chunks of
        this many tokens (default 512)."""
        _check(lib().tmq_model_set_prefill(self.handle, int(chunk)))

    def prompt(self, tokens):
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        _check(lib().tmq_model_prompt(self.handle, _p(t), t.size))

    def feed_capture(self, token: int) -> np.ndarray:
        """one more position; the fp32 input of every matmul per layer:
        [attn_norm out (H) | context (H) | ffn_norm out (H) | silu*up (I)]"""
        c = self.config
        out = np.empty((c["n_layers"], 3 * c["hidden"] + c["inter"]), dtype=np.float32)
        _check(lib().tmq_model_feed_capture(self.handle, int(token), _p(out)))
        return out

    def feed(self, token: int, dump: bool = False):
        if dump:
            out = np.empty((self.config["n_layers"] + 1, self.config["hidden"]), dtype=np.float32)
            _check(lib().tmq_model_feed_dump(self.handle, int(token), _p(out)))
            return out
        _check(lib().tmq_model_feed(self.handle, int(token)))
        return None

    def logits(self) -> np.ndarray:
        out = np.empty(self.config["vocab"], dtype=np.float32)
        _check(lib().tmq_model_logits(self.handle, _p(out)))
        return out

    def generate(self, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.int32)
        _check(lib().tmq_model_generate(self.handle, n, _p(out)))
        return out

    def generate_async(self, n: int):
        _check(lib().tmq_model_generate_async(self.handle, n))

    def tokens(self, first: int, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.int32)
        _check(lib().tmq_model_tokens(self.handle, first, n, _p(out)))
        return out

    def hidden(self) -> np.ndarray:
        out = np.empty(self.config["hidden"], dtype=np.float32)
        _check(lib().tmq_model_hidden(self.handle, _p(out)))
        return out

    def free(self):
        if self.handle:
            lib().tmq_model_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
