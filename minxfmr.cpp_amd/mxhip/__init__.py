"""ctypes binding of the gfx950 backend's C ABI (include/minxfmr_hip.h).

The shared library is built in-tree by ``make -C minxfmr.cpp_amd``; importing
this module loads it and fails loudly if it is missing.  There is no CPU
fallback: every call runs on the GPU or returns an error.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

PKG_DIR = Path(__file__).resolve().parent.parent
LIB_PATH = PKG_DIR / "lib" / "libminxfmr_hip.so"

F32, F16, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 6, 8, 12, 13, 14
Q1_0 = 41  # GGUF type 41: one byte per element, the byte's value (widened to F32 at load)
FORM_REF, FORM_GGML = 0, 1
BLOCK = {F32: (1, 4), F16: (1, 2), Q5_0: (32, 22), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176),
         Q6_K: (256, 210), Q1_0: (1, 1)}
TYPE_NAMES = {F32: "F32", F16: "F16", Q5_0: "Q5_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K",
              Q1_0: "Q1_0"}


class MxhError(RuntimeError):
    pass


def row_bytes(type_: int, cols: int) -> int:
    be, bb = BLOCK[type_]
    if cols % be:
        raise ValueError(f"cols={cols} not a multiple of {be}")
    return cols // be * bb


class ModelConfig(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_layer", "n_embd", "n_head", "n_head_kv", "head_dim", "n_ff", "n_vocab",
                                       "n_ctx")] + \
               [("eps", C.c_float), ("rope_theta", C.c_float)] + \
               [(n, C.c_int) for n in ("has_qk_norm", "has_bias", "type_wq", "type_wv", "type_wffn_down",
                                       "type_output", "type_embd")] + \
               [("weight_bytes", C.c_int64), ("step_read_bytes", C.c_int64)]


class SynthArch(C.Structure):
    _fields_ = [("arch", C.c_char_p)] + \
               [(n, C.c_int) for n in ("n_layer", "n_embd", "n_head", "n_head_kv", "head_dim", "n_ff", "n_vocab",
                                       "ctx")] + \
               [("rope_theta", C.c_float), ("eps", C.c_float)] + \
               [(n, C.c_int) for n in ("qk_norm", "tied", "wtype", "out_type", "embd_type", "attn_v_type",
                                       "ffn_down_type")]


MODEL_ROPE_NEOX, MODEL_GGML_FORM, MODEL_NO_QK_NORM, MODEL_NO_GRAPH, MODEL_TOKEN_PREFILL, MODEL_GGUF_LAYOUT = 1, 4, 8, 16, 32, 64
TILED_FLAG = 0x100
MODEL_BF16_PREFILL = 128


def _load() -> C.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(f"{LIB_PATH} is not built; run `make -C {PKG_DIR}` (or __graft_entry__.build())")
    lib = C.CDLL(str(LIB_PATH))
    vp, i64, sz, fp, ip = C.c_void_p, C.c_int64, C.c_size_t, C.POINTER(C.c_float), C.c_int
    sig = {
        "mxh_init": (ip, [ip]),
        "mxh_is_available": (ip, []),
        "mxh_last_error": (C.c_char_p, []),
        "mxh_synchronize": (ip, []),
        "mxh_stream": (vp, []),
        "mxh_alloc": (ip, [C.POINTER(vp), sz]),
        "mxh_free": (ip, [vp]),
        "mxh_upload": (ip, [vp, vp, sz]),
        "mxh_download": (ip, [vp, vp, sz]),
        "mxh_memset": (ip, [vp, ip, sz]),
        "mxh_copy": (ip, [vp, vp, sz]),
        "mxh_gemm_q_bf16": (ip, [ip, vp, i64, vp, i64, i64, vp, ip]),
        "mxh_gemm_q_f16": (ip, [ip, vp, i64, vp, i64, i64, vp, ip]),
        "mxh_gemm_q_f16_noalloc": (ip, [ip, vp, i64, vp, i64, i64, vp, ip]),
        "mxh_attention_prefill": (ip, [vp, vp, vp, vp, ip, ip, ip, ip, ip]),
        "mxh_tile_rows": (ip, [ip, vp, i64, i64, C.POINTER(C.c_int)]),
        "mxh_timer_begin": (ip, []),
        "mxh_timer_end": (ip, [fp]),
        "mxh_gemv": (ip, [ip, vp, vp, vp, i64, i64, ip]),
        "mxh_matmul_rhs_t": (ip, [ip, vp, i64, vp, i64, i64, vp, ip]),
        "mxh_dequant": (ip, [ip, vp, vp, i64, i64, ip]),
        "mxh_preload": (ip, [vp, sz]),
        "mxh_release_resources": (None, []),
        "mxh_host_matmul_rhs_t": (ip, [ip, vp, i64, i64, vp, sz, i64, vp, ip]),
        "mxh_host_matmul_f32": (ip, [vp, vp, vp, i64, i64, i64]),
        "mxh_host_matmul_q": (ip, [ip, vp, i64, i64, vp, sz, i64, vp, ip]),
        "mxh_host_matvec_strided": (ip, [vp, vp, vp, sz, sz, sz]),
        "mxh_host_vec_dot_rows": (ip, [vp, vp, vp, sz, sz, sz]),
        "mxh_host_vec_dot_rows_ring": (ip, [vp, vp, sz, sz, sz, sz, sz, vp]),
        "mxh_host_vec_mul_rows_cols": (ip, [vp, vp, vp, sz, sz, sz]),
        "mxh_model_open": (ip, [C.c_char_p, ip, ip, C.POINTER(vp)]),
        "mxh_model_config_get": (ip, [vp, C.POINTER(ModelConfig)]),
        "mxh_model_reset": (ip, [vp]),
        "mxh_model_position": (ip, [vp]),
        "mxh_model_step": (ip, [vp, ip, vp, vp]),
        "mxh_model_prefill": (ip, [vp, vp, ip]),
        "mxh_model_set_sampling": (ip, [vp, ip, C.c_double, C.c_double, C.c_double, C.c_uint64]),
        "mxh_model_set_logit_edits": (ip, [vp, vp, ip, ip, C.c_double, C.c_double, C.c_double]),
        "mxh_sample": (ip, [vp, ip, ip, C.c_double, C.c_double, C.c_double, C.c_uint64, C.c_uint64, C.POINTER(C.c_int)]),
        "mxh_model_generate": (ip, [vp, vp, ip, ip, vp, C.POINTER(C.c_float), C.POINTER(C.c_float)]),
        "mxh_model_close": (None, [vp]),
        "mxh_model_decode": (ip, [vp, ip, vp, C.POINTER(C.c_float)]),
        "mxh_model_set_token": (ip, [vp, ip]),
        "mxh_model_bench_gemv": (ip, [vp, ip, ip, C.POINTER(C.c_float), C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
        "mxh_model_bench_attention": (ip, [vp, ip, C.POINTER(C.c_float), C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
        "mxh_write_synthetic_gguf": (ip, [C.c_char_p, C.POINTER(SynthArch), C.c_uint64, ip]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()
EXPORTED = (
    "mxh_init mxh_is_available mxh_last_error mxh_synchronize mxh_stream mxh_alloc mxh_free mxh_upload "
    "mxh_download mxh_memset mxh_copy mxh_gemm_q_bf16 mxh_gemm_q_f16 mxh_gemm_q_f16_noalloc mxh_attention_prefill mxh_tile_rows mxh_timer_begin mxh_timer_end mxh_gemv mxh_matmul_rhs_t mxh_dequant mxh_preload "
    "mxh_release_resources mxh_host_matmul_rhs_t mxh_host_matmul_f32 mxh_host_matmul_q mxh_host_matvec_strided "
    "mxh_host_vec_dot_rows mxh_host_vec_dot_rows_ring mxh_host_vec_mul_rows_cols mxh_model_open "
    "mxh_model_config_get mxh_model_reset mxh_model_position mxh_model_step mxh_model_prefill mxh_model_set_sampling mxh_model_set_logit_edits mxh_sample mxh_model_generate mxh_model_close "
    "mxh_write_synthetic_gguf mxh_model_decode mxh_model_set_token mxh_model_bench_gemv mxh_model_bench_attention"
).split()


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = lib.mxh_last_error().decode(errors="replace")
        raise MxhError(f"{what or 'mxh call'} failed ({rc}): {msg}")


def ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


class DeviceBuffer:
    """A device allocation owned by Python (freed on close / garbage collection)."""

    def __init__(self, nbytes: int):
        p = C.c_void_p()
        check(lib.mxh_alloc(C.byref(p), max(int(nbytes), 1)), "mxh_alloc")
        self.ptr = p.value
        self.nbytes = int(nbytes)

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        buf = cls(a.nbytes)
        if a.nbytes:
            check(lib.mxh_upload(buf.ptr, ptr(a), a.nbytes), "upload")
        return buf

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        check(lib.mxh_upload(self.ptr + offset, ptr(a), a.nbytes), "upload")

    def download(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        if out.nbytes:
            check(lib.mxh_download(ptr(out), self.ptr + offset, out.nbytes), "download")
        return out

    def close(self) -> None:
        if self.ptr:
            lib.mxh_free(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def init(device: int = 0) -> None:
    check(lib.mxh_init(device), "mxh_init")


def available() -> bool:
    return bool(lib.mxh_is_available())


def synchronize() -> None:
    check(lib.mxh_synchronize(), "synchronize")


def gemv(type_: int, w: DeviceBuffer | int, x: DeviceBuffer | int, y: DeviceBuffer | int, n: int, k: int,
         form: int = FORM_REF) -> None:
    addr = lambda b: b.ptr if isinstance(b, DeviceBuffer) else int(b)
    check(lib.mxh_gemv(type_, addr(w), addr(x), addr(y), n, k, form), "mxh_gemv")


def gemm_bf16(type_: int, a: DeviceBuffer, m: int, w: DeviceBuffer, n: int, k: int, out: DeviceBuffer,
              form: int = FORM_REF) -> None:
    """out[m x n] = bf16(a) . bf16(dequant(w))^T on the matrix cores."""
    check(lib.mxh_gemm_q_bf16(type_, a.ptr, m, w.ptr, n, k, out.ptr, form), "mxh_gemm_q_bf16")


def gemm_f16(type_: int, a: DeviceBuffer, m: int, w: DeviceBuffer, n: int, k: int, out: DeviceBuffer,
             form: int = FORM_REF) -> None:
    """out[m x n] = a . dequant(w)^T on the fp16 matrix cores with exact weight codes."""
    check(lib.mxh_gemm_q_f16(type_, a.ptr, m, w.ptr, n, k, out.ptr, form), "mxh_gemm_q_f16")


def tile_rows(type_: int, w: DeviceBuffer, rows: int, cols: int) -> int:
    """Regroup device weight rows in place into the tiled order; returns the type id for gemv from then on."""
    t = C.c_int(-1)
    check(lib.mxh_tile_rows(type_, w.ptr, rows, cols, C.byref(t)), "mxh_tile_rows")
    return t.value


def attention_prefill(q: DeviceBuffer, kc: DeviceBuffer, vc: DeviceBuffer, att: DeviceBuffer, p0: int, m: int,
                      nh: int, nkv: int, hd: int) -> None:
    """Causal attention of m prompt tokens at positions p0.. over the fp16 K/V cache (matrix cores)."""
    check(lib.mxh_attention_prefill(q.ptr, kc.ptr, vc.ptr, att.ptr, p0, m, nh, nkv, hd), "mxh_attention_prefill")


def sample(logits: DeviceBuffer, n: int, top_k: int, temperature: float, top_p: float = 1.0, min_p: float = 0.0,
           seed: int = 0, draw: int = 0) -> int:
    """One device sampling decision over n logits (draw number `draw` of the seeded stream)."""
    tok = C.c_int(-1)
    check(lib.mxh_sample(logits.ptr, n, top_k, temperature, top_p, min_p, seed, draw, C.byref(tok)), "mxh_sample")
    return tok.value


def memset(buf: DeviceBuffer, value: int) -> None:
    check(lib.mxh_memset(buf.ptr, value, buf.nbytes), "mxh_memset")


def copy(dst: DeviceBuffer, src: DeviceBuffer, nbytes: int) -> None:
    """Device-to-device copy on the library stream (asynchronous)."""
    assert nbytes <= dst.nbytes and nbytes <= src.nbytes
    check(lib.mxh_copy(dst.ptr, src.ptr, nbytes), "mxh_copy")


def dequant(type_: int, w: DeviceBuffer, rows: int, cols: int, form: int = FORM_REF) -> np.ndarray:
    out = DeviceBuffer(rows * cols * 4)
    check(lib.mxh_dequant(type_, w.ptr, out.ptr, rows, cols, form), "mxh_dequant")
    res = out.download(np.float32, rows * cols).reshape(rows, cols)
    out.close()
    return res


def host_matmul_rhs_t(type_: int, a: np.ndarray, w: np.ndarray, n: int, form: int = FORM_REF) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    m, k = a.shape
    out = np.empty((m, n), dtype=np.float32)
    check(lib.mxh_host_matmul_rhs_t(type_, ptr(a), m, k, ptr(w), w.nbytes, n, ptr(out), form), "matmul_rhs_t")
    return out


class Timer:
    """Elapsed milliseconds of the work enqueued on the library stream."""

    def __enter__(self):
        check(lib.mxh_timer_begin(), "timer_begin")
        return self

    def __exit__(self, *exc):
        ms = C.c_float()
        check(lib.mxh_timer_end(C.byref(ms)), "timer_end")
        self.ms = ms.value
        return False


def write_synthetic_gguf(path, arch: str = "qwen3", *, n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab,
                         ctx=4096, rope_theta=1e6, eps=1e-6, qk_norm=True, tied=False, wtype=Q4_K, out_type=Q8_0,
                         embd_type=Q8_0, attn_v_type=-1, ffn_down_type=-1, seed=0, threads=0) -> None:
    """Seeded synthetic GGUF written by the library's C++ writer (host only)."""
    a = SynthArch(arch.encode(), n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab, ctx, rope_theta, eps,
                  int(qk_norm), int(tied), wtype, out_type, embd_type, attn_v_type, ffn_down_type)
    check(lib.mxh_write_synthetic_gguf(str(path).encode(), C.byref(a), seed, threads), "write_synthetic_gguf")


class Model:
    """A GGUF decoder model resident in HBM (device-side decode step)."""

    def __init__(self, path, n_ctx: int, flags: int = 0):
        h = C.c_void_p()
        check(lib.mxh_model_open(str(path).encode(), n_ctx, flags, C.byref(h)), "mxh_model_open")
        self.h = h.value
        cfg = ModelConfig()
        check(lib.mxh_model_config_get(self.h, C.byref(cfg)), "config")
        self.cfg = cfg

    def reset(self) -> None:
        check(lib.mxh_model_reset(self.h), "reset")

    @property
    def position(self) -> int:
        return lib.mxh_model_position(self.h)

    def set_sampling(self, top_k: int, temperature: float, top_p: float = 1.0, min_p: float = 0.0, seed: int = 0):
        """Top-k / temperature sampling on the device (temperature <= 0: greedy)."""
        check(lib.mxh_model_set_sampling(self.h, top_k, temperature, top_p, min_p, seed), "set_sampling")

    def set_logit_edits(self, suppress=(), repeat_last_n: int = 64, repeat_penalty: float = 1.0,
                        frequency_penalty: float = 0.0, presence_penalty: float = 0.0):
        """Suppressed ids and repetition / frequency / presence penalties applied before each choice."""
        ids = np.ascontiguousarray(suppress, np.int32)
        check(lib.mxh_model_set_logit_edits(self.h, ptr(ids) if ids.size else None, ids.size, repeat_last_n,
                                            repeat_penalty, frequency_penalty, presence_penalty), "set_logit_edits")

    def prefill(self, tokens) -> None:
        """Feed prompt ids at the current position (no logits)."""
        t = np.ascontiguousarray(tokens, np.int32)
        check(lib.mxh_model_prefill(self.h, ptr(t) if t.size else None, t.size), "prefill")

    def step(self, token: int, logits: bool = True, trace: bool = False):
        c = self.cfg
        lg = np.empty(c.n_vocab, np.float32) if logits else None
        tr = np.empty((c.n_layer + 1) * c.n_embd, np.float32) if trace else None
        check(lib.mxh_model_step(self.h, token, ptr(lg) if lg is not None else None,
                                 ptr(tr) if tr is not None else None), "step")
        return lg, (tr.reshape(c.n_layer + 1, c.n_embd) if tr is not None else None)

    def generate(self, prompt, n_gen: int):
        """Greedy ids; returns (ids, prefill_ms, decode_ms)."""
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(n_gen, np.int32)
        pm, dm = C.c_float(), C.c_float()
        check(lib.mxh_model_generate(self.h, ptr(p), p.size, n_gen, ptr(out), C.byref(pm), C.byref(dm)), "generate")
        return out, pm.value, dm.value

    def decode(self, n_gen: int):
        """Continue greedy decoding; returns (ids, decode_ms)."""
        out = np.empty(n_gen, np.int32)
        ms = C.c_float()
        check(lib.mxh_model_decode(self.h, n_gen, ptr(out), C.byref(ms)), "decode")
        return out, ms.value

    def set_token(self, token: int) -> None:
        """Make `token` the id at the current position (the next decode input)."""
        check(lib.mxh_model_set_token(self.h, token), "set_token")

    def bench_attention(self, reps: int = 1):
        """(device ms, launches, algorithmic bytes) of every layer's decode attention at the current position."""
        ms, n, b = C.c_float(), C.c_int64(), C.c_int64()
        check(lib.mxh_model_bench_attention(self.h, reps, C.byref(ms), C.byref(n), C.byref(b)), "bench_attention")
        return ms.value, n.value, b.value

    def bench_gemv(self, type_: int, reps: int = 1):
        """(device ms, launches, algorithmic bytes) of every `type_` GEMV of the model."""
        ms, n, b = C.c_float(), C.c_int64(), C.c_int64()
        check(lib.mxh_model_bench_gemv(self.h, type_, reps, C.byref(ms), C.byref(n), C.byref(b)), "bench_gemv")
        return ms.value, n.value, b.value

    def close(self) -> None:
        if self.h:
            lib.mxh_model_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
