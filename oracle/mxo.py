"""ctypes binding of the CPU oracle (liboracle.so) and of the reference build
(_ref/libmxref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
CPU-baseline leg of bench.py, as the checker.  The product never imports it.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
REF_LIB = HERE / "_ref" / "libmxref.so"

F32, F16, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 6, 8, 12, 13, 14
Q1_0 = 41  # GGUF type 41: one byte per element, the byte's value (widened to F32 at load)
FORM_REF, FORM_GGML = 0, 1
OPEN_ROPE_NEOX, OPEN_KV_FP16, OPEN_GGML_FORM, OPEN_NO_QK_NORM = 1, 2, 4, 8
BLOCK = {F32: (1, 4), F16: (1, 2), Q5_0: (32, 22), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176),
         Q6_K: (256, 210), Q1_0: (1, 1)}


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "array must be C-contiguous"
    return a.ctypes.data


class ModelInfo(C.Structure):
    _fields_ = [(n, C.c_int) for n in
                ("n_layer", "n_embd", "n_head", "n_head_kv", "head_dim", "n_ff", "n_vocab", "n_ctx")] + \
               [("eps", C.c_float), ("rope_theta", C.c_float)] + \
               [(n, C.c_int) for n in ("has_qk_norm", "has_bias", "tied_output", "type_wq", "type_wffn_down",
                                       "type_output", "type_embd")]


def _load():
    if not LIB.exists():
        raise ImportError(f"{LIB} not built; run `make -C {HERE}`")
    lib = C.CDLL(str(LIB))
    vp, sz, ip, fp = C.c_void_p, C.c_size_t, C.c_int, C.c_float
    sig = {
        "mxo_fp16_to_fp32": (fp, [C.c_uint16]),
        "mxo_fp32_to_fp16": (C.c_uint16, [fp]),
        "mxo_dequant_rows": (ip, [ip, vp, sz, sz, vp, ip]),
        "mxo_matmul_rhs_t": (ip, [ip, vp, sz, sz, vp, sz, vp, ip, ip]),
        "mxo_quantize_q8_0_row": (None, [vp, sz, vp]),
        "mxo_quantize_q4k_row": (None, [vp, sz, vp]),
        "mxo_quantize_q5k_row": (None, [vp, sz, vp]),
        "mxo_quantize_q5_0_row": (None, [vp, sz, vp]),
        "mxo_quantize_q6k_row": (None, [vp, sz, vp]),
        "mxo_rmsnorm": (None, [vp, vp, vp, sz, fp]),
        "mxo_rope": (None, [vp, sz, sz, sz, sz, fp, ip]),
        "mxo_softmax": (None, [vp, sz]),
        "mxo_silu": (fp, [fp]),
        "mxo_model_open": (vp, [C.c_char_p, ip, ip, ip]),
        "mxo_model_close": (None, [vp]),
        "mxo_model_info_get": (None, [vp, C.POINTER(ModelInfo)]),
        "mxo_model_reset": (None, [vp]),
        "mxo_model_step": (ip, [vp, ip, vp, vp]),
        "mxo_model_pos": (ip, [vp]),
        "mxo_model_set_pos": (ip, [vp, ip]),
        "mxo_argmax": (ip, [vp, sz]),
        "mxo_sample": (ip, [vp, sz, ip, C.c_double, C.c_double, C.c_double, C.POINTER(C.c_uint64)]),
        "mxo_logit_edits": (None, [vp, sz, vp, sz, vp, sz, ip, C.c_double, C.c_double, C.c_double]),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype, f.argtypes = res, args
    return lib


lib = _load()


def row_bytes(t: int, cols: int) -> int:
    be, bb = BLOCK[t]
    assert cols % be == 0
    return cols // be * bb


def fp16_to_fp32(h: int) -> float:
    return lib.mxo_fp16_to_fp32(h)


def dequant(t: int, w: np.ndarray, rows: int, cols: int, form: int = FORM_REF) -> np.ndarray:
    out = np.empty((rows, cols), np.float32)
    w = np.ascontiguousarray(w)
    assert lib.mxo_dequant_rows(t, _p(w), rows, cols, _p(out), form) == 0
    return out


def matmul_rhs_t(t: int, a: np.ndarray, w: np.ndarray, n: int, form: int = FORM_REF, threads: int = 8) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    if a.ndim == 1:
        a = a[None, :]
    m, k = a.shape
    out = np.empty((m, n), np.float32)
    w = np.ascontiguousarray(w)
    assert lib.mxo_matmul_rhs_t(t, _p(a), m, k, _p(w), n, _p(out), form, threads) == 0
    return out


_QUANT = {Q8_0: "mxo_quantize_q8_0_row", Q4_K: "mxo_quantize_q4k_row", Q5_K: "mxo_quantize_q5k_row",
          Q5_0: "mxo_quantize_q5_0_row", Q6_K: "mxo_quantize_q6k_row"}


def quantize(t: int, x: np.ndarray) -> np.ndarray:
    """Quantize a [rows x cols] float32 matrix into raw GGUF bytes (uint8)."""
    x = np.ascontiguousarray(x, np.float32)
    if t == F32:
        return x.view(np.uint8).reshape(-1).copy()
    if t == F16:
        return x.astype(np.float16).view(np.uint8).reshape(-1).copy()
    if t == Q1_0:  # the synthetic writer's bytes: small non-negative integers
        return np.clip(np.rint(x * np.float32(64) + np.float32(2)), 0, 255).astype(np.uint8).reshape(-1)
    n = x.size
    out = np.empty(n // BLOCK[t][0] * BLOCK[t][1], np.uint8)
    getattr(lib, _QUANT[t])(_p(x), n, _p(out))
    return out


def rmsnorm(x: np.ndarray, w: np.ndarray | None, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib.mxo_rmsnorm(_p(x), _p(w) if w is not None else None, _p(y), x.size, eps)
    return y


def rope(v: np.ndarray, n_heads: int, head_dim: int, pos: int, theta: float, neox: bool = False) -> np.ndarray:
    v = np.array(v, np.float32, copy=True)
    lib.mxo_rope(_p(v), n_heads, head_dim, 0, pos, theta, int(neox))
    return v


def softmax(x: np.ndarray) -> np.ndarray:
    x = np.array(x, np.float32, copy=True)
    lib.mxo_softmax(_p(x), x.size)
    return x


def sample(logits: np.ndarray, top_k: int, temperature: float, top_p: float, min_p: float, state: int):
    st = C.c_uint64(state)
    logits = np.ascontiguousarray(logits, np.float32)
    tok = lib.mxo_sample(_p(logits), logits.size, top_k, temperature, top_p, min_p, C.byref(st))
    return tok, st.value


def logit_edits(logits: np.ndarray, history, suppress=(), repeat_last_n: int = 64, repeat_penalty: float = 1.0,
                frequency_penalty: float = 0.0, presence_penalty: float = 0.0) -> np.ndarray:
    """The reference's logit edits (minxfmr.cpp:2047-2089) on a copy of logits."""
    out = np.array(logits, np.float32, copy=True)
    h = np.ascontiguousarray(history, np.int32)
    s = np.ascontiguousarray(suppress, np.int32)
    lib.mxo_logit_edits(_p(out), out.size, _p(h) if h.size else None, h.size, _p(s) if s.size else None, s.size,
                        repeat_last_n, repeat_penalty, frequency_penalty, presence_penalty)
    return out


class Model:
    """Whole-model CPU oracle over a GGUF file (one token per step)."""

    def __init__(self, path: str, n_ctx: int, flags: int = 0, threads: int = 8):
        self.h = lib.mxo_model_open(str(path).encode(), n_ctx, flags, threads)
        if not self.h:
            raise RuntimeError(f"oracle could not open {path}")
        info = ModelInfo()
        lib.mxo_model_info_get(self.h, C.byref(info))
        self.info = info

    def step(self, token: int, want_logits: bool = True, trace: bool = False):
        i = self.info
        logits = np.empty(i.n_vocab, np.float32) if want_logits else None
        tr = np.empty((i.n_layer + 1) * i.n_embd, np.float32) if trace else None
        rc = lib.mxo_model_step(self.h, token, _p(logits) if logits is not None else None,
                                _p(tr) if tr is not None else None)
        if rc != 0:
            raise RuntimeError("oracle step failed")
        return logits, (tr.reshape(i.n_layer + 1, i.n_embd) if tr is not None else None)

    def reset(self):
        lib.mxo_model_reset(self.h)

    def set_pos(self, pos: int):
        """Jump to position `pos` (cache rows below keep their contents); for timing."""
        if lib.mxo_model_set_pos(self.h, pos) != 0:
            raise ValueError(f"position {pos} outside the context")

    def close(self):
        if self.h:
            lib.mxo_model_close(self.h)
            self.h = None

    def __del__(self):
        self.close()


def load_ref():
    """The reference's own CPU code (compiled by oracle/Makefile), or None."""
    if not REF_LIB.exists():
        return None
    r = C.CDLL(str(REF_LIB))
    vp, sz, ip, fp = C.c_void_p, C.c_size_t, C.c_int, C.c_float
    sig = {
        "ref_fp16_to_fp32": (fp, [C.c_uint16]),
        "ref_dequant_block": (ip, [ip, vp, vp]),
        "ref_matmul_rhs_t": (ip, [ip, vp, sz, sz, vp, sz, vp]),
        "ref_rmsnorm": (ip, [vp, vp, sz, sz, fp]),
        "ref_rope": (None, [vp, sz, sz, sz, sz, sz, fp, ip]),
        "ref_softmax": (None, [vp, sz]),
        "ref_cache_new": (vp, [sz, sz, sz]),
        "ref_cache_free": (None, [vp]),
        "ref_layer_forward": (ip, [vp, vp, sz, sz, vp, sz, sz, sz, vp, vp, vp, vp, vp, vp, fp, fp, ip]),
        "ref_gguf_to_f32": (ip, [ip, vp, sz, C.c_uint32, C.c_uint32, vp]),
    }
    for name, (res, args) in sig.items():
        f = getattr(r, name)
        f.restype, f.argtypes = res, args
    return r
