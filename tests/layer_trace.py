"""Reference decoder-stack trace helper (test infrastructure).

Drives the reference's transformer_forward_single_layer (via oracle/_ref) over
a token sequence, mirroring run_stack_forward (src/api/minxfmr.cpp:544-663):
embedding row dequantized, layers in order with a shared KV cache.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

import mxo

TINY = dict(name="qwen3", n_layer=2, n_embd=256, n_head=4, n_head_kv=2, head_dim=64, n_ff=512, n_vocab=300,
            qk_norm=False, tied=False, wtype=mxo.Q4_K, out_type=mxo.Q8_0, embd_type=mxo.Q8_0)
TOKENS = [5, 17, 299, 0, 42, 42, 7]
# a cache of RING_SEQ_MAX rows run past its end: the reference's ring
# (kv_cache.cpp:50-75) overwrites the oldest row and RoPE positions stop at
# seq_max (transformer.cpp:506)
RING_SEQ_MAX = 5
RING_TOKENS = [5, 17, 299, 0, 42, 42, 7, 3, 250, 11, 11, 64, 128, 9]


def ref_stack_trace(keep: dict, arch: dict, tokens: list[int], seq_max: int = 64) -> np.ndarray:
    ref = mxo.load_ref()
    d, nl = arch["n_embd"], arch["n_layer"]
    kvd = arch["n_head_kv"] * arch["head_dim"]
    cache = ref.ref_cache_new(nl, seq_max, kvd)
    t_e, ne_e, emb = keep["token_embd.weight"]
    emb_rows = mxo.dequant(t_e, emb, arch["n_vocab"], d)
    roles = ["attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"]
    out = []
    for tok in tokens:
        x = np.ascontiguousarray(emb_rows[tok:tok + 1])
        per_layer = []
        for l in range(nl):
            ws = [keep[f"blk.{l}.{r}.weight"] for r in roles]
            types = (C.c_int * 7)(*[w[0] for w in ws])
            ptrs = (C.c_void_p * 7)(*[w[2].ctypes.data for w in ws])
            rows = (C.c_size_t * 7)(*[w[1][1] for w in ws])
            cols = (C.c_size_t * 7)(*[w[1][0] for w in ws])
            an = keep[f"blk.{l}.attn_norm.weight"][2].view(np.float32)
            fn = keep[f"blk.{l}.ffn_norm.weight"][2].view(np.float32)
            y = np.empty_like(x)
            rc = ref.ref_layer_forward(x.ctypes.data, y.ctypes.data, 1, d, cache, l, arch["n_head"],
                                       arch["n_head_kv"], types, ptrs, rows, cols, an.ctypes.data, fn.ctypes.data,
                                       C.c_float(1e6), C.c_float(1e-6), 0)
            assert rc == 0
            per_layer.append(y[0].copy())
            x = y
        out.append(np.stack(per_layer))
    ref.ref_cache_free(cache)
    return np.stack(out)
