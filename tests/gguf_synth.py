"""Seeded synthetic GGUF models for tests and the benchmark's parity legs.

Writes GGUF v3 files with llama.cpp tensor names and `<arch>.*` metadata; 2D
weights are N(0, 0.02) fp32 quantized by the oracle's quantizers, norm weights
are F32 ones (plus a small seeded perturbation so they are not trivial).
Test infrastructure: uses the oracle's quantizers.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

import mxo

GGUF_MAGIC = 0x46554747
ALIGN = 32


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _kv(key: str, val) -> bytes:
    out = _str(key)
    if isinstance(val, bool):
        out += struct.pack("<IB", 7, int(val))
    elif isinstance(val, int):
        out += struct.pack("<II", 4, val)
    elif isinstance(val, float):
        out += struct.pack("<If", 6, val)
    elif isinstance(val, str):
        out += struct.pack("<I", 8) + _str(val)
    elif isinstance(val, list):
        out += struct.pack("<IIQ", 9, 8, len(val)) + b"".join(_str(s) for s in val)
    else:
        raise TypeError(key)
    return out


def write_gguf(path: Path, meta: dict, tensors: list[tuple[str, int, list[int], np.ndarray]]) -> None:
    """tensors: (name, ggml type, ne (fastest first), raw bytes as uint8)."""
    head = struct.pack("<IIQQ", GGUF_MAGIC, 3, len(tensors), len(meta) + 1)
    head += _kv("general.alignment", ALIGN)
    for k, v in meta.items():
        head += _kv(k, v)
    offs, off = [], 0
    for name, t, ne, data in tensors:
        off = (off + ALIGN - 1) // ALIGN * ALIGN
        offs.append(off)
        off += data.nbytes
    for (name, t, ne, data), o in zip(tensors, offs):
        head += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        head += struct.pack("<IQ", t, o)
    pad = (-len(head)) % ALIGN
    with open(path, "wb") as f:
        f.write(head + b"\0" * pad)
        pos = 0
        for (name, t, ne, data), o in zip(tensors, offs):
            if o > pos:
                f.write(b"\0" * (o - pos))
                pos = o
            f.write(np.ascontiguousarray(data).tobytes())
            pos += data.nbytes


@dataclass
class Arch:
    name: str = "qwen3"
    n_layer: int = 2
    n_embd: int = 256
    n_head: int = 4
    n_head_kv: int = 2
    head_dim: int = 64
    n_ff: int = 512
    n_vocab: int = 512
    ctx: int = 4096
    rope_theta: float = 1e6
    eps: float = 1e-6
    qk_norm: bool = True
    tied: bool = False
    wtype: int = mxo.Q4_K
    out_type: int = mxo.Q8_0
    embd_type: int = mxo.Q8_0
    overrides: dict = field(default_factory=dict)  # tensor suffix -> type (e.g. "attn_v": Q5_K)


QWEN3_06B = dict(name="qwen3", n_layer=28, n_embd=1024, n_head=16, n_head_kv=8, head_dim=128, n_ff=3072,
                 n_vocab=151936, qk_norm=True, tied=True, wtype=mxo.Q8_0, out_type=mxo.Q8_0, embd_type=mxo.Q8_0)
QWEN3_8B = dict(name="qwen3", n_layer=36, n_embd=4096, n_head=32, n_head_kv=8, head_dim=128, n_ff=12288,
                n_vocab=151936, qk_norm=True, tied=False, wtype=mxo.Q4_K, out_type=mxo.Q8_0, embd_type=mxo.Q4_K)
LLAMA3_8B = dict(name="llama", n_layer=32, n_embd=4096, n_head=32, n_head_kv=8, head_dim=128, n_ff=14336,
                 n_vocab=128256, qk_norm=False, tied=False, wtype=mxo.Q4_K, out_type=mxo.Q8_0, embd_type=mxo.Q4_K,
                 rope_theta=5e5, overrides={"attn_v": mxo.Q5_K, "ffn_down": mxo.Q5_K})


def _weight(rng, rows, cols, t):
    w = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02)
    return mxo.quantize(t, w)


def build(path: Path, arch: Arch, seed: int = 0, keep: dict | None = None) -> Path:
    """Write the synthetic model; returns the path.  Deterministic in `seed`.
    When `keep` is a dict it receives name -> (type, ne, raw bytes)."""
    rng = np.random.default_rng(seed)
    a = arch
    qd, kvd = a.n_head * a.head_dim, a.n_head_kv * a.head_dim
    tensors = []

    def add(name, t, rows, cols):
        tensors.append((name, t, [cols, rows], _weight(rng, rows, cols, t)))

    def add_norm(name, n):
        v = (1.0 + 0.02 * rng.standard_normal(n)).astype(np.float32)
        tensors.append((name, mxo.F32, [n], v.view(np.uint8)))

    # output.weight first in the directory, as GGUF writers emit it
    if not a.tied:
        add("output.weight", a.out_type, a.n_vocab, a.n_embd)
    add("token_embd.weight", a.embd_type, a.n_vocab, a.n_embd)
    add_norm("output_norm.weight", a.n_embd)
    for l in range(a.n_layer):
        def t_of(role):
            return a.overrides.get(role, a.wtype)
        add_norm(f"blk.{l}.attn_norm.weight", a.n_embd)
        add(f"blk.{l}.attn_q.weight", t_of("attn_q"), qd, a.n_embd)
        add(f"blk.{l}.attn_k.weight", t_of("attn_k"), kvd, a.n_embd)
        add(f"blk.{l}.attn_v.weight", t_of("attn_v"), kvd, a.n_embd)
        if a.qk_norm:
            add_norm(f"blk.{l}.attn_q_norm.weight", a.head_dim)
            add_norm(f"blk.{l}.attn_k_norm.weight", a.head_dim)
        add(f"blk.{l}.attn_output.weight", t_of("attn_output"), a.n_embd, qd)
        add_norm(f"blk.{l}.ffn_norm.weight", a.n_embd)
        add(f"blk.{l}.ffn_gate.weight", t_of("ffn_gate"), a.n_ff, a.n_embd)
        add(f"blk.{l}.ffn_up.weight", t_of("ffn_up"), a.n_ff, a.n_embd)
        add(f"blk.{l}.ffn_down.weight", t_of("ffn_down"), a.n_embd, a.n_ff)
    p = a.name
    meta = {
        "general.architecture": p,
        "general.name": f"synthetic-{p}-seed{seed}",
        f"{p}.block_count": a.n_layer,
        f"{p}.context_length": a.ctx,
        f"{p}.embedding_length": a.n_embd,
        f"{p}.feed_forward_length": a.n_ff,
        f"{p}.attention.head_count": a.n_head,
        f"{p}.attention.head_count_kv": a.n_head_kv,
        f"{p}.attention.key_length": a.head_dim,
        f"{p}.attention.value_length": a.head_dim,
        f"{p}.rope.freq_base": float(a.rope_theta),
        f"{p}.attention.layer_norm_rms_epsilon": float(a.eps),
    }
    write_gguf(Path(path), meta, tensors)
    if keep is not None:
        for name, t, ne, data in tensors:
            keep[name] = (t, ne, data)
    return Path(path)
