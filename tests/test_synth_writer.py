"""The library's C++ synthetic GGUF writer (host code, CPU only): the oracle
reads what it writes, shapes/types/metadata are as requested, weights are
N(0, 0.02) after dequantization, and output is independent of thread count."""
from __future__ import annotations

import hashlib

import numpy as np

import mxhip
import mxo


def _write(path, threads, **kw):
    args = dict(n_layer=2, n_embd=256, n_head=4, n_head_kv=2, head_dim=64, n_ff=512, n_vocab=300, seed=7)
    args.update(kw)
    mxhip.write_synthetic_gguf(path, threads=threads, **args)
    return path


def test_oracle_reads_writer_output(tmp_path):
    p = _write(tmp_path / "m.gguf", 3, wtype=mxhip.Q4_K, out_type=mxhip.Q8_0, embd_type=mxhip.Q8_0,
               attn_v_type=mxhip.Q5_K)
    m = mxo.Model(p, 16)
    i = m.info
    assert (i.n_layer, i.n_embd, i.n_head, i.n_head_kv, i.head_dim, i.n_ff, i.n_vocab) == (2, 256, 4, 2, 64, 512, 300)
    assert i.has_qk_norm == 1 and i.tied_output == 0 and i.type_wq == mxo.Q4_K and i.type_output == mxo.Q8_0
    lg, tr = m.step(3, trace=True)
    assert np.all(np.isfinite(lg)) and np.all(np.isfinite(tr))


def test_thread_count_does_not_change_bytes(tmp_path):
    a = _write(tmp_path / "a.gguf", 1)
    b = _write(tmp_path / "b.gguf", 5)
    assert hashlib.sha256(a.read_bytes()).digest() == hashlib.sha256(b.read_bytes()).digest()


def test_writer_quantizers_round_trip(tmp_path):
    """Dequantized weights (ggml scale form, which the writer packs for) have
    the requested N(0, 0.02) statistics."""
    import struct
    for t in (mxhip.Q4_K, mxhip.Q5_K, mxhip.Q6_K, mxhip.Q8_0, mxhip.Q5_0, mxhip.F16):
        p = _write(tmp_path / f"w{t}.gguf", 2, wtype=t, n_layer=1)
        raw = p.read_bytes()
        # locate blk.0.ffn_gate.weight through the oracle-independent header walk
        m = mxo.Model(p, 4)
        assert m.info.type_wq == t
        m.close()
        # statistics of the whole gate matrix: rows 512 x cols 256
        name = b"blk.0.ffn_gate.weight"
        at = raw.index(name) + len(name)
        n_dims = struct.unpack_from("<I", raw, at)[0]
        ne = struct.unpack_from("<" + "Q" * n_dims, raw, at + 4)
        ttype, off = struct.unpack_from("<IQ", raw, at + 4 + 8 * n_dims)
        assert ttype == t and ne == (256, 512)
        # data section starts at the first 32-aligned offset after the directory,
        # whose last entry is blk.0.ffn_down.weight (2 dims)
        dirend = raw.index(b"blk.0.ffn_down.weight") + len(b"blk.0.ffn_down.weight") + 4 + 16 + 12
        data0 = (dirend + 31) // 32 * 32
        nb = mxo.row_bytes(t, 256) * 512
        w = np.frombuffer(raw, np.uint8, nb, data0 + off)
        vals = mxo.dequant(t, w, 512, 256, mxo.FORM_GGML)
        assert abs(vals.mean()) < 2e-3
        assert abs(vals.std() - 0.02) < 0.02 * (0.12 if t == mxhip.Q4_K else 0.06)


def test_q4_k_m_mix_opens_in_the_oracle(tmp_path):
    """A llama.cpp Q4_K_M-style mix (Q6_K head, attn_v and ffn_down, F16
    embedding) written by the library opens in the oracle, which multiplies
    Q6_K and F16 rows as the F32 values the reference's loader makes of
    them; the step is finite and the types are as written."""
    p = _write(tmp_path / "q4km.gguf", 2, wtype=mxhip.Q4_K, out_type=mxhip.Q6_K, embd_type=mxhip.F16,
               attn_v_type=mxhip.Q6_K, ffn_down_type=mxhip.Q6_K)
    m = mxo.Model(p, 4)
    i = m.info
    assert (i.type_wq, i.type_wffn_down, i.type_output, i.type_embd) == (mxo.Q4_K, mxo.Q6_K, mxo.Q6_K, mxo.F16)
    lg, tr = m.step(1, trace=True)
    assert np.all(np.isfinite(lg)) and np.all(np.isfinite(tr))
    m.close()


def test_type41_tensors(tmp_path):
    """GGUF type 41 (one byte per element, the byte's value) for attn_v and
    ffn_down: the file holds rows * cols bytes for them, the writer's bytes
    are round(64 x + 2) of its N(0, 0.02) draws, and the oracle opens and
    steps the model."""
    import struct
    p = _write(tmp_path / "t41.gguf", 2, wtype=mxhip.Q4_K, out_type=mxhip.Q8_0, embd_type=mxhip.Q8_0,
               attn_v_type=mxhip.Q1_0, ffn_down_type=mxhip.Q1_0, n_layer=1)
    raw = p.read_bytes()
    name = b"blk.0.ffn_down.weight"
    at = raw.index(name) + len(name)
    n_dims = struct.unpack_from("<I", raw, at)[0]
    ne = struct.unpack_from("<" + "Q" * n_dims, raw, at + 4)
    ttype, off = struct.unpack_from("<IQ", raw, at + 4 + 8 * n_dims)
    assert ttype == 41 and ne == (512, 256)
    data0 = (at + 4 + 8 * n_dims + 12 + 31) // 32 * 32
    w = np.frombuffer(raw, np.uint8, 256 * 512, data0 + off).astype(np.float64)
    assert abs(w.mean() - 2.0) < 0.05 and abs(w.std() - 1.28) < 0.08
    m = mxo.Model(p, 4)
    assert m.info.type_wffn_down == mxo.Q1_0
    lg, tr = m.step(5, trace=True)
    assert np.all(np.isfinite(lg)) and np.all(np.isfinite(tr))
    m.close()
