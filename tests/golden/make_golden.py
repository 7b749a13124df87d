"""Regenerate the golden fixtures in this directory.

Run in the build container (needs oracle/_ref/libmxref.so, which
`make -C oracle` compiles from the reference's own CPU sources):

    python tests/golden/make_golden.py

Outputs
  reference_kat.json  the reference's own known-answer blocks
                      (tests/test_cuda_quantized_matmul.cpp:18-42,
                      tests/test_cuda_quant_kernel_parity.cpp:26-67) with the
                      values the reference CPU code produces for them.
  ref_vectors.npz     seeded random inputs and the reference CPU outputs for:
                      Q4_K/Q8_0/Q5_0 block dequant, rhs-transposed matmul,
                      rmsnorm, rope (both pairings), softmax, and a 2-layer
                      decoder stack (transformer_forward_single_layer).
The reference's sources never leave the build container.  The CPU library
compiled from them (oracle/_ref/libmxref.so, git-ignored, so never committed)
travels with the working tree to GPU runs, where only the tests' checkers and
bench.py's reference-kind CPU-baseline leg load it; these vectors are the
committed record of its outputs.
"""
from __future__ import annotations

import ctypes as C
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT / "oracle"))
import mxo  # noqa: E402

REF = mxo.load_ref()
if REF is None:
    raise SystemExit("oracle/_ref/libmxref.so missing: run `make -C oracle` with /root/reference present")


def p(a):
    return a.ctypes.data


def ref_dequant(t, blocks: np.ndarray, be: int) -> np.ndarray:
    out = np.empty((len(blocks), be), np.float32)
    for i, b in enumerate(blocks):
        b = np.ascontiguousarray(b)
        assert REF.ref_dequant_block(t, p(b), p(out[i])) == 0
    return out


def ref_matmul(t, a, w, n):
    a = np.ascontiguousarray(a, np.float32)
    m, k = a.shape
    out = np.empty((m, n), np.float32)
    assert REF.ref_matmul_rhs_t(t, p(a), m, k, p(w), n, p(out)) == 0
    return out


def kat_blocks():
    q4 = np.zeros(144, np.uint8)
    q4[0:2] = [0x00, 0x3C]  # d = 1.0
    q4[2:4] = [0x00, 0x3C]  # dmin = 1.0
    q4[4 + 4] = 0x40
    q4[4 + 8] = 0x10
    q4[16 + 64] = 0x01
    q5 = np.zeros(22, np.uint8)
    q5[0:2] = [0x00, 0x3C]
    q5[6] = 0x0F
    q8 = np.zeros(34, np.uint8)
    q8[0:2] = [0x00, 0x3C]
    q8[2] = 0xFF
    return {"Q4_K": (mxo.Q4_K, q4, 256), "Q5_0": (mxo.Q5_0, q5, 32), "Q8_0": (mxo.Q8_0, q8, 32)}


def main():
    kat = {}
    for name, (t, blk, be) in kat_blocks().items():
        deq = ref_dequant(t, blk[None, :], be)[0]
        # parity test: every row is the crafted block, A = ones (K = N = block elems)
        w = np.tile(blk, be)
        y = ref_matmul(t, np.ones((1, be), np.float32), w, be)[0]
        kat[name] = {"type": t, "block_hex": blk.tobytes().hex(), "dequant": deq.tolist(), "ones_dot": float(y[0]),
                     "ones_dot_all_equal": bool(np.all(y == y[0]))}
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    kat["F32_matmul"] = {"a": a.tolist(), "b": b.tolist(), "c": [[58.0, 64.0], [139.0, 154.0]]}
    (HERE / "reference_kat.json").write_text(json.dumps(kat, indent=1))

    rng = np.random.default_rng(0x5EED)
    vec = {}
    # random raw blocks (any bit pattern, fp16 d limited to finite values)
    for t, be, bb in ((mxo.Q4_K, 256, 144), (mxo.Q8_0, 32, 34), (mxo.Q5_0, 32, 22)):
        blocks = rng.integers(0, 256, size=(512, bb), dtype=np.uint8)
        d = (rng.standard_normal((512, 2)) * 0.01).astype(np.float16).view(np.uint8)
        blocks[:, 0:2] = d[:, 0:2]
        if t == mxo.Q4_K:
            blocks[:, 2:4] = d[:, 2:4]
        vec[f"blocks_{t}"] = blocks
        vec[f"dequant_{t}"] = ref_dequant(t, blocks, be)
    # rhs-transposed matmul on quantizer-produced weights
    for t, k, n, m in ((mxo.Q4_K, 512, 48, 1), (mxo.Q4_K, 1024, 16, 3), (mxo.Q8_0, 512, 40, 1), (mxo.Q5_0, 256, 24, 2)):
        wf = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        wq = mxo.quantize(t, wf)
        a = rng.standard_normal((m, k)).astype(np.float32)
        vec[f"mm_{t}_{k}_{n}_{m}_w"] = wq
        vec[f"mm_{t}_{k}_{n}_{m}_a"] = a
        vec[f"mm_{t}_{k}_{n}_{m}_out"] = ref_matmul(t, a, wq, n)
    # rmsnorm
    x = rng.standard_normal((3, 1024)).astype(np.float32) * 3
    y = np.empty_like(x)
    assert REF.ref_rmsnorm(p(x), p(y), 3, 1024, C.c_float(1e-6)) == 0
    vec["rms_x"], vec["rms_y"] = x, y
    # rope, both pairings, several positions
    for neox in (0, 1):
        v = rng.standard_normal((1, 8 * 128)).astype(np.float32)
        outs = []
        for pos in (0, 1, 7, 1000, 8191):
            t_ = v.copy()
            REF.ref_rope(p(t_), 1, 8, 128, 0, pos, C.c_float(1e6), neox)
            outs.append(t_[0])
        vec[f"rope{neox}_x"], vec[f"rope{neox}_y"] = v[0], np.stack(outs)
    # softmax
    s = (rng.standard_normal(777) * 4).astype(np.float32)
    so = s.copy()
    REF.ref_softmax(p(so), so.size)
    vec["sm_x"], vec["sm_y"] = s, so
    np.savez_compressed(HERE / "ref_vectors.npz", **vec)
    print("wrote", HERE / "reference_kat.json", HERE / "ref_vectors.npz")


if __name__ == "__main__":
    main()


def layer_trace():
    """Per-layer hidden states of the reference decoder stack on the tiny model."""
    import tempfile
    sys.path.insert(0, str(ROOT / "tests"))
    import gguf_synth
    from layer_trace import TINY, TOKENS, ref_stack_trace
    keep = {}
    with tempfile.TemporaryDirectory() as td:
        gguf_synth.build(Path(td) / "tiny.gguf", gguf_synth.Arch(**TINY), seed=123, keep=keep)
    hidden = ref_stack_trace(keep, TINY, TOKENS)
    np.savez_compressed(HERE / "ref_layer_trace.npz", hidden=hidden, tokens=np.array(TOKENS))
    print("wrote", HERE / "ref_layer_trace.npz", hidden.shape)


if __name__ == "__main__" and "--layers" in sys.argv:
    layer_trace()


def ring_trace():
    """The same stack with a cache of RING_SEQ_MAX rows run past its end."""
    import tempfile
    sys.path.insert(0, str(ROOT / "tests"))
    import gguf_synth
    from layer_trace import RING_SEQ_MAX, RING_TOKENS, TINY, ref_stack_trace
    keep = {}
    with tempfile.TemporaryDirectory() as td:
        gguf_synth.build(Path(td) / "tiny.gguf", gguf_synth.Arch(**TINY), seed=123, keep=keep)
    hidden = ref_stack_trace(keep, TINY, RING_TOKENS, seq_max=RING_SEQ_MAX)
    np.savez_compressed(HERE / "ref_ring_trace.npz", hidden=hidden, tokens=np.array(RING_TOKENS),
                        seq_max=np.array(RING_SEQ_MAX))
    print("wrote", HERE / "ref_ring_trace.npz", hidden.shape)


if __name__ == "__main__" and "--ring" in sys.argv:
    ring_trace()
