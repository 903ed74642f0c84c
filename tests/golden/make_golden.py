"""Writes the golden fixtures in tests/golden (run from the repo root:
python tests/golden/make_golden.py).

  dequant_golden.npz  random + edge blocks of Q8_0 / Q4_K / Q6_K / F16 and
                      their dequantized values; every expected value is
                      computed twice, by the oracle's row decoders and by the
                      independent element-wise forms (tests/npref.py), and the
                      script refuses to write unless both agree bit-for-bit.
  decode_golden.npz   the synthetic 'tiny-q4_k' model (seed fixed in its
                      spec): oracle logits (f16 KV) for 4 teacher-forced
                      tokens, and 16 greedy ids from token 0.
The reference ships no fixtures (oracle_harness/fixtures/.gitignore); these
are the builder's, regenerated only when the oracle changes on purpose.
"""
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(REPO, "odin-infer_amd"), os.path.join(REPO, "oracle"), os.path.dirname(HERE)]

import npref  # noqa: E402
import refcpu  # noqa: E402
from helpers import random_blocks  # noqa: E402
from oi import synth  # noqa: E402

BLOCK = {8: (32, 34), 12: (256, 144), 14: (256, 210), 1: (1, 2)}


def edge_blocks(kind):
    out = []
    edge16 = [0x7BFF, 0x0001, 0x8000, 0x3C00, 0xFBFF, 0x0400, 0x03FF, 0x0000]
    e, b = BLOCK[kind]
    for i, d in enumerate(edge16):
        blk = (np.arange(b, dtype=np.int64) * (37 + 2 * i) % 256).astype(np.uint8)
        if kind == 12:
            blk[0:2] = np.array([d], np.uint16).view(np.uint8)
            blk[2:4] = np.array([edge16[-1 - i]], np.uint16).view(np.uint8)
        elif kind == 14:
            blk[208:210] = np.array([d], np.uint16).view(np.uint8)
        elif kind == 8:
            blk[0:2] = np.array([d], np.uint16).view(np.uint8)
        else:
            blk = np.array([d], np.uint16).view(np.uint8)
        out.append(blk)
    return np.concatenate(out)


def main():
    rng = np.random.default_rng(20261201)
    arrays = {}
    for kind, (e, b) in BLOCK.items():
        nb = 48 if e > 1 else 512
        blocks = np.concatenate([random_blocks(kind, nb, rng), edge_blocks(kind)])
        n = len(blocks) // b * e
        a = refcpu.dequant_row(kind, blocks, n)
        c = npref.dequant(kind, blocks, n)
        assert np.array_equal(np.isnan(a), np.isnan(c)) and np.array_equal(a[~np.isnan(a)].view(np.uint32),
                                                                           c[~np.isnan(c)].view(np.uint32))
        arrays["blocks_%d" % kind] = blocks
        arrays["values_%d" % kind] = a
    np.savez_compressed(os.path.join(HERE, "dequant_golden.npz"), **arrays)

    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "tiny.gguf")
        synth.write_gguf(path, "tiny-q4_k")
        r = refcpu.RefEngine(path, max_ctx=64, num_threads=4, kv_f16=True)
        tokens = np.array([0, 7, 123, 4000], np.int32)
        logits = np.stack([r.forward(int(t), i) for i, t in enumerate(tokens)])
        r.close()
        r = refcpu.RefEngine(path, max_ctx=64, num_threads=4, kv_f16=True)
        tok, ids = 0, []
        for pos in range(16):
            tok = refcpu.argmax(r.forward(tok, pos))
            ids.append(tok)
        r.close()
    np.savez_compressed(os.path.join(HERE, "decode_golden.npz"), model=np.array("tiny-q4_k"), tokens=tokens,
                        logits=logits.astype(np.float32), greedy=np.array(ids, np.int32))
    print("wrote", os.listdir(HERE))


if __name__ == "__main__":
    main()
