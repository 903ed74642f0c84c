"""Replays the committed golden fixtures (tests/golden, written by
make_golden.py): the oracle on the CPU, and the HIP path on the GPU."""
import os
import tempfile

import numpy as np
import pytest

import refcpu
from helpers import same_bits, scaled_err
from oi import ggml, infer, synth

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DQ = np.load(os.path.join(HERE, "dequant_golden.npz"))
DEC = np.load(os.path.join(HERE, "decode_golden.npz"))
KINDS = [8, 12, 14, 1]


@pytest.mark.parametrize("kind", KINDS)
def test_oracle_dequant_golden(kind):
    blocks, values = DQ["blocks_%d" % kind], DQ["values_%d" % kind]
    assert same_bits(refcpu.dequant_row(kind, blocks, len(values)), values)


@pytest.fixture(scope="module")
def golden_model():
    with tempfile.TemporaryDirectory(prefix="oi_golden_") as d:
        path = os.path.join(d, "tiny.gguf")
        synth.write_gguf(path, str(DEC["model"]))
        yield path


def test_oracle_decode_golden(golden_model):
    r = refcpu.RefEngine(golden_model, max_ctx=64, num_threads=4, kv_f16=True)
    try:
        for i, t in enumerate(DEC["tokens"]):
            assert scaled_err(r.forward(int(t), i), DEC["logits"][i]) <= 1e-6
    finally:
        r.close()


@pytest.mark.gpu
@pytest.mark.parametrize("kind", KINDS)
def test_gpu_dequant_golden(kind):
    blocks, values = DQ["blocks_%d" % kind], DQ["values_%d" % kind]
    e = 256 if kind in (12, 14) else 64
    n = len(values) // e * e
    nbytes = ggml.row_byte_size(kind, n)
    assert same_bits(ggml.dequant_row(kind, blocks[:nbytes], n), values[:n])


@pytest.mark.gpu
def test_gpu_decode_golden(golden_model):
    e, _ = infer.engine_load(golden_model, infer.Engine_Opts(max_ctx=64))
    try:
        for i, t in enumerate(DEC["tokens"]):
            assert scaled_err(infer.engine_forward(e, int(t), i), DEC["logits"][i]) <= 1e-3
        assert np.array_equal(infer.engine_decode_greedy(e, 0, 0, 16), DEC["greedy"])
    finally:
        infer.engine_destroy(e)
