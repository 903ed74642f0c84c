"""CPU tests of the product around the kernels: the C ABI library loads and
exports every declared symbol, the loader reports malformed models as error
codes in the reference's order (file and model checks before the device), the
synthetic models are what the measurement plan says, and the Python mirror of
the Engine API keeps the reference's names and tables.  No GPU needed."""
import ctypes
import os
import re
import struct
import subprocess
import sys

import numpy as np
import pytest

import refcpu
from oi import _native, ggml, infer, synth

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header):
    text = open(os.path.join(REPO, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(oi_[a-z0-9_]+)\s*\(", text)))


@pytest.mark.parametrize("header,lib", [("oi.h", _native.LIB_HIP), ("oi_synth.h", _native.LIB_SYNTH)])
def test_library_exports_every_declared_symbol(header, lib):
    names = declared(header)
    assert len(names) >= 5
    L = ctypes.CDLL(lib)
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    if header == "oi.h":
        # the Python binding covers exactly the C ABI header of the HIP library
        assert set(declared("oi.h")) == set(_native.HIP_SYMBOLS)


def prototypes(header):
    """name -> number of parameters of every function declared in header."""
    text = open(os.path.join(REPO, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(oi_[a-z0-9_]+)\s*\(([^()]*)\)\s*;", text):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


@pytest.mark.parametrize("header", ["oi.h"])
def test_binding_arity_matches_header(header):
    """The ctypes argument lists have as many entries as the C prototypes
    (a short list silently passes garbage in the missing registers)."""
    protos = prototypes(header)
    assert protos
    for name, n in protos.items():
        assert len(_native.HIP_SYMBOLS[name][1]) == n, (name, n, len(_native.HIP_SYMBOLS[name][1]))


def _load_rc(path, max_ctx=64):
    L = _native.hip()
    o = _native.Opts(max_ctx, 1, 1, 0)
    h = ctypes.c_void_p()
    rc = L.oi_engine_load(str(path).encode(), ctypes.byref(o), ctypes.byref(h))
    if rc == 0:
        L.oi_engine_destroy(h)
    return rc, L.oi_last_error().decode()


def _patch_tensor_type(data, name, new_type):
    """Rewrite the type id of tensor `name` in a GGUF byte string."""
    key = struct.pack("<Q", len(name)) + name.encode()
    i = data.index(key) + len(key)
    nd = struct.unpack_from("<I", data, i)[0]
    t = i + 4 + 8 * nd
    return data[:t] + struct.pack("<I", new_type) + data[t + 4:]


def test_engine_load_errors(make_model, tmp_path):
    OI_E_IO, OI_E_FORMAT, OI_E_MODEL, OI_E_UNSUPPORTED, OI_E_DEVICE = -2, -3, -4, -5, -7
    assert _load_rc(tmp_path / "missing.gguf")[0] == OI_E_IO
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUX" + bytes(100))
    assert _load_rc(bad) == (OI_E_FORMAT, "not a GGUF file (bad magic)")
    path = make_model("tiny-q8_0")
    data = open(path, "rb").read()
    (tmp_path / "v9.gguf").write_bytes(data[:4] + struct.pack("<I", 9) + data[8:])
    assert _load_rc(tmp_path / "v9.gguf")[0] == OI_E_FORMAT
    (tmp_path / "trunc.gguf").write_bytes(data[: len(data) // 3])
    assert _load_rc(tmp_path / "trunc.gguf")[0] == OI_E_FORMAT
    (tmp_path / "nokey.gguf").write_bytes(data.replace(b"qwen3.block_count", b"qwen3.block_xxxxx"))
    rc, msg = _load_rc(tmp_path / "nokey.gguf")
    assert rc == OI_E_MODEL and "qwen3.block_count" in msg
    (tmp_path / "notensor.gguf").write_bytes(data.replace(b"blk.1.ffn_up.weight", b"blk.1.ffn_xx.weight"))
    rc, msg = _load_rc(tmp_path / "notensor.gguf")
    assert rc == OI_E_MODEL and "missing required tensor: blk.1.ffn_up.weight" in msg
    # a type the reference's dequant turns into zeros (ggml/quant.odin:170-173)
    # is refused by name here rather than read as zeros (Q2_K = 10)
    q2 = _patch_tensor_type(data, "blk.0.attn_q.weight", 10)
    (tmp_path / "q2_k.gguf").write_bytes(q2)
    rc, msg = _load_rc(tmp_path / "q2_k.gguf")
    assert rc in (OI_E_UNSUPPORTED, OI_E_FORMAT) and "blk.0.attn_q.weight" in msg
    # norm weights must be F32 (infer/model.odin:74-80)
    (tmp_path / "f16norm.gguf").write_bytes(_patch_tensor_type(data, "output_norm.weight", 1))
    rc, msg = _load_rc(tmp_path / "f16norm.gguf")
    assert rc in (OI_E_MODEL, OI_E_FORMAT)
    # a valid file gets past every model check; without a GPU it stops at the device
    rc, msg = _load_rc(path)
    assert rc in (0, OI_E_DEVICE), msg


def test_forward_rejects_null_engine():
    L = _native.hip()
    assert not L.oi_engine_forward(None, 0, 0)
    assert "null engine" in L.oi_last_error().decode()
    assert L.oi_engine_decode_greedy(None, 0, 0, 1, None) == -1


def test_synth_file_matches_measurement_plan(make_model):
    path = make_model("tiny-q4_k")
    r = refcpu.RefEngine(path, max_ctx=128)
    spec = synth.CONFIGS["tiny-q4_k"]
    try:
        assert (r.dim, r.hidden_dim, r.n_layers, r.n_heads, r.n_kv_heads, r.head_dim, r.vocab_size) == (
            spec["dim"], spec["hidden_dim"], spec["n_layers"], spec["n_heads"], spec["n_kv_heads"],
            spec["head_dim"], spec["vocab_size"])
        assert r.seq_len == min(spec["context_length"], 128)
        assert abs(r.rope_freq - 1e6) < 1 and abs(r.rms_eps - 1e-6) < 1e-12
    finally:
        r.close()


def test_synth_weights_and_quantizers():
    w = synth.tensor_f32(9, "blk.0.attn_q.weight", 64, 1024)
    assert abs(w.std() - 0.02) < 0.002 and abs(w.mean()) < 0.002
    assert np.array_equal(w, synth.tensor_f32(9, "blk.0.attn_q.weight", 64, 1024, n_threads=1))  # thread-free
    assert not np.array_equal(w, synth.tensor_f32(9, "blk.0.attn_k.weight", 64, 1024))
    for kind, tol in [(8, 0.01), (12, 0.1), (14, 0.03), (1, 0.001), (2, 0.15), (3, 0.12), (6, 0.06), (7, 0.06)]:
        blocks = synth.quantize_rows(kind, w)
        assert len(blocks) == 64 * ggml.row_byte_size(kind, 1024)
        y = refcpu.dequant_row(kind, blocks, w.size).reshape(w.shape)
        rms = np.sqrt(np.mean((y - w) ** 2)) / np.sqrt(np.mean(w ** 2))
        assert rms < tol, (kind, rms)


def test_kv_prefill_is_standard_normal_f16():
    k, v = synth.kv_prefill(5, 2, 2, 64, 128)
    assert k.shape == (2, 2, 64, 128) and k.dtype == np.uint16
    kf = k.view(np.float16).astype(np.float64)
    assert abs(kf.std() - 1) < 0.02 and abs(kf.mean()) < 0.02
    assert not np.array_equal(k, v)


def test_ggml_tables_match_oracle():
    for t in ggml.GGML_Type:
        e, b = ggml.ggml_block_info(t)
        ce, cb = ctypes.c_int(), ctypes.c_int()
        refcpu.lib().ref_block_info(int(t), ctypes.byref(ce), ctypes.byref(cb))
        assert (e, b) == (ce.value, cb.value)
        assert ggml.row_byte_size(t, 4096) == refcpu.row_byte_size(int(t), 4096)
        assert ggml.is_supported_quant(t) == bool(refcpu.lib().ref_is_supported_quant(int(t)))


def test_engine_api_mirror():
    o = infer.Engine_Opts()
    assert (o.max_ctx, o.use_hip, o.num_threads) == (4096, True, 1)
    assert [f for f in infer.Config.__dataclass_fields__] == [
        "dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "vocab_size", "seq_len", "max_seq",
        "head_dim", "rope_freq", "rms_eps"]  # infer/model.odin:12-24


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr
