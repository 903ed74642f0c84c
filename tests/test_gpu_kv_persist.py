"""GPU state persistence against the CPU oracle (oracle/refcpu.c, the restated
qwen3_5/kv_persist.odin and engine.odin snapshot procedures):

  * a file the GPU engine writes has the oracle's header byte for byte and a
    body within f16 rounding of the oracle's (the GPU's K/V differ from the
    oracle's by the decode path's tolerance, so the body is compared, not
    bit-matched);
  * a file the oracle writes, loaded by the GPU engine, continues with logits
    within 1e-3 of the oracle's own continuation (a misplaced position, head
    or layer would be far off);
  * save -> reset -> load and full / speculative snapshots (host and device
    memory) reproduce the next logits bit for bit;
  * a refused file (CRC, fingerprint) leaves the state as it was.
Dense, routed-expert and hybrid layouts.
"""
import os
import struct

import numpy as np
import pytest

import refcpu
from helpers import DeviceBuffer, scaled_err
from oi import infer

pytestmark = pytest.mark.gpu
TOL = 1e-3
NT = min(16, os.cpu_count() or 1)
MODELS = ["tiny-q8_0", "moe-tiny", "qwen35-tiny"]
TOKENS = [3, 17, 5, 99, 42, 7, 1, 250, 31]


def _engines(path, max_ctx=64):
    e, ok = infer.engine_load(path, infer.Engine_Opts(max_ctx=max_ctx))
    assert ok
    return e, refcpu.RefEngine(path, max_ctx=max_ctx, num_threads=NT, kv_f16=True)


def _feed_gpu(e, tokens, pos0=0):
    for i, t in enumerate(tokens):
        infer.engine_forward(e, t, pos0 + i)


def _feed_ref(r, tokens, pos0=0):
    for i, t in enumerate(tokens):
        r.forward(t, pos0 + i)


@pytest.mark.parametrize("name", MODELS)
def test_gpu_file_matches_oracle_file(make_model, tmp_path, name):
    path = make_model(name)
    e, r = _engines(path)
    try:
        _feed_gpu(e, TOKENS)
        _feed_ref(r, TOKENS)
        fg, fr = tmp_path / "gpu.oikv", tmp_path / "ref.oikv"
        assert infer.engine_save_kv(e, fg, len(TOKENS))
        r.save_kv(fr, len(TOKENS))
        g, o = fg.read_bytes(), fr.read_bytes()
        assert len(g) == len(o)
        assert g[:60] == o[:60]
        bg, bo = np.frombuffer(g[60:-4], np.float32), np.frombuffer(o[60:-4], np.float32)
        n, _, n_full, n_lin, kv_dim, conv_dim, kern, nv, hk, hv = struct.unpack_from("<10I", o, 20)
        sizes = [("K/V", 2 * n_full * n * kv_dim), ("conv", n_lin * conv_dim * max(kern - 1, 0)),
                 ("recurrent", n_lin * nv * hk * hv)]
        off = 0
        for what, size in sizes:
            if size:
                err = scaled_err(bg[off:off + size], bo[off:off + size])
                print("%s: %s section, scaled difference GPU vs oracle %.3g" % (name, what, err))
                assert err <= TOL, what
            off += size
        assert off == bo.size
        # the oracle reads the GPU's file and continues where the GPU does
        r2 = refcpu.RefEngine(path, max_ctx=64, num_threads=NT, kv_f16=True)
        try:
            assert r2.load_kv(fg) == len(TOKENS)
            assert scaled_err(infer.engine_forward(e, 11, len(TOKENS)), r2.forward(11, len(TOKENS))) <= TOL
        finally:
            r2.close()
    finally:
        infer.engine_destroy(e)
        r.close()


@pytest.mark.parametrize("name", MODELS)
def test_oracle_file_loads_on_gpu(make_model, tmp_path, name):
    path = make_model(name)
    e, r = _engines(path)
    try:
        _feed_ref(r, TOKENS)
        f = tmp_path / "ref.oikv"
        r.save_kv(f, len(TOKENS))
        n, ok = infer.engine_load_kv(e, f)
        assert ok and n == len(TOKENS)
        tok, worst = 11, 0.0
        for i in range(6):
            got = infer.engine_forward(e, tok, n + i).copy()
            ref = r.forward(tok, n + i)
            worst = max(worst, scaled_err(got, ref))
            tok = int(refcpu.argmax(ref))
        print("%s: continuation after loading the oracle's file, worst scaled error %.3g" % (name, worst))
        assert worst <= TOL
    finally:
        infer.engine_destroy(e)
        r.close()


@pytest.mark.parametrize("name", MODELS)
def test_save_reset_load_bit_exact(make_model, tmp_path, name):
    """The reference's acceptance check (docs/KV_CACHE.md:104-113)."""
    path = make_model(name)
    e, ok = infer.engine_load(path, infer.Engine_Opts(max_ctx=64))
    try:
        _feed_gpu(e, TOKENS)
        f = tmp_path / "s.oikv"
        assert infer.engine_save_kv(e, f, len(TOKENS))
        want = infer.engine_forward(e, 11, len(TOKENS)).copy()
        infer.engine_reset_state(e)
        assert not np.array_equal(infer.engine_forward(e, 11, len(TOKENS)), want)
        infer.engine_reset_state(e)
        n, ok = infer.engine_load_kv(e, f)
        assert ok and n == len(TOKENS)
        assert np.array_equal(infer.engine_forward(e, 11, len(TOKENS)), want)
        # a second save of the restored state is the same file
        f2 = tmp_path / "s2.oikv"
        infer.engine_reset_state(e)
        infer.engine_load_kv(e, f)
        assert infer.engine_save_kv(e, f2, len(TOKENS))
        assert f2.read_bytes() == f.read_bytes()
    finally:
        infer.engine_destroy(e)


@pytest.mark.parametrize("name", MODELS)
def test_snapshots_host_and_device(make_model, name):
    path = make_model(name)
    e, ok = infer.engine_load(path, infer.Engine_Opts(max_ctx=64))
    dev = []
    try:
        _feed_gpu(e, TOKENS[:5])
        snap = infer.engine_save_full_state(e)
        assert [s.size for s in snap] == list(infer.engine_state_sizes(e))
        want = infer.engine_forward(e, 8, 5).copy()
        _feed_gpu(e, [9, 10, 12], 6)
        infer.engine_restore_full_state(e, *snap)
        assert np.array_equal(infer.engine_forward(e, 8, 5), want)
        # the same through device buffers (a prefix snapshot kept in HBM)
        dev = [DeviceBuffer(n) for n in infer.engine_state_sizes(e)]
        infer.engine_restore_full_state(e, *snap)
        L = infer._native.hip()
        assert L.oi_engine_save_full_state(e.handle, *[d.ptr for d in dev]) == 0
        _feed_gpu(e, [9, 10, 12], 5)
        assert L.oi_engine_restore_full_state(e.handle, *[d.ptr for d in dev]) == 0
        assert np.array_equal(infer.engine_forward(e, 8, 5), want)
        for d, s in zip(dev, snap):
            assert np.array_equal(d.to_host(s.size), s)
    finally:
        for d in dev:
            d.free()
        infer.engine_destroy(e)


def test_spec_state_rollback_hybrid(make_model):
    """Speculative rollback (qwen3_5/engine.odin:153-165): the DeltaNet states
    restored, the draft positions of the cache overwritten by the re-run."""
    e, ok = infer.engine_load(make_model("qwen35-tiny"), infer.Engine_Opts(max_ctx=64))
    try:
        _feed_gpu(e, TOKENS[:4])
        conv, rec = infer.engine_save_spec_state(e)
        assert conv.size > 0 and rec.size > 0
        want = [infer.engine_forward(e, t, 4 + i).copy() for i, t in enumerate([5, 6, 7])]
        infer.engine_restore_spec_state(e, conv, rec)
        got = [infer.engine_forward(e, t, 4 + i).copy() for i, t in enumerate([5, 6, 7])]
        for a, b in zip(want, got):
            assert np.array_equal(a, b)
    finally:
        infer.engine_destroy(e)


def test_refused_files_leave_the_gpu_state(make_model, tmp_path):
    path = make_model("qwen35-tiny")
    e, ok = infer.engine_load(path, infer.Engine_Opts(max_ctx=64))
    other, _ = infer.engine_load(make_model("qwen35-moe-tiny"), infer.Engine_Opts(max_ctx=64))
    try:
        _feed_gpu(e, TOKENS[:3])
        good = tmp_path / "g.oikv"
        assert infer.engine_save_kv(e, good, 3)
        data = bytearray(good.read_bytes())
        data[80] ^= 1
        bad = tmp_path / "b.oikv"
        bad.write_bytes(bytes(data))
        assert infer.engine_load_kv(e, bad) == (0, False)
        assert "CRC mismatch" in infer._native.hip().oi_last_error().decode()
        assert infer.engine_load_kv(other, good) == (0, False)
        assert "fingerprint mismatch" in infer._native.hip().oi_last_error().decode()
        after = tmp_path / "a.oikv"
        assert infer.engine_save_kv(e, after, 3)
        assert after.read_bytes() == good.read_bytes()
        assert not infer.engine_save_kv(e, after, 65)  # past seq_len
        assert struct.unpack_from("<I", good.read_bytes(), 8)[0] == 2
    finally:
        infer.engine_destroy(e)
        infer.engine_destroy(other)
