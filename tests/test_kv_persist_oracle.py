"""The .oikv v1 state file (qwen3_5/kv_persist.odin:1-381) on the CPU oracle,
pinned independently of both writers:

  * the header is read back field by field with struct (60 bytes, the order of
    write_header, kv_persist.odin:141-156), the fingerprint recomputed as
    FNV-1a 64 from the GGUF's own metadata (kv_persist.odin:74-93), the
    checksum with zlib.crc32 (IEEE CRC-32, what core:hash crc32 computes);
  * the body layout (per attention layer K then V as f32 [pos][kv_heads *
    head_dim], then every conv state, then every recurrent state) is checked
    against values planted through kv_fill in head-major order, so a missed
    head-major -> position-major transposition fails;
  * save -> reset -> load reproduces the next logits bit for bit (the
    reference's own acceptance check, docs/KV_CACHE.md:104-113), for the dense
    and the hybrid layout;
  * every refusal the reference makes (bad magic, version, arch, fingerprint,
    seq_len, CRC) leaves the state untouched.  CPU only.
"""
import struct
import zlib

import numpy as np
import pytest

import npref
import refcpu
from oi import synth

HEADER = struct.Struct("<IIIQ10I")
assert HEADER.size == 60


def _fnv(vals):
    h = 0xcbf29ce484222325
    for v in vals:
        h = ((h ^ (v & (2 ** 64 - 1))) * 0x100000001b3) % 2 ** 64
    return h


def _expected_fingerprint(path, arch):
    """From the file's metadata, not from either engine's config."""
    W = npref.GGUFWeights(path)
    m = W.meta
    a = m["general.architecture"]
    heads, kv = m[a + ".attention.head_count"], m[a + ".attention.head_count_kv"]
    dim = m[a + ".embedding_length"]
    hd = m.get(a + ".attention.key_length", dim // heads)
    vocab = W.tensors["token_embd.weight"][0][1]
    if arch == 2:
        nk, nv = m[a + ".ssm.group_count"], m[a + ".ssm.time_step_rank"]
        hk = m[a + ".ssm.state_size"]
        hv = m[a + ".ssm.inner_size"] // nv
        kern = m[a + ".ssm.conv_kernel"]
    else:
        nk = nv = hk = hv = kern = 0
    return _fnv([dim, m[a + ".block_count"], heads, kv, hd, nk, nv, hk, hv, kern, vocab])


def _run(r, tokens):
    for p, t in enumerate(tokens):
        r.forward(t, p)


@pytest.mark.parametrize("name,arch", [("tiny-q8_0", 1), ("qwen35-tiny", 2), ("moe-tiny", 3)])
def test_save_reset_load_is_bit_exact(make_model, tmp_path, name, arch):
    path = make_model(name)
    r = refcpu.RefEngine(path, max_ctx=64, num_threads=4, kv_f16=True)
    try:
        toks = [3, 17, 5, 99, 42, 7, 1]
        _run(r, toks)
        f = tmp_path / "s.oikv"
        r.save_kv(f, len(toks))
        want = r.forward(11, len(toks)).copy()
        r.reset_state()
        assert not np.array_equal(r.forward(11, len(toks)), want)  # the state matters
        r.reset_state()
        assert r.load_kv(f) == len(toks)
        assert np.array_equal(r.forward(11, len(toks)), want)
        data = f.read_bytes()
        h = HEADER.unpack_from(data)
        assert h[:3] == (0x4F494B56, 1, arch)
        assert h[3] == _expected_fingerprint(path, arch)
        assert h[4:6] == (len(toks), r.seq_len)
        assert struct.unpack_from("<I", data, len(data) - 4)[0] == zlib.crc32(data[:-4])
        n_full, n_lin, kv_dim, conv_dim, kern, nv, hk, hv = h[6:]
        body = 2 * n_full * len(toks) * kv_dim * 4 + n_lin * (conv_dim * max(kern - 1, 0) + nv * hk * hv) * 4
        assert len(data) == 60 + body + 4
        assert kv_dim == r.n_kv_heads * r.head_dim
        if arch == 2:
            assert n_lin == 3 and n_full == 1  # 3 DeltaNet : 1 full attention
        else:
            assert (n_full, n_lin) == (r.n_layers, 0)
    finally:
        r.close()


def test_body_layout_from_planted_cache(make_model, tmp_path):
    """kv_fill plants K/V in head-major order; the file must hold them as
    [pos][kv_head * head_dim] f32 rows, layer by layer, K before V."""
    path = make_model("tiny-q8_0")
    r = refcpu.RefEngine(path, max_ctx=64, num_threads=2, kv_f16=True)
    try:
        n, H, hd = 9, r.n_kv_heads, r.head_dim
        rng = np.random.default_rng(5)
        planted = []
        for l in range(r.n_layers):
            k = rng.standard_normal((H, n, hd)).astype(np.float16)
            v = rng.standard_normal((H, n, hd)).astype(np.float16)
            r.kv_fill(l, 0, k.view(np.uint16), v.view(np.uint16))
            planted.append((k, v))
        f = tmp_path / "p.oikv"
        r.save_kv(f, n)
        body = np.frombuffer(f.read_bytes()[60:-4], np.float32)
        off = 0
        for k, v in planted:
            for t in (k, v):
                rows = body[off:off + n * H * hd].reshape(n, H * hd)
                assert np.array_equal(rows, t.astype(np.float32).transpose(1, 0, 2).reshape(n, H * hd))
                off += n * H * hd
        assert off == body.size
    finally:
        r.close()


def test_refusals_leave_the_state_alone(make_model, tmp_path):
    path = make_model("qwen35-tiny")
    r = refcpu.RefEngine(path, max_ctx=64, num_threads=2, kv_f16=True)
    r2 = refcpu.RefEngine(make_model("qwen35-moe-tiny"), max_ctx=64, num_threads=2, kv_f16=True)
    r3 = refcpu.RefEngine(path, max_ctx=32, num_threads=2, kv_f16=True)
    r4 = refcpu.RefEngine(make_model("tiny-q8_0"), max_ctx=64, num_threads=2, kv_f16=True)
    try:
        _run(r, [1, 2, 3])
        good = tmp_path / "g.oikv"
        r.save_kv(good, 3)
        data = bytearray(good.read_bytes())

        def variant(name, mutate):
            d = bytearray(data)
            mutate(d)
            p = tmp_path / name
            p.write_bytes(bytes(d))
            return p

        def fix_crc(d):
            struct.pack_into("<I", d, len(d) - 4, zlib.crc32(bytes(d[:-4])))

        cases = {
            "bad magic": variant("m", lambda d: (struct.pack_into("<I", d, 0, 0x12345678), fix_crc(d))),
            "version mismatch": variant("v", lambda d: (struct.pack_into("<I", d, 4, 2), fix_crc(d))),
            "arch mismatch": variant("a", lambda d: (struct.pack_into("<I", d, 8, 1), fix_crc(d))),
            "fingerprint mismatch": variant("f", lambda d: (struct.pack_into("<Q", d, 12, 1), fix_crc(d))),
            "CRC mismatch": variant("c", lambda d: d.__setitem__(100, d[100] ^ 1)),
            "header truncated": variant("t", lambda d: d.__delitem__(slice(40, None))),
        }
        after = tmp_path / "after.oikv"
        for msg, p in cases.items():
            with pytest.raises(RuntimeError, match=msg):
                r.load_kv(p)
            r.save_kv(after, 3)  # the state, unchanged: the same file again
            assert after.read_bytes() == bytes(data), msg
        with pytest.raises(RuntimeError, match="fingerprint mismatch"):
            r2.load_kv(good)  # another hybrid model
        with pytest.raises(RuntimeError, match="arch mismatch"):
            r4.load_kv(good)  # a dense model
        with pytest.raises(RuntimeError, match="seq_len mismatch"):
            r3.load_kv(good)  # same model, another -c
        with pytest.raises(RuntimeError, match="n_valid_pos"):
            r.save_kv(tmp_path / "x.oikv", r.seq_len + 1)
    finally:
        for e in (r, r2, r3, r4):
            e.close()


def test_f32_cache_file_loads_into_the_f16_mode_rounded(make_model, tmp_path):
    """A file from the reference CPU path (f32 cache) read by an f16-cache
    engine is rounded to f16 on load, as metal_load_kv does."""
    path = make_model("tiny-q8_0")
    a = refcpu.RefEngine(path, max_ctx=64, num_threads=2, kv_f16=False)
    b = refcpu.RefEngine(path, max_ctx=64, num_threads=2, kv_f16=True)
    try:
        _run(a, [4, 8, 15, 16])
        fa, fb = tmp_path / "a.oikv", tmp_path / "b.oikv"
        a.save_kv(fa, 4)
        assert b.load_kv(fa) == 4
        b.save_kv(fb, 4)
        ka = np.frombuffer(fa.read_bytes()[60:-4], np.float32)
        kb = np.frombuffer(fb.read_bytes()[60:-4], np.float32)
        assert not np.array_equal(ka, kb)  # the f32 cache carries bits f16 cannot
        assert np.array_equal(ka.astype(np.float16).astype(np.float32), kb)
    finally:
        a.close()
        b.close()


def test_synth_hybrid_metadata_keys_used_above(make_model):
    """The fingerprint test reads the hybrid's DeltaNet dims from these keys."""
    W = npref.GGUFWeights(make_model("qwen35-tiny"))
    spec = synth.CONFIGS["qwen35-tiny"]
    m = W.meta
    assert m["qwen35.ssm.group_count"] == spec["lin_n_k_heads"]
    assert m["qwen35.ssm.time_step_rank"] == spec["lin_n_v_heads"]
    assert m["qwen35.ssm.state_size"] == spec["lin_head_k_dim"]
    assert m["qwen35.ssm.inner_size"] == spec["lin_n_v_heads"] * spec["lin_head_v_dim"]
    assert m["qwen35.ssm.conv_kernel"] == spec["lin_conv_kernel"]
