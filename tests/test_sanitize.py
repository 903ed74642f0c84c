"""The host code that reads untrusted files, built with AddressSanitizer and
UndefinedBehaviorSanitizer (tests/sanitize/Makefile) and run over malformed
files: the product's GGUF reader and model loader (csrc/gguf.cpp,
csrc/engine.cpp), its .oikv checks (csrc/oikv.cpp), and the oracle's readers
(oracle/refcpu.c).

Malformed inputs: truncations at every header field boundary, header fields
overwritten with boundary values (counts, string lengths, value types,
dimension counts, dimensions that overflow or leave partial blocks, tensor
types, data offsets past the end or wrapping, metadata values that size the
model), and seeded random byte flips in the header region.  The test passes
when no sanitizer reports (the build aborts on the first one), every
structurally broken file is rejected by both readers, and the untouched files
are accepted.  CPU only: the harness loads no device code paths (an accepted
model ends in OI_E_DEVICE where no GPU is present)."""
import os
import shutil
import struct
import subprocess
import sys

import numpy as np
import pytest

from helpers import gguf_fields

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = os.path.join(REPO, "tests", "sanitize")
EXE = os.path.join(SAN, "_build", "san_readers")
sys.path.insert(0, os.path.join(REPO, "odin-infer_amd"))

OI_E_FORMAT, OI_E_MODEL, OI_E_UNSUPPORTED, OI_E_DEVICE = -3, -4, -5, -7
U64 = 2 ** 64 - 1

pytestmark = pytest.mark.skipif(shutil.which("g++") is None or shutil.which("make") is None,
                                reason="needs g++ and make")


@pytest.fixture(scope="module")
def harness():
    objs = os.path.join(REPO, "odin-infer_amd", "_build")
    if not os.path.isdir(objs) or not any(f.endswith(".hip.o") for f in os.listdir(objs)):
        sys.path.insert(0, os.path.join(REPO, "odin-infer_amd"))
        import build
        build.build()
    r = subprocess.run(["make", "-C", SAN, "-j8"], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    return EXE


def _env():
    env = dict(os.environ)
    env["ASAN_OPTIONS"] = "detect_leaks=1:abort_on_error=0:exitcode=86"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1:exitcode=87"
    env["HIP_VISIBLE_DEVICES"] = ""  # the loader must stop at its device check here
    return env


def _run(exe, args):
    try:
        r = subprocess.run([exe, *args], capture_output=True, text=True, env=_env(), timeout=300)
    except subprocess.TimeoutExpired as ex:
        done = (ex.stdout or b"").decode(errors="replace").count("\n")
        raise AssertionError("the harness did not finish within 300 s; it stopped after %d of its files, "
                             "at %s" % (done, args[1 + done] if 1 + done < len(args) else "?")) from None
    report = "AddressSanitizer" in r.stderr or "runtime error" in r.stderr or "LeakSanitizer" in r.stderr
    assert r.returncode == 0 and not report, "sanitizer or harness failure (rc %d):\n%s" % (
        r.returncode, r.stderr[-6000:])
    rows = {}
    for line in r.stdout.splitlines():
        parts = line.split(" ", 3 if args[0] == "gguf" else 2)
        rows[parts[-1]] = tuple(int(x) for x in parts[:-1])
    return rows


def _put(data, off, size, v):
    b = bytearray(data)
    b[off:off + size] = int(v & (2 ** (8 * size) - 1)).to_bytes(size, "little")
    return bytes(b)


def gguf_mutations(data):
    """(label, bytes, must_reject) for one valid GGUF."""
    fields = gguf_fields(data)
    end = fields[-1][1]
    muts = [("identity", data, False)]
    cuts = sorted({0, 3, 23, 24, end - 1, end, end + (len(data) - end) // 2, len(data) - 1} |
                  {o for _, o, _ in fields if 0 < o < end} | {o + 1 for _, o, _ in fields[:40]})
    for c in cuts:
        if c < len(data):
            muts.append(("truncate@%d" % c, data[:c], True))
    tensors = sorted({n.split(":")[1].rsplit(".", 1)[0] for n, _, _ in fields if n.startswith("tensor:")})
    pick = set(tensors[:2] + tensors[len(tensors) // 2:len(tensors) // 2 + 1] + tensors[-2:])
    for name, off, size in fields:
        if name in ("end",):
            continue
        vals = []
        if name == "magic":
            vals = [(0x46554748, True)]
        elif name == "version":
            vals = [(1, True), (4, True), (2 ** 32 - 1, True)]
        elif name in ("n_tensors", "n_meta"):
            vals = [((1 << 24) + 1, True), (U64, True), (2 ** 63, True)]
        elif name.endswith(".keylen") or name.endswith(".strlen") or name.endswith(".namelen"):
            vals = [(U64, True), (2 ** 63, True), (len(data), True)]
        elif name.endswith(".type") and name.startswith("meta:"):
            vals = [(13, True), (2 ** 32 - 1, True)]
        elif name.endswith(".atype"):
            vals = [(13, True), (9, True)]
        elif name.endswith(".count"):
            vals = [(U64, True), (2 ** 61, True)]
        elif name.startswith("meta:") and name.endswith(".value") and size >= 4:
            vals = [(0, None), (1, None), (2 ** 31, None), (2 ** (8 * size) - 1, None)]
        elif name.startswith("tensor:"):
            t = name.split(":")[1].rsplit(".", 1)[0]
            if t not in pick:
                continue
            f = name.rsplit(".", 1)[1]
            if f == "n_dims":
                vals = [(0, True), (5, True), (2 ** 32 - 1, True)]
            elif f.startswith("dim"):
                vals = [(0, None), (2 ** 63, True), (2 ** 32 + 1, True), (U64, True), (7, True)]
            elif f == "type":
                vals = [(99, True), (16, True), (0, None), (15, None)]
            elif f == "offset":
                vals = [(U64, True), (2 ** 63, True), (len(data), True), (U64 - 31, True)]
        for v, rej in vals:
            muts.append(("%s=%d" % (name, v), _put(data, off, size, v), rej))
    rng = np.random.default_rng(1234)
    for i in range(120):
        b = bytearray(data)
        for _ in range(int(rng.integers(1, 5))):
            b[int(rng.integers(0, end))] ^= 1 << int(rng.integers(0, 8))
        muts.append(("flip%d" % i, bytes(b), None))
    return muts


MODELS = {
    "dense": dict(kind="spec", args=(256, 512, 1, 2, 1, 128, 256, 64), types=("Q4_K", "Q6_K", "Q8_0", "Q4_K", "Q6_K")),
    "moe": dict(kind="config", name="moe-tiny", over=dict(vocab_size=256, n_layers=1)),
    "hybrid": dict(kind="config", name="qwen35-moe-tiny", over=dict(vocab_size=256)),
}


def _write_model(path, m):
    from oi import synth
    from oi.ggml import GGML_Type as T
    if m["kind"] == "spec":
        spec = synth._spec(*m["args"], *(getattr(T, t) for t in m["types"]), seed=5)
        synth.write_gguf(path, spec)
    else:
        synth.write_gguf(path, m["name"], **m["over"])


@pytest.mark.parametrize("model", sorted(MODELS))
def test_gguf_readers_under_sanitizers(harness, tmp_path, model):
    good = str(tmp_path / ("%s.gguf" % model))
    _write_model(good, MODELS[model])
    data = open(good, "rb").read()
    muts = gguf_mutations(data)
    paths, expect = [], {}
    for i, (label, b, rej) in enumerate(muts):
        p = str(tmp_path / ("m%04d.gguf" % i))
        with open(p, "wb") as fh:
            fh.write(b)
        paths.append(p)
        expect[p] = (label, rej)
    rows = {}
    for i in range(0, len(paths), 200):
        rows.update(_run(harness, ["gguf", *paths[i:i + 200]]))
    assert len(rows) == len(paths)
    bad = []
    for p, (prc, orc, grc) in rows.items():
        label, rej = expect[p]
        if rej is False and (prc != OI_E_DEVICE or orc != 0):
            bad.append("%s: valid file not accepted (product %d, oracle %d)" % (label, prc, orc))
        if rej is True and (prc in (0, OI_E_DEVICE) or orc == 0):
            bad.append("%s: broken file accepted (product %d, oracle %d)" % (label, prc, orc))
    assert not bad, "\n".join(bad)
    n_rej = sum(1 for p in rows if rows[p][0] not in (0, OI_E_DEVICE))
    print("%s: %d files, %d rejected by the product loader" % (model, len(rows), n_rej))


def test_oikv_readers_under_sanitizers(harness, tmp_path):
    from oracle import refcpu
    model = str(tmp_path / "hybrid.gguf")
    _write_model(model, MODELS["hybrid"])
    ref = refcpu.RefEngine(model, max_ctx=32, kv_f16=False)
    for pos, tok in enumerate([1, 7, 3]):
        ref.forward(tok, pos)
    good = str(tmp_path / "good.oikv")
    ref.save_kv(good, 3)
    ref.close()
    data = open(good, "rb").read()
    muts = [("identity", data, False)]
    for c in [0, 4, 59, 60, 61, len(data) // 2, len(data) - 4, len(data) - 1]:
        muts.append(("truncate@%d" % c, data[:c], True))
    muts.append(("extended", data + b"\0", True))
    for i in range(15):  # the 15 header words
        w = struct.unpack_from("<I", data, 4 * i)[0]
        for v in {0, 1, w + 1, 2 ** 31, 2 ** 32 - 1} - {w}:
            muts.append(("word%d=%d" % (i, v), _put(data, 4 * i, 4, v), True))
    muts.append(("crc", _put(data, len(data) - 4, 4, struct.unpack_from("<I", data, len(data) - 4)[0] ^ 1), True))
    muts.append(("body", _put(data, 100, 1, data[100] ^ 0x10), True))
    paths, expect = [], {}
    for i, (label, b, rej) in enumerate(muts):
        p = str(tmp_path / ("k%03d.oikv" % i))
        with open(p, "wb") as fh:
            fh.write(b)
        paths.append(p)
        expect[p] = (label, rej)
    rows = _run(harness, ["oikv", model, good, *paths])
    assert len(rows) == len(paths)
    bad = []
    for p, (prc, orc) in rows.items():
        label, rej = expect[p]
        if rej and (prc == 0 or orc >= 0):
            bad.append("%s: accepted (product %d, oracle %d)" % (label, prc, orc))
        if not rej and (prc != 0 or orc != 3):
            bad.append("%s: rejected (product %d, oracle %d)" % (label, prc, orc))
    assert not bad, "\n".join(bad)
