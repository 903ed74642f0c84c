#!/usr/bin/env python3
"""Decode throughput of the token loop on one MI355X.

Workload (the measured configuration): Qwen3-8B-shaped dense decoder,
Q4_K_M-style weights (Q4_K, Q6_K for attn_v and output), f16 KV cache
pre-filled with N(0,1) to context 4096, then greedy decode at batch 1 from
position 4096.  A step is one token of the device-side greedy loop
(oi_engine_decode_greedy): embedding, 36 layers, logits, argmax.

Prints one JSON line.  `roofline` is for the dominant kernel (gate/up GEMV),
timed with HIP events on the engine's stream; `token_loop` gives the whole
step's algorithmic HBM bytes and rate.  `cpu_baseline` times the CPU oracle
(oracle/refcpu.c, the restated reference CPU forward) on a bounded sample of
the same workload and checks its greedy ids against the GPU's.

usage: python bench.py [--gpus 1] [--steps 512] [--warmup 16]
"""
import argparse
import json
import os
import shutil
import sys
import tempfile
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "odin-infer_amd"))

PEAK_HBM_GBPS = 8000.0
METRIC = "decode tok/s @bs1 Qwen3-8B-shape Q4_K; achieved HBM GB/s as % of peak"
CONTEXT = 4096
MODEL = "qwen3-8b-q4_k_m"


def log(msg):
    print("[bench] " + msg, file=sys.stderr, flush=True)


def algorithmic_bytes_per_token(cfg, wbytes, pos):
    """Weights read once per token + KV read over pos+1 positions + KV write
    + logits write (f16 KV, f32 logits)."""
    kvd = cfg.n_kv_heads * cfg.head_dim
    return wbytes + cfg.n_layers * 2 * kvd * 2 * (pos + 1) + cfg.n_layers * 2 * kvd * 2 + cfg.vocab_size * 4


def weight_bytes(spec):
    from oi.ggml import row_byte_size
    D, H, L, V = spec["dim"], spec["hidden_dim"], spec["n_layers"], spec["vocab_size"]
    QD, KVD = spec["n_heads"] * spec["head_dim"], spec["n_kv_heads"] * spec["head_dim"]
    td, tv, tdown = spec["type_default"], spec["type_attn_v"], spec["type_ffn_down"]
    per_layer = (row_byte_size(td, D) * (QD + KVD + 2 * H) + row_byte_size(tv, D) * KVD +
                 row_byte_size(td, QD) * D + row_byte_size(tdown, H) * D + 4 * (2 * D + 2 * spec["head_dim"]))
    out = row_byte_size(spec["type_output"], D) * V if spec["type_output"] >= 0 else 0
    # per token the embedding contributes one row
    return L * per_layer + out + 4 * D + row_byte_size(spec["type_embd"], D)


def cpu_threads():
    """Threads for the CPU baseline: the host's cores (nproc), capped at the
    worker-pool share the GPU box grants one GPU (OMP_NUM_THREADS there)."""
    nproc = os.cpu_count() or 1
    cap = int(os.environ.get("OMP_NUM_THREADS", nproc) or nproc)
    return max(1, min(nproc, cap)), nproc


def cpu_baseline(path, k, v, cfg, gpu_tokens, budget_s, max_steps=64):
    """The oracle (restated reference CPU forward) on the host's cores: greedy
    steps from pos 4096 of the same model and pre-filled f16 KV, up to
    max_steps or budget_s; its ids are compared with the GPU's.  Then a
    1-thread figure on one step."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import refcpu  # the oracle, timed here as the CPU baseline
    threads, nproc = cpu_threads()
    r = refcpu.RefEngine(path, max_ctx=cfg.seq_len, num_threads=threads, kv_f16=True)
    try:
        for layer in range(cfg.n_layers):
            r.kv_fill(layer, 0, k[layer], v[layer])
        tok, ids, t0 = 0, [], time.perf_counter()
        while True:
            logits = r.forward(tok, CONTEXT + len(ids))
            tok = refcpu.argmax(logits)
            ids.append(tok)
            el = time.perf_counter() - t0
            if el > budget_s or len(ids) >= min(max_steps, len(gpu_tokens)):
                break
        n = len(ids)
    finally:
        r.close()
    # 1 thread, one step (the same forward at the next position)
    r1 = refcpu.RefEngine(path, max_ctx=cfg.seq_len, num_threads=1, kv_f16=True)
    try:
        for layer in range(cfg.n_layers):
            r1.kv_fill(layer, 0, k[layer], v[layer])
        t1 = time.perf_counter()
        r1.forward(0, CONTEXT)
        el1 = time.perf_counter() - t1
    finally:
        r1.close()
    match = 0
    while match < n and gpu_tokens[match] == ids[match]:
        match += 1
    return {
        "value": n / el, "unit": "tok/s", "cores": threads, "kind": "port", "nproc": nproc,
        "sample": "%d greedy decode steps from pos %d of the same model and pre-filled f16 KV, "
                  "oracle/refcpu.c (restated reference CPU forward, row work queue over %d threads; the host "
                  "reports nproc=%d, the box grants one GPU a %d-thread share)" % (n, CONTEXT, threads, nproc, threads),
        "ms_per_token": 1000 * el / n,
        "one_thread": {"value": 1.0 / el1, "unit": "tok/s", "ms_per_token": 1000 * el1, "sample": "1 step"},
        "greedy_ids_match_gpu": bool(match == n), "compared_steps": n, "matching_prefix": match,
    }


def c1_cpu_run(budget_s=60.0):
    """Qwen3-0.6B shape, Q8_0, f32 KV cache, max_ctx 4096,
    token 0 then 256 greedy steps on the CPU reference path (the oracle, host
    cores), and the same workload on the GPU (f16 KV) beside it."""
    import numpy as np
    from oi import infer, synth
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import refcpu
    threads, nproc = cpu_threads()
    d = tempfile.mkdtemp(prefix="oi_c1_")
    try:
        path = os.path.join(d, "c1.gguf")
        synth.write_gguf(path, "qwen3-0.6b-q8_0")
        spec = synth.CONFIGS["qwen3-0.6b-q8_0"]
        r = refcpu.RefEngine(path, max_ctx=4096, num_threads=threads, kv_f16=False)
        try:
            tok, ids, t0 = 0, [], time.perf_counter()
            for pos in range(256):
                tok = refcpu.argmax(r.forward(tok, pos))
                ids.append(tok)
                if time.perf_counter() - t0 > budget_s:
                    break
            el = time.perf_counter() - t0
        finally:
            r.close()
        n = len(ids)
        e, _ = infer.engine_load(path, infer.Engine_Opts(max_ctx=4096))
        try:
            infer.engine_decode_greedy(e, 0, 0, 16)  # warm
            g0 = time.perf_counter()
            gids = infer.engine_decode_greedy(e, 0, 0, 256)
            gel = time.perf_counter() - g0
        finally:
            infer.engine_destroy(e)
        match = 0
        while match < n and gids[match] == ids[match]:
            match += 1
        # the GPU's greedy path teacher-forced through the oracle with the
        # GPU's cache precision (f16 KV): its pick against the oracle's argmax
        # at each step, and where they differ the oracle's margin between the
        # two (a near-tie that the cache precision alone can decide: at step
        # 1 of this model the f32- and f16-KV oracles pick different ids)
        K = min(64, len(gids))
        r16 = refcpu.RefEngine(path, max_ctx=4096, num_threads=threads, kv_f16=True)
        try:
            agree, worst, prev = 0, 0.0, 0
            for i in range(K):
                lg = np.asarray(r16.forward(prev, i), np.float64)
                pick = refcpu.argmax(lg)
                if pick == int(gids[i]):
                    agree += 1
                else:
                    worst = max(worst, float(lg[pick] - lg[int(gids[i])]) / float(np.abs(lg).max()))
                prev = int(gids[i])
        finally:
            r16.close()
        wb = weight_bytes(spec)
        return {"workload": "Qwen3-0.6B shape Q8_0, token 0 + %d greedy steps, f32 KV (CPU) / f16 KV (GPU), "
                            "max_ctx 4096" % n,
                "cpu": {"value": round(n / el, 2), "unit": "tok/s", "cores": threads, "nproc": nproc, "kind": "port",
                        "ms_per_token": round(1000 * el / n, 2),
                        "GBps": round(wb * n / el / 1e9, 2)},
                "gpu": {"value": round(256 / gel, 1), "unit": "tok/s", "ms_per_token": round(1000 * gel / 256, 4),
                        "GBps": round(wb * 256 / gel / 1e9, 1)},
                "greedy_matching_prefix": match, "compared_steps": n,
                "gpu_path_vs_f16kv_oracle": {"steps": K, "argmax_equal": agree,
                                             "max_rel_margin_where_different": worst}}
    finally:
        shutil.rmtree(d, ignore_errors=True)


def gemv_microbench(iters=100, cpu=True):
    """the quantized GEMV alone at batch 1 for Q4_K, Q6_K
    and Q8_0 at 12288x4096, 4096x12288, 4096x4096 and 151936x4096, weights
    N(0,0.02) quantized, x ~ N(0,1) f32.  Copies of the weights totalling
    >= 1 GiB are cycled (the 256 MB Infinity Cache cannot serve repeats);
    max(iters, copies) launches of oi_gemv_launch in one HIP graph, HIP events
    around the graph launch; the median of 3 graph launches of the mean time
    per GEMV.  Bytes: weights + 4 in + 4 out."""
    import ctypes
    import numpy as np
    from oi import ggml, synth
    hip = ctypes.CDLL("libamdhip64.so")
    vp = ctypes.c_void_p

    def ok(rc, what):
        if rc != 0:
            raise RuntimeError("%s failed (%d)" % (what, rc))

    threads, _ = cpu_threads()
    out = []
    names = {12: "Q4_K", 14: "Q6_K", 8: "Q8_0"}
    for rows, cols in ((12288, 4096), (4096, 12288), (4096, 4096), (151936, 4096)):
        w32 = synth.tensor_f32(9, "microbench.%dx%d" % (rows, cols), rows, cols, sigma=0.02)
        x = np.random.default_rng(rows + cols).standard_normal(cols).astype(np.float32)
        for kind in (12, 14, 8):
            blocks = synth.quantize_rows(kind, w32)
            w0 = ggml.DeviceWeights(kind, blocks, rows, cols)
            ncopy = max(1, -(-ROTATE_BYTES // w0.nbytes))
            ws = [w0] + [ggml.DeviceWeights(kind, blocks, rows, cols) for _ in range(ncopy - 1)]
            xd, yd, st = vp(), vp(), vp()
            ok(hip.hipMalloc(ctypes.byref(xd), ctypes.c_size_t(cols * 4)), "hipMalloc")
            ok(hip.hipMalloc(ctypes.byref(yd), ctypes.c_size_t(rows * 4)), "hipMalloc")
            ok(hip.hipMemcpy(xd, x.ctypes.data_as(vp), ctypes.c_size_t(cols * 4), 1), "hipMemcpy")
            ok(hip.hipStreamCreate(ctypes.byref(st)), "hipStreamCreate")
            n = max(iters, ncopy)
            runs = sorted(_graph_us(hip, st, lambda i: ws[i % ncopy].launch(xd.value, yd.value, st.value), n)
                          for _ in range(3))
            us = runs[1]
            hip.hipStreamDestroy(st)
            hip.hipFree(xd)
            hip.hipFree(yd)
            byts = w0.nbytes + 4 * cols + 4 * rows
            rec = {"type": names[kind], "rows": rows, "cols": cols, "median_us": round(us, 3),
                   "runs_us": [round(u, 3) for u in runs], "launches": n, "weight_copies": ncopy,
                   "bytes": int(byts), "GBps": round(byts / us / 1e3, 1),
                   "frac_hbm_peak": round(byts / us / 1e3 / PEAK_HBM_GBPS, 4)}
            for wc in ws:
                wc.free()
            if cpu:
                rc = _oracle()
                t0 = time.perf_counter()
                rc.matmul_t(blocks, kind, x, rows, threads)
                el = time.perf_counter() - t0
                rec["cpu_baseline"] = {"value": round(1e6 * el, 1), "unit": "us/GEMV", "cores": threads,
                                       "kind": "port", "sample": "one oracle/refcpu.c matmul_t (restated "
                                       "infer/matmul.odin:77-109) of the same matrix and x"}
            out.append(rec)
            log("GEMV %s %dx%d: %.2f us, %.0f GB/s" % (names[kind], rows, cols, us, byts / us / 1e3))
        del w32
    return out


PEAK_F16_TFLOPS = 2500.0  # MI355X dense f16 MFMA
ROTATE_BYTES = 1 << 30  # secondary benches cycle through >= 1 GiB of weights / state


def prefill_gemm(iters=50, cpu=True, tokens=64, shapes=((12, 4096, 4096), (12, 12288, 4096), (14, 4096, 12288))):
    """Batched projection (oi_gemm_launch, the prefill GEMM on the matrix cores)
    at the reference harness's projection shapes with 64 tokens: weights
    resident in HBM (copies totalling >= 1 GiB, cycled, so the Infinity Cache
    cannot serve repeats), f16 activations, f32 output.  max(iters, copies)
    launches (the K-split kernel and, when K is split, the reduction of the
    partial products) are captured in one HIP graph, so that the time is the
    device's and not the Python launch loop's; mean time per projection from
    HIP events around the graph launch.  Device buffers, streams, graphs and events come from the HIP
    runtime the library itself is linked against (libamdhip64)."""
    import ctypes
    import numpy as np
    from oi import ggml
    hip = ctypes.CDLL("libamdhip64.so")
    vp = ctypes.c_void_p

    def ok(rc, what):
        if rc != 0:
            raise RuntimeError("%s failed (%d)" % (what, rc))

    rng = np.random.default_rng(7)
    out = []
    for kind, m, k in shapes:
        n = tokens
        e, b = {12: (256, 144), 14: (256, 210)}[kind]
        nb = m * (k // e)
        raw = rng.integers(0, 256, size=(nb, b), dtype=np.uint8)
        d = (rng.random(nb) * 0.18 + 0.02).astype(np.float16).view(np.uint8).reshape(nb, 2)
        if kind == 12:
            raw[:, 0:2] = d
            raw[:, 2:4] = (rng.random(nb) * 0.05).astype(np.float16).view(np.uint8).reshape(nb, 2)
        else:
            raw[:, 208:210] = d
        # copies of the weights totalling >= 1 GiB, launch i reads copy i mod
        # ncopy, so the 256 MB Infinity Cache cannot serve repeats
        w0 = ggml.DeviceWeights(kind, raw.reshape(-1), m, k)
        ncopy = max(1, -(-ROTATE_BYTES // w0.nbytes))
        nlaunch = max(iters, ncopy)
        ws_list = [w0] + [ggml.DeviceWeights(kind, raw.reshape(-1), m, k) for _ in range(ncopy - 1)]
        w = w0
        xh = np.ascontiguousarray(rng.uniform(-1, 1, size=(n, k)).astype(np.float16))
        wsb = w.gemm_workspace_bytes(n)
        x, c, ws, st = vp(), vp(), vp(), vp()
        ok(hip.hipMalloc(ctypes.byref(x), ctypes.c_size_t(xh.nbytes)), "hipMalloc")
        ok(hip.hipMalloc(ctypes.byref(c), ctypes.c_size_t(n * m * 4)), "hipMalloc")
        if wsb:
            ok(hip.hipMalloc(ctypes.byref(ws), ctypes.c_size_t(wsb)), "hipMalloc")
        ok(hip.hipMemcpy(x, xh.ctypes.data_as(vp), ctypes.c_size_t(xh.nbytes), 1), "hipMemcpy")
        ok(hip.hipStreamCreate(ctypes.byref(st)), "hipStreamCreate")
        for _ in range(3):
            w.launch_gemm(x.value, n, c.value, ws.value, wsb, st.value)
        ok(hip.hipStreamSynchronize(st), "hipStreamSynchronize")
        graph, exe = vp(), vp()
        ok(hip.hipStreamBeginCapture(st, 0), "hipStreamBeginCapture")
        for i in range(nlaunch):
            ws_list[i % ncopy].launch_gemm(x.value, n, c.value, ws.value, wsb, st.value)
        ok(hip.hipStreamEndCapture(st, ctypes.byref(graph)), "hipStreamEndCapture")
        ok(hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, ctypes.c_size_t(0)), "hipGraphInstantiate")
        ok(hip.hipGraphLaunch(exe, st), "hipGraphLaunch")
        ok(hip.hipStreamSynchronize(st), "hipStreamSynchronize")
        e0, e1 = vp(), vp()
        ok(hip.hipEventCreate(ctypes.byref(e0)), "hipEventCreate")
        ok(hip.hipEventCreate(ctypes.byref(e1)), "hipEventCreate")
        ok(hip.hipEventRecord(e0, st), "hipEventRecord")
        ok(hip.hipGraphLaunch(exe, st), "hipGraphLaunch")
        ok(hip.hipEventRecord(e1, st), "hipEventRecord")
        ok(hip.hipEventSynchronize(e1), "hipEventSynchronize")
        ms = ctypes.c_float()
        ok(hip.hipEventElapsedTime(ctypes.byref(ms), e0, e1), "hipEventElapsedTime")
        us = ms.value * 1000.0 / nlaunch
        hip.hipEventDestroy(e0)
        hip.hipEventDestroy(e1)
        hip.hipGraphExecDestroy(exe)
        hip.hipGraphDestroy(graph)
        hip.hipStreamDestroy(st)
        hip.hipFree(x)
        hip.hipFree(c)
        if wsb:
            hip.hipFree(ws)
        flops = 2.0 * m * n * k
        byts = w.nbytes + n * k * 2 + n * m * 4
        out.append({"type": "Q4_K" if kind == 12 else "Q6_K", "rows": m, "cols": k, "tokens": n,
                    "avg_us": round(us, 3), "TFLOPs": round(flops / us / 1e6, 1),
                    "frac_f16_peak": round(flops / us / 1e6 / PEAK_F16_TFLOPS, 4),
                    "GBps": round(byts / us / 1e3, 1), "frac_hbm_peak": round(byts / us / 1e3 / PEAK_HBM_GBPS, 4)})
        for wc in ws_list:
            wc.free()
        out[-1]["weight_copies"] = ncopy
        if cpu:
            rc = _oracle()
            rows = 128
            t0 = time.perf_counter()
            rc.gemm_f16(raw.reshape(m, -1)[:rows].reshape(-1), kind, rows, k, xh.view(np.uint16))
            el = (time.perf_counter() - t0) * m / rows
            out[-1]["cpu_baseline"] = {
                "value": round(1e6 * el, 1), "unit": "us/projection", "cores": 1, "kind": "port",
                "sample": "oracle/refcpu.c ref_gemm_f16 (f16-staged operands, float64 sums, as the reference "
                          "harness's CPU check) on the first %d rows, scaled to %d" % (rows, m)}
    return out


def _oracle():
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import refcpu  # the oracle, timed as the CPU baseline
    return refcpu


def deltanet_step(iters=200, cpu=True):
    """Gated DeltaNet token step (oi_deltanet_step_launch) at the Qwen3.5 shape
    of the measurement plan: 16 k heads, 32 v heads, head dims 128, conv kernel
    4.  Inputs resident in HBM; the recurrent and conv states cycle through
    copies totalling >= 1 GiB (as the 36 layers' states do between two visits
    of one layer), so the Infinity Cache cannot serve them; the steps are
    captured in one HIP graph; mean time per step from HIP events around the
    graph launch.  Bytes: the recurrent state read and
    written (2 * 32*128*128*4) plus the conv window read and written and the
    step's vectors."""
    import ctypes
    import numpy as np
    from oi import _native
    hip = ctypes.CDLL("libamdhip64.so")
    vp = ctypes.c_void_p
    L = _native.hip()

    def ok(rc, what):
        if rc != 0:
            raise RuntimeError("%s failed (%d)" % (what, rc))

    n_kh, n_vh, hk, hv, kern = 16, 32, 128, 128, 4
    kd, vd = n_kh * hk, n_vh * hv
    cd = 2 * kd + vd
    rng = np.random.default_rng(3)
    f = np.float32
    host = {"qkv": rng.standard_normal(cd).astype(f), "z": rng.standard_normal(vd).astype(f),
            "b": rng.standard_normal(n_vh).astype(f), "a": rng.standard_normal(n_vh).astype(f),
            "conv_w": (rng.standard_normal(cd * kern) * 0.5).astype(f),
            "a_decay": (-np.exp(rng.standard_normal(n_vh) * 0.5)).astype(f),
            "dt_bias": (rng.standard_normal(n_vh) * 0.5).astype(f), "norm_w": np.ones(hv, f),
            "conv_state": rng.standard_normal(cd * (kern - 1)).astype(f),
            "rec_state": (rng.standard_normal(n_vh * hk * hv) * 0.1).astype(f),
            "scratch": np.zeros(cd, f), "out": np.zeros(vd, f)}
    dev = {}
    for k, arr in host.items():
        p = vp()
        ok(hip.hipMalloc(ctypes.byref(p), ctypes.c_size_t(arr.nbytes)), "hipMalloc")
        ok(hip.hipMemcpy(p, arr.ctypes.data_as(vp), ctypes.c_size_t(arr.nbytes), 1), "hipMemcpy")
        dev[k] = p
    d = _native.DeltaNetDims(n_kh, n_vh, hk, hv, kern, 1e-6)
    # one layer's states per copy, >= 1 GiB cycled (a decode step visits each
    # layer's state once, with the weights of every layer in between)
    st_bytes = host["rec_state"].nbytes + host["conv_state"].nbytes
    ncopy = -(-ROTATE_BYTES // st_bytes)
    big = {}
    for k in ("rec_state", "conv_state"):
        p = vp()
        nb = host[k].nbytes
        ok(hip.hipMalloc(ctypes.byref(p), ctypes.c_size_t(nb * ncopy)), "hipMalloc")
        for c in range(ncopy):
            ok(hip.hipMemcpy(vp(p.value + c * nb), host[k].ctypes.data_as(vp), ctypes.c_size_t(nb), 1), "hipMemcpy")
        big[k] = (p, nb)
    st = vp()
    ok(hip.hipStreamCreate(ctypes.byref(st)), "hipStreamCreate")
    order = ("qkv", "z", "b", "a", "conv_w", "a_decay", "dt_bias", "norm_w")

    def launch(i):
        c = i % ncopy
        cs = vp(big["conv_state"][0].value + c * big["conv_state"][1])
        rs = vp(big["rec_state"][0].value + c * big["rec_state"][1])
        ok(L.oi_deltanet_step_launch(ctypes.byref(d), *[dev[k] for k in order], cs, rs, dev["scratch"], dev["out"],
                                     st), "oi_deltanet_step_launch")

    iters = max(iters, ncopy)
    us = _graph_us(hip, st, launch, iters)
    hip.hipStreamDestroy(st)
    for p in dev.values():
        hip.hipFree(p)
    for p, _ in big.values():
        hip.hipFree(p)
    byts = 2 * n_vh * hk * hv * 4 + 2 * cd * (kern - 1) * 4 + cd * kern * 4 + (cd + 2 * vd + 2 * n_vh) * 4
    out = {"shape": "n_k_heads 16, n_v_heads 32, head dims 128, conv kernel 4", "avg_us": round(us, 3),
           "state_copies": ncopy, "bytes": byts, "GBps": round(byts / us / 1e3, 1), "frac_hbm_peak": round(byts / us / 1e3 / PEAK_HBM_GBPS, 4),
           "kernels": "dn_step_kernel (conv, gates and delta rule in one launch)"}
    if cpu:
        rc = _oracle()
        n = 20
        t0 = time.perf_counter()
        rc.deltanet_steps(n_kh, n_vh, hk, hv, kern, 1e-6, np.tile(host["qkv"], (n, 1)), np.tile(host["z"], (n, 1)),
                          np.tile(host["b"], (n, 1)), np.tile(host["a"], (n, 1)), host["conv_w"], host["a_decay"],
                          host["dt_bias"], host["norm_w"], host["conv_state"], host["rec_state"])
        el = time.perf_counter() - t0
        out["cpu_baseline"] = {"value": round(1e6 * el / n, 3), "unit": "us/step", "cores": 1, "kind": "port",
                               "sample": "%d steps of oracle/refcpu.c ref_deltanet_steps (restated qwen3_5/ops.odin "
                                         "and qwen3_5/forward.odin:172-219), same shape" % n}
    return out


def _graph_us(hip, st, launch, iters):
    """Mean device time of `launch(i)` over `iters` launches (i = 0..iters-1)
    captured in one HIP graph on stream st (HIP events around a second graph
    launch)."""
    import ctypes
    vp = ctypes.c_void_p

    def ok(rc, what):
        if rc != 0:
            raise RuntimeError("%s failed (%d)" % (what, rc))

    launch(0)
    ok(hip.hipStreamSynchronize(st), "hipStreamSynchronize")
    graph, exe = vp(), vp()
    ok(hip.hipStreamBeginCapture(st, 0), "hipStreamBeginCapture")
    for i in range(iters):
        launch(i)
    ok(hip.hipStreamEndCapture(st, ctypes.byref(graph)), "hipStreamEndCapture")
    ok(hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, ctypes.c_size_t(0)), "hipGraphInstantiate")
    ok(hip.hipGraphLaunch(exe, st), "hipGraphLaunch")
    ok(hip.hipStreamSynchronize(st), "hipStreamSynchronize")
    e0, e1 = vp(), vp()
    ok(hip.hipEventCreate(ctypes.byref(e0)), "hipEventCreate")
    ok(hip.hipEventCreate(ctypes.byref(e1)), "hipEventCreate")
    ok(hip.hipEventRecord(e0, st), "hipEventRecord")
    ok(hip.hipGraphLaunch(exe, st), "hipGraphLaunch")
    ok(hip.hipEventRecord(e1, st), "hipEventRecord")
    ok(hip.hipEventSynchronize(e1), "hipEventSynchronize")
    ms = ctypes.c_float()
    ok(hip.hipEventElapsedTime(ctypes.byref(ms), e0, e1), "hipEventElapsedTime")
    for h in (e0, e1):
        hip.hipEventDestroy(h)
    hip.hipGraphExecDestroy(exe)
    hip.hipGraphDestroy(graph)
    return ms.value * 1000.0 / iters


def qwen35_attn_step(iters=100, seq_len=4096, cpu=True):
    """Attention of a Qwen3.5 full-attention layer for one token
    (oi_qwen35_attn_step_launch) at the measurement-plan shape: 16 q heads of
    256 with gate, 2 kv heads, partial RoPE over 64 dimensions, at the last
    position of a 4096-token f16 cache; the launches cycle through cache copies
    totalling >= 1 GiB (one per layer, as a decode step visits them).  Bytes: the K and V rows read
    (2 * 2 * 4096 * 256 * 2) plus q/gate, k, v and the output."""
    import ctypes
    import numpy as np
    from oi import _native
    hip = ctypes.CDLL("libamdhip64.so")
    vp = ctypes.c_void_p
    L = _native.hip()

    def ok(rc, what):
        if rc != 0:
            raise RuntimeError("%s failed (%d)" % (what, rc))

    nh, nkv, hd, rd = 16, 2, 256, 64
    rng = np.random.default_rng(4)
    f = np.float32
    d = _native.Qwen35AttnDims(nh, nkv, hd, rd, seq_len, 1e-6)
    host = {"qproj": rng.standard_normal(nh * 2 * hd).astype(f), "k": rng.standard_normal(nkv * hd).astype(f),
            "v": rng.standard_normal(nkv * hd).astype(f), "q_norm": np.ones(hd, f), "k_norm": np.ones(hd, f),
            "inv_freq": (1e7 ** (-(np.arange(rd // 2) / (rd / 2.0)))).astype(f),
            "kc": rng.standard_normal(nkv * seq_len * hd).astype(np.float16),
            "vc": rng.standard_normal(nkv * seq_len * hd).astype(np.float16),
            "ws": np.zeros(L.oi_qwen35_attn_workspace_bytes(ctypes.byref(d)) // 4, f), "out": np.zeros(nh * hd, f)}
    dev = {}
    for k, arr in host.items():
        p = vp()
        ok(hip.hipMalloc(ctypes.byref(p), ctypes.c_size_t(arr.nbytes)), "hipMalloc")
        ok(hip.hipMemcpy(p, arr.ctypes.data_as(vp), ctypes.c_size_t(arr.nbytes), 1), "hipMemcpy")
        dev[k] = p
    # one layer's K and V cache per copy, >= 1 GiB cycled
    cb = host["kc"].nbytes
    ncopy = -(-ROTATE_BYTES // (2 * cb))
    big = vp()
    ok(hip.hipMalloc(ctypes.byref(big), ctypes.c_size_t(2 * cb * ncopy)), "hipMalloc")
    for c in range(ncopy):
        ok(hip.hipMemcpy(vp(big.value + 2 * c * cb), host["kc"].ctypes.data_as(vp), ctypes.c_size_t(cb), 1), "hipMemcpy")
        ok(hip.hipMemcpy(vp(big.value + (2 * c + 1) * cb), host["vc"].ctypes.data_as(vp), ctypes.c_size_t(cb), 1),
           "hipMemcpy")
    st = vp()
    ok(hip.hipStreamCreate(ctypes.byref(st)), "hipStreamCreate")
    order = ("qproj", "k", "v", "q_norm", "k_norm", "inv_freq")

    def launch(i):
        c = i % ncopy
        kc, vc = vp(big.value + 2 * c * cb), vp(big.value + (2 * c + 1) * cb)
        ok(L.oi_qwen35_attn_step_launch(ctypes.byref(d), seq_len - 1, *[dev[k] for k in order], kc, vc, dev["ws"],
                                        dev["out"], st), "oi_qwen35_attn_step_launch")

    us = _graph_us(hip, st, launch, max(iters, ncopy))
    hip.hipStreamDestroy(st)
    for p in dev.values():
        hip.hipFree(p)
    hip.hipFree(big)
    byts = 2 * 2 * nkv * seq_len * hd + 4 * (nh * 2 * hd + 2 * nkv * hd + nh * hd)
    out = {"shape": "16 q heads x 256 (+gate), 2 kv heads, rotary 64, position 4095 of a 4096 f16 cache",
           "avg_us": round(us, 3), "cache_copies": ncopy, "bytes": byts, "GBps": round(byts / us / 1e3, 1),
           "frac_hbm_peak": round(byts / us / 1e3 / PEAK_HBM_GBPS, 4),
           "kernels": "q35_lane_kernel (q/k norm + RoPE fused; 64 splits x 2 kv heads, one wave per query head) + q35_combine_kernel"}
    if cpu:
        rc = _oracle()
        kc16 = host["kc"].view(np.uint16).reshape(nkv, seq_len, hd)
        vc16 = host["vc"].view(np.uint16).reshape(nkv, seq_len, hd)
        t0 = time.perf_counter()
        rc.qwen35_attn_steps(nh, nkv, hd, rd, seq_len, 1e-6, seq_len - 1, host["qproj"], host["k"], host["v"],
                             host["q_norm"], host["k_norm"], host["inv_freq"], kc16, vc16)
        el = time.perf_counter() - t0
        out["cpu_baseline"] = {"value": round(1e6 * el, 1), "unit": "us/step", "cores": 1, "kind": "port",
                               "sample": "1 step at position 4095 of oracle/refcpu.c ref_qwen35_attn_steps "
                                         "(restated qwen3_5/forward.odin:69-127), same shape and cache"}
    return out


def moe_step(iters=100, cpu=True):
    """Routed-expert FFN for one token (oi_moe_ffn_launch) at the config-4
    shape: 128 experts, top 8, dim 2048, expert inner 768, Q4_K experts, F32
    router; weights resident in HBM (whole weight sets cycled, >= 1 GiB, so the
    Infinity Cache cannot serve the chosen experts again), experts chosen on
    the device.  Bytes: the
    router and the 8 chosen experts' gate, up and down matrices."""
    import ctypes
    import numpy as np
    from oi import _native, ggml, synth
    hip = ctypes.CDLL("libamdhip64.so")
    vp = ctypes.c_void_p
    L = _native.hip()

    def ok(rc, what):
        if rc != 0:
            raise RuntimeError("%s failed (%d)" % (what, rc))

    E, k, dim, inter = 128, 8, 2048, 768
    rng = np.random.default_rng(8)
    router = (rng.standard_normal((E, dim)) * 0.1).astype(np.float32)
    mats = [synth.quantize_rows(12, (rng.standard_normal((E * inter, dim)) * 0.05).astype(np.float32)),
            synth.quantize_rows(12, (rng.standard_normal((E * inter, dim)) * 0.05).astype(np.float32)),
            synth.quantize_rows(12, (rng.standard_normal((E * dim, inter)) * 0.05).astype(np.float32))]
    # whole weight sets (router + all experts) cycled, >= 1 GiB in total
    sets = []
    while True:
        sets.append((ggml.DeviceWeights(0, router.view(np.uint8).reshape(-1), E, dim),
                     ggml.DeviceWeights(12, mats[0], E * inter, dim), ggml.DeviceWeights(12, mats[1], E * inter, dim),
                     ggml.DeviceWeights(12, mats[2], E * dim, inter)))
        if len(sets) * sum(w.nbytes for w in sets[0]) >= ROTATE_BYTES:
            break
    wr, wg, wu, wd = sets[0]
    d = _native.MoeDims(E, k, dim, inter, 1)
    x, y, ws, st = vp(), vp(), vp(), vp()
    xh = rng.standard_normal(dim).astype(np.float32)
    ok(hip.hipMalloc(ctypes.byref(x), ctypes.c_size_t(dim * 4)), "hipMalloc")
    ok(hip.hipMalloc(ctypes.byref(y), ctypes.c_size_t(dim * 4)), "hipMalloc")
    ok(hip.hipMalloc(ctypes.byref(ws), ctypes.c_size_t(L.oi_moe_workspace_bytes(ctypes.byref(d)))), "hipMalloc")
    ok(hip.hipMemcpy(x, xh.ctypes.data_as(vp), ctypes.c_size_t(dim * 4), 1), "hipMemcpy")
    ok(hip.hipStreamCreate(ctypes.byref(st)), "hipStreamCreate")

    def launch(i):
        r, g, u, dn = sets[i % len(sets)]
        ok(L.oi_moe_ffn_launch(ctypes.byref(d), r.h, g.h, u.h, dn.h, x, ws, y, st), "oi_moe_ffn_launch")

    us = _graph_us(hip, st, launch, max(iters, len(sets)))
    hip.hipStreamDestroy(st)
    for p in (x, y, ws):
        hip.hipFree(p)
    per_expert = (wg.nbytes + wu.nbytes + wd.nbytes) / E
    byts = wr.nbytes + k * per_expert
    for ws_ in sets:
        for w in ws_:
            w.free()
    out = {"shape": "128 experts, top 8, dim 2048, inter 768, Q4_K experts, F32 router", "avg_us": round(us, 3),
           "weight_sets": len(sets),
           "bytes": int(byts), "GBps": round(byts / us / 1e3, 1), "frac_hbm_peak": round(byts / us / 1e3 / PEAK_HBM_GBPS, 4),
           "kernels": "router GEMV + gemv_q_kernel rows mode (routing in its prologue, gate/up) + "
                      "gemv_q_kernel columns mode (down)"}
    if cpu:
        rc = _oracle()
        t0 = time.perf_counter()
        rc.moe_ffn(E, k, dim, inter, 1, 0, router.view(np.uint8).reshape(-1), 12, mats[0], mats[1], mats[2], xh)
        el = time.perf_counter() - t0
        out["cpu_baseline"] = {"value": round(1e6 * el, 1), "unit": "us/token", "cores": 1, "kind": "port",
                               "sample": "1 token of oracle/refcpu.c ref_moe_ffn (HF Qwen3-MoE convention restated), "
                                         "same weights and input"}
    return out


def _free_gb(path):
    st = os.statvfs(path)
    return st.f_bavail * st.f_frsize / 1e9


def model_decode(name, context, steps, warmup=8, prompt=0, cpu=True, cpu_budget=20.0, chunks=(64, 512)):
    """A whole-model decode measurement at batch 1 for the routed-expert and
    hybrid configurations: the synthetic model `name` (full size), then either
    the f16 KV cache pre-filled with N(0,1) to `context` positions (config 4)
    or a `prompt`-token random-id prompt through engine_forward_batch (config
    5, the hybrid's DeltaNet states need the prompt itself), then `steps`
    greedy steps of the device-side loop.  Bytes per token: every launch's
    algorithmic bytes (routed experts: only the chosen ones) from the engine's
    own accounting at the mean position.  CPU baseline: the oracle on a bounded
    sample of the same decode."""
    import numpy as np
    from oi import infer, synth
    spec = synth.CONFIGS[name]
    d = tempfile.mkdtemp(prefix="oi_%s_" % name)
    try:
        need = 1.2 * weight_bytes_any(spec) / 1e9 + 1
        if _free_gb(d) < need:
            return {"skipped": "needs %.0f GB of temporary disk, %.0f GB free" % (need, _free_gb(d))}
        path = os.path.join(d, name + ".gguf")
        t = time.time()
        synth.write_gguf(path, name)
        log("wrote synthetic %s (%.2f GB) in %.1fs" % (name, os.path.getsize(path) / 1e9, time.time() - t))
        start = context if not prompt else prompt
        e, _ = infer.engine_load(path, infer.Engine_Opts(max_ctx=start + steps + warmup + 8))
        cfg = infer.engine_config(e)
        out = {"model": name, "layers": cfg.n_layers, "dim": cfg.dim, "vocab": cfg.vocab_size}
        try:
            if prompt:
                toks = np.random.default_rng(5).integers(0, cfg.vocab_size, size=prompt).astype(np.int32)
                infer.engine_forward_batch(e, toks[:64], 0)  # allocates the prefill buffers
                pf = {"tokens": prompt}
                for chunk in chunks:
                    best = None
                    for _ in range(3):
                        infer.engine_reset_state(e)
                        t0 = time.perf_counter()
                        for i in range(0, prompt, chunk):
                            logits = infer.engine_forward_batch(e, toks[i:i + chunk], i)
                        pel = time.perf_counter() - t0
                        best = pel if best is None else min(best, pel)
                    wk = hybrid_prefill_work(spec, prompt, chunk)
                    pf["chunk%d" % chunk] = {
                        "ms": round(1000 * best, 1), "tok_s": round(prompt / best, 1),
                        "algorithmic_bytes": wk["bytes"], "GBps": round(wk["bytes"] / best / 1e9, 1),
                        "frac_hbm_peak": round(wk["bytes"] / best / 1e9 / PEAK_HBM_GBPS, 4),
                        "TFLOPs": round(wk["flops"] / best / 1e12, 2),
                        "frac_f16_peak": round(wk["flops"] / best / 1e12 / PEAK_F16_TFLOPS, 4),
                        "distinct_experts_per_call": wk["distinct_experts_per_call"]}
                    log("%s prefill, %d-token chunks: %d tokens in %.1f ms (%.0f tok/s)" % (
                        name, chunk, prompt, 1000 * best, prompt / best))
                first = int(np.argmax(logits))
                pf["note"] = ("batched prefill (oi_engine_prefill) from a reset state, one call per chunk, host "
                              "wall clock, best of 3; decode continues from the last chunk length's run; bytes and "
                              "FLOPs from bench.hybrid_prefill_work (routed experts: expected distinct experts "
                              "per call under uniform routing)")
                out["prefill"] = pf
                snap = None
            else:
                k, v = synth.kv_prefill(777, cfg.n_layers, cfg.n_kv_heads, context, cfg.head_dim)
                infer.engine_kv_fill(e, 0, 0, k, v)
                first = 0
                snap = (k, v)
            if warmup and not prompt:
                infer.engine_decode_greedy(e, first, start, warmup)
            t0 = time.perf_counter()
            toks = infer.engine_decode_greedy(e, first, start, steps)
            el = time.perf_counter() - t0
            tok_s = steps / el
            infer.engine_forward(e, int(toks[-1]), start + steps - 1)
            us, bpt = infer.engine_time_kernel(e, "token", min(steps, 64))
            kern = {}
            for kn in ("qkv", "attn", "wo", "router", "gateup", "down", "shared", "linear_in", "deltanet",
                       "linear_out", "output"):
                try:
                    infer.engine_time_kernel(e, kn, 16)
                    ku, kb = infer.engine_time_kernel(e, kn, 64)
                    kern[kn] = {"avg_us": round(ku, 3), "GBps": round(kb / ku / 1e3, 1)}
                except Exception:
                    pass
            gbps = bpt * tok_s / 1e9
            out.update({"decode_tok_s": round(tok_s, 2), "ms_per_token": round(1000 * el / steps, 4),
                        "steps": steps, "from_pos": start, "bytes_per_token": int(bpt),
                        "achieved_GBps": round(gbps, 1), "frac_hbm_peak": round(gbps / PEAK_HBM_GBPS, 4),
                        "kernels_us": kern})
            log("%s decode: %.1f tok/s, %.0f GB/s (%.1f%% of peak)" % (name, tok_s, gbps,
                                                                        100 * gbps / PEAK_HBM_GBPS))
        finally:
            infer.engine_destroy(e)
        if cpu:
            sys.path.insert(0, os.path.join(REPO, "oracle"))
            import refcpu
            threads, nproc = cpu_threads()
            r = refcpu.RefEngine(path, max_ctx=start + 64, num_threads=threads, kv_f16=True)
            try:
                if snap is not None:
                    for layer in range(cfg.n_layers):
                        r.kv_fill(layer, 0, snap[0][layer], snap[1][layer])
                    tok, n, t0 = first, 0, time.perf_counter()
                    while True:
                        tok = refcpu.argmax(r.forward(tok, start + n))
                        n += 1
                        if time.perf_counter() - t0 > cpu_budget or n >= 16:
                            break
                    el = time.perf_counter() - t0
                    sample = "%d greedy steps from pos %d of the same model and pre-filled cache" % (n, start)
                else:
                    # the hybrid's state needs the prompt: time the oracle's first prompt tokens
                    n, t0 = 0, time.perf_counter()
                    ptoks = np.random.default_rng(5).integers(0, cfg.vocab_size, size=16)
                    for t in ptoks:
                        r.forward(int(t), n)
                        n += 1
                        if time.perf_counter() - t0 > cpu_budget:
                            break
                    el = time.perf_counter() - t0
                    sample = "%d forward steps from position 0 (the prompt's first tokens) of the same model" % n
                out["cpu_baseline"] = {"value": round(n / el, 4), "unit": "tok/s", "cores": threads, "nproc": nproc,
                                       "kind": "port", "sample": sample + ", oracle/refcpu.c"}
            finally:
                r.close()
        return out
    finally:
        shutil.rmtree(d, ignore_errors=True)


def hybrid_prefill_work(spec, prompt, chunk):
    """Algorithmic HBM bytes and FLOPs of a Qwen3.5 hybrid routed-expert
    prompt of `prompt` tokens run in `chunk`-token calls (oi_engine_prefill,
    qwen3_5/forward.odin:46-225 per token).  Per call: every dense weight once
    (attention / DeltaNet projections, router, shared expert, the output
    projection for the call's last row), the routed experts that the call's
    tokens select -- counted as the expected number of distinct experts under
    uniform routing, E (1 - (1 - k/E)^T) of E, since a call streams each
    selected expert once -- the K/V of the full-attention layers read up to the
    call's last position and written for its tokens, and the DeltaNet conv and
    recurrent states read and written once.  FLOPs: 2 per weight element per
    token for the dense weights and the k routed experts, plus 4 hd per key
    per head for attention (scores and values) and 4 hk hv per token per value
    head for the delta rule."""
    from oi.ggml import row_byte_size
    D, V, L = spec["dim"], spec["vocab_size"], spec["n_layers"]
    Q, KV, hd = spec["n_heads"] * spec["head_dim"], spec["n_kv_heads"] * spec["head_dim"], spec["head_dim"]
    E, k, EF, SF = spec["n_experts"], spec["n_experts_used"], spec["expert_ffn"], spec["shared_expert_ffn"]
    nv, hk, hv = spec["lin_n_v_heads"], spec["lin_head_k_dim"], spec["lin_head_v_dim"]
    KD, VD = spec["lin_n_k_heads"] * hk, nv * hv
    CD, ck = 2 * KD + VD, spec["lin_conv_kernel"]
    t, tv, tdn, tr = spec["type_default"], spec["type_attn_v"], spec["type_ffn_down"], spec["type_router"]
    n_full = sum(1 for l in range(L) if (l + 1) % spec["full_attn_interval"] == 0)
    n_lin = L - n_full
    rb = row_byte_size
    full_w = rb(t, D) * (2 * Q + KV) + rb(tv, D) * KV + rb(t, Q) * D
    full_p = D * (2 * Q + 2 * KV) + Q * D
    lin_w = rb(t, D) * (CD + VD + 2 * nv) + rb(t, VD) * D + 4 * CD * ck
    lin_p = D * (CD + VD + 2 * nv) + VD * D
    ffn_w = rb(tr, D) * (E + 1) + rb(t, D) * 2 * SF + rb(tdn, SF) * D
    ffn_p = D * (E + 1) + 3 * SF * D
    exp_w = rb(t, D) * 2 * EF + rb(tdn, EF) * D
    exp_p = 3 * EF * D
    dense_w = n_full * full_w + n_lin * lin_w + L * ffn_w + rb(spec["type_output"], D) * V
    per_tok_p = n_full * full_p + n_lin * lin_p + L * (ffn_p + k * exp_p)
    state = n_lin * (nv * hk * hv * 4 + CD * (ck - 1) * 4)
    byts = flops = 0.0
    for p0 in range(0, prompt, chunk):
        T = min(chunk, prompt - p0)
        distinct = E * (1.0 - (1.0 - k / E) ** T)
        byts += dense_w + L * distinct * exp_w + T * rb(spec["type_embd"], D)
        byts += n_full * 2 * KV * 2 * (p0 + T) + n_full * 2 * KV * 2 * T + 2 * state
        flops += 2.0 * T * per_tok_p + 2.0 * D * V
        keys = T * p0 + T * (T + 1) / 2  # causal keys over the call's rows
        flops += n_full * 4.0 * spec["n_heads"] * hd * keys + n_lin * 4.0 * T * nv * hk * hv
    return {"bytes": int(byts), "flops": flops,
            "distinct_experts_per_call": round(E * (1.0 - (1.0 - k / E) ** min(chunk, prompt)), 1)}


def weight_bytes_any(spec):
    """GGUF bytes of a synthetic model of any architecture (for disk checks)."""
    from oi.ggml import row_byte_size
    D, L, V = spec["dim"], spec["n_layers"], spec["vocab_size"]
    QD, KVD = spec["n_heads"] * spec["head_dim"], spec["n_kv_heads"] * spec["head_dim"]
    t = spec["type_default"]
    per = row_byte_size(t, D) * (2 * QD + 2 * KVD) + row_byte_size(t, QD) * D
    if spec["n_experts"]:
        per += 3 * spec["n_experts"] * spec["expert_ffn"] * row_byte_size(t, D)
        per += 3 * spec.get("shared_expert_ffn", 0) * row_byte_size(t, D)
    else:
        per += 3 * spec["hidden_dim"] * row_byte_size(t, D)
    return L * per + 2 * V * row_byte_size(t, D)


def measure_prefill(e, cfg, n, reps=7):
    """Batched prefill of an n-token prompt at position 0 (engine_forward_batch,
    synchronous): host wall clock per call after one warm call (which also
    allocates the prefill buffers); the median of `reps` calls (single calls
    vary by several percent), with the fastest and slowest."""
    import numpy as np
    from oi import infer
    ptoks = np.random.default_rng(99).integers(0, cfg.vocab_size, size=n).astype(np.int32)
    infer.engine_forward_batch(e, ptoks, 0)
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        infer.engine_forward_batch(e, ptoks, 0)
        times.append(time.perf_counter() - t0)
    times.sort()
    pel = times[len(times) // 2]
    D, QD, KVD, H = cfg.dim, cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim, cfg.hidden_dim
    proj_flop = 2.0 * n * cfg.n_layers * (2 * D * QD + 2 * D * KVD + 3 * D * H)
    log("prefill: %d tokens in %.2f ms -> %.0f tok/s" % (n, 1000 * pel, n / pel))
    return {"tokens": n, "tok_s": round(n / pel, 1), "ms": round(1000 * pel, 3),
            "ms_min": round(1000 * times[0], 3), "ms_max": round(1000 * times[-1], 3), "calls": reps,
            "projection_TFLOPs": round(proj_flop / pel / 1e12, 1),
            "note": "host wall clock around oi_engine_prefill (synchronous), median of the calls, chunks of "
                    "<=512 tokens; the prompt overwrites the cache from position 0 after the decode measurement"}


def remove_stale_models(min_age_s=120):
    """Delete the synthetic models that an earlier bench run left in the
    temporary directory when it ended abnormally (each is up to 45 GB; left
    behind they make later runs skip the whole-model measurements for lack
    of disk).  Only this script's directories (oi_bench_*, oi_c1_*, oi_<model>_*
    holding nothing but .gguf files) older than min_age_s are removed."""
    root = tempfile.gettempdir()
    removed = 0
    try:
        names = os.listdir(root)
    except OSError:
        return 0
    for name in names:
        p = os.path.join(root, name)
        if not name.startswith("oi_") or not os.path.isdir(p) or os.path.islink(p):
            continue
        try:
            files = os.listdir(p)
            if not files or not all(f.endswith(".gguf") for f in files):
                continue
            if time.time() - os.path.getmtime(p) < min_age_s:
                continue
            shutil.rmtree(p, ignore_errors=True)
            removed += 1
        except OSError:
            continue
    if removed:
        log("removed %d stale synthetic-model directories from %s" % (removed, root))
    return removed


def prompt_breakdown(path, layers=48, calls=32):
    """Kernel time of the first 64-token-chunk prompt in a rocprofv3 kernel trace
    of --only c5: the first `calls` consecutive prefill calls (each starts with
    embed_rows_kernel) whose routing runs on 64 tokens (pf_moe_topk_kernel over
    64 workgroups, once per layer), summed by kernel and grid."""
    import csv
    import collections
    rows = []
    with open(path) as f:
        for r in csv.DictReader(f):
            nm = r["Kernel_Name"]
            nm = nm[:nm.rfind("(")] if nm.endswith(")") else nm
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), nm,
                         int(r["Grid_Size_X"]) // max(1, int(r["Workgroup_Size_X"]))))
    rows.sort()
    starts = [i for i, r in enumerate(rows) if r[2].endswith("embed_rows_kernel")] + [len(rows)]
    for k in range(len(starts) - calls):
        seg = rows[starts[k]:starts[k + calls]]
        topk = [r for r in seg if r[2].endswith("pf_moe_topk_kernel")]
        if len(topk) == calls * layers and all(r[3] == 64 for r in topk):
            break
    else:
        sys.exit("no %d-call prompt of 64-token chunks in the trace" % calls)
    span = (seg[-1][1] - seg[0][0]) / 1e6
    d = collections.defaultdict(list)
    for st, en, nm, g in seg:
        d[(nm, g)].append((en - st) / 1e3)
    tot = sum(sum(v) for v in d.values())
    print("first 64-token-chunk prompt: span %.1f ms, kernel time %.1f ms, %d dispatches" % (span, tot / 1e3, len(seg)))
    for (nm, g), v in sorted(d.items(), key=lambda kv: -sum(kv[1])):
        v.sort()
        print("%-48s grid %5d n %5d median %6.1f us total %7.2f ms (%4.1f%%)" %
              (nm[-48:], g, len(v), v[len(v) // 2], sum(v) / 1e3, 100 * sum(v) / tot))


def layer_timeline(path):
    """Per-layer timeline of one decode token from a rocprofv3 kernel trace: the
    dispatches of the last whole token (embed_kernel to the next embed_kernel),
    grouped into the 36 layers' six launches (QKV GEMV, attention splits,
    split merge, wo GEMV, gate/up GEMV, down GEMV); for each launch its mean
    duration and the mean gap from the previous dispatch's end to its start."""
    import csv
    rows = []
    with open(path) as f:
        for r in csv.DictReader(f):
            nm = r["Kernel_Name"]
            nm = nm[:nm.rfind("(")] if nm.endswith(")") else nm  # without the parameter list
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), nm))
    rows.sort()
    starts = [i for i, r in enumerate(rows) if r[2].endswith("embed_kernel")]
    # the last whole greedy token (the run ends with sampled tokens)
    toks = [rows[a:b] for a, b in zip(starts, starts[1:])
            if b - a > 1 + 36 * 6 and not any("sample" in r[2] for r in rows[a:b])]
    if not toks:
        sys.exit("no whole greedy token in the trace")
    tok = toks[-1]
    body = tok[1:]  # after the embedding
    nl = 36
    per = 6
    if len(body) < nl * per:
        sys.exit("unexpected dispatch count %d" % len(tok))
    names = ["QKV GEMV (RMSNorm prologue)", "attention splits", "split merge", "wo GEMV (+ residual)",
             "gate/up GEMV (RMSNorm prologue, SwiGLU)", "down GEMV (+ residual)"]
    dur = [[] for _ in range(per)]
    gap = [[] for _ in range(per)]
    prev_end = tok[0][1]
    for l in range(nl):
        for k in range(per):
            st, en, _ = body[l * per + k]
            dur[k].append((en - st) / 1e3)
            gap[k].append((st - prev_end) / 1e3)
            prev_end = en
    tail = body[nl * per:]
    span = (tok[-1][1] - tok[0][0]) / 1e3
    busy = sum((r[1] - r[0]) / 1e3 for r in tok)
    print("token: %d dispatches, span %.1f us, kernel time %.1f us (%.1f%%)" % (len(tok), span, busy, 100 * busy / span))
    print("%-42s %10s %10s %10s" % ("launch (mean over the 36 layers)", "gap us", "kernel us", "kernel"))
    for k in range(per):
        print("%-42s %10.2f %10.2f  %s" % (names[k], sum(gap[k]) / nl, sum(dur[k]) / nl, body[k][2][-60:]))
    lay = sum(sum(d) for d in dur) / nl
    lg = sum(sum(g) for g in gap) / nl
    print("%-42s %10.2f %10.2f" % ("layer", lg, lay))
    for st, en, nm in tail:
        print("after the layers: %s %.2f us" % (nm[-60:], (en - st) / 1e3))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=512)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--cpu-budget", type=float, default=40.0, help="seconds of CPU baseline work (decode sample)")
    ap.add_argument("--no-microbench", action="store_true", help="skip the config-2 GEMV microbench")
    ap.add_argument("--no-models", action="store_true", help="skip the config-4 / config-5 whole-model decodes")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--model-path", default=None, help="reuse an existing synthetic GGUF")
    ap.add_argument("--no-gemm", action="store_true", help="skip the prefill GEMM measurement")
    ap.add_argument("--no-prefill", action="store_true", help="skip the batched prefill measurement")
    ap.add_argument("--prefill-tokens", type=int, default=512)
    ap.add_argument("--only", choices=["prefill", "gemm", "deltanet", "qwen35_attn", "moe", "gemv", "c1", "decode",
                                       "c4", "c5"],
                    default=None,
                    help="run one secondary measurement alone (for profiling) and print its JSON")
    ap.add_argument("--c5-model", default="qwen35-hybrid-moe",
                    help="synthetic model of --only c5 (a shorter model of the same shapes, such as "
                         "qwen35-hybrid-moe-4layer, gives the same per-launch kernels for profiling)")
    ap.add_argument("--c5-chunks", default="64,512", help="prompt chunk lengths of --only c5, comma-separated")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a device-to-device copy of MIB MiB (3 times), to calibrate HBM counters")
    ap.add_argument("--prompt-breakdown", default=None, metavar="TRACE_CSV",
                    help="only summarise a rocprofv3 kernel trace of --only c5: kernel time of the first "
                         "64-token-chunk prompt, by kernel and grid")
    ap.add_argument("--layer-timeline", default=None, metavar="TRACE_CSV",
                    help="only summarise a rocprofv3 kernel trace of the decode (--only decode, OI_NO_GRAPH=1): "
                         "per-layer kernel durations and gaps of its last whole token")
    args = ap.parse_args()
    if args.layer_timeline:
        layer_timeline(args.layer_timeline)
        return
    if args.prompt_breakdown:
        prompt_breakdown(args.prompt_breakdown)
        return
    remove_stale_models()
    if args.copy_calibration:
        import torch
        n = args.copy_calibration << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_per_dispatch": n}))
        return
    if args.gpus != 1:
        print("bench.py measures one GPU only: the token loop runs on a single MI355X "
              "(multi-GPU sharding is a design note, not built); got --gpus %d" % args.gpus, file=sys.stderr)
        sys.exit(2)
    if CONTEXT + args.steps > 4608 + 8192:
        sys.exit("too many steps")

    from oi import infer, synth
    import numpy as np

    if args.only == "gemm":
        print(json.dumps({"prefill_gemm": prefill_gemm()}), flush=True)
        return
    if args.only == "deltanet":
        print(json.dumps({"deltanet_step": deltanet_step()}), flush=True)
        return
    if args.only == "qwen35_attn":
        print(json.dumps({"qwen35_attn_step": qwen35_attn_step()}), flush=True)
        return
    if args.only == "moe":
        print(json.dumps({"moe_step": moe_step()}), flush=True)
        return
    if args.only == "gemv":
        print(json.dumps({"gemv_microbench": gemv_microbench(cpu=not args.no_cpu)}), flush=True)
        return
    if args.only == "c1":
        print(json.dumps({"c1": c1_cpu_run()}), flush=True)
        return
    if args.only == "c4":
        print(json.dumps({"c4": model_decode("qwen3-30b-a3b-q4_k", 2048, 256, cpu=not args.no_cpu)}), flush=True)
        return
    if args.only == "c5":
        chunks = tuple(int(c) for c in args.c5_chunks.split(","))
        print(json.dumps({"c5": model_decode(args.c5_model, 0, 256, prompt=2048, cpu=not args.no_cpu,
                                             chunks=chunks)}), flush=True)
        return

    tmpdir = None
    path = args.model_path
    spec = dict(synth.CONFIGS[MODEL])
    if path is None:
        tmpdir = tempfile.mkdtemp(prefix="oi_bench_")
        path = os.path.join(tmpdir, MODEL + ".gguf")
        t = time.time()
        synth.write_gguf(path, MODEL)
        log("wrote synthetic %s (%.2f GB) in %.1fs" % (MODEL, os.path.getsize(path) / 1e9, time.time() - t))
    try:
        max_ctx = CONTEXT + max(args.steps, args.warmup) + 1
        t = time.time()
        e, _ = infer.engine_load(path, infer.Engine_Opts(max_ctx=max_ctx))
        cfg = infer.engine_config(e)
        log("engine loaded in %.1fs (seq_len %d)" % (time.time() - t, cfg.seq_len))
        if args.only == "prefill":
            print(json.dumps({"prefill": measure_prefill(e, cfg, args.prefill_tokens)}), flush=True)
            infer.engine_destroy(e)
            return
        k, v = synth.kv_prefill(4242, cfg.n_layers, cfg.n_kv_heads, CONTEXT, cfg.head_dim)
        infer.engine_kv_fill(e, 0, 0, k, v)
        log("KV pre-filled to %d" % CONTEXT)

        if args.warmup:
            infer.engine_decode_greedy(e, 0, CONTEXT, args.warmup)
        t0 = time.perf_counter()
        toks = infer.engine_decode_greedy(e, 0, CONTEXT, args.steps)  # synchronizes
        el = time.perf_counter() - t0
        tok_s = args.steps / el
        log("decode: %d steps in %.3fs -> %.1f tok/s" % (args.steps, el, tok_s))

        # the same loop with the sampler on the device (serve_harness's
        # temperature and top-p, serve.odin:1544, with a nonzero seed)
        smp = infer.Sampler(0.6, 0.95, rng_seed=42)
        infer.engine_decode_sample(e, 0, CONTEXT, min(16, args.steps), smp)  # warm, captures its graph
        t0 = time.perf_counter()
        infer.engine_decode_sample(e, 0, CONTEXT, args.steps, smp)
        el_s = time.perf_counter() - t0
        sampled = {"temperature": 0.6, "topp": 0.95, "tok_s": round(args.steps / el_s, 2),
                   "ms_per_token": round(1000 * el_s / args.steps, 4),
                   "sampler_us_per_token": round(1e6 * (el_s - el) / args.steps, 2)}
        log("sampled decode (T 0.6, top-p 0.95): %.1f tok/s, sampler %.1f us/token" % (
            sampled["tok_s"], sampled["sampler_us_per_token"]))

        # whole-step algorithmic bytes at the mean position of the timed steps
        wb = weight_bytes(spec)
        mean_pos = CONTEXT + (args.steps - 1) / 2.0
        bpt = algorithmic_bytes_per_token(cfg, wb, mean_pos)
        loop_gbps = bpt * tok_s / 1e9

        # dominant kernel, timed alone with HIP events on the engine stream
        infer.engine_forward(e, int(toks[-1]), CONTEXT + args.steps - 1)
        kern = {}
        for name in ("gateup", "qkv", "wo", "down", "attn", "output"):
            iters = cfg.n_layers * 4 if name != "output" else 8
            infer.engine_time_kernel(e, name, iters)  # warm
            us, b = infer.engine_time_kernel(e, name, iters)
            kern[name] = {"us": us, "bytes": b, "GBps": b / us / 1e3}
        if args.only == "decode":
            print(json.dumps({"decode_tok_s": round(tok_s, 2), "ms_per_step": round(1000 * el / args.steps, 4),
                              "sampled_decode": sampled, "kernels": {n: {"avg_us": round(d["us"], 3), "GBps": round(d["GBps"], 1)}
                                          for n, d in kern.items()}}), flush=True)
            infer.engine_destroy(e)
            return
        dom = "gateup"
        roofline = {
            "bound": "hbm", "kernel": "gemv_kernel gate/up Q4_K (RMSNorm prologue, SwiGLU epilogue)",
            "achieved": round(kern[dom]["GBps"], 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
            "frac": round(kern[dom]["GBps"] / PEAK_HBM_GBPS, 4), "traffic": None,
            "bytes_per_launch": kern[dom]["bytes"], "avg_launch_us": round(kern[dom]["us"], 3),
        }
        traffic_file = os.path.join(REPO, "profiles", "traffic_gateup.json")
        if os.path.exists(traffic_file):
            with open(traffic_file) as f:
                roofline["traffic"] = json.load(f).get("traffic_bytes_per_launch")

        gemm = None
        if not args.no_gemm:
            gemm = prefill_gemm(cpu=not args.no_cpu)
            log("prefill GEMM: " + ", ".join("%s %dx64x%d %.1f us %.0f TFLOP/s" % (
                g["type"], g["rows"], g["cols"], g["avg_us"], g["TFLOPs"]) for g in gemm))

        prefill = None if args.no_prefill else measure_prefill(e, cfg, args.prefill_tokens)
        dn = None if args.no_gemm else deltanet_step(cpu=not args.no_cpu)
        q35 = None if args.no_gemm else qwen35_attn_step(cpu=not args.no_cpu)
        moe = None if args.no_gemm else moe_step(cpu=not args.no_cpu)
        if dn:
            log("deltanet step: %.2f us, %.0f GB/s; qwen3.5 attention step: %.2f us, %.0f GB/s" % (
                dn["avg_us"], dn["GBps"], q35["avg_us"], q35["GBps"]))

        micro = None if args.no_microbench else gemv_microbench(cpu=not args.no_cpu)
        c4 = c5 = None
        if not args.no_models:
            c4 = model_decode("qwen3-30b-a3b-q4_k", 2048, 256, cpu=not args.no_cpu)
            c5 = model_decode("qwen35-hybrid-moe", 0, 256, prompt=2048, cpu=not args.no_cpu)
        c1 = None if args.no_cpu else c1_cpu_run()
        if c1:
            fk = c1["gpu_path_vs_f16kv_oracle"]
            log("C1: CPU %.2f tok/s (%d threads), GPU %.1f tok/s, greedy prefix %d/%d against the f32-KV oracle; "
                "GPU path through the f16-KV oracle: argmax equal at %d/%d steps (max relative margin where "
                "different %.2g)" % (c1["cpu"]["value"], c1["cpu"]["cores"], c1["gpu"]["value"],
                                     c1["greedy_matching_prefix"], c1["compared_steps"], fk["argmax_equal"],
                                     fk["steps"], fk["max_rel_margin_where_different"]))

        cpu = None
        if not args.no_cpu:
            log("CPU baseline (oracle) for up to %.0fs ..." % args.cpu_budget)
            cpu = cpu_baseline(path, k, v, cfg, list(toks), args.cpu_budget)
            log("CPU baseline: %.3f tok/s, greedy ids match: %s" % (cpu["value"], cpu["greedy_ids_match_gpu"]))
            if prefill:
                # the reference's CPU engine has no batched path: a prompt is
                # forward() token by token (qwen3_5/engine.odin:86-91)
                prefill["cpu_baseline"] = {
                    "value": round(cpu["value"], 3), "unit": "tok/s", "cores": cpu["cores"], "kind": "port",
                    "sample": "the decode sample above: the reference's CPU prefill runs forward per token"}

        out = {
            "metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(1000 * el / args.steps, 4), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "q4k/q6k x i22 dot4, f32",
            "dtype_note": "weights Q4_K/Q6_K decoded in registers; activations quantized per 32 elements to 22-bit "
                          "integers (three int8 planes) for v_dot4_i32_i8, f32 scales, sums and accumulation; "
                          "norms, RoPE, softmax and attention in f32 over an f16 KV cache",
            "data": "synthetic (seeded N(0,0.02) weights quantized Q4_K/Q6_K; N(0,1) f16 KV prefill)",
            "config": {"workload": "Qwen3-8B-shape dense decode, bs1, greedy, f16 KV pre-filled to 4096, "
                                   "%d steps from pos 4096" % args.steps,
                       "hidden": cfg.dim, "layers": cfg.n_layers, "heads": "%d/%d" % (cfg.n_heads, cfg.n_kv_heads),
                       "ffn": cfg.hidden_dim, "vocab": cfg.vocab_size, "weights": "Q4_K + Q6_K(attn_v, output)",
                       "kv_cache": "f16", "parallelism": "single GPU"},
            "roofline": roofline,
            "token_loop": {"bytes_per_token": int(bpt), "achieved_GBps": round(loop_gbps, 1),
                           "frac_of_peak": round(loop_gbps / PEAK_HBM_GBPS, 4),
                           "roofline_tok_s": round(PEAK_HBM_GBPS * 1e9 / bpt, 1)},
            "kernels": {n: {"avg_us": round(d["us"], 3), "GBps": round(d["GBps"], 1)} for n, d in kern.items()},
            "sampled_decode": sampled,
            "cpu_baseline": cpu,
            "prefill_gemm": gemm,
            "prefill": prefill,
            "deltanet_step": dn,
            "qwen35_attn_step": q35,
            "moe_step": moe,
            "gemv_microbench": micro,
            "c1": c1,
            "c4_moe_decode": c4,
            "c5_hybrid": c5,
        }
        print(json.dumps(out), flush=True)
        infer.engine_destroy(e)
    finally:
        if tmpdir:
            shutil.rmtree(tmpdir, ignore_errors=True)


if __name__ == "__main__":
    main()
