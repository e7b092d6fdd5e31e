#!/usr/bin/env python3
"""bench.py -- Q4_0 decode-GEMV throughput on one MI355X.

A "step" is one pass of the Llama-3-8B per-layer decode GEMV set at batch 1
(Wq 4096x4096, Wk/Wv 1024x4096, Wo 4096x4096, W_gate/W_up 14336x4096,
W_down 4096x14336; Q4_0 weights, fp32 activations ~ N(0,1)), executed as the
decode step runs it: Q|K|V as one launch, W_gate|W_up as one, Wo and W_down
alone, each straight from its fp32 input (the digit planes of x are made
inside the GEMV launch).
The K timed steps run as one captured HIP graph (4K launches, as a decode
step runs its layers back to back), step i using weight set i % LAYERS of
LAYERS distinct sets (4 x 136.6 MB), so the 256 MB MALL cannot serve
repeats.  Inputs are resident in HBM when the timed region starts.

value  = algorithmic bytes of the K timed steps / wall time of those steps,
         algorithmic bytes per step = sum over the 7 matrices of
         (weights + 4*N + 4*M) = 136,642,560 B.
roofline = the dominant kernel (the fused W_gate|W_up GEMV launch), timed
         with HIP events on its stream around a graph of K back-to-back
         launches: achieved = its algorithmic bytes / (elapsed / K), vs
         8 TB/s.  The same K-launch graph times each of the four launches
         for the "kernels" breakdown; each launch shape rotates >= 300 MB of
         distinct weight copies (so the 256 MB MALL serves no repeat), and
         each line carries the time of a device-to-device copy of the same
         bytes (its "copy floor", which moves twice the bytes: read + write).
config1 = BASELINE config 1, one 4096x4096 GEMV from fp32 x, timed the same
         way over 32 rotated copies.
cpu_baseline = the reference's own q_gemv_q4_f32_avx2 (compiled from its
         sources into oracle/_ref) running the same 7-matrix set on one
         pinned host core of this machine, for a bounded sample.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--cpu-seconds S]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "project-ia_amd"))
sys.path.insert(0, str(REPO))

METRIC = "Q4_0 GEMV HBM GB/s (% peak) + decode tok/s, Llama-3-8B shape, 1 GPU"
HBM_PEAK_GBS = 8000.0
DIM, KV, HID = 4096, 1024, 14336
SHAPES = [("wq", DIM, DIM), ("wk", KV, DIM), ("wv", KV, DIM), ("wo", DIM, DIM),
          ("w_gate", HID, DIM), ("w_up", HID, DIM), ("w_down", DIM, HID)]
LAYERS = 4
ROT_BYTES = 300 << 20  # distinct weight bytes each timed launch shape rotates over


def alg_bytes(M, N):
    return M * (N // 32) * 20 + 4 * N + 4 * M


STEP_BYTES = sum(alg_bytes(M, N) for _, M, N in SHAPES)
GATE_UP_BYTES = alg_bytes(HID, DIM) * 2
assert STEP_BYTES == 136_642_560


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class LayerSet:
    """Device-resident weights of one layer + tensor views."""

    def __init__(self, qa, mats):
        self.bufs = {k: qa.DeviceBuffer.from_numpy(w) for k, w in mats.items()}
        self.t = {k: qa.q4_tensor(self.bufs[k].ptr, M, N) for k, M, N in SHAPES}


def gen_layer(seed):
    from qorus_amd import synthetic as syn
    rng = syn.rng_for(seed)
    return {k: syn.gen_q4(M, N, rng) for k, M, N in SHAPES}


def ptr_array(ptrs, ctype=C.c_void_p):
    return (ctype * len(ptrs))(*ptrs)


def run_gpu(args):
    import qorus_amd as qa
    from qorus_amd import synthetic as syn
    lib = qa.lib()
    if not qa.gpu_available():
        raise SystemExit("bench.py: no usable GPU (" + lib.qh_last_error().decode() + ")")
    log(f"[bench] device {lib.qh_arch_name().decode()}; generating {LAYERS} layers "
        f"({LAYERS * STEP_BYTES / 1e6:.0f} MB)")
    layers = [LayerSet(qa, gen_layer(1000 + l)) for l in range(LAYERS)]
    rng = syn.rng_for(77)
    xin = {k: qa.DeviceBuffer.from_numpy(syn.gen_f32(n, rng)) for k, n in
           (("h", DIM), ("o", DIM), ("h2", DIM), ("m", HID))}
    outs = {k: qa.DeviceBuffer(M * 4) for k, M, _ in SHAPES}
    ws = {k: qa.DeviceBuffer(lib.qh_gemv_workspace_bytes(n)) for k, n in
          (("h", DIM), ("o", DIM), ("h2", DIM), ("m", HID))}
    stream = qa.Stream()
    s = stream.handle

    def gemv_group(L, xk, mats):
        """One launch: ys = Ws . x straight from the fp32 x (digit planes
        made inside the GEMV)."""
        Ws = ptr_array([L.t[m].addr for m in mats])
        ys = ptr_array([outs[m].ptr for m in mats])
        qa.check(lib.qh_gemv_q4_f32_multi(Ws, None, ys, len(mats), xin[xk].ptr, ws[xk].ptr, s), "gemv")

    groups = [("qkv", "h", ["wq", "wk", "wv"]), ("wo", "o", ["wo"]), ("gate_up", "h2", ["w_gate", "w_up"]),
              ("down", "m", ["w_down"])]

    def enqueue_step(L):
        """The 4 GEMV launches of one layer pass."""
        for _, xk, mats in groups:
            gemv_group(L, xk, mats)

    def capture(n_steps):
        """One graph of n_steps consecutive steps (weight set i % LAYERS),
        as a decode step runs its layers back to back in one graph."""
        qa.check(lib.qh_stream_begin_capture(s), "begin_capture")
        for i in range(n_steps):
            enqueue_step(layers[i % LAYERS])
        g = C.c_void_p()
        qa.check(lib.qh_stream_end_capture(s, C.byref(g)), "end_capture")
        return g.value

    warm, timed = capture(args.warmup), capture(args.steps)
    qa.check(lib.qh_graph_launch(warm, s))
    stream.sync()

    # ---- timed region: exactly K steps, synchronized on both sides ----
    qa.check(lib.qh_device_synchronize())
    t0 = time.perf_counter()
    qa.check(lib.qh_graph_launch(timed, s))
    stream.sync()
    qa.check(lib.qh_device_synchronize())
    t1 = time.perf_counter()
    wall = t1 - t0
    graphs = [warm, timed]

    # ---- per-launch kernel time: K launches of one GEMV group captured back
    # to back in one graph, HIP events on the stream around its replay;
    # mean = elapsed / K.  Inside a graph the launches follow each other with
    # no dispatch gap, so this is the kernel's own duration (what rocprofv3
    # --kernel-trace reports).  Each launch shape rotates at least ROT_BYTES
    # of distinct weight copies (device copies of the layer sets), so the
    # 256 MB MALL cannot serve a repeat.
    kbytes = {"qkv": sum(alg_bytes(M, N) for k, M, N in SHAPES if k in ("wq", "wk", "wv")),
              "wo": alg_bytes(DIM, DIM), "gate_up": GATE_UP_BYTES, "down": alg_bytes(DIM, HID)}
    extra = []  # keeps the copies alive

    def rotated(mats, min_sets=0):
        """Tensor sets of `mats` totalling >= ROT_BYTES (and at least
        min_sets of them): the LAYERS generated sets, then device copies."""
        sets = [{m: L.t[m] for m in mats} for L in layers]
        wbytes = sum(M * (N // 32) * 20 for k, M, N in SHAPES if k in mats)
        i = 0
        while len(sets) * wbytes < ROT_BYTES or len(sets) < min_sets:
            src = layers[i % LAYERS]
            cp = {}
            for m in mats:
                M, N = next((M, N) for k, M, N in SHAPES if k == m)
                b = qa.DeviceBuffer(M * (N // 32) * 20)
                qa.check(lib.qh_memcpy_dtod(b.ptr, src.bufs[m].ptr, b.nbytes, s), "copy")
                extra.append(b)
                cp[m] = qa.q4_tensor(b.ptr, M, N)
            sets.append(cp)
            i += 1
        stream.sync()
        return sets

    def time_graph(enqueue, n):
        qa.check(lib.qh_stream_begin_capture(s), "begin_capture")
        for i in range(n):
            enqueue(i)
        g = C.c_void_p()
        qa.check(lib.qh_stream_end_capture(s, C.byref(g)), "end_capture")
        qa.check(lib.qh_graph_launch(g.value, s))  # warm
        e0, e1 = qa.Event(), qa.Event()
        e0.record(stream)
        qa.check(lib.qh_graph_launch(g.value, s))
        e1.record(stream)
        stream.sync()
        lib.qh_graph_destroy(g.value)
        return e0.elapsed_ms(e1) / n

    def time_group(xk, mats, sets):
        def enq(i):
            st = sets[i % len(sets)]
            Ws = ptr_array([st[m].addr for m in mats])
            ys = ptr_array([outs[m].ptr for m in mats])
            qa.check(lib.qh_gemv_q4_f32_multi(Ws, None, ys, len(mats), xin[xk].ptr, ws[xk].ptr, s), "gemv")
        return time_graph(enq, max(args.steps, 2 * len(sets)))

    # The copy floor of a launch: a device-to-device copy of the launch's
    # algorithmic bytes, from a rotated source region into a rotated
    # destination region (each >= ROT_BYTES of distinct addresses), timed
    # the same way.  It moves twice the bytes the GEMV reads (read + write),
    # so copy_us / us > 1 means the GEMV streams its bytes faster than a
    # copy of them completes.
    pool_bytes = ROT_BYTES + (80 << 20)
    src_pool, dst_pool = qa.DeviceBuffer(pool_bytes), qa.DeviceBuffer(pool_bytes)

    def time_copy(nbytes):
        nbytes = (nbytes + 255) & ~255
        slots = max(2, pool_bytes // nbytes)

        def enq(i):
            off = (i % slots) * nbytes
            qa.check(lib.qh_memcpy_dtod(dst_pool.ptr + off, src_pool.ptr + off, nbytes, s), "copy")
        return time_graph(enq, max(args.steps, 2 * slots))

    breakdown = {}
    per_kernel = {}
    for name, xk, mats in groups:
        sets = rotated(mats)
        ms = time_group(xk, mats, sets)
        per_kernel[name] = ms
        us = ms * 1e3
        cus = time_copy(kbytes[name]) * 1e3
        gbs = kbytes[name] / (us * 1e-6) / 1e9
        breakdown[name] = {"us": round(us, 2), "GB_s": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                           "copies_rotated": len(sets), "rotated_MB": round(len(sets) * kbytes[name] / 1e6),
                           "copy_floor_us": round(cus, 2), "frac_of_copy_floor": round(cus / us, 3)}
        log(f"[bench] {name}: {us:.2f} us ({gbs:.0f} GB/s, {len(sets)} copies); copy of the same bytes {cus:.2f} us")
    mean_ms = per_kernel["gate_up"]
    for g in graphs:
        lib.qh_graph_destroy(g)
    achieved = GATE_UP_BYTES / (mean_ms * 1e-3) / 1e9
    # one 4096 x 4096 GEMV from fp32 x (the Wo shape as a
    # standalone launch), >= 32 rotated copies.
    c1_sets = rotated(["wo"], min_sets=32)
    c1_ms = time_group("o", ["wo"], c1_sets)
    c1_bytes = alg_bytes(DIM, DIM)
    c1_gbs = c1_bytes / (c1_ms * 1e-3) / 1e9
    config1 = {"workload": "config1: one Q4_0 GEMV 4096x4096 from fp32 x ~ N(0,1) (digit planes made in the launch)",
               "us": round(c1_ms * 1e3, 2), "alg_bytes": c1_bytes, "GB_s": round(c1_gbs, 1),
               "frac_hbm_peak": round(c1_gbs / HBM_PEAK_GBS, 4), "copies_rotated": len(c1_sets),
               "copy_floor_us": breakdown["wo"]["copy_floor_us"],
               "frac_of_copy_floor": round(breakdown["wo"]["copy_floor_us"] / (c1_ms * 1e3), 3)}
    log(f"[bench] config1: {c1_ms * 1e3:.2f} us ({c1_gbs:.0f} GB/s, {len(c1_sets)} copies)")
    return wall, achieved, mean_ms, breakdown, config1


def run_cpu_baseline(seconds):
    """Reference q_gemv_q4_f32_avx2 (oracle/_ref) on one pinned core."""
    from oracle import oracle as orc
    kind = "reference" if orc.ref_available() else "port"
    mats = gen_layer(1000)
    rng = orc.rng_for(78)
    xs = {DIM: orc.aligned_copy(orc.gen_f32(DIM, rng)), HID: orc.aligned_copy(orc.gen_f32(HID, rng))}
    ys = {k: orc.aligned_empty((M,), np.float32) for k, M, _ in SHAPES}
    Wa = {k: orc.aligned_copy(mats[k].reshape(-1)) for k, _, _ in SHAPES}
    tens = {k: orc.q4_tensor(Wa[k].ctypes.data, M, N) for k, M, N in SHAPES}
    if kind == "reference":
        fn = orc.ref().q_gemv_q4_f32_avx2

        def one_pass():
            for k, M, N in SHAPES:
                rc = fn(C.addressof(tens[k][0]), xs[N].ctypes.data, ys[k].ctypes.data)
                assert rc == 0
    else:
        L = orc.lib()

        def one_pass():
            for k, M, N in SHAPES:
                L.or_gemv_q4(Wa[k], M, N, xs[N], ys[k])
    try:
        old = os.sched_getaffinity(0)
        core = min(old)
        os.sched_setaffinity(0, {core})
    except (AttributeError, OSError):
        old = None
    try:
        one_pass()  # warm-up
        n = 0
        t0 = time.perf_counter()
        while True:
            one_pass()
            n += 1
            el = time.perf_counter() - t0
            if el >= seconds or n >= 1000:
                break
    finally:
        if old is not None:
            os.sched_setaffinity(0, old)
    gbs = n * STEP_BYTES / el / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": 1, "kind": kind,
            "sample": f"{n} passes of the config-2 per-layer Q4_0 GEMV set ({STEP_BYTES / 1e6:.1f} MB/pass) "
                      f"in {el:.1f} s on 1 pinned core ({orc.cpu_model_name()})"}


# ---------------------------------------------------------------------------
# Decode step
# ---------------------------------------------------------------------------
DEC = dict(vocab=128256, dim=4096, hidden=14336, n_layers=32, n_heads=32, n_kv=8)
DEC_POS = 2047


def decode_bytes_per_token(n_layers=32, ctx=2048):
    """Algorithmic HBM bytes of one decode step: every weight byte once
    (32 layers + Q4_0 LM head + the fp32 embedding row and norm weights) and
    the fp32 K and V rows of `ctx` cached positions."""
    d, hid, v, kvd = 4096, 14336, 128256, 1024
    q4 = lambda r, c: r * (c // 32) * 20
    layer = q4(d, d) * 2 + q4(kvd, d) * 2 + q4(hid, d) * 2 + q4(d, hid) + 2 * d * 4
    kv = n_layers * 8 * ctx * 2 * 128 * 4
    return n_layers * layer + q4(v, d) + d * 4 + d * 4 + kv


def scratch_dir(need_bytes):
    import shutil
    import tempfile
    for base in ("/dev/shm", None):
        try:
            d = tempfile.mkdtemp(prefix="qorus_bench_", dir=base)
            if shutil.disk_usage(d).free > need_bytes * 1.2:
                return d
            shutil.rmtree(d, ignore_errors=True)
        except OSError:
            continue
    raise SystemExit("bench.py: no scratch space for the synthetic model")


def graph_node_floor_us(n_nodes=200):
    """Replay time per node of a captured graph of n_nodes back-to-back
    one-workgroup launches (qh_add_f32 over 64 floats, each reading the
    previous one's output): the fixed cost every node of a decode graph
    pays, whatever its work."""
    import qorus_amd as qa
    lib = qa.lib()
    a = qa.DeviceBuffer.from_numpy(np.ones(64, np.float32))
    b = qa.DeviceBuffer.from_numpy(np.zeros(64, np.float32))
    stream = qa.Stream()
    s = stream.handle
    qa.check(lib.qh_stream_begin_capture(s), "begin_capture")
    for i in range(n_nodes):
        src, dst = (a, b) if i % 2 == 0 else (b, a)
        qa.check(lib.qh_add_f32(src.ptr, src.ptr, dst.ptr, 64, s), "add")
    g = C.c_void_p()
    qa.check(lib.qh_stream_end_capture(s, C.byref(g)), "end_capture")
    qa.check(lib.qh_graph_launch(g.value, s))  # warm
    best = None
    for _ in range(3):
        e0, e1 = qa.Event(), qa.Event()
        e0.record(stream)
        qa.check(lib.qh_graph_launch(g.value, s))
        e1.record(stream)
        stream.sync()
        ms = e0.elapsed_ms(e1)
        best = ms if best is None else min(best, ms)
    lib.qh_graph_destroy(g.value)
    return round(best * 1e3 / n_nodes, 3)


def run_decode(args):
    import shutil
    import qorus_amd as qa
    from qorus_amd import synthetic as syn
    steps = args.decode_steps
    max_seq = DEC_POS + 1 + args.decode_warmup + steps + 8
    h = qa.QorusHeader(max_seq=max_seq, **DEC)
    size = qa.model_layout(h)["_size"]
    d = scratch_dir(size)
    path = Path(d) / "llama3_8b_q4_0.qorus"
    try:
        t0 = time.perf_counter()
        syn.write_synthetic_model(path, h, seed=2024)
        log(f"[bench] decode: wrote {size / 1e9:.2f} GB synthetic model in {time.perf_counter() - t0:.1f} s")
        m = qa.Model(path)
        hd = 128
        rng = syn.rng_for(2025)
        kv = np.zeros((h.n_layers, h.n_kv, max_seq, 2, hd), np.float32)
        kv[:, :, :DEC_POS] = rng.standard_normal((h.n_layers, h.n_kv, DEC_POS, 2, hd), dtype=np.float32)
        m.upload_kv(kv)
        first_tok = 1
        # warm-up (captures the graph), then the timed greedy decode from pos 2047
        m.generate(first_tok, DEC_POS, args.decode_warmup)
        m.upload_kv(kv)
        toks, ms = m.generate(first_tok, DEC_POS, steps)
        # the same decode with each token sampled on the device
        # (temperature 0.8, top-k 40, top-p 0.95)
        ms_s = None
        if not args.no_sampled_decode:
            m.upload_kv(kv)
            m.generate_sampled(first_tok, DEC_POS, args.decode_warmup, 0.8, 40, 0.95)
            m.upload_kv(kv)
            _, ms_s = m.generate_sampled(first_tok, DEC_POS, steps, 0.8, 40, 0.95)
        prefills = [] if args.no_prompt else [run_prompt(m, h, T) for T in args.prompt_tokens]
        m.close()
        avg_ctx = DEC_POS + 1 + (steps - 1) / 2
        bpt = decode_bytes_per_token(ctx=int(round(avg_ctx)))
        out = {"tok_s": round(1e3 / ms, 1), "ms_per_token": round(ms, 4), "steps": steps,
               "warmup": args.decode_warmup,
               "workload": "config4: 32-layer Llama-3-8B shape, Q4_0 weights + Q4_0 LM head, fp32 KV pre-filled "
                           "N(0,1) to pos 2047, greedy decode from pos 2047 (context 2048..%d), hipGraph per step"
                           % (DEC_POS + steps),
               "hbm_bytes_per_token": bpt,
               "achieved_GB_s": round(bpt / (ms * 1e-3) / 1e9, 1),
               "frac_of_hbm_peak": round(bpt / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
               "roofline_tok_s_at_peak": round(HBM_PEAK_GBS * 1e9 / bpt, 1),
               "sampled_tok_s": None if ms_s is None else round(1e3 / ms_s, 1),
               "sampled_workload": "same steps, each token drawn on the device by q_sample_token's pipeline "
                                   "(temperature 0.8, top-k 40, top-p 0.95); only the tokens leave the GPU"}
        out["graph_node_floor_us"] = graph_node_floor_us()
        out["graph_node_floor_workload"] = ("replay time per node of a captured graph of 200 back-to-back "
                                            "one-workgroup qh_add_f32 launches: the fixed cost of every node "
                                            "of the decode graph (7 per layer, 3 per token besides)")
        for pf in prefills:
            out["prefill_%d" % pf["tokens"]] = pf
        if not args.no_cpu:
            out["cpu_baseline"], out["first_token_matches_cpu"] = run_cpu_decode(path, kv, first_tok, int(toks[0]),
                                                                                args.cpu_decode_tokens)
        return out
    finally:
        shutil.rmtree(d, ignore_errors=True)


PROMPT_T = 512
PROMPT_TS = (512, 2048)  # prompts the decode leg times by default


def prompt_flop(n_layers=32, T=PROMPT_T):
    """Useful flops of a T-token prompt through llama_forward: 2*T per weight
    of the 32 layers (Q|K|V, Wo, W_gate|W_up, W_down) plus the causal
    attention (q.k and p.v over keys 0..t of each query, 32 heads x 128) and
    the LM head of the last token."""
    d, hid, v, kvd = 4096, 14336, 128256, 1024
    w = d * d * 2 + 2 * kvd * d + 3 * hid * d
    attn = 2 * 2 * 32 * 128 * (T * (T + 1) // 2)
    return n_layers * (2 * T * w + attn) + 2 * v * d


def run_prompt(m, h, T=PROMPT_T, reps=3):
    """llama_forward of a T-token prompt (512 by default) at position 0 on
    the 32-layer model (the batched prefill, in chunks of up to 2048 tokens),
    wall clock around the synchronous call."""
    if T < 1 or T > h.max_seq:
        raise SystemExit(f"bench.py: --prompt-tokens must be 1..{h.max_seq}")
    rng = np.random.default_rng(2026)
    toks = [int(t) for t in rng.integers(0, h.vocab, T)]
    m.forward(toks, 0)  # first call allocates the prefill buffers
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        m.forward(toks, 0)
        times.append(time.perf_counter() - t0)
    ms = 1e3 * sum(times) / len(times)
    fl = prompt_flop(T=T)
    log(f"[bench] prompt: {T} tokens in {ms:.2f} ms ({T / ms * 1e3:.0f} tok/s)")
    return {"tokens": T, "ms": round(ms, 3), "tok_s": round(T / ms * 1e3, 1), "reps": reps,
            "useful_tflop_s": round(fl / (ms * 1e-3) / 1e12, 1),
            "frac_of_fp16_mfma_peak": round(fl / (ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
            "workload": "llama_forward(%d tokens, pos 0) on the config-4 model (32 layers, Llama-3-8B shape, "
                        "Q4_0; chunks of up to 2048 tokens): every projection an MFMA GEMM, causal attention with "
                        "q.k and P.V on fp16 hi/lo MFMA, KV rows 0..%d "
                        "written, LM head of the last token; wall clock of the synchronous call incl. the "
                        "token upload and the 513 KB logits download" % (T, T - 1)}


def run_cpu_decode(path, kv, first_tok, gpu_tok0, n_tokens):
    """The oracle's corrected decode step (or_decode_step), one pinned core."""
    from oracle import oracle as orc
    blob = np.memmap(path, dtype=np.uint8, mode="r")
    ref = orc.DecodeOracle(blob, kv.copy())
    try:
        old = os.sched_getaffinity(0)
        os.sched_setaffinity(0, {min(old)})
    except (AttributeError, OSError):
        old = None
    try:
        t = first_tok
        t0 = time.perf_counter()
        toks = []
        for i in range(n_tokens):
            t, _ = ref.step(t, DEC_POS + i)
            toks.append(t)
        el = time.perf_counter() - t0
    finally:
        if old is not None:
            os.sched_setaffinity(0, old)
    cpu = {"value": round(n_tokens / el, 4), "unit": "tok/s", "cores": 1, "kind": "port",
           "sample": f"{n_tokens} greedy decode steps of the 32-layer model from pos 2047 with the oracle's "
                     f"C restatement (or_decode_step; the reference's own forward cannot run at these shapes) "
                     f"in {el:.1f} s on 1 pinned core ({orc.cpu_model_name()})"}
    return cpu, bool(toks[0] == gpu_tok0)


# ---------------------------------------------------------------------------
# LM head + softmax + argmax
# ---------------------------------------------------------------------------
VOCAB = 128256
LM_COPIES = 2  # 2 x 328 MB: more than the 256 MB MALL holds


def lmhead_bytes():
    """Algorithmic HBM bytes of one config-3 step: the Q4_0 LM head once,
    x, the logits written and read back by softmax and argmax, the
    probabilities written."""
    return alg_bytes(VOCAB, DIM) + 3 * 4 * VOCAB


def run_lmhead(args):
    import qorus_amd as qa
    from qorus_amd import synthetic as syn
    lib = qa.lib()
    rng = syn.rng_for(4242)
    Ws = [qa.DeviceBuffer.from_numpy(syn.gen_q4(VOCAB, DIM, rng)) for _ in range(LM_COPIES)]
    ts = [qa.q4_tensor(w.ptr, VOCAB, DIM) for w in Ws]
    x = qa.DeviceBuffer.from_numpy(syn.gen_f32(DIM, rng))
    ws = qa.DeviceBuffer(lib.qh_gemv_workspace_bytes(DIM))
    logits, probs = qa.DeviceBuffer(VOCAB * 4), qa.DeviceBuffer(VOCAB * 4)
    tok = qa.DeviceBuffer(4)
    stream = qa.Stream()
    s = stream.handle
    ys = ptr_array([logits.ptr])

    def gemv(t):
        qa.check(lib.qh_gemv_q4_f32_multi(ptr_array([t.addr]), None, ys, 1, x.ptr, ws.ptr, s))

    fws = qa.DeviceBuffer(lib.qh_gemv_softmax_workspace_bytes(VOCAB))

    def step(t):
        """LM head + softmax of the logits + their greedy argmax (results:
        q_gemv_q4_f32_avx2, q_softmax_f32_avx2 and main.c:870-881); the
        GEMV leaves the argmax's per-workgroup partials, then the softmax's
        exp and normalize passes (3 launches)."""
        qa.check(lib.qh_gemv_q4_f32_softmax_argmax(t.addr, x.ptr, logits.ptr, probs.ptr, tok.ptr, fws.ptr, s))

    def capture(n):
        """One graph of n consecutive steps (weight copy i % LM_COPIES), as
        the config-2 leg runs its steps."""
        qa.check(lib.qh_stream_begin_capture(s))
        for i in range(n):
            step(ts[i % LM_COPIES])
        g = C.c_void_p()
        qa.check(lib.qh_stream_end_capture(s, C.byref(g)))
        return g.value

    steps = max(10, args.steps // 4)
    graphs = [capture(8), capture(steps)]
    qa.check(lib.qh_graph_launch(graphs[0], s))
    stream.sync()
    qa.check(lib.qh_device_synchronize())
    t0 = time.perf_counter()
    qa.check(lib.qh_graph_launch(graphs[1], s))
    stream.sync()
    qa.check(lib.qh_device_synchronize())
    wall = time.perf_counter() - t0
    # correctness spot check: the device argmax is the host argmax
    lg = logits.download(np.float32, (VOCAB,))
    tk = int(tok.download(np.uint32, (1,))[0])
    ok = tk == int(np.argmax(lg))
    # stage timings with events (eager launches on the same stream): the
    # whole step, and the plain GEMV launch alone for comparison
    stages = {"gemv": [], "step": []}
    for i in range(16):
        for name, fn in (("gemv", lambda: gemv(ts[i % LM_COPIES])), ("step", lambda: step(ts[i % LM_COPIES]))):
            a, b = qa.Event(), qa.Event()
            a.record(stream)
            fn()
            b.record(stream)
            stream.sync()
            stages[name].append(a.elapsed_ms(b))
    for g in graphs:
        lib.qh_graph_destroy(g)
    ms = wall / steps * 1e3
    nbytes = lmhead_bytes()
    cpu = None if args.no_cpu else run_cpu_lmhead()
    return {"workload": "config3: LM head 128256x4096 Q4_0 GEMV + softmax over 128256 logits + argmax "
                        "(qh_gemv_q4_f32_softmax_argmax: 3 launches), one hipGraph of all timed steps, "
                        "2 rotated weight copies",
            "ms_per_step": round(ms, 5), "steps": steps, "alg_bytes": nbytes,
            "GB_s": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "frac_of_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "stage_us": {k: round(float(np.median(v)) * 1e3, 2) for k, v in stages.items()},
            "argmax_matches_host": ok, "cpu_baseline": cpu}


def run_cpu_lmhead(n_steps=3):
    """Config 3 on one pinned host core: the reference's own
    q_gemv_q4_f32_avx2 and q_softmax_f32_avx2 (oracle/_ref) plus the
    oracle's argmax, n_steps times on one synthetic LM head."""
    from oracle import oracle as orc
    if not orc.ref_available():
        return None
    from qorus_amd import synthetic as syn
    R = orc.ref()
    rng = syn.rng_for(4243)
    W = orc.aligned_copy(syn.gen_q4(VOCAB, DIM, rng).reshape(-1))
    x = orc.aligned_copy(syn.gen_f32(DIM, rng))
    lg = orc.aligned_empty((VOCAB,), np.float32)
    pr = orc.aligned_empty((VOCAB,), np.float32)
    t = orc.q4_tensor(W.ctypes.data, VOCAB, DIM)
    try:
        old = os.sched_getaffinity(0)
        os.sched_setaffinity(0, {min(old)})
    except (AttributeError, OSError):
        old = None
    try:
        def step():
            assert R.q_gemv_q4_f32_avx2(C.addressof(t[0]), x.ctypes.data, lg.ctypes.data) == 0
            assert R.q_softmax_f32_avx2(lg.ctypes.data, pr.ctypes.data, VOCAB) == 0
            orc.argmax(lg)
        step()
        t0 = time.perf_counter()
        for _ in range(n_steps):
            step()
        el = time.perf_counter() - t0
    finally:
        if old is not None:
            os.sched_setaffinity(0, old)
    return {"value": round(n_steps / el, 3), "unit": "steps/s", "ms_per_step": round(el / n_steps * 1e3, 2),
            "cores": 1, "kind": "reference",
            "sample": f"{n_steps} steps of the reference's q_gemv_q4_f32_avx2 (128256x4096) + q_softmax_f32_avx2 "
                      f"+ argmax on 1 pinned core ({orc.cpu_model_name()})"}


# ---------------------------------------------------------------------------
# Config 5: batched prefill GEMM on MFMA
# ---------------------------------------------------------------------------
PREFILL_T = 512
PREFILL_COPIES = 3
MFMA_F16_PEAK_TFLOPS = 2500.0
PREFILL_FLOP = 3 * 2 * PREFILL_T * HID * DIM  # useful flops of one step


def run_prefill(args):
    """Config 5: X [512 x 4096] fp32 against W_gate|W_up [14336 x 4096] (one
    qh_gemm_q4_f32_multi launch), then H [512 x 14336] against W_down
    [4096 x 14336] (qh_gemm_q4_f32): the prefill projections of one MLP, as
    the reference runs them one token row at a time (model.c:1485-1561).
    The timed steps run as one captured graph, step i using weight copy
    i % PREFILL_COPIES (330 MB, past the MALL); inputs resident in HBM."""
    import qorus_amd as qa
    from qorus_amd import synthetic as syn
    lib = qa.lib()
    rng = syn.rng_for(5555)
    T = PREFILL_T
    sets = []
    for _ in range(PREFILL_COPIES):
        bufs = [qa.DeviceBuffer.from_numpy(syn.gen_q4(M, N, rng)) for M, N in ((HID, DIM), (HID, DIM), (DIM, HID))]
        ts = [qa.q4_tensor(b.ptr, M, N) for b, (M, N) in zip(bufs, ((HID, DIM), (HID, DIM), (DIM, HID)))]
        sets.append((bufs, ts))
    X = qa.DeviceBuffer.from_numpy(rng.standard_normal((T, DIM), dtype=np.float32))
    H = qa.DeviceBuffer.from_numpy(rng.standard_normal((T, HID), dtype=np.float32))
    G, U, Y = qa.DeviceBuffer(T * HID * 4), qa.DeviceBuffer(T * HID * 4), qa.DeviceBuffer(T * DIM * 4)
    ws_gu = qa.DeviceBuffer(lib.qh_gemm_workspace_bytes(DIM, T, 2 * HID))
    ws_d = qa.DeviceBuffer(lib.qh_gemm_workspace_bytes(HID, T, DIM))
    stream = qa.Stream()
    s = stream.handle
    ys = ptr_array([G.ptr, U.ptr])

    def gate_up(i):
        ts = sets[i % PREFILL_COPIES][1]
        qa.check(lib.qh_gemm_q4_f32_multi(ptr_array([ts[0].addr, ts[1].addr]), ys, 2, X.ptr, T, ws_gu.ptr, s))

    def down(i):
        ts = sets[i % PREFILL_COPIES][1]
        qa.check(lib.qh_gemm_q4_f32(ts[2].addr, H.ptr, T, Y.ptr, ws_d.ptr, s))

    def capture(fns, n):
        qa.check(lib.qh_stream_begin_capture(s))
        for i in range(n):
            for f in fns:
                f(i)
        g = C.c_void_p()
        qa.check(lib.qh_stream_end_capture(s, C.byref(g)))
        return g.value

    steps = max(6, args.steps // 20)
    warm = capture([gate_up, down], 3)
    qa.check(lib.qh_graph_launch(warm, s))
    stream.sync()

    def time_graph(fns):
        g = capture(fns, steps)
        a, b = qa.Event(), qa.Event()
        a.record(stream)
        qa.check(lib.qh_graph_launch(g, s))
        b.record(stream)
        stream.sync()
        lib.qh_graph_destroy(g)
        return a.elapsed_ms(b) / steps

    qa.check(lib.qh_device_synchronize())
    t0 = time.perf_counter()
    ms_step = time_graph([gate_up, down])
    wall = time.perf_counter() - t0
    ms_gu = time_graph([gate_up])
    ms_d = time_graph([down])
    lib.qh_graph_destroy(warm)
    tflops = PREFILL_FLOP / (ms_step * 1e-3) / 1e12
    cpu = None if args.no_cpu else run_cpu_prefill()
    return {"workload": "config5: 512-token prefill GEMM, X 512x4096 vs W_gate|W_up 14336x4096 (one launch) then "
                        "512x14336 vs W_down 4096x14336; one hipGraph of all timed steps, 3 rotated weight copies",
            "dtype": "q4_0 x f32 on fp16 MFMA (exact q-8 operand, x as fp16 hi + fp16 lo (x - hi), fp32 accumulate)",
            "ms_per_step": round(ms_step, 4), "steps": steps, "tokens_per_s": round(T / (ms_step * 1e-3), 1),
            "useful_flop_per_step": PREFILL_FLOP, "TFLOP_s": round(tflops, 1),
            "mfma_util": round(tflops / MFMA_F16_PEAK_TFLOPS, 4), "peak_TFLOP_s": MFMA_F16_PEAK_TFLOPS,
            # each useful product takes two MFMA products (x's fp16 hi and lo parts against the
            # same exact weight operand), so the matrix cores run at twice the useful rate
            "mfma_issue_util": round(2 * tflops / MFMA_F16_PEAK_TFLOPS, 4),
            "launch_us": {"gate_up": round(ms_gu * 1e3, 1), "down": round(ms_d * 1e3, 1)},
            "wall_s": round(wall, 3), "cpu_baseline": cpu}


def run_cpu_prefill(rows=12):
    """Config 5 on one pinned host core as the reference runs it: one
    q_gemv_q4_f32_avx2 (oracle/_ref) per token row and matrix; a bounded
    sample of `rows` token rows of each of the three matrices, reported as
    prefill tokens per second."""
    from oracle import oracle as orc
    if not orc.ref_available():
        return None
    from qorus_amd import synthetic as syn
    R = orc.ref()
    rng = syn.rng_for(5556)
    mats = []
    for M, N in ((HID, DIM), (HID, DIM), (DIM, HID)):
        W = orc.aligned_copy(syn.gen_q4(M, N, rng).reshape(-1))
        mats.append((W, orc.q4_tensor(W.ctypes.data, M, N), N, orc.aligned_empty((M,), np.float32)))
    xs = {N: orc.aligned_copy(syn.gen_f32(N, rng)) for N in (DIM, HID)}
    try:
        old = os.sched_getaffinity(0)
        os.sched_setaffinity(0, {min(old)})
    except (AttributeError, OSError):
        old = None
    try:
        for W, t, N, y in mats:
            assert R.q_gemv_q4_f32_avx2(C.addressof(t[0]), xs[N].ctypes.data, y.ctypes.data) == 0
        t0 = time.perf_counter()
        for _ in range(rows):
            for W, t, N, y in mats:
                R.q_gemv_q4_f32_avx2(C.addressof(t[0]), xs[N].ctypes.data, y.ctypes.data)
        el = time.perf_counter() - t0
    finally:
        if old is not None:
            os.sched_setaffinity(0, old)
    return {"value": round(rows / el, 3), "unit": "prefill tokens/s", "cores": 1, "kind": "reference",
            "sample": f"{rows} token rows x 3 matrices of the reference's q_gemv_q4_f32_avx2 on 1 pinned core "
                      f"({orc.cpu_model_name()})"}


# ---------------------------------------------------------------------------
# HBM traffic of the dominant kernel (rocprofv3 --pmc passes)
# ---------------------------------------------------------------------------
COPY_BYTES = 256 << 20
TRAFFIC_LAUNCHES = 12


TRAFFIC_SHAPES = [("qkv", "h", ["wq", "wk", "wv"]), ("wo", "o", ["wo"]), ("gate_up", "h2", ["w_gate", "w_up"]),
                  ("down", "m", ["w_down"]), ("lm_head", "h", ["lm"])]
LM_VOCAB = 128256


def traffic_alg_bytes(name):
    if name == "lm_head":
        return alg_bytes(LM_VOCAB, DIM)
    mats = dict((n, m) for n, _, m in TRAFFIC_SHAPES)[name]
    return sum(alg_bytes(M, N) for k, M, N in SHAPES if k in mats)


def run_traffic():
    """Workload of the counter passes: for each GEMV launch shape of the
    decode step (Q|K|V, Wo, W_gate|W_up, W_down, each from its fp32 input)
    and the config-3 LM head (128256 x 4096), TRAFFIC_LAUNCHES launches in
    a block (rotating the weight sets), then 4 device copies of COPY_BYTES
    whose counter readings calibrate the KiB-per-dispatch scale.  Run it
    under `rocprofv3 --pmc FETCH_SIZE` and, separately, `--pmc WRITE_SIZE`;
    then --summarize-traffic."""
    import qorus_amd as qa
    from qorus_amd import synthetic as syn
    lib = qa.lib()
    if not qa.gpu_available():
        raise SystemExit("bench.py: no usable GPU")
    layers = [LayerSet(qa, gen_layer(1000 + l)) for l in range(LAYERS)]
    rng = syn.rng_for(91)
    lm = [qa.DeviceBuffer.from_numpy(syn.gen_q4(LM_VOCAB, DIM, rng)) for _ in range(2)]
    lm_t = [qa.q4_tensor(b.ptr, LM_VOCAB, DIM) for b in lm]
    xin = {k: qa.DeviceBuffer.from_numpy(syn.gen_f32(n, syn.rng_for(77))) for k, n in
           (("h", DIM), ("o", DIM), ("h2", DIM), ("m", HID))}
    ws = {k: qa.DeviceBuffer(lib.qh_gemv_workspace_bytes(n)) for k, n in
          (("h", DIM), ("o", DIM), ("h2", DIM), ("m", HID))}
    outs = {k: qa.DeviceBuffer(M * 4) for k, M, _ in SHAPES}
    outs["lm"] = qa.DeviceBuffer(LM_VOCAB * 4)
    src, dst = qa.DeviceBuffer(COPY_BYTES), qa.DeviceBuffer(COPY_BYTES)
    stream = qa.Stream()
    s = stream.handle
    for name, xk, mats in TRAFFIC_SHAPES:
        for i in range(TRAFFIC_LAUNCHES):
            L = layers[i % LAYERS]
            Ws = ptr_array([(lm_t[i % 2] if m == "lm" else L.t[m]).addr for m in mats])
            ys = ptr_array([outs[m].ptr for m in mats])
            qa.check(lib.qh_gemv_q4_f32_multi(Ws, None, ys, len(mats), xin[xk].ptr, ws[xk].ptr, s))
        stream.sync()
    for _ in range(4):
        qa.check(lib.qh_memcpy_dtod(dst.ptr, src.ptr, COPY_BYTES, s))
    stream.sync()
    print(json.dumps({"traffic_workload": [n for n, _, _ in TRAFFIC_SHAPES], "launches": TRAFFIC_LAUNCHES,
                      "copy_bytes": COPY_BYTES}))


def _counter_rows(d):
    import csv
    rows = []
    for f in Path(d).rglob("*counter_collection.csv"):
        rows += list(csv.DictReader(open(f)))
    if not rows:
        raise SystemExit(f"no counter_collection.csv under {d}")
    return rows


def summarize_traffic(fetch_dir, write_dir, cmd):
    """profiles/gemv_traffic.json from the two counter passes.  The GEMV
    dispatches, in dispatch order, are the blocks of TRAFFIC_SHAPES; each
    counter's KiB-per-dispatch reading (median of a block, its first two
    launches left out) is scaled by copy_bytes / (what the same counter
    reads for the device copy), so the figure is in bytes of the copy's own
    accounting."""
    per = {n: {} for n, _, _ in TRAFFIC_SHAPES}
    cal = {}
    for cname, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        rows = [r for r in _counter_rows(d) if r.get("Counter_Name") == cname]
        gemv = sorted((r for r in rows if "k_gemv" in r["Kernel_Name"]), key=lambda r: int(r["Dispatch_Id"]))
        copies = [r for r in rows if "copyBuffer" in r["Kernel_Name"]]
        gmax = max((int(r["Grid_Size"]) for r in copies), default=0)
        copy = [float(r["Counter_Value"]) for r in copies if int(r["Grid_Size"]) == gmax]
        if len(gemv) != TRAFFIC_LAUNCHES * len(TRAFFIC_SHAPES) or not copy:
            raise SystemExit(f"{cname}: {len(gemv)} gemv dispatches, {len(copy)} copies")
        c = float(np.median(copy))
        factor = COPY_BYTES / (c * 1024.0)
        cal[cname] = {"copy_kib_per_dispatch": c, "copy_bytes": COPY_BYTES, "scale": factor}
        for i, (name, _, _) in enumerate(TRAFFIC_SHAPES):
            block = [float(r["Counter_Value"]) for r in gemv[i * TRAFFIC_LAUNCHES:(i + 1) * TRAFFIC_LAUNCHES]]
            g = float(np.median(block[2:]))
            per[name][cname] = {"kib_per_dispatch": g, "bytes_per_dispatch": g * 1024.0 * factor}
    shapes = {}
    for name, _, _ in TRAFFIC_SHAPES:
        t = per[name]["FETCH_SIZE"]["bytes_per_dispatch"] + per[name]["WRITE_SIZE"]["bytes_per_dispatch"]
        alg = traffic_alg_bytes(name)
        shapes[name] = {"alg_bytes_per_launch": alg, "traffic_bytes_per_launch": round(t),
                        "traffic_over_alg": round(t / alg, 4), "counters": per[name]}
    res = {"kernel": "k_gemv_p fused W_gate|W_up 28672x4096 (config 2)", "alg_bytes_per_launch": GATE_UP_BYTES,
           "traffic_bytes_per_launch": shapes["gate_up"]["traffic_bytes_per_launch"],
           "traffic_over_alg": shapes["gate_up"]["traffic_over_alg"], "shapes": shapes, "calibration": cal,
           "command": cmd}
    p = REPO / "profiles" / "gemv_traffic.json"
    p.write_text(json.dumps(res, indent=1) + "\n")
    print(json.dumps(res))


# Decode attention at context 2048 (config 4, pos 2047 onward): algorithmic
# bytes per dispatch of the three kernels, per layer (8 KV heads x 2048
# positions x 128 floats of K or V; 32 query heads).  The cache rows hold K
# and V side by side, so each kernel reads half of every 1-KB row.
ATTN_KEYS, ATTN_HEADS, ATTN_KV, ATTN_HD = 2048, 32, 8, 128
ATTN_CHUNKS_PV = (ATTN_KEYS + 255) // 256
ATTN_ALG = {
    # K rows + q, scores and 64-key chunk maxima written
    "k_attn_scores": ATTN_KV * ATTN_KEYS * ATTN_HD * 4 + ATTN_HEADS * ATTN_HD * 4 + ATTN_HEADS * ATTN_KEYS * 4
    + ATTN_HEADS * (ATTN_KEYS // 64) * 4,
    # V rows + scores and chunk maxima read, P.V partials and chunk sums written
    "k_attn_pv": ATTN_KV * ATTN_KEYS * ATTN_HD * 4 + ATTN_HEADS * ATTN_KEYS * 4 + ATTN_HEADS * (ATTN_KEYS // 64) * 4
    + ATTN_CHUNKS_PV * ATTN_HEADS * ATTN_HD * 4 + ATTN_CHUNKS_PV * ATTN_HEADS * 4,
    # partials and sums read, the 4096-float output's digit planes written
    "k_attn_combine": ATTN_CHUNKS_PV * ATTN_HEADS * ATTN_HD * 4 + ATTN_CHUNKS_PV * ATTN_HEADS * 4 + 13 * 16 * 128,
}


def summarize_attn_traffic(fetch_dir, write_dir, cmd):
    """profiles/attention_traffic.json: FETCH_SIZE and WRITE_SIZE per
    dispatch of the decode-step attention kernels, from two --pmc passes
    over the config-4 decode leg (median over every dispatch of a kernel),
    scaled by the plain-copy calibration of profiles/gemv_traffic.json (the
    same counters on the same part)."""
    cal = json.loads((REPO / "profiles" / "gemv_traffic.json").read_text())["calibration"]
    per = {k: {} for k in ATTN_ALG}
    for cname, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        rows = [r for r in _counter_rows(d) if r.get("Counter_Name") == cname]
        for k in ATTN_ALG:
            vals = [float(r["Counter_Value"]) for r in rows if ("qh::" + k + "<") in r["Kernel_Name"]
                    or ("qh::" + k + "(") in r["Kernel_Name"]]
            if not vals:
                raise SystemExit(f"{cname}: no {k} dispatches under {d}")
            g = float(np.median(vals))
            per[k][cname] = {"dispatches": len(vals), "kib_per_dispatch": g,
                             "bytes_per_dispatch": g * 1024.0 * cal[cname]["scale"]}
    res = {"workload": "config-4 decode step, context 2048..2080 (the bench's decode leg), per layer",
           "kernels": {k: {"alg_bytes_per_dispatch": ATTN_ALG[k],
                           "traffic_bytes_per_dispatch": round(per[k]["FETCH_SIZE"]["bytes_per_dispatch"]
                                                               + per[k]["WRITE_SIZE"]["bytes_per_dispatch"]),
                           "traffic_over_alg": round((per[k]["FETCH_SIZE"]["bytes_per_dispatch"]
                                                      + per[k]["WRITE_SIZE"]["bytes_per_dispatch"]) / ATTN_ALG[k], 4),
                           "counters": per[k]} for k in ATTN_ALG},
           "calibration": "profiles/gemv_traffic.json (FETCH_SIZE x%.4f, WRITE_SIZE x%.4f)"
           % (cal["FETCH_SIZE"]["scale"], cal["WRITE_SIZE"]["scale"]),
           "command": cmd}
    p = REPO / "profiles" / "attention_traffic.json"
    p.write_text(json.dumps(res, indent=1) + "\n")
    print(json.dumps(res))


def traffic_from_profiles():
    """HBM bytes per launch of the dominant kernel from the committed
    rocprofv3 --pmc summary (profiles/gemv_traffic.json), or None."""
    p = REPO / "profiles" / "gemv_traffic.json"
    try:
        return json.loads(p.read_text()).get("traffic_bytes_per_launch")
    except (OSError, ValueError):
        return None


def run_sample(n_calls=40, warmup=5):
    """q_sample_token (reference main.c:852-992) at the Llama-3 vocabulary
    (128256) on synthetic logits, host logits in and token out as the
    reference's API takes them: wall time per call (H2D of the logits, the
    device pipeline, the token's D2H), median over n_calls."""
    import qorus_amd as qa
    lib = qa.lib()
    V = 128256
    rng = np.random.default_rng(12)
    raw = np.empty(V * 4 + 64, np.uint8)  # 64-byte aligned float32 logits
    off = (-raw.ctypes.data) % 64
    lg = raw[off:off + V * 4].view(np.float32)
    lg[:] = rng.standard_normal(V).astype(np.float32) * np.float32(3.0)
    tok = C.c_uint32()
    lib.qh_sample_set_state(123456789)
    out = {}
    for name, T, k, p in (("greedy", 0.0, 0, 0.0), ("T0.8_topk40", 0.8, 40, 0.0), ("T0.8_topp0.9", 0.8, 0, 0.9),
                          ("T0.8_topk40_topp0.95", 0.8, 40, 0.95), ("T1.0_no_filter", 1.0, 0, 0.0)):
        ts = []
        for i in range(warmup + n_calls):
            t0 = time.perf_counter()
            rc = lib.q_sample_token(lg.ctypes.data, V, T, k, p, C.byref(tok), None)
            t1 = time.perf_counter()
            if rc != 0:
                raise SystemExit(f"q_sample_token failed: {lib.qh_last_error().decode()}")
            if i >= warmup:
                ts.append(t1 - t0)
        out[name] = round(float(np.median(ts)) * 1e6, 1)
    log(f"[bench] q_sample_token us/call at V={V}: {out}")
    return {"vocab": V, "us_per_call": out,
            "logits": "synthetic N(0,1)*3, host memory (the reference API's contract)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--no-decode", action="store_true", help="skip the config-4 decode leg")
    ap.add_argument("--decode-steps", type=int, default=32)
    ap.add_argument("--decode-warmup", type=int, default=4)
    ap.add_argument("--no-sampled-decode", action="store_true",
                    help="config-4 leg: greedy decode only (no device-sampled generation)")
    ap.add_argument("--cpu-decode-tokens", type=int, default=3)
    ap.add_argument("--no-lmhead", action="store_true", help="skip the config-3 LM-head leg")
    ap.add_argument("--no-sample", action="store_true", help="skip the q_sample_token leg")
    ap.add_argument("--no-prefill", action="store_true", help="skip the config-5 prefill GEMM leg")
    ap.add_argument("--no-prompt", action="store_true",
                    help="skip the llama_forward prompt on the config-4 model")
    ap.add_argument("--prompt-tokens", type=int, nargs="+", default=list(PROMPT_TS),
                    help="tokens of those prompts (default 512 2048; up to the decode model's context)")
    ap.add_argument("--traffic", action="store_true",
                    help="run only the workload of the rocprofv3 --pmc traffic passes")
    ap.add_argument("--summarize-traffic", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="write profiles/gemv_traffic.json from two --pmc output dirs")
    ap.add_argument("--summarize-attn-traffic", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="write profiles/attention_traffic.json from two --pmc passes over the decode leg")
    ap.add_argument("--traffic-cmd", default="", help="command line recorded with the summary")
    ap.add_argument("--only", choices=("prefill", "decode", "lmhead"),
                    help="run one leg alone and print its JSON (for profiler runs; not the bench line)")
    args = ap.parse_args()
    if args.summarize_traffic:
        summarize_traffic(*args.summarize_traffic, args.traffic_cmd)
        return
    if args.summarize_attn_traffic:
        summarize_attn_traffic(*args.summarize_attn_traffic, args.traffic_cmd)
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (batch-1 decode of an 8B model is not "
              f"sharded); --gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)
    if args.traffic:
        run_traffic()
        return
    if args.only:
        leg = {"prefill": run_prefill, "decode": run_decode, "lmhead": run_lmhead}[args.only]
        print(json.dumps({"leg": args.only, "result": leg(args)}), flush=True)
        return

    wall, achieved, kern_ms, breakdown, config1 = run_gpu(args)
    ms_per_step = wall / args.steps * 1e3
    value = STEP_BYTES * args.steps / wall / 1e9
    cpu = None if args.no_cpu else run_cpu_baseline(args.cpu_seconds)
    lmhead = None if args.no_lmhead else run_lmhead(args)
    decode = None if args.no_decode else run_decode(args)
    sample = None if args.no_sample else run_sample()
    prefill = None if args.no_prefill else run_prefill(args)
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 x f32 (int4 digit-plane dot, f32 scale/accumulate)",
        "data": "synthetic (seeded: nibbles U{0..15}, scale |N(0,1)|*0.02, x ~ N(0,1))",
        "config": {"workload": "config2: Llama-3-8B per-layer decode GEMV set at batch 1 "
                               "(Wq,Wk,Wv,Wo,W_gate,W_up,W_down Q4_0; fp32 x)",
                   "layers_rotated": LAYERS, "bytes_per_step": STEP_BYTES,
                   "launches_per_step": 4, "step_exec": "one hipGraph of all K steps"},
        "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles(),
                     "kernel": "k_gemv (fused W_gate|W_up, 28672x4096)",
                     "alg_bytes_per_launch": GATE_UP_BYTES, "mean_launch_us": round(kern_ms * 1e3, 2)},
        "kernels": breakdown,
        "config1": config1,
        "cpu_baseline": cpu,
        "lmhead": lmhead,
        "decode": decode,
        "sample": sample,
        "prefill": prefill,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
