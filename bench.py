"""Headline benchmark: batch-1 Q4 decode of the Llama-3-8B-shaped model
(hidden 4096, 32 layers, 32/8 heads of 128, intermediate 14336, vocab
128256, GGUF Q4_K weights repacked at load into the reference's 32-blocks
with Q4_K's own scales kept beside them, fp16 KV cache of 4096) on one
MI355X.

A step is one greedy decode token (one replay of the captured token graph:
32 layers of Q4_K GEMVs, attention over the cache, the head and the pick).
The prompt of random ids fills the cache to position ctx - warmup - steps
first, so the timed tokens attend over ~4,000 keys.

Printed (one JSON line): tok/s, plus
- roofline: the dominant kernel, the gate|up GEMV (28672 x 4096), launched as
  the decode launches it and timed with HIP events on its own stream across
  the 32 layers' distinct matrices: algorithmic bytes / average launch time
  vs 8 TB/s;
- cpu_baseline: the oracle's shader-order float32 restatement of the
  reference's split matmul (OpenMP, the host's cores) on one layer's four
  matmuls and the head, extrapolated to a 32-layer token.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q4 GEMV HBM GB/s (% of peak); decode tok/s, 8B-shape Q4 batch 1"
HBM_PEAK_GBPS = 8000.0

# Algorithmic bytes a weight of each weight file format: what a GEMV must
# read at least, whatever layout the device keeps (GGUF Q4_0 18 B / 32,
# Q4_K 144 B / 256, MatMulNBits q4 16 B of nibbles + a half scale + half a
# byte of zero point / 32, Q8_0 34 B / 32, Q6_K 210 B / 256).
BPW = {"q4_0": 18 / 32, "q4_k": 144 / 256, "q4_k_rowgroup": 144 / 256,
       "q4_k_records": 144 / 256, "nbits": 18.5 / 32,
       "q8_0": 34 / 32, "q8": 34 / 32, "q6_k": 210 / 256}


def gemv_bytes(N, K, M, fmt):
    """Algorithmic bytes of an N x K GEMV over M rows: the weights at their
    file format's bytes a weight, the half inputs and float32 outputs."""
    return int(round(N * K * BPW[fmt])) + M * K * 2 + M * N * 4


def token_bytes(shape, keys, M=1):
    """Algorithmic bytes of one forward of M rows of a model shape: every
    layer's GEMVs, the head, the keys and values of `keys` cache positions in
    every attention layer (read once for all M rows), and the conv states."""
    s, D, F = shape, shape.hidden, shape.intermediate
    total = 0
    for i in range(s.layers):
        if s.layer_type(i) == "conv":
            total += gemv_bytes(3 * D, D, M, s.fmt) + gemv_bytes(D, D, M, s.fmt)
            total += (s.conv_kernel - 1) * D * 4 * 2  # state read and written
        else:
            total += gemv_bytes(s.qkv_rows, D, M, s.fmt)
            total += gemv_bytes(D, s.heads * s.head_dim, M, s.fmt)
            total += 2 * s.kv_heads * s.head_dim * 2 * keys
        total += gemv_bytes(2 * F, D, M, s.fmt) + gemv_bytes(D, F, M, s.fmt)
    return total + gemv_bytes(s.vocab, D, M, s.embed_fmt or s.fmt)


def host_threads():
    """Threads for a CPU baseline: every CPU in the process's affinity mask,
    capped by OMP_NUM_THREADS where the host sets it (a shared machine's CPU
    share for one GPU job). Returns (threads, a note saying so)."""
    allowed = len(os.sched_getaffinity(0))
    host = os.cpu_count() or allowed
    env = os.environ.get("OMP_NUM_THREADS", "")
    threads = allowed
    note = f"{allowed} CPUs in the affinity mask, {host} on the host"
    if env.isdigit() and 0 < int(env) < allowed:
        threads = int(env)
        note += f"; OMP_NUM_THREADS={env}, the host's CPU share for one GPU job"
    return threads, note


def gemv_roofline(mats, x, parts, out16, eps, reps=6, fmt="q4_k"):
    """Average duration of the gate|up GEMV, launched as the decode launches
    it (prescaled norm in, SwiGLU out), over distinct matrices. `achieved`
    counts the GEMV's algorithmic bytes at the weight file format's bytes a
    weight (gemv_bytes); the bytes of the layout the device keeps are
    reported beside them."""
    import torch
    from webgllm_amd import lib as L, ops
    m = mats[0]
    F, D = m.N // 2, m.K
    ep = L.Epilogue(mode=L.EPI_SWIGLU, out16=out16.data_ptr(), ld_out16=F,
                    norm_parts=parts.data_ptr(), n_parts=D // 4, ld_parts_in=D // 4,
                    norm_count=D, eps=eps, norm_mult=32.0)
    # one pass over the matrices captured as a graph and replayed `reps`
    # times: launch to launch on the GPU, with no host time between launches
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for mm in mats[:4]:
            ops.gemv(mm, x, epilogue=ep)
        stream.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for mm in mats:
                ops.gemv(mm, x, epilogue=ep)
        g.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            g.replay()
        e1.record(stream)
    stream.synchronize()
    launches = reps * len(mats)
    us = e0.elapsed_time(e1) * 1e3 / launches
    algo = gemv_bytes(m.N, m.K, 1, fmt)
    achieved = algo / (us * 1e-6) / 1e9
    # the device layout's bytes: nibbles and scales (Q4_K records, or half
    # scales and zero points), x (halves), the norm's parts and the half
    # SwiGLU output
    stored = m.nbytes + D * 2 + (D // 4) * 4 + F * 2
    scales = ("Q4_K scale records (d, dmin, 6-bit scales and mins: 0.5625 bytes a weight "
              "with the nibbles)" if m.zero == L.ZERO_Q4K else "half scale + half zero per 32 "
              "weights")
    stored_gbps = stored / (us * 1e-6) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": measured_traffic(),
            "kernel": f"gemv_stream_kernel gate|up {m.N}x{m.K}, SwiGLU epilogue",
            "bytes_per_launch": algo,
            "bytes_rule": f"N*K*{BPW[fmt]:.4f} ({fmt} file bytes a weight) + K*2 (half x) "
                          f"+ N*4 (float32 y)",
            "avg_launch_us": round(us, 3), "launches": launches,
            "stored_layout": {"bytes_per_launch": stored, "achieved": round(stored_gbps, 1),
                              "frac": round(stored_gbps / HBM_PEAK_GBPS, 4),
                              "what": f"the device's layout: 4-bit + {scales}, x, norm "
                                      "parts, half SwiGLU out"}}


def measured_traffic():
    """HBM bytes per launch of the gate|up GEMV from the FETCH_SIZE and
    WRITE_SIZE counter runs of `bench.py --roofline-only`, each scaled by
    what the counter reads for a copy of known size; the figure is kept in
    the traffic summary beside the kernel's rocprof summary."""
    path = os.path.join(ROOT, "profiles", "gemv_gate_up_llama8b_traffic.txt")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1].replace(",", "").strip())
    except OSError:
        pass
    return None


def roofline_only(args):
    """The gate|up GEMV alone over 32 distinct 28672 x 4096 Q4_K matrices,
    then a 256 MiB device copy: a short program for counter runs."""
    import torch
    from webgllm_amd import engine as E
    shape = E.LLAMA3_8B
    F, D = shape.intermediate, shape.hidden
    w = E.Weights.blank(shape, seed=0)
    mats = [w.matrix(2 * F, D, E.gate_up_row_order(F)) for _ in range(shape.layers)]
    x = (torch.randn((1, D), device="cuda") * 0.1).half()
    parts = torch.ones((1, D // 4), device="cuda")
    out16 = torch.zeros((1, F), dtype=torch.float16, device="cuda")
    torch.cuda.synchronize()
    roof = gemv_roofline(mats, x, parts, out16, shape.eps, reps=args.reps)
    n = 256 << 20
    src = torch.ones(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)  # reads and writes 256 MiB: the counters' scale
    torch.cuda.synchronize()
    print(json.dumps({"roofline": roof, "copy_bytes_each_way": n, "copies": 3}), flush=True)


def oracle_matrix(m):
    """The oracle's QuantMatrix holding a device matrix's arrays (row order
    as stored; the timing does not depend on it)."""
    import numpy as np
    from oracle import oracle as O
    from webgllm_amd import lib as L
    if m.layout == L.LAYOUT_Q4K:
        G, S = m.N // 4, m.K // 256
        rec = m.quants.cpu().numpy().reshape(G, S, 4, 144)
        src = np.ascontiguousarray(rec.transpose(0, 2, 1, 3)).reshape(-1)
        qm = O.QuantMatrix(m.N, m.K, "halves")
        O.pack_q4_k(qm, 0, src, m.N)
        return qm
    if m.zero == L.ZERO_Q4K:  # the super-blocks behind the records, packed as the reference does
        src = O.q4k_from_records(m.quants.cpu().numpy(), m.scales.cpu().numpy().view(np.uint8),
                                 m.N, m.K)
        qm = O.QuantMatrix(m.N, m.K, "halves")
        O.pack_q4_k(qm, 0, src.reshape(-1), m.N)
        return qm
    qm = O.QuantMatrix(m.N, m.K, {L.ZERO_8: False, L.ZERO_U8: True, L.ZERO_F16: "halves"}[m.zero])
    qm.quants[:] = m.quants.cpu().numpy().view(np.uint32)
    qm.scales[:] = m.scales.cpu().numpy().view(np.uint16)
    if m.zero == L.ZERO_U8:
        qm.zeros[:] = m.zeros.cpu().numpy()
    elif m.zero == L.ZERO_F16:
        qm.zero_halves[:] = m.zeros.cpu().numpy().view(np.uint16)
    return qm


def cpu_step_time(groups, M, threads, seconds=12.0):
    """The oracle's shader-order float32 split matmul (OpenMP) over one matrix
    of each group, M rows of half activations, repeated for about `seconds`.
    groups: (label, device matrix, times a step uses it). Returns (seconds
    per step, a description of the sample)."""
    import numpy as np
    from oracle import oracle as O
    qms = [(label, oracle_matrix(m), k) for label, m, k in groups]
    rng = np.random.default_rng(0)
    xs = {qm.K: O.f32_to_h2(rng.standard_normal((M, qm.K)).astype(np.float32))
          for _, qm, _ in qms}
    O.matmul_split(qms[0][1], xs[qms[0][1].K], threads)  # warm the threads
    spent = {label: 0.0 for label, _, _ in qms}
    reps = 0
    while reps < 100000 and (sum(spent.values()) < seconds or reps < 2):
        for label, qm, _ in qms:
            t0 = O.now()
            O.matmul_split(qm, xs[qm.K], threads)
            spent[label] += O.now() - t0
        reps += 1
    per_step = sum(spent[label] / reps * k for label, _, k in qms)
    parts = ", ".join(f"{label} {spent[label] / reps * 1e3:.1f} ms x{k}" for label, _, k in qms)
    desc = (f"oracle shader-order fp32 split matmul (OpenMP, {threads} threads: "
            f"{host_threads()[1]}), {M} row(s): {parts}; {reps} repetitions "
            f"({sum(spent.values()):.1f} s), extrapolated to the step")
    return per_step, desc


def cpu_attention_time(engine, layer, keys, threads, seconds=2.0):
    """The oracle's float32 attention (the shaders' scores and attend, heads
    in parallel) of one query row over `keys` rows of a layer's cache."""
    import numpy as np
    from oracle import oracle as O
    s = engine.shape
    kc = engine.k_cache[layer][:keys].cpu().numpy().view(np.uint16)
    vc = engine.v_cache[layer][:keys].cpu().numpy().view(np.uint16)
    q = (np.random.default_rng(0).standard_normal(s.heads * s.head_dim) /
         np.sqrt(s.head_dim)).astype(np.float32)
    kvd = s.kv_heads * s.head_dim
    O.attention_f32(q, kc, vc, s.heads, s.kv_heads, s.head_dim, keys, kvd, threads)
    spent, n = 0.0, 0
    while spent < seconds or n < 2:
        t0 = O.now()
        O.attention_f32(q, kc, vc, s.heads, s.kv_heads, s.head_dim, keys, kvd, threads)
        spent += O.now() - t0
        n += 1
    return spent / n


def cpu_baseline(engine, threads, seconds=12.0, keys=None):
    """Oracle split matmul (float32, shader order) on one layer + the head,
    repeated for about `seconds` of CPU time, plus the float32 attention of
    one layer over `keys` cache rows, extrapolated to a token (norms, the
    embedding row and the pick are left out: under 0.1% of the bytes)."""
    s = engine.shape
    lw = engine.w.layers[0]
    groups = [(k, lw[k], s.layers) for k in ("qkv", "o", "gate_up", "down")]
    groups.append(("head", engine.w.embedding, 1))
    per_token, desc = cpu_step_time(groups, 1, threads, seconds)
    if keys:
        att = cpu_attention_time(engine, 0, keys, threads)
        per_token += att * s.layers
        desc += (f"; attention: the oracle's float32 scores/attend over {keys} keys, "
                 f"{att * 1e3:.2f} ms x{s.layers}")
    return {"value": round(1.0 / per_token, 4), "unit": "tok/s", "cores": threads,
            "kind": "port", "sample": desc}


def line(metric, value, unit, steps, warmup, ms, config, roofline, cpu, dtype="f32", **extra):
    out = {"metric": metric, "value": value, "unit": unit, "n_gpus": 1, "steps": steps,
           "warmup": warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": dtype, "data": "synthetic",
           "config": config, "roofline": roofline, "cpu_baseline": cpu}
    out.update(extra)
    return out


def timed(fn, reps):
    """Average milliseconds of fn() over reps runs, between HIP events on the
    current stream."""
    import torch
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(reps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def workload_q4_0_gemv(args):
    """Q4_0 GEMV 2048 x 2048, batch 1 (a decode step's matmul): graph-captured
    launches over 256 distinct weight copies (604 MB, more than the 256 MB
    infinity cache), each moving 2,359,296 weight bytes + the half input + the
    float32 output."""
    import torch
    from webgllm_amd import engine as E, ops
    N = K = 2048
    copies = 256
    shape = E.ModelShape("q4_0-gemv", K, 1, 1, 1, 4, 4, 4, "q4_0")
    w = E.Weights.blank(shape, seed=0)
    mats = [w.matrix(N, K) for _ in range(copies)]
    x = (torch.randn((1, K), device="cuda", generator=torch.Generator(device="cuda")
                     .manual_seed(1))).half()
    y = torch.empty((1, N), device="cuda")
    algo = mats[0].nbytes + K * 2 + N * 4
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for m in mats[:4]:
            ops.gemv(m, x, out=y)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for m in mats:
                ops.gemv(m, x, out=y)
    torch.cuda.synchronize()
    reps = max(1, args.steps // 16)
    for _ in range(args.warmup // 8 + 1):
        g.replay()
    ms_graph = timed(g.replay, reps)
    us = ms_graph * 1e3 / copies
    gbps = algo / (us * 1e-6) / 1e9
    # the same matrix over and over (held in the caches)
    with torch.cuda.stream(s):
        gh = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gh, stream=s):
            for _ in range(copies):
                ops.gemv(mats[0], x, out=y)
    torch.cuda.synchronize()
    gh.replay()
    hot = timed(gh.replay, reps) * 1e3 / copies
    cpu = None
    if not args.no_cpu:
        threads = host_threads()[0]
        t, desc = cpu_step_time([("2048x2048", mats[0], 1)], 1, threads, 10.0)
        cpu = {"value": round(algo / t / 1e9, 3), "unit": "GB/s", "cores": threads,
               "kind": "port", "sample": desc}
    roof = {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None,
            "kernel": "gemv_stream_kernel 2048x2048 Q4_0 (cold: 256 distinct copies)",
            "bytes_per_launch": algo, "avg_launch_us": round(us, 3),
            "launches": reps * copies}
    cfg = {"workload": "Q4_0 GEMV 2048x2048 batch 1, half input, float32 output, 256 "
                       "distinct weight copies in one captured graph",
           "weights": "random GGUF Q4_0 blocks (18 bytes / 32 weights) repacked on the GPU "
                      "(packQ4_0)", "global_batch": 1, "parallelism": "none"}
    return line("Q4_0 GEMV HBM GB/s", round(gbps, 1), "GB/s", reps * copies, args.warmup,
                ms_graph / copies, cfg, roof, cpu, hot_launch_us=round(hot, 3),
                hot_GBps=round(algo / (hot * 1e-6) / 1e9, 1))


def workload_nbits_gemm(args, fmt="nbits"):
    """Prefill GEMM on MFMA: A half [512 x 4096] times MatMulNBits weights
    (4-bit, half scales, u8 zero points, block 32) at N = 4096 and 14336,
    float32 output. With fmt "q8": 8-bit matrices (floats requantized as
    the GGUF loader does) on the same kernel."""
    import torch
    from webgllm_amd import engine as E, ops
    M, K = 512, 4096
    shape = E.ModelShape(f"{fmt}-gemm", K, 1, 1, 1, 4, 4, 4, fmt)
    w = E.Weights.blank(shape, seed=0)
    a = torch.randn((M, K), device="cuda", generator=torch.Generator(device="cuda")
                    .manual_seed(2)).half()
    res = {}
    for N in (4096, 14336):
        mats = [w.matrix(N, K) for _ in range(4)]
        c = torch.empty((M, N), device="cuda")
        # a few milliseconds of warm-up: the first launches after new weights
        # run ~10% slow while the clocks come up
        for i in range(40):
            ops.gemm(mats[i % 4], a, out=c)
        it = iter(range(1 << 30))
        ms = timed(lambda: ops.gemm(mats[next(it) % 4], a, out=c), max(100, 2 * args.steps))
        res[N] = (ms, 2.0 * M * N * K / (ms * 1e-3) / 1e12, mats[0])
    tot_flop = sum(2.0 * M * N * K for N in res)
    tot_ms = sum(r[0] for r in res.values())
    tflops = tot_flop / (tot_ms * 1e-3) / 1e12
    cpu = None
    if not args.no_cpu and fmt == "nbits":
        threads = host_threads()[0]
        t, desc = cpu_step_time([("4096x4096", res[4096][2], 1),
                                 ("14336x4096", res[14336][2], 1)], 8, threads, 10.0)
        cpu = {"value": round(tot_flop / 64 / t / 1e12, 5), "unit": "TFLOP/s",
               "cores": threads, "kind": "port",
               "sample": desc + " (8 of the 512 rows; the rate scales with rows)"}
    elif not args.no_cpu:
        import numpy as np
        from oracle import oracle as O
        from webgllm_amd import lib as L
        threads = host_threads()[0]
        m = res[14336][2]
        wm = O.WideMatrix(m.N, m.K, 8)
        wm.quants[:] = m.quants.cpu().numpy()
        wm.scales[:] = m.scales.cpu().numpy().view(np.uint16)
        x16 = O.f32_to_h2(np.random.default_rng(0).standard_normal((8, K)).astype(np.float32))
        spent, n = 0.0, 0
        while spent < 10.0 or n < 2:
            t0 = O.now()
            wm.matmul(x16, threads)
            spent += O.now() - t0
            n += 1
        cpu = {"value": round(2.0 * 8 * m.N * K / (spent / n) / 1e12, 5), "unit": "TFLOP/s",
               "cores": threads, "kind": "port",
               "sample": f"oracle float32 8-bit block form (OpenMP, {threads} threads), 8 rows x "
                         f"the 14336x4096 matrix, {n} repetitions ({spent:.1f} s)"}
    roof = {"bound": "mfma", "achieved": round(tflops, 1), "peak": 2500.0, "unit": "TFLOP/s",
            "frac": round(tflops / 2500.0, 4), "traffic": None,
            "kernel": "gemm_q4_kernel (v_mfma_f32_32x32x16_f16, dequant in registers)",
            "flops_per_launch": {str(N): 2 * M * N * K for N in res},
            "avg_launch_us": {str(N): round(r[0] * 1e3, 2) for N, r in res.items()}}
    what = "MatMulNBits q4" if fmt == "nbits" else "8-bit"
    cfg = {"workload": f"{what} prefill GEMM, M=512, K=4096, N in {{4096, 14336}}",
           "weights": "random MatMulNBits q4 rows (u8 zero points) repacked on the GPU"
                      if fmt == "nbits" else "random floats requantized to 8 bits on the GPU "
                                             "(quantizeQ8)",
           "global_batch": M, "parallelism": "none"}
    return line(f"prefill GEMM TFLOP/s ({what}, M=512)", round(tflops, 1), "TFLOP/s",
                args.steps, 4, tot_ms, cfg, roof, cpu, dtype="f16 x f16 -> f32",
                per_shape_tflops={str(N): round(r[1], 1) for N, r in res.items()})


def decode_engine_run(shape, ctx, prompt_len, steps, warmup):
    """Prefill random ids, capture the token step, warm up, then time
    `steps` graph replays. Returns (engine, weights, ms a token, first
    timed position)."""
    import torch
    from webgllm_amd import engine as E
    w = E.Weights(shape, seed=0)
    eng = E.Engine(w, ctx)
    prompt = torch.randint(0, shape.vocab, (prompt_len,),
                           generator=torch.Generator().manual_seed(1)).tolist()
    first = int(eng.forward(prompt)[-1])
    # the timed replays run past what decode() reserves: room for all of them
    eng.reserve(min(ctx, eng.position + warmup + steps + 1))
    eng.capture_step(first)
    eng.decode(first, warmup)
    p0 = eng.position
    eng.ids[0] = int(eng.hist[p0].item())
    eng.pos.fill_(p0)
    ms = timed(eng.graph.replay, steps)
    eng.position += steps
    return eng, w, ms, p0


def workload_qwen2_decode(args):
    """Qwen2-0.5B-shape greedy decode (MatMulNBits q4, fp16 KV cache of 1024):
    a 512-id random prompt, then decode to position 1024."""
    from webgllm_amd import engine as E
    shape = E.QWEN2_05B
    steps = 1024 - 512 - args.warmup - 1
    eng, w, ms, p0 = decode_engine_run(shape, 1024, 512, steps, args.warmup)
    keys = p0 + (steps + 1) // 2
    tok_bytes = token_bytes(shape, keys)
    cpu = cpu_baseline(eng, host_threads()[0], 10.0, keys=keys) if not args.no_cpu else None
    gbps = tok_bytes / (ms * 1e-3) / 1e9
    roof = {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None,
            "kernel": "whole token (MatMulNBits weights at 18.5 B / 32, ~286 MB, about the "
                      "infinity cache's size: 'effective' GB/s)", "bytes_per_launch": tok_bytes,
            "avg_launch_us": round(ms * 1e3, 2), "launches": steps}
    cfg = {"workload": f"Qwen2-0.5B-shape greedy decode, positions {p0}..{p0 + steps - 1}",
           "model": shape.name, "layers": shape.layers, "hidden": shape.hidden,
           "vocab": shape.vocab, "weights": "random MatMulNBits q4 (u8 zero points)",
           "global_batch": 1, "seq_len": 1024, "parallelism": "none"}
    return line("decode tok/s, Qwen2-0.5B-shape MatMulNBits batch 1", round(1000.0 / ms, 2),
                "tok/s", steps, args.warmup, ms, cfg, roof, cpu)


def workload_lfm2_verify(args):
    """LFM2-1.2B-shape hybrid (10 short-conv + 6 attention layers, Q4_0):
    speculative verify of a token and 4 random draft ids (M = 5), keeping
    the agreeing prefix + 1 and rolling the conv states back (the
    reference's handler loop, src/handler.ts:1811-1887)."""
    import torch
    from webgllm_amd import engine as E
    shape = E.LFM2_12B
    w = E.Weights(shape, seed=0)
    ctx = 2048
    eng = E.Engine(w, ctx)
    g = torch.Generator().manual_seed(3)
    prompt = torch.randint(0, shape.vocab, (256,), generator=g).tolist()
    token = int(eng.forward(prompt)[-1])
    steps = min(args.steps, (ctx - 300) // 5)

    def verify(n):
        nonlocal token
        written = 0
        for _ in range(n):
            drafts = torch.randint(0, shape.vocab, (4,), generator=g).tolist()
            rows = eng.forward([token] + drafts, draft=True).tolist()
            kept = 1
            for i in range(4):
                if rows[i] != drafts[i]:
                    break
                kept += 1
            eng.accept(kept)
            token = rows[kept - 1]
            written += kept
        return written

    # the host loop (a readback and the accept on the host every step)
    verify(args.warmup)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    written_host = verify(steps)
    torch.cuda.synchronize()
    dt_host = time.perf_counter() - t0

    # the device loop: every step one graph replay (drafts from a device
    # table; the picks, accept and conv-state rollback on the device), the
    # kept counts read back once after the timed steps
    eng.reserve(min(ctx, eng.position + 5 * (args.warmup + steps)))
    eng.capture_verify(5)
    v = eng._verify
    eng.ids[0] = token
    eng.pos.fill_(eng.position)
    n = args.warmup + steps
    v["table"][:n].copy_(torch.randint(0, shape.vocab, (n, 4), generator=g, dtype=torch.int32))
    v["cursor"].zero_()
    for _ in range(args.warmup):
        v["graph"].replay()
    pos_start = int(eng.pos.item())
    ms = timed(v["graph"].replay, steps)
    kept = v["kept"][args.warmup:n].tolist()
    written = sum(kept)
    eng.position = pos_start + written
    assert int(eng.pos.item()) == eng.position
    dt = ms * steps * 1e-3
    # a step's algorithmic bytes: the Q4_0 weights once for the 5 rows, the
    # cache rows the batch reads (keys at the steps' mean position + 5)
    keys = (pos_start + eng.position) // 2 + 5
    step_bytes = token_bytes(shape, keys, M=5)
    gbps = step_bytes / (ms * 1e-3) / 1e9
    roof = {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None,
            "kernel": "whole verify step, one graph replay (5 rows: Q4_0 weights at 18 B / 32 "
                      "read once, the cache, the picks, accept and rollback on the device)",
            "bytes_per_launch": step_bytes, "avg_launch_us": round(ms * 1e3, 2),
            "launches": steps}
    cpu = None
    if not args.no_cpu:
        threads = host_threads()[0]
        conv = next(i for i in range(shape.layers) if shape.layer_type(i) == "conv")
        att = next(i for i in range(shape.layers) if shape.layer_type(i) == "attn")
        n_conv = len(shape.conv_layers)
        n_att = shape.layers - n_conv
        lc, la = w.layers[conv], w.layers[att]
        groups = [("in_proj", lc["in_proj"], n_conv), ("out_proj", lc["out_proj"], n_conv),
                  ("qkv", la["qkv"], n_att), ("o", la["o"], n_att),
                  ("gate_up", lc["gate_up"], shape.layers), ("down", lc["down"], shape.layers),
                  ("head", w.embedding, 1)]
        t, desc = cpu_step_time(groups, 5, threads, 10.0)
        cpu = {"value": round(1.0 / t, 4), "unit": "verify steps/s", "cores": threads,
               "kind": "port", "sample": desc}
    cfg = {"workload": "LFM2-1.2B-shape speculative verify, token + 4 random draft ids a "
                       "step (M = 5), accept + conv-state rollback on the device, one graph "
                       "replay a step",
           "model": shape.name, "layers": shape.layers, "hidden": shape.hidden,
           "vocab": shape.vocab, "weights": "random GGUF Q4_0", "global_batch": 5,
           "seq_len": ctx, "parallelism": "none"}
    return line("verify steps/s, LFM2-1.2B-shape Q4_0, 4 drafts", round(steps / dt, 2),
                "verify steps/s", steps, args.warmup, ms, cfg, roof, cpu,
                tokens_per_s=round(written / dt, 2), tokens_per_step=round(written / steps, 3),
                weight_bytes=w.nbytes,
                host_loop={"steps_per_s": round(steps / dt_host, 2),
                           "ms_per_step": round(dt_host * 1e3 / steps, 4),
                           "tokens_per_step": round(written_host / steps, 3),
                           "what": "forward(draft=True), the picks read back, accept on the "
                                   "host, every step"})


def workload_llama8b_prefill(args):
    """Llama-3-8B-shape prompt processing: a 2048-token random prompt from
    position 0, its first 2040 rows in GEMM batches of 512 (MFMA GEMMs, flash
    prefill attention), the last 8 through the few-token path with the head
    and the picks; tokens/s of the whole prompt, repeated from a reset
    cache."""
    import torch
    from webgllm_amd import engine as E, ops
    shape = E.LLAMA3_8B
    w = E.Weights(shape, seed=0)
    n = 2048
    eng = E.Engine(w, n + 8)
    assert eng._prefill_ok()
    prompt = torch.randint(0, shape.vocab, (n,),
                           generator=torch.Generator().manual_seed(4)).tolist()

    def run():
        eng.reset()
        eng.forward(prompt)
    for _ in range(2):
        run()
    reps = max(3, args.steps // 16)
    ms = timed(run, reps)
    tok_s = n / (ms * 1e-3)
    # the dominant kernel: layer 0's gate|up GEMM at 512 rows, as the batches launch it
    lw = w.layers[0]
    F, D = shape.intermediate, shape.hidden
    a = torch.randn((512, D), device="cuda").half()
    gu = torch.empty((512, 2 * F), device="cuda")
    col = eng._col_of(lw["gate_up"])
    for _ in range(20):
        ops.gemm(lw["gate_up"], a, out=gu, col_of=col)
    gms = timed(lambda: ops.gemm(lw["gate_up"], a, out=gu, col_of=col), 60)
    flop = 2.0 * 512 * 2 * F * D
    tf = flop / (gms * 1e-3) / 1e12
    roof = {"bound": "mfma", "achieved": round(tf, 1), "peak": 2500.0, "unit": "TFLOP/s",
            "frac": round(tf / 2500.0, 4), "traffic": None,
            "kernel": f"gemm_q4_kernel gate|up 512 x {2 * F} x {D} (Q4_K repacked; f16 zero "
                      f"points, rebuilt from the Q4_K records by one launch before it), column "
                      f"map to gate | up", "flops_per_launch": flop,
            "avg_launch_us": round(gms * 1e3, 2), "launches": 60}
    cpu = None
    if not args.no_cpu:
        threads = host_threads()[0]
        t, desc = cpu_step_time([("qkv", lw["qkv"], shape.layers), ("o", lw["o"], shape.layers),
                                 ("gate_up", lw["gate_up"], shape.layers),
                                 ("down", lw["down"], shape.layers)], 8, threads, 10.0)
        cpu = {"value": round(8 / t, 3), "unit": "tok/s", "cores": threads, "kind": "port",
               "sample": desc + " (8 prompt rows a step; the head is left out)"}
    cfg = {"workload": f"Llama-3-8B-shape Q4_K prompt of {n} random ids from position 0",
           "model": shape.name, "layers": shape.layers, "hidden": shape.hidden,
           "weights": "random GGUF Q4_K super-blocks, repacked on the GPU (packQ4_K)",
           "global_batch": n, "seq_len": n, "parallelism": "none"}
    return line("prefill tok/s, Llama-3-8B-shape Q4_K", round(tok_s, 1), "tok/s", reps, 2, ms,
                cfg, roof, cpu, dtype="f16 x f16 -> f32")


def workload_wide_gemv(args, fmt, N, K, copies, what):
    """A batch-1 GEMV over an 8-bit or Q6_K matrix as the decode launches the
    head (prescaled-norm input from the sums of squares, float32 out),
    graph-captured over `copies` distinct matrices."""
    import numpy as np
    import torch
    from oracle import oracle as O
    from webgllm_amd import engine as E, lib as L, ops
    shape = E.ModelShape(f"{fmt}-gemv", K, 1, 1, 1, 4, 4, 4, fmt)
    w = E.Weights.blank(shape, seed=0)
    mats = [w.matrix(N, K) for _ in range(copies)]
    x = (torch.randn((1, K), device="cuda", generator=torch.Generator(device="cuda")
                     .manual_seed(1)) * 0.1).half()
    parts = torch.ones((1, K // 4), device="cuda")
    y = torch.empty((1, N), device="cuda")
    ep = L.Epilogue(mode=L.EPI_STORE, norm_parts=parts.data_ptr(), n_parts=K // 4,
                    ld_parts_in=K // 4, norm_count=K, eps=1e-5, norm_mult=32.0)
    algo = mats[0].nbytes + K * 2 + (K // 4) * 4 + N * 4
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for m in mats:
            ops.gemv(m, x, out=y, epilogue=ep)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for m in mats:
                ops.gemv(m, x, out=y, epilogue=ep)
    torch.cuda.synchronize()
    # warm up for a third of a second: the first launches after the
    # matrices are made run slower
    t_end = time.time() + 0.33
    n_warm = 0
    while n_warm < max(3, args.warmup) or time.time() < t_end:
        g.replay()
        torch.cuda.synchronize()
        n_warm += 1
    reps = max(10, args.steps // 2)
    ms_graph = timed(g.replay, reps)
    us = ms_graph * 1e3 / copies
    gbps = algo / (us * 1e-6) / 1e9
    cpu = None
    if not args.no_cpu:
        threads = host_threads()[0]
        m = mats[0]
        wm = O.WideMatrix(m.N, m.K, 8 if m.layout == L.LAYOUT_Q8 else 6)
        wm.quants[:] = m.quants.cpu().numpy()
        wm.scales[:] = m.scales.cpu().numpy().view(np.uint16)
        x16 = x.cpu().numpy().view(np.uint16)
        wm.matmul(x16, threads)
        spent, n = 0.0, 0
        while spent < 10.0 or n < 2:
            t0 = O.now()
            wm.matmul(x16, threads)
            spent += O.now() - t0
            n += 1
        cpu = {"value": round(algo / (spent / n) / 1e9, 3), "unit": "GB/s", "cores": threads,
               "kind": "port",
               "sample": f"oracle float32 block form of the reference's shader (OpenMP, "
                         f"{threads} threads) on one {N}x{K} matrix, 1 row, {n} repetitions "
                         f"({spent:.1f} s)"}
    kname = "gemv_wide_stream_kernel<Q6K>" if fmt == "q6_k" else "gemv_wide_stream_kernel<Q8>"
    roof = {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None,
            "kernel": f"{kname} {N}x{K} ({what}), prescaled-norm input",
            "bytes_per_launch": algo, "avg_launch_us": round(us, 3), "launches": reps * copies}
    cfg = {"workload": f"{what}: {fmt} GEMV {N}x{K} batch 1, {copies} distinct matrices in "
                       f"one captured graph", "global_batch": 1, "parallelism": "none"}
    return line(f"{fmt} GEMV HBM GB/s", round(gbps, 1), "GB/s", reps * copies, args.warmup,
                ms_graph / copies, cfg, roof, cpu)


def workload_q6_k_head(args):
    """The Llama-3-8B output head as a Q4_K_M GGUF stores it (Q6_K,
    128256 x 4096, 431 MB a copy)."""
    return workload_wide_gemv(args, "q6_k", 128256, 4096, 2, "Llama-3-8B Q6_K output head")


def workload_q8_gemv(args):
    """The 8B gate|up matrix (28672 x 4096) requantized to 8 bits, as the
    reference's GGUF loader stores tensors it does not keep in 4 bits."""
    return workload_wide_gemv(args, "q8", 28672, 4096, 8, "Llama-3-8B gate|up, 8-bit")


def workload_gguf_load(args):
    """Loading an LFM2-1.2B-shape GGUF (16 layers, 10 of them short conv;
    Q4_0 layer matrices and a Q6_K embedding as Liquid AI's files have them)
    from a file into the engine's device layout: read through the library's
    memory-mapped reader, copied over, repacked on the GPU. GB/s of file
    bytes, best of a few loads of the page-cached file."""
    import tempfile
    import numpy as np
    import torch
    from tests import gguf_writer as W
    from webgllm_amd import load_gguf as LG, ops
    D, layers, heads, kv, hd, F, V = 2048, 16, 32, 8, 64, 8192, 65536
    conv = (0, 1, 3, 4, 6, 7, 9, 11, 13, 15)
    rng = np.random.default_rng(0)

    def q4_0(rows, K):
        b = rng.integers(0, 256, (rows * K // 32, 18), dtype=np.uint8)
        h = rng.uniform(0.002, 0.006, b.shape[0]).astype(np.float16).view(np.uint16)
        b[:, 0], b[:, 1] = h & 255, h >> 8
        return b

    tensors = []
    for i in range(layers):
        p = f"blk.{i}."
        for n in ("attn_norm", "ffn_norm"):
            tensors.append((p + n + ".weight", (D,), 0, np.ones(D, np.float32)))
        if i in conv:
            tensors += [(p + "shortconv.in_proj.weight", (D, 3 * D), 2, q4_0(3 * D, D)),
                        (p + "shortconv.out_proj.weight", (D, D), 2, q4_0(D, D)),
                        (p + "shortconv.conv.weight", (3, D), 0,
                         rng.standard_normal(3 * D).astype(np.float32))]
        else:
            tensors += [(p + "attn_q.weight", (D, heads * hd), 2, q4_0(heads * hd, D)),
                        (p + "attn_k.weight", (D, kv * hd), 2, q4_0(kv * hd, D)),
                        (p + "attn_v.weight", (D, kv * hd), 2, q4_0(kv * hd, D)),
                        (p + "attn_output.weight", (heads * hd, D), 2, q4_0(D, heads * hd)),
                        (p + "attn_q_norm.weight", (hd,), 0, np.ones(hd, np.float32)),
                        (p + "attn_k_norm.weight", (hd,), 0, np.ones(hd, np.float32))]
        tensors += [(p + "ffn_gate.weight", (D, F), 2, q4_0(F, D)),
                    (p + "ffn_up.weight", (D, F), 2, q4_0(F, D)),
                    (p + "ffn_down.weight", (F, D), 2, q4_0(D, F))]
    tensors.append(("token_embd_norm.weight", (D,), 0, np.ones(D, np.float32)))
    emb = rng.integers(0, 256, (V * D // 256, 210), dtype=np.uint8)
    h = rng.uniform(1e-5, 2e-5, emb.shape[0]).astype(np.float16).view(np.uint16)
    emb[:, 208], emb[:, 209] = h & 255, h >> 8
    tensors.append(("token_embd.weight", (D, V), 14, emb))
    kvs = [0 if i in conv else kv for i in range(layers)]
    meta = [("general.architecture", W.STRING, "lfm2"), ("lfm2.block_count", W.U32, layers),
            ("lfm2.embedding_length", W.U32, D), ("lfm2.attention.head_count", W.U32, heads),
            ("lfm2.attention.head_count_kv", W.ARRAY, (W.I32, kvs)),
            ("lfm2.feed_forward_length", W.U32, F), ("lfm2.rope.freq_base", W.F32, 1e6),
            ("lfm2.attention.layer_norm_rms_epsilon", W.F32, 1e-5),
            ("lfm2.shortconv.l_cache", W.U32, 3)]
    path = os.path.join(tempfile.mkdtemp(), "lfm2-1.2b-shape-q4_0.gguf")
    W.write_gguf(path, meta, tensors)
    size = os.path.getsize(path)
    del tensors
    times = []
    for _ in range(3):
        torch.cuda.synchronize()
        t0 = time.time()
        w = LG.load_gguf(path)
        torch.cuda.synchronize()
        times.append(time.time() - t0)
        del w
    best = min(times)
    gbps = size / best / 1e9
    # the dominant kernel: packQ4_0 of one gate|up-sized matrix, HIP events
    src = torch.from_numpy(q4_0(2 * F, D).reshape(-1)).cuda()
    m = ops.Q4Matrix(2 * F, D)
    m.repack_q4_0(0, 2 * F, src)
    ms = timed(lambda: m.repack_q4_0(0, 2 * F, src), 20)
    kbytes = 2 * src.numel()  # block bytes read, the same written
    kgbps = kbytes / (ms * 1e-3) / 1e9
    roof = {"bound": "hbm", "achieved": round(kgbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(kgbps / HBM_PEAK_GBPS, 4), "traffic": None,
            "kernel": f"repack_q4_0_kernel {2 * F}x{D} (packQ4_0: 18-byte blocks read, "
                      f"written as 16-byte rows + half scales)",
            "bytes_per_launch": kbytes, "avg_launch_us": round(ms * 1e3, 2), "launches": 20}
    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O
        blocks = q4_0(2 * F, D).reshape(-1)
        qm = O.QuantMatrix(2 * F, D)
        spent, n = 0.0, 0
        while spent < 5.0 or n < 2:
            t0 = O.now()
            O.pack_q4_0(qm, 0, blocks, 2 * F)
            spent += O.now() - t0
            n += 1
        cpu = {"value": round(blocks.size / (spent / n) / 1e9, 3), "unit": "GB/s", "cores": 1,
               "kind": "port", "sample": f"oracle packQ4_0 (one thread) of one {2 * F}x{D} "
                                         f"matrix, {n} repetitions ({spent:.1f} s)"}
    cfg = {"workload": f"LFM2-1.2B-shape GGUF ({size / 1e9:.2f} GB: Q4_0 layer matrices, "
                       f"Q6_K embedding) loaded into the device layout, page-cached file",
           "loads_s": [round(t, 3) for t in times], "parallelism": "none"}
    return line("GGUF load GB/s (file bytes into the device layout)", round(gbps, 2), "GB/s",
                3, 0, best * 1e3, cfg, roof, cpu, dtype="u8")


def workload_sample_pick(args):
    """The sampling pick of one Llama-3-8B-vocabulary row (128256 logits):
    wg_pick_candidates with a repetition and presence penalty and a window
    of 64 seen tokens, the best 64 chunks (16384 candidates) gathered; then
    their read-back and the host sampler (top-k 40, top-p 0.95, temperature
    0.8). Microseconds a pick."""
    import numpy as np
    import torch
    from webgllm_amd import lib as L, ops
    from webgllm_amd.sampler import GpuPick, Sampler, draw
    V, count = 128256, 64
    g = torch.Generator(device="cuda").manual_seed(3)
    logits = torch.randn((1, V), device="cuda", generator=g) * 3
    mask = torch.zeros(V, dtype=torch.uint8, device="cuda")
    mask[torch.randint(0, V, (64,), device="cuda", generator=g)] = 1
    scratch = torch.empty(int(L.load().wg_pick_scratch_bytes(1, V)), dtype=torch.uint8,
                          device="cuda")

    chunks_out = torch.empty((1, count), dtype=torch.int32, device="cuda")
    cand_out = torch.empty((1, count, 256), device="cuda")
    lib = L.load()
    stream = torch.cuda.current_stream().cuda_stream

    def launch():  # the C call alone, outputs preallocated
        L.check(lib.wg_pick_candidates(logits.data_ptr(), 1, V, V, mask.data_ptr(), None, 0, 0,
                                       1.1, 0.2, None, 0, 0, count, chunks_out.data_ptr(),
                                       cand_out.data_ptr(), scratch.data_ptr(), scratch.numel(),
                                       stream))
    for _ in range(20):
        launch()
    reps = max(100, 4 * args.steps)
    ms = timed(launch, reps)
    algo = V * 4 + V + 2 * count * 256 * 4 + count * 4  # logits, mask, gather reread + out
    gbps = algo / (ms * 1e-3) / 1e9
    s = Sampler(0.8, 40, top_p=0.95, repetition_penalty=1.1, presence_penalty=0.2)
    gp = GpuPick(V, count)
    gp.mask.copy_(mask)
    r = np.random.default_rng(0)
    for _ in range(20):
        draw(gp(logits[0], s), r.random)
    t0 = time.time()
    n = 200
    for _ in range(n):
        draw(gp(logits[0], s), r.random)
    host_ms = (time.time() - t0) * 1e3 / n
    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O
        lg, mk = logits.cpu().numpy(), mask.cpu().numpy()
        spent, k = 0.0, 0
        while spent < 5.0 or k < 2:
            t1 = O.now()
            O.pick_candidates(lg, count, mask=mk, penalty=1.1, presence=0.2)
            spent += O.now() - t1
            k += 1
        cpu = {"value": round(spent / k * 1e6, 1), "unit": "us", "cores": 1, "kind": "port",
               "sample": f"oracle restatement of the pick (one thread), the same row, {k} "
                         f"repetitions ({spent:.1f} s)"}
    roof = {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 5), "traffic": None,
            "kernel": "chunk_max_kernel + chunk_gather_kernel (one row, 128256 logits, 64 chunks)",
            "bytes_per_launch": algo, "avg_launch_us": round(ms * 1e3, 2), "launches": reps}
    cfg = {"workload": "sampling pick of one 128256-logit row: penalties, best 64 chunks, "
                       "then the host sampler", "pick_and_sample_ms": round(host_ms, 3),
           "parallelism": "none"}
    return line("sampling pick us (128256-logit row, 64 chunks)", round(ms * 1e3, 2), "us",
                reps, 20, ms, cfg, roof, cpu, higher_is_better=False)


def workload_delta_rule(args):
    """A Qwen3.5-shaped Gated DeltaNet layer's recurrence (16 heads, key and
    value dims 128): wg_delta_rule for one decode row, cycling over 320
    layers' states (320 MB, past the 256 MB MALL, so every launch reads its
    state from HBM); also a 2048-row prompt batch in one launch.
    Microseconds a decode row."""
    import ctypes as C
    import torch
    from webgllm_amd import lib as L
    H, dk, dv = 16, 128, 128
    K, V = H * dk, H * dv
    layers = 320
    g = torch.Generator(device="cuda").manual_seed(5)
    states = torch.randn((layers, H, dk, dv), device="cuda", generator=g) * 0.1
    qkv = torch.randn((2048, 2 * K + V), device="cuda", generator=g)
    ba = torch.randn((2048, 2 * H), device="cuda", generator=g)
    A = -torch.rand(H, device="cuda", generator=g) - 0.5
    dt = torch.randn(H, device="cuda", generator=g) * 0.5
    out = torch.empty((2048, V), device="cuda")
    lib = L.load()
    shape = L.DeltaShape(H, dk, dv)

    def launch(st, M, stream):
        L.check(lib.wg_delta_rule(qkv.data_ptr(), M, qkv.stride(0), ba.data_ptr(), ba.stride(0),
                                  A.data_ptr(), dt.data_ptr(), C.byref(shape), st.data_ptr(),
                                  None, 0, out.data_ptr(), out.stride(0), stream))
    # One decode row for each of the 320 layers' states, captured in a graph
    # so that the host's call overhead is not what gets timed.
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        launch(states[0], 1, side.cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(graph):
        cur = torch.cuda.current_stream().cuda_stream
        for layer in range(layers):
            launch(states[layer], 1, cur)
    for _ in range(2):
        graph.replay()
    reps = max(4, args.steps // 8)
    ms = timed(graph.replay, reps) / layers
    state_bytes = H * dk * dv * 4
    algo = 2 * state_bytes + (2 * K + V) * 4 + 2 * H * 4 + V * 4  # state in and out, row, out
    gbps = algo / (ms * 1e-3) / 1e9
    cur = torch.cuda.current_stream().cuda_stream
    for _ in range(3):
        launch(states[0], 2048, cur)
    pf_ms = timed(lambda: launch(states[0], 2048, cur), 10)
    need = int(lib.wg_delta_chunk_scratch_bytes(2048, C.byref(shape), 0))
    scratch = torch.empty(need // 4 + 4, device="cuda")

    def chunked():
        L.check(lib.wg_delta_rule_chunked(
            qkv.data_ptr(), 2048, qkv.stride(0), ba.data_ptr(), ba.stride(0), A.data_ptr(),
            dt.data_ptr(), C.byref(shape), states[0].data_ptr(), None, 0, out.data_ptr(),
            out.stride(0), scratch.data_ptr(), need, cur))
    for _ in range(3):
        chunked()
    pf_chunked_ms = timed(chunked, 10)
    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O
        q1, b1 = qkv[:1].cpu().numpy(), ba[:1].cpu().numpy()
        a1, d1, s1 = A.cpu().numpy(), dt.cpu().numpy(), states[0].cpu().numpy()
        spent, k = 0.0, 0
        while spent < 5.0 or k < 2:
            t1 = O.now()
            O.delta_rule(q1, b1, a1, d1, H, dk, dv, s1)
            spent += O.now() - t1
            k += 1
        cpu = {"value": round(spent / k * 1e6, 1), "unit": "us", "cores": 1, "kind": "port",
               "sample": f"oracle restatement of the recurrence for one row (float64, one "
                         f"thread), {k} repetitions ({spent:.1f} s)"}
    roof = {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None,
            "kernel": "delta_rule_kernel<16> (one row, 16 heads of 128, state from HBM)",
            "bytes_per_launch": algo, "avg_launch_us": round(ms * 1e3, 2),
            "launches": reps * layers}
    cfg = {"workload": "Gated DeltaNet recurrence of one Qwen3.5-shaped layer (16 heads, "
                       "key/value dims 128), one decode row", "heads": H, "key_dim": dk,
           "value_dim": dv, "prompt_rows": 2048, "prompt_ms": round(pf_ms, 3),
           "prompt_rows_per_s": round(2048 / (pf_ms * 1e-3)),
           "prompt_chunked_ms": round(pf_chunked_ms, 3),
           "prompt_chunked_rows_per_s": round(2048 / (pf_chunked_ms * 1e-3)),
           "parallelism": "none"}
    return line("Gated DeltaNet recurrence us a decode row (16 heads of 128)",
                round(ms * 1e3, 2), "us", reps * layers, 3 * layers, ms, cfg, roof, cpu,
                higher_is_better=False)


def workload_onnx_load(args):
    """Loading the MatMulNBits weights of an LFM2-350M q4f16 ONNX export
    (the onnxruntime-genai graph, with zero points) into the device layout:
    the graph read by the library's reader, each weight's quants, scales and
    zero points read from the external data file and repacked on the GPU
    (wg_repack_nbits). The data file holds random weights at the graph's
    offsets. GB/s of weight bytes, best of a few loads of the page-cached
    file."""
    import shutil
    import tempfile
    import numpy as np
    import torch
    from webgllm_amd.onnx import OnnxFile, OnnxModel, upload_nbits
    src = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tests", "golden", "onnx",
                       "lfm2-350m", "model_q4f16.onnx")
    d = tempfile.mkdtemp()
    graph = os.path.join(d, "model_q4f16.onnx")
    shutil.copy(src, graph)
    f = OnnxFile(graph)
    m = OnnxModel(f)
    paths = sorted({n.name.rsplit("/", 1)[0] + "/" for n in f.nodes
                    if n.op_type == "MatMulNBits"})
    weights = [m.nbits(p) for p in paths]
    rng = np.random.default_rng(0)
    total = 0
    with open(os.path.join(d, "model_q4f16.onnx_data"), "wb") as out:
        for w in weights:
            for t in (w.quant, w.scales, w.zp):
                if t is None:
                    continue
                n = t.external[2]
                if t is w.scales:
                    data = rng.uniform(0.002, 0.02, n // 2).astype(np.float16).view(np.uint8)
                else:
                    data = rng.integers(0, 256, n, dtype=np.uint8)
                out.seek(t.external[1])
                out.write(data.tobytes())
                total += n
    times = []
    for _ in range(3):
        torch.cuda.synchronize()
        t0 = time.time()
        mats = [upload_nbits(f, w) for w in weights]
        torch.cuda.synchronize()
        times.append(time.time() - t0)
        del mats
    best = min(times)
    gbps = total / best / 1e9
    f.close()
    shutil.rmtree(d, ignore_errors=True)
    cfg = {"workload": "LFM2-350M q4f16 ONNX export's MatMulNBits weights (random values at "
                       "the graph's offsets) into the device layout",
           "matrices": len(weights), "weight_bytes": total,
           "load_s": [round(t, 3) for t in times], "parallelism": "none"}
    return line("ONNX MatMulNBits load GB/s (LFM2-350M export)", round(gbps, 2), "GB/s", 3, 0,
                best * 1e3, cfg, None, None)


WORKLOADS = {"q4_0-gemv": workload_q4_0_gemv, "nbits-gemm": workload_nbits_gemm,
             "sample-pick": workload_sample_pick, "delta-rule": workload_delta_rule,
             "gguf-load": workload_gguf_load, "onnx-load": workload_onnx_load,
             "q8-gemm": lambda args: workload_nbits_gemm(args, "q8"),
             "q6_k-head": workload_q6_k_head, "q8-gemv": workload_q8_gemv,
             "qwen2-decode": workload_qwen2_decode, "lfm2-verify": workload_lfm2_verify,
             "llama8b-prefill": workload_llama8b_prefill}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--layers", type=int, default=None, help=argparse.SUPPRESS)
    ap.add_argument("--roofline-only", action="store_true",
                    help="only the gate|up GEMV launches and a copy (for counter runs)")
    ap.add_argument("--reps", type=int, default=6, help=argparse.SUPPRESS)
    ap.add_argument("--workload", default="llama8b-decode",
                    choices=["llama8b-decode"] + sorted(WORKLOADS),
                    help="the headline Llama-3-8B-shape decode (default) or another "
                         "configuration's measurement")
    ap.add_argument("--tuning", action="append", default=[], metavar="NAME=VALUE",
                    help="set a launch-shape knob of the library (wg_tuning_set) first")
    args = ap.parse_args()
    for kv in args.tuning:
        from webgllm_amd import lib as _L
        name, value = kv.split("=")
        _L.check(_L.load().wg_tuning_set(name.encode(), int(value)))
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(--gpus {args.gpus} asked)", file=sys.stderr)
        sys.exit(2)
    if args.roofline_only:
        roofline_only(args)
        return
    if args.workload != "llama8b-decode":
        print(json.dumps(WORKLOADS[args.workload](args)), flush=True)
        return

    import dataclasses

    import torch

    from webgllm_amd import engine as E

    shape = E.LLAMA3_8B
    if args.layers:
        shape = dataclasses.replace(shape, layers=args.layers)
    t0 = time.time()
    w = E.Weights(shape, seed=0)
    eng = E.Engine(w, args.ctx)
    prompt_len = args.ctx - args.warmup - args.steps - 1
    rng = torch.Generator().manual_seed(1)
    prompt = torch.randint(0, shape.vocab, (prompt_len,), generator=rng).tolist()
    picks = eng.forward(prompt)
    # the timed replays run past what decode() reserves: room for all of them
    eng.reserve(args.ctx)
    torch.cuda.synchronize()
    t_prefill = time.time() - t0
    first = int(picks[-1])
    eng.capture_step(first)
    # warmup, then exactly `steps` timed tokens
    eng.decode(first, args.warmup)
    last = int(eng.hist[eng.position].item())
    stream = torch.cuda.current_stream()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    p0 = eng.position
    eng.ids[0] = last
    eng.pos.fill_(p0)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(args.steps):
        eng.graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    eng.position += args.steps
    ms = e0.elapsed_time(e1) / args.steps
    tok_s = 1000.0 / ms

    roof = gemv_roofline([lw["gate_up"] for lw in w.layers], eng.x16[:1], eng.parts[:1],
                         eng.ff16[:1], shape.eps)
    # keys a timed token attends over, on average (positions p0 .. p0 + steps - 1)
    keys = p0 + (args.steps + 1) // 2
    tok_bytes = token_bytes(shape, keys)
    kv_bytes = shape.layers * 2 * shape.kv_heads * shape.head_dim * 2 * keys
    stored_bytes = w.nbytes + kv_bytes
    cpu = None
    if not args.no_cpu:
        threads = host_threads()[0]
        cpu = cpu_baseline(eng, threads, keys=keys)
    out = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "Llama-3-8B-shape Q4_K batch-1 greedy decode, fp16 KV cache 4096 "
                        f"(timed positions {p0}..{p0 + args.steps - 1})",
            "model": shape.name, "layers": shape.layers, "hidden": shape.hidden,
            "vocab": shape.vocab,
            "weights": "random GGUF Q4_K super-blocks, repacked on the GPU to the "
                       "reference's 32-blocks (packQ4_K's quants) with Q4_K's own scales and "
                       "mins kept in 64-byte records a row group (0.5625 bytes a weight)",
            "activations": "f16", "accumulate": "f32",
            "global_batch": 1, "seq_len": args.ctx, "parallelism": "none",
        },
        "roofline": roof,
        "cpu_baseline": cpu,
        # a token's algorithmic bytes: Q4_K weights at 144 B / 256, the
        # keys and values of the cache rows it reads, activations
        "token_bytes": tok_bytes,
        "token_roofline_tok_s": round(HBM_PEAK_GBPS * 1e9 / tok_bytes, 1),
        "token_roofline_ratio": round(HBM_PEAK_GBPS * 1e9 / tok_bytes / tok_s, 3),
        "decode_effective_GBps": round(tok_bytes / (ms * 1e-3) / 1e9, 1),
        "stored_layout_token_bytes": stored_bytes,
        "setup_s": round(t_prefill, 1),
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
