"""Headline benchmark: batch-1 Q4 decode of the Llama-3-8B-shaped model
(hidden 4096, 32 layers, 32/8 heads of 128, intermediate 14336, vocab
128256, GGUF Q4_K weights repacked at load as the reference does, fp16 KV
cache of 4096) on one MI355X.

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


def gemv_roofline(mats, x, parts, out16, eps, reps=6):
    """Average duration of the gate|up GEMV, launched as the decode launches
    it (prescaled norm in, SwiGLU out), over distinct matrices."""
    import torch
    from webgllm_amd import lib as L, ops
    m = mats[0]
    F, D = m.N // 2, m.K
    ep = L.Epilogue(mode=L.EPI_SWIGLU, out16=out16.data_ptr(), ld_out16=F,
                    norm_parts=parts.data_ptr(), n_parts=D // 4, ld_parts_in=D // 4,
                    norm_count=D, eps=eps, norm_mult=32.0)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for mm in mats[:4]:
            ops.gemv(mm, x, epilogue=ep)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            for mm in mats:
                ops.gemv(mm, x, epilogue=ep)
        e1.record(stream)
    stream.synchronize()
    launches = reps * len(mats)
    us = e0.elapsed_time(e1) * 1e3 / launches
    # weights (nibbles, half scales, half zero points) + x (halves) + the
    # norm's parts + the half SwiGLU output
    algo = m.nbytes + D * 2 + (D // 4) * 4 + F * 2
    achieved = algo / (us * 1e-6) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": measured_traffic(),
            "kernel": f"gemv_stream_kernel gate|up {m.N}x{m.K} (Q4_K repacked: 4-bit + "
                      f"half scale + half zero per 32), SwiGLU epilogue",
            "bytes_per_launch": algo, "avg_launch_us": round(us, 3), "launches": launches}


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
    qm = O.QuantMatrix(m.N, m.K, {L.ZERO_8: False, L.ZERO_U8: True, L.ZERO_F16: "halves"}[m.zero])
    qm.quants[:] = m.quants.cpu().numpy().view(np.uint32)
    qm.scales[:] = m.scales.cpu().numpy().view(np.uint16)
    if m.zero == L.ZERO_U8:
        qm.zeros[:] = m.zeros.cpu().numpy()
    elif m.zero == L.ZERO_F16:
        qm.zero_halves[:] = m.zeros.cpu().numpy().view(np.uint16)
    return qm


def cpu_baseline(engine, threads, seconds=12.0):
    """Oracle split matmul (float32, shader order) on one layer + the head,
    repeated for about `seconds` of CPU time."""
    import numpy as np
    from oracle import oracle as O
    s = engine.shape
    lw = engine.w.layers[0]
    layer = [oracle_matrix(lw[k]) for k in ("qkv", "o", "gate_up", "down")]
    head = oracle_matrix(engine.w.embedding)
    rng = np.random.default_rng(0)
    xs = {m.K: O.f32_to_h2(rng.standard_normal((1, m.K)).astype(np.float32))
          for m in layer + [head]}
    O.matmul_split(layer[0], xs[layer[0].K], threads)  # warm the threads
    # repeat the layer + head sample until about `seconds` of CPU work is done
    t_layer = t_head = 0.0
    reps = 0
    while reps < 400 and (t_layer + t_head < seconds or reps < 2):
        t0 = O.now()
        for m in layer:
            O.matmul_split(m, xs[m.K], threads)
        t1 = O.now()
        O.matmul_split(head, xs[head.K], threads)
        t_layer += t1 - t0
        t_head += O.now() - t1
        reps += 1
    per_token = (s.layers * t_layer + t_head) / reps
    return {"value": round(1.0 / per_token, 4), "unit": "tok/s", "cores": threads,
            "kind": "port",
            "sample": f"oracle shader-order fp32 split matmul (OpenMP, {threads} threads) on "
                      f"layer 0's qkv/o/gate|up/down and the 128256x4096 head at batch 1, "
                      f"{reps} repetitions ({t_layer + t_head:.1f} s: {t_layer / reps * 1e3:.1f} ms "
                      f"a layer, {t_head / reps * 1e3:.1f} ms the head), extrapolated to 32 "
                      f"layers; attention and norms not included"}


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
    ap.add_argument("--persistent", action="store_true",
                    help="decode every layer in one persistent launch (wg_decode_run)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(--gpus {args.gpus} asked)", file=sys.stderr)
        sys.exit(2)
    if args.roofline_only:
        roofline_only(args)
        return

    import dataclasses

    import torch

    from webgllm_amd import engine as E

    shape = E.LLAMA3_8B
    if args.layers:
        shape = dataclasses.replace(shape, layers=args.layers)
    t0 = time.time()
    w = E.Weights(shape, seed=0)
    eng = E.Engine(w, args.ctx, persistent=args.persistent)
    prompt_len = args.ctx - args.warmup - args.steps - 1
    rng = torch.Generator().manual_seed(1)
    prompt = torch.randint(0, shape.vocab, (prompt_len,), generator=rng).tolist()
    picks = eng.forward(prompt)
    torch.cuda.synchronize()
    t_prefill = time.time() - t0
    first = int(picks[-1])
    eng.capture_step()
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
    kv_bytes = shape.layers * 2 * shape.kv_heads * shape.head_dim * 2 * (p0 + args.steps // 2)
    token_bytes = w.nbytes + kv_bytes
    cpu = None
    if not args.no_cpu:
        threads = min(os.cpu_count() or 1, 16)
        cpu = cpu_baseline(eng, threads)
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
                       "reference's 32-blocks (packQ4_K)",
            "activations": "f16", "accumulate": "f32",
            "global_batch": 1, "seq_len": args.ctx, "parallelism": "none",
            "decode_path": "persistent" if eng.plan is not None else "per-op kernels",
        },
        "roofline": roof,
        "cpu_baseline": cpu,
        "token_bytes": token_bytes,
        "token_roofline_tok_s": round(HBM_PEAK_GBPS * 1e9 / token_bytes, 1),
        "decode_effective_GBps": round(token_bytes / (ms * 1e-3) / 1e9, 1),
        "setup_s": round(t_prefill, 1),
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
