#!/usr/bin/env python3
"""Benchmark of the quantized-matmul hot path on one MI355X.

Headline workload: Qwen3-235B-shape attention projections,
decode batch 1, hidden 4096.  One step = the projections of all 94 layers for one token:
Q Q4_K 4096->8192 with K (Q4_K) + V (Q6_K) 4096->512 each in one launch
(mnemo_matvec_qkv), then O Q4_K 8192->4096 with fp32 residual -- 188 launches over
3.83 GB of distinct weights (so the 256 MB MALL cannot serve them), captured once in a
hipGraph and replayed.  value = algorithmic bytes per step / step time (GB/s), inputs
resident in HBM.  The Q / dual K+V split the reference engine uses is timed beside it.

Also reported (secondary, same JSON line under "extra"): the M=512 Q4_K prefill GEMM
(TOPS vs the 5.0 POP/s int8 peak) and per-kernel GEMV bandwidths.

cpu_baseline: a vectorised fp32 dequant+dot port of the reference arithmetic
(oracle/cpu_baseline.c, AVX-512 or AVX2 build by the host CPU) over one layer's attention
projections, rows split over every host core this process may use, plus a single-core run,
timed for a bounded ~10 s sample.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
# The GEMM's exact per-sub-block arithmetic needs one fp32 rescale (a VALU lane-op) per output and
# 32-value sub-block: 32 MACs per lane-op at 16 lane-ops per clock per SIMD caps it at the dense
# f16 MFMA rate, 2.5 POP/s (the semantics' own roof, beside the 5.0 POP/s int8 peak).
F16_ROOF_TOPS = 2500.0
GEMM_ROTATE_BYTES = 600 << 20
CPU_ROTATE_LAYERS = 16  # host copies of one layer's weights, 653 MB: more than the host's L3
H, QD, KVD, LAYERS = 4096, 8192, 512, 94
Q4K, Q6K = 12, 14


def rb(t, cols):
    return (cols + 255) // 256 * (144 if t == Q4K else 210)


# algorithmic bytes per call: weights + x + y (+ residual)
BYTES_Q = QD * rb(Q4K, H) + 4 * H + 4 * QD
BYTES_KV = KVD * rb(Q4K, H) + KVD * rb(Q6K, H) + 4 * H + 2 * 4 * KVD
BYTES_O = H * rb(Q4K, QD) + 4 * QD + 4 * H + 4 * H
BYTES_QKV = BYTES_Q + BYTES_KV - 4 * H  # x read once
BYTES_LAYER = BYTES_QKV + BYTES_O


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-gemm", action="store_true")
    ap.add_argument("--no-moe", action="store_true")
    ap.add_argument("--no-decode", action="store_true", help="skip the full decode-step tok/s (147 GB of experts)")
    ap.add_argument("--decode-tokens", type=int, default=20)
    ap.add_argument("--decode-pos", type=int, default=2048, help="KV-cache position of the first decoded token")
    ap.add_argument("--decode-long-pos", type=int, default=32768,
                    help="a second position the same graph is timed at (long-context decode; 0: skip)")
    ap.add_argument("--decode-max-ctx", type=int, default=40960,
                    help="KV-cache allocation in positions (the model's context length, as a server allocates it)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="end with a 256 MiB device copy (torch.neg) whose HBM counters scale rocprofv3 "
                         "FETCH_SIZE/WRITE_SIZE readings (mnemocuda_amd/profiling.py)")
    return ap.parse_args()


def time_launches(fn, n, stream, reps=5):
    """Average device time per launch of fn(i), i = 0..n-1, captured back to back in one
    hipGraph and replayed reps times between two HIP events on the launch stream (the
    launch-to-launch time of a dependent chain; rocprof's per-kernel duration excludes
    only the short gap between kernels)."""
    import torch
    with torch.cuda.stream(stream):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for i in range(n):
                fn(i)
        g.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(reps):
            g.replay()
        b.record(stream)
        torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e-3 / (reps * n)


def time_eager(fn, n, stream):
    """Average device time per call of fn(i) for calls long enough that the host stays
    ahead: n calls enqueued back to back between two HIP events."""
    import torch
    with torch.cuda.stream(stream):
        fn(0)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for i in range(n):
            fn(i)
        b.record(stream)
        torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e-3 / n


def gpu_bench(args):
    import torch
    import mnemocuda_amd as m
    from mnemocuda_amd import ops, synth

    torch.cuda.set_device(0)
    ops.init()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1234)
    dev = torch.device("cuda")
    layers = []
    for _ in range(LAYERS):
        layers.append(dict(
            q=synth.weights_torch(gen, Q4K, QD, H, dev),
            k=synth.weights_torch(gen, Q4K, KVD, H, dev),
            v=synth.weights_torch(gen, Q6K, KVD, H, dev),
            o=synth.weights_torch(gen, Q4K, H, QD, dev),
        ))
    x = torch.randn(H, device=dev, generator=gen)
    res = torch.randn(H, device=dev, generator=gen)
    q, k, v = torch.empty(QD, device=dev), torch.empty(KVD, device=dev), torch.empty(KVD, device=dev)
    hid = torch.empty(H, device=dev)
    attn = torch.randn(QD, device=dev, generator=gen)
    torch.cuda.synchronize()

    def step():
        for L in layers:
            ops.matvec_qkv(L["q"], Q4K, L["k"], Q4K, L["v"], Q6K, x, q, k, v, QD, KVD, H)
            ops.matvec_q4k_add(L["o"], attn, res, hid, H, QD)

    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        step()  # eager once (also validates arguments outside capture)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            step()
        for _ in range(args.warmup):
            g.replay()
        torch.cuda.synchronize()
        # untimed replays until at least 100 ms of warm-up have run, so that the clocks have
        # settled before the timed steps whatever W is (W = 3: 2.93 TB/s; 200: 2.97 TB/s)
        warm0 = time.perf_counter()
        while time.perf_counter() - warm0 < 0.1:
            for _ in range(8):
                g.replay()
            torch.cuda.synchronize()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record(s)
        wall0 = time.perf_counter()
        for _ in range(args.steps):
            g.replay()
        t1.record(s)
        torch.cuda.synchronize()
        wall = time.perf_counter() - wall0
        step_s = t0.elapsed_time(t1) * 1e-3 / args.steps

        # per-kernel durations (HIP events on the launch stream), rotating over layers
        n = LAYERS
        d_qkv = time_launches(lambda i: ops.matvec_qkv(layers[i]["q"], Q4K, layers[i]["k"], Q4K, layers[i]["v"], Q6K,
                                                       x, q, k, v, QD, KVD, H), n, s)
        d_q = time_launches(lambda i: ops.matvec_q4k(layers[i]["q"], x, q, QD, H), n, s)
        d_kv = time_launches(lambda i: ops.matvec_dual(layers[i]["k"], Q4K, layers[i]["v"], Q6K, x, k, v, KVD, H), n, s)
        d_o = time_launches(lambda i: ops.matvec_q4k_add(layers[i]["o"], attn, res, hid, H, QD), n, s)

        gemm = None
        if not args.no_gemm:
            M_TOK = 512
            acts = torch.randn(M_TOK, H, device=dev, generator=gen)
            aq = torch.empty(M_TOK * (H // 128) * 144, dtype=torch.uint8, device=dev)
            ops.quantize_q8_1(acts, aq, H, M_TOK)
            res_g = {}
            for name, N_ in (("n8192", QD), ("n1536", 1536)):
                # distinct weight buffers over 2.3x the 256 MB MALL, rotated call by call
                nbuf = -(-GEMM_ROTATE_BYTES // (N_ * rb(Q4K, H)))
                ws = [synth.weights_torch(gen, Q4K, N_, H, dev) for _ in range(nbuf)]
                out = torch.empty(M_TOK, N_, device=dev)
                for w_ in ws[:4]:
                    ops.gemm(w_, Q4K, aq, out, N_, H, M_TOK)
                d = time_eager(lambda i: ops.gemm(ws[i % nbuf], Q4K, aq, out, N_, H, M_TOK), max(nbuf, 32), s)
                ops_ = 2.0 * M_TOK * N_ * H
                res_g[name] = {"us": d * 1e6, "tops": ops_ / d / 1e12, "frac_int8_peak": ops_ / d / 1e12 / INT8_PEAK_TOPS,
                               "frac_f16_rescale_roof": ops_ / d / 1e12 / F16_ROOF_TOPS,
                               "weight_buffers_rotated": nbuf, "weight_bytes_rotated": nbuf * N_ * rb(Q4K, H)}
                del ws
            gemm = res_g

        moe = None
        if not args.no_moe:
            moe = moe_prefill_bench(gen, s)
        decode = attn = None
        if not args.no_decode:
            attn = attention_bench(s)
            decode = decode_bench(gen, s, layers, args.decode_tokens, args.decode_pos, args.decode_max_ctx,
                                  args.decode_long_pos)
    return dict(step_s=step_s, wall=wall, d_qkv=d_qkv, d_q=d_q, d_kv=d_kv, d_o=d_o, gemm=gemm, moe=moe,
                decode=decode, attn=attn)


def decode_bench(gen, stream, layers, tokens, ctx_pos, cache_ctx=40960, long_pos=0):
    """configs[2] inside a full decode step (forward.c:687-1077 per layer, then the lm_head
    and sampling, forward.c:1601-1707), one token at cache position ctx_pos, ctx_pos+1, ...:
    per layer  fused Q/K/V with the attention RMS norm -> GQA decode attention over 0..pos
    with the QK norm, RoPE and f16 KV store in its launch (position in device memory) -> O (+ residual) ->
    MoE block with its RMS norm with device-side dispatch (router 128 x 4096 fp32, top-8, gate+up
    Q4_K 4096->1536 x 8, down Q6_K 1536->4096 x 8, weighted sum added to the residual);
    then the final norm, lm_head Q6_K 151936 x 4096 and top-p sampling.  All 128 experts of
    all 94 layers are resident (147 GB); the KV cache rows below ctx_pos hold random
    earlier tokens.  One hipGraph per token (the position advances on the device); with
    long_pos the same graph is timed again from that position (long-context decode)."""
    import torch
    from mnemocuda_amd import ops, synth
    E, k, EFF, VOCAB = 128, 8, 1536, 151936
    NH, NKV, HD, EPS, THETA = 64, 4, 128, 1e-6, 1e6
    max_ctx = max(cache_ctx, ctx_pos + tokens + 8)
    stride, g_off, u_off, d_off = synth.expert_layout(H, EFF, Q6K)
    tables = [synth.expert_table_torch(gen, E, H, EFF, Q6K, "cuda") for _ in range(LAYERS)]
    routers = [torch.randn(E, H, device="cuda", generator=gen) / 64 for _ in range(LAYERS)]
    norms = [dict(attn=1 + 0.05 * torch.randn(H, device="cuda", generator=gen),
                  ffn=1 + 0.05 * torch.randn(H, device="cuda", generator=gen),
                  q=1 + 0.05 * torch.randn(HD, device="cuda", generator=gen),
                  k=1 + 0.05 * torch.randn(HD, device="cuda", generator=gen)) for _ in range(LAYERS)]
    kcache = [(torch.randn(max_ctx * NKV * HD, device="cuda", generator=gen)).half() for _ in range(LAYERS)]
    vn = ops.v_cache_bytes(NKV, HD, max_ctx, 0, 1) // 2  # V in the blocked layout of attention_decode
    vcache = [(torch.randn(vn, device="cuda", generator=gen)).half() for _ in range(LAYERS)]
    lm_head = synth.weights_torch(gen, Q6K, VOCAB, H, "cuda")
    final_norm = 1 + 0.05 * torch.randn(H, device="cuda", generator=gen)
    X0 = torch.randn(H, device="cuda", generator=gen)
    res = torch.empty(H, device="cuda")
    hid = torch.empty(H, device="cuda")
    normed = torch.empty(H, device="cuda")
    q, kk, v = torch.empty(QD, device="cuda"), torch.empty(KVD, device="cuda"), torch.empty(KVD, device="cuda")
    attn = torch.empty(QD, device="cuda")
    logits = torch.empty(VOCAB, device="cuda")
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    pos = torch.zeros(1, dtype=torch.int32, device="cuda")
    ws = torch.zeros(ops.moe_decode_workspace_bytes(H, EFF, E, k), dtype=torch.uint8, device="cuda")
    aws = torch.empty(ops.attention_decode_workspace_bytes(NKV, max_ctx), dtype=torch.uint8, device="cuda")
    sws = torch.empty(ops.sample_workspace_bytes(), dtype=torch.uint8, device="cuda")
    scale = 1.0 / HD ** 0.5

    def token():
        bufs = (res, hid)  # the residual stream alternates between two buffers, layer by layer
        for li, L in enumerate(layers):
            n, src, dst = norms[li], bufs[li % 2], bufs[(li + 1) % 2]
            # attention norm inside the projection launch
            ops.matvec_qkv_rmsnorm(L["q"], Q4K, L["k"], Q4K, L["v"], Q6K, src, n["attn"], EPS, q, kk, v, QD, KVD, H)
            # QK norm + RoPE + KV store inside the attention launch
            ops.attention_decode_prep(q, kk, v, n["q"], n["k"], EPS, THETA, kcache[li], vcache[li], attn, NH, HD, NKV,
                                      max_ctx, pos, scale, aws, v_layout=1)
            ops.matvec_q4k_add(L["o"], attn, src, dst, H, QD)  # dst = src + W_o attn
            # dst += moe(rms_norm(dst) * ffn_norm): the norm inside the router and gate/up launches
            ops.moe_decode_rmsnorm(routers[li], tables[li], stride, g_off, u_off, d_off, Q6K, dst, n["ffn"], EPS, H,
                                   EFF, E, k, ws, dst)
        ops.rms_norm(bufs[len(layers) % 2], final_norm, normed, EPS)
        ops.matvec_q6k(lm_head, normed, logits, VOCAB, H)
        ops.sample_token_ws(logits, VOCAB, 0.7, 0.9, 12345, sws, tok)
        pos.add_(1)

    with torch.cuda.stream(stream):
        res.copy_(X0)
        pos.fill_(ctx_pos)
        token()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            token()
        for _ in range(2):
            res.copy_(X0)
            g.replay()
        torch.cuda.synchronize()
        def timed(p0):
            pos.fill_(p0)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            for t in range(tokens):
                res.copy_(X0)
                g.replay()
            b.record(stream)
            torch.cuda.synchronize()
            return a.elapsed_time(b) / tokens

        ms = timed(ctx_pos)
        # the same graph later in the context (the position lives on the device)
        long_ms = timed(long_pos) if 0 < long_pos and long_pos + tokens <= max_ctx else None
    moe_bytes = (E * H * 4 + H * 4 + E * 4) + k * (2 * EFF * (H // 256) * 144 + H * (EFF // 256) * 210)
    kv_bytes = 2 * NKV * HD * 2 * (ctx_pos + tokens // 2)  # K + V rows read per layer, mean position
    per_tok = (BYTES_LAYER + moe_bytes + kv_bytes) * LAYERS + VOCAB * (H // 256) * 210
    del tables, routers, lm_head, kcache, vcache
    torch.cuda.empty_cache()
    return {"tok_s": round(1e3 / ms, 1), "ms_per_token": round(ms, 3), "tokens": tokens,
            "context_position": ctx_pos, "cache_positions": max_ctx, "bytes_per_token": per_tok, "GBps": round(per_tok / ms / 1e6, 1),
            "frac_hbm_peak": round(per_tok / ms / 1e6 / HBM_PEAK_GBS, 4),
            "experts_resident_GB": round(E * LAYERS * stride / 1e9, 1),
            "launches_per_token": LAYERS * 7 + 5,
            "long_context": None if long_ms is None else {"context_position": long_pos, "tok_s": round(1e3 / long_ms, 1),
                                                          "ms_per_token": round(long_ms, 3)}}


def attention_bench(stream, lengths=(1024, 4096, 16384, 32768)):
    """Decode attention for one layer (64 query heads, 4 KV heads, head_dim 128, f16 cache)
    at several sequence lengths: the GQA-batched split kernel with V in the blocked layout
    (the decode path) and in the reference's row layout, and the reference-form entry point
    cuda_attention_f16kv (host sequence length, the reference's caches), graph-timed over 20
    launches."""
    import torch
    from mnemocuda_amd import ops
    NH, NKV, HD = 64, 4, 128
    out = {}
    ops.attention_reserve(20 * len(lengths))  # every captured entry-point call holds a slot
    for L in lengths:
        kc = torch.randn(L * NKV * HD, device="cuda").half()
        vc = torch.randn(L * NKV * HD, device="cuda").half()
        q = torch.randn(NH * HD, device="cuda")
        o = torch.empty(NH * HD, device="cuda")
        pos = torch.tensor([L - 1], dtype=torch.int32, device="cuda")
        ws = torch.empty(ops.attention_decode_workspace_bytes(NKV, L), dtype=torch.uint8, device="cuda")
        fast = time_launches(lambda i: ops.attention_decode(q, kc, vc, o, NH, HD, NKV, L, pos, 0.088, ws, v_layout=1),
                             20, stream)
        rows = time_launches(lambda i: ops.attention_decode(q, kc, vc, o, NH, HD, NKV, L, pos, 0.088, ws), 20, stream)
        ref = time_launches(lambda i: ops.attention(q, kc, vc, o, NH, HD, NKV, L, 0.088), 20, stream)
        kv = 2 * L * NKV * HD * 2
        out[str(L)] = {"gqa_split_us": round(fast * 1e6, 2), "gqa_split_rowsV_us": round(rows * 1e6, 2),
                       "entry_point_us": round(ref * 1e6, 2), "gqa_split_kv_GBps": round(kv / fast / 1e9, 1)}
        del kc, vc
    return out


def moe_prefill_bench(gen, stream):
    """grouped-expert prefill, 512 tokens x top-8 of 128 experts (Zipf 1.1),
    gate+up Q4_K 4096->1536, down Q6_K 1536->4096, router-weighted scatter-add."""
    import numpy as np
    import torch
    from mnemocuda_amd import ops, synth
    T, E, k, EFF = 512, 128, 8, 1536
    idx, w = synth.zipf_routing(np.random.default_rng(7), T, E, k)
    table = synth.expert_table_torch(gen, E, H, EFF, Q6K, "cuda")
    stride, g_off, u_off, d_off = synth.expert_layout(H, EFF, Q6K)
    x = torch.randn(T, H, device="cuda", generator=gen)
    out = torch.zeros(T, H, device="cuda")
    idx_d, w_d = torch.from_numpy(idx).cuda(), torch.from_numpy(w).cuda()
    ws = torch.empty(ops.moe_prefill_workspace_bytes(T, H, EFF, E, k), dtype=torch.uint8, device="cuda")

    def run(_i):
        ops.moe_prefill(table, stride, g_off, u_off, d_off, Q6K, x, idx_d, w_d, T, H, EFF, E, k, ws, out)

    for i in range(3):
        run(i)
    d = time_eager(run, 10, stream)
    active = int(np.unique(idx).size)
    flops = 2.0 * T * k * 3 * H * EFF
    wbytes = active * (stride)
    return {"us": round(d * 1e6, 1), "tops": round(flops / d / 1e12, 1),
            "frac_int8_peak": round(flops / d / 1e12 / INT8_PEAK_TOPS, 4),
            "active_experts": active, "expert_weight_GBps": round(wbytes / d / 1e9, 1)}


def cpu_baseline(seconds):
    """The reference's arithmetic on the host CPU (oracle/cpu_baseline.c: fused dequant+dot,
    fp32 accumulation, vectorised, OpenMP rows), timed on every core this process may run on
    and on one core.  A reported baseline only."""
    import numpy as np
    import oracle
    from mnemocuda_amd import synth

    b = oracle.load_baseline()
    cores = len(os.sched_getaffinity(0))
    rng = np.random.default_rng(7)
    wq = synth.weights(rng, Q4K, QD, H)
    wk = synth.weights(rng, Q4K, KVD, H)
    wv = synth.weights(rng, Q6K, KVD, H)
    wo = synth.weights(rng, Q4K, H, QD)
    x = rng.standard_normal(QD).astype(np.float32)
    # distinct copies, visited in turn, so that no pass finds its weights in the host caches
    copies = [tuple(a.copy() for a in (wq, wk, wv, wo)) for _ in range(CPU_ROTATE_LAYERS)]

    def rate(threads, budget):
        reps, t0 = 0, time.perf_counter()
        while True:
            cq, ck, cv, co = copies[reps % CPU_ROTATE_LAYERS]
            b.gemv(Q4K, cq, x[:H], QD, H, threads)
            b.gemv(Q4K, ck, x[:H], KVD, H, threads)
            b.gemv(Q6K, cv, x[:H], KVD, H, threads)
            b.gemv(Q4K, co, x, H, QD, threads)
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget:
                return BYTES_LAYER * reps / el / 1e9, reps, el

    v_all, reps, el = rate(cores, 0.6 * seconds)
    v_one, reps1, el1 = rate(1, 0.4 * seconds)
    return {"value": round(v_all, 2), "unit": "GB/s", "cores": cores, "kind": "port",
            "single_core_GBps": round(v_one, 2), "isa": f"x86-64-{b.level}",
            "sample": f"one layer's attention projections (Q 8192x4096 Q4_K, K 512x4096 Q4_K, V 512x4096 "
                      f"Q6_K, O 4096x8192 Q4_K; {CPU_ROTATE_LAYERS} copies in turn, {CPU_ROTATE_LAYERS * BYTES_LAYER / 1e6:.0f} MB): {reps} passes in {el:.1f} s on {cores} cores, {reps1} in "
                      f"{el1:.1f} s on 1 core; fused dequant+dot in fp32, vectorised, OpenMP rows"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the hot path "
              "would shard by weight rows and experts with no exchange between GPUs", file=sys.stderr)
        sys.exit(2)
    r = gpu_bench(args)
    if args.copy_calibration:
        import torch
        src = torch.ones(64 << 20, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
    value = BYTES_LAYER * LAYERS / r["step_s"] / 1e9
    ach = BYTES_QKV / r["d_qkv"] / 1e9
    prof = ROOT / "profiles" / "gemv_qkv_fused_traffic.json"
    traffic, kname = None, "gemv_split_kernel<8, 4, 0, 3>"
    if prof.exists():
        try:
            pj = json.loads(prof.read_text())
            traffic, kname = pj.get("hbm_bytes_per_launch"), pj.get("kernel", kname)
        except Exception:
            traffic = None
    line = {
        "metric": "Q4K/Q6K GEMV HBM GB/s (% of peak); Q4K GEMM int8-MFMA TOPS; decode tok/s",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["step_s"] * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8 dot4 (q4/q6 weights x int8 digits of x), fp32 rescale and accumulate",
        "data": "synthetic (seeded GGUF Q4_K/Q6_K blocks with the benchmark configs' value distributions, generated in HBM)",
        "config": {"workload": "configs[1]: Qwen3-235B attention projections, decode batch=1, hidden 4096, "
                               "94 layers per step (Q 4096->8192 Q4_K + K Q4_K + V Q6_K 4096->512 in one "
                               "launch, O 8192->4096 Q4_K + residual), hipGraph replay",
                   "global_batch": 1, "layers": LAYERS, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": kname + " (fused Q 8192 + K 512 Q4_K + V 512 Q6_K, 4096 cols)",
                     "bytes_per_launch": BYTES_QKV, "avg_launch_us": round(r["d_qkv"] * 1e6, 3)},
        "extra": {
            "fraction_of_hbm_peak": round(value / HBM_PEAK_GBS, 4),
            "per_kernel_GBps": {"qkv_fused": round(BYTES_QKV / r["d_qkv"] / 1e9, 1),
                                "o_proj_res": round(BYTES_O / r["d_o"] / 1e9, 1),
                                "q_proj_alone": round(BYTES_Q / r["d_q"] / 1e9, 1),
                                "kv_dual_alone": round(BYTES_KV / r["d_kv"] / 1e9, 1)},
            "per_kernel_us": {"qkv_fused": round(r["d_qkv"] * 1e6, 2), "o_proj_res": round(r["d_o"] * 1e6, 2),
                              "q_proj_alone": round(r["d_q"] * 1e6, 2), "kv_dual_alone": round(r["d_kv"] * 1e6, 2)},
            "gemm_q4k_m512": r["gemm"],
            "moe_prefill_cfg4": r["moe"],
            "decode_tok_s": r["decode"],
            "decode_attention_one_layer": r["attn"],
            "wall_s_timed": round(r["wall"], 3),
        },
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
