"""Summaries of rocprofv3 output for the kernels of this library (used to write profiles/).

    python -m mnemocuda_amd.profiling stats <trace_dir> <out.md> "<command>" [<top> <name filter>]
    python -m mnemocuda_amd.profiling traffic <fetch_dir> <write_dir> <out.json> <out.md> "<command>"
    python -m mnemocuda_amd.profiling probe [qkv|gemm|moe]
    python -m mnemocuda_amd.profiling counters <out.md> "<command>" <filter> <pmc_dir>...

`probe` is the program the `--pmc` passes profile, each ending with the calibration copy:
  qkv  -- the fused QKV GEMV of bench.py's workload (one layer's weights, 4 launches);
  gemm -- the M=512 Q4_K prefill GEMMs of bench.py (N=8192 and N=1536, one launch per weight
          buffer over 600 MB of distinct buffers);
  moe  -- bench.py's grouped-expert prefill (configs[4], 3 calls);
  decode -- bench.py's decode layer (fused QKV with the norm, attention at position 2048, O +
          residual, the MoE block with 128 resident experts) over 4 layers of distinct
          weights, 3 tokens, then the lm_head Q6_K 151,936 x 4096 GEMV and top-p sampling.
`counters` merges several `--pmc` runs of one probe into a table per kernel (counters summed
over a dispatch's XCD / shader-engine instances, averaged over dispatches) with derived
figures: VALU and MFMA instructions per wave, the share of wave time waiting on counters,
the LDS bank-conflict ratio, and HBM bytes per launch from FETCH_SIZE scaled by the copy.

`stats` turns a `rocprofv3 --kernel-trace --stats --output-format csv` run into a table of
kernel durations.  `traffic` reads two `--pmc` runs (FETCH_SIZE, then WRITE_SIZE) of
`probe`, which ends with a device copy of known size (torch.neg
over 256 MiB of fp32: 256 MiB read, 256 MiB written): the copy's
counter reading gives the bytes-per-count factor, and the fused QKV GEMV's readings times
that factor give its HBM bytes per launch (bench.py reports them as roofline.traffic).
"""
from __future__ import annotations

import csv
import json
import sys
from collections import defaultdict
from pathlib import Path

# the fused QKV GEMV: a mixed-type launch (TM = 3) of the split-columns GEMV (8 lanes per row,
# 4 waves of 1024 columns, plain x), which the library picks for the QKV shape
QKV_KERNEL = "gemv_split_kernel<8, 4, 0, 3>"


def _is_qkv(name: str) -> bool:
    return "gemv_split_kernel<8, 4, 0, 3>" in name


COPY_BYTES = 256 << 20  # bench.py --copy-calibration copies this many bytes


def _find(d: Path, suffix: str) -> Path:
    hits = sorted(Path(d).rglob(f"*{suffix}"))
    if not hits:
        raise FileNotFoundError(f"no *{suffix} under {d}")
    return hits[0]


def stats(trace_dir: str, out_md: str, command: str, top: int = 16, only: str | None = None) -> None:
    """only: keep the kernels whose name contains this text (e.g. 'mnemo::').  With the
    kernel trace present, a kernel launched with several grid sizes gets a row per size."""
    rows = list(csv.DictReader(open(_find(Path(trace_dir), "kernel_stats.csv"))))
    if only:
        rows = [r for r in rows if only in r["Name"]]
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    lines = [f"command: `{command}`", "",
             "| kernel | calls | avg us | min us | max us | % time |", "|---|---|---|---|---|---|"]
    for r in rows[:top]:
        lines.append(f"| `{r['Name'][:90]}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                     f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | {float(r['Percentage']):.1f} |")
    hits = sorted(Path(trace_dir).rglob("*kernel_trace.csv"))
    if hits:
        per: dict[tuple[str, int], list[float]] = defaultdict(list)
        for r in csv.DictReader(open(hits[0])):
            if only and only not in r["Kernel_Name"]:
                continue
            grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
            per[(r["Kernel_Name"], grid)].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        names = [r["Name"] for r in rows[:top]]
        split = [(k, v) for k, v in per.items() if k[0] in names and sum(1 for kk in per if kk[0] == k[0]) > 1]
        if split:
            lines += ["", "Per launch shape (kernel trace):", "", "| kernel | grid (threads) | calls | avg us | min us | max us |",
                      "|---|---|---|---|---|---|"]
            for (name, grid), v in sorted(split, key=lambda kv: (kv[0][0], -kv[0][1])):
                lines.append(f"| `{name[:90]}` | {grid} | {len(v)} | {sum(v) / len(v):.2f} | {min(v):.2f} | {max(v):.2f} |")
    Path(out_md).write_text("\n".join(lines) + "\n")


def _per_kernel(pmc_dir: Path, counter: str) -> dict[tuple[str, int], list[float]]:
    """counter value per dispatch, grouped by (kernel name, grid size)"""
    per_dispatch: dict[tuple[str, int, str], float] = defaultdict(float)
    for r in csv.DictReader(open(_find(pmc_dir, "counter_collection.csv"))):
        if r["Counter_Name"] != counter:
            continue
        per_dispatch[(r["Kernel_Name"], int(r["Grid_Size"]), r["Dispatch_Id"])] += float(r["Counter_Value"])
    out: dict[tuple[str, int], list[float]] = defaultdict(list)
    for (name, grid, _), v in per_dispatch.items():
        out[(name, grid)].append(v)
    return out


def _pick(per: dict[tuple[str, int], list[float]], key) -> tuple[str, float]:
    """the largest-grid launch shape of the matching kernel (the same template also serves
    smaller launches, e.g. the K+V dual GEMV)"""
    keys = [k for k in per if key(k[0])]
    if not keys:
        raise KeyError("kernel not found in counter output")
    k = max(keys, key=lambda k: k[1])
    vals = per[k]
    return f"{k[0]} grid={k[1]}", sum(vals) / len(vals)


def traffic(fetch_dir: str, write_dir: str, out_json: str, out_md: str, command: str) -> dict:
    res = {}
    for counter, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        per = _per_kernel(Path(d), counter)
        qn, q = _pick(per, _is_qkv)
        cn, c = _pick(per, lambda n: "neg_kernel" in n)
        factor = COPY_BYTES / c  # bytes per counter unit, from the copy of known size
        res[counter] = {"kernel": qn, "per_launch_counter": q, "copy_kernel": cn, "copy_counter": c,
                        "bytes_per_unit": factor, "bytes_per_launch": q * factor}
    total = res["FETCH_SIZE"]["bytes_per_launch"] + res["WRITE_SIZE"]["bytes_per_launch"]
    out = {"kernel": res["FETCH_SIZE"]["kernel"], "hbm_bytes_per_launch": round(total), "algorithmic_bytes_per_launch": 21827584,
           "counters": res, "command": command}
    Path(out_json).write_text(json.dumps(out, indent=1) + "\n")
    lines = [f"command: `{command}`", "",
             f"fused QKV GEMV (`{res['FETCH_SIZE']['kernel']}`), HBM bytes per launch from FETCH_SIZE + WRITE_SIZE, each scaled",
             f"by the same counter over a {COPY_BYTES >> 20} MiB device copy (read {COPY_BYTES >> 20} MiB, "
             f"write {COPY_BYTES >> 20} MiB):", "",
             "| counter | per launch (counter units) | copy reading | bytes per unit | bytes per launch |",
             "|---|---|---|---|---|"]
    for k, v in res.items():
        lines.append(f"| {k} | {v['per_launch_counter']:.1f} | {v['copy_counter']:.1f} | {v['bytes_per_unit']:.1f} | "
                     f"{v['bytes_per_launch']:.0f} |")
    lines += ["", f"total HBM bytes per launch: {total:.0f} (algorithmic: 21,827,584)"]
    Path(out_md).write_text("\n".join(lines) + "\n")
    return out


def counters(out_md: str, command: str, only: str, *pmc_dirs: str) -> None:
    per: dict[tuple[str, int], dict[str, list[float]]] = defaultdict(lambda: defaultdict(list))
    copy: dict[str, float] = {}
    for d in pmc_dirs:
        cur: dict[tuple[str, int, str, str], float] = defaultdict(float)
        for r in csv.DictReader(open(_find(Path(d), "counter_collection.csv"))):
            cur[(r["Kernel_Name"], int(r["Grid_Size"]), r["Dispatch_Id"], r["Counter_Name"])] += float(r["Counter_Value"])
        for (name, grid, _, c), v in cur.items():
            if "neg_kernel" in name and c == "FETCH_SIZE":
                copy[c] = max(copy.get(c, 0.0), v)
            elif only in name:
                per[(name, grid)][c].append(v)
    lines = [f"command: `{command}`", ""]
    for (name, grid), cs in sorted(per.items(), key=lambda kv: kv[0][0]):
        avg = {c: sum(v) / len(v) for c, v in cs.items()}
        lines += [f"`{name[:150]}` grid={grid}", "", "| counter | per dispatch |", "|---|---|"]
        lines += [f"| {c} | {v:.6g} |" for c, v in sorted(avg.items())]
        waves = avg.get("SQ_WAVES")
        derived = []
        if waves:
            for c, label in (("SQ_INSTS_VALU", "VALU instructions per wave"), ("SQ_INSTS_MFMA", "MFMA instructions per wave"),
                             ("SQ_INSTS_LDS", "LDS instructions per wave"), ("SQ_INSTS_VMEM_RD", "vector memory reads per wave")):
                if c in avg:
                    derived.append(f"| {label} | {avg[c] / waves:.1f} |")
        if "SQ_INSTS_VALU" in avg and avg.get("SQ_INSTS_MFMA"):
            derived.append(f"| VALU per MFMA instruction | {avg['SQ_INSTS_VALU'] / avg['SQ_INSTS_MFMA']:.2f} |")
        if "SQ_WAIT_INST_ANY" in avg and avg.get("SQ_WAVE_CYCLES"):
            derived.append(f"| share of wave time waiting on counters | {avg['SQ_WAIT_INST_ANY'] / avg['SQ_WAVE_CYCLES']:.2f} |")
        if "SQ_LDS_BANK_CONFLICT" in avg and avg.get("SQ_LDS_IDX_ACTIVE"):
            derived.append(f"| LDS bank-conflict cycles / LDS active cycles | {avg['SQ_LDS_BANK_CONFLICT'] / avg['SQ_LDS_IDX_ACTIVE']:.2f} |")
        if "FETCH_SIZE" in avg and copy.get("FETCH_SIZE"):
            derived.append(f"| HBM bytes fetched per launch (FETCH_SIZE x {COPY_BYTES / copy['FETCH_SIZE']:.1f} B, the copy's factor) | "
                           f"{avg['FETCH_SIZE'] * COPY_BYTES / copy['FETCH_SIZE']:.4g} |")
        if derived:
            lines += ["", "| derived | value |", "|---|---|", *derived]
        lines.append("")
    Path(out_md).write_text("\n".join(lines) + "\n")


def _copy_tail() -> None:
    import torch
    src = torch.ones(COPY_BYTES // 4, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()


def _decode_probe(torch, ops, synth, gen, layers: int = 4, tokens: int = 3, pos0: int = 2048,
                  max_ctx: int = 4096) -> None:
    """the calls of bench.py's decode step, eager, on `layers` layers of distinct weights"""
    Q4K, Q6K, H, QD, KVD = 12, 14, 4096, 8192, 512
    E, k, EFF, VOCAB = 128, 8, 1536, 151936
    NH, NKV, HD, EPS, THETA = 64, 4, 128, 1e-6, 1e6
    stride, g_off, u_off, d_off = synth.expert_layout(H, EFF, Q6K)
    L = [dict(q=synth.weights_torch(gen, Q4K, QD, H, "cuda"), k=synth.weights_torch(gen, Q4K, KVD, H, "cuda"),
              v=synth.weights_torch(gen, Q6K, KVD, H, "cuda"), o=synth.weights_torch(gen, Q4K, H, QD, "cuda"),
              table=synth.expert_table_torch(gen, E, H, EFF, Q6K, "cuda"),
              router=torch.randn(E, H, device="cuda", generator=gen) / 64,
              kc=torch.randn(max_ctx * NKV * HD, device="cuda", generator=gen).half(),
              vc=torch.randn(ops.v_cache_bytes(NKV, HD, max_ctx, 0, 1) // 2, device="cuda", generator=gen).half())
         for _ in range(layers)]
    nw = 1 + 0.05 * torch.randn(H, device="cuda", generator=gen)
    qn = 1 + 0.05 * torch.randn(HD, device="cuda", generator=gen)
    lm_head = synth.weights_torch(gen, Q6K, VOCAB, H, "cuda")
    bufs = (torch.randn(H, device="cuda", generator=gen), torch.empty(H, device="cuda"))
    q, kk, v = torch.empty(QD, device="cuda"), torch.empty(KVD, device="cuda"), torch.empty(KVD, device="cuda")
    attn, normed, logits = torch.empty(QD, device="cuda"), torch.empty(H, device="cuda"), torch.empty(VOCAB, device="cuda")
    tok, pos = torch.zeros(1, dtype=torch.int32, device="cuda"), torch.full((1,), pos0, dtype=torch.int32, device="cuda")
    ws = torch.zeros(ops.moe_decode_workspace_bytes(H, EFF, E, k), dtype=torch.uint8, device="cuda")
    aws = torch.empty(ops.attention_decode_workspace_bytes(NKV, max_ctx), dtype=torch.uint8, device="cuda")
    sws = torch.empty(ops.sample_workspace_bytes(), dtype=torch.uint8, device="cuda")
    for _ in range(tokens):
        for li, W in enumerate(L):
            src, dst = bufs[li % 2], bufs[(li + 1) % 2]
            ops.matvec_qkv_rmsnorm(W["q"], Q4K, W["k"], Q4K, W["v"], Q6K, src, nw, EPS, q, kk, v, QD, KVD, H)
            ops.attention_decode_prep(q, kk, v, qn, qn, EPS, THETA, W["kc"], W["vc"], attn, NH, HD, NKV, max_ctx, pos,
                                      1.0 / HD ** 0.5, aws, v_layout=1)
            ops.matvec_q4k_add(W["o"], attn, src, dst, H, QD)
            ops.moe_decode_rmsnorm(W["router"], W["table"], stride, g_off, u_off, d_off, Q6K, dst, nw, EPS, H, EFF,
                                   E, k, ws, dst)
        ops.rms_norm(bufs[layers % 2], nw, normed, EPS)
        ops.matvec_q6k(lm_head, normed, logits, VOCAB, H)
        ops.sample_token_ws(logits, VOCAB, 0.7, 0.9, 12345, sws, tok)
        pos.add_(1)
    torch.cuda.synchronize()


def probe(which: str = "qkv", launches: int = 4) -> None:
    import torch
    from mnemocuda_amd import ops, synth
    Q4K, Q6K, H, QD, KVD = 12, 14, 4096, 8192, 512
    torch.cuda.set_device(0)
    ops.init()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1234)
    if which == "gemm":
        T = 512
        acts = torch.randn(T, H, device="cuda", generator=gen)
        aq = torch.empty(T * (H // 128) * 144, dtype=torch.uint8, device="cuda")
        ops.quantize_q8_1(acts, aq, H, T)
        for n in (QD, 1536):
            # distinct weight buffers over 600 MB (more than the 256 MB MALL), one launch each,
            # as bench.py times them
            nbuf = -(-(600 << 20) // (n * (H // 256) * 144))
            out = torch.empty(T, n, device="cuda")
            for _ in range(nbuf):
                w = synth.weights_torch(gen, Q4K, n, H, "cuda")
                ops.gemm(w, Q4K, aq, out, n, H, T)
                del w
        _copy_tail()
        print("probe done", flush=True)
        return
    if which == "moe":
        import numpy as np
        T, E, k, EFF = 512, 128, 8, 1536
        idx, wt = synth.zipf_routing(np.random.default_rng(7), T, E, k)
        table = synth.expert_table_torch(gen, E, H, EFF, Q6K, "cuda")
        stride, g_off, u_off, d_off = synth.expert_layout(H, EFF, Q6K)
        x = torch.randn(T, H, device="cuda", generator=gen)
        out = torch.zeros(T, H, device="cuda")
        idx_d, w_d = torch.from_numpy(idx).cuda(), torch.from_numpy(wt).cuda()
        ws = torch.empty(ops.moe_prefill_workspace_bytes(T, H, EFF, E, k), dtype=torch.uint8, device="cuda")
        for _ in range(3):
            ops.moe_prefill(table, stride, g_off, u_off, d_off, Q6K, x, idx_d, w_d, T, H, EFF, E, k, ws, out)
        _copy_tail()
        print("probe done", flush=True)
        return
    if which in ("decode", "decode_long"):
        # decode_long: the same step from KV position 32,768 of a 40,960-position cache
        _decode_probe(torch, ops, synth, gen, **({"pos0": 32768, "max_ctx": 40960} if which == "decode_long" else {}))
        _copy_tail()
        print("probe done", flush=True)
        return
    wq, wk = synth.weights_torch(gen, Q4K, QD, H, "cuda"), synth.weights_torch(gen, Q4K, KVD, H, "cuda")
    wv = synth.weights_torch(gen, Q6K, KVD, H, "cuda")
    x = torch.randn(H, device="cuda", generator=gen)
    q, k, v = torch.empty(QD, device="cuda"), torch.empty(KVD, device="cuda"), torch.empty(KVD, device="cuda")
    for _ in range(launches):
        ops.matvec_qkv(wq, Q4K, wk, Q4K, wv, Q6K, x, q, k, v, QD, KVD, H)
    src = torch.ones(COPY_BYTES // 4, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    print("probe done", flush=True)


if __name__ == "__main__":
    if sys.argv[1] == "stats":
        stats(sys.argv[2], sys.argv[3], sys.argv[4], *([int(sys.argv[5]), sys.argv[6]] if len(sys.argv) > 6 else []))
    elif sys.argv[1] == "traffic":
        traffic(sys.argv[2], sys.argv[3], sys.argv[4], sys.argv[5], sys.argv[6])
    elif sys.argv[1] == "probe":
        probe(*sys.argv[2:3])
    elif sys.argv[1] == "counters":
        counters(sys.argv[2], sys.argv[3], sys.argv[4], *sys.argv[5:])
    else:
        raise SystemExit(__doc__)
