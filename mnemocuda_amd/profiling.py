"""Summaries of rocprofv3 output for the kernels of this library (used to write profiles/).

    python -m mnemocuda_amd.profiling stats <trace_dir> <out.md> "<command>" [<top> <name filter>]
    python -m mnemocuda_amd.profiling traffic <fetch_dir> <write_dir> <out.json> <out.md> "<command>"
    python -m mnemocuda_amd.profiling probe

`probe` is the program the two `--pmc` passes profile: the fused QKV GEMV of bench.py's
workload (one layer's weights, 4 launches), then the calibration copy.

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

# the fused QKV GEMV: a mixed-type launch (TM = 3) of the 32-lanes-per-row GEMV; the library
# builds it for 512- and 256-thread workgroups and the QKV shape runs the 256-thread one
QKV_KERNEL = "gemv_kernel<32, 1, *, 0, 3>"


def _is_qkv(name: str) -> bool:
    # template arguments <LPR 32, UPL 1, XPT, x mode 0 (plain x), types 3 (Q4_K and Q6_K)>
    return "gemv_kernel<32, 1, " in name and (", 0, 3>" in name or ", false, 3>" in name)
COPY_BYTES = 256 << 20  # bench.py --copy-calibration copies this many bytes


def _find(d: Path, suffix: str) -> Path:
    hits = sorted(Path(d).rglob(f"*{suffix}"))
    if not hits:
        raise FileNotFoundError(f"no *{suffix} under {d}")
    return hits[0]


def stats(trace_dir: str, out_md: str, command: str, top: int = 16, only: str | None = None) -> None:
    """only: keep the kernels whose name contains this text (e.g. 'mnemo::')"""
    rows = list(csv.DictReader(open(_find(Path(trace_dir), "kernel_stats.csv"))))
    if only:
        rows = [r for r in rows if only in r["Name"]]
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    lines = [f"command: `{command}`", "",
             "| kernel | calls | avg us | min us | max us | % time |", "|---|---|---|---|---|---|"]
    for r in rows[:top]:
        lines.append(f"| `{r['Name'][:90]}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                     f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | {float(r['Percentage']):.1f} |")
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


def probe(launches: int = 4) -> None:
    import torch
    from mnemocuda_amd import ops, synth
    Q4K, Q6K, H, QD, KVD = 12, 14, 4096, 8192, 512
    torch.cuda.set_device(0)
    ops.init()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1234)
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
        probe()
    else:
        raise SystemExit(__doc__)
