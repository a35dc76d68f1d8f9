"""Turns rocprofv3 output into the short text summaries kept under profiles/.

  python -m surge_amd.profile_summary stats KERNEL_STATS_CSV --tokens N > summary.md
      per-kernel calls, total/avg time and time per decode token from a
      `rocprofv3 --kernel-trace --stats` run;
  python -m surge_amd.profile_summary pmc COUNTER_CSV --counter FETCH_SIZE --calib-bytes B
      per-kernel average of one counter (KiB per dispatch) from a
      `rocprofv3 --pmc <counter>` run, and the same figure scaled into bytes by
      the counter's reading for the largest plain copy kernel
      (__amd_rocclr_copyBuffer) of known size B bytes in the same run;
  python -m surge_amd.profile_summary decode KERNEL_TRACE_CSV
      per decode token: calls, average and total time of each kernel over the
      device-resident greedy steps of a `rocprofv3 --kernel-trace` run of
      bench.py (from the third k_embed launch to the last k_step_advance: the
      prefill and the first warm-up steps are left out), the span per token
      and the time between kernels;
  python -m surge_amd.profile_summary prefill KERNEL_TRACE_CSV
      per kernel: calls, average and total time over the prefill of a
      `rocprofv3 --kernel-trace` run of bench.py (from the first k_embed_rows
      launch to the last launch before the first decode k_embed);
  python -m surge_amd.profile_summary counters COUNTER_CSV --kernel NAME
      every counter of a `rocprofv3 --pmc` run averaged over the dispatches of
      kernel NAME (prefix match), with derived fractions: wave cycles spent
      waiting for instruction issue (SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES) or on
      memory (SQ_WAIT_ANY / SQ_WAVE_CYCLES), and MFMA busy per SIMD
      (SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 XCDs * 4 SIMDs * CUs));
  python -m surge_amd.profile_summary traffic FETCH_CSV WRITE_CSV --kernel NAME --calib-bytes B
         --algo-bytes A --json OUT
      HBM bytes per dispatch of kernel NAME (prefix match): FETCH_SIZE from the
      first run plus WRITE_SIZE from the second, each scaled by its reading for
      the plain copy kernel of B bytes in the same run, against its algorithmic
      bytes A; written as the JSON bench.py reports as roofline.traffic;
  python -m surge_amd.profile_summary hbm FETCH_CSV WRITE_CSV --trace KERNEL_TRACE_CSV --calib-bytes B
      per decode kernel: HBM bytes per dispatch (FETCH_SIZE + WRITE_SIZE, each
      calibrated by the plain copy of B bytes in its run), the average duration
      over the decode region of the trace, and the achieved HBM GB/s and its
      fraction of the 8 TB/s peak;
  python -m surge_amd.profile_summary floor KERNEL_TRACE_CSV
      per decode kernel of one token: its average duration against that of
      the plain read of its algorithmic bytes at the same place of the
      token's launch sequence, from a `rocprofv3 --kernel-trace` run of
      `SURGE_HIP_GRAPH=0 bench.py --fill` (decode tokens k_embed ..
      k_step_advance after the first two; the floor's k_read dispatches in
      tokens of the same length after the first), and the time lost per token;
  python -m surge_amd.profile_summary trace KERNEL_TRACE_CSV --kernel NAME --last N
      average duration of the last N dispatches of kernel NAME (prefix match)
      from a `rocprofv3 --kernel-trace` run, next to the average over all of
      its dispatches: bench.py times its GEMV roofline leg last, so the last
      N dispatches are exactly the launches it timed with HIP events.
"""
import argparse
import csv
import json
import sys
from collections import defaultdict


def short(name: str) -> str:
    return name.split("(")[0].replace("void ", "")[:70]


def stats(path, tokens):
    rows = list(csv.DictReader(open(path)))
    tot = sum(float(r["TotalDurationNs"]) for r in rows)
    print("| kernel | calls | calls/token | avg us | total ms | ms/token | % |")
    print("|---|---|---|---|---|---|---|")
    for r in rows:
        t = float(r["TotalDurationNs"])
        print(f"| `{short(r['Name'])}` | {r['Calls']} | {int(r['Calls']) / tokens:.2f} | "
              f"{float(r['AverageNs']) / 1e3:.2f} | {t / 1e6:.1f} | {t / tokens / 1e6:.4f} | {100 * t / tot:.1f} |")
    print(f"\nTotal kernel time {tot / 1e6:.1f} ms over {tokens} tokens = {tot / tokens / 1e6:.3f} ms/token.")


def decode(path):
    rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Start_Timestamp"]))
    names = [short(r["Kernel_Name"]) for r in rows]
    embeds = [i for i, n in enumerate(names) if n == "k_embed"]
    ends = [i for i, n in enumerate(names) if n == "k_step_advance"]
    if len(embeds) < 3 or not ends:
        print("no device-resident decode steps in this trace")
        return
    seg = rows[embeds[2]:ends[-1] + 1]
    ntok = sum(1 for r in seg if short(r["Kernel_Name"]) == "k_embed")
    span = int(seg[-1]["End_Timestamp"]) - int(seg[0]["Start_Timestamp"])
    agg = defaultdict(lambda: [0, 0])
    busy = 0
    for r in seg:
        d = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
        key = f"{short(r['Kernel_Name'])} (grid {int(r['Grid_Size_X']) // max(1, int(r['Workgroup_Size_X']))}x{r['Grid_Size_Y']})"
        agg[key][0] += 1
        agg[key][1] += d
        busy += d
    print(f"{ntok} decode tokens: span {span / ntok / 1e3:.1f} us/token, kernels busy {busy / ntok / 1e3:.1f} "
          f"us/token, between kernels {(span - busy) / ntok / 1e3:.1f} us/token\n")
    print("| kernel (workgroups) | calls/token | avg us | us/token | % of busy |")
    print("|---|---|---|---|---|")
    for k, (n, t) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        print(f"| `{k}` | {n / ntok:.2f} | {t / n / 1e3:.2f} | {t / ntok / 1e3:.1f} | {100 * t / busy:.1f} |")


def prefill(path):
    rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Start_Timestamp"]))
    names = [short(r["Kernel_Name"]) for r in rows]
    st = next((i for i, n in enumerate(names) if n == "k_embed_rows"), None)
    en = next((i for i, n in enumerate(names) if n == "k_embed"), None)
    if st is None or en is None or en <= st:
        print("no prefill in this trace")
        return
    seg = rows[st:en]
    span = int(seg[-1]["End_Timestamp"]) - int(seg[0]["Start_Timestamp"])
    agg = defaultdict(lambda: [0, 0])
    busy = 0
    for r in seg:
        d = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
        key = f"{short(r['Kernel_Name'])} (grid {int(r['Grid_Size_X']) // max(1, int(r['Workgroup_Size_X']))}" \
              f"x{r['Grid_Size_Y']}x{r.get('Grid_Size_Z', '1')})"
        agg[key][0] += 1
        agg[key][1] += d
        busy += d
    print(f"prefill: span {span / 1e6:.1f} ms, kernels busy {busy / 1e6:.1f} ms\n")
    print("| kernel (workgroups) | calls | avg us | total ms | % of busy |")
    print("|---|---|---|---|---|")
    for k, (n, t) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        if t < 0.001 * busy:
            continue
        print(f"| `{k}` | {n} | {t / n / 1e3:.1f} | {t / 1e6:.1f} | {100 * t / busy:.1f} |")


def counters(path, kernel, cus=256):
    vals = defaultdict(list)
    for r in csv.DictReader(open(path)):
        if short(r["Kernel_Name"]).startswith(kernel):
            vals[r["Counter_Name"]].append(float(r["Counter_Value"]))
    if not vals:
        print(f"no dispatches of {kernel}")
        return None
    avg = {c: sum(v) / len(v) for c, v in vals.items()}
    print(f"`{kernel}`: {len(next(iter(vals.values())))} dispatches\n")
    print("| counter | average per dispatch |")
    print("|---|---|")
    for c in sorted(avg):
        print(f"| {c} | {avg[c]:.0f} |")
    out = {"kernel": kernel, "counters": avg}
    wc = avg.get("SQ_WAVE_CYCLES")
    if wc:
        for c in ("SQ_WAIT_INST_ANY", "SQ_WAIT_ANY", "SQ_ACTIVE_INST_ANY"):
            if c in avg:
                out[c + "/SQ_WAVE_CYCLES"] = avg[c] / wc
    if "SQ_VALU_MFMA_BUSY_CYCLES" in avg and avg.get("GRBM_GUI_ACTIVE"):
        out["mfma_busy_per_simd"] = avg["SQ_VALU_MFMA_BUSY_CYCLES"] / (avg["GRBM_GUI_ACTIVE"] / 8 * 4 * cus)
    print()
    for k, v in out.items():
        if k not in ("kernel", "counters"):
            print(f"- {k}: {v:.3f}")
    return out


def pmc(path, counter, calib_bytes):
    vals = defaultdict(list)
    for r in csv.DictReader(open(path)):
        if r.get("Counter_Name", counter) != counter:
            continue
        vals[r["Kernel_Name"]].append(float(r["Counter_Value"]))
    copies = vals.get("__amd_rocclr_copyBuffer", [])
    ref = max(copies) if copies else 0.0
    scale = calib_bytes / (ref * 1024.0) if ref else None
    out = {}
    print(f"| kernel | dispatches | avg {counter} (KiB) | bytes/dispatch (calibrated) |")
    print("|---|---|---|---|")
    for k, v in sorted(vals.items(), key=lambda kv: -sum(kv[1])):
        avg = sum(v) / len(v)
        b = avg * 1024.0 * scale if scale else None
        out[short(k)] = {"dispatches": len(v), "avg_kib": avg, "bytes": b}
        print(f"| `{short(k)}` | {len(v)} | {avg:.1f} | {b / 1e6:.2f} MB |" if b else
              f"| `{short(k)}` | {len(v)} | {avg:.1f} | - |")
    print(f"\nCalibration: largest __amd_rocclr_copyBuffer read {ref:.1f} KiB for a {calib_bytes} B copy "
          f"(scale {scale:.4f})." if scale else "\nNo calibration copy found.")
    return out, scale


def traffic(fetch_csv, write_csv, kernel, calib_bytes, algo_bytes):
    def one(path, counter):
        vals, copies = [], []
        for r in csv.DictReader(open(path)):
            if r.get("Counter_Name", counter) != counter:
                continue
            name = short(r["Kernel_Name"])
            if name == "__amd_rocclr_copyBuffer":
                copies.append(float(r["Counter_Value"]))
            elif name.startswith(kernel):
                vals.append(float(r["Counter_Value"]))
        scale = calib_bytes / (max(copies) * 1024.0)
        return sum(vals) / len(vals) * 1024.0 * scale, len(vals), scale
    fb, n, fs = one(fetch_csv, "FETCH_SIZE")
    wb, _, ws = one(write_csv, "WRITE_SIZE")
    return {"kernel": kernel, "kernels_sha256": kernels_sha256(),
            "fetch_bytes_per_dispatch": int(fb), "write_bytes_per_dispatch": int(wb),
            "bytes_per_dispatch": int(fb + wb), "algorithmic_bytes": int(algo_bytes),
            "traffic_over_algorithmic": round((fb + wb) / algo_bytes, 4), "dispatches": n,
            "fetch_scale": fs, "write_scale": ws}


def kernels_sha256() -> str:
    """The build a measurement belongs to: sha256 of the kernel source
    (surge_amd/csrc/kernels.hip). bench.py reports a recorded counter figure
    only when it matches the source it was built from."""
    import hashlib
    import os
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "csrc", "kernels.hip")
    return hashlib.sha256(open(path, "rb").read()).hexdigest()


def hbm(fetch_csv, write_csv, trace_csv, calib_bytes, peak_gbs=8000.0):
    def per_kernel(path, counter):
        # counters of the decode steps only (from the third k_embed to the
        # last k_step_advance, in dispatch order), so kernels that prefill also
        # launches are not averaged with their prefill dispatches
        vals, copies, rows = defaultdict(list), [], []
        for r in csv.DictReader(open(path)):
            if r.get("Counter_Name", counter) != counter:
                continue
            name = short(r["Kernel_Name"])
            if name == "__amd_rocclr_copyBuffer":
                copies.append(float(r["Counter_Value"]))
            else:
                rows.append((int(r.get("Dispatch_Id", len(rows))), name, float(r["Counter_Value"])))
        rows.sort()
        embeds = [i for i, x in enumerate(rows) if x[1] == "k_embed"]
        ends = [i for i, x in enumerate(rows) if x[1] == "k_step_advance"]
        if len(embeds) >= 3 and ends:
            rows = rows[embeds[2]:ends[-1] + 1]
        for _, name, v in rows:
            vals[name].append(v)
        scale = calib_bytes / (max(copies) * 1024.0)
        return {k: sum(v) / len(v) * 1024.0 * scale for k, v in vals.items()}, scale
    fb, fs = per_kernel(fetch_csv, "FETCH_SIZE")
    wb, ws = per_kernel(write_csv, "WRITE_SIZE")
    rows = sorted(csv.DictReader(open(trace_csv)), key=lambda r: int(r["Start_Timestamp"]))
    names = [short(r["Kernel_Name"]) for r in rows]
    embeds = [i for i, n in enumerate(names) if n == "k_embed"]
    ends = [i for i, n in enumerate(names) if n == "k_step_advance"]
    seg = rows[embeds[2]:ends[-1] + 1] if len(embeds) >= 3 and ends else rows
    durs = defaultdict(list)
    for r in seg:
        durs[short(r["Kernel_Name"])].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    print(f"Calibration: FETCH_SIZE x{fs:.4f}, WRITE_SIZE x{ws:.4f} (plain copy of {calib_bytes:.0f} B).\n")
    print("| kernel | HBM MB per dispatch (fetch + write) | avg us (decode) | HBM GB/s | of 8 TB/s |")
    print("|---|---|---|---|---|")
    out = {}
    for k in sorted(durs, key=lambda k: -sum(durs[k])):
        if k not in fb:
            continue
        b = fb[k] + wb.get(k, 0.0)
        us = sum(durs[k]) / len(durs[k]) / 1e3
        gbs = b / (us * 1e3)
        out[k] = {"hbm_bytes": b, "avg_us": us, "hbm_gbs": gbs}
        print(f"| `{k}` | {fb[k] / 1e6:.2f} + {wb.get(k, 0.0) / 1e6:.2f} | {us:.2f} | {gbs:.0f} | {gbs / peak_gbs:.3f} |")
    return out


def floor(path):
    rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Start_Timestamp"]))
    dur = lambda r: (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    # decode tokens: k_embed .. k_step_advance, in launch order
    toks, cur = [], None
    for r in rows:
        n = short(r["Kernel_Name"])
        if n == "k_embed":
            cur = [r]
        elif cur is not None:
            cur.append(r)
            if n == "k_step_advance":
                toks.append(cur)
                cur = None
    toks = toks[2:]
    if not toks:
        print("no decode tokens in the trace")
        return None
    n = len(toks[0])
    toks = [t for t in toks if len(t) == n]

    def kind(i):
        nm = short(toks[0][i]["Kernel_Name"])
        if nm.startswith(("k_gemv_ring<2, 1, 0>", "k_gemv_q8<2, 1, 0>")):
            return "lm_head" if i + 1 < n and short(toks[0][i + 1]["Kernel_Name"]) == "k_argmax" else "input projection"
        if nm.startswith("k_gemv_bal") and i and short(toks[0][i - 1]["Kernel_Name"]).startswith("k_attn_combine"):
            return "output projection (attention)"     # the attention output projection on the balanced GEMV
        for pre, k in (("k_embed", "embedding"), ("k_attn_partial", "attention partial"),
                       ("k_attn_combine", "attention combine"), ("k_gdn_step", "DeltaNet step"),
                       ("k_gemv_q8<2, 0, 1>", "output projection (attention)"),
                       ("k_gemv_ring<2, 2, 1>", "output projection (DeltaNet, gated prologue)"),
                       ("k_gemv_q8<2, 2, 1>", "output projection (DeltaNet, gated prologue)"),
                       ("k_gemv_bal<0, 0", "output projection (attention)"), ("k_gemv_ring<2, 1, 2>", "gate/up"),
                       ("k_gemv_q8<2, 1, 2>", "gate/up"),
                       ("k_gemv_bal", "down projection"), ("k_argmax", "argmax"), ("k_step_advance", "step advance")):
            if nm.startswith(pre):
                return k
        return nm
    reads = [r for r in rows if short(r["Kernel_Name"]).startswith("k_read")]
    nfl = len(reads) // n
    fl = [reads[t * n:(t + 1) * n] for t in range(1, nfl)]
    if not fl:
        print("no floor reads in the trace")
        return None
    kinds = [kind(i) for i in range(n)]
    order = list(dict.fromkeys(kinds))
    agg = {k: [0, 0.0, 0.0] for k in order}
    for i, k in enumerate(kinds):
        agg[k][0] += 1
        agg[k][1] += sum(dur(t[i]) for t in toks) / len(toks)
        agg[k][2] += sum(dur(t[i]) for t in fl) / len(fl)
    print(f"{len(toks)} decode tokens and {len(fl)} floor tokens of {n} kernels each (eager launches)")
    print()
    print("| kernel | launches/token | plain read of its bytes us | decode kernel us | lost per token us |")
    print("|---|---|---|---|---|")
    tot_d = tot_f = 0.0
    for k in order:
        c, d, f = agg[k]
        tot_d += d
        tot_f += f
        print(f"| {k} | {c} | {f / c:.2f} | {d / c:.2f} | {d - f:.1f} |")
    print(f"| all | {n} | | | {tot_d - tot_f:.1f} |")
    print()
    print(f"busy per token: decode {tot_d:.1f} us, plain reads {tot_f:.1f} us")
    return agg


def trace(path, kernel, last):
    durs = []
    for r in csv.DictReader(open(path)):
        if short(r["Kernel_Name"]).startswith(kernel):
            durs.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]) - int(r["Start_Timestamp"])))
    durs.sort()
    if not durs:
        print(f"no dispatches of {kernel}")
        return None
    tail = [d for _, d in durs[-last:]] if last else [d for _, d in durs]
    all_avg = sum(d for _, d in durs) / len(durs) / 1e3
    avg = sum(tail) / len(tail) / 1e3
    print(f"`{kernel}`: {len(durs)} dispatches, average {all_avg:.2f} us; "
          f"last {len(tail)} dispatches average {avg:.2f} us (min {min(tail) / 1e3:.2f}, max {max(tail) / 1e3:.2f}).")
    return {"kernel": kernel, "dispatches": len(durs), "avg_us": all_avg, "last": len(tail), "last_avg_us": avg}


def micro(micro_jsonl, shapes_jsonl):
    """The micro-config tables from `bench.py --micro` and `bench.py
    --gemv-shapes` output (one JSON object per line each)."""
    rows = [json.loads(l) for l in open(micro_jsonl) if l.strip().startswith("{")]
    print("| unit | GPU us (rotated) | GB/s | of 8 TB/s | GPU us (resident) | ref.c us (1 core) |")
    print("|---|---|---|---|---|---|")
    split = []
    for r in rows:
        if "cpu_us_median" in r:
            print(f"| {r['unit']} | {r['gpu_us']} | {r['gpu_GBs']} | {r['frac']} | {r['gpu_us_cache_resident']} | "
                  f"{r['cpu_us_median']} |")
            if "gpu_us_partial" in r:
                keys = r["unit"].split(" at ")[1].split(",")[0]
                split.append(f"{keys}: {r['gpu_us_partial']} / {r['gpu_us_combine']}")
    if split:
        print("\nAttention split: partial / combine us (rotated): " + "; ".join(split) + ".")
    print("\n| read | us (rotated) | GB/s | of 8 TB/s | us (resident) |")
    print("|---|---|---|---|---|")
    for r in rows:
        if r.get("unit", "").startswith("plain streaming read"):
            print(f"| {r['algo_bytes'] / 1e6:.1f} MB | {r['gpu_us']} | {r['gpu_GBs']} | {r['frac']} | "
                  f"{r['gpu_us_cache_resident']} |")
    for r in rows:
        if r.get("unit", "").startswith("empty kernel"):
            print(f"\nEmpty kernel: {r['gpu_us_per_launch_eager']} us per launch issued one by one, "
                  f"{r['gpu_us_per_launch_in_graph']} us replayed from a captured HIP graph ({r['reps']} launches).")
    if not shapes_jsonl:
        return
    sh = [json.loads(l) for l in open(shapes_jsonl) if l.strip().startswith("{")]
    shapes, variants, t = [], [], {}
    for r in sh:
        if r["shape"] not in shapes:
            shapes.append(r["shape"])
        if r["variant"] not in variants:
            variants.append(r["variant"])
        t[(r["shape"], r["variant"])] = r["us"]
    print("\n| shape | " + " | ".join(variants) + " |")
    print("|---|" + "---|" * len(variants))
    for s_ in shapes:
        print(f"| {s_} | " + " | ".join(str(t.get((s_, v), "-")) for v in variants) + " |")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("mode", choices=["stats", "pmc", "trace", "decode", "traffic", "prefill", "counters", "hbm",
                                     "micro", "floor"])
    ap.add_argument("--trace", default=None)
    ap.add_argument("csv")
    ap.add_argument("csv2", nargs="?", default=None)
    ap.add_argument("--algo-bytes", type=float, default=0)
    ap.add_argument("--tokens", type=int, default=1)
    ap.add_argument("--counter", default="FETCH_SIZE")
    ap.add_argument("--calib-bytes", type=float, default=0)
    ap.add_argument("--json", default=None)
    ap.add_argument("--kernel", default="k_gemv_ring<2, 1, 2>")
    ap.add_argument("--last", type=int, default=0)
    a = ap.parse_args()
    if a.mode == "stats":
        stats(a.csv, a.tokens)
    elif a.mode == "micro":
        micro(a.csv, a.csv2)
    elif a.mode == "decode":
        decode(a.csv)
    elif a.mode == "floor":
        floor(a.csv)
    elif a.mode == "prefill":
        prefill(a.csv)
    elif a.mode == "hbm":
        out = hbm(a.csv, a.csv2, a.trace, a.calib_bytes)
        if a.json:
            json.dump(out, open(a.json, "w"), indent=1)
    elif a.mode == "counters":
        out = counters(a.csv, a.kernel)
        if a.json and out:
            json.dump(out, open(a.json, "w"), indent=1)
    elif a.mode == "traffic":
        out = traffic(a.csv, a.csv2, a.kernel, a.calib_bytes, a.algo_bytes)
        print(json.dumps(out, indent=1))
        if a.json:
            json.dump(out, open(a.json, "w"), indent=1)
    elif a.mode == "trace":
        out = trace(a.csv, a.kernel, a.last)
        if a.json and out:
            json.dump(out, open(a.json, "w"), indent=1)
    else:
        out, scale = pmc(a.csv, a.counter, a.calib_bytes)
        if a.json:
            json.dump({"counter": a.counter, "scale": scale, "kernels": out}, open(a.json, "w"), indent=1)


if __name__ == "__main__":
    sys.exit(main())
