"""Summarises rocprofv3 output of bench.py runs into the text files kept under profiles/.

  python talos-xii_amd/prof_summary.py --stats <kernel_stats.csv> [--fetch <fetch counter_collection.csv>
      --write <write counter_collection.csv>] [--mfma <mfma counter_collection.csv>] --bench-json <bench lines>
      [--metric <metric prefix>] --title <title> --command "<command>" --out <file.md>
      [--traffic-json profiles/traffic.json]

Kernel-trace stats give each kernel's launch count and average duration. The FETCH_SIZE and
WRITE_SIZE passes (one counter per run; the values are KiB per dispatch) are scaled by what the
same counters read for the known-size device-to-device copy that bench.py --copy-calibration-mb
performs (__amd_rocclr_copyBuffer): factor = copied bytes / counted bytes. The HBM traffic per
launch of every kernel is written to traffic.json, which bench.py reports next to the
algorithmic bytes of its dominant kernel.
"""
import argparse
import collections
import csv
import json
import re


def short(name):
    """'void talos::gemm_f32_kernel<true, false, 768>(talos::GemmArgs)' -> 'gemm_f32_kernel<true, false, 768>'."""
    n = re.sub(r"^void ", "", name)
    n = re.sub(r"^talos::", "", n)
    depth, out = 0, []
    for ch in n:
        if ch == "(" and depth == 0:
            break
        depth += ch == "<"
        depth -= ch == ">"
        out.append(ch)
    return "".join(out)


def counters(path, counter, scale=1024.0):
    """Per kernel symbol, the counter's value of each dispatch (FETCH_SIZE / WRITE_SIZE are KiB:
    scale 1024 gives bytes)."""
    per = collections.defaultdict(list)
    for r in csv.DictReader(open(path)):
        if r["Counter_Name"] == counter:
            per[short(r["Kernel_Name"])].append(float(r["Counter_Value"]) * scale)
    return per


def calibration(per, copy_bytes):
    vals = sorted(per.get("__amd_rocclr_copyBuffer", []))
    big = [v for v in vals if v >= 0.2 * copy_bytes]
    if not big:
        raise SystemExit("no calibration copy found in the counter file")
    return copy_bytes / (sum(big) / len(big)), len(big), sum(big) / len(big)


def pick_line(path, metric_prefix):
    """The bench JSON line whose metric starts with metric_prefix (the last line when empty)."""
    lines = [json.loads(l) for l in open(path).read().strip().splitlines() if l.startswith("{")]
    for d in lines:
        if metric_prefix and d.get("metric", "").startswith(metric_prefix):
            return d
    return lines[-1]


def bench_sentence(bench):
    if isinstance(bench.get("value"), dict):  # per-kernel lines (C2)
        parts = [f"`{k}` {v['us_per_launch']} us per launch ({v['GB/s']} GB/s)" for k, v in bench["value"].items()]
        return "bench line under the profiler: " + "; ".join(parts) + "."
    s = f"bench line under the profiler: {bench['value']} {bench['unit']}"
    if "ms_per_step" in bench:
        s += f", {bench['ms_per_step']} ms/step"
    roof = bench.get("roofline")
    if roof:
        s += (f"; dominant kernel `{roof['kernel']}` bench-measured average {roof['avg_launch_us']} us per launch "
              f"({roof['achieved']} {roof['unit']}, {100 * roof['frac']:.1f}% of the {roof['bound']} peak)")
    return s + "."


def mfma_table(path, stats, simds):
    """Per kernel: MFMA busy (SQ_VALU_MFMA_BUSY_CYCLES over GRBM_GUI_ACTIVE x SIMDs) and the MFMA
    flops counted per launch (SQ_INSTS_VALU_MFMA_MOPS_F32, and _BF16 when the pass collected it,
    x 512). GRBM_GUI_ACTIVE is reported summed over the XCDs; the per-XCD cycle count is that sum
    divided by the XCD count, found as the ratio of the sum to the cycles the kernel's duration
    holds at the measured clock."""
    busy, gui, mops, mops16 = (counters(path, c, scale=1.0) for c in
                               ("SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE", "SQ_INSTS_VALU_MFMA_MOPS_F32",
                                "SQ_INSTS_VALU_MFMA_MOPS_BF16"))
    dur = {short(r["Name"]): float(r["AverageNs"]) for r in stats}
    rows = []
    for k in sorted(busy, key=lambda k: -sum(busy[k])):
        if k.startswith("__amd") or not gui.get(k):
            continue
        g = sum(gui[k]) / len(gui[k])
        xcds = max(1, round(g / (dur.get(k, 0) * 2.1))) if dur.get(k) else 1  # ~2.1 GHz under load
        util = sum(busy[k]) / len(busy[k]) / (g / xcds * simds)
        fl = 512.0 * sum(mops.get(k, [0.0])) / max(1, len(mops.get(k, [])))
        fl16 = 512.0 * sum(mops16.get(k, [0.0])) / max(1, len(mops16.get(k, [])))
        clock = g / xcds / dur[k] if dur.get(k) else 0.0
        rows.append((k, len(busy[k]), util, fl, fl16, clock))
    return rows


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--stats", required=True)
    ap.add_argument("--fetch")
    ap.add_argument("--write")
    ap.add_argument("--mfma", help="counter CSV of a --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_VALU_MFMA_MOPS_F32 "
                                   "GRBM_GUI_ACTIVE pass")
    ap.add_argument("--simds", type=int, default=1024)
    ap.add_argument("--bench-json", required=True)
    ap.add_argument("--metric", default="", help="prefix of the bench line's metric to quote")
    ap.add_argument("--title", default="C4 PPO minibatch fwd+bwd")
    ap.add_argument("--command", required=True)
    ap.add_argument("--pmc-command", default="")
    ap.add_argument("--mfma-command", default="")
    ap.add_argument("--out", required=True)
    ap.add_argument("--traffic-json")
    ap.add_argument("--top", type=int, default=16)
    a = ap.parse_args()

    bench = pick_line(a.bench_json, a.metric)
    stats = list(csv.DictReader(open(a.stats)))
    total_ns = sum(float(r["TotalDurationNs"]) for r in stats)
    lines = [f"# rocprofv3 kernel summary: {a.title}", "",
             "Command (kernel trace + stats):", "", "```", a.command, "```", ""]
    lines += [bench_sentence(bench), ""]
    lines += ["| kernel | calls | avg us | total % |", "|---|---:|---:|---:|"]
    for r in stats[:a.top]:
        lines.append(f"| `{short(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                     f"{100 * float(r['TotalDurationNs']) / total_ns:.2f} |")
    if a.mfma:
        rows = mfma_table(a.mfma, stats, a.simds)
        lines += ["", "Matrix-core counters (rocprofv3 --pmc, one pass):", "", "```", a.mfma_command, "```", "",
                  f"MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE per XCD x {a.simds} SIMDs); fp32 and "
                  "bf16 MFMA flops = SQ_INSTS_VALU_MFMA_MOPS_F32 / _BF16 x 512 per launch (bf16 blank when the pass "
                  "did not collect it); clock = GRBM_GUI_ACTIVE per XCD / the kernel's average duration from the "
                  "trace above.", "",
                  "| kernel | launches | MFMA busy % | fp32 MFMA GFLOP/launch | bf16 MFMA GFLOP/launch | clock GHz |",
                  "|---|---:|---:|---:|---:|---:|"]
        for k, n, util, fl, fl16, clock in rows[:a.top]:
            lines.append(f"| `{k}` | {n} | {100 * util:.1f} | {fl / 1e9:.3f} | {fl16 / 1e9:.3f} | {clock:.2f} |")
    traffic = {}
    if a.fetch and a.write:
        copy_bytes = bench.get("copy_calibration_bytes") or (1024 << 20)
        f, w = counters(a.fetch, "FETCH_SIZE"), counters(a.write, "WRITE_SIZE")
        ff, nf, cf = calibration(f, copy_bytes)
        fw, nw, cw = calibration(w, copy_bytes)
        lines += ["", "HBM traffic (rocprofv3 --pmc, one counter per run):", "", "```", a.pmc_command, "```", "",
                  f"Calibration: a {copy_bytes >> 20} MiB device-to-device copy (x{nf}) reads FETCH_SIZE = "
                  f"{cf / 2**20:.1f} MiB and WRITE_SIZE = {cw / 2**20:.1f} MiB, so the factors are "
                  f"fetch x{ff:.3f}, write x{fw:.3f}.", "",
                  "Achieved = (read + write) / the kernel's average traced duration above, against the 8 TB/s "
                  "HBM peak (the tracer adds its own time to short launches).", "",
                  "| kernel | launches | HBM read MB/launch | HBM write MB/launch | achieved GB/s | of HBM peak |",
                  "|---|---:|---:|---:|---:|---:|"]
        for k in sorted(f, key=lambda k: -sum(f[k])):
            # the runtime's copies (the calibration) and the set-up fills of plan buffers, whose
            # launches differ in size between the traced and the counted run
            if k.startswith("__amd") or k.startswith("fill_zero"):
                continue
            rd = ff * sum(f[k]) / len(f[k])
            wr = fw * sum(w.get(k, [0.0])) / max(1, len(w.get(k, [])))
            traffic[k] = {"fetch_bytes": rd, "write_bytes": wr, "bytes": rd + wr}
        dur = {short(r["Name"]): float(r["AverageNs"]) for r in stats}
        for k in list(traffic)[:a.top]:
            t = traffic[k]
            gbs = t["bytes"] / dur[k] if dur.get(k) else 0.0  # bytes / ns = GB/s
            lines.append(f"| `{k}` | {len(f[k])} | {t['fetch_bytes'] / 1e6:.1f} | {t['write_bytes'] / 1e6:.1f} | "
                         f"{gbs:.0f} | {gbs / 8000.0:.2f} |")
        if a.traffic_json:
            old = {}
            try:
                old = json.load(open(a.traffic_json))
            except (OSError, ValueError):
                pass
            old.update(traffic)
            json.dump(old, open(a.traffic_json, "w"), indent=1, sort_keys=True)
    open(a.out, "w").write("\n".join(lines) + "\n")


if __name__ == "__main__":
    main()
