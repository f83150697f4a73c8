"""Summarises rocprofv3 output of bench.py runs into the text files kept under profiles/.

  python talos-xii_amd/prof_summary.py --stats <kernel_stats.csv> [--fetch <fetch counter_collection.csv>
      --write <write counter_collection.csv>] --bench-json <bench line> --command "<command>" --out <file.md>
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


def counters(path, counter):
    per = collections.defaultdict(list)
    for r in csv.DictReader(open(path)):
        if r["Counter_Name"] == counter:
            per[short(r["Kernel_Name"])].append(float(r["Counter_Value"]) * 1024.0)  # KiB -> bytes
    return per


def calibration(per, copy_bytes):
    vals = sorted(per.get("__amd_rocclr_copyBuffer", []))
    big = [v for v in vals if v >= 0.2 * copy_bytes]
    if not big:
        raise SystemExit("no calibration copy found in the counter file")
    return copy_bytes / (sum(big) / len(big)), len(big), sum(big) / len(big)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--stats", required=True)
    ap.add_argument("--fetch")
    ap.add_argument("--write")
    ap.add_argument("--bench-json", required=True)
    ap.add_argument("--command", required=True)
    ap.add_argument("--pmc-command", default="")
    ap.add_argument("--out", required=True)
    ap.add_argument("--traffic-json")
    ap.add_argument("--top", type=int, default=16)
    a = ap.parse_args()

    bench = json.loads(open(a.bench_json).read().strip().splitlines()[-1])
    stats = list(csv.DictReader(open(a.stats)))
    total_ns = sum(float(r["TotalDurationNs"]) for r in stats)
    lines = [f"# rocprofv3 kernel summary: {bench['config']['workload'].split(':')[0]} PPO minibatch fwd+bwd", "",
             "Command (kernel trace + stats):", "", "```", a.command, "```", ""]
    lines += [f"bench line under the profiler: {bench['value']} samples/s, {bench['ms_per_step']} ms/step; "
              f"dominant kernel `{bench['roofline']['kernel']}` bench-measured average "
              f"{bench['roofline']['avg_launch_us']} us per launch.", ""]
    lines += ["| kernel | calls | avg us | total % |", "|---|---:|---:|---:|"]
    for r in stats[:a.top]:
        lines.append(f"| `{short(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                     f"{100 * float(r['TotalDurationNs']) / total_ns:.2f} |")
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
                  "| kernel | launches | HBM read MB/launch | HBM write MB/launch |", "|---|---:|---:|---:|"]
        for k in sorted(f, key=lambda k: -sum(f[k])):
            if k.startswith("__amd"):
                continue
            rd = ff * sum(f[k]) / len(f[k])
            wr = fw * sum(w.get(k, [0.0])) / max(1, len(w.get(k, [])))
            traffic[k] = {"fetch_bytes": rd, "write_bytes": wr, "bytes": rd + wr}
        for k in list(traffic)[:a.top]:
            t = traffic[k]
            lines.append(f"| `{k}` | {len(f[k])} | {t['fetch_bytes'] / 1e6:.1f} | {t['write_bytes'] / 1e6:.1f} |")
        if a.traffic_json:
            json.dump(traffic, open(a.traffic_json, "w"), indent=1, sort_keys=True)
    open(a.out, "w").write("\n".join(lines) + "\n")


if __name__ == "__main__":
    main()
