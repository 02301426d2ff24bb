"""Summaries of the rocprofv3 runs of csrspmm_amd/profile_configs.sh.

    python -m csrspmm_amd.profile_summary [PROF_DIR]     # default gpurun_out/prof

For every NAME with a NAME.trace.log under PROF_DIR, writes profiles/NAME.md
(kernel trace, calibrated HBM traffic, L2 hit rate and VALU busy per kernel,
and the three fractions of the 8 TB/s peak) and the entry "CONFIG/KEY" of
profiles/traffic.json, where KEY is the algorithm, "plan" + algorithm for a
stored plan, or algorithm + "NoPanels".  Each traffic entry records the
kernel-source digest the run printed (csrspmm_amd.kernel_source_digest), so
bench.py can tell whether the figure belongs to the kernels it runs.  A
bench_xl directory (profile_configs.sh bench) becomes
profiles/bench_xl_trace.md.

Counter calibration: FETCH_SIZE and WRITE_SIZE are read, in KiB per
dispatch, for the SpMM dispatches of 3 calls, and scaled by what they read
for a 1 GiB device-to-device copy in the same run (FETCH_SIZE reads 512 MiB
for it, so its factor is about 2; WRITE_SIZE reads 1 GiB).
"""
from __future__ import annotations

import csv
import glob
import json
import os
import re
import subprocess
import sys

from . import configs

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PEAK = 8.0e12
XCDS = 8


def short(n: str) -> str:
    n = n.replace("csrspmm_hip::(anonymous namespace)::", "").replace("csrspmm_hip::Problem",
                                                                      "Problem")
    n = re.sub(r"^void ", "", n)
    return re.sub(r"\(.*\)$", "", n)


def _rows(pattern):
    files = glob.glob(pattern)
    if not files:
        raise FileNotFoundError(pattern)
    with open(files[0]) as f:
        return list(csv.DictReader(f))


def _run_info(log_path):
    with open(log_path) as f:
        log = f.read()
    m = re.search(r"\[profile_run\] (\S+) (\S+) M=(\d+) nnz=(\d+) N=(\d+) bytes_alg=(\d+) "
                  r"bytes_min=(\d+) U=(\d+) sources=(\S+)", log)
    if not m:
        raise ValueError(f"{log_path}: no profile_run header")
    cfg, algo = m.group(1), m.group(2)
    M, nnz, N, balg, bmin, U = map(int, m.groups()[2:8])
    mode = "plan" if "[profile_run] plan " in log else ("nopanels" if "no column panels" in log
                                                         else "")
    # a stored plan resolves Auto with the matrix's true longest row
    pm = re.search(r"\[profile_run\] plan (\w+):", log)
    return dict(cfg=cfg, algo=algo, M=M, nnz=nnz, N=N, balg=balg, bmin=bmin, U=U,
                digest=m.group(9), mode=mode, plan_algo=pm.group(1) if pm else None)


def _command(name, info, kind):
    extra = {"plan": " --plan", "nopanels": " --no-panels"}.get(info["mode"], "")
    run = f"python3 -m csrspmm_amd.profile_run --config {info['cfg']} --algo {info['algo']}{extra}"
    if kind == "trace":
        return (f"rocprofv3 --kernel-trace --stats -d OUT/{name}/trace -o {name} "
                f"--output-format csv -- {run} --calls 20")
    if kind == "hit":
        return (f"rocprofv3 --pmc TCC_HIT_sum TCC_MISS_sum VALUBusy -d OUT/{name}/hit -o {name} "
                f"--output-format csv -- {run} --calls 3")
    if kind == "busy":
        return (f"rocprofv3 --pmc TCC_BUSY_avr GRBM_GUI_ACTIVE TA_BUSY_avr -d OUT/{name}/busy "
                f"-o {name} --output-format csv -- {run} --calls 3")
    d = kind.split("_")[0].lower()
    return (f"rocprofv3 --pmc {kind} -d OUT/{name}/{d} -o {name} --output-format csv -- {run} "
            f"--calls 3 --copy-mib 1024")


def _commit():
    try:
        return subprocess.run(["git", "-C", ROOT, "rev-parse", "--short=12", "HEAD"],
                              capture_output=True, text=True, check=True).stdout.strip()
    except (OSError, subprocess.CalledProcessError):
        return None


def summarize(prof: str, name: str):
    d = os.path.join(prof, name)
    info = _run_info(os.path.join(prof, name + ".trace.log"))
    cfg = configs.CONFIGS[info["cfg"]]
    calls = 20
    spmm = [r for r in _rows(f"{d}/trace/*kernel_stats.csv") if "csrspmm_hip" in r["Name"]]
    per_call_us = sum(float(r["TotalDurationNs"]) for r in spmm) / calls / 1000

    def pmc(kind):
        rows = _rows(f"{d}/{kind}/*counter_collection.csv")
        copy = [float(r["Counter_Value"]) for r in rows
                if "copyBuffer" in r["Kernel_Name"] and int(r["Grid_Size"]) >= 131072]
        tot = sum(float(r["Counter_Value"]) for r in rows if "csrspmm_hip" in r["Kernel_Name"])
        return copy[0], tot / 3.0

    fcopy, fkib = pmc("fetch")
    wcopy, wkib = pmc("write")
    ff, wf = 1048576.0 / fcopy, 1048576.0 / wcopy
    fb, wb = fkib * 1024 * ff, wkib * 1024 * wf
    tr = fb + wb
    t = per_call_us * 1e-6
    from . import capi

    lib = capi.hip()
    resolved = info["plan_algo"] or lib.csrspmm_algorithm_name(lib.csrspmm_resolve_algorithm_ex(
        capi.ALGO[info["algo"]], info["M"], cfg.K(), info["N"], info["nnz"], -1)).decode()
    what = {"plan": "stored plan, ", "nopanels": "no column panels (base-size workspace), "}.get(
        info["mode"], "")
    lines = [
        f"# rocprofv3: {what}{info['algo']}"
        + (f" ({resolved})" if info["algo"] == "Auto" else "")
        + f" on config `{info['cfg']}` ({cfg.description})", "",
        "Commands (repository root on the MI355X box; `bash csrspmm_amd/profile_configs.sh "
        f"{name}:{info['cfg']}:{info['algo']}" + (f":{info['mode']}" if info["mode"] else "")
        + "` runs them):", "```",
        _command(name, info, "trace"), _command(name, info, "FETCH_SIZE"),
        _command(name, info, "WRITE_SIZE"), _command(name, info, "hit"),
        _command(name, info, "busy"), "```", "",
        f"Kernel sources: digest `{info['digest']}` (csrspmm_amd.kernel_source_digest).", "",
        f"M={info['M']} nnz={info['nnz']} N={info['N']}, distinct columns U={info['U']}; per call: "
        f"gather-model bytes {info['balg']:,}, compulsory bytes {info['bmin']:,}.", "",
        "## Kernel trace (`--stats`, 20 calls; the torch fill/copy kernels of data setup left out)",
        "", "| kernel | calls | avg us | min us | max us |", "|---|---|---|---|---|"]
    for r in spmm:
        lines.append(f"| `{short(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1000:.1f} "
                     f"| {float(r['MinNs']) / 1000:.1f} | {float(r['MaxNs']) / 1000:.1f} |")
    lines += [
        "", f"SpMM GPU time per call (sum over the call's dispatches): {per_call_us:.1f} us", "",
        "## HBM traffic per call (`--pmc`, KiB per dispatch summed over a call's SpMM "
        "dispatches, mean of 3 calls)", "",
        f"Calibration: a 1 GiB device copy (`__amd_rocclr_copyBuffer`) reads FETCH_SIZE = "
        f"{fcopy:.0f} KiB and WRITE_SIZE = {wcopy:.0f} KiB, so FETCH_SIZE is scaled by {ff:.4f} "
        f"and WRITE_SIZE by {wf:.4f}.", "",
        "| counter | raw KiB | scaled bytes |", "|---|---|---|",
        f"| FETCH_SIZE | {fkib:.0f} | {int(fb):,} |", f"| WRITE_SIZE | {wkib:.0f} | {int(wb):,} |",
        f"| total | | {int(tr):,} |", "",
        "## Against the 8 TB/s HBM peak, per call", "",
        "| figure | bytes | GB/s | fraction of peak |", "|---|---|---|---|",
        f"| measured traffic (FETCH + WRITE, scaled) | {int(tr):,} | {tr / t / 1e9:.0f} | "
        f"**{tr / t / PEAK:.3f}** |",
        f"| compulsory (each distinct B row once) | {info['bmin']:,} | {info['bmin'] / t / 1e9:.0f} "
        f"| {info['bmin'] / t / PEAK:.3f} |",
        f"| gather model (a B row per nonzero; above 1 = served from caches) | {info['balg']:,} | "
        f"{info['balg'] / t / 1e9:.0f} | {info['balg'] / t / PEAK:.3f} |", "",
        f"Measured traffic is {tr / info['bmin']:.2f} x the compulsory bytes and "
        f"{tr / info['balg']:.3f} x the gather model."]
    hit = {}
    for r in _rows(f"{d}/hit/*counter_collection.csv"):
        if "csrspmm_hip" not in r["Kernel_Name"]:
            continue
        e = hit.setdefault(short(r["Kernel_Name"]),
                           {"TCC_HIT_sum": 0.0, "TCC_MISS_sum": 0.0, "VALUBusy": []})
        if r["Counter_Name"] == "VALUBusy":
            e["VALUBusy"].append(float(r["Counter_Value"]))
        else:
            e[r["Counter_Name"]] += float(r["Counter_Value"])
    lines += ["", "## L2 hit rate and VALU busy per kernel (`--pmc TCC_HIT_sum TCC_MISS_sum "
              "VALUBusy`, 3 calls)", "",
              "| kernel | L2 hits | L2 misses | L2 hit rate | VALUBusy % (mean per dispatch) |",
              "|---|---|---|---|---|"]
    for k, e in hit.items():
        h, m = e["TCC_HIT_sum"] / 3, e["TCC_MISS_sum"] / 3
        vb = sum(e["VALUBusy"]) / max(len(e["VALUBusy"]), 1)
        lines.append(f"| `{k}` | {h / 1e6:.2f} M | {m / 1e6:.2f} M | {h / max(h + m, 1):.3f} | "
                     f"{vb:.1f} |")
    # L2 (TCC) and texture-address (TA) busy: each counter's mean over its
    # instances, in cycles, over the dispatch's GRBM_GUI_ACTIVE cycles, which
    # rocprofv3 sums over the 8 XCDs (divided by 8 it matches the kernel
    # durations at the ~2.4 GHz clock)
    busy = {}
    for r in _rows(f"{d}/busy/*counter_collection.csv"):
        if "csrspmm_hip" not in r["Kernel_Name"]:
            continue
        e = busy.setdefault(short(r["Kernel_Name"]), {})
        e.setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))

    def frac(e, c):
        g = sum(e.get("GRBM_GUI_ACTIVE", [])) / XCDS
        return sum(e.get(c, [])) / g if g > 0 else 0.0

    lines += ["", "## L2 and TA busy per kernel (`--pmc TCC_BUSY_avr GRBM_GUI_ACTIVE TA_BUSY_avr`, "
              "3 calls)", "",
              "Busy cycles (mean over the TCC channels / TA units) over the dispatch's cycles "
              "(GRBM_GUI_ACTIVE / 8 XCDs).  An L2 busy near 1 is the L2's request rate, the "
              "bound of a gather kernel whose B rows come from L2 and the MALL.", "",
              "| kernel | GRBM cycles per XCD | L2 (TCC) busy | TA busy |", "|---|---|---|---|"]
    for k, e in busy.items():
        g = sum(e.get("GRBM_GUI_ACTIVE", [])) / max(len(e.get("GRBM_GUI_ACTIVE", [])), 1) / XCDS
        lines.append(f"| `{k}` | {g:,.0f} | {frac(e, 'TCC_BUSY_avr'):.3f} | "
                     f"{frac(e, 'TA_BUSY_avr'):.3f} |")
    main_k = max(busy, key=lambda k: sum(busy[k].get("GRBM_GUI_ACTIVE", [0])), default=None)
    tot_g = sum(sum(e.get("GRBM_GUI_ACTIVE", [])) for e in busy.values()) / XCDS
    tot_b = sum(sum(e.get("TCC_BUSY_avr", [])) for e in busy.values())
    with open(os.path.join(ROOT, "profiles", name + ".md"), "w") as f:
        f.write("\n".join(lines) + "\n")
    key = {"plan": f"{info['cfg']}/plan{info['algo']}",
           "nopanels": f"{info['cfg']}/{info['algo']}NoPanels"}.get(
        info["mode"], f"{info['cfg']}/{info['algo']}")
    entry = {"bytes_per_call": int(tr), "fetch_bytes": int(fb), "write_bytes": int(wb),
             "fetch_factor": round(ff, 4), "write_factor": round(wf, 4),
             "spmm_us_per_call": round(per_call_us, 1), "bytes_alg": info["balg"],
             "bytes_min": info["bmin"], "source_digest": info["digest"], "summary": f"{name}.md",
             "kernels": [short(r["Name"]) for r in spmm],
             "l2_busy_main": round(frac(busy[main_k], "TCC_BUSY_avr"), 4) if main_k else None,
             "l2_busy_main_kernel": main_k,
             "l2_busy_call": round(tot_b / tot_g, 4) if tot_g > 0 else None}
    print(f"{name}: {per_call_us:.1f} us, measured {tr / t / PEAK:.3f} of peak, "
          f"compulsory {info['bmin'] / t / PEAK:.3f}, sources {info['digest']}")
    return key, entry


def summarize_bench(prof: str):
    d = os.path.join(prof, "bench_xl")
    spmm = [r for r in _rows(f"{d}/trace/*kernel_stats.csv") if "csrspmm_hip" in r["Name"]]
    calls = int(spmm[0]["Calls"])
    per_call = sum(float(r["TotalDurationNs"]) for r in spmm) / calls / 1000
    with open(os.path.join(prof, "bench_xl.log")) as f:
        j = json.loads([ln for ln in f.read().splitlines() if ln.startswith("{")][-1])
    lines = [
        "# rocprofv3 kernel trace of the default bench run (config `xl`, Auto = "
        f"{j['config']['resolved_algo']} at N={j['config']['N']})", "",
        "Command (repository root on the MI355X box; `bash csrspmm_amd/profile_configs.sh "
        "bench` runs it):", "```",
        "rocprofv3 --kernel-trace --stats -d OUT/bench_xl/trace -o bench_xl --output-format csv "
        "-- python3 bench.py --cpu-seconds 0 --variants none --plan-algo none --configs none", "```", "",
        f"bench.py times {j['warmup']} warmup + {j['steps']} timed calls (plus its timing-mode "
        "calls); its live HIP-event figure for one call (`roofline.kernel_ms`) should match the "
        "per-call sum of the SpMM kernels below.", "",
        f"Kernel sources: digest `{j['roofline'].get('kernel_source_digest')}`.", "",
        "| kernel | calls | avg us | min us | max us |", "|---|---|---|---|---|"]
    for r in spmm:
        lines.append(f"| `{short(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1000:.1f} "
                     f"| {float(r['MinNs']) / 1000:.1f} | {float(r['MaxNs']) / 1000:.1f} |")
    lines += ["", f"SpMM GPU time per call (sum of the averages): {per_call:.1f} us", "",
              f"bench.py output in the same run: ms_per_step {j['ms_per_step']}, SpMM call (all "
              f"launches) {j['roofline']['kernel_ms']} ms, roofline frac {j['roofline']['frac']} "
              f"({j['roofline'].get('frac_basis')})."]
    with open(os.path.join(ROOT, "profiles", "bench_xl_trace.md"), "w") as f:
        f.write("\n".join(lines) + "\n")
    print(f"bench: {per_call:.1f} us per call by trace, {j['roofline']['kernel_ms']} ms live")


def main(argv=None):
    argv = sys.argv[1:] if argv is None else argv
    prof = argv[0] if argv else os.path.join(ROOT, "gpurun_out", "prof")
    tj = os.path.join(ROOT, "profiles", "traffic.json")
    traffic = {}
    if os.path.exists(tj):
        with open(tj) as f:
            traffic = json.load(f)
    commit = _commit()
    for log in sorted(glob.glob(os.path.join(prof, "*.trace.log"))):
        name = os.path.basename(log)[:-len(".trace.log")]
        key, entry = summarize(prof, name)
        entry["commit"] = commit
        traffic[key] = entry
    # An entry whose summary file is gone describes a run nobody can read.
    traffic = {k: v for k, v in traffic.items()
               if os.path.exists(os.path.join(ROOT, "profiles", v.get("summary", "")))}
    with open(tj, "w") as f:
        json.dump(traffic, f, indent=1)
        f.write("\n")
    if os.path.isdir(os.path.join(prof, "bench_xl")):
        summarize_bench(prof)
    return 0


if __name__ == "__main__":
    sys.exit(main())
