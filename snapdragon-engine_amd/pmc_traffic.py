"""HBM traffic of the timed kernel from rocprofv3 counter runs (profiling helper).

Reads three pairs of `rocprofv3 --pmc FETCH_SIZE` / `--pmc WRITE_SIZE` CSV outputs: the bench's
`--pmc-probe` run (the fused verify launches) and `--calibrate-copy` (a 1 GiB device copy, whose
true read and write bytes are known), scales the probe's per-dispatch counters by the copy's
measured/true ratio and writes profiles/<key>_traffic.json, which bench.py uses for the roofline's
`traffic` field.

    python snapdragon-engine_amd/pmc_traffic.py --probe-fetch DIR --probe-write DIR \\
        --copy-fetch DIR --copy-write DIR --probe-json FILE [--out profiles/fused_verify_traffic.json]

For a kernel launched outside the engine (a fixed shape, e.g. the K-quant GEMV of `bench.py --kquant`),
--algorithmic BYTES replaces --probe-json and every dispatch of --kernel (a name substring) counts:

    python snapdragon-engine_amd/pmc_traffic.py --probe-fetch DIR --probe-write DIR --copy-fetch DIR \\
        --copy-write DIR --kernel "vl_gemv_kernel<6, 2, 8>" --algorithmic 419168832 \\
        --out profiles/kquant_lm_head_traffic.json
"""
import argparse
import csv
import glob
import json
import os


def rows(d):
    out = []
    for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
        with open(f) as fh:
            out.extend(csv.DictReader(fh))
    if not out:
        raise SystemExit(f"no counter_collection.csv under {d}")
    return out


def per_dispatch(d, counter, name_sub):
    """{dispatch id: counter value (KiB)} for kernels whose name contains name_sub."""
    vals = {}
    for r in rows(d):
        if r.get("Counter_Name") != counter or name_sub not in r.get("Kernel_Name", ""):
            continue
        k = int(r["Dispatch_Id"])
        vals[k] = vals.get(k, 0.0) + float(r["Counter_Value"])
    return vals


def largest(vals, n):
    """The n largest dispatches (the verify runs: ~10x the draft run's bytes)."""
    return sorted(vals.values(), reverse=True)[:n]


def main():
    ap = argparse.ArgumentParser()
    for k in ("probe-fetch", "probe-write", "copy-fetch", "copy-write"):
        ap.add_argument("--" + k, required=True)
    ap.add_argument("--probe-json")
    ap.add_argument("--algorithmic", type=int)
    ap.add_argument("--kernel", default="fused_kernel")
    ap.add_argument("--out", default=os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "profiles",
                                                  "fused_verify_traffic.json"))
    a = ap.parse_args()
    if a.probe_json:
        with open(a.probe_json) as f:
            probe = next(json.loads(line) for line in f if line.startswith("{") and "pmc_probe" in line)
    elif a.algorithmic:
        probe = {"pmc_probe": a.kernel, "algorithmic_bytes_per_launch": a.algorithmic,
                 "launches": len(per_dispatch(a.probe_fetch, "FETCH_SIZE", a.kernel))}
    else:
        raise SystemExit("--probe-json or --algorithmic is required")
    n = probe["launches"]
    copy_bytes = 1 << 30
    cf = largest(per_dispatch(a.copy_fetch, "FETCH_SIZE", ""), 1)[0] * 1024
    cw = largest(per_dispatch(a.copy_write, "WRITE_SIZE", ""), 1)[0] * 1024
    kf = sum(largest(per_dispatch(a.probe_fetch, "FETCH_SIZE", a.kernel), n)) / n * 1024
    kw = sum(largest(per_dispatch(a.probe_write, "WRITE_SIZE", a.kernel), n)) / n * 1024
    ff, fw = copy_bytes / cf, copy_bytes / cw
    fetch, write = kf * ff, kw * fw
    res = {
        "kernel": probe["pmc_probe"],
        "launches": n,
        "fetch_bytes_per_launch_raw": int(kf),
        "write_bytes_per_launch_raw": int(kw),
        "copy_calibration": {"bytes": copy_bytes, "fetch_raw": int(cf), "write_raw": int(cw),
                             "fetch_factor": round(ff, 4), "write_factor": round(fw, 4)},
        "hbm_bytes_per_launch": int(fetch + write),
        "algorithmic_bytes_per_launch": probe["algorithmic_bytes_per_launch"],
        "traffic_over_algorithmic": round((fetch + write) / probe["algorithmic_bytes_per_launch"], 4),
    }
    for k in ("positions", "union_experts_per_moe_layer"):
        if k in probe:
            res[k] = probe[k]
    os.makedirs(os.path.dirname(os.path.abspath(a.out)), exist_ok=True)
    with open(a.out, "w") as f:
        json.dump(res, f, indent=1)
    print(json.dumps(res))


if __name__ == "__main__":
    main()
