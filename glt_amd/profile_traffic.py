"""HBM traffic per launch from rocprofv3 counter passes.

FETCH_SIZE and WRITE_SIZE (KiB per dispatch) are read for the path's kernels
and for a plain device copy of known size (bench.py --calibrate-copy), whose
readings give the factor between counted and true bytes. Usage:

    python -m glt_amd.profile_traffic --fetch F.csv --write W.csv \
        --calib-fetch CF.csv --calib-write CW.csv --out-dir profiles

writes traffic_<label>.json per kernel and prints a markdown table.
"""
import argparse
import collections
import csv
import json
import os

# launch label -> (kernel-name substring, grid-size predicate)
KERNELS = {
    "gate_up": ("gemm_mfma_kernel<unsigned short, 1, true>", None),
    "dinter": ("gemm_mfma_kernel<unsigned short, 2, false>", None),
    "down": ("gemm_mfma_kernel<unsigned short, 0, false>", None),
    # dx and wgrad share an instantiation: dx fills the grid (1024 tiles),
    # wgrad's 3 x 64 tiles do not
    "dx": ("gemm_mfma_kernel<float, 0, false>", lambda g: g >= 256 * 256),
    "wgrad": ("gemm_mfma_kernel<float, 0, false>", lambda g: g < 256 * 256),
    "rmsnorm_fwd": ("rmsnorm_fwd", None),
    "rmsnorm_bwd": ("rmsnorm_bwd", None),
    "adamw_pack": ("adamw_pack_kernel", None),
    "rope": ("rope", None),
    "bake": ("bake_kernel", None),
    "clip_sumsq": ("sumsq_partial_kernel", None),
    "shuffle_tr": ("shuffle_tr16_kernel<true>", None),
    "transpose16": ("transpose16_kernel", None),
}


def per_dispatch(path, counter):
    """{kernel name: [value per dispatch]} for one counter."""
    out = collections.defaultdict(list)
    for r in csv.DictReader(open(path)):
        if r["Counter_Name"] != counter:
            continue
        out[(r["Kernel_Name"], int(r["Grid_Size"]))].append(float(r["Counter_Value"]))
    return out


def pick(table, name_sub, grid_ok):
    vals = []
    for (name, grid), v in table.items():
        if name_sub in name and (grid_ok is None or grid_ok(grid)):
            vals.extend(v)
    return sum(vals) / len(vals) if vals else None


def copy_reading(table, nbytes):
    """Mean reading (KiB) of the calibration copy: the dispatches whose name
    says copy, else the largest non-fill kernel."""
    cands = {k: v for k, v in table.items() if "copy" in k[0].lower()}
    if not cands:
        cands = {k: v for k, v in table.items() if "fill" not in k[0].lower()}
    vals = max(cands.values(), key=lambda v: sum(v) / len(v))
    return sum(vals) / len(vals)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--fetch", required=True)
    ap.add_argument("--write", required=True)
    ap.add_argument("--calib-fetch", required=True)
    ap.add_argument("--calib-write", required=True)
    ap.add_argument("--calib-bytes", type=int, default=1 << 30)
    ap.add_argument("--out-dir", default=None)
    args = ap.parse_args()

    fetch, write = per_dispatch(args.fetch, "FETCH_SIZE"), per_dispatch(args.write, "WRITE_SIZE")
    cf = copy_reading(per_dispatch(args.calib_fetch, "FETCH_SIZE"), args.calib_bytes) * 1024 / args.calib_bytes
    cw = copy_reading(per_dispatch(args.calib_write, "WRITE_SIZE"), args.calib_bytes) * 1024 / args.calib_bytes
    print(f"copy calibration: FETCH_SIZE reads {cf:.4f} x true bytes, WRITE_SIZE {cw:.4f} x\n")
    print("| kernel | FETCH_SIZE KiB/launch | WRITE_SIZE KiB/launch | HBM bytes/launch (calibrated) |")
    print("|---|---|---|---|")
    for label, (sub, grid_ok) in KERNELS.items():
        f, w = pick(fetch, sub, grid_ok), pick(write, sub, grid_ok)
        if f is None or w is None:
            continue
        hbm = f * 1024 / cf + w * 1024 / cw
        print(f"| {label} | {f:,.0f} | {w:,.0f} | {hbm:,.0f} |")
        if args.out_dir:
            with open(os.path.join(args.out_dir, f"traffic_{label}.json"), "w") as fh:
                json.dump({"kernel": label, "fetch_kib_per_launch": f, "write_kib_per_launch": w,
                           "copy_fetch_factor": cf, "copy_write_factor": cw,
                           "hbm_bytes_per_launch": round(hbm)}, fh, indent=1)


if __name__ == "__main__":
    main()
