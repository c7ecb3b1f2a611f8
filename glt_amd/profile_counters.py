"""Per-dispatch SQ/TA counters of this library's GEMM kernels beside the
vendor library's kernels on the same shapes, from rocprofv3 --pmc passes of
`bench.py --vendor` (one pass per counter group; commands in
profiles/gemm_vs_hipblaslt_counters.md). Usage:

    python -m glt_amd.profile_counters P1.csv P2.csv ... > table.md

Each column is the median over a kernel's dispatches of one shape. The
vendor's launches are told apart by order: `bench.py --vendor` times gate/up,
down and dInter (one kernel name, equal dispatch counts, in that order), then
dX (another kernel name).
"""
import collections
import csv
import statistics
import sys

OURS = {
    "gate_up (ours)": "gemm_mfma_kernel<unsigned short, 1, true>",
    "down (ours)": "gemm_mfma_kernel<unsigned short, 0, false>",
    "dinter (ours)": "gemm_mfma_kernel<unsigned short, 2, false>",
    "dx (ours)": "gemm_mfma_kernel<float, 0, false>",
}
VENDOR_TN = "Cijk_Alik_Bljk"   # gate/up, down, dInter in that order
VENDOR_NN = "Cijk_Ailk_Bljk"   # dX
# algorithmic FLOP of each shape (16384 tokens, hidden 4096, N = 14336 + 1024)
_M, _D, _N = 16384, 4096, 15360
FLOP = {"gate_up": 2 * _M * _D * 2 * _N, "down": 2 * _M * _N * _D, "dinter": 2 * _M * _D * _N,
        "dx": 2 * _M * 2 * _N * _D}
TILE_STEP = 2 * 256 * 256 * 64   # FLOP of one 64-deep step of a 256 x 256 tile


def load(paths):
    """{(dispatch id, kernel name, grid): {counter: value}}"""
    out = collections.defaultdict(dict)
    for p in paths:
        for r in csv.DictReader(open(p)):
            key = (int(r["Dispatch_Id"]), r["Kernel_Name"], int(r["Grid_Size"]))
            out[key][r["Counter_Name"]] = out[key].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    return out


def groups(d):
    g = {}
    for label, sub in OURS.items():
        # the dX launches fill the grid with 1024 tiles; the weight-gradient
        # launch of the same instantiation has 192
        g[label] = [v for (i, n, gr), v in sorted(d.items()) if sub in n and "Cijk" not in n]
    tn = [v for (i, n, gr), v in sorted(d.items()) if VENDOR_TN in n and gr >= 256 * 256]
    k = len(tn) // 3
    for j, name in enumerate(("gate_up", "down", "dinter")):
        g[f"{name} (hipBLASLt)"] = tn[j * k:(j + 1) * k]
    g["dx (hipBLASLt)"] = [v for (i, n, gr), v in sorted(d.items()) if VENDOR_NN in n and gr >= 256 * 256]
    return g


def med(vals, c):
    xs = [v[c] for v in vals if c in v]
    return statistics.median(xs) if xs else None


def main():
    d = load(sys.argv[1:])
    g = {k: v for k, v in groups(d).items() if v}
    # dX (ours): the launches that are not the weight-gradient one are the
    # largest by MFMA count
    if "dx (ours)" in g:
        mx = max(v.get("SQ_INSTS_MFMA", 0) for v in g["dx (ours)"])
        g["dx (ours)"] = [v for v in g["dx (ours)"] if v.get("SQ_INSTS_MFMA", 0) > 0.5 * mx]
    counters = sorted({c for vals in g.values() for v in vals for c in v})
    cols = list(g)
    print("| counter | " + " | ".join(cols) + " |")
    print("|---" * (len(cols) + 1) + "|")
    for c in counters:
        print(f"| {c} | " + " | ".join(f"{med(g[k], c):,.0f}" if med(g[k], c) is not None else "" for k in cols) + " |")
    # per 64-deep step of a 256 x 256 tile (one workgroup's K-step in both
    # kernels), so the two MFMA shapes compare on equal work
    print()
    print("| per 256x256x64 tile step | " + " | ".join(cols) + " |")
    print("|---" * (len(cols) + 1) + "|")
    for c in counters:
        row = []
        for k in cols:
            a = med(g[k], c)
            steps = FLOP[k.split(" ")[0]] / TILE_STEP
            row.append(f"{a / steps:.2f}" if a is not None else "")
        print(f"| {c} | " + " | ".join(row) + " |")


if __name__ == "__main__":
    main()
