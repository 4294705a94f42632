"""HBM traffic per verify GEMM launch from two rocprofv3 counter runs of
`bench.py --mode gemm` (one with --pmc FETCH_SIZE, one with --pmc WRITE_SIZE).

Counters are KiB per dispatch.  They are scaled by what the same counter
reads for the calibration copy (a device-to-device copy of 256 MiB,
__amd_rocclr_copyBuffer) and grouped by (kernel, grid size): bench.py runs
one grid size per shape, in the order of SHAPES.  The verify-step figure is
the launch-weighted mean over one target forward at M = 9: 32 layers x
(QKV, O, gate/up, down) + the output projection.

usage: python traffic_summary.py fetch_counter_collection.csv write_counter_collection.csv
"""
import csv
import sys
from collections import OrderedDict

SHAPES = ["Q4_0 4096x4096", "Q4_0 12288x4096", "Q4_0 4096x11008", "Q4_0 22016x4096",
          "Q4_0 32000x4096", "Q8_0 11008x4096", "Q8_0 4096x11008"]
ALG = {  # algorithmic bytes per launch at M = 9
    s: (r * c // 32 * (18 if s.startswith("Q4") else 34) + 4 * 9 * c + 4 * 9 * r)
    for s, (r, c) in zip(SHAPES, [(4096, 4096), (12288, 4096), (4096, 11008), (22016, 4096),
                                  (32000, 4096), (11008, 4096), (4096, 11008)])}
VERIFY_MIX = {"Q4_0 12288x4096": 32, "Q4_0 4096x4096": 32, "Q4_0 22016x4096": 32,
              "Q4_0 4096x11008": 32, "Q4_0 32000x4096": 1}
CAL_BYTES = 256 << 20


def load(path, counter):
    groups = OrderedDict()
    cal = []
    with open(path) as f:
        for d in csv.DictReader(f):
            if d.get("Counter_Name") != counter:
                continue
            name, v = d["Kernel_Name"], float(d["Counter_Value"]) * 1024.0
            if name.startswith("__amd_rocclr_copyBuffer") and v > CAL_BYTES / 2:
                cal.append(v)
            elif name.startswith("void vx_gemm_kernel"):
                key = (name.split("(")[0], d["Grid_Size"])
                groups.setdefault(key, []).append(v)
    return groups, cal


def main():
    fetch, fcal = load(sys.argv[1], "FETCH_SIZE")
    write, wcal = load(sys.argv[2], "WRITE_SIZE")
    ff = CAL_BYTES / (sum(fcal) / len(fcal))
    wf = CAL_BYTES / (sum(wcal) / len(wcal))
    print(f"calibration: copy of {CAL_BYTES} B reads FETCH {sum(fcal)/len(fcal):.0f} B "
          f"(factor {ff:.4f}), WRITE {sum(wcal)/len(wcal):.0f} B (factor {wf:.4f})")
    keys = list(fetch.keys())
    if len(keys) != len(SHAPES):
        print(f"expected {len(SHAPES)} GEMM groups, found {len(keys)}: {keys}")
    per = {}
    print(f"{'shape (M=9)':18s} {'kernel':34s} {'launches':>8s} {'alg MB':>8s} {'fetch MB':>9s} {'write MB':>9s} {'traffic/alg':>11s}")
    for shape, key in zip(SHAPES, keys):
        fv = sum(fetch[key]) / len(fetch[key]) * ff
        wv = sum(write.get(key, [0.0])) / max(1, len(write.get(key, []))) * wf
        per[shape] = fv + wv
        print(f"{shape:18s} {key[0][5:39]:34s} {len(fetch[key]):8d} {ALG[shape]/1e6:8.2f} {fv/1e6:9.2f} "
              f"{wv/1e6:9.2f} {(fv + wv)/ALG[shape]:11.3f}")
    n = sum(VERIFY_MIX.values())
    t = sum(per[s] * c for s, c in VERIFY_MIX.items()) / n
    a = sum(ALG[s] * c for s, c in VERIFY_MIX.items()) / n
    print(f"verify mix (32 x QKV/O/gate-up/down + output, M=9): algorithmic {a:.0f} B/launch")
    print(f"traffic_bytes_per_launch: {t:.0f}")


if __name__ == "__main__":
    main()
