"""CPU tests of bench.py's profile readers: the SQ-counter summary matches each
case's dispatches by launch order (warm-up call dropped, other kernels
skipped) and derives its figures from the counters as its docstring states.
The counter files are synthetic, written the way rocprofv3 --pmc writes them."""

import csv
import os

import bench
from sglite_amd import ops

CU = ops.device_cu_count()
SIMDS, XCDS = 4 * CU, max(1, CU // 32)


def _plan():
    plan = [(f"MFMA probe, {label.replace('_', ' ')}", "mfma_probe_kernel", grid, 256)
            for label, grid in bench.probe_grids(ops).items()]
    for label, M, K, N in bench.SQ_CASES:
        info = ops.plan_info(M, N, K, bench.G)
        plan.append((label, info.function, info.workgroups, info.threads))
    plan += [(label, "Cijk_Ailk_Bljk_HHS_BH", 1024, 256) for label, *_ in bench.SQ_DENSE]
    return plan


def _counters(case: int, warm: bool) -> dict:
    """Counter values of one dispatch: the counted calls of case i give MFMA busy 0.1 + 0.01 i and
    VALU busy 0.2, a wait-issue fraction of 0.3 and 5 + i MFMA instructions per wave; the warm-up
    call gives other values, so a summary that kept it would show them."""
    cyc = 1000.0
    busy = 0.0 if warm else 0.1 + 0.01 * case
    return {"GRBM_GUI_ACTIVE": cyc * XCDS, "SQ_VALU_MFMA_BUSY_CYCLES": busy * SIMDS * cyc,
            "SQ_ACTIVE_INST_VALU": 0.2 * SIMDS * cyc / 4, "SQ_WAVE_CYCLES": 1000.0,
            "SQ_WAIT_INST_ANY": 0.0 if warm else 300.0, "SQ_WAVES": 10.0,
            "SQ_INSTS_MFMA": 10.0 * (5 + case), "SQ_VALU_MFMA_COEXEC_CYCLES": 0.0}


def _write_pass(d: str, counters: list, plan) -> None:
    os.makedirs(d)
    with open(os.path.join(d, "pmc_counter_collection.csv"), "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Grid_Size", "Workgroup_Size", "Counter_Name", "Counter_Value",
                    "Start_Timestamp", "End_Timestamp"])
        did = 0
        for i, (_, fn, wgs, block) in enumerate(plan):
            name = fn + ("_MT64x64(args)" if fn.startswith("Cijk_") else "(args)" if fn == "mfma_probe_kernel"
                         else "<1, 2>(args)")
            name = "void sgl_awq::(anonymous namespace)::" + name if not fn.startswith("Cijk_") else name
            for call in range(1 + bench.SQ_REPS):
                did += 1
                vals = _counters(i, warm=call == 0)
                for c in counters:
                    if c in vals:
                        w.writerow([did, name, wgs * block, block, c, vals[c], 0, 100_000])
                did += 1  # an unrelated dispatch between calls (torch's own kernels)
                for c in counters:
                    w.writerow([did, "elementwise_kernel(args)", 65536, 256, c, 12345.0, 0, 1000])


def test_sq_summary_matches_dispatch_order_and_drops_the_warm_up(tmp_path):
    plan = _plan()
    dirs = []
    for i, p in enumerate(bench.SQ_PASSES):
        d = str(tmp_path / f"pass{i}")
        _write_pass(d, p.split(), plan)
        dirs.append(d)
    md = bench.sq_summary(dirs)
    rows = {r.split("|")[1].strip(): [c.strip() for c in r.split("|")[2:-1]]
            for r in md.splitlines() if r.startswith("| ") and not r.startswith("| case")}
    assert len(rows) == len(plan)
    for i, (label, *_rest) in enumerate(plan):
        cols = rows[label]
        # columns: kernel, us, clock, MFMA busy, rate, VALU busy, co-exec, wait issue, ...
        assert cols[1] == "100.0"
        ghz = 1000.0 / 100_000.0
        assert cols[2] == f"{ghz:.2f}"
        assert cols[3] == f"{0.1 + 0.01 * i:.2f}", (label, cols)
        assert cols[4] == f"{(0.1 + 0.01 * i) * ghz / bench.MFMA_PEAK_GHZ:.2f}"
        assert cols[5] == "0.20"
        assert cols[7] == "0.30"
        assert cols[-1].split(" / ")[1] == str(5 + i)
