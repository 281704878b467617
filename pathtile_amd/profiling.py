"""Summaries of rocprofv3 results (rocpd SQLite ``*_results.db``) as Markdown.

Seven reports, each written for one workload:

``trace``   kernel-trace statistics: calls and average/min/max duration per
            kernel, plus the launch geometry and resources of the largest
            dispatch of each kernel.
``traffic`` HBM bytes per launch from two ``--pmc`` runs (``FETCH_SIZE`` in
            one, ``WRITE_SIZE`` in the other).  Both counters are read in KiB
            per dispatch.  They are scaled by what the same counter reads for
            a plain device-to-device copy of known size (torch ``copy_`` →
            ``__amd_rocclr_copyBuffer``); on MI355X ``FETCH_SIZE`` reads half
            of the bytes a copy loads, ``WRITE_SIZE`` reads them exactly.
``valu``    VALU instruction counts and the VALU-busy fraction from
            ``SQ_INSTS_VALU`` / ``SQ_ACTIVE_INST_VALU`` / ``SQ_BUSY_CYCLES`` /
            ``GRBM_GUI_ACTIVE``, the MFMA-busy fraction from
            ``SQ_VALU_MFMA_BUSY_CYCLES`` when collected, and the useful
            FP32 work as a fraction of the vector and of the matrix FP32
            peaks.
``mfma``    Matrix flops each kernel issues per dispatch, from
            ``SQ_INSTS_VALU_MFMA_MOPS_F32`` / ``..._BF16`` (units of 512
            flops), beside its useful flops; ``--emit SUBSTR=KEY`` writes a
            ``KEY: flops`` line per kernel for bench.py.
``mix``     VALU instruction mix from the ``SQ_INSTS_VALU_*`` class counters:
            each class's share of ``SQ_INSTS_VALU`` and the FP32 fraction
            (FMA + add + multiply in FP32).
``stall``   achieved occupancy (waves per CU and SIMD), the share of wave
            cycles spent waiting, MemUnitStalled, DRAM-credit stalls of the
            L2 channels and the UTCL1 translation miss rate, from counters
            collected over several passes.
``lds``     LDS instructions per wave, LDS-busy fraction per CU, bank-conflict
            share of the LDS cycles and the share of wave cycles waiting for
            LDS, from ``SQ_INSTS_LDS`` / ``SQ_LDS_IDX_ACTIVE`` /
            ``SQ_LDS_BANK_CONFLICT`` / ``SQ_WAIT_INST_LDS`` /
            ``SQ_WAVE_CYCLES`` / ``GRBM_GUI_ACTIVE``.

Only the dispatches with the largest grid of each kernel, and none below a
quarter of its median duration or counter value, are kept, so the small
correctness-gate launches that run before the timed loops are left out.

Usage::

    python -m pathtile_amd.profiling trace   DB --command CMD --out FILE
    python -m pathtile_amd.profiling traffic FETCH_DB WRITE_DB --kernel SUBSTR \
        --tag fwd --algorithmic-bytes N --copy-bytes N --command CMD --out FILE
    python -m pathtile_amd.profiling valu    DB --command CMD --out FILE \
        --useful-fma SUBSTR=N --clock-mhz F
    python -m pathtile_amd.profiling mfma    DB --command CMD --out FILE \
        --useful-fma SUBSTR=N --emit SUBSTR=KEY
    python -m pathtile_amd.profiling mix     DB --command CMD --out FILE
    python -m pathtile_amd.profiling lds     DB --command CMD --out FILE
    python -m pathtile_amd.profiling stall   [LABEL=]DB ... --command CMD --out FILE
"""

from __future__ import annotations

import argparse
import sqlite3
import statistics
from pathlib import Path

COPY_KERNEL = "__amd_rocclr_copyBuffer"
PEAK_FP32_VECTOR = 78.6e12   # MI355X, non-packed FP32 FMA on the SIMDs
PEAK_FP32_MATRIX = 157.3e12  # MI355X dense FP32 matrix cores
# MI355X: 256 CUs x 4 SIMDs; a wave64 VALU op occupies its SIMD16 for 4 cycles.
NUM_SIMDS = 1024
NUM_CUS = 256
CYCLES_PER_WAVE_VALU = 4
NUM_XCD = 8


def short_name(name: str) -> str:
    """Kernel name without the parameter list (template arguments kept)."""
    depth = 0
    for i, ch in enumerate(name):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            return name[:i].replace("void ", "")
    return name


def _largest_dispatches(rows, key_grid, key_value=None):
    """Keep, per kernel name, only the rows whose grid equals its maximum and,
    with `key_value`, whose value is at least a quarter of that kernel's
    median: kernels that size their grid by the GPU rather than the batch
    (persistent and sample-range grids) launch the same grid for the small
    correctness-gate batch, which the value filter then drops."""
    best = {}
    for r in rows:
        best[r["name"]] = max(best.get(r["name"], 0), r[key_grid])
    rows = [r for r in rows if r[key_grid] == best[r["name"]]]
    if key_value is None:
        return rows
    med = {}
    for name in best:
        v = [r[key_value] for r in rows if r["name"] == name]
        med[name] = statistics.median(v) if v else 0
    return [r for r in rows if r[key_value] >= 0.25 * med[r["name"]]]


def kernel_rows(db: str):
    con = sqlite3.connect(db)
    con.row_factory = sqlite3.Row
    rows = [dict(r) for r in con.execute(
        "select name, duration, grid_x*grid_y*grid_z as grid, "
        "workgroup_x*workgroup_y*workgroup_z as wg, lds_size, scratch_size, "
        "vgpr_count, accum_vgpr_count, sgpr_count from kernels")]
    con.close()
    return rows


def counter_rows(db: str, counter: str):
    con = sqlite3.connect(db)
    con.row_factory = sqlite3.Row
    rows = [dict(r) for r in con.execute(
        "select kernel_name as name, dispatch_id, grid_size as grid, value "
        "from counters_collection where counter_name = ?", (counter,))]
    con.close()
    return rows


def trace_report(db: str, command: str, match: str = "pt::") -> str:
    rows = [r for r in kernel_rows(db) if match in r["name"] or r["name"] == COPY_KERNEL]
    rows = _largest_dispatches(rows, "grid", "duration")
    by = {}
    for r in rows:
        by.setdefault(r["name"], []).append(r)
    out = ["| kernel | calls | avg us | min us | median us | max us | grid | wg | VGPR | AGPR | SGPR | LDS B | scratch B |",
           "|---|---|---|---|---|---|---|---|---|---|---|---|---|"]
    for name, rs in sorted(by.items(), key=lambda kv: -sum(r["duration"] for r in kv[1])):
        d = [r["duration"] / 1e3 for r in rs]
        r0 = rs[0]
        out.append(f"| `{short_name(name)}` | {len(rs)} | {statistics.mean(d):.2f} | {min(d):.2f} | "
                   f"{statistics.median(d):.2f} | {max(d):.2f} | {r0['grid']} | {r0['wg']} | "
                   f"{r0['vgpr_count']} | {r0['accum_vgpr_count']} | {r0['sgpr_count']} | "
                   f"{r0['lds_size']} | {r0['scratch_size']} |")
    head = ["Command:", "", "```", command, "```", "",
            "Dispatches with each kernel's largest grid only, and none shorter than a "
            "quarter of that kernel's median (the timed loops; the small "
            "correctness-gate launches are dropped).", ""]
    return "\n".join(head + out) + "\n"


def _mean_counter(db: str, counter: str, match: str):
    rows = _largest_dispatches(
        [r for r in counter_rows(db, counter) if match in r["name"]], "grid", "value")
    if not rows:
        raise SystemExit(f"no {counter} rows for kernels matching {match!r} in {db}")
    vals = [r["value"] for r in rows]
    return statistics.mean(vals), min(vals), max(vals), len(vals), rows[0]["name"]


def _copy_counter(db: str, counter: str):
    """Counter value of the largest plain copy dispatch (KiB)."""
    rows = [r for r in counter_rows(db, counter) if r["name"] == COPY_KERNEL]
    if not rows:
        raise SystemExit(f"no {COPY_KERNEL} dispatches in {db} (run bench.py with --copy-probe)")
    top = max(r["value"] for r in rows)
    vals = [r["value"] for r in rows if r["value"] > 0.9 * top]
    return statistics.mean(vals), len(vals)


def traffic_report(fetch_db: str, write_db: str, kernel: str, tag: str,
                   algorithmic_bytes: int, copy_bytes: int, command: str) -> str:
    kib = 1024.0
    f_mean, f_min, f_max, f_n, name = _mean_counter(fetch_db, "FETCH_SIZE", kernel)
    w_mean, w_min, w_max, w_n, _ = _mean_counter(write_db, "WRITE_SIZE", kernel)
    cf, cf_n = _copy_counter(fetch_db, "FETCH_SIZE")
    cw, cw_n = _copy_counter(write_db, "WRITE_SIZE")
    fetch_factor = copy_bytes / (cf * kib)
    write_factor = copy_bytes / (cw * kib)
    fetch_bytes = f_mean * kib * fetch_factor
    write_bytes = w_mean * kib * write_factor
    lines = [
        f"# HBM traffic per launch: {tag} (`{short_name(name)}`)", "",
        "Commands (two separate passes, one counter each):", "", "```", command, "```", "",
        "| counter | dispatches | mean KiB | min KiB | max KiB | copy probe KiB (n) | scale | bytes/launch |",
        "|---|---|---|---|---|---|---|---|",
        f"| FETCH_SIZE | {f_n} | {f_mean:.1f} | {f_min:.1f} | {f_max:.1f} | {cf:.1f} ({cf_n}) | "
        f"{fetch_factor:.4f} | {fetch_bytes:.0f} |",
        f"| WRITE_SIZE | {w_n} | {w_mean:.1f} | {w_min:.1f} | {w_max:.1f} | {cw:.1f} ({cw_n}) | "
        f"{write_factor:.4f} | {write_bytes:.0f} |",
        "",
        f"Copy probe: {copy_bytes} bytes read and {copy_bytes} bytes written per copy; "
        "scale = copy bytes / (counter KiB x 1024).",
        f"Algorithmic bytes per launch: {algorithmic_bytes}; measured/algorithmic = "
        f"{(fetch_bytes + write_bytes) / algorithmic_bytes:.4f}.",
        "",
        f"FETCH_BYTES_PER_LAUNCH: {fetch_bytes:.0f}",
        f"WRITE_BYTES_PER_LAUNCH: {write_bytes:.0f}",
        "",
    ]
    return "\n".join(lines)


def valu_report(db: str, command: str, useful_fma: dict[str, int], clock_mhz: float,
                match: str = "pt::") -> str:
    counters = ("SQ_WAVES", "SQ_INSTS_VALU", "SQ_ACTIVE_INST_VALU", "SQ_BUSY_CYCLES",
                "GRBM_GUI_ACTIVE", "SQ_WAVE_CYCLES", "SQ_VALU_MFMA_BUSY_CYCLES")
    per = {}
    for c in counters:
        rows = _largest_dispatches(
            [r for r in counter_rows(db, c) if match in r["name"]], "grid", "value")
        for r in rows:
            per.setdefault(r["name"], {}).setdefault(c, []).append(r["value"])
    out = ["Command:", "", "```", command, "```", "",
           f"VALU-busy = SQ_ACTIVE_INST_VALU x {CYCLES_PER_WAVE_VALU} / ({NUM_SIMDS} SIMDs x "
           f"GRBM_GUI_ACTIVE / {NUM_XCD} XCDs). Useful FP32 work = 2 x useful FMAs (multiply-adds "
           f"that touch a real element) / duration, as a fraction of the 78.6 TFLOP/s "
           f"non-packed vector FP32 peak (packed FP32 is off in this build) and of the "
           f"157.3 TFLOP/s dense FP32 matrix peak; duration = GRBM_GUI_ACTIVE / {NUM_XCD} / "
           f"{clock_mhz:.0f} MHz.", "",
           f"MFMA-busy = SQ_VALU_MFMA_BUSY_CYCLES / ({NUM_SIMDS} SIMDs x GRBM_GUI_ACTIVE / "
           f"{NUM_XCD} XCDs) (n/a when that counter was not collected).", "",
           "| kernel | dispatches | waves | VALU insts | VALU insts / wave | VALU-busy | MFMA-busy | useful FMA | of vector FP32 peak | of matrix FP32 peak |",
           "|---|---|---|---|---|---|---|---|---|---|"]
    for name, cs in per.items():
        m = {c: statistics.mean(v) for c, v in cs.items()}
        n = len(cs.get("SQ_INSTS_VALU", []))
        gui = m["GRBM_GUI_ACTIVE"] / NUM_XCD
        busy = m["SQ_ACTIVE_INST_VALU"] * CYCLES_PER_WAVE_VALU / (NUM_SIMDS * gui)
        fma = next((v for k, v in useful_fma.items() if k in name), None)
        if fma is not None:
            secs = gui / (clock_mhz * 1e6)
            frac = f"{2 * fma / secs / PEAK_FP32_VECTOR:.3f}"
            frac_m = f"{2 * fma / secs / PEAK_FP32_MATRIX:.3f}"
            fma_s = str(fma)
        else:
            frac, frac_m, fma_s = "n/a", "n/a", "n/a"
        mfma = (f"{m['SQ_VALU_MFMA_BUSY_CYCLES'] / (NUM_SIMDS * gui):.3f}"
                if "SQ_VALU_MFMA_BUSY_CYCLES" in m else "n/a")
        out.append(f"| `{short_name(name)}` | {n} | {m['SQ_WAVES']:.0f} | {m['SQ_INSTS_VALU']:.0f} | "
                   f"{m['SQ_INSTS_VALU'] / max(m['SQ_WAVES'], 1):.0f} | {busy:.3f} | {mfma} | {fma_s} | "
                   f"{frac} | {frac_m} |")
    return "\n".join(out) + "\n"


def mfma_report(db: str, command: str, useful_fma: dict[str, int], emit: dict[str, str],
                match: str = "pt::") -> str:
    """Matrix flops issued per dispatch (MOPS counters x 512) per kernel."""
    counters = ("SQ_INSTS_VALU_MFMA_MOPS_F32", "SQ_INSTS_VALU_MFMA_MOPS_BF16")
    per = {}
    for c in counters:
        rows = _largest_dispatches(
            [r for r in counter_rows(db, c) if match in r["name"]], "grid", "value")
        for r in rows:
            per.setdefault(r["name"], {}).setdefault(c, []).append(r["value"])
    out = ["Command:", "", "```", command, "```", "",
           "Issued matrix flops per dispatch = SQ_INSTS_VALU_MFMA_MOPS_<type> x 512 (mean over "
           "the dispatches with each kernel's largest grid). Useful flops = 2 x multiply-adds "
           "that touch a real element.", "",
           "| kernel | dispatches | FP32 matrix flops | BF16 matrix flops | useful flops | issued / useful |",
           "|---|---|---|---|---|---|"]
    lines = []
    for name, cs in per.items():
        m = {c: statistics.mean(v) for c, v in cs.items()}
        f32 = m.get("SQ_INSTS_VALU_MFMA_MOPS_F32", 0.0) * 512
        bf16 = m.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", 0.0) * 512
        if f32 == 0 and bf16 == 0:
            continue
        fma = next((v for k, v in useful_fma.items() if k in name), None)
        useful = 2 * fma if fma is not None else None
        ratio = f"{(f32 + bf16) / useful:.2f}" if useful else "n/a"
        n = max(len(v) for v in cs.values())
        out.append(f"| `{short_name(name)}` | {n} | {f32:.4g} | {bf16:.4g} | "
                   f"{useful if useful is not None else 'n/a'} | {ratio} |")
        for sub, key in emit.items():
            if sub in name:
                lines.append(f"{key}: {bf16 if bf16 > 0 else f32:.0f}")
    return "\n".join(out + [""] + sorted(lines)) + "\n"


MIX_COUNTERS = ("SQ_INSTS_VALU", "SQ_INSTS_VALU_FMA_F32", "SQ_INSTS_VALU_ADD_F32",
                "SQ_INSTS_VALU_MUL_F32", "SQ_INSTS_VALU_INT32", "SQ_INSTS_VALU_CVT",
                "SQ_INSTS_VALU_MFMA_F32", "SQ_INSTS_VALU_MFMA_BF16")


def mix_report(db: str, command: str, match: str = "pt::") -> str:
    """VALU instruction mix per kernel: each class as a share of all VALU
    instructions, and the FP32 fraction (FMA + add + multiply in FP32)."""
    per = {}
    for c in MIX_COUNTERS:
        rows = _largest_dispatches(
            [r for r in counter_rows(db, c) if match in r["name"]], "grid", "value")
        for r in rows:
            per.setdefault(r["name"], {}).setdefault(c, []).append(r["value"])
    out = ["Command:", "", "```", command, "```", "",
           "Wave-level instruction counts per dispatch (mean over the dispatches with each "
           "kernel's largest grid), each as a share of SQ_INSTS_VALU. FP32 fraction = "
           "(FMA_F32 + ADD_F32 + MUL_F32) / VALU; MFMA = MFMA_F32 + MFMA_BF16 instructions.", "",
           "| kernel | dispatches | VALU insts | FP32 fraction | FMA_F32 | ADD_F32 | MUL_F32 | INT32 | CVT | MFMA |",
           "|---|---|---|---|---|---|---|---|---|---|"]
    for name, cs in per.items():
        if not all(c in cs for c in MIX_COUNTERS):
            continue
        m = {c: statistics.mean(v) for c, v in cs.items()}
        tot = m["SQ_INSTS_VALU"]
        if tot == 0:
            continue
        sh = {c: m[c] / tot for c in MIX_COUNTERS[1:]}
        fp32 = sh["SQ_INSTS_VALU_FMA_F32"] + sh["SQ_INSTS_VALU_ADD_F32"] + sh["SQ_INSTS_VALU_MUL_F32"]
        mfma = sh["SQ_INSTS_VALU_MFMA_F32"] + sh["SQ_INSTS_VALU_MFMA_BF16"]
        n = len(cs["SQ_INSTS_VALU"])
        out.append(f"| `{short_name(name)}` | {n} | {tot:.0f} | {fp32:.3f} | "
                   f"{sh['SQ_INSTS_VALU_FMA_F32']:.3f} | {sh['SQ_INSTS_VALU_ADD_F32']:.3f} | "
                   f"{sh['SQ_INSTS_VALU_MUL_F32']:.3f} | {sh['SQ_INSTS_VALU_INT32']:.3f} | "
                   f"{sh['SQ_INSTS_VALU_CVT']:.3f} | {mfma:.3f} |")
    return "\n".join(out) + "\n"


def lds_report(db: str, command: str, match: str = "pt::") -> str:
    """LDS load per kernel: instructions per wave, how busy the LDS of a CU
    is, the share of its busy cycles lost to bank conflicts and the share of
    wave cycles spent waiting for LDS results."""
    counters = ("SQ_WAVES", "SQ_INSTS_LDS", "SQ_LDS_IDX_ACTIVE", "SQ_LDS_BANK_CONFLICT",
                "SQ_WAIT_INST_LDS", "SQ_WAVE_CYCLES", "GRBM_GUI_ACTIVE")
    per = {}
    for c in counters:
        rows = _largest_dispatches(
            [r for r in counter_rows(db, c) if match in r["name"]], "grid", "value")
        for r in rows:
            per.setdefault(r["name"], {}).setdefault(c, []).append(r["value"])
    out = ["Command:", "", "```", command, "```", "",
           f"LDS-busy = SQ_LDS_IDX_ACTIVE / ({NUM_CUS} CUs x GRBM_GUI_ACTIVE / {NUM_XCD} XCDs): "
           "the fraction of cycles a CU's LDS serves indexed reads and writes. "
           "Conflict share = SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE: the part of those "
           "cycles spent replaying bank conflicts. LDS wait = SQ_WAIT_INST_LDS / "
           "SQ_WAVE_CYCLES: the fraction of a wave's life spent waiting for LDS results.", "",
           "| kernel | dispatches | waves | LDS insts / wave | LDS-busy | conflict share | LDS wait |",
           "|---|---|---|---|---|---|---|"]
    for name, cs in per.items():
        if not all(c in cs for c in counters):
            continue
        m = {c: statistics.mean(v) for c, v in cs.items()}
        if m["SQ_INSTS_LDS"] == 0:
            continue
        gui = m["GRBM_GUI_ACTIVE"] / NUM_XCD
        busy = m["SQ_LDS_IDX_ACTIVE"] / (NUM_CUS * gui)
        conflict = m["SQ_LDS_BANK_CONFLICT"] / max(m["SQ_LDS_IDX_ACTIVE"], 1)
        wait = m["SQ_WAIT_INST_LDS"] / max(m["SQ_WAVE_CYCLES"], 1)
        n = len(cs["SQ_INSTS_LDS"])
        out.append(f"| `{short_name(name)}` | {n} | {m['SQ_WAVES']:.0f} | "
                   f"{m['SQ_INSTS_LDS'] / max(m['SQ_WAVES'], 1):.0f} | {busy:.3f} | "
                   f"{conflict:.3f} | {wait:.3f} |")
    return "\n".join(out) + "\n"


STALL_COUNTERS = ("MeanOccupancyPerCU", "SQ_WAVE_CYCLES", "SQ_WAIT_ANY", "SQ_WAIT_INST_ANY",
                  "MemUnitStalled", "GRBM_GUI_ACTIVE", "TCC_EA0_RDREQ_DRAM_CREDIT_STALL_sum",
                  "TCC_EA0_WRREQ_DRAM_CREDIT_STALL_sum", "TCP_UTCL1_TRANSLATION_MISS_sum",
                  "TCP_UTCL1_TRANSLATION_HIT_sum")
NUM_TCC = 128  # 16 L2 channels per XCD


def stall_report(dbs: list[str], command: str, match: str = "pt::",
                 labels: list[str] | None = None) -> str:
    """Achieved occupancy and where the waves wait, per kernel (and per
    database, `labels` naming each): mean resident waves per CU
    (MeanOccupancyPerCU) and per SIMD; the share of wave cycles spent
    waiting on anything (SQ_WAIT_ANY / SQ_WAVE_CYCLES) and on an issued
    instruction (SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES); MemUnitStalled (% of
    the time the texture units' data path is stalled); the share of L2
    channel cycles with a read or write request held for lack of DRAM
    credits ((TCC_EA0_*_DRAM_CREDIT_STALL summed over the 128 channels) /
    (128 x GRBM_GUI_ACTIVE / 8)); and the UTCL1 (first-level address
    translation) miss rate. Every counter is read from whichever database
    holds it: collect them in passes that fit the counter blocks."""
    labels = labels or [""] * len(dbs)
    per = {}
    for db, label in zip(dbs, labels):
        for c in STALL_COUNTERS:
            try:
                rows = counter_rows(db, c)
            except sqlite3.Error:
                continue
            rows = _largest_dispatches([r for r in rows if match in r["name"]], "grid", "value")
            for r in rows:
                per.setdefault((label, r["name"]), {}).setdefault(c, []).append(r["value"])
    out = ["Command:", "", "```", command, "```", "",
           "Occupancy = MeanOccupancyPerCU (waves per CU; per SIMD = / 4). Wait = "
           "SQ_WAIT_ANY / SQ_WAVE_CYCLES; wait-inst = SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES. "
           "MemUnitStalled: % of time the TA data path stalls. DRAM credit stall = "
           "TCC_EA0_{RD,WR}REQ_DRAM_CREDIT_STALL summed / (128 L2 channels x GRBM_GUI_ACTIVE / "
           "8 XCDs). UTCL1 miss = misses / (hits + misses). Dispatches with each kernel's "
           "largest grid, none below a quarter of its median counter value.", "",
           "| run | kernel | dispatches | waves/CU | waves/SIMD | wait | wait-inst | "
           "MemUnitStalled % | DRAM credit stall rd | wr | UTCL1 miss |",
           "|---|---|---|---|---|---|---|---|---|---|---|"]

    def fmt(v, spec):
        return "-" if v is None else format(v, spec)

    for (label, name), cs in per.items():
        m = {c: statistics.mean(v) for c, v in cs.items()}
        n = max(len(v) for v in cs.values())
        occ = m.get("MeanOccupancyPerCU")
        wait = (m["SQ_WAIT_ANY"] / m["SQ_WAVE_CYCLES"]
                if "SQ_WAIT_ANY" in m and m.get("SQ_WAVE_CYCLES") else None)
        wait_i = (m["SQ_WAIT_INST_ANY"] / m["SQ_WAVE_CYCLES"]
                  if "SQ_WAIT_INST_ANY" in m and m.get("SQ_WAVE_CYCLES") else None)
        gui = m.get("GRBM_GUI_ACTIVE")
        rd = wr = None
        if gui:
            denom = NUM_TCC * gui / NUM_XCD
            if "TCC_EA0_RDREQ_DRAM_CREDIT_STALL_sum" in m:
                rd = m["TCC_EA0_RDREQ_DRAM_CREDIT_STALL_sum"] / denom
            if "TCC_EA0_WRREQ_DRAM_CREDIT_STALL_sum" in m:
                wr = m["TCC_EA0_WRREQ_DRAM_CREDIT_STALL_sum"] / denom
        miss = None
        if "TCP_UTCL1_TRANSLATION_MISS_sum" in m and "TCP_UTCL1_TRANSLATION_HIT_sum" in m:
            tot = m["TCP_UTCL1_TRANSLATION_MISS_sum"] + m["TCP_UTCL1_TRANSLATION_HIT_sum"]
            miss = m["TCP_UTCL1_TRANSLATION_MISS_sum"] / tot if tot else None
        out.append(f"| {label} | `{short_name(name)}` | {n} | {fmt(occ, '.2f')} | "
                   f"{fmt(None if occ is None else occ / 4, '.2f')} | {fmt(wait, '.3f')} | "
                   f"{fmt(wait_i, '.3f')} | {fmt(m.get('MemUnitStalled'), '.1f')} | "
                   f"{fmt(rd, '.3f')} | {fmt(wr, '.3f')} | {fmt(miss, '.4f')} |")
    return "\n".join(out) + "\n"


def main(argv=None) -> int:
    p = argparse.ArgumentParser(prog="python -m pathtile_amd.profiling")
    sub = p.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("trace")
    t.add_argument("db")
    t.add_argument("--command", required=True)
    t.add_argument("--title", default="Kernel trace")
    t.add_argument("--out", required=True)
    f = sub.add_parser("traffic")
    f.add_argument("fetch_db")
    f.add_argument("write_db")
    f.add_argument("--kernel", required=True, help="substring of the kernel name")
    f.add_argument("--tag", required=True)
    f.add_argument("--algorithmic-bytes", type=int, required=True)
    f.add_argument("--copy-bytes", type=int, required=True)
    f.add_argument("--command", required=True)
    f.add_argument("--out", required=True)
    v = sub.add_parser("valu")
    v.add_argument("db")
    v.add_argument("--command", required=True)
    v.add_argument("--useful-fma", action="append", default=[],
                   help="KERNEL_SUBSTR=N useful FMAs per dispatch (repeatable)")
    v.add_argument("--clock-mhz", type=float, default=2400.0)
    v.add_argument("--title", default="VALU utilisation")
    v.add_argument("--out", required=True)
    m = sub.add_parser("mfma")
    m.add_argument("db")
    m.add_argument("--command", required=True)
    m.add_argument("--useful-fma", action="append", default=[],
                   help="KERNEL_SUBSTR=N useful FMAs per dispatch (repeatable)")
    m.add_argument("--emit", action="append", default=[],
                   help="KERNEL_SUBSTR=KEY: write 'KEY: flops' for that kernel (repeatable)")
    m.add_argument("--title", default="Issued matrix flops")
    m.add_argument("--out", required=True)
    x = sub.add_parser("mix")
    x.add_argument("db")
    x.add_argument("--command", required=True)
    x.add_argument("--title", default="VALU instruction mix")
    x.add_argument("--out", required=True)
    d = sub.add_parser("lds")
    d.add_argument("db")
    d.add_argument("--command", required=True)
    d.add_argument("--title", default="LDS load")
    d.add_argument("--out", required=True)
    st = sub.add_parser("stall")
    st.add_argument("dbs", nargs="+", help="databases of the counter passes; LABEL=DB "
                    "to name a run (several DBs of one run share its label)")
    st.add_argument("--command", required=True)
    st.add_argument("--title", default="Occupancy and stalls")
    st.add_argument("--out", required=True)
    a = p.parse_args(argv)

    def pairs(items, conv):
        d = {}
        for item in items:
            k, _, n = item.rpartition("=")
            d[k] = conv(n)
        return d

    if a.cmd == "trace":
        text = f"# {a.title}\n\n" + trace_report(a.db, a.command)
    elif a.cmd == "traffic":
        text = traffic_report(a.fetch_db, a.write_db, a.kernel, a.tag, a.algorithmic_bytes,
                              a.copy_bytes, a.command)
    elif a.cmd == "valu":
        text = f"# {a.title}\n\n" + valu_report(a.db, a.command, pairs(a.useful_fma, int),
                                                a.clock_mhz)
    elif a.cmd == "mix":
        text = f"# {a.title}\n\n" + mix_report(a.db, a.command)
    elif a.cmd == "lds":
        text = f"# {a.title}\n\n" + lds_report(a.db, a.command)
    elif a.cmd == "stall":
        labels = [d.rpartition("=")[0] if "=" in d else "" for d in a.dbs]
        dbs = [d.rpartition("=")[2] for d in a.dbs]
        text = f"# {a.title}\n\n" + stall_report(dbs, a.command, labels=labels)
    else:
        text = f"# {a.title}\n\n" + mfma_report(a.db, a.command, pairs(a.useful_fma, int),
                                                pairs(a.emit, str))
    Path(a.out).parent.mkdir(parents=True, exist_ok=True)
    Path(a.out).write_text(text)
    print(text)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
