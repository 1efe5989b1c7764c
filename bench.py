"""Benchmark of the CRESSO5 hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c1|c2|c3|c4|c5|copy] [--no-cpu]

With no --workload, the headline configs run first: C2 gives the line's
`value`, `ms_per_step`, `roofline`, `cpu_baseline` and `parity`; C3 (the
metric's second config, with its own CPU leg and parity) and the timing-only
C4 and C5 lines follow under `secondary`.
    python bench.py --rocprof-summary DIR [DIR ...] [--calib DIR ...] [--launches N]

Workloads:
  c1: one fp32 (2048,2048) parameter, rank 8 (the reference's CPU-runnable case).
  c2: one fp32 (4096,4096) parameter, spectral/hash route, rank 8, F=5, B=64, T=2;
      grads N(0,1e-3) with 1% of entries x50, fresh per step.
  c3: 840 LoRA-thin fp32 matrices alternating (4096,16)/(16,4096), scalar route,
      rank 4; per-tensor scale 10^U(-4,-1) times N(0,1e-2).
  c4: the 1.2 B-element transformer set (fp32, rank 8; inputs drawn on the device).
  c5: bf16 (8192,8192) and fp32 conv / 3-D tensors at rank 16, F=7, B=256, T=4.
  copy: calibration only -- torch's device copy of a 256 MiB fp32 buffer, the
      plain copy kernel of known size that scales rocprofv3's FETCH_SIZE and
      WRITE_SIZE counters to bytes.
Inputs are resident in HBM before the timed region; each step's grads are
pre-generated on the device (C2: a pool of 4 grad sets cycled through; C3 and
C4: one set, assigned before the first step), so the timed region holds only
optimizer.step() (and, for C2, one p.grad assignment a step).

The --rocprof-summary mode turns rocprofv3 CSV output (--output-format csv)
in DIR into markdown tables: per-kernel durations from *kernel_stats.csv, and
per-kernel counter means per dispatch from *counter_collection.csv, with the
HBM byte counters scaled by the copy calibration in --calib (FETCH_SIZE and
WRITE_SIZE of the known-size copy) and summed per launch of the hot path
(--launches = optimizer steps the profiled run executed).

Prints ONE JSON line.  `value` is the algorithmic HBM throughput of a step
(grad read + param read + param write, 12 B per fp32 element) in GB/s.
`roofline.achieved` is the same algorithmic bytes over one step's mean
duration in the timed region: one pair of HIP events on the launch stream
around the K steps (an event pair around every step would add its own cost,
7-15 us a step, so the timed region holds none).  `roofline.traffic` is the
HBM bytes per step from the committed rocprofv3 counter summary, reported only
when that summary was measured on the current kernel sources (a digest of
cresso_amd/csrc/ recorded in it).  `cpu_baseline` times the CPU oracle (a port
of the reference's cuda_ops="off" path) on the host cores, and `parity`
compares a fresh GPU optimizer with it after the same steps on the timed
leg's own inputs (cpu_and_parity).
"""

from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
METRIC = "optimizer ms/step + achieved HBM GB/s (% peak): 4096² rank-8, 840 LoRA-thin"


def lora_shapes(count=840):
    return [(4096, 16) if i % 2 == 0 else (16, 4096) for i in range(count)]


def make_c3(device, pool=4, seed=0):
    gen = torch.Generator().manual_seed(seed)
    shapes = lora_shapes()
    scales = (10.0 ** (torch.rand(len(shapes), generator=gen, dtype=torch.float64) * 3.0 - 4.0)).tolist()
    params = [torch.nn.Parameter((0.02 * torch.randn(s, generator=gen)).to(device)) for s in shapes]
    grads = []
    for _ in range(pool):
        grads.append([(sc * 1e-2 * torch.randn(s, generator=gen)).to(device) for s, sc in zip(shapes, scales)])
    kwargs = dict(lr=2e-3, rank=4, hash_bins=64, hash_tables=2)
    return params, grads, kwargs, shapes, scales


def make_forms(device, pool=1, seed=0):
    """Profile-only group (not a bench line) for the scalar route's other launch
    forms: 256 small thin tensors (scalar_stream_kernel), 4 large thin tensors
    (the wide form's passes and finishes) and 64 micro-route tensors
    (micro_kernel), one scalar plan."""
    gen = torch.Generator().manual_seed(seed)
    shapes = [(999, 7)] * 256 + [(262144, 32)] * 4 + [(64, 64)] * 64
    params = [torch.nn.Parameter((0.02 * torch.randn(s, generator=gen)).to(device)) for s in shapes]
    grads = []
    for _ in range(pool):
        grads.append([(1e-3 * torch.randn(s, generator=gen)).to(device) for s in shapes])
    kwargs = dict(lr=2e-3, rank=4, hash_bins=64, hash_tables=2, micro_field_max_size=4096)
    return params, grads, kwargs, shapes, None


def make_c2(device, pool=4, seed=0):
    gen = torch.Generator().manual_seed(seed)
    shape = (4096, 4096)
    params = [torch.nn.Parameter((0.02 * torch.randn(shape, generator=gen)).to(device))]
    grads = []
    for _ in range(pool):
        g = 1e-3 * torch.randn(shape, generator=gen)
        mask = torch.rand(shape, generator=gen) < 0.01
        grads.append([torch.where(mask, g * 50.0, g).to(device)])
    kwargs = dict(lr=2e-3, rank=8, max_frequency=5, hash_bins=64, hash_tables=2)
    return params, grads, kwargs, [shape], None


def make_c1(device, pool=10, seed=0):
    """C1 (the reference's CPU-runnable case): one fp32 (2048,2048) param, p0 = 0.02 randn, then
    a fresh grad 1e-3 randn per step from the same generator (seed 0); rank 8, F = 5, B = 64, T = 2."""
    gen = torch.Generator().manual_seed(seed)
    shape = (2048, 2048)
    params = [torch.nn.Parameter((0.02 * torch.randn(shape, generator=gen)).to(device))]
    grads = [[(1e-3 * torch.randn(shape, generator=gen)).to(device)] for _ in range(pool)]
    kwargs = dict(lr=2e-3, rank=8, max_frequency=5, hash_bins=64, hash_tables=2)
    return params, grads, kwargs, [shape], None


C4_SHAPES = [(32000, 2048), (2048, 2048), (5632, 2048), (2048, 5632), (2048,)]


def c4_layer_shapes(layers=22):
    """The full C4 set: embedding, then per layer q,k,v,o, gate, up, down and two RMSNorm weights."""
    out = [(32000, 2048)]
    for _ in range(layers):
        out += [(2048, 2048)] * 4 + [(5632, 2048)] * 2 + [(2048, 5632)] + [(2048,)] * 2
    return out


def make_c4(device, pool=2, seed=0, shapes=None, on_device=False):
    """C4: fp32 tensors, grads N(0, sigma) with sigma = 10^U(-5,-2) per tensor; p0 = 0.02 randn.
    shapes=None is the full 1.2 B-element set; C4_SHAPES is one tensor of each distinct shape.
    on_device: draw params and grads with a generator on `device` (the timing leg of the full
    set; 3.6 G draws on the host would take minutes)."""
    shapes = c4_layer_shapes() if shapes is None else shapes
    gen = torch.Generator().manual_seed(seed)
    sig = (10.0 ** (torch.rand(len(shapes), generator=gen, dtype=torch.float64) * 3.0 - 5.0)).tolist()
    if on_device:
        gen = torch.Generator(device=device).manual_seed(seed)
        draw = lambda s: torch.randn(s, generator=gen, device=device)   # noqa: E731
    else:
        draw = lambda s: torch.randn(s, generator=gen).to(device)   # noqa: E731
    params = [torch.nn.Parameter(0.02 * draw(s)) for s in shapes]
    grads = [[sc * draw(s) for s, sc in zip(shapes, sig)] for _ in range(pool)]
    kwargs = dict(lr=2e-3, rank=8, max_frequency=5, hash_bins=64, hash_tables=2)
    return params, grads, kwargs, shapes, sig


C5_SHAPES = [(8192, 8192), (512, 256, 3, 3), (256, 256, 3, 3), (64, 512, 512)]
C5_DTYPES = [torch.bfloat16, torch.float32, torch.float32, torch.float32]


def make_c5(device, pool=2, seed=0):
    """C5: bf16 (8192,8192) with bf16 grads, fp32 conv and 3-D tensors; grads N(0, 1e-3) in the
    parameter dtype (drawn in fp32, then cast); p0 = 0.02 randn.  rank 16, F = 7, B = 256, T = 4."""
    gen = torch.Generator().manual_seed(seed)
    params = [torch.nn.Parameter((0.02 * torch.randn(s, generator=gen)).to(dt).to(device))
              for s, dt in zip(C5_SHAPES, C5_DTYPES)]
    grads = [[(1e-3 * torch.randn(s, generator=gen)).to(dt).to(device) for s, dt in zip(C5_SHAPES, C5_DTYPES)]
             for _ in range(pool)]
    kwargs = dict(lr=2e-3, rank=16, max_frequency=7, hash_bins=256, hash_tables=4)
    return params, grads, kwargs, C5_SHAPES, None


TRAFFIC_FILES = {"c2": "profiles/spectral_step_c2_hbm_traffic.md", "c3": "profiles/scalar_step_c3_hbm_traffic.md",
                 "c4": "profiles/spectral_step_c4_hbm_traffic.md", "c5": "profiles/spectral_step_c5_hbm_traffic.md"}
SOURCE_GLOBS = ("cresso_amd/csrc/*.hip", "cresso_amd/csrc/*.hpp", "cresso_amd/csrc/*.cpp")


def source_digest():
    """Digest of the library's kernel sources: a traffic figure measured on other sources is stale."""
    import hashlib
    h = hashlib.sha256()
    for pat in SOURCE_GLOBS:
        for path in sorted(ROOT.glob(pat)):
            h.update(path.name.encode())
            h.update(path.read_bytes())
    return h.hexdigest()[:16]


def measured_traffic(workload):
    """HBM bytes per launch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary of
    this workload (scaled by the copy calibration) -> (bytes or None, note).  The summary
    records the digest of the kernel sources it was measured on; a figure measured on other
    sources is not reported."""
    path = ROOT / TRAFFIC_FILES.get(workload, "-")
    if not path.is_file():
        return None, "no profile"
    nbytes, digest = None, None
    for line in path.read_text().splitlines():
        if line.startswith("- scaled HBM bytes"):
            nbytes = int(float(line.rsplit(":", 1)[1]))
        if line.startswith("- kernel source digest:"):
            digest = line.rsplit(":", 1)[1].strip()
    cur = source_digest()
    if digest != cur:
        return None, f"{TRAFFIC_FILES[workload]} was measured on kernel sources {digest}, these are {cur}"
    return nbytes, f"{TRAFFIC_FILES[workload]} (rocprofv3 FETCH_SIZE + WRITE_SIZE, kernel sources {cur})"


def algorithmic_bytes(params):
    """Compulsory bytes of a step: grad read + param read + param write per element, in the
    param's dtype (12 B fp32, 6 B bf16); state traffic (< 4 KiB a tensor) is ignored."""
    n = sum(p.numel() for p in params)
    return sum(3 * p.element_size() * p.numel() for p in params), n


def time_gpu(workload, steps, warmup, maker=None):
    import cresso_amd

    device = torch.device("cuda:0")
    params, grads, kwargs, shapes, _ = (maker or TIMING_MAKERS.get(workload, MAKERS[workload]))(device)
    nbytes, n = algorithmic_bytes(params)
    opt = cresso_amd.CRESSO5(params, cuda_ops="required", **kwargs)
    pool = len(grads)

    def set_grads(k):
        if pool == 1 and k > 0:
            return   # the same grads every step (set before the first)
        for p, g in zip(params, grads[k % pool]):
            p.grad = g

    for k in range(warmup):
        set_grads(k)
        opt.step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(device)
    # the timed region: K steps between two events (events recorded between
    # the steps would add their own cost, about 7-15 us a step, to the steps)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for k in range(steps):
        set_grads(warmup + k)
        opt.step()
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    total_ms = start.elapsed_time(end)
    # host cost of the grad assignments alone (no optimizer work): what a
    # caller that swaps grad sets every step pays on top of the step
    t1 = time.perf_counter()
    for k in range(steps):
        for p, g in zip(params, grads[k % pool]):
            p.grad = g
    assign_ms = 1e3 * (time.perf_counter() - t1) / steps
    return dict(ms_per_step=total_ms / steps, wall_ms_per_step=1e3 * wall / steps, shapes=shapes, kwargs=kwargs,
                nbytes=nbytes, n=n, pool=pool, assign_ms=assign_ms)


def copy_calibration(steps, warmup, nbytes=256 << 20):
    """Plain device copy of a known size, for scaling the HBM byte counters."""
    device = torch.device("cuda:0")
    src = torch.randn(nbytes // 4, device=device)
    dst = torch.empty_like(src)
    for _ in range(warmup):
        dst.copy_(src)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        dst.copy_(src)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    return dict(read_bytes=nbytes, write_bytes=nbytes, ms_per_copy=round(ms, 4),
                gb_s=round(2 * nbytes / (ms * 1e-3) / 1e9, 1))


# ---------------------------------------------------------------------------
# rocprofv3 CSV summaries
# ---------------------------------------------------------------------------
_SETUP = ("ws_", "zero_u64")  # one-time workspace set-up kernels of the library


def _hot(name: str) -> bool:
    """A kernel of the library's per-step launch (not torch's, not set-up)."""
    return "cresso::" in name and not _short_kernel(name).startswith(_SETUP)


def _short_kernel(name: str) -> str:
    import re
    m = re.search(r"cresso::(?:\(anonymous namespace\)::)?(\w+)", name)
    if m:
        return m.group(1)
    if "copyBuffer" in name:
        return "__amd_rocclr_copyBuffer"
    return name.split("(")[0][-60:]


def _read_csv(path):
    import csv
    with open(path, newline="") as fh:
        return list(csv.DictReader(fh))


def _counter_means(paths, by_grid=False):
    """{kernel: {counter: (mean value per dispatch, dispatches)}}; rows of one
    dispatch (counter dimensions) are summed first.  by_grid: keyed by
    "kernel @ workgroups" instead."""
    from collections import defaultdict
    per = defaultdict(float)
    names = {}
    for path in paths:
        for row in _read_csv(path):
            key = (path, row["Dispatch_Id"], row["Counter_Name"])
            per[key] += float(row["Counter_Value"])
            name = ("*" if _hot(row["Kernel_Name"]) else "") + _short_kernel(row["Kernel_Name"])
            if by_grid:
                name += f" @ {int(row['Grid_Size']) // max(1, int(row['Workgroup_Size']))}"
            names[(path, row["Dispatch_Id"])] = name
    agg = defaultdict(lambda: defaultdict(list))
    for (path, did, cn), v in per.items():
        agg[names[(path, did)]][cn].append(v)
    return {k: {cn: (sum(v) / len(v), len(v)) for cn, v in d.items()} for k, d in agg.items()}


def _trace_means(paths):
    """{"kernel @ workgroups": mean duration in us} of the library's kernels
    over the given kernel-trace files."""
    from collections import defaultdict
    acc = defaultdict(lambda: [0, 0.0])
    for path in paths:
        for r in _read_csv(path):
            if not _hot(r["Kernel_Name"]):
                continue
            wg = max(1, int(r["Workgroup_Size_X"]) * int(r["Workgroup_Size_Y"]) * int(r["Workgroup_Size_Z"]))
            blocks = (int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])) // wg
            a = acc[f"{_short_kernel(r['Kernel_Name'])} @ {blocks}"]
            a[0] += 1
            a[1] += (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    return {k: tot / n for k, (n, tot) in acc.items()}


def _copy_reading(calib_dirs, counter):
    """Median reading of `counter` over the 256 MiB copies of `bench.py --workload copy`."""
    import glob
    from collections import defaultdict
    vals = defaultdict(float)
    for d in calib_dirs:
        for path in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for row in _read_csv(path):
                if row["Counter_Name"] == counter and "copyBuffer" in row["Kernel_Name"]:
                    vals[(path, row["Dispatch_Id"])] += float(row["Counter_Value"])
    if not vals:
        return None
    big = sorted(v for v in vals.values() if v >= 0.5 * max(vals.values()))
    return big[len(big) // 2]


def rocprof_summary(dirs, calib=None, launches=None):
    import glob
    if isinstance(dirs, str):
        dirs = [dirs]
    out = []

    def found(pattern):
        return sorted(p for d in dirs for p in glob.glob(os.path.join(d, "**", pattern), recursive=True))

    for path in found("*kernel_stats.csv"):
        rows = _read_csv(path)
        out.append(f"### Kernel durations ({os.path.basename(path)})\n")
        out.append("| kernel | calls | avg us | min us | max us | % |")
        out.append("|---|---:|---:|---:|---:|---:|")
        per_launch = 0.0
        for r in rows:
            k = _short_kernel(r["Name"])
            avg = float(r["AverageNs"]) / 1e3
            calls = int(r["Calls"])
            out.append(f"| {k} | {calls} | {avg:.2f} | {float(r['MinNs'])/1e3:.2f} | {float(r['MaxNs'])/1e3:.2f} | "
                       f"{float(r['Percentage']):.1f} |")
            if launches and _hot(r["Name"]):
                per_launch += float(r["TotalDurationNs"]) / 1e3 / launches
        if launches:
            out.append(f"\nkernel time per launch of the hot path (library kernels without one-time set-up, "
                       f"{launches} launches): {per_launch:.2f} us\n")
    for path in found("*kernel_trace.csv"):
        # per (kernel, grid): workloads of several shapes launch each kernel at several grids
        from collections import defaultdict
        acc = defaultdict(lambda: [0, 0.0])
        for r in _read_csv(path):
            if not _hot(r["Kernel_Name"]):
                continue
            wg = max(1, int(r["Workgroup_Size_X"]) * int(r["Workgroup_Size_Y"]) * int(r["Workgroup_Size_Z"]))
            blocks = (int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])) // wg
            a = acc[(_short_kernel(r["Kernel_Name"]), blocks)]
            a[0] += 1
            a[1] += (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        if len({k for k, _ in acc}) == len(acc):
            continue   # one grid per kernel: the table above says it all
        out.append(f"### Kernel durations per grid ({os.path.basename(path)}, library kernels of the step)\n")
        out.append("| kernel | workgroups | calls | avg us | us per launch |")
        out.append("|---|---:|---:|---:|---:|")
        for (k, blocks), (calls, tot) in sorted(acc.items(), key=lambda kv: -kv[1][1]):
            per = f"{tot / launches:.1f}" if launches else ""
            out.append(f"| {k} | {blocks} | {calls} | {tot / calls:.2f} | {per} |")
        out.append("")
    cc = found("*counter_collection.csv")
    if cc:
        means = _counter_means(cc)
        scale = {}
        if calib:
            for cn in ("FETCH_SIZE", "WRITE_SIZE"):
                kib = _copy_reading(calib, cn)
                if kib:
                    nbytes = 256 << 20
                    scale[cn] = nbytes / (kib * 1024.0)
                    out.append(f"{cn} calibration: device copy of {nbytes} B reads {kib:.1f} KiB per dispatch "
                               f"-> bytes = KiB x 1024 x {scale[cn]:.4f}")
        counters = sorted({cn for d_ in means.values() for cn in d_})
        out.append("\n### Counters, mean per dispatch (* = kernel of the per-step launch)\n")
        out.append("| kernel | dispatches | " + " | ".join(counters) + " |")
        out.append("|---|---:|" + "---:|" * len(counters))
        totals = {cn: 0.0 for cn in counters}
        for k, d_ in sorted(means.items(), key=lambda kv: kv[0]):
            n = max(v[1] for v in d_.values())
            out.append(f"| {k} | {n} | " + " | ".join(f"{d_[cn][0]:.5g}" if cn in d_ else "" for cn in counters) + " |")
            if launches and k.startswith("*"):
                for cn in counters:
                    if cn in d_:
                        totals[cn] += d_[cn][0] * d_[cn][1] / launches
        if launches:
            out.append(f"\nper launch of the hot path (* kernels, {launches} launches):")
            tb = 0
            for cn in counters:
                line = f"- {cn}: {totals[cn]:.6g}"
                if cn in scale:
                    b = totals[cn] * 1024.0 * scale[cn]
                    tb += b
                    line += f" KiB -> {b:.0f} bytes"
                out.append(line)
            if tb:
                out.append(f"- scaled HBM bytes (those counters above): {tb:.0f}")
                out.append(f"- kernel source digest: {source_digest()}")
        if "SQ_INSTS_VALU" in counters:
            # issue-time floor of each kernel's vector work on the whole chip:
            # a wave64 VALU op holds a 16-lane SIMD 4 cycles (transcendentals
            # 16), an fp32 16x16x4 MFMA 32 cycles; 1024 SIMDs at 2.4 GHz
            out.append("\n### VALU and MFMA issue time per dispatch (1024 SIMDs, 2.4 GHz)\n")
            out.append("| kernel | VALU instr | transcendental % | VALU issue us | MFMA instr | MFMA busy us |")
            out.append("|---|---:|---:|---:|---:|---:|")
            for k, d_ in sorted(means.items(), key=lambda kv: kv[0]):
                if "SQ_INSTS_VALU" not in d_:
                    continue
                iv = d_["SQ_INSTS_VALU"][0]
                tr = d_.get("SQ_INSTS_VALU_TRANS_F32", (0.0, 0))[0]
                mf = d_.get("SQ_INSTS_MFMA", (0.0, 0))[0]
                t_v = (iv - mf + 3.0 * tr) * 4 / 1024 / 2.4e9 * 1e6
                t_m = mf * 32 / 1024 / 2.4e9 * 1e6
                out.append(f"| {k} | {iv:.4g} | {100 * tr / max(iv, 1):.1f} | {t_v:.1f} | {mf:.4g} | {t_m:.1f} |")
        # achieved HBM bandwidth of each library kernel of the step, per launch
        # grid: the scaled FETCH_SIZE + WRITE_SIZE bytes per dispatch over the
        # mean duration of that kernel at that grid in the kernel trace given
        # with the counter directories
        dur = _trace_means(found("*kernel_trace.csv"))
        if dur and "FETCH_SIZE" in scale and "WRITE_SIZE" in scale:
            gmb = _counter_means(cc, by_grid=True)
            rows_bw = []
            for k, d_ in gmb.items():
                if not k.startswith("*") or "FETCH_SIZE" not in d_ or "WRITE_SIZE" not in d_:
                    continue
                key = k[1:]
                if key not in dur:
                    continue
                b = d_["FETCH_SIZE"][0] * 1024.0 * scale["FETCH_SIZE"] + d_["WRITE_SIZE"][0] * 1024.0 * scale["WRITE_SIZE"]
                us = dur[key]
                rows_bw.append((key, b, us, b / (us * 1e3)))
            if rows_bw:
                out.append("\n### Achieved HBM bandwidth per kernel and launch grid (counter bytes / trace duration)\n")
                out.append("| kernel @ workgroups | HBM bytes per dispatch | mean us | GB/s | of 8 TB/s |")
                out.append("|---|---:|---:|---:|---:|")
                for key, b, us, gbs in sorted(rows_bw, key=lambda r: -r[2]):
                    out.append(f"| {key} | {b:.4g} | {us:.2f} | {gbs:.0f} | {gbs / HBM_PEAK_GBS:.3f} |")
        # workloads of several shapes: the same per launch grid of the library's kernels
        gm = {k: d_ for k, d_ in _counter_means(cc, by_grid=True).items() if k.startswith("*")}
        if len(gm) > len([k for k in means if k.startswith("*")]):
            hdr = [cn for cn in ("SQ_INSTS_VALU", "SQ_INSTS_MFMA", "FETCH_SIZE", "WRITE_SIZE") if cn in counters]
            out.append("\n### Per launch grid (kernel @ workgroups), mean per dispatch\n")
            cols = hdr + (["VALU issue us", "MFMA busy us"] if "SQ_INSTS_VALU" in hdr else [])
            cols += [f"{cn} bytes" for cn in ("FETCH_SIZE", "WRITE_SIZE") if cn in hdr and cn in scale]
            out.append("| kernel @ workgroups | dispatches | " + " | ".join(cols) + " |")
            out.append("|---|---:|" + "---:|" * len(cols))
            for k, d_ in sorted(gm.items(), key=lambda kv: kv[0]):
                n = max(v[1] for v in d_.values())
                vals = [f"{d_[cn][0]:.5g}" if cn in d_ else "" for cn in hdr]
                if "SQ_INSTS_VALU" in hdr:
                    iv = d_.get("SQ_INSTS_VALU", (0.0, 0))[0]
                    tr = d_.get("SQ_INSTS_VALU_TRANS_F32", (0.0, 0))[0]
                    mf = d_.get("SQ_INSTS_MFMA", (0.0, 0))[0]
                    vals += [f"{(iv - mf + 3.0 * tr) * 4 / 1024 / 2.4e9 * 1e6:.1f}", f"{mf * 32 / 1024 / 2.4e9 * 1e6:.1f}"]
                vals += [f"{d_[cn][0] * 1024.0 * scale[cn]:.4g}" for cn in ("FETCH_SIZE", "WRITE_SIZE")
                         if cn in hdr and cn in scale and cn in d_]
                out.append(f"| {k} | {n} | " + " | ".join(vals) + " |")
    print("\n".join(out))


MAKERS = {"c1": make_c1, "c2": make_c2, "c3": make_c3, "c4": make_c4, "c5": make_c5, "forms": make_forms}
# the timing leg of the full C4 set draws its inputs on the device
# C3's 840 grads are set once: assigning p.grad for 840 tensors in Python costs
# ~0.3 us each, more than the GPU step, and is input refresh, not optimizer work
# (autograd writes .grad in C++); the step's work does not depend on the values
TIMING_MAKERS = {"c3": lambda device: make_c3(device, pool=1),
                 "c4": lambda device: make_c4(device, pool=1, on_device=True)}
CPU_LEG = ("c2", "c3")   # C4/C5 take minutes per step on the CPU: their parity is tests/test_gpu_full_configs.py


def cpu_and_parity(workload, steps=4):
    """The CPU baseline and the in-run parity check, on identical inputs.

    The CPU oracle (a port of the reference's cuda_ops="off" path) and a fresh
    GPU optimizer both take `steps` steps from the timed leg's own seeded
    inputs (seed 0: the same params and grad pool, cycled the same way).  The
    first CPU step (state set-up) is untimed; the others give the median and
    mean.  Then params, every state tensor and the last step's update
    dp = p_after - p_before are compared; for the spectral route the
    workspace's hash bins and bin counts are compared with the oracle's
    integer restatement, bit for bit."""
    import numpy as np
    import cresso_amd
    from oracle.cresso_oracle import OracleCRESSO5, hash_index_np

    torch.set_num_threads(os.cpu_count() or 1)
    params, grads, kwargs, shapes, _ = MAKERS[workload](torch.device("cpu"))
    pool = len(grads)
    # the reference's sequential fp32 scatter_add carries ~1e-5 relative error
    # of its own at 262144 elements per bin: fp64 bin sums break the tie
    accum = "fp64" if workload == "c2" else "native"
    cpu_ps = [p.detach().clone() for p in params]
    oracle = OracleCRESSO5(cpu_ps, hash_accum=accum, **kwargs)
    dev = torch.device("cuda:0")
    gpu_ps = [torch.nn.Parameter(p.detach().clone().to(dev)) for p in params]
    gopt = cresso_amd.CRESSO5(gpu_ps, cuda_ops="required", **kwargs)
    gdev = [[g.to(dev) for g in gs] for gs in grads]
    times = []
    for k in range(steps):
        last = k == steps - 1
        if last:
            torch.cuda.synchronize()
            before_g = [p.detach().double().cpu() for p in gpu_ps]
            before_o = [p.double() for p in cpu_ps]
        t0 = time.perf_counter()
        oracle.step(grads[k % pool])
        if k:
            times.append(time.perf_counter() - t0)
        for p, g in zip(gpu_ps, gdev[k % pool]):
            p.grad = g
        gopt.step()
    torch.cuda.synchronize()
    # parity
    p_err, p_ok, dp_err, s_err, s_ok = 0.0, True, 0.0, 0.0, True
    for i, (a, b) in enumerate(zip(gpu_ps, cpu_ps)):
        got, exp = a.detach().double().cpu(), b.double()
        d = (got - exp).abs()
        p_err = max(p_err, float(d.max()))
        p_ok = p_ok and bool((d <= 1e-6 + 1e-5 * exp.abs()).all())
        dg, de = got - before_g[i], exp - before_o[i]
        scale = float(de.pow(2).mean().sqrt())
        dp_err = max(dp_err, float(((dg - de).abs() / (de.abs() + scale + 1e-30)).max()))
        sa, sb = gopt.state[a], oracle.state[i]
        for key, v in sb.items():
            if not torch.is_tensor(v) or key == "freqs":
                s_ok = s_ok and (key not in sa or (sa[key] == v if not torch.is_tensor(v)
                                                   else bool(torch.equal(sa[key].cpu(), v))))
                continue
            gv, ev = sa[key].double().cpu(), v.double()
            dd = (gv - ev).abs()
            s_err = max(s_err, float((dd / (ev.abs() + 1e-6)).max()))
            s_ok = s_ok and bool((dd <= 1e-6 + 1e-5 * ev.abs()).all())
    parity = {"steps": steps, "inputs": "identical to the timed leg's (seed 0, same grad pool)",
              "oracle_hash_accum": accum, "tolerance": "rtol 1e-5, atol 1e-6 (fp32)",
              "param_max_abs_err": float(f"{p_err:.3e}"), "params_within_tol": p_ok,
              "state_max_rel_err": float(f"{s_err:.3e}"), "states_within_tol": s_ok,
              "update_max_err_of_scale": float(f"{dp_err:.3e}")}
    if workload == "c2":
        eng = gopt._spectral_engine
        ws = next(iter(eng.ws.values()))
        n = gpu_ps[0].numel()
        T, B = kwargs["hash_tables"], kwargs["hash_bins"]
        bins = torch.empty(T, n, dtype=torch.int32, device=dev)
        counts = torch.empty(T, B, dtype=torch.int64, device=dev)
        import ctypes
        from cresso_amd import _native
        _native.check(eng.lib.cresso_spectral_workspace_bins(
            ws.plan, ctypes.c_void_p(ws.buf.data_ptr()), ctypes.c_size_t(ws.buf.numel()),
            ctypes.c_void_p(bins.data_ptr()), ctypes.c_void_p(counts.data_ptr()),
            ctypes.c_void_p(_native.stream_handle(dev))), "workspace bins")
        torch.cuda.synchronize()
        bins_ok, counts_ok = True, True
        for t in range(T):
            ref = hash_index_np(n, B, t)
            bins_ok = bins_ok and bool(np.array_equal(bins[t].cpu().numpy(), ref))
            counts_ok = counts_ok and bool(np.array_equal(counts[t].cpu().numpy(), np.bincount(ref, minlength=B)))
        parity["bins_bit_exact"] = bins_ok
        parity["counts_bit_exact"] = counts_ok
    parity["ok"] = bool(p_ok and s_ok and parity.get("bins_bit_exact", True) and parity.get("counts_bit_exact", True))
    times.sort()
    med = times[len(times) // 2] if len(times) % 2 else 0.5 * (times[len(times) // 2 - 1] + times[len(times) // 2])
    what = "the full (4096,4096) tensor" if workload == "c2" else "all 840 tensors"
    cpu = dict(value=round(med * 1e3, 3), unit="ms/step", median_ms=round(med * 1e3, 3),
               mean_ms=round(sum(times) / len(times) * 1e3, 3), cores=torch.get_num_threads(), kind="port",
               sample=f"{what}, {len(times)} timed steps after 1 untimed set-up step, on the timed leg's inputs",
               cpu=_cpu_model(), os_cpu_count=os.cpu_count())
    return cpu, parity


def _cpu_model():
    try:
        out = subprocess.run(["lscpu"], stdout=subprocess.PIPE, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return "unknown"


WORKLOAD_NAMES = {"c1": "C1: (2048,2048) fp32 spectral/hash route, rank 8, F=5, B=64, T=2",
                  "c2": "C2: (4096,4096) fp32 spectral/hash route, rank 8, F=5, B=64, T=2",
                  "c3": "C3: 840 LoRA-thin fp32 (4096,16)/(16,4096), scalar route, rank 4",
                  "c4": "C4: 1.2 B fp32 params (embedding (32000,2048), 22 layers of q,k,v,o (2048,2048), gate/up "
                        "(5632,2048), down (2048,5632), two (2048,) norms), rank 8, F=5, B=64, T=2",
                  "c5": "C5: bf16 (8192,8192), fp32 (512,256,3,3), (256,256,3,3), (64,512,512), rank 16, F=7, "
                        "B=256, T=4",
                  "forms": "profile-only: 256 x (999,7) scalar stream form, 4 x (262144,32) wide form, 64 x (64,64) "
                           "micro route, fp32"}


def measure(workload, args):
    """Time one workload on the GPU (and its CPU baseline); one record."""
    res = time_gpu(workload, args.steps, args.warmup)
    nbytes, n = res["nbytes"], res["n"]
    traffic, traffic_note = measured_traffic(workload)
    ms = res["ms_per_step"]
    achieved = nbytes / (ms * 1e-3) / 1e9   # the launch = one step; its mean duration over the timed region
    rec = {
        "workload": workload,
        "value": round(nbytes / (ms * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "ms_per_step": round(ms, 4),
        "config": {"workload": WORKLOAD_NAMES[workload], "elements": n, "algorithmic_bytes_per_step": nbytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_source": traffic_note,
                     "launch": "one optimizer step (the library's kernel sequence); mean over the timed region, "
                               "HIP events on the launch stream"},
    }
    if workload == "c3":
        # the same step with two grad sets alternating (840 p.grad assignments
        # a step inside the timed region); the assignments' host cost alone
        # is reported beside it
        alt = time_gpu(workload, args.steps, args.warmup, maker=lambda device: make_c3(device, pool=2))
        rec["alternating_grads"] = {"grad_sets": 2, "ms_per_step": round(alt["ms_per_step"], 4),
                                    "host_grad_assignment_ms_per_step": round(alt["assign_ms"], 4),
                                    "note": "840 p.grad assignments a step inside the timed region; the line's "
                                            "value is timed with one grad set assigned before the first step"}
    if not args.no_cpu and workload in CPU_LEG:
        rec["cpu_baseline"], rec["parity"] = cpu_and_parity(workload)
        if workload == "c2":
            rec["cpu_baseline"]["note"] = ("the oracle sums the hash bins in fp64 (hash_accum='fp64'); the "
                                           "reference's cuda_ops='off' path sums them sequentially in fp32, "
                                           "the same torch ops otherwise")
    elif workload not in CPU_LEG:
        rec["parity"] = {"in_run": False, "covered_by": "tests/test_gpu_full_configs.py (oracle trajectories at "
                         "this config's shapes)"}
    return rec


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", choices=["c1", "c2", "c3", "c4", "c5", "forms", "copy"], default=None)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--rocprof-summary", default=None, nargs="+", metavar="DIR")
    ap.add_argument("--calib", default=None, nargs="+", metavar="DIR")
    ap.add_argument("--launches", type=int, default=None)
    args = ap.parse_args()
    if args.rocprof_summary:
        rocprof_summary(args.rocprof_summary, args.calib, args.launches)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported in this build "
              "(every GPU box here has one GPU)", file=sys.stderr)
        sys.exit(2)
    workloads = [args.workload] if args.workload else ["c2", "c3", "c4", "c5"]
    if workloads == ["copy"]:
        print(json.dumps({"calibration": "device copy", **copy_calibration(args.steps, args.warmup)}))
        return
    recs = [measure(w, args) for w in workloads]
    first = recs[0]
    out = {
        "metric": METRIC,
        "value": first["value"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": first["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded torch CPU generator, copied to HBM before timing)",
        "config": first["config"],
        "roofline": first["roofline"],
    }
    if "cpu_baseline" in first:
        out["cpu_baseline"] = first["cpu_baseline"]
        out["parity"] = first["parity"]
    if "alternating_grads" in first:
        out["alternating_grads"] = first["alternating_grads"]
    if len(recs) > 1:
        # the metric names both headline configs: the second rides along with
        # the same fields (value = algorithmic GB/s, ms_per_step, roofline, CPU)
        out["secondary"] = recs[1:]
    print(json.dumps(out))


if __name__ == "__main__":
    main()
